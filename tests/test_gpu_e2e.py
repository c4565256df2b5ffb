"""SlideFSDP end to end on small Llama and Qwen2 models, across the runtime's
options: staging order, update parity with the oracle (bit-exact), parity
with a non-offloaded PyTorch bf16 run over 10 steps (bit-identical gradients
and losses where the output unit computes the loss as the reference does),
padding masks, learning-rate changes and save_pretrained.

The non-offloaded run starts from the same bf16 weights and fp32 rotary
frequencies (``fullsize.gpu_bf16_copy``): the same kernels then see the same
bits, so offloading, recomputing from offloaded checkpoints and staging
change nothing."""

import os

import numpy as np
import pytest
import torch

import oracle
from fullsize import gpu_bf16_copy

pytestmark = pytest.mark.gpu

V, H, I, L = 1024, 256, 512, 3
LR, BETAS, EPS, WD = 1e-3, (0.9, 0.999), 1e-8, 0.01


def make_model(arch: str = "llama", vocab: int = V):
    """A small model of the Llama-3 family, or of the Qwen2 family (q/k/v
    projections with biases, as Qwen2.5-14B)."""
    if arch == "llama":
        from transformers import LlamaConfig as C, LlamaForCausalLM as M
    else:
        from transformers import Qwen2Config as C, Qwen2ForCausalLM as M
    cfg = C(vocab_size=vocab, hidden_size=H, intermediate_size=I, num_hidden_layers=L,
            num_attention_heads=8, num_key_value_heads=4, max_position_embeddings=512,
            rope_theta=500000.0, tie_word_embeddings=False)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(1234)
    model = M(cfg)
    if arch != "llama":
        with torch.no_grad():  # non-zero biases, so that their updates are checked too
            for name, p in model.named_parameters():
                if name.endswith(".bias"):
                    p.normal_(0.0, 0.02)
    return model


def units_of(model):
    m = model.model
    return [[m.embed_tokens.weight]] + [list(l.parameters()) for l in m.layers] + [[m.norm.weight, model.lm_head.weight]]


def batches(n, B=2, S=128, vocab=V):
    g = torch.Generator().manual_seed(99)
    return [torch.randint(0, vocab, (B, S), generator=g) for _ in range(n)]


def u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("resident", [0, L - 1])
def test_schedule_matches_oracle(dev, resident):
    from test1_amd import SlideFSDP, SlideFSDPConfig

    sf = SlideFSDP(make_model(), SlideFSDPConfig(device=dev, lr=LR, weight_decay=WD), wait_timeout=120,
                   resident_layers=resident)
    ids = batches(2)
    for k in range(2):
        sf.runtime.trace = []
        sf(input_ids=ids[k].to(dev), labels=ids[k].to(dev))
        sf.wait_for_updates()
        # resident decoders are units L - resident .. L - 1
        exp = oracle.step_schedule(L, first_decoder_first=True, resident_units=tuple(range(L - resident, L)))
        assert sf.runtime.trace == exp, f"step {k}"
    sf.close()


# (parameter H2D format, resident decoder layers, gradient D2H engine, host gradient slots:
#  None = one per unit, k = a ring of k; the model family; the fused chunked cross entropy)
MODES = [("fp32", 0, "sdma", None, "llama", False), ("bf16", 0, "sdma", None, "llama", False),
         ("fp32", L - 1, "sdma", None, "llama", False), ("bf16", L - 1, "sdma", None, "llama", False),
         ("fp32", 0, "kernel", None, "llama", False), ("bf16", L - 1, "kernel", None, "llama", False),
         ("fp32", L - 1, "sdma", 2, "llama", False), ("bf16", 0, "kernel", 2, "llama", False),
         ("fp32", L - 1, "sdma", None, "qwen2", False), ("bf16", 0, "kernel", None, "qwen2", False),
         ("fp32", L - 1, "sdma", None, "llama", True), ("bf16", 0, "sdma", None, "qwen2", True)]


@pytest.mark.parametrize("h2d_format,resident,d2h_engine,ring,arch,fused", MODES)
def test_updates_match_oracle_bit_exact(dev, h2d_format, resident, d2h_engine, ring, arch, fused):
    """Every unit's host update equals the oracle AdamW applied to the same
    (captured) bf16 grads and fp32 master, for 3 steps.  With bf16 H2D the
    host bf16 copy of every unit is the oracle cast of its master after each
    step, so both formats stage the same bits.  ``resident`` decoder layers
    keep their forward weights for the backward."""
    check_updates_against_oracle(dev, arch, h2d_format, {}, dict(
        resident_layers=resident, d2h_engine=d2h_engine, grad_ring_depth=ring, fused_cross_entropy=fused))


@pytest.mark.parametrize("bf16_reload", [False, True])
def test_pool_schedule_reloads(dev, bf16_reload):
    """The reference's schedule (every unit in the 2-unit pool, reloaded for
    its backward) with the backward's reloads as fp32 + cast at use
    (``bf16_reload=False``) or from the bf16 copy each update writes (the
    default with fp32 H2D): every update bit-exact vs the oracle over 3 steps,
    and step-1 gradients and the 10-step losses equal to the non-offloaded
    run's (a reload copy an update left stale would change a later step's
    gradients)."""
    sf = check_updates_against_oracle(dev, "llama", "fp32", {}, dict(resident_layers=0, bf16_reload=bf16_reload),
                                      keep=True)
    try:
        assert sf.bf16_reload_units == (list(range(1, L)) if bf16_reload else [])
    finally:
        sf.close()
    check_loss_parity(dev, "llama", False, {}, dict(resident_layers=0, bf16_reload=bf16_reload))


# Updates in pieces of 40,000 elements: a decoder (590,336 elements) comes back, is
# updated and is staged in 15 pieces, the output unit in 7, cutting parameters
# inside their vector body.  (H2D format, resident decoders, D2H engine, slot ring, family)
PIECE = 40000
PIECE_MODES = [("fp32", L - 1, "sdma", None, "llama"), ("bf16", L - 1, "sdma", None, "llama"),
               ("fp32", 0, "sdma", None, "qwen2"), ("fp32", L - 1, "kernel", 2, "llama"),
               ("bf16", 0, "copy", None, "llama")]


@pytest.mark.parametrize("h2d_format,resident,d2h_engine,ring,arch", PIECE_MODES)
def test_piecewise_updates_match_oracle_bit_exact(dev, h2d_format, resident, d2h_engine, ring, arch):
    """Units updated in pieces: each piece's gradients are waited for just
    before its AdamW (SDMA: one copy per piece), and own units are copied to
    the device piece by piece right after each piece's update, then cast in
    one launch.  The updates, the staged weights the next forward computes
    with, and the moments stay the oracle's, bit for bit, over 3 steps; with
    every unit in a buffer of its own the staging really ran in pieces (at
    least two decoders' worth of piece copies; each fp32 cast one whole unit)."""
    sf = check_updates_against_oracle(dev, arch, h2d_format, {}, dict(
        resident_layers=resident, d2h_engine=d2h_engine, grad_ring_depth=ring, update_piece_elems=PIECE),
        keep=True, timing=True)
    plan = sf.layer_states[1]._piece_plan()
    assert plan is not None and len(plan[0]) == 15
    assert len(sf.layer_states[L + 1]._piece_plan()[0]) == 7
    st = sf.runtime.stager
    sizes = [n // (4 if h2d_format == "fp32" else 2) for _, _, n in st.copy_timing]
    assert sizes
    if resident == L - 1:
        # the first forward stages the units whole, later stagings run in pieces
        # (a unit whose backward still holds it when its update starts is
        # staged whole by the next forward instead)
        assert sum(1 for n in sizes if n <= PIECE + 15) >= 2 * 15, sizes
        if h2d_format == "fp32":
            unit_sizes = {s.total_size for s in sf.layer_states}
            assert {n for _, _, n in st.cast_timing} <= unit_sizes
    sf.close()


def test_piecewise_updates_with_moments_on_storage(dev, tmp_path):
    """Updates in pieces with the first moment on local storage (2 buffers,
    so moments are evicted and read back within every step): bit-exact
    against the oracle over 3 steps."""
    check_updates_against_oracle(dev, "llama", "fp32", storage_config(tmp_path, "cpu", 0.3),
                                 dict(update_piece_elems=PIECE), nvme_buffers=2)


# (cast where the unit is next used, byte cap of the whole-unit slots: None = default)
CAST_PLACEMENTS = [(True, None), (False, None), (True, 0)]


@pytest.mark.parametrize("cast_at_use,slot_cap", CAST_PLACEMENTS)
def test_cast_placement_matches_oracle(dev, cast_at_use, slot_cap):
    """Units staged after their update (every unit resident, fp32 H2D): copied
    into a whole-unit device slot and cast on the forward's stream right
    before the unit's forward (default), cast on the cast stream as soon as
    the copy lands (``cast_at_use=False``), or, with no slot to be had, staged
    through the ring.  Updates, staged weights and moments stay the oracle's,
    bit for bit, over 3 steps, and the slots are used only by the first."""
    def setup(sf):
        if slot_cap is not None:
            sf.runtime.stager.slots.cap_bytes = slot_cap

    sf = check_updates_against_oracle(dev, "llama", "fp32", {}, dict(resident_layers=L - 1, cast_at_use=cast_at_use),
                                      keep=True, setup=setup)
    assert sf.runtime.cast_at_use == cast_at_use
    used = sf.runtime.stager.slots.bytes
    assert (used > 0) == (cast_at_use and slot_cap is None), used
    sf.close()


def test_dropped_stagings_restage_from_the_master(dev):
    """Stagings for the next forward dropped between steps (``refresh_host_copy``,
    as after writing a master directly): units copied but not cast give their
    slot back, and the next forward stages them from the master through the
    ring; every update stays the oracle's, bit for bit, and no slot is lost
    (free slots plus those still held by a staging add up to the pool)."""
    from test1_amd.layer_state import PendingCast

    dropped = []

    def between(sf, k):
        if k == 1:
            held = [s for s in sf.layer_states if s._prefetched is not None and isinstance(s._prefetched[1], PendingCast)]
            dropped.append(len(held))
            for s in sf.layer_states:
                s.refresh_host_copy()

    sf = check_updates_against_oracle(dev, "llama", "fp32", {}, dict(resident_layers=L - 1), keep=True, between=between)
    assert dropped and dropped[0] > 0
    pool = sf.runtime.stager.slots
    free = sum(t.numel() * 4 for lst in pool._free.values() for t, _ in lst)
    held = sum(4 * s._prefetched[1].n for s in sf.layer_states
               if s._prefetched is not None and isinstance(s._prefetched[1], PendingCast))
    held += sum(4 * s._pending_cast.n for s in sf.layer_states if s._pending_cast is not None)
    assert free + held == pool.bytes, (free, held, pool.bytes)
    sf.close()
    assert pool.bytes == 0 and not pool._free     # close gives every slot back


@pytest.mark.parametrize("grad", [False, True])
def test_evaluation_forwards_between_steps(dev, grad):
    """Forwards without labels between training steps, under ``no_grad`` or
    with autograd on and no backward (checkpoints packed, nothing unpacked):
    two such forwards give identical logits, and every update of the
    training that follows stays the oracle's, bit for bit."""
    seen = []

    def between(sf, k):
        ids = batches(1)[0].to(dev)
        with torch.set_grad_enabled(grad):
            a = sf(input_ids=ids).logits.detach().float().clone()
            b = sf(input_ids=ids).logits.detach().float().clone()
        assert torch.equal(a, b), f"step {k}"
        seen.append(a)

    check_updates_against_oracle(dev, "llama", "fp32", {}, dict(resident_layers=L - 1), between=between)
    assert len(seen) == 2


@pytest.mark.parametrize("h2d_format", ["fp32", "bf16"])
def test_masters_written_between_steps(dev, h2d_format):
    """Masters written directly between training steps (``load_state_dict``
    after a forward without labels, which leaves the units with own buffers,
    the last decoder and the output unit loaded), between
    ``release_device_units`` and ``refresh_host_copies``: the next forward
    computes with the cast of the new masters, and every update that follows
    is the oracle's on the new masters, bit for bit."""
    def between(sf, k):
        model = sf.base_model
        with torch.no_grad():
            sf(input_ids=batches(1)[0].to(dev))
        assert sum(s.is_resident() for s in sf.layer_states) >= 2
        sf.release_device_units()
        assert not any(s.is_resident() for s in sf.layer_states)
        g = torch.Generator().manual_seed(100 + k)
        new = {n: p.detach() + 0.01 * torch.randn(p.shape, generator=g) for n, p in model.named_parameters()}
        model.load_state_dict(new, strict=False)
        sf.refresh_host_copies()
        name_of = {id(p): n for n, p in model.named_parameters()}
        arrays = {u: [new[name_of[id(p)]].numpy() for p in ps] for u, ps in enumerate(units_of(model))}
        # the next forward stages the new masters
        with torch.no_grad():
            sf(input_ids=batches(1)[0].to(dev))
        torch.cuda.synchronize()
        staged = 0
        for u, st in enumerate(sf.layer_states):
            if st.is_resident():
                exp = oracle.cast_f32_bf16(np.concatenate([a.reshape(-1) for a in arrays[u]]))
                assert np.array_equal(u16(st._current_gpu_cache["param"][:st.total_size]), exp), (k, u)
                staged += 1
        assert staged >= 2
        return arrays

    check_updates_against_oracle(dev, "llama", h2d_format, {}, dict(resident_layers=L - 1), between=between)


@pytest.mark.parametrize("early", [True, False])
def test_embedding_early_rows(dev, early):
    """The embedding's update in two parts (default): the rows the batch does
    not touch as the backward starts, the batch's rows after their gradient.
    Every update stays the oracle's, bit for bit, over 3 steps (batches of
    changing shape), and the early part ran once in every step; with
    ``early_embedding_update=False`` the table is updated in one part after
    the backward."""
    def setup(sf):
        sf.runtime.timeline = []

    sf = check_updates_against_oracle(dev, "llama", "fp32", {}, dict(early_embedding_update=early), keep=True,
                                      setup=setup, shapes=[(2, 128), (1, 96), (2, 128)])
    marks = [w for _, _, w, u in sf.runtime.timeline if u == 0 and w in ("early_update_done", "update_start")]
    assert marks.count("update_start") == 3, marks
    # one early part per step (run by the late part itself if it came first)
    assert marks.count("early_update_done") == (3 if early else 0), marks
    sf.close()


def test_out_of_range_input_id_raises_at_the_update(dev):
    """An input id just past the vocabulary (labels valid): the lookup's
    bounds check flags it instead of reading outside the host table, the
    backward's dense embedding gradient stays inside the table, the
    embedding's early rows are skipped, and its update raises ValueError,
    which wait_for_updates reports."""
    from test1_amd import SlideFSDP, SlideFSDPConfig

    sf = SlideFSDP(make_model(), SlideFSDPConfig(device=dev, lr=LR, weight_decay=WD), wait_timeout=120)
    ids = batches(1)[0]
    labels = ids.clone()
    ids[0, 5] = V
    sf(input_ids=ids.to(dev), labels=labels.to(dev))
    with pytest.raises(ValueError, match="outside"):
        sf.wait_for_updates()
    assert sf.layer_optimizer._early_rows == {}
    try:
        sf.close()
    except ValueError:
        pass


def test_failed_backward_leaves_the_wrapper_usable(dev):
    """A backward that raises part-way (a host-side hook on the first
    decoder's weight raises; every kernel completes normally): the error
    reaches the caller, the offloads and updates already queued finish, no
    unit stays on the device (with the 2-unit pool, a unit left loaded would
    block the next step's load), the embedding's early update part is closed,
    and the next two steps train every unit."""
    from test1_amd import SlideFSDP, SlideFSDPConfig

    sf = SlideFSDP(make_model(), SlideFSDPConfig(device=dev, lr=LR, weight_decay=WD), wait_timeout=120,
                   resident_layers=0)
    ids = batches(3)

    def boom(grad):
        raise RuntimeError("injected backward failure")

    h = sf.layer_states[1].layer.self_attn.q_proj.weight.register_hook(boom)
    with pytest.raises(RuntimeError, match="injected"):
        sf(input_ids=ids[0].to(dev), labels=ids[0].to(dev))
    h.remove()
    assert not any(s.is_resident() for s in sf.layer_states)
    assert sf.buffer_pool.available() == sf.buffer_pool.pool_size
    assert sf.layer_states[0]._early is None and sf.layer_optimizer._early_rows == {}
    before = [g["step"] for g in sf.layer_optimizer.param_groups]
    assert before[2:] == [1] * L and before[1] == 0      # units above the failure were updated
    for k in (1, 2):
        loss = sf(input_ids=ids[k].to(dev), labels=ids[k].to(dev)).loss.item()
        sf.wait_for_updates()
        assert np.isfinite(loss)
    after = [g["step"] for g in sf.layer_optimizer.param_groups]
    assert [b - a for a, b in zip(before, after)] == [2] * (L + 2)
    sf.close()


def test_cast_at_use_loss_parity(dev):
    """Casts where the unit is next used, against the non-offloaded run:
    first-step gradients and 10 losses."""
    check_loss_parity(dev, "llama", False, {}, dict(resident_layers=L - 1, cast_at_use=True))


# checkpoint offload mode, optimizer moments on storage (fraction), H2D format
STORAGE_MODES = [("nvme", 0.0, "fp32"), ("cpu", 0.3, "fp32"), ("nvme", 0.8, "bf16")]


def storage_config(tmp_path, ac_mode, fraction):
    return dict(ac_offload_mode=ac_mode, ac_offload_dir=str(tmp_path / "ac"),
                optimizer_nvme_offload_fraction=fraction, optimizer_offload_dir=str(tmp_path / "opt"))


@pytest.mark.parametrize("ac_mode,fraction,h2d_format", STORAGE_MODES)
def test_storage_offload_updates_match_oracle_bit_exact(dev, tmp_path, ac_mode, fraction, h2d_format):
    """Checkpoint inputs on local storage (``ac_offload_mode="nvme"``) and/or
    AdamW moments on local storage (``optimizer_nvme_offload_fraction``: the
    first moment above 0, both above 0.5): the updates stay those of the
    oracle AdamW, bit for bit, over 3 steps (2 moment buffers, so moments
    are evicted and read back within every step)."""
    check_updates_against_oracle(dev, "llama", h2d_format, storage_config(tmp_path, ac_mode, fraction), {},
                                 nvme_buffers=2)


def test_changing_batch_shapes_match_oracle(dev):
    """Batches of different sizes and lengths in one run ([2,128], [1,96],
    [3,64], [2,128]): checkpoint slots, embedding row buffers and rotary
    tables follow the shape, and every update stays the oracle's, bit for
    bit."""
    check_updates_against_oracle(dev, "llama", "fp32", {}, {}, shapes=[(2, 128), (1, 96), (3, 64), (2, 128)])


@pytest.mark.parametrize("h2d_format", ["fp32", "bf16"])
def test_without_activation_checkpoints(dev, h2d_format):
    """``enable_activation_checkpoint=False`` with every unit in a device
    buffer of its own: the activations stay in HBM and nothing is recomputed;
    updates stay the oracle's, bit for bit, and the losses match the
    non-offloaded run."""
    check_updates_against_oracle(dev, "llama", h2d_format, dict(enable_activation_checkpoint=False), {})
    check_loss_parity(dev, "llama", False, dict(enable_activation_checkpoint=False), dict(h2d_format=h2d_format))


def test_without_activation_checkpoints_needs_own_buffers(dev):
    from test1_amd import SlideFSDP, SlideFSDPConfig

    with pytest.raises(NotImplementedError):
        SlideFSDP(make_model(), SlideFSDPConfig(device=dev, enable_activation_checkpoint=False), resident_layers=0)


def test_fallback_slot_ring_when_per_unit_slots_do_not_fit(dev, monkeypatch):
    """Pinning one gradient slot per unit fails (as for Qwen2.5-14B with fp32
    masters on hosts with a pinned-memory cap): the output unit (vocab 8192,
    more than twice a decoder) gets a slot of its own, the decoders share a
    ring of decoder-sized slots, widened after the first step; updates stay
    the oracle's, bit for bit, over 4 steps."""
    from test1_amd import _native, layer_state

    class Refused(layer_state.GradSlotsPerUnit):
        def __init__(self, *a, **k):
            raise _native.NativeError("sf_host_alloc failed: out of memory", _native.HIP_ERROR_OUT_OF_MEMORY)

    monkeypatch.setattr(layer_state, "GradSlotsPerUnit", Refused)
    sf = check_updates_against_oracle(dev, "llama", "fp32", {}, {}, steps=4, vocab=8192, keep=True)
    ring = sf.runtime.grad_ring
    assert isinstance(ring, layer_state.GradSlotRing)
    assert set(ring.big) == {L + 1} and ring.depth == L     # grown to one slot per decoder
    sf.close()


@pytest.mark.parametrize("refused", [(1,), (0, 1)])
def test_checkpoints_kept_on_device_when_slots_cannot_be_pinned(dev, monkeypatch, refused):
    """Pinning the checkpoint slot of decoders ``refused`` fails (the
    driver's pinned-memory limit): those decoders keep their checkpoints in
    HBM, the others still go through pinned slots; updates stay the
    oracle's, bit for bit, over 3 steps, and the first-step gradients and 10
    losses are the non-offloaded run's, bit for bit."""
    from test1_amd import _native, sliding_checkpoint
    from test1_amd.sliding_checkpoint import KeptOnDevice

    real = sliding_checkpoint.pinned_empty
    calls = []

    def pinned_empty(shape, dtype):
        calls.append(tuple(shape))
        # the per-decoder slots come first, in decoder order, once per run
        if (len(calls) - 1) % L in refused:
            raise _native.NativeError("sf_host_alloc failed: out of memory", _native.HIP_ERROR_OUT_OF_MEMORY)
        return real(shape, dtype)

    monkeypatch.setattr(sliding_checkpoint, "pinned_empty", pinned_empty)
    with pytest.warns(UserWarning, match="could not be pinned"):
        sf = check_updates_against_oracle(dev, "llama", "fp32", {}, {}, keep=True)
    kept = [i for i, t in enumerate(sf.layer_tensors) if isinstance(t[0], KeptOnDevice)]
    assert kept == list(refused)
    assert all(isinstance(t[0], torch.Tensor) for i, t in enumerate(sf.layer_tensors) if i not in refused)
    sf.close()
    calls.clear()
    with pytest.warns(UserWarning, match="could not be pinned"):
        check_loss_parity(dev, "llama", False, {}, {})


def check_updates_against_oracle(dev, arch, h2d_format, cfg_kw, sf_kw, steps=3, nvme_buffers=None, shapes=None,
                                 vocab=V, keep=False, timing=False, setup=None, between=None):
    from test1_amd import SlideFSDP, SlideFSDPConfig

    model = make_model(arch, vocab=vocab)
    sf = SlideFSDP(model, SlideFSDPConfig(device=dev, lr=LR, weight_decay=WD, adam_betas=BETAS, adam_eps=EPS,
                                          **cfg_kw),
                   wait_timeout=120, h2d_format=h2d_format, **sf_kw)
    if setup is not None:
        setup(sf)
    if timing:
        sf.runtime.stager.cast_timing, sf.runtime.stager.copy_timing = [], []
    if nvme_buffers is not None and sf.layer_optimizer.offloader is not None:
        sf.layer_optimizer.offloader.n_buffers = nvme_buffers
    orc = oracle.LayerAdamOracle(lr=LR, betas=BETAS, eps=EPS, weight_decay=WD)
    ref_units = []
    for ps in units_of(model):
        arrs = [p.detach().numpy().copy() for p in ps]
        ref_units.append(arrs)
        orc.add_layer(arrs)
    if shapes is None:
        steps_ids = batches(steps, vocab=vocab)
    else:
        steps_ids = [batches(1, B, S, vocab=vocab)[0] for B, S in shapes]
    for k, ids in enumerate(steps_ids):
        if between is not None and k > 0:
            # a hook that writes the masters returns their new values per unit
            for u, arrs in (between(sf, k) or {}).items():
                for a, b in zip(ref_units[u], arrs):
                    a[...] = b
        sf.runtime.capture = {}
        ids = ids.to(dev)
        sf(input_ids=ids, labels=ids)
        sf.wait_for_updates()
        cap = sf.runtime.capture
        assert sorted(k for k in cap if isinstance(k, int)) == list(range(L + 2))
        for u in range(L + 2):
            # the packed host grads are the device grads, bit for bit, in layout order
            dev_grads = cap[("device_grads", u)]
            exp = oracle.pack_b16([u16(g) for g in dev_grads])
            assert np.array_equal(u16(cap[u][0]), exp), f"unit {u} packed grads"
        for u in range(L + 1, -1, -1):  # update order of the runtime
            grads, master_before = cap[u]
            flat_before = np.concatenate([a.reshape(-1) for a in ref_units[u]])
            assert np.array_equal(master_before.numpy().view(np.uint32), flat_before.view(np.uint32)), f"unit {u}"
            g = u16(grads)
            if sf.dtype == torch.float16:
                g = g.view(np.float16)
            parts, off = [], 0
            for a in ref_units[u]:
                parts.append(g[off:off + a.size].reshape(a.shape))
                off += a.size
            orc.step_layer(u, parts)
        for u, ps in enumerate(units_of(model)):
            for p, a in zip(ps, ref_units[u]):
                assert np.array_equal(p.detach().numpy().view(np.uint32), a.view(np.uint32)), f"unit {u}"
            if h2d_format == "bf16":
                flat = np.concatenate([a.reshape(-1) for a in ref_units[u]])
                assert np.array_equal(u16(sf.layer_states[u]._cpu_params_bf16), oracle.cast_f32_bf16(flat)), f"unit {u}"
    opt = sf.layer_optimizer
    for u in range(L + 2):
        m, v = opt.layer_states(u)
        om, ov = orc.moments(u)
        assert np.array_equal(m.numpy().view(np.uint32), om.view(np.uint32)), f"unit {u} exp_avg"
        assert np.array_equal(v.numpy().view(np.uint32), ov.view(np.uint32)), f"unit {u} exp_avg_sq"
    if keep:
        return sf
    sf.close()


def reference_losses(model, steps_ids, dev, dtype=torch.bfloat16):
    """Non-offloaded run: the model on the GPU in ``dtype``, same loss as
    OutputLayer, fp32 masters updated by the oracle AdamW unit by unit (last
    unit first)."""
    cast = oracle.cast_f32_bf16 if dtype == torch.bfloat16 else oracle.cast_f32_f16
    gm = gpu_bf16_copy(model, dev, dtype)
    units_gpu = units_of(gm)
    masters = [[p.detach().float().numpy().copy() for p in ps] for ps in units_of(model)]
    orc = oracle.LayerAdamOracle(lr=LR, betas=BETAS, eps=EPS, weight_decay=WD)
    for arrs in masters:
        orc.add_layer(arrs)
    losses, first_grads = [], None
    for ids in steps_ids:
        with torch.no_grad():
            for ps, arrs in zip(units_gpu, masters):
                for p, a in zip(ps, arrs):
                    b = cast(a)
                    p.data.copy_(torch.from_numpy(b.view(np.int16)).view(dtype).view(p.shape))
        ids = ids.to(dev)
        gm.zero_grad(set_to_none=True)
        hidden = gm.model(input_ids=ids).last_hidden_state
        logits = gm.lm_head(hidden)
        loss = torch.nn.functional.cross_entropy(logits[..., :-1, :].reshape(-1, V), ids[..., 1:].reshape(-1))
        loss.backward()
        losses.append(loss.item())
        grads = [[u16(p.grad).reshape(p.shape) for p in ps] for ps in units_gpu]
        if first_grads is None:
            first_grads = grads
        for u in range(len(units_gpu) - 1, -1, -1):
            orc.step_layer(u, grads[u] if dtype == torch.bfloat16 else [g.view(np.float16) for g in grads[u]])
    return losses, first_grads


@pytest.mark.parametrize("h2d_format,resident,d2h_engine,ring,arch,fused", MODES)
def test_loss_parity_with_non_offloaded_run(dev, h2d_format, resident, d2h_engine, ring, arch, fused):
    check_loss_parity(dev, arch, fused, {}, dict(h2d_format=h2d_format, resident_layers=resident,
                                                 d2h_engine=d2h_engine, grad_ring_depth=ring,
                                                 fused_cross_entropy=fused))


@pytest.mark.parametrize("h2d_format", ["fp32", "bf16"])
def test_whole_embedding_matches_oracle_bit_exact(dev, h2d_format):
    """``row_sparse_embedding=False``: the embedding unit is staged whole and
    its whole gradient offloaded, as the reference does; every update is the
    oracle's over 3 steps, and the 10-step losses equal the non-offloaded
    run's."""
    sf = check_updates_against_oracle(dev, "llama", h2d_format, {}, dict(row_sparse_embedding=False), keep=True)
    assert not sf.layer_states[0].row_sparse
    sf.close()
    check_loss_parity(dev, "llama", False, {}, dict(h2d_format=h2d_format, row_sparse_embedding=False))


@pytest.mark.parametrize("resident,d2h_engine", [(0, "sdma"), (L - 1, "kernel")])
def test_float16_units_match_oracle_bit_exact(dev, resident, d2h_engine):
    """dtype=float16 (the reference's config allows it, config.py:110-113):
    units staged with the fp32 -> fp16 cast, fp16 gradients offloaded and
    widened exactly by the host AdamW; every update, moment and packed
    gradient is the oracle's over 3 steps.  The embedding is staged whole
    (its row gathers round to bf16)."""
    sf = check_updates_against_oracle(dev, "llama", "fp32", dict(dtype=torch.float16),
                                      dict(resident_layers=resident, d2h_engine=d2h_engine), keep=True)
    assert sf.dtype == torch.float16 and not sf.layer_states[0].row_sparse
    assert sf.buffer_pool.pool[0]["param"].dtype == torch.float16
    sf.close()


def test_float16_loss_parity_with_non_offloaded_run(dev):
    """float16 units against a non-offloaded fp16 run of the same weights:
    step-1 gradients and the 10 losses bit-identical."""
    check_loss_parity(dev, "qwen2", False, dict(dtype=torch.float16), dict(resident_layers=L - 1))


def test_piecewise_loss_parity(dev):
    """Updates in pieces against the non-offloaded run: first-step gradients
    and 10 losses (no capture after the first step: every piece's AdamW
    starts as soon as its own gradient copy has landed)."""
    check_loss_parity(dev, "llama", False, {}, dict(resident_layers=L - 1, update_piece_elems=PIECE))


# Copy options that change only the speed, in the pool schedule where both
# matter: checkpoints by the pack kernel beside SDMA gradient copies, and the
# unit-load issue limit off and at its tightest.
COPY_OPTIONS = [dict(checkpoint_d2h="kernel"), dict(h2d_issue_limit=0), dict(h2d_issue_limit=1)]


@pytest.mark.parametrize("opts", COPY_OPTIONS, ids=["ckpt_kernel", "issue_unlimited", "issue_1"])
def test_copy_options_match_oracle_and_non_offloaded_run(dev, opts):
    """Every update the oracle's over 3 steps, and step-1 gradients and 10
    losses equal to the non-offloaded run's, with each option set."""
    kw = dict(resident_layers=0, d2h_engine="sdma", **opts)
    sf = check_updates_against_oracle(dev, "llama", "fp32", {}, kw, keep=True)
    assert sf._checkpoint_d2h == opts.get("checkpoint_d2h", "sdma")
    assert sf.runtime.h2d_issue_limit == opts.get("h2d_issue_limit", 3)
    sf.close()
    check_loss_parity(dev, "llama", False, {}, kw)


@pytest.mark.parametrize("ac_mode,fraction,h2d_format", STORAGE_MODES)
def test_storage_offload_loss_parity(dev, tmp_path, ac_mode, fraction, h2d_format):
    """The storage modes against the non-offloaded run: first-step gradients
    (through checkpoints read back from files) and 10 losses."""
    check_loss_parity(dev, "llama", False, storage_config(tmp_path, ac_mode, fraction), dict(h2d_format=h2d_format))


def check_loss_parity(dev, arch, fused, cfg_kw, sf_kw):
    from test1_amd import SlideFSDP, SlideFSDPConfig

    model = make_model(arch)
    steps = batches(10)
    ref_losses, ref_grads = reference_losses(model, steps, dev, cfg_kw.get("dtype", torch.bfloat16))
    sf = SlideFSDP(model, SlideFSDPConfig(device=dev, lr=LR, weight_decay=WD, adam_betas=BETAS, adam_eps=EPS,
                                          **cfg_kw),
                   wait_timeout=120, **sf_kw)
    losses = []
    for k, ids in enumerate(steps):
        if k == 0:
            sf.runtime.capture = {}
        ids = ids.to(dev)
        losses.append(sf(input_ids=ids, labels=ids).loss.item())
        sf.wait_for_updates()
        if k == 0:
            cap, sf.runtime.capture = sf.runtime.capture, None
            for u, ref_u in enumerate(ref_grads):
                got = u16(cap[u][0]).view(np.int16).view(np.uint16)
                exp = np.concatenate([g.reshape(-1) for g in ref_u])
                gf = torch.from_numpy(got.view(np.int16).copy()).view(torch.bfloat16).float()
                ef = torch.from_numpy(exp.view(np.int16).copy()).view(torch.bfloat16).float()
                rel = ((gf - ef).norm() / ef.norm().clamp_min(1e-30)).item()
                exact = float((got == exp).mean())
                print(f"unit {u}: grad rel-L2 {rel:.2e}, bit-exact fraction {exact:.4f}")
                if fused:
                    # the chunked cross entropy sums the loss gradient in
                    # another order than the reference's full-logits loss
                    assert rel < 1e-2, f"unit {u} grads"
                else:
                    assert exact == 1.0, f"unit {u}: step-1 gradients differ from the non-offloaded run's"
    print("losses", [round(x, 5) for x in losses])
    print("ref   ", [round(x, 5) for x in ref_losses])
    if not fused:
        # same gradients and the same AdamW (the oracle's bits): the whole
        # trajectory is the non-offloaded run's
        assert losses == ref_losses, (losses, ref_losses)
    for a, b in zip(losses, ref_losses):
        assert abs(a - b) <= 1e-2 * abs(b), (a, b)
    # first step, same weights: equal up to the reference's bf16 loss (the
    # fused path returns the fp32 loss; half a bf16 ulp is 2**-9 relative)
    assert abs(losses[0] - ref_losses[0]) <= (2.0 ** -8 if fused else 1e-3) * abs(ref_losses[0])
    sf.close()


def test_padding_mask_matches_non_offloaded_run(dev):
    """Left-padded batch: the padding mask reaches every layer (the causal
    mask is built as the model itself builds it) and the checkpointed mask
    round-trips through host memory.  The logits of the padded sequence's
    real tokens equal a non-offloaded run's with the mask, bit for bit, and
    differ from the run without it; the loss is finite over two steps."""
    from test1_amd import SlideFSDP, SlideFSDPConfig

    model = make_model()
    gm = gpu_bf16_copy(model, dev)
    ids = batches(1)[0].to(dev)
    mask = torch.ones_like(ids)
    mask[1, :40] = 0  # second sequence: 40 padding tokens in front
    labels = ids.masked_fill(mask == 0, -100)
    with torch.no_grad():
        ref = gm.lm_head(gm.model(input_ids=ids, attention_mask=mask).last_hidden_state).float()
        ref_nomask = gm.lm_head(gm.model(input_ids=ids).last_hidden_state).float()
    del gm
    sf = SlideFSDP(model, SlideFSDPConfig(device=dev, lr=LR, weight_decay=WD), wait_timeout=120)
    out = sf(input_ids=ids, attention_mask=mask, labels=labels)
    got = out.logits.detach().float()
    sf.wait_for_updates()

    def rel(a, b):
        return ((a - b).norm() / b.norm()).item()

    d_mask = rel(got[1, 40:], ref[1, 40:])
    d_nomask = rel(got[1, 40:], ref_nomask[1, 40:])
    print("padded sequence logits: rel-L2 vs masked reference", d_mask, "vs unmasked", d_nomask)
    # same weights and kernels: the real tokens' logits are the masked run's, bit for bit
    assert torch.equal(got[1, 40:], ref[1, 40:])
    assert d_nomask > 1e-3
    assert torch.equal(got[0], ref[0])  # the unpadded sequence is unaffected
    loss2 = sf(input_ids=ids, attention_mask=mask, labels=labels).loss.item()
    sf.wait_for_updates()
    assert np.isfinite(out.loss.item()) and np.isfinite(loss2)
    sf.close()


def test_learning_rate_change_and_save_pretrained(dev, tmp_path):
    """update_learning_rate takes effect at the next update (two steps checked
    bit-exact against the oracle with the same learning rates), and
    save_pretrained writes the bf16 rounding of every fp32 master, then leaves
    the parameters on their masters."""
    from safetensors.torch import load_file

    from test1_amd import SlideFSDP, SlideFSDPConfig

    model = make_model()
    sf = SlideFSDP(model, SlideFSDPConfig(device=dev, lr=LR, weight_decay=WD, adam_betas=BETAS, adam_eps=EPS),
                   wait_timeout=120)
    orc = oracle.LayerAdamOracle(lr=LR, betas=BETAS, eps=EPS, weight_decay=WD)
    ref_units = []
    for ps in units_of(model):
        arrs = [p.detach().numpy().copy() for p in ps]
        ref_units.append(arrs)
        orc.add_layer(arrs)
    for k, (ids, lr) in enumerate(zip(batches(2), (LR, LR / 7))):
        if k == 1:
            sf.update_learning_rate(lr)
            orc.lr = lr
        sf.runtime.capture = {}
        ids = ids.to(dev)
        sf(input_ids=ids, labels=ids)
        sf.wait_for_updates()
        for u in range(L + 1, -1, -1):
            g = u16(sf.runtime.capture[u][0])
            parts, off = [], 0
            for a in ref_units[u]:
                parts.append(g[off:off + a.size].reshape(a.shape))
                off += a.size
            orc.step_layer(u, parts)
    for u, ps in enumerate(units_of(model)):
        for p, a in zip(ps, ref_units[u]):
            assert np.array_equal(p.detach().numpy().view(np.uint32), a.view(np.uint32)), f"unit {u}"

    # As the reference: gradients are released as each unit is offloaded, so
    # the norm is taken over none and nothing is scaled.
    assert float(sf.clip_grad_norm_(1.0)) == 0.0
    out = sf.save_pretrained(str(tmp_path / "ckpt"))
    saved = {}
    for name in os.listdir(out):
        if name.endswith(".safetensors"):
            saved.update(load_file(os.path.join(out, name)))
    named = dict(model.named_parameters())
    assert set(saved) == set(named)
    for n, t in saved.items():
        p = named[n]
        assert t.dtype == torch.bfloat16
        assert np.array_equal(u16(t).reshape(-1), oracle.cast_f32_bf16(p.detach().numpy().reshape(-1))), n
    for p in named.values():
        assert p.dtype == torch.float32 and p.device.type == "cpu"
    sf.close()
