"""Helpers of the full-size end-to-end GPU tests (Llama-3.1-8B and
Qwen2.5-14B shapes): a non-offloaded bf16 copy of the model on the GPU, the
oracle AdamW driven over a few captured units, and the checks of captured
gradients, updates and staged weights.

The oracle keeps real arrays only for the captured units; every other unit is
stepped with one-element stand-ins per parameter.  The reference's AdamW
scalars (beta^t, bias corrections) depend on the sequence of calls across all
units and parameters (optimizer/layer_adam/csrc/cpu_adam.h:57-89), not on the
data, so the stand-ins reproduce them exactly while the captured units get
the full arithmetic."""

import time

import numpy as np
import torch

import oracle


def say(*a):
    print(*a, flush=True)


def u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def same_bits(a, b) -> bool:
    """Two 16-bit tensors (any device, any shape of equal numel) hold the same bits."""
    return np.array_equal(u16(a).reshape(-1), u16(b).reshape(-1))


def grad_word_sums(grads):
    """Per gradient, the sum of its 16-bit words (None for a missing one):
    the checksum the runtime records as ``("grad_sums", unit)``."""
    return [None if g is None else int(g.detach().view(torch.int16).sum(dtype=torch.int64)) for g in grads]


def check_step1_against_reference(cap, ref_grads, units, ref_sums=None):
    """SlideFSDP's step-1 device gradients of ``units`` equal the
    non-offloaded run's, bit for bit, and (with ``ref_sums``, per unit the
    reference's ``grad_word_sums``) every other unit's gradients have the
    reference's checksums.  A failure lists every unit that differs, with
    the fraction of its elements that still match or the parameters whose
    checksums differ, so that the highest unit listed is where the
    backward first went apart."""
    bad = []
    if ref_sums is not None:
        for u in sorted(ref_sums, reverse=True):
            got = cap.get(("grad_sums", u))
            if got is None:
                continue      # the row-sparse embedding records none
            got = [None if t is None else int(t) for t in got]
            diff = [j for j, (a, b) in enumerate(zip(got, ref_sums[u])) if a != b]
            if len(got) != len(ref_sums[u]) or diff:
                bad.append(f"unit {u} checksums of parameters {diff}")
    for u in units:
        got, exp = cap[("device_grads", u)], ref_grads[u]
        assert len(got) == len(exp), f"unit {u}: {len(got)} gradients, expected {len(exp)}"
        for j, (a, b) in enumerate(zip(got, exp)):
            assert a.numel() == b.numel(), f"unit {u} parameter {j}: {a.numel()} elements, expected {b.numel()}"
            if not same_bits(a, b):
                frac = float(np.mean(u16(a).reshape(-1) == u16(b).reshape(-1)))
                bad.append(f"unit {u} parameter {j} ({frac:.4f} of elements equal)")
    assert not bad, "step-1 gradients differ from the non-offloaded run's: " + "; ".join(bad)


def unit_params(model):
    """Parameters of each SlideFSDP unit in its flat order: [embedding] +
    decoder layers + [final norm, lm_head]."""
    m = model.model
    return ([[m.embed_tokens.weight]] + [list(l.parameters()) for l in m.layers]
            + [[m.norm.weight, model.lm_head.weight]])


def gpu_bf16_copy(model, dev, dtype=torch.bfloat16):
    """The model's architecture on the GPU in ``dtype`` (bf16 or fp16), each
    weight the RNE cast of its fp32 weight (cast on the GPU parameter by
    parameter, so no second host copy is made); rotary frequencies rebuilt in
    fp32 as in the host model."""
    cfg = model.config
    with torch.device("meta"):
        gm = type(model)(cfg)
    gm = gm.to(dtype).to_empty(device=dev)
    gm.model.rotary_emb = type(model.model.rotary_emb)(config=cfg).to(dev)
    with torch.no_grad():
        for (n, gp), (n2, p) in zip(gm.named_parameters(), model.named_parameters()):
            assert n == n2, (n, n2)
            gp.copy_(p.detach().to(dev))
    return gm


def reference_step(gm, ids, vocab, units, layer_inputs=None, grad_sums=None):
    """One forward/backward of the non-offloaded model with transformers' own
    decoder forward (causal mask, rotary) and per-layer recompute; returns the
    loss and the bf16 gradients of ``units`` (host).  A list passed as
    ``layer_inputs`` receives each decoder layer's input hidden states (host);
    a dict passed as ``grad_sums`` receives every unit's ``grad_word_sums``."""
    gm.gradient_checkpointing_enable(gradient_checkpointing_kwargs={"use_reentrant": False})
    gm.train()
    gm.zero_grad(set_to_none=True)
    out = gm.model(input_ids=ids, use_cache=False, output_hidden_states=layer_inputs is not None)
    if layer_inputs is not None:
        n_dec = len(gm.model.layers)
        layer_inputs.extend(h.detach().cpu() for h in out.hidden_states[:n_dec])
    hidden = out.last_hidden_state
    del out
    logits = gm.lm_head(hidden)
    del hidden
    loss = torch.nn.functional.cross_entropy(logits[..., :-1, :].reshape(-1, vocab), ids[..., 1:].reshape(-1))
    del logits
    loss.backward()
    ups = unit_params(gm)
    grads = {u: [p.grad.detach().cpu() for p in ups[u]] for u in units}
    if grad_sums is not None:
        grad_sums.update({u: grad_word_sums([p.grad for p in ps]) for u, ps in enumerate(ups)})
    return loss.item(), grads


def check_served_checkpoints(served, layer_inputs):
    """Each decoder layer's recompute was given its input hidden states of
    the non-offloaded forward, bit for bit (``served`` is the runtime's
    ``capture_served`` after a step: the first tensor each layer's recompute
    received, copied on its stream after the prefetch wait).  Returns the
    layers checked."""
    checked, bad = [], []
    for i, h in enumerate(layer_inputs):
        got = served.get((i, 0))
        assert got is not None, f"decoder {i}: nothing served to its recompute"
        assert tuple(got.shape) == tuple(h.shape), f"decoder {i}: served {tuple(got.shape)}"
        if not same_bits(got, h):
            bad.append(i)
        checked.append(i)
    if bad:
        i = bad[0]
        got, exp = u16(served[(i, 0)]).reshape(-1), u16(layer_inputs[i]).reshape(-1)
        diff = np.flatnonzero(got != exp)
        stale = [j for j, h in enumerate(layer_inputs)
                 if j != i and np.array_equal(got[diff], u16(h).reshape(-1)[diff])]
        raise AssertionError(
            f"the recompute of decoders {bad} was given other inputs than the non-offloaded forward's; "
            f"decoder {i}: {diff.size} of {got.size} elements, flat [{diff[0]}, {diff[-1]}], "
            f"zero there: {bool((got[diff] == 0).all())}, equal there to the inputs of decoders {stale}")
    return checked


def unit_weight_sums(gm):
    """Per unit, the sum of the 16-bit words of its bf16 weights (the
    checksum the runtime records with ``capture_served``)."""
    return [int(sum(int(p.detach().view(torch.int16).sum(dtype=torch.int64)) for p in ps))
            for ps in unit_params(gm)]


def master_weight_sums(sf):
    """Per unit, the checksum of the RNE bf16 cast of SlideFSDP's current
    fp32 master (torch's CPU cast, the oracle's rounding): the weights a
    step computes with, taken before the step (after the previous step's
    updates)."""
    sf.wait_for_updates()
    out = []
    for st in sf.layer_states:
        m = st._cpu_params_flat
        out.append(int(m.to(torch.bfloat16).view(torch.int16).sum(dtype=torch.int64)))
    return out


def check_backward_weights(served, sums, units):
    """Each unit's device weights at the start and at the end of its
    backward have the checksum of its bf16 weights in the non-offloaded run
    (step 1: no update has reached them yet).  Returns the units checked."""
    bad = []
    for u in units:
        for what in ("weights_start", "weights_end"):
            got = served.get((what, u))
            assert got is not None, f"unit {u}: no {what} checksum"
            if int(got) != sums[u]:
                bad.append(f"unit {u} {what}")
    assert not bad, "device weights read by the backward differ from the forward's: " + ", ".join(bad)
    return list(units)


def _bits(t):
    return t.detach().contiguous().view(-1).view(torch.uint8)


def check_served_side_inputs(served, n_dec):
    """The checkpoint tensors after the hidden states (rotary tables, mask)
    that each decoder's recompute was given equal those of the last decoder,
    which keeps the forward's own device tensors.  Returns their number."""
    last, k = n_dec - 1, 1
    while (last, k) in served:
        ref = _bits(served[(last, k)])
        bad = [i for i in range(n_dec) if not torch.equal(_bits(served[(i, k)]), ref)]
        assert not bad, f"checkpoint tensor {k} given to the recompute of decoders {bad} differs from the forward's"
        k += 1
    return k - 1


def check_checkpoint_slots(sf, layer_inputs):
    """After a step, the pinned checkpoint slot of every offloaded decoder
    layer holds that layer's input hidden states bit for bit (the forward is
    the non-offloaded run's, so its inputs are ``layer_inputs``).  The last
    decoder keeps its checkpoint on the device, as does a layer whose slot
    could not be pinned.  Returns the layers checked."""
    from test1_amd.sliding_checkpoint import KeptOnDevice

    checked, bad = [], []
    for i, h in enumerate(layer_inputs[:-1]):
        slot = sf.layer_tensors[i][0]
        if isinstance(slot, KeptOnDevice):
            continue
        assert slot.shape == h.shape, f"decoder {i}: checkpoint slot of shape {tuple(slot.shape)}"
        if not same_bits(slot, h):
            bad.append(i)
        checked.append(i)
    if bad:
        i = bad[0]
        got, exp = u16(sf.layer_tensors[i][0]).reshape(-1), u16(layer_inputs[i]).reshape(-1)
        diff = np.flatnonzero(got != exp)
        stale = [j for j, h in enumerate(layer_inputs)
                 if j != i and np.array_equal(got[diff], u16(h).reshape(-1)[diff])]
        raise AssertionError(
            f"checkpoint slots of decoders {bad} differ from the layers' inputs in the non-offloaded forward; "
            f"decoder {i}: {diff.size} of {got.size} elements, flat [{diff[0]}, {diff[-1]}], "
            f"zero there: {bool((got[diff] == 0).all())}, equal there to the inputs of decoders {stale}")
    return checked


class CapturedOracle:
    """LayerAdamOracle over every unit: real fp32 arrays for ``units``,
    one-element stand-ins for the others (same calls, so the same scalars)."""

    def __init__(self, model, units, lr, betas, eps, wd):
        self.units = set(units)
        self.orc = oracle.LayerAdamOracle(lr=lr, betas=betas, eps=eps, weight_decay=wd)
        self.arrays = {}
        self.nparams = []
        for u, ps in enumerate(unit_params(model)):
            if u in self.units:
                arrs = [p.detach().numpy().copy() for p in ps]
                self.arrays[u] = arrs
            else:
                arrs = [np.zeros(1, np.float32) for _ in ps]
            self.nparams.append(len(ps))
            self.orc.add_layer(arrs)

    def flat(self, u):
        return np.concatenate([a.reshape(-1) for a in self.arrays[u]])

    def step(self, cap):
        """Check and apply one step: for each captured unit, the runtime's
        fp32 master before its update must equal the oracle's, and its packed
        host gradients feed the oracle update.  Units are stepped last first,
        the order the reference runs updates in."""
        n_units = len(self.nparams)
        for u in range(n_units - 1, -1, -1):
            if u in self.units:
                grads, master_before = cap[u]
                before = self.flat(u)
                assert np.array_equal(master_before.numpy().view(np.uint32), before.view(np.uint32)), \
                    f"unit {u}: master before the update differs from the oracle's"
                g = u16(grads)
                parts, off = [], 0
                for a in self.arrays[u]:
                    parts.append(g[off:off + a.size].reshape(a.shape))
                    off += a.size
                assert off == g.size, f"unit {u}: {g.size} packed gradient elements, expected {off}"
                self.orc.step_layer(u, parts)
            else:
                self.orc.step_layer(u, [np.zeros(1, np.float32)] * self.nparams[u])


def check_packed_grads(cap, units):
    """The packed host gradients equal the device gradients, bit for bit, in
    layout order."""
    for u in units:
        exp = oracle.pack_b16([u16(g) for g in cap[("device_grads", u)]])
        assert np.array_equal(u16(cap[u][0]), exp), f"unit {u}: packed grads differ from the device grads"


def check_masters(sf, orc, units):
    """The runtime's fp32 masters after the step equal the oracle's."""
    for u in units:
        got = sf.layer_states[u]._cpu_params_flat.numpy()
        assert np.array_equal(got.view(np.uint32), orc.flat(u).view(np.uint32)), f"unit {u}: master after update"


def check_moments(sf, orc, units):
    for u in units:
        m, v = sf.layer_optimizer.layer_states(u)
        om, ov = orc.orc.moments(u)
        assert np.array_equal(m.numpy().view(np.uint32), om.view(np.uint32)), f"unit {u} exp_avg"
        assert np.array_equal(v.numpy().view(np.uint32), ov.view(np.uint32)), f"unit {u} exp_avg_sq"


def check_staged(sf, orc, units, ids):
    """A forward without labels stages every unit with its current master;
    each captured unit that keeps a device buffer of its own stays bound
    after it: its bf16 weights must be the oracle's cast of the oracle's
    master.  Returns the units checked."""
    with torch.no_grad():
        sf(input_ids=ids)
    torch.cuda.synchronize()
    checked = []
    for u in units:
        st = sf.layer_states[u]
        unit = st._current_gpu_cache
        if unit is None:
            continue
        got = u16(unit["param"][:st.total_size])
        assert np.array_equal(got, oracle.cast_f32_bf16(orc.flat(u))), f"unit {u}: staged bf16 weights"
        checked.append(u)
    return checked


def timed(what, fn, *a, **k):
    t = time.time()
    r = fn(*a, **k)
    say(f"{what}: {time.time() - t:.1f} s")
    return r
