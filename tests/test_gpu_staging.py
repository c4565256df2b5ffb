"""Parameter streaming (fp32 pinned masters -> bf16 pool units) and the unit
fences, against the oracle."""

import numpy as np
import pytest
import torch

import oracle
from test1_amd.layer_state import BF16Loader, H2DStager, LayerBufferPool
from test1_amd.optimizer import cpu_adam
from test1_amd.pinned import pinned_empty

pytestmark = pytest.mark.gpu


def bits16(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("chunk", [1 << 14, 100_003, 1 << 22, "bf16"])
def test_stream_layers_into_two_unit_pool(dev, chunk):
    """8 layers of ragged sizes streamed through a 2-unit pool, each layer's
    bf16 unit checked bit-exact before the unit is reused; a GEMM reads each
    unit on the compute stream (so a missing fence would corrupt it).
    ``chunk`` is the fp32 staging chunk, or "bf16": host-cast copies loaded
    without a device cast."""
    rng = np.random.default_rng(0)
    sizes = [int(s) for s in rng.integers(200_000, 1_500_000, 8)]
    masters = []
    for i, n in enumerate(sizes):
        m = pinned_empty(n, torch.float32)
        m.copy_(torch.randn(n, generator=torch.Generator().manual_seed(i)) * 0.02)
        masters.append(m)
    h2d, cast = torch.cuda.Stream(), torch.cuda.Stream()
    pool = LayerBufferPool(max(sizes), torch.bfloat16, dev, 2)
    if chunk == "bf16":
        st = BF16Loader(h2d)
        sources = []
        for m in masters:
            b = pinned_empty(m.numel(), torch.bfloat16)
            sources.append(cpu_adam.cast_f32_bf16(m, b))
    else:
        st = H2DStager(dev, chunk, 2, h2d, cast)
        sources = masters
    comp = torch.cuda.current_stream()
    results = []
    cur = None
    units = {}
    for i in range(len(sizes) + 1):
        if i < len(sizes):  # prefetch layer i while layer i-1 "computes"
            unit = pool.acquire(timeout=30)
            units[i] = (unit, st.load(sources[i], unit["param"], unit["ready"]))
            unit["ready"] = None
        if i >= 1:
            j = i - 1
            unit, done = units.pop(j)
            comp.wait_event(done)
            w = unit["param"][: sizes[j] // 1024 * 1024].view(-1, 1024)
            results.append((j, (w.float() @ torch.ones(1024, device=dev)).sum(), unit["param"][: sizes[j]].clone()))
            ev = torch.cuda.Event()
            ev.record(comp)
            unit["ready"] = ev
            pool.release(unit)
    torch.cuda.synchronize()
    for j, tot, snap in results:
        exp = oracle.cast_f32_bf16(masters[j].numpy())
        assert np.array_equal(bits16(snap), exp), f"layer {j}"
        w = torch.from_numpy(exp[: sizes[j] // 1024 * 1024].view(np.int16).copy()).view(torch.bfloat16)
        assert torch.allclose(tot.cpu(), w.float().view(-1, 1024).sum(), rtol=1e-4, atol=1e-3)


def test_param_streaming_llama3_8b_32_layers(dev):
    """32 Llama-3-8B decoder layers (218,112,000 fp32 parameters each, seeded
    per layer, in pinned host memory) streamed through a 2-unit bf16 pool:
    the load of layer i+1 is issued before layer i's forward, on [1, 1024,
    4096] bf16 N(0, 1) hidden states.  Every unit equals the RNE cast of its
    master (whole layer against torch's device cast, a slice against the
    oracle), and the output equals the same forward with weights cast by
    torch."""
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer, LlamaRotaryEmbedding

    cfg = LlamaConfig(hidden_size=4096, intermediate_size=14336, num_attention_heads=32, num_key_value_heads=8,
                      head_dim=128, rope_theta=500000.0, max_position_embeddings=2048)
    cfg._attn_implementation = "sdpa"
    L = 32
    with torch.device("meta"):
        layer = LlamaDecoderLayer(cfg, 0)
    names = [(n, p.shape, p.numel()) for n, p in layer.named_parameters()]
    N = sum(k for _, _, k in names)
    assert N == 218_112_000
    layer = layer.to_empty(device=dev).to(torch.bfloat16)
    rope = LlamaRotaryEmbedding(config=cfg).to(dev)

    masters = []
    for i in range(L):
        g = torch.Generator(device=dev).manual_seed(1000 + i)
        m = pinned_empty(N, torch.float32)
        m.copy_(torch.randn(N, generator=g, device=dev) * 0.02)
        masters.append(m)
    h0 = torch.randn(1, 1024, 4096, generator=torch.Generator(device=dev).manual_seed(7), device=dev).bfloat16()
    pos = rope(h0, torch.arange(1024, device=dev).unsqueeze(0))

    def bind(flat):
        off = 0
        for (name, shape, k), p in zip(names, layer.parameters()):
            p.data = flat[off:off + k].view(shape)
            off += k

    def fwd(h):
        with torch.no_grad():
            out = layer(h, attention_mask=None, position_embeddings=pos)
        return out[0] if isinstance(out, tuple) else out

    h2d, cast = torch.cuda.Stream(), torch.cuda.Stream()
    pool = LayerBufferPool(N, torch.bfloat16, dev, 2)
    st = H2DStager(dev, N, 2, h2d, cast)
    comp = torch.cuda.current_stream()
    mismatched = []
    units = {}
    h = h0
    nxt = pool.acquire(timeout=60)
    units[0] = (nxt, st.load(masters[0], nxt["param"], nxt["ready"]))
    for i in range(L):
        if i + 1 < L:  # prefetch layer i+1 before layer i's forward
            u = pool.acquire(timeout=60)
            units[i + 1] = (u, st.load(masters[i + 1], u["param"], u["ready"]))
        unit, done = units.pop(i)
        comp.wait_event(done)
        ref = masters[i].to(dev, non_blocking=False).to(torch.bfloat16)
        if not torch.equal(unit["param"][:N].view(torch.int16), ref.view(torch.int16)):
            mismatched.append(i)
        if i in (0, L - 1):
            sl = slice(N - 4_000_000, N)
            assert np.array_equal(bits16(unit["param"][sl]), oracle.cast_f32_bf16(masters[i].numpy()[sl])), i
        bind(unit["param"])
        h = fwd(h)
        ev = torch.cuda.Event()
        ev.record(comp)
        unit["ready"] = ev
        pool.release(unit)
    assert not mismatched, f"units differ from the cast of their master: {mismatched}"
    # reference: the same 32 forwards with weights cast by torch
    r = h0
    for i in range(L):
        bind(masters[i].to(dev).to(torch.bfloat16))
        r = fwd(r)
    torch.cuda.synchronize()
    assert torch.equal(h.view(torch.int16), r.view(torch.int16))


def test_stager_slots_are_taken_on_the_stream_that_copies_into_them(dev):
    """Whole-unit slots of units staged after their update are allocated on
    the H2D stream, which copies into them.  Taken on the compute stream, a
    slot could be memory the backward has just freed while its kernels on it
    are still queued, and the copy, on another stream, would overwrite it
    under them (step-1 gradients of the Qwen2.5-14B-shaped step differed from
    a non-offloaded run's from the middle of the backward down).  The slot's
    cast is the oracle's."""
    h2d, cast = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    stager = H2DStager(dev, 1 << 20, 3, h2d, cast, slot_cap_bytes=1 << 30)
    # a block freed on the current stream that the slot would fit in
    junk = torch.empty(1 << 23, dtype=torch.float32, device=dev)
    del junk
    n = 3_000_001
    g = torch.Generator().manual_seed(11)
    host = pinned_empty(n, torch.float32)
    host.copy_(torch.randn(n, generator=g) * 0.02)
    p = stager.copy_for_later(host, None)
    assert p is not None
    addr = p.slot.data_ptr()
    seg = [sg for sg in torch.cuda.memory_snapshot()
           if sg["address"] <= addr < sg["address"] + sg["total_size"]]
    assert len(seg) == 1 and seg[0]["stream"] == h2d.cuda_stream, \
        "slot not allocated on the stream that copies into it"
    dst = torch.empty(n, dtype=torch.bfloat16, device=dev)
    stager.cast_pending(p, dst, torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert np.array_equal(bits16(dst), oracle.cast_f32_bf16(host.numpy()))


def test_noop_sync_copies_are_bit_exact(dev):
    """The one-GPU transfer strategy (reference distributed_sync.py:324-354):
    ``gather_params_to_gpu`` copies a pinned bf16 layer into the device buffer
    and ``reduce_gradients_to_master`` copies device grads into a pinned host
    buffer, returning once they are there; both bit for bit, for an odd size
    into larger buffers (the rest untouched)."""
    from test1_amd import SlideFSDPConfig
    from test1_amd.distributed_sync import create_distributed_sync

    sync = create_distributed_sync(SlideFSDPConfig(device=dev))
    g = torch.Generator().manual_seed(5)
    n = 3_000_017
    host = pinned_empty(n, torch.bfloat16)
    host.copy_(torch.randn(n, generator=g).bfloat16())
    gpu = torch.full((n + 64,), 7.0, dtype=torch.bfloat16, device=dev)
    sync.gather_params_to_gpu(host, gpu)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(gpu[:n]), bits16(host))
    assert bool((gpu[n:] == 7.0).all())

    grads = (torch.randn(n, generator=g) * 1e-3).bfloat16().to(dev)
    back = pinned_empty(n + 64, torch.bfloat16)
    back.fill_(3.0)
    sync.reduce_gradients_to_master(grads, back)   # synchronises before returning
    assert np.array_equal(bits16(back[:n]), bits16(grads))
    assert bool((back[n:] == 3.0).all())
