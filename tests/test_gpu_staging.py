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
