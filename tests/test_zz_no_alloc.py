"""The staging entry point that allocates nothing (sf_stage_f32_bf16_noalloc,
its pieces through the library's static device scratch buffer) against the
one with a caller workspace (sf_stage_f32_bf16), through the C ABI: two
calls in a row, the second with a smaller input, bit for bit, and both equal
to the oracle's cast; once the runtime's pools are warm, repeating the two
calls leaves the free device memory unchanged;
a piece larger than the scratch is refused with its own status before
anything is enqueued."""

import numpy as np
import pytest
import torch

import oracle
from test1_amd import _native
from test1_amd.pinned import pinned_empty

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def test_noalloc_stage_matches_workspace_stage(dev):
    lib = _native.hip()
    scratch = _native.SF_STAGE_SCRATCH_ELEMS
    # (elements, piece): three pieces of the whole scratch with a ragged last
    # one, then a smaller input in pieces of an odd size
    cases = [(2 * scratch + 100_003, 0), (1_000_003, 4099)]
    g = torch.Generator().manual_seed(11)
    bufs = []
    for n, chunk in cases:
        x = pinned_empty(n, torch.float32)
        x.copy_(torch.randn(n, generator=g) * 0.02)
        x[:3] = torch.tensor([float("nan"), float("-inf"), -0.0])
        a = torch.full((n + 8,), 7.0, dtype=torch.bfloat16, device=dev)
        b = torch.full((n + 8,), 7.0, dtype=torch.bfloat16, device=dev)
        work = torch.empty(chunk or scratch, dtype=torch.float32, device=dev)
        bufs.append((x, a, b, work, chunk))
    st = torch.cuda.current_stream()

    def two_calls():
        for k, (x, a, b, work, chunk) in enumerate(bufs):
            print(f"call {k}: {x.numel()} elements, pieces of {chunk or scratch}", flush=True)
            assert lib.sf_stage_f32_bf16_noalloc(x.data_ptr(), a.data_ptr(), x.numel(), chunk,
                                                 st.cuda_stream) == 0
        torch.cuda.synchronize()

    # The first rounds load the library's code object on this device (the
    # scratch array comes with it), create its ordering event, and let the
    # HIP runtime size its own launch, copy and event pools for ~250 launches
    # and the event waits between calls (in a fresh process its pools still
    # grew by 2 MiB in the second round); two further identical rounds, with
    # nothing else in between, leave the free device memory unchanged.
    two_calls()
    two_calls()
    free_before = torch.cuda.mem_get_info(dev)[0]
    two_calls()
    two_calls()
    free_after = torch.cuda.mem_get_info(dev)[0]
    # the same stagings through the workspace entry point
    for x, a, b, work, chunk in bufs:
        assert lib.sf_stage_f32_bf16(x.data_ptr(), b.data_ptr(), x.numel(), work.data_ptr(), work.numel(),
                                     st.cuda_stream) == 0
    torch.cuda.synchronize()
    for k, (x, a, b, work, chunk) in enumerate(bufs):
        n = x.numel()
        assert np.array_equal(_bits(a), _bits(b)), f"call {k}: differs from the workspace entry point"
        assert np.array_equal(_bits(a[:n]), oracle.cast_f32_bf16(x.numpy())), f"call {k}: differs from the oracle"
        assert bool((a[n:] == 7.0).all()), f"call {k}: wrote past the end"
    assert free_after == free_before, (free_before, free_after)

    x, a = bufs[1][0], bufs[1][1]
    rc = lib.sf_stage_f32_bf16_noalloc(x.data_ptr(), a.data_ptr(), x.numel(), scratch + 8, st.cuda_stream)
    assert rc == _native.SF_ETOOBIG and b"scratch" in lib.sf_error_string(rc)


def test_noalloc_calls_on_two_streams_are_ordered(dev):
    """Calls on two streams, issued back to back with nothing between them on
    the host: the second call's copies into the shared scratch buffer wait
    for the first call's last cast (the library's ordering event), so both
    outputs are the oracle's cast.  Without that ordering the second
    stream's copies would overwrite pieces the first stream had not cast."""
    lib = _native.hip()
    scratch = _native.SF_STAGE_SCRATCH_ELEMS
    g = torch.Generator().manual_seed(12)
    sizes = (3 * scratch + 17, 2 * scratch + 5)
    xs, outs = [], []
    for n in sizes:
        x = pinned_empty(n, torch.float32)
        x.copy_(torch.randn(n, generator=g) * 0.02)
        xs.append(x)
        outs.append(torch.full((n + 8,), 7.0, dtype=torch.bfloat16, device=dev))
    streams = [torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)]
    torch.cuda.synchronize()
    for rnd in range(2):
        for k, (x, out, st) in enumerate(zip(xs, outs, streams)):
            print(f"round {rnd} call {k}: {x.numel()} elements on stream {k}", flush=True)
            assert lib.sf_stage_f32_bf16_noalloc(x.data_ptr(), out.data_ptr(), x.numel(), 0, st.cuda_stream) == 0
        torch.cuda.synchronize()
        for k, (x, out) in enumerate(zip(xs, outs)):
            n = x.numel()
            assert np.array_equal(_bits(out[:n]), oracle.cast_f32_bf16(x.numpy())), f"round {rnd} call {k}"
            assert bool((out[n:] == 7.0).all()), f"round {rnd} call {k}: wrote past the end"
            out.fill_(7.0)
        torch.cuda.synchronize()
