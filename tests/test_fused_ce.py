"""Chunked linear + cross entropy (the output unit's fused variant) against
plain PyTorch cross entropy on the same bf16 GEMM outputs, in fp32."""

import pytest
import torch

from test1_amd.fused_ce import chunked_linear_cross_entropy


def reference(h, w, y, ignore_index=-100):
    """fp32 reference on the bf16 GEMM's output, with autograd."""
    h32 = h.detach().float().requires_grad_(True)
    w32 = w.detach().float().requires_grad_(True)
    logits = h32 @ w32.t()
    loss = torch.nn.functional.cross_entropy(logits, y, ignore_index=ignore_index)
    loss.backward()
    return loss.detach(), h32.grad, w32.grad


def rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-30)).item()


@pytest.mark.parametrize("chunk", [1, 7, 64, 0])
def test_matches_fp32_reference(chunk):
    g = torch.Generator().manual_seed(5)
    N, H, V = 150, 64, 1000
    h = (torch.randn(N, H, generator=g)).bfloat16().requires_grad_(True)
    w = (torch.randn(V, H, generator=g) * 0.05).bfloat16().requires_grad_(True)
    y = torch.randint(0, V, (N,), generator=g)
    y[::11] = -100  # ignored rows
    loss = chunked_linear_cross_entropy(h, w, y, chunk_rows=chunk)
    (2.0 * loss).backward()  # the backward scales by the incoming gradient
    ref_loss, ref_gh, ref_gw = reference(h, w, y)
    assert abs(loss.item() - ref_loss.item()) <= 1e-3 * abs(ref_loss.item())
    assert rel(h.grad, 2.0 * ref_gh) < 1e-2
    assert rel(w.grad, 2.0 * ref_gw) < 1e-2
    assert h.grad.dtype == torch.bfloat16 and w.grad.dtype == torch.bfloat16
    # ignored rows get no gradient
    assert h.grad[::11].abs().max().item() == 0.0


def test_all_rows_ignored_gives_nan_like_cross_entropy():
    h = torch.randn(4, 16).bfloat16()
    w = torch.randn(32, 16).bfloat16()
    y = torch.full((4,), -100)
    assert torch.isnan(chunked_linear_cross_entropy(h, w, y))
    assert torch.isnan(torch.nn.functional.cross_entropy(h.float() @ w.float().t(), y))


def test_shape_errors():
    with pytest.raises(ValueError):
        chunked_linear_cross_entropy(torch.zeros(4, 8), torch.zeros(10, 9), torch.zeros(4, dtype=torch.long))
    with pytest.raises(ValueError):
        chunked_linear_cross_entropy(torch.zeros(4, 8), torch.zeros(10, 8), torch.zeros(5, dtype=torch.long))
