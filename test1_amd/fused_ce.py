"""Chunked linear + cross entropy for the output unit: the loss of
``cross_entropy(hidden @ weight.T, labels)`` without materialising the
[N, V] logits.

The reference's output unit uses a fused linear-cross-entropy kernel when one
is installed (slide_fsdp.py:57-63, 85-97: ``LigerFusedLinearCrossEntropyLoss``,
mean reduction, no logits returned) and full logits + ``nn.CrossEntropyLoss``
otherwise.  This is the fused variant built from hipBLASLt GEMMs: rows are
processed in chunks of ``chunk_rows``; for each chunk the logits are formed in
fp32, the chunk's loss terms are summed, and since the step's backward follows
at once, the gradients with respect to the hidden rows and the weight are
formed right away from ``softmax - onehot`` (as the fused kernel does) and
only scaled in the backward.  Peak extra memory is one chunk of fp32 logits
plus an fp32 weight-gradient accumulator, instead of the [N, V] logits in bf16
and fp32 and their gradient.

Numerics: logsumexp, softmax and the loss are fp32; the logits are the bf16
GEMM's output widened, as ``nn.CrossEntropyLoss`` on bf16 logits sees them;
the gradient of the logits is rounded to bf16 for the two gradient GEMMs and
the weight gradient is accumulated over chunks in fp32.  Rows whose label is
``ignore_index`` contribute nothing; the mean is over the other rows (NaN if
there are none, as ``nn.CrossEntropyLoss``).
"""

from __future__ import annotations

import torch


class ChunkedLinearCrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor, ignore_index: int,
                chunk_rows: int) -> torch.Tensor:
        if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
            raise ValueError("chunked linear cross entropy: hidden [N, H] and weight [V, H] expected")
        if labels.shape != hidden.shape[:1]:
            raise ValueError("chunked linear cross entropy: one label per hidden row expected")
        n, h = hidden.shape
        v = weight.shape[0]
        dev = hidden.device
        grad_hidden = torch.empty_like(hidden)
        grad_weight = torch.zeros((v, h), dtype=torch.float32, device=dev)
        loss_sum = torch.zeros((), dtype=torch.float32, device=dev)
        valid_all = labels != ignore_index
        n_valid = valid_all.sum().to(torch.float32)
        wt = weight.t()
        for s in range(0, n, max(1, int(chunk_rows))):
            e = min(n, s + int(chunk_rows))
            hc = hidden[s:e]
            yc = labels[s:e]
            valid = valid_all[s:e]
            ysafe = torch.where(valid, yc, torch.zeros_like(yc))
            logits = torch.mm(hc, wt).float()                       # [C, V], widened bf16 GEMM output
            lse = torch.logsumexp(logits, dim=1)
            target = logits.gather(1, ysafe.unsqueeze(1)).squeeze(1)
            loss_sum += torch.where(valid, lse - target, torch.zeros_like(lse)).sum()
            logits.sub_(lse.unsqueeze(1)).exp_()                    # softmax, in place
            rows = torch.arange(e - s, device=dev)
            logits[rows, ysafe] -= 1.0                              # - onehot
            logits.mul_(valid.unsqueeze(1).to(logits.dtype))        # ignored rows: no gradient
            g = logits.to(hidden.dtype)
            del logits
            grad_hidden[s:e] = torch.mm(g, weight)
            grad_weight.add_(torch.mm(g.t(), hc))
        ctx.save_for_backward(grad_hidden, grad_weight, n_valid)
        ctx.weight_dtype = weight.dtype
        return loss_sum / n_valid

    @staticmethod
    def backward(ctx, grad_loss: torch.Tensor):
        grad_hidden, grad_weight, n_valid = ctx.saved_tensors
        scale = (grad_loss.to(torch.float32) / n_valid)
        gh = (grad_hidden.to(torch.float32) * scale).to(grad_hidden.dtype)
        gw = (grad_weight * scale).to(ctx.weight_dtype)
        return gh, gw, None, None, None


def chunked_linear_cross_entropy(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor,
                                 ignore_index: int = -100, chunk_rows: int = 0) -> torch.Tensor:
    """Mean cross entropy of ``hidden @ weight.T`` against ``labels``.
    ``chunk_rows`` <= 0 picks chunks of ~256 MiB of fp32 logits."""
    if chunk_rows <= 0:
        chunk_rows = max(1, (256 << 20) // (4 * weight.shape[0]))
    return ChunkedLinearCrossEntropy.apply(hidden, weight, labels, int(ignore_index), int(chunk_rows))
