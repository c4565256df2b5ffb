"""End-to-end loss parity at the full Llama-3.1-8B shape (32 layers, hidden
4096, vocab 128256; batch 4 x 1024, uniform random tokens), 10 training steps:
SlideFSDP with its defaults against a non-offloaded bf16 run on the same GPU
whose fp32 masters and AdamW moments live in HBM (torch AdamW, same
hyperparameters).  The bar is 1e-2 relative per step.

Each run builds and trains two 8B-parameter models (~30 s on an MI355X box,
~150 GB of host and ~190 GB of device memory).  lr 1e-5 (the bench's) runs
always; lr 1e-4 with SF_FULL_E2E=1.  At lr 1e-3 every Adam step moves each
weight by ~5 % of its spread and the two runs' trajectories part after a few
steps (their gradients differ in the last bits, as any two GEMM kernel
choices do), so that rate tests nothing.  Measured: every step within one
bf16 ulp of the loss (0.0625 at 12.5) at lr 1e-5 and 1e-4.  The file sorts
after the other GPU tests, which a failure here should not hide."""

import copy
import gc
import os
import sys
import time

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

_FULL = os.environ.get("SF_FULL_E2E") == "1"

BETAS, EPS, WD, STEPS = (0.9, 0.999), 1e-8, 0.01, 10


def _say(*a):
    print(*a, flush=True)


def _batches(w):
    g = torch.Generator().manual_seed(42)
    return [torch.randint(0, w["vocab"], (w["batch"], w["seq"]), generator=g) for _ in range(STEPS)]


def _reference_losses(model, batches, dev, vocab, LR):
    """bf16 weights on the GPU, fp32 masters and AdamW moments in HBM."""
    gm = copy.deepcopy(model).to(dev, torch.bfloat16)
    gparams = list(gm.parameters())
    masters = [p.detach().to(dev, torch.float32) for p in model.parameters()]
    opt = torch.optim.AdamW(masters, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD)
    losses = []
    for k, ids in enumerate(batches):
        ids = ids.to(dev)
        gm.zero_grad(set_to_none=True)
        logits = gm.lm_head(gm.model(input_ids=ids).last_hidden_state)
        loss = torch.nn.functional.cross_entropy(logits[..., :-1, :].reshape(-1, vocab), ids[..., 1:].reshape(-1))
        del logits
        loss.backward()
        losses.append(loss.item())
        with torch.no_grad():
            for m, p in zip(masters, gparams):
                m.grad = p.grad.float()
                p.grad = None
            opt.step()
            for m, p in zip(masters, gparams):
                p.copy_(m)          # round to nearest even, as the staging cast
                m.grad = None
        _say(f"[reference] step {k}: loss {losses[-1]:.5f}")
    del gm, masters, opt, gparams
    torch.cuda.empty_cache()
    return losses


@pytest.mark.parametrize("LR", [1e-5, pytest.param(1e-4, marks=pytest.mark.skipif(
    not _FULL, reason="second full-size run: set SF_FULL_E2E=1"))])
def test_llama31_8b_loss_parity_10_steps(dev, LR):
    sys.path.insert(0, ROOT)
    import bench
    from test1_amd import SlideFSDP, SlideFSDPConfig

    w = dict(bench.WORKLOADS["llama3-8b"])
    t0 = time.time()
    model = bench.build_model(w)
    _say(f"model built in {time.time() - t0:.0f} s")
    batches = _batches(w)
    ref = _reference_losses(model, batches, dev, w["vocab"], LR)

    cfg = SlideFSDPConfig(device=dev, lr=LR, adam_betas=BETAS, adam_eps=EPS, weight_decay=WD,
                          attention_implementation="sdpa")
    sf = SlideFSDP(model, cfg)
    got = []
    try:
        for k, ids in enumerate(batches):
            ids = ids.to(dev)
            got.append(sf(input_ids=ids, labels=ids).loss.item())
            _say(f"[SlideFSDP] step {k}: loss {got[-1]:.5f}")
        sf.wait_for_updates()
    finally:
        # the pinned masters (48 GB with the gradient slots) must go before
        # another run in this process pins its own
        sf.close()
        del sf, model
        gc.collect()
        torch.cuda.empty_cache()
    _say("reference", [round(x, 5) for x in ref])
    _say("SlideFSDP", [round(x, 5) for x in got])
    for k, (a, b) in enumerate(zip(got, ref)):
        assert abs(a - b) <= 1e-2 * abs(b), (k, a, b)
