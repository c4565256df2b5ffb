"""End-to-end parity at the full Llama-3.1-8B shape (32 layers, hidden 4096,
vocab 128256; batch 4 x 1024, uniform random tokens), 10 training steps at
lr 1e-4: SlideFSDP with its defaults against a non-offloaded bf16 run on the
same GPU whose fp32 masters and AdamW moments live in HBM (torch AdamW, same
hyperparameters).  Both start from the same bf16 weights and fp32 rotary
frequencies (the reference model is built parameter by parameter on the GPU;
``Module.to(bfloat16)`` would also round the rotary ``inv_freq`` buffer).

* Step 1: the loss and the gradients of the first decoder and the output
  unit equal the non-offloaded run's bit for bit (same kernels on the same
  bits: offload, recompute from the offloaded checkpoints and the staged
  weights change nothing), and every offloaded decoder's pinned checkpoint
  slot holds that layer's input in the non-offloaded forward.
* Loss: every step within 1e-2 relative (the returned loss, bf16 as the
  reference's).  The loss also recomputed in fp32 from the returned bf16
  logits, where the ten steps' drop is visible (a bf16 loss near 12.5 has a
  0.0625 ulp): SlideFSDP's drop from step 1 must track the reference's (the
  two AdamW implementations differ in operation order only).
* Steps 1-3: those units' packed host gradients equal their device gradients
  and every update is the oracle AdamW's, bit for bit (reference
  layer_state.py:410-437); a forward after step 3 computes with the oracle's
  bf16 cast of the updated masters.  A run whose updates were skipped or
  corrupted fails here.

At lr 1e-3 every Adam step moves each weight by ~5 % of its spread and the
two runs' trajectories part after a few steps (their AdamW steps differ in
the last bits), so that rate tests nothing.  Each run builds and trains two
8B-parameter models (~150 GB of host and ~190 GB of device memory).  The file
sorts after the other GPU tests, which a failure here should not hide."""

import gc
import os
import sys
import time

import pytest
import torch

from fullsize import (CapturedOracle, check_backward_weights, check_checkpoint_slots, check_served_checkpoints,
                      check_served_side_inputs, grad_word_sums, unit_weight_sums, check_masters, check_moments, check_packed_grads,
                      check_staged, check_step1_against_reference, gpu_bf16_copy, say, timed, unit_params)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

LR, BETAS, EPS, WD, STEPS, CHECKED_STEPS = 1e-4, (0.9, 0.999), 1e-8, 0.01, 10, 3


def _batches(w):
    g = torch.Generator().manual_seed(42)
    return [torch.randint(0, w["vocab"], (w["batch"], w["seq"]), generator=g) for _ in range(STEPS + 1)]


def _fp32_loss(logits, ids, vocab):
    return torch.nn.functional.cross_entropy(logits[..., :-1, :].float().reshape(-1, vocab),
                                             ids[..., 1:].reshape(-1)).item()


def _reference(model, batches, dev, vocab, units):
    """bf16 weights on the GPU, fp32 masters and AdamW moments in HBM.
    Returns the bf16 losses, the fp32 losses, step 1's gradients of
    ``units``, step 1's decoder layer inputs (host), the weight checksums
    and step 1's gradient checksums of every unit."""
    gm = gpu_bf16_copy(model, dev)
    sums = unit_weight_sums(gm)
    gparams = list(gm.parameters())
    masters = [p.detach().to(dev, torch.float32) for p in model.parameters()]
    opt = torch.optim.AdamW(masters, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD)
    losses, losses32, grads, layer_inputs, grad_sums = [], [], None, None, None
    for k, ids in enumerate(batches[:STEPS]):
        ids = ids.to(dev)
        gm.zero_grad(set_to_none=True)
        out = gm.model(input_ids=ids, output_hidden_states=k == 0)
        if k == 0:
            layer_inputs = [h.detach().cpu() for h in out.hidden_states[:len(gm.model.layers)]]
        logits = gm.lm_head(out.last_hidden_state)
        del out
        loss = torch.nn.functional.cross_entropy(logits[..., :-1, :].reshape(-1, vocab), ids[..., 1:].reshape(-1))
        losses32.append(_fp32_loss(logits.detach(), ids, vocab))
        del logits
        loss.backward()
        losses.append(loss.item())
        if k == 0:
            ups = unit_params(gm)
            grads = {u: [p.grad.detach().cpu() for p in ups[u]] for u in units}
            grad_sums = {u: grad_word_sums([p.grad for p in ps]) for u, ps in enumerate(ups)}
        with torch.no_grad():
            for m, p in zip(masters, gparams):
                m.grad = p.grad.float()
                p.grad = None
            opt.step()
            for m, p in zip(masters, gparams):
                p.copy_(m)          # round to nearest even, as the staging cast
                m.grad = None
        say(f"[reference] step {k}: loss {losses[-1]:.5f} (fp32 {losses32[-1]:.6f})")
    del gm, masters, opt, gparams
    torch.cuda.empty_cache()
    return losses, losses32, grads, layer_inputs, sums, grad_sums


def test_llama31_8b_parity_10_steps(dev):
    sys.path.insert(0, ROOT)
    import bench
    from test1_amd import SlideFSDP, SlideFSDPConfig

    w = dict(bench.WORKLOADS["llama3-8b"])
    L = w["layers"]
    units = (1, L + 1)
    model = timed("model built", bench.build_model, w)
    batches = _batches(w)
    ref, ref32, ref_grads, layer_inputs, sums, ref_sums = timed("reference run", _reference, model, batches, dev,
                                                                w["vocab"], units)

    orc = CapturedOracle(model, units, LR, BETAS, EPS, WD)
    cfg = SlideFSDPConfig(device=dev, lr=LR, adam_betas=BETAS, adam_eps=EPS, weight_decay=WD,
                          attention_implementation="sdpa")
    sf = SlideFSDP(model, cfg, wait_timeout=600)
    sf.runtime.capture_units = set(units)
    got, got32 = [], []
    try:
        for k, ids in enumerate(batches[:STEPS]):
            ids = ids.to(dev)
            checked = k < CHECKED_STEPS
            sf.runtime.capture = {} if checked else None
            sf.runtime.capture_served = {} if k == 0 else None
            t = time.time()
            out = sf(input_ids=ids, labels=ids)
            got.append(out.loss.item())
            got32.append(_fp32_loss(out.logits.detach(), ids, w["vocab"]))
            del out
            sf.wait_for_updates()
            say(f"[SlideFSDP] step {k}: loss {got[-1]:.5f} (fp32 {got32[-1]:.6f}) {time.time() - t:.1f} s")
            if not checked:
                continue
            cap = sf.runtime.capture
            if k == 0:
                assert got[0] == ref[0] and got32[0] == ref32[0], (got[0], ref[0], got32[0], ref32[0])
                n = len(check_checkpoint_slots(sf, layer_inputs))
                say(f"step 1: checkpoint slots of {n} decoders equal the non-offloaded forward's layer inputs")
                served, sf.runtime.capture_served = sf.runtime.capture_served, None
                n = len(check_served_checkpoints(served, layer_inputs))
                n_side = check_served_side_inputs(served, L)
                n_units = len(check_backward_weights(served, sums, range(1, L + 2)))
                del served, layer_inputs
                say(f"step 1: the recomputes of {n} decoders were given the non-offloaded forward's layer inputs "
                    f"and {n_side} more tensors of the forward's; the backward of {n_units} units read the forward's "
                    f"weights")
                check_step1_against_reference(cap, ref_grads, units, ref_sums)
                del ref_grads
                say(f"step 1: loss and gradients of units {units} equal the non-offloaded run's bit for bit, and every "
                    f"unit's gradient checksums")
            check_packed_grads(cap, units)
            orc.step(cap)
            check_masters(sf, orc, units)
            del cap
            sf.runtime.capture = None
            if k == CHECKED_STEPS - 1:
                check_moments(sf, orc, units)
                owned = {u for u in units if sf.layer_states[u].resident_across_steps}
                staged = check_staged(sf, orc, units, batches[STEPS].to(dev))
                say(f"staged bf16 weights checked for units {staged} (own buffers: {sorted(owned)})")
                assert set(staged) == owned and 1 in owned, (staged, owned)
        sf.wait_for_updates()
    finally:
        # the pinned masters (48 GB with the gradient slots) must go before
        # another run in this process pins its own
        sf.close()
        del sf, model
        gc.collect()
        torch.cuda.empty_cache()
    say("reference", [round(x, 5) for x in ref], [round(x, 6) for x in ref32])
    say("SlideFSDP", [round(x, 5) for x in got], [round(x, 6) for x in got32])
    for k, (a, b) in enumerate(zip(got, ref)):
        assert abs(a - b) <= 1e-2 * abs(b), (k, a, b)
    # the fp32 loss moves over the ten steps, and SlideFSDP's drop from step 1
    # tracks the reference's
    drop_ref, drop_got = ref32[0] - ref32[-1], got32[0] - got32[-1]
    say(f"fp32 loss drop over {STEPS} steps: reference {drop_ref:.5f}, SlideFSDP {drop_got:.5f}")
    assert drop_ref > 0.0
    assert abs(drop_got - drop_ref) <= 0.2 * drop_ref, (drop_got, drop_ref)
