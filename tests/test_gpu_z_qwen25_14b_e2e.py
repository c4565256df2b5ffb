"""The Qwen2.5-14B-shaped training step at its full size (48 layers, hidden
5120, intermediate 13824, 40/8 heads, vocab 152064, q/k/v biases; batch
2 x 4096 uniform random tokens) through SlideFSDP with its defaults, against
a non-offloaded bf16 run and the oracle (reference slide_fsdp.py:507-640).

Step 1: the loss and the gradients SlideFSDP offloads for the embedding, the
first, two middle and last decoders and the output unit equal, bit for bit, those of a
non-offloaded bf16 forward/backward of the same weights (transformers' own
forward with per-layer recompute; same kernels on the same bits, so the
offload, the recompute from offloaded checkpoints and the staged weights
change nothing), and every offloaded decoder's pinned checkpoint slot holds
that layer's input in the non-offloaded forward.  Steps 1-3: those units' packed host gradients equal their
device gradients, every update is the oracle AdamW's bit for bit, and so are
the moments; a forward after step 3 computes with the oracle's bf16 cast of
the updated masters.

With fp32 masters (59 GB pinned) one gradient slot per unit does not fit
under the pinned-memory cap of these hosts, so this also runs the slot ring
(the output unit in a slot of its own, the decoders in a ring).  Host memory
~230 GB."""

import gc
import os
import sys
import time

import pytest
import torch

from fullsize import (CapturedOracle, check_backward_weights, check_checkpoint_slots, check_served_checkpoints,
                      check_served_side_inputs, unit_weight_sums, check_masters, check_moments, check_packed_grads,
                      check_staged, check_step1_against_reference, gpu_bf16_copy, reference_step, say, timed)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

LR, BETAS, EPS, WD = 1e-5, (0.9, 0.999), 1e-8, 0.01
STEPS = 3


def test_qwen25_14b_step_against_reference_and_oracle(dev):
    sys.path.insert(0, ROOT)
    import bench
    from test1_amd import SlideFSDP, SlideFSDPConfig
    from test1_amd.grad_slots import GradSlotRing

    w = dict(bench.WORKLOADS["qwen2.5-14b"])
    L = w["layers"]
    units = (0, 1, L // 3, 2 * L // 3, L, L + 1)
    model = timed("model built", bench.build_model, w)
    g = torch.Generator().manual_seed(7)
    batches = [torch.randint(0, w["vocab"], (w["batch"], w["seq"]), generator=g) for _ in range(STEPS + 1)]

    from test1_amd.pinned import pinned_bytes_live
    say(f"pinned memory live at the start: {pinned_bytes_live() / 2**30:.1f} GiB")
    gm = timed("bf16 copy on the GPU", gpu_bf16_copy, model, dev)
    layer_inputs, ref_sums = [], {}
    ref_loss, ref_grads = timed("reference step", reference_step, gm, batches[0].to(dev), w["vocab"], units,
                                layer_inputs, ref_sums)
    sums = unit_weight_sums(gm)
    del gm
    gc.collect()
    torch.cuda.empty_cache()
    say(f"reference step-1 loss {ref_loss:.5f}")

    orc = timed("oracle set up", CapturedOracle, model, units, LR, BETAS, EPS, WD)
    cfg = SlideFSDPConfig(device=dev, lr=LR, adam_betas=BETAS, adam_eps=EPS, weight_decay=WD,
                          attention_implementation="sdpa")
    sf = timed("SlideFSDP set up", SlideFSDP, model, cfg, wait_timeout=600)
    say(f"pinned memory live after set-up: {pinned_bytes_live() / 2**30:.1f} GiB")
    ring = sf.runtime.grad_ring
    say(f"gradient slots: {type(ring).__name__}"
        + (f", own slots for units {sorted(ring.big)}, ring of {ring.depth}" if isinstance(ring, GradSlotRing) else ""))
    sf.runtime.capture_units = set(units)
    try:
        for k in range(STEPS):
            sf.runtime.capture = {}
            sf.runtime.capture_served = {} if k == 0 else None
            ids = batches[k].to(dev)
            t = time.time()
            loss = sf(input_ids=ids, labels=ids).loss.item()
            sf.wait_for_updates()
            say(f"[SlideFSDP] step {k + 1}: loss {loss:.5f} ({time.time() - t:.1f} s)")
            cap = sf.runtime.capture
            assert sorted(u for u in cap if isinstance(u, int)) == sorted(units)
            if k == 0:
                assert loss == ref_loss, (loss, ref_loss)
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
            timed(f"oracle step {k + 1}", orc.step, cap)
            check_masters(sf, orc, units)
            del cap
            sf.runtime.capture = None
        check_moments(sf, orc, units)
        owned = {u for u in units if sf.layer_states[u].resident_across_steps}
        checked = check_staged(sf, orc, units, batches[STEPS].to(dev))
        say(f"staged bf16 weights checked for units {checked} (units with own buffers: {sorted(owned)})")
        assert set(checked) == owned and owned & {1, L}, (checked, owned)
    finally:
        sf.close()
        del sf, model
        gc.collect()
        torch.cuda.empty_cache()
