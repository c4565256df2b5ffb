"""The reference's own schedule at the full Llama-3.1-8B shape (32 layers,
hidden 4096, vocab 128256; batch 4 x 1024, uniform random tokens): every unit
in the 2-unit ``LayerBufferPool`` and reloaded for its backward
(``resident_layers=0``, reference slide_fsdp.py:432-448, layer_state.py:28-101,
279-326), nothing staged after its update (``stage_after_update=False``), so
the backward's checkpoint prefetches run on the parameter H2D stream behind
the weight reloads, as in the reference.

* The schedule: in step 1 the forward loads every unit, and the backward
  reloads every decoder below the last and skips the embedding (whose
  backward reads no weights) and the two units still loaded.
* Step 1: the loss and the device gradients of the first, a middle and the
  last decoder, the output unit and the embedding equal, bit for bit, those
  of a non-offloaded bf16 forward/backward of the same weights (transformers'
  own forward with per-layer recompute), and every other unit's gradients
  have the non-offloaded run's checksums.  Every offloaded decoder's pinned
  checkpoint slot holds its layer's input in the non-offloaded forward, each
  recompute was given that input, and each unit's reloaded weights at the
  start and end of its backward have the checksum of the non-offloaded run's
  bf16 weights.
* Steps 1-3: those units' packed host gradients equal their device
  gradients, every update and moment is the oracle AdamW's bit for bit, and a
  forward after step 3 computes with the oracle's cast of the updated masters
  in the units it leaves loaded (the last decoder and the output unit).
* The backward's reloads come from the bf16 copies the updates write
  (``bf16_reload``, the default with fp32 H2D): in every step each unit's
  weights at the start and end of its backward have the checksum of the RNE
  cast of its current master, so a copy an update left stale fails.

Host memory ~140 GB; the file sorts after the other GPU tests."""

import gc
import os
import sys
import time

import pytest
import torch

from fullsize import (CapturedOracle, check_backward_weights, check_checkpoint_slots, check_masters, check_moments,
                      check_packed_grads, check_served_checkpoints, check_served_side_inputs, check_staged,
                      check_step1_against_reference, gpu_bf16_copy, master_weight_sums, reference_step, say, timed,
                      unit_weight_sums)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

LR, BETAS, EPS, WD = 1e-5, (0.9, 0.999), 1e-8, 0.01
STEPS = 3


def test_llama31_8b_reference_schedule_parity(dev):
    sys.path.insert(0, ROOT)
    import bench
    from test1_amd import SlideFSDP, SlideFSDPConfig

    w = dict(bench.WORKLOADS["llama3-8b"])
    L = w["layers"]
    units = (0, 1, L // 2, L, L + 1)
    model = timed("model built", bench.build_model, w)
    g = torch.Generator().manual_seed(5)
    batches = [torch.randint(0, w["vocab"], (w["batch"], w["seq"]), generator=g) for _ in range(STEPS + 1)]

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
    sf = timed("SlideFSDP set up", SlideFSDP, model, cfg, resident_layers=0, stage_after_update=False,
               wait_timeout=600)
    assert sf.resident_layers == 0 and not any(st.resident_across_steps for st in sf.layer_states)
    assert sf._act_prefetch_stream() is sf.runtime.h2d_stream
    assert sf.bf16_reload_units == list(range(1, L)), sf.bf16_reload_units
    sf.runtime.capture_units = set(units)
    try:
        for k in range(STEPS):
            sf.runtime.capture = {}
            sf.runtime.capture_served = {}
            if k > 0:
                sums = timed(f"master checksums before step {k + 1}", master_weight_sums, sf)
            sf.runtime.trace = [] if k == 0 else None
            ids = batches[k].to(dev)
            t = time.time()
            loss = sf(input_ids=ids, labels=ids).loss.item()
            sf.wait_for_updates()
            say(f"[SlideFSDP] step {k + 1}: loss {loss:.5f} ({time.time() - t:.1f} s)")
            cap = sf.runtime.capture
            assert sorted(u for u in cap if isinstance(u, int)) == sorted(units)
            if k == 0:
                loads = [(e[1], e[2]) for e in sf.runtime.trace if e[0] == "h2d"]
                fwd = sorted(u for u, bwd in loads[:L + 2])
                bwd = sorted(u for u, b in loads[L + 2:])
                assert fwd == list(range(L + 2)), loads
                # reloaded for the backward: every decoder below the last; the
                # embedding's reload reads no weights and copies nothing
                assert bwd == list(range(0, L)), loads
                say(f"step 1: forward loaded {len(fwd)} units, backward reloaded units 0..{L - 1}")
                assert loss == ref_loss, (loss, ref_loss)
                n = len(check_checkpoint_slots(sf, layer_inputs))
                say(f"step 1: checkpoint slots of {n} decoders equal the non-offloaded forward's layer inputs")
                served, sf.runtime.capture_served = sf.runtime.capture_served, None
                n = len(check_served_checkpoints(served, layer_inputs))
                n_side = check_served_side_inputs(served, L)
                n_units = len(check_backward_weights(served, sums, range(1, L + 2)))
                del served, layer_inputs
                say(f"step 1: the recomputes of {n} decoders were given the non-offloaded forward's layer inputs "
                    f"and {n_side} more tensors of the forward's; the backward of {n_units} reloaded units read "
                    f"the forward's weights")
                check_step1_against_reference(cap, ref_grads, units, ref_sums)
                del ref_grads
                say(f"step 1: loss and gradients of units {units} equal the non-offloaded run's bit for bit, and "
                    f"every unit's gradient checksums")
            else:
                served, sf.runtime.capture_served = sf.runtime.capture_served, None
                n_units = len(check_backward_weights(served, sums, range(1, L + 2)))
                del served
                say(f"step {k + 1}: the backward of {n_units} units read the cast of their current masters")
            check_packed_grads(cap, units)
            timed(f"oracle step {k + 1}", orc.step, cap)
            check_masters(sf, orc, units)
            del cap
            sf.runtime.capture = None
        check_moments(sf, orc, units)
        checked = check_staged(sf, orc, units, batches[STEPS].to(dev))
        say(f"staged bf16 weights checked for units {checked}")
        assert set(checked) == {L, L + 1}, checked
    finally:
        sf.close()
        del sf, model
        gc.collect()
        torch.cuda.empty_cache()
