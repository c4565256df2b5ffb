"""CPU oracle for the layer-streaming path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the CPU-baseline leg of ``bench.py`` may import this package, and only to
check results.  The product (``test1_amd``) never imports, links or runs it.

Contents (each function cites the reference file:line it restates):
  cast_f32_bf16    layer_state.py:301                fp32 -> bf16 RNE cast
  cast_f32_f16     layer_state.py:301 (float16 units) fp32 -> fp16 RNE cast
  widen_f16        optimizer/layer_adam/layer_adam.py:404   fp16 -> fp32
  widen_bf16       optimizer/layer_adam/layer_adam.py:404   bf16 -> fp32
  pack_b16         layer_state.py:241-264, distributed_sync.py:353
  layer_layout     layer_state.py:241-264            flat offsets and views
  OracleAdam       optimizer/layer_adam/csrc/cpu_adam.h:57-192,
                   cpu_adam_impl.cpp:21-68, 211-237
  LayerAdamOracle  optimizer/layer_adam/layer_adam.py:131-195, 358-425
  step_schedule    slide_fsdp.py:507-640, 363-464; layer_state.py:273-457

How each part is pinned is stated in each docstring; a part with no
independent check says "parity unpinned".
"""

from .oracle import (  # noqa: F401
    LLAMA3_8B_LAYER_TABLE,
    LayerAdamOracle,
    OracleAdam,
    cast_f32_bf16,
    cast_f32_bf16_c,
    cast_f32_f16,
    cast_f32_f16_c,
    layer_layout,
    lib_path,
    pack_b16,
    step_schedule,
    widen_bf16,
    widen_f16,
)
