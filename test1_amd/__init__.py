"""MI355X-native single-GPU layer-streaming training (SlideFSDP drop-in).

Public API, matching the reference's:
    SlideFSDPConfig, SlideFSDP, LayerAdam, SlidingCheckpoint,
    LayerBufferPool, LayerRuntimeState
The device work runs in hand-written HIP kernels for gfx950 behind the C ABI
declared in include/slidefsdp.h (``test1_amd/lib/libsf_hip.so``); the host
AdamW runs in ``test1_amd/lib/libsf_cpu.so``.
"""

from .config import SlideFSDPConfig  # noqa: F401


def __getattr__(name):
    # Lazy imports: the config (and the CPU optimizer) import without a GPU;
    # the runtime classes need transformers and the HIP library.
    if name in ("SlideFSDP", "OutputLayer"):
        from . import slide_fsdp
        return getattr(slide_fsdp, name)
    if name in ("LayerBufferPool", "LayerRuntimeState", "H2DStager", "GradStagingRing", "GradSlotRing"):
        from . import layer_state
        return getattr(layer_state, name)
    if name in ("SlidingCheckpoint", "ActivationRing", "StorageSpill", "save_on_cpu"):
        from . import sliding_checkpoint
        return getattr(sliding_checkpoint, name)
    if name == "LayerAdam":
        from .optimizer import LayerAdam
        return LayerAdam
    raise AttributeError(name)
