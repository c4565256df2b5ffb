"""Transfer strategy of the layer-streaming path: single GPU only.

Reference distributed_sync.py:313-377.  With one GPU the reference picks
``NoOpSync``: a full-layer H2D copy (``gather_params_to_gpu``) and a D2H copy
of the gradients (``reduce_gradients_to_master``).  Here those copies are
issued by ``layer_state`` itself on dedicated streams, so ``NoOpSync`` only
keeps the reference's object and method names for code that calls them
directly; ``SlideFSDP.close`` calls its ``cleanup`` as the reference's
``__del__`` does (slide_fsdp.py:744).  Several GPUs (``DistributedSync``:
shard-mode all-gather, grad reduce) are not part of this build;
``create_distributed_sync`` raises when a multi-rank process group is
initialised.
"""

from __future__ import annotations

import torch
import torch.distributed as dist

from . import kernels


class NoOpSync:
    """One-GPU copies (reference distributed_sync.py:313-362), asynchronous on
    the current stream through the library's copy entry point."""

    def __init__(self, config):
        self.config = config
        self.device = config.device
        self.dtype = config.dtype
        self.world_size = 1
        self.rank = 0
        self.is_distributed = False
        # the reference reads it for its CPU-side barriers (layer_state.py:270, 433)
        self.cpu_group = None

    def gather_params_to_gpu(self, cpu_params: torch.Tensor, gpu_buffer: torch.Tensor, layer_state=None) -> None:
        n = cpu_params.numel()
        kernels.memcpy_async(gpu_buffer[:n], cpu_params[:n])

    def reduce_gradients_to_master(self, gpu_grads: torch.Tensor, cpu_buffer: torch.Tensor, layer_state=None) -> None:
        n = gpu_grads.numel()
        kernels.memcpy_async(cpu_buffer[:n], gpu_grads[:n])
        torch.cuda.current_stream().synchronize()

    sync_gradients_to_cpu = reduce_gradients_to_master

    def cleanup(self) -> None:
        pass


def create_distributed_sync(config) -> NoOpSync:
    """NoOpSync on one process; several ranks are not supported by this build
    (reference distributed_sync.py:365-377 would return DistributedSync)."""
    if dist.is_available() and dist.is_initialized() and dist.get_world_size() > 1:
        raise NotImplementedError("SlideFSDP in this build runs on a single GPU (world_size must be 1)")
    return NoOpSync(config)
