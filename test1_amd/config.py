"""SlideFSDPConfig: the reference's configuration dataclass, field for field.

Same names, defaults, validation and dict round trip as reference
config.py:16-165, so existing JSON configs and call sites work unchanged.
Fields that only matter for several GPUs (``param_transfer_mode="shard"``,
``grad_sync_mode``) are accepted and validated here; ``SlideFSDP`` rejects
the ones a single GPU cannot honour.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, fields
from typing import Optional, Tuple

import torch

_DTYPES = {"bf16": torch.bfloat16, "bfloat16": torch.bfloat16, "fp16": torch.float16, "float16": torch.float16}


@dataclass
class SlideFSDPConfig:
    """Configuration of the layer-streaming trainer (reference config.py:16-93).

    Runtime knobs that the reference declares but does not read
    (``prefetch_layers``, ``max_workers``: its executors are fixed at one
    worker, slide_fsdp.py:161-163) are kept for compatibility and likewise
    unused: the prefetch distance is one unit by design.
    """

    dtype: torch.dtype = torch.bfloat16
    device: Optional[torch.device] = None

    param_transfer_mode: str = "full"
    grad_sync_mode: str = "gpu_reduce"

    lr: float = 1e-5
    weight_decay: float = 0.01
    adam_betas: Tuple[float, float] = (0.9, 0.999)
    adam_eps: float = 1e-8
    bias_correction: bool = True

    prefetch_layers: int = 1
    max_workers: int = 1
    enable_activation_checkpoint: bool = True
    gpu_buffer_pool_size: int = 2

    model_path: str = ""
    max_seq_length: int = 1024
    train_batch_size: int = 4
    num_epochs: int = 1
    log_every_n_steps: int = 1
    seed: int = 42
    use_liger_kernel: bool = True
    attention_implementation: str = "flash_attention_2"

    ac_offload_mode: str = "cpu"
    ac_offload_dir: str = "/tmp/ac_offload"

    optimizer_nvme_offload_fraction: float = 0.0
    optimizer_offload_dir: str = "/tmp/opt_offload"

    clip_grad_norm: float = 1.0

    def __post_init__(self):
        # Validation order and messages follow reference config.py:95-124.
        if self.param_transfer_mode not in ("full", "shard"):
            raise ValueError(f"param_transfer_mode must be 'full' or 'shard', got {self.param_transfer_mode}")
        if self.grad_sync_mode not in ("gpu_reduce", "cpu_reduce"):
            raise ValueError(f"grad_sync_mode must be 'gpu_reduce' or 'cpu_reduce', got {self.grad_sync_mode}")
        if self.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError(f"dtype must be torch.bfloat16 or torch.float16, got {self.dtype}")
        if self.device is None:
            self.device = torch.device("cuda", int(os.environ.get("LOCAL_RANK", 0)))
        if self.ac_offload_mode not in ("cpu", "nvme", "none"):
            raise ValueError(f"ac_offload_mode must be 'cpu', 'nvme', or 'none', got {self.ac_offload_mode}")

    @classmethod
    def from_dict(cls, config_dict: dict) -> "SlideFSDPConfig":
        """Build from a dict: string dtypes and devices, list betas, unknown keys
        dropped (reference config.py:126-153).  Like the reference, the input
        dict is updated in place with the converted values."""
        d = config_dict
        if isinstance(d.get("dtype"), str):
            d["dtype"] = _DTYPES.get(d["dtype"].lower(), torch.bfloat16)
        if isinstance(d.get("device"), str):
            d["device"] = torch.device(d["device"])
        if isinstance(d.get("adam_betas"), list):
            d["adam_betas"] = tuple(d["adam_betas"])
        names = {f.name for f in fields(cls)}
        return cls(**{k: v for k, v in d.items() if k in names})

    def to_dict(self) -> dict:
        """Plain dict with dtype as e.g. "bfloat16" and device as "cuda:0"
        (reference config.py:155-165)."""
        out = {}
        for f in fields(self):
            v = getattr(self, f.name)
            if isinstance(v, torch.dtype):
                v = str(v).replace("torch.", "")
            elif isinstance(v, torch.device):
                v = str(v)
            out[f.name] = v
        return out
