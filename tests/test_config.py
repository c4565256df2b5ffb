"""SlideFSDPConfig is a field-for-field drop-in (reference config.py:16-165)."""

import dataclasses

import pytest
import torch

from test1_amd import SlideFSDPConfig

REFERENCE_FIELDS = {
    "dtype": torch.bfloat16, "device": None, "param_transfer_mode": "full", "grad_sync_mode": "gpu_reduce",
    "lr": 1e-5, "weight_decay": 0.01, "adam_betas": (0.9, 0.999), "adam_eps": 1e-8, "bias_correction": True,
    "prefetch_layers": 1, "max_workers": 1, "enable_activation_checkpoint": True, "gpu_buffer_pool_size": 2,
    "model_path": "", "max_seq_length": 1024, "train_batch_size": 4, "num_epochs": 1, "log_every_n_steps": 1,
    "seed": 42, "use_liger_kernel": True, "attention_implementation": "flash_attention_2",
    "ac_offload_mode": "cpu", "ac_offload_dir": "/tmp/ac_offload", "optimizer_nvme_offload_fraction": 0.0,
    "optimizer_offload_dir": "/tmp/opt_offload", "clip_grad_norm": 1.0,
}


def test_fields_and_defaults():
    fields = {f.name: f.default for f in dataclasses.fields(SlideFSDPConfig)}
    assert list(fields) == list(REFERENCE_FIELDS)
    assert fields == REFERENCE_FIELDS


def test_device_from_local_rank(monkeypatch):
    monkeypatch.setenv("LOCAL_RANK", "3")
    assert SlideFSDPConfig().device == torch.device("cuda", 3)


@pytest.mark.parametrize("kw", [{"param_transfer_mode": "x"}, {"grad_sync_mode": "x"},
                                {"dtype": torch.float32}, {"ac_offload_mode": "disk"}])
def test_validation(kw):
    with pytest.raises(ValueError):
        SlideFSDPConfig(device=torch.device("cpu"), **kw)


def test_from_dict_to_dict_round_trip():
    d = {"dtype": "fp16", "device": "cuda:1", "adam_betas": [0.8, 0.95], "lr": 3e-4, "unknown": 1}
    c = SlideFSDPConfig.from_dict(d)
    assert c.dtype == torch.float16 and c.device == torch.device("cuda", 1) and c.adam_betas == (0.8, 0.95)
    out = c.to_dict()
    assert out["dtype"] == "float16" and out["device"] == "cuda:1" and out["lr"] == 3e-4
    assert SlideFSDPConfig.from_dict(dict(out)) == c
    assert SlideFSDPConfig.from_dict({"dtype": "weird", "device": "cpu"}).dtype == torch.bfloat16
