"""The bf16 reload copies of the units the backward reloads, on the CPU:
which units get one, the pinned reserve held while they are pinned (and
given back), the fall-back to fp32 reloads when the host cannot pin more,
and that an update writes the copy (the RNE cast of the updated master)."""

import threading
from types import SimpleNamespace

import pytest
import torch

from test1_amd import _native


def _oom():
    return _native.NativeError("sf_host_alloc failed: out of memory", _native.HIP_ERROR_OUT_OF_MEMORY)


class _State:
    def __init__(self, idx, own=False, ok=True, log=None):
        self.layer_idx, self.resident_across_steps, self.ok, self.log = idx, own, ok, log

    def enable_bf16_reload(self):
        self.log.append(("enable", self.layer_idx))
        return self.ok


def _model(states):
    from test1_amd import slide_fsdp

    sf = object.__new__(slide_fsdp.SlideFSDP)
    sf.__dict__["layer_states"] = states
    return sf


def test_reload_copies_for_reloaded_decoders_only(monkeypatch):
    from test1_amd import pinned

    log = []
    # embedding, decoders 1..5 (4 and 5 with own buffers; 5 is the last), output
    states = ([_State(0, log=log)] + [_State(i, own=i >= 4, log=log) for i in range(1, 6)]
              + [_State(6, log=log)])
    monkeypatch.setattr(pinned, "pinned_empty", lambda shape, dtype: log.append(("reserve", shape)) or
                        torch.empty(0, dtype=dtype))
    got = _model(states)._enable_bf16_reloads(reserve_bytes=123)
    assert got == [1, 2, 3]
    assert log == [("reserve", 123), ("enable", 1), ("enable", 2), ("enable", 3)]


def test_reload_copies_stop_at_the_pinned_limit(monkeypatch):
    from test1_amd import pinned

    log = []
    states = [_State(0, log=log)] + [_State(i, ok=i < 3, log=log) for i in range(1, 7)] + [_State(7, log=log)]
    monkeypatch.setattr(pinned, "pinned_empty", lambda shape, dtype: torch.empty(0, dtype=dtype))
    assert _model(states)._enable_bf16_reloads() == [1, 2]
    assert log == [("enable", 1), ("enable", 2), ("enable", 3)]


def test_no_reload_copies_without_room_for_the_reserve(monkeypatch):
    from test1_amd import pinned

    def refuse(shape, dtype):
        raise _oom()

    log = []
    monkeypatch.setattr(pinned, "pinned_empty", refuse)
    states = [_State(0, log=log)] + [_State(i, log=log) for i in range(1, 4)] + [_State(4, log=log)]
    assert _model(states)._enable_bf16_reloads() == [] and log == []


def _unit(monkeypatch, n=48, refuse=False, fmt="fp32"):
    from test1_amd import layer_state

    st = object.__new__(layer_state.LayerRuntimeState)
    master = torch.randn(n) * 0.02
    st.__dict__.update(
        _reload_bf16=None, _cpu_params_bf16=None, row_sparse=False, backward_reads_params=True,
        buffer_pool=SimpleNamespace(dtype=torch.bfloat16), runtime=SimpleNamespace(h2d_format=fmt),
        total_size=n, _cpu_params_flat=master, update_lock=threading.Lock(), _param_maps={}, _params=[])
    st.wait_for_update = lambda timeout=None: None

    def pin(shape, dtype):
        if refuse:
            raise _oom()
        return torch.empty(shape, dtype=dtype)

    monkeypatch.setattr(layer_state, "pinned_empty", pin)
    return st


def test_reload_copy_is_the_cast_of_the_master(monkeypatch):
    st = _unit(monkeypatch)
    assert st.enable_bf16_reload()
    assert torch.equal(st._reload_bf16.view(torch.int16), st._cpu_params_flat.to(torch.bfloat16).view(torch.int16))
    assert st._bf16_host() is st._reload_bf16


def test_reload_copy_refused_keeps_fp32_reloads(monkeypatch):
    st = _unit(monkeypatch, refuse=True)
    assert not st.enable_bf16_reload() and st._reload_bf16 is None and st._bf16_host() is None


@pytest.mark.parametrize("fmt", ["bf16"])
def test_no_reload_copy_with_bf16_h2d(monkeypatch, fmt):
    st = _unit(monkeypatch, fmt=fmt)
    assert not st.enable_bf16_reload() and st._reload_bf16 is None


def test_update_writes_the_reload_copy(monkeypatch):
    """The host AdamW's fused pass writes the bf16 copy of each updated
    parameter: after an update through LayerAdam with the unit's bf16 views,
    the reload copy is the RNE cast of the new master."""
    from test1_amd.optimizer import LayerAdam

    n = 64
    p = torch.nn.Parameter(torch.randn(n) * 0.02)
    opt = LayerAdam(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, num_layer=1)
    opt.add_layer_params(0, [p])
    copy = p.data.to(torch.bfloat16)
    grad = (torch.randn(n) * 1e-3).to(torch.bfloat16)
    with torch.no_grad():
        opt.step_with_grad_views(0, {p: grad}, param_views={p: p.data}, bf16_views={p: copy})
    assert torch.equal(copy.view(torch.int16), p.data.to(torch.bfloat16).view(torch.int16))
