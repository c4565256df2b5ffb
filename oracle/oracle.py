"""Scalar / numpy restatement of the reference's layer-streaming arithmetic.

TEST INFRASTRUCTURE ONLY (see the package docstring): results are checked
against it; it is never the thing measured or shipped.
"""

from __future__ import annotations

import ctypes
import os
from typing import Dict, Iterable, List, Sequence, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))


def lib_path() -> str:
    return os.path.join(_HERE, "lib", "libsf_oracle.so")


_LIB = None


def _lib() -> ctypes.CDLL:
    """The compiled scalar C restatement (oracle/sf_oracle.c)."""
    global _LIB
    if _LIB is None:
        path = lib_path()
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run `make -C oracle`)")
        lib = ctypes.CDLL(path)
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        f = ctypes.c_float
        lib.oracle_cast_f32_bf16.argtypes = [vp, vp, sz]
        lib.oracle_cast_f32_f16.argtypes = [vp, vp, sz]
        lib.oracle_widen_bf16.argtypes = [vp, vp, sz]
        lib.oracle_adam_init.argtypes = [vp, f, f, f, f, f, ctypes.c_int]
        lib.oracle_adam_update.argtypes = [vp, sz, f, f, f, f, f, ctypes.c_int, vp, vp, vp, vp, sz]
        lib.oracle_adam_scalars.argtypes = [vp, vp, vp]
        _LIB = lib
    return _LIB


# ---------------------------------------------------------------------------
# Cast, widen, pack
# ---------------------------------------------------------------------------

def cast_f32_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even, NaN -> 0xFFFF.

    Restates the CPU cast of reference layer_state.py:301
    (``_bf16_convert_buffer[:n].copy_(_cpu_params_flat)``), i.e. torch's
    vectorised CPU float->bfloat16 conversion.  Pinned by: torch CPU
    ``.to(torch.bfloat16)`` itself (the routine the reference calls) on the
    golden fixtures and on exhaustive bit-pattern sweeps, and by closed forms
    (exactly representable values map to their top half; ties go to even;
    overflow past the largest bf16 gives inf).
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16))
    r = r.astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r[nan] = np.uint16(0xFFFF)
    return r


def cast_f32_bf16_c(x: np.ndarray) -> np.ndarray:
    """The same cast through the scalar C restatement (oracle/sf_oracle.c)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    _lib().oracle_cast_f32_bf16(x.ctypes.data, out.ctypes.data, x.size)
    return out


def cast_f32_f16(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 bit patterns (uint16): IEEE round to nearest even with
    subnormals, overflow to infinity, NaN -> quiet NaN keeping the sign and
    the top 9 payload bits (sign | 0x7E00 | mantissa >> 13).

    Restates the CPU cast of reference layer_state.py:301 for units of dtype
    float16 (the convert buffer takes the config's dtype, slide_fsdp.py:
    181-186; config.py:110-113 allows float16): torch's CPU float -> half
    conversion.  Pinned by: torch CPU ``.to(torch.float16)`` itself on bit
    sweeps and specials; numpy's own float -> half conversion (an independent
    IEEE implementation) on every non-NaN input of the sweeps; closed forms
    (exact halves map to themselves, the largest half 65504, the tie 65520 to
    infinity, the smallest subnormal 2**-24 and the tie 2**-25 to zero)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    sign = ((u >> 16) & 0x8000).astype(np.uint64)
    a = u & 0x7FFFFFFF
    out = np.zeros(u.shape, dtype=np.uint64)
    nan = a > 0x7F800000
    inf = ~nan & (a >= 0x477FF000)
    normal = ~nan & ~inf & (a >= 0x38800000)
    sub = ~nan & ~inf & ~normal
    out[nan] = 0x7E00 | ((a[nan] >> 13) & 0x1FF)
    out[inf] = 0x7C00
    r = a[normal] - 0x38000000
    out[normal] = (r + 0xFFF + ((r >> 13) & 1)) >> 13
    e = a[sub] >> 23
    m = (a[sub] & 0x7FFFFF) | 0x800000
    shift = np.clip(126 - e.astype(np.int64), 14, 40).astype(np.uint64)
    q = m >> shift
    rem = m & ((np.uint64(1) << shift) - 1)
    half = np.uint64(1) << (shift - 1)
    up = (rem > half) | ((rem == half) & ((q & 1) == 1))
    val = q + up.astype(np.uint64)
    val[e < 102] = 0
    out[sub] = val
    return (out | sign).astype(np.uint16)


def cast_f32_f16_c(x: np.ndarray) -> np.ndarray:
    """The same fp16 cast through the scalar C restatement (oracle/sf_oracle.c)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    _lib().oracle_cast_f32_f16(x.ctypes.data, out.ctypes.data, x.size)
    return out


def widen_f16(h: np.ndarray) -> np.ndarray:
    """fp16 bit patterns -> fp32, exact: the ``grad.float()`` of reference
    optimizer/layer_adam/layer_adam.py:404 for float16 units.  Pinned by torch
    CPU ``.float()`` on all 65536 fp16 patterns, NaN payloads included (a
    signaling NaN comes back quiet)."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = h.view(np.float16).astype(np.float32).view(np.uint32)   # exact for every non-NaN
    nan = ((h & 0x7C00) == 0x7C00) & ((h & 0x3FF) != 0)
    hn = h[nan].astype(np.uint32)
    out[nan] = ((hn & 0x8000) << 16) | 0x7FC00000 | ((hn & 0x3FF) << 13)
    return out.view(np.float32)


def widen_bf16(b: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> fp32, the exact ``grad.float()`` of reference
    optimizer/layer_adam/layer_adam.py:404 (simd.h:47-54: a 16-bit shift).
    Pinned by torch CPU ``.float()`` on all 65536 bf16 patterns."""
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def pack_b16(parts: Sequence[np.ndarray]) -> np.ndarray:
    """Concatenate 16-bit tensors in order: the flat layout of reference
    layer_state.py:241-264 (view k starts where view k-1 ends), which is what
    the grad D2H of distributed_sync.py:353 moves.  Pinned by the invariant
    ``flat == torch.cat([p.flatten() for p in layer.parameters()])`` and the
    closed-form offset table of a Llama-3-8B layer."""
    if not parts:
        return np.empty(0, dtype=np.uint16)
    return np.concatenate([np.ascontiguousarray(p).reshape(-1).view(np.uint16) for p in parts])


# ---------------------------------------------------------------------------
# Flat layout of a unit
# ---------------------------------------------------------------------------

def layer_layout(named_shapes: Iterable[Tuple[str, Tuple[int, ...]]]) -> List[Tuple[str, int, Tuple[int, ...], int]]:
    """(name, offset, shape, numel) for each parameter in ``named_parameters()``
    order, offsets accumulating from 0 with no padding: reference
    layer_state.py:241-264 (``_param_maps[name] = (offset, shape, size)``)."""
    out = []
    off = 0
    for name, shape in named_shapes:
        n = int(np.prod(shape)) if len(shape) else 1
        out.append((name, off, tuple(shape), n))
        off += n
    return out


# Closed-form table of one Llama-3-8B decoder layer (hidden 4096, 32 heads /
# 8 KV heads of 128, intermediate 14336), in transformers' named_parameters()
# order: (name, offset, numel).  Total 218,112,000.
LLAMA3_8B_LAYER_TABLE = [
    ("self_attn.q_proj.weight", 0, 16_777_216),
    ("self_attn.k_proj.weight", 16_777_216, 4_194_304),
    ("self_attn.v_proj.weight", 20_971_520, 4_194_304),
    ("self_attn.o_proj.weight", 25_165_824, 16_777_216),
    ("mlp.gate_proj.weight", 41_943_040, 58_720_256),
    ("mlp.up_proj.weight", 100_663_296, 58_720_256),
    ("mlp.down_proj.weight", 159_383_552, 58_720_256),
    ("input_layernorm.weight", 218_103_808, 4_096),
    ("post_attention_layernorm.weight", 218_107_904, 4_096),
]


# ---------------------------------------------------------------------------
# AdamW
# ---------------------------------------------------------------------------

class _AdamStruct(ctypes.Structure):
    _fields_ = [
        ("alpha", ctypes.c_float), ("beta1", ctypes.c_float), ("beta2", ctypes.c_float),
        ("eps", ctypes.c_float), ("weight_decay", ctypes.c_float),
        ("beta1_t", ctypes.c_float), ("beta2_t", ctypes.c_float),
        ("step", ctypes.c_size_t), ("adamw_mode", ctypes.c_int),
        ("bc1", ctypes.c_float), ("bc2", ctypes.c_float),
    ]


class OracleAdam:
    """One reference ``Adam_Optimizer`` (cpu_adam.h:26-106), restated in scalar C.

    ``update`` mirrors ``ds_adam_step`` (cpu_adam_impl.cpp:211-237): advance
    the beta^t state (cpu_adam.h:57-76), set lr/eps/wd and bias corrections
    (cpu_adam.h:77-89), then update every element in the vector-body order of
    Step_AVX (cpu_adam.h:170-191), with the last n % 16 elements in the scalar
    tail order (cpu_adam_impl.cpp:45-64) as the reference's compiler fuses it.

    Pinned by: the reference's own cpu_adam compiled from its sources
    (oracle/_ref, when /root/reference is present) and the fixtures it wrote
    under tests/golden; closed forms at t = 1 (m = (1-b1) g, v = (1-b2) g^2,
    update = -lr * m / (bc1 * (sqrt(v)/sqrt(bc2') + eps))); and
    torch.optim.AdamW within float tolerance.
    """

    def __init__(self, alpha=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, adamw_mode=True):
        self._s = _AdamStruct()
        _lib().oracle_adam_init(ctypes.byref(self._s), alpha, betas[0], betas[1], eps,
                                weight_decay, 1 if adamw_mode else 0)

    def update(self, step: int, lr: float, beta1: float, beta2: float, eps: float, wd: float,
               bias_correction: bool, p: np.ndarray, g: np.ndarray, m: np.ndarray, v: np.ndarray) -> None:
        for a in (p, g, m, v):
            if a.dtype != np.float32 or not a.flags.c_contiguous:
                raise TypeError("OracleAdam.update takes C-contiguous float32 arrays")
        n = p.size
        if not (g.size == m.size == v.size == n):
            raise ValueError("size mismatch")
        _lib().oracle_adam_update(ctypes.byref(self._s), step, lr, beta1, beta2, eps, wd,
                                  1 if bias_correction else 0, p.ctypes.data, g.ctypes.data,
                                  m.ctypes.data, v.ctypes.data, n)

    def scalars(self) -> Tuple[float, float]:
        """(bias_correction1, bias_correction2) of the last update."""
        a, b = ctypes.c_float(), ctypes.c_float()
        _lib().oracle_adam_scalars(ctypes.byref(self._s), ctypes.byref(a), ctypes.byref(b))
        return a.value, b.value


class LayerAdamOracle:
    """Restates LayerAdam's per-layer bookkeeping over OracleAdam.

    Reference optimizer/layer_adam/layer_adam.py: one optimizer id for all
    layers (:59-69); ``add_layer_params`` (:131-195) gives each layer a param
    group with its own ``step`` and zeroed fp32 flat moments laid out in
    parameter order; ``step_with_grad_views`` (:358-425) increments that
    layer's step once, then calls ``adam_update`` per parameter in order with
    ``grad.float()``.  Layer groups are indexed by insertion order, as the
    reference indexes ``param_groups[layer_idx]``.
    Pinned by: running it against the compiled reference driven the same way
    (tests), and the t = 1 closed form.
    """

    def __init__(self, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0,
                 bias_correction=True, adamw_mode=True):
        self.lr, self.betas, self.eps, self.wd = lr, tuple(betas), eps, weight_decay
        self.bias_correction = bias_correction
        self.adam = OracleAdam(lr, betas, eps, weight_decay, adamw_mode)
        self.groups: List[Dict] = []

    def add_layer(self, params: Sequence[np.ndarray]) -> int:
        n = sum(p.size for p in params)
        m = np.zeros(n, np.float32)
        v = np.zeros(n, np.float32)
        views, off = [], 0
        for p in params:
            views.append((m[off:off + p.size], v[off:off + p.size]))
            off += p.size
        self.groups.append({"params": list(params), "step": 0, "m": m, "v": v, "views": views})
        return len(self.groups) - 1

    def moments(self, idx: int):
        """The layer's flat (exp_avg, exp_avg_sq)."""
        return self.groups[idx]["m"], self.groups[idx]["v"]

    def step_layer(self, idx: int, grads: Sequence[np.ndarray]) -> None:
        """grads: per-parameter arrays, float32, bf16 bit patterns (uint16) or
        float16."""
        grp = self.groups[idx]
        grp["step"] += 1
        for p, g, (m, v) in zip(grp["params"], grads, grp["views"]):
            if g.dtype == np.uint16:
                g32 = widen_bf16(g)
            elif g.dtype == np.float16:
                g32 = widen_f16(g.view(np.uint16))
            else:
                g32 = np.ascontiguousarray(g, np.float32)
            self.adam.update(grp["step"], self.lr, self.betas[0], self.betas[1], self.eps, self.wd,
                             self.bias_correction, p.reshape(-1), g32.reshape(-1), m, v)


# ---------------------------------------------------------------------------
# Unit schedule of one training step
# ---------------------------------------------------------------------------

def step_schedule(num_decoders: int, act_offload: bool = True, first_decoder_first: bool = False,
                  resident_units: Tuple[int, ...] = ()) -> List[Tuple]:
    """Expected order of staging events for one training step of a model with
    ``num_decoders`` decoder layers, units numbered 0 (embedding),
    1..L (decoders), L+1 (norm + lm_head).

    Events: ("h2d", unit, grads) parameter load, ``grads`` True where the
    reference loads with grad buffers (is_backward); ("d2h", unit) gradient
    offload; ("act_d2h", unit) checkpoint input packed to its host slot;
    ("act_h2d", unit) checkpoint input prefetched back.

    Follows reference slide_fsdp.py:535-541 (embedding and first decoder
    loaded up front), :366-381 (each PreLayerFunction prefetches the next
    unit, the output unit with grads, :372-373), :399-400 and :576 (the last
    decoder and the output unit stay resident: no reload in backward,
    layer_state.py:286-287), :432-448 (each unit's backward prefetches the
    unit before it with grads), :450-464 (gradient offload after the unit's
    backward), sliding_checkpoint.py:58-59, 62-75 (every decoder but the
    last packs its checkpoint input) and :88-108 (decoder j's first unpack
    prefetches decoder j-1).  One deliberate difference: the offload of a
    unit's gradients is triggered after all of its gradients exist, not by
    the first parameter's pre-hook (slide_fsdp.py:419-430), which fires
    before the unit's backward is complete; the order of events is the same.
    ``first_decoder_first`` swaps the two initial loads (an ordering the
    reference does not use; the set of events is unchanged).
    ``resident_units`` (not in the reference) keep their forward load for the
    backward: their backward ("h2d", u, True) event is absent.
    Pinned by (tests/test_schedule.py): an event model of the reference's
    autograd nodes and residency flags (its forward records the nodes, its
    backward replays them in reverse), which must give the same schedule for
    every L = 1..8, every resident set, with and without checkpoint offload
    and in both first-load orders; invariants read off the reference's hook
    order; and planted mistakes (last decoder reloaded, prefetch two ahead,
    grads flag dropped, late checkpoint prefetch, embedding reload missing)
    that both checks must reject.
    """
    L = num_decoders
    out: List[Tuple] = [("h2d", 0, False), ("h2d", 1, False)]
    if first_decoder_first:
        out.reverse()
    for i in range(1, L + 1):
        nxt = i + 1
        out.append(("h2d", nxt, nxt == L + 1))
        if act_offload and i < L:
            out.append(("act_d2h", i))
    # backward: output unit first, then decoders L..1, then the embedding
    out.append(("d2h", L + 1))
    for i in range(L, 0, -1):
        if i - 1 not in resident_units:
            out.append(("h2d", i - 1, True))
        if act_offload and i >= 2:
            out.append(("act_h2d", i - 1))
        out.append(("d2h", i))
    out.append(("d2h", 0))
    return out
