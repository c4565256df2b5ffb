"""The oracle, pinned: against the golden fixtures (torch's CPU cast, the
reference's compiled CPU Adam), against closed forms and exhaustive sweeps,
and with planted mistakes that these checks must catch."""

import os

import numpy as np
import pytest
import torch

import oracle
from conftest import GOLDEN, load_ref_adam


# ---------------------------------------------------------------- cast
def test_cast_matches_golden_fixture():
    d = np.load(os.path.join(GOLDEN, "cast_f32_bf16.npz"))
    x = d["x_bits"].view(np.float32)
    assert np.array_equal(oracle.cast_f32_bf16(x), d["bf16_bits"])
    assert np.array_equal(oracle.cast_f32_bf16_c(x), d["bf16_bits"])


def test_cast_matches_torch_on_bit_sweep():
    # every high half-word with a spread of low half-words: 65536 x 8 patterns
    hi = np.arange(1 << 16, dtype=np.uint32)
    lo = np.array([0, 1, 0x7FFF, 0x8000, 0x8001, 0xC000, 0xFFFE, 0xFFFF], dtype=np.uint32)
    bits = (hi[:, None] << 16 | lo[None, :]).reshape(-1)
    x = bits.view(np.float32)
    exp = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.cast_f32_bf16(x), exp)
    assert np.array_equal(oracle.cast_f32_bf16_c(x), exp)


def test_cast_closed_forms():
    # exactly representable values keep their top half; ties go to even;
    # the largest values round to infinity; every NaN becomes 0xFFFF
    vals = np.array([1.0, -2.5, 0.0, -0.0], dtype=np.float32)
    assert np.array_equal(oracle.cast_f32_bf16(vals), (vals.view(np.uint32) >> 16).astype(np.uint16))
    ties = np.array([0x3F808000, 0x3F818000], dtype=np.uint32).view(np.float32)
    assert oracle.cast_f32_bf16(ties).tolist() == [0x3F80, 0x3F82]
    assert oracle.cast_f32_bf16(np.array([0x7F7FFFFF], np.uint32).view(np.float32))[0] == 0x7F80
    nans = np.array([0x7FC00000, 0xFF800001, 0x7F800001], np.uint32).view(np.float32)
    assert oracle.cast_f32_bf16(nans).tolist() == [0xFFFF] * 3


def test_cast_check_catches_truncation():
    # a planted mistake (truncation instead of rounding) must fail the fixture
    d = np.load(os.path.join(GOLDEN, "cast_f32_bf16.npz"))
    trunc = (d["x_bits"] >> 16).astype(np.uint16)
    assert not np.array_equal(trunc, d["bf16_bits"])


def test_widen_all_bf16_patterns():
    b = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    exp = torch.from_numpy(b.view(np.int16).copy()).view(torch.bfloat16).float().numpy()
    got = oracle.widen_bf16(b)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


# ---------------------------------------------------------------- fp16 cast (float16 units)
def _f16_sweep():
    # every high half-word with low half-words around the rounding point of
    # fp16's 13 dropped bits, plus random patterns
    hi = np.arange(1 << 16, dtype=np.uint32)
    lo = np.array([0, 1, 0x0FFF, 0x1000, 0x1001, 0x2000, 0x3000, 0xF000, 0xFFFF], dtype=np.uint32)
    bits = (hi[:, None] << 16 | lo[None, :]).reshape(-1)
    rnd = np.random.default_rng(5).integers(0, 1 << 32, 500_000, dtype=np.uint64).astype(np.uint32)
    return np.concatenate([bits, rnd]).view(np.float32)


def test_f16_cast_matches_torch_on_bit_sweep():
    x = _f16_sweep()
    exp = torch.from_numpy(x.copy()).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.cast_f32_f16(x), exp)
    assert np.array_equal(oracle.cast_f32_f16_c(x), exp)


def test_f16_cast_matches_numpy_on_non_nan():
    # numpy's float -> half conversion is an independent IEEE implementation
    x = _f16_sweep()
    ok = ~np.isnan(x)
    with np.errstate(over="ignore"):
        exp = x[ok].astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.cast_f32_f16(x)[ok], exp)


def test_f16_cast_closed_forms():
    f = lambda v: oracle.cast_f32_f16(np.array(v, dtype=np.float32)).tolist()   # noqa: E731
    assert f([1.0, -2.0, 0.0, -0.0, 65504.0]) == [0x3C00, 0xC000, 0x0000, 0x8000, 0x7BFF]
    assert f([65519.996, 65520.0, -1e30]) == [0x7BFF, 0x7C00, 0xFC00]     # the tie 65520 goes to inf
    assert f([2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -25, 2.0 ** -14]) == [0x0001, 0x0000, 0x0002, 0x0400]
    assert f([1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11]) == [0x3C00, 0x3C02]  # ties to even
    nans = np.array([0x7FC00000, 0xFF800001, 0x7FBFFFFF], np.uint32).view(np.float32)
    assert oracle.cast_f32_f16(nans).tolist() == [0x7E00, 0xFE00, 0x7FFF]


def test_f16_cast_check_catches_truncation():
    # a planted mistake (the 13 dropped bits truncated) must fail the torch sweep
    x = _f16_sweep()
    ok = (np.abs(x) < 60000) & (np.abs(x) > 1e-4)
    u = x[ok].view(np.uint32)
    trunc = (((u >> 16) & 0x8000) | (((u & 0x7FFFFFFF) - 0x38000000) >> 13)).astype(np.uint16)
    exp = torch.from_numpy(x[ok].copy()).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    assert not np.array_equal(trunc, exp)
    assert np.array_equal(oracle.cast_f32_f16(x[ok]), exp)


def test_widen_all_f16_patterns():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    exp = torch.from_numpy(h.view(np.int16).copy()).view(torch.float16).float().numpy()
    assert np.array_equal(oracle.widen_f16(h).view(np.uint32), exp.view(np.uint32))


# ---------------------------------------------------------------- pack / layout
def test_pack_is_concatenation_and_inverts():
    rng = np.random.default_rng(0)
    parts = [rng.integers(0, 1 << 16, n, dtype=np.uint16) for n in (5, 0, 4096, 3)]
    flat = oracle.pack_b16(parts)
    assert flat.size == sum(p.size for p in parts)
    off = 0
    for p in parts:
        assert np.array_equal(flat[off:off + p.size], p)
        off += p.size


def _llama_layer():
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer

    cfg = LlamaConfig(hidden_size=4096, intermediate_size=14336, num_attention_heads=32,
                      num_key_value_heads=8, head_dim=128)
    with torch.device("meta"):
        return LlamaDecoderLayer(cfg, layer_idx=0)


def test_layout_of_llama3_8b_layer_matches_closed_form_table():
    layer = _llama_layer()
    lay = oracle.layer_layout((n, tuple(p.shape)) for n, p in layer.named_parameters())
    assert [(n, o, k) for n, o, _, k in lay] == oracle.LLAMA3_8B_LAYER_TABLE
    assert lay[-1][1] + lay[-1][3] == 218_112_000


def test_layout_flat_equals_cat_of_parameters():
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer

    cfg = LlamaConfig(hidden_size=64, intermediate_size=96, num_attention_heads=4, num_key_value_heads=2)
    layer = LlamaDecoderLayer(cfg, layer_idx=0)
    lay = oracle.layer_layout((n, tuple(p.shape)) for n, p in layer.named_parameters())
    flat = torch.cat([p.detach().flatten() for p in layer.parameters()])
    params = dict(layer.named_parameters())
    for name, off, shape, n in lay:
        assert torch.equal(flat[off:off + n].view(shape), params[name].detach())


# ---------------------------------------------------------------- Adam
def _run_adam_case(d, name, update_fn):
    sizes = [int(s) for s in d["sizes"]]
    adamw, wd, bc, lr, eps, nsteps = d[f"{name}/meta"]
    betas = d[f"{name}/betas"]
    p = d[f"{name}/p0"].copy()
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    opt = oracle.OracleAdam(lr, tuple(betas[0]), eps, wd, bool(adamw))
    for step in range(1, int(nsteps) + 1):
        g = oracle.widen_bf16(d[f"{name}/g{step}"])
        off = 0
        for n in sizes:
            sl = slice(off, off + n)
            pp, mm, vv = p[sl].copy(), m[sl].copy(), v[sl].copy()
            update_fn(opt, step, float(lr), float(betas[step - 1][0]), float(betas[step - 1][1]), float(eps),
                      float(wd), bool(bc), pp, np.ascontiguousarray(g[sl]), mm, vv)
            p[sl], m[sl], v[sl] = pp, mm, vv
            off += n
        yield step, p, m, v


@pytest.mark.parametrize("name", ["adamw", "l2", "nobc"])
def test_oracle_adam_matches_reference_fixture(name):
    d = np.load(os.path.join(GOLDEN, "adam_ref.npz"))
    for step, p, m, v in _run_adam_case(d, name, lambda o, *a: o.update(*a)):
        for arr, key in ((p, "p"), (m, "m"), (v, "v")):
            exp = d[f"{name}/{key}{step}"]
            assert np.array_equal(arr.view(np.uint32), exp.view(np.uint32)), f"{name} step {step} {key}"


def test_adam_fixture_catches_dropped_bias_correction():
    # planted mistake: bias correction off must not match the fixture
    d = np.load(os.path.join(GOLDEN, "adam_ref.npz"))

    def wrong(o, step, lr, b1, b2, eps, wd, bc, p, g, m, v):
        o.update(step, lr, b1, b2, eps, wd, False, p, g, m, v)

    step, p, m, v = next(_run_adam_case(d, "adamw", wrong))
    assert not np.array_equal(p, d["adamw/p1"])


def test_adam_first_step_closed_form():
    # t = 1, no decay: m = (1-b1) g, v = (1-b2) g^2, p -= lr * m / (bc1 * (sqrt(v) / sqrt(bc2') + eps))
    rng = np.random.default_rng(3)
    n = 1024 + 7
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    p0 = p.copy()
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    lr, b1, b2, eps = 1e-3, 0.9, 0.999, 1e-8
    opt = oracle.OracleAdam(lr, (b1, b2), eps, 0.0, True)
    opt.update(1, lr, b1, b2, eps, 0.0, True, p, g, m, v)
    f32 = np.float32
    b1m1, b2m1 = float(f32(1) - f32(b1)), float(f32(1) - f32(b2))  # the float32 constants
    bc1, bc2 = b1m1, 1 / np.sqrt(b2m1)
    m_exp = b1m1 * g.astype(np.float64)
    v_exp = b2m1 * g.astype(np.float64) ** 2
    p_exp = p0 - lr / bc1 * m_exp / (np.sqrt(v_exp) * bc2 + eps)
    np.testing.assert_allclose(m, m_exp, rtol=6e-8)
    np.testing.assert_allclose(v, v_exp, rtol=1.2e-7)
    np.testing.assert_allclose(p, p_exp, rtol=1.2e-7, atol=1e-9)  # one float32 rounding of p
    # at t = 1 the step is lr * sign(g), up to eps / |g|
    big = np.abs(g) > 1e-4
    assert np.all(np.abs((p0 - p) - lr * np.sign(g))[big] < 2e-7)


def test_adam_tracks_torch_adamw():
    rng = np.random.default_rng(5)
    n = 4096 + 3
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    pt = torch.nn.Parameter(torch.from_numpy(p.copy()))
    topt = torch.optim.AdamW([pt], lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    opt = oracle.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    for step in range(1, 11):
        g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
        pt.grad = torch.from_numpy(g.copy())
        topt.step()
        opt.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, p, g, m, v)
    np.testing.assert_allclose(p, pt.detach().numpy(), rtol=0, atol=5e-7)


def test_oracle_adam_matches_compiled_reference_live():
    ref = load_ref_adam()
    if ref is None:
        pytest.skip("reference CPU Adam not built here (needs the reference sources)")
    rng = np.random.default_rng(11)
    sizes = [1000, 33, 4096, 5, 128]
    ps = [(rng.standard_normal(n) * 0.02).astype(np.float32) for n in sizes]
    tp = [torch.from_numpy(p.copy()) for p in ps]
    ms = [np.zeros(n, np.float32) for n in sizes]
    vs = [np.zeros(n, np.float32) for n in sizes]
    tm = [torch.zeros(n) for n in sizes]
    tv = [torch.zeros(n) for n in sizes]
    ref.create_adam(3, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, False)
    opt = oracle.OracleAdam(1e-5, (0.9, 0.999), 1e-8, 0.01, True)
    for step in range(1, 25):
        for i, n in enumerate(sizes):
            g = torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32)).bfloat16().float()
            ref.adam_update(3, step, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, tp[i], g, tm[i], tv[i])
            opt.update(step, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, ps[i], g.numpy().copy(), ms[i], vs[i])
            assert np.array_equal(ps[i].view(np.uint32), tp[i].numpy().view(np.uint32)), (step, i)
            assert np.array_equal(vs[i].view(np.uint32), tv[i].numpy().view(np.uint32)), (step, i)
    ref.destroy_adam(3)


# ---------------------------------------------------------------- schedule
def test_step_schedule_shape():
    s = oracle.step_schedule(4)
    h2d = [e for e in s if e[0] == "h2d"]
    d2h = [e[1] for e in s if e[0] == "d2h"]
    assert d2h == [5, 4, 3, 2, 1, 0]                       # every unit offloads once, in reverse
    assert [e[1] for e in h2d[:6]] == [0, 1, 2, 3, 4, 5]   # forward loads in order
    assert ("h2d", 5, True) in s                           # output unit loads with grads
    assert [e[1] for e in h2d[6:]] == [3, 2, 1, 0]         # backward reloads all but last decoder/output
    assert [e[1] for e in s if e[0] == "act_d2h"] == [1, 2, 3]
    assert [e[1] for e in s if e[0] == "act_h2d"] == [3, 2, 1]
