"""Write the golden fixtures under tests/golden (run from the repo root).

    python tests/golden/make_golden.py

cast_f32_bf16.npz
    Inputs: seeded N(0, 0.02) fp32 values plus special bit patterns (signed
    zeros, infinities, NaNs with several payloads, denormals, round-to-even
    ties, the values either side of the bf16 overflow boundary).
    Expected: torch CPU ``x.to(torch.bfloat16)``, the routine the reference's
    host cast calls (layer_state.py:301).
adam_ref.npz
    The reference's own CPU Adam (optimizer/layer_adam/csrc, compiled from
    its sources into oracle/_ref by oracle/Makefile), driven like
    LayerAdam.step_with_grad_views: one optimizer id, several tensors per
    step with sizes that exercise the vector body and the n % 16 scalar tail,
    bf16 grads widened with .float(), AdamW with weight decay, a change of
    betas, an L2 (adamw_mode=False) optimizer and bias_correction=False.
    Needs oracle/_ref/cpu_adam_ref.so (built only where the reference
    sources exist).
"""

import importlib.util
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))


def special_f32_bits() -> np.ndarray:
    pats = [
        0x00000000, 0x80000000,              # +0, -0
        0x7F800000, 0xFF800000,              # +inf, -inf
        0x7FC00000, 0xFFC00000, 0x7F800001, 0x7FBFFFFF, 0xFF812345,  # NaNs
        0x00000001, 0x807FFFFF, 0x00008000, 0x00018000, 0x0000FFFF,  # denormals
        0x3F808000, 0x3F818000, 0x3F80FFFF, 0x3F807FFF,              # ties / near ties
        0x7F7F7FFF, 0x7F7F8000, 0x7F7FFFFF, 0xFF7FFFFF,              # overflow boundary
        0x3F800000, 0xBF800000, 0x3E4CCCCD, 0x33D6BF95,              # 1, -1, 0.2, 1e-7
    ]
    return np.array(pats, dtype=np.uint32)


def make_cast() -> None:
    g = torch.Generator().manual_seed(42)
    x = (torch.randn(4093, generator=g) * 0.02).numpy().view(np.uint32)
    # every rounding situation of the low half-word, on a few exponents
    lo = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF], dtype=np.uint32)
    hi = np.array([0x3F80, 0x3F81, 0xBC23, 0x0080, 0x7F7F], dtype=np.uint32)
    grid = (hi[:, None] << 16 | lo[None, :]).reshape(-1)
    bits = np.concatenate([special_f32_bits(), grid, x])
    t = torch.from_numpy(bits.view(np.float32).copy())
    out = t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.savez_compressed(os.path.join(HERE, "cast_f32_bf16.npz"), x_bits=bits, bf16_bits=out)
    print("cast_f32_bf16.npz:", bits.size, "values")


def load_ref():
    path = os.path.join(ROOT, "oracle", "_ref", "cpu_adam_ref.so")
    if not os.path.exists(path):
        sys.exit(f"{path} missing: build it with `make -C oracle ref`")
    spec = importlib.util.spec_from_file_location("cpu_adam_ref", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def make_adam() -> None:
    ref = load_ref()
    g = torch.Generator().manual_seed(7)
    sizes = [257, 777, 16, 129]
    cases = {
        # name: (adamw_mode, weight_decay, bias_correction, betas per step)
        "adamw": (True, 0.01, True, [(0.9, 0.999)] * 3 + [(0.8, 0.99)] * 3),
        "l2": (False, 0.01, True, [(0.9, 0.999)] * 4),
        "nobc": (True, 0.0, False, [(0.9, 0.999)] * 3),
    }
    arrays = {"sizes": np.array(sizes)}
    for case_id, (name, (adamw, wd, bc, betas)) in enumerate(cases.items()):
        oid = 10 + case_id
        lr, eps = 1e-3, 1e-8
        ref.create_adam(oid, lr, betas[0][0], betas[0][1], eps, wd, adamw, False)
        ps = [torch.randn(n, generator=g) * 0.02 for n in sizes]
        ms = [torch.zeros(n) for n in sizes]
        vs = [torch.zeros(n) for n in sizes]
        arrays[f"{name}/p0"] = torch.cat(ps).numpy().copy()
        for step, (b1, b2) in enumerate(betas, start=1):
            gs = [(torch.randn(n, generator=g) * 1e-3).bfloat16() for n in sizes]
            arrays[f"{name}/g{step}"] = torch.cat(gs).view(torch.int16).numpy().view(np.uint16).copy()
            for p, gg, m, v in zip(ps, gs, ms, vs):
                ref.adam_update(oid, step, lr, b1, b2, eps, wd, bc, p, gg.float(), m, v)
            arrays[f"{name}/p{step}"] = torch.cat(ps).numpy().copy()
            arrays[f"{name}/m{step}"] = torch.cat(ms).numpy().copy()
            arrays[f"{name}/v{step}"] = torch.cat(vs).numpy().copy()
        arrays[f"{name}/meta"] = np.array([1.0 if adamw else 0.0, wd, 1.0 if bc else 0.0, lr, eps, len(betas)])
        arrays[f"{name}/betas"] = np.array(betas, dtype=np.float64)
        ref.destroy_adam(oid)
    np.savez_compressed(os.path.join(HERE, "adam_ref.npz"), **arrays)
    print("adam_ref.npz:", ", ".join(cases))


if __name__ == "__main__":
    make_cast()
    make_adam()
