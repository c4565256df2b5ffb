"""The product's host AdamW (libsf_cpu.so) and the LayerAdam drop-in, against
the oracle and the reference fixtures, bit for bit."""

import os

import numpy as np
import pytest
import torch

import oracle
from conftest import GOLDEN, load_ref_adam
from test1_amd.optimizer import LayerAdam, cpu_adam


@pytest.fixture(autouse=True)
def _threads():
    cpu_adam.set_num_threads(4)
    yield
    cpu_adam.set_num_threads(0)


@pytest.mark.parametrize("name", ["adamw", "l2", "nobc"])
@pytest.mark.parametrize("grad_dtype", [torch.float32, torch.bfloat16])
def test_adam_update_matches_reference_fixture(name, grad_dtype):
    d = np.load(os.path.join(GOLDEN, "adam_ref.npz"))
    sizes = [int(s) for s in d["sizes"]]
    adamw, wd, bc, lr, eps, nsteps = d[f"{name}/meta"]
    betas = d[f"{name}/betas"]
    oid = 40 + ["adamw", "l2", "nobc"].index(name)
    cpu_adam.create_adam(oid, float(lr), float(betas[0][0]), float(betas[0][1]), float(eps), float(wd), bool(adamw))
    p = torch.from_numpy(d[f"{name}/p0"].copy())
    m = torch.zeros_like(p)
    v = torch.zeros_like(p)
    for step in range(1, int(nsteps) + 1):
        g16 = torch.from_numpy(d[f"{name}/g{step}"].view(np.int16).copy()).view(torch.bfloat16)
        g = g16 if grad_dtype == torch.bfloat16 else g16.float()
        off = 0
        for n in sizes:
            sl = slice(off, off + n)
            cpu_adam.adam_update(oid, step, float(lr), float(betas[step - 1][0]), float(betas[step - 1][1]),
                                 float(eps), float(wd), bool(bc), p[sl], g[sl], m[sl], v[sl])
            off += n
        for t, key in ((p, "p"), (m, "m"), (v, "v")):
            assert np.array_equal(t.numpy().view(np.uint32), d[f"{name}/{key}{step}"].view(np.uint32)), (step, key)
    cpu_adam.destroy_adam(oid)


def test_stateless_step_matches_oracle_on_large_tensor():
    # large enough for many threads, with a ragged tail, bf16 grads
    rng = np.random.default_rng(1)
    n = 3_000_017
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    g = torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32)).bfloat16()
    tp, tm, tv = torch.from_numpy(p.copy()), torch.zeros(n), torch.zeros(n)
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    cpu_adam.create_adam(50, 1e-5, 0.9, 0.999, 1e-8, 0.01, True)
    opt = oracle.OracleAdam(1e-5, (0.9, 0.999), 1e-8, 0.01, True)
    for step in (1, 2, 3):
        cpu_adam.adam_update(50, step, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, tp, g, tm, tv)
        opt.update(step, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, p, g.float().numpy().copy(), m, v)
    assert np.array_equal(tp.numpy().view(np.uint32), p.view(np.uint32))
    assert np.array_equal(tv.numpy().view(np.uint32), v.view(np.uint32))
    cpu_adam.destroy_adam(50)


def test_fp16_grads_match_the_oracle_on_widened_grads():
    """float16 units: fp16 gradients read directly give the bits of the update
    on ``grad.float()`` (reference layer_adam.py:404), including subnormal
    and large fp16 values, over a vector body and a ragged tail."""
    rng = np.random.default_rng(2)
    n = 1_000_003
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    g32 = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    g32[:64] = np.array([2.0 ** -24, -(2.0 ** -20), 6e-8, 65504.0, -1000.0, 0.0, -0.0, 1e-7] * 8, np.float32)
    g = torch.from_numpy(g32).half()
    tp, tm, tv = torch.from_numpy(p.copy()), torch.zeros(n), torch.zeros(n)
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    cpu_adam.create_adam(51, 1e-5, 0.9, 0.999, 1e-8, 0.01, True)
    opt = oracle.OracleAdam(1e-5, (0.9, 0.999), 1e-8, 0.01, True)
    for step in (1, 2, 3):
        cpu_adam.adam_update(51, step, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, tp, g, tm, tv)
        widened = oracle.widen_f16(g.view(torch.int16).numpy().view(np.uint16))
        opt.update(step, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, p, widened, m, v)
    assert np.array_equal(tp.numpy().view(np.uint32), p.view(np.uint32))
    assert np.array_equal(tm.numpy().view(np.uint32), m.view(np.uint32))
    assert np.array_equal(tv.numpy().view(np.uint32), v.view(np.uint32))
    cpu_adam.destroy_adam(51)


def test_adam_update_errors_like_reference():
    cpu_adam.create_adam(60, 1e-3)
    p = torch.zeros(8)
    with pytest.raises(RuntimeError, match="not supported"):
        cpu_adam.adam_update(60, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, True, p.half(), p.half(), p, p.clone())
    with pytest.raises(RuntimeError, match="unknown optimizer"):
        cpu_adam.adam_update(12345, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, True, p, p.clone(), p.clone(), p.clone())
    with pytest.raises(ValueError, match="contiguous"):
        q = torch.zeros(8, 2)[:, 0]
        cpu_adam.adam_update(60, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, True, q, q.clone(), q.clone(), q.clone())
    cpu_adam.destroy_adam(60)


def _layer_params(rng, shapes):
    return [torch.nn.Parameter(torch.from_numpy((rng.standard_normal(s) * 0.02).astype(np.float32)))
            for s in shapes]


def test_layer_adam_step_with_grad_views_matches_oracle():
    """LayerAdam driven like the runtime (one unit at a time, bf16 grad views into
    a flat staging buffer) against LayerAdamOracle (reference layer_adam.py:358-425)."""
    rng = np.random.default_rng(2)
    units = [[(64, 32), (32,)], [(128, 64), (64, 64), (64,)], [(100,), (7, 3)]]
    params = [_layer_params(rng, u) for u in units]
    ref_params = [[p.detach().numpy().copy() for p in u] for u in params]
    opt = LayerAdam(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    orc = oracle.LayerAdamOracle(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    for i, u in enumerate(params):
        assert opt.add_layer_params(i, u) == i
        orc.add_layer(ref_params[i])
    for _ in range(3):
        for i in reversed(range(len(units))):  # backward order, as the runtime
            flat = torch.from_numpy((rng.standard_normal(sum(p.numel() for p in params[i])) * 1e-3)
                                    .astype(np.float32)).bfloat16()
            views, off = {}, 0
            for p in params[i]:
                views[p] = flat[off:off + p.numel()].view(p.shape)
                off += p.numel()
            opt.step_with_grad_views(i, views)
            orc.step_layer(i, [views[p].view(torch.int16).numpy().view(np.uint16) for p in params[i]])
    for u, ru in zip(params, ref_params):
        for p, rp in zip(u, ru):
            assert np.array_equal(p.detach().numpy().view(np.uint32), rp.view(np.uint32))


def test_layer_adam_matches_compiled_reference_driven_identically():
    ref = load_ref_adam()
    if ref is None:
        pytest.skip("reference CPU Adam not built here")
    rng = np.random.default_rng(4)
    units = [[(33, 17), (17,)], [(64, 64), (64,)]]
    params = [_layer_params(rng, u) for u in units]
    rparams = [[p.detach().clone() for p in u] for u in params]
    rstate = [[(torch.zeros(p.shape), torch.zeros(p.shape)) for p in u] for u in params]
    opt = LayerAdam(lr=1e-4, weight_decay=0.01)
    for i, u in enumerate(params):
        opt.add_layer_params(i, u)
    ref.create_adam(0, 1e-4, 0.9, 0.999, 1e-8, 0.01, True, False)
    steps = [0, 0]
    for _ in range(4):
        for i in (1, 0):
            steps[i] += 1
            grads = [torch.from_numpy((rng.standard_normal(p.shape) * 1e-3).astype(np.float32)).bfloat16()
                     for p in params[i]]
            opt.step_with_grad_views(i, dict(zip(params[i], grads)))
            for rp, g, (m, v) in zip(rparams[i], grads, rstate[i]):
                ref.adam_update(0, steps[i], 1e-4, 0.9, 0.999, 1e-8, 0.01, True, rp, g.float(), m, v)
    for u, ru in zip(params, rparams):
        for p, rp in zip(u, ru):
            assert torch.equal(p.detach().view(torch.int32), rp.view(torch.int32))


def test_adam_update_writes_rounded_bf16_copy():
    # The fused bf16 output leaves p/m/v unchanged and equals the cast of the
    # updated params; ragged tail (n % 16 != 0) and one non-finite value.
    rng = np.random.default_rng(2)
    n = 2_000_003
    p0 = torch.from_numpy((rng.standard_normal(n) * 0.02).astype(np.float32))
    g = torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32)).bfloat16()
    g[n - 2] = float("nan")
    runs = []
    for with_copy in (False, True):
        p, m, v = p0.clone(), torch.zeros(n), torch.zeros(n)
        pb = torch.empty(n, dtype=torch.bfloat16) if with_copy else None
        cpu_adam.create_adam(70, 1e-5, 0.9, 0.999, 1e-8, 0.01, True)
        for step in (1, 2):
            cpu_adam.adam_update(70, step, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, p, g, m, v, params_bf16=pb)
        cpu_adam.destroy_adam(70)
        runs.append((p, m, v, pb))
    for a, b in zip(runs[0][:3], runs[1][:3]):
        assert np.array_equal(a.numpy().view(np.uint32), b.numpy().view(np.uint32))
    p, pb = runs[1][0], runs[1][3]
    assert np.isnan(p[n - 2].item())
    assert np.array_equal(pb.view(torch.int16).numpy().view(np.uint16), oracle.cast_f32_bf16(p.numpy()))


def test_host_cast_matches_golden():
    d = np.load(os.path.join(GOLDEN, "cast_f32_bf16.npz"))
    x = torch.from_numpy(d["x_bits"].view(np.float32).copy())
    out = torch.empty(x.numel(), dtype=torch.bfloat16)
    cpu_adam.cast_f32_bf16(x, out)
    assert np.array_equal(out.view(torch.int16).numpy().view(np.uint16), d["bf16_bits"])
    with pytest.raises(ValueError, match="same size"):
        cpu_adam.cast_f32_bf16(x, out[:-1])
    with pytest.raises(ValueError, match="params_bf16"):
        cpu_adam.create_adam(71, 1e-3)
        try:
            q = torch.zeros(8)
            cpu_adam.adam_update(71, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, True, q, q.clone(), q.clone(), q.clone(),
                                 params_bf16=torch.empty(8))
        finally:
            cpu_adam.destroy_adam(71)


@pytest.mark.parametrize("grad_dtype", [torch.float32, torch.bfloat16])
def test_row_sparse_update_equals_dense_update(grad_dtype):
    # A [V, H] table whose gradient is zero outside a few rows: the row-sparse
    # update gives the dense update's bits for params, moments and the bf16
    # copy, over three steps (the bias-correction state advances the same way).
    rng = np.random.default_rng(3)
    V, H = 1000, 64
    p0 = torch.from_numpy((rng.standard_normal((V, H)) * 0.02).astype(np.float32))
    dense = [p0.clone(), torch.zeros(V, H), torch.zeros(V, H), torch.empty(V, H, dtype=torch.bfloat16)]
    sparse = [p0.clone(), torch.zeros(V, H), torch.zeros(V, H), torch.empty(V, H, dtype=torch.bfloat16)]
    cpu_adam.create_adam(80, 1e-3, 0.9, 0.999, 1e-8, 0.01, True)
    cpu_adam.create_adam(81, 1e-3, 0.9, 0.999, 1e-8, 0.01, True)
    for step in (1, 2, 3):
        ids = torch.from_numpy(rng.integers(0, V, 37))  # with repeats
        rows = torch.from_numpy((rng.standard_normal((37, H)) * 1e-3).astype(np.float32)).to(grad_dtype)
        # repeated ids carry the same (summed) row, as gathered from a dense grad
        first = {}
        for k, r in enumerate(ids.tolist()):
            first.setdefault(r, k)
        for k, r in enumerate(ids.tolist()):
            rows[k] = rows[first[r]]
        g = torch.zeros(V, H, dtype=grad_dtype)
        g[ids] = rows
        cpu_adam.adam_update(80, step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, dense[0], g, dense[1], dense[2],
                             params_bf16=dense[3])
        row_slot = torch.full((V,), -1, dtype=torch.int64)
        row_slot[ids] = torch.arange(37)
        cpu_adam.adam_update_rows(81, step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, sparse[0], sparse[1], sparse[2],
                                  row_slot, rows, params_bf16=sparse[3])
        for a, b in zip(dense, sparse):
            assert torch.equal(a.view(torch.int16 if a.dtype == torch.bfloat16 else torch.int32),
                               b.view(torch.int16 if b.dtype == torch.bfloat16 else torch.int32)), step
    cpu_adam.destroy_adam(80)
    cpu_adam.destroy_adam(81)


def test_row_sparse_update_rejects_bad_shapes():
    cpu_adam.create_adam(82, 1e-3)
    p, m, v = torch.zeros(4, 24), torch.zeros(4, 24), torch.zeros(4, 24)
    slot = torch.tensor([0, -1, -1, -1])
    with pytest.raises(RuntimeError, match="failed"):  # row length not a multiple of 16
        cpu_adam.adam_update_rows(82, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, True, p, m, v, slot, torch.zeros(1, 24))
    p, m, v = torch.zeros(4, 32), torch.zeros(4, 32), torch.zeros(4, 32)
    with pytest.raises(RuntimeError, match="failed"):  # a slot beyond the gradient rows
        cpu_adam.adam_update_rows(82, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, True, p, m, v,
                                  torch.tensor([0, 1, -1, -1]), torch.zeros(1, 32))
    cpu_adam.destroy_adam(82)


def _run_layer_adam(order_fn, reference_order, steps=6, seed=3, piece_elems=None, calls=None, early=False):
    """Units 0 (a [64, 32] table, row-sparse updates) and 1..4 (several
    params each), stepped ``steps`` times in the order ``order_fn(step)``.
    With ``piece_elems``, units 1..4 are updated in pieces of that size (the
    runtime's split), and ``calls`` collects the piece callbacks."""
    g = torch.Generator().manual_seed(seed)
    shapes = {1: [(48, 32), (32,)], 2: [(40, 16), (16,), (16,)], 3: [(33, 7)], 4: [(64, 16), (64,)]}
    units = {0: [torch.nn.Parameter(torch.randn(64, 32, generator=g) * 0.02)]}
    for u, shp in shapes.items():
        units[u] = [torch.nn.Parameter(torch.randn(s, generator=g) * 0.02) for s in shp]
    opt = LayerAdam(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, num_layer=5)
    opt.reference_order = reference_order
    for u in sorted(units):
        opt.add_layer_params(u, units[u])
    gg = torch.Generator().manual_seed(seed + 1)
    for step in range(steps):
        grads = {u: [(torch.randn(p.shape, generator=gg) * 1e-3).bfloat16() for p in units[u]] for u in units}
        ids = torch.randperm(64, generator=gg)[:9]
        for u in order_fn(step):
            if u == 0 and early:
                # the gradient-free rows first, the batch's rows once their gradient is there
                untouched = torch.full((64,), -1, dtype=torch.int64)
                untouched[ids] = -2
                opt.step_rows_early(0, untouched, units[0][0].data)
                row_slot = torch.full((64,), -2, dtype=torch.int64)
                row_slot[ids] = torch.arange(ids.numel())
                opt.step_rows(0, row_slot, grads[0][0][ids].contiguous(), units[0][0].data)
            elif u == 0:
                row_slot = torch.full((64,), -1, dtype=torch.int64)
                row_slot[ids] = torch.arange(ids.numel())
                opt.step_rows(0, row_slot, grads[0][0][ids].contiguous(), units[0][0].data)
            elif piece_elems is None:
                opt.step_with_grad_views(u, dict(zip(units[u], grads[u])))
            else:
                pieces = _pieces_of(units[u], piece_elems)
                log = []
                opt.step_with_grad_views(u, dict(zip(units[u], grads[u])), pieces=pieces,
                                         before_piece=lambda j: log.append(("before", j)),
                                         after_piece=lambda j: log.append(("after", j)))
                if calls is not None:
                    calls.append((u, len(pieces), log))
    return units, opt


def _pieces_of(params, piece_elems):
    from test1_amd.layer_state import overlap_ranges, split_into_pieces

    sizes = [p.numel() for p in params]
    offs = [sum(sizes[:i]) for i in range(len(sizes))]
    spans = list(zip(offs, sizes))
    return [[(params[i], lo, hi) for i, lo, hi in overlap_ranges(spans, a, b)]
            for a, b in split_into_pieces(sizes, piece_elems)]


def test_reference_order_scalars_give_the_reference_bits_in_any_order():
    """LayerAdam updates units in the reference's order (last unit first)
    through the stateful native update, pinned against the reference's
    compiled cpu_adam above.  With ``reference_order`` the same updates in
    shuffled orders give the same bits over 6 steps (beta2^t by product and
    by pow differ at t = 3, 4 and 6, so the first call of those steps is
    checked), while the stateful update in a shuffled order does not."""
    import random

    descending = lambda step: [4, 3, 2, 1, 0]  # noqa: E731
    rng = random.Random(7)
    orders = {s: rng.sample(range(5), 5) for s in range(6)}
    assert any(o[0] != 4 for o in orders.values())
    ref_units, _ = _run_layer_adam(descending, reference_order=False)
    got_units, _ = _run_layer_adam(lambda s: orders[s], reference_order=True)
    same_order, _ = _run_layer_adam(descending, reference_order=True)
    stateful_shuffled, _ = _run_layer_adam(lambda s: orders[s], reference_order=False)
    differs = False
    for u in ref_units:
        for a, b, c, d in zip(ref_units[u], got_units[u], same_order[u], stateful_shuffled[u]):
            ai = a.data.view(torch.int32)
            assert torch.equal(ai, b.data.view(torch.int32)), f"unit {u}"
            assert torch.equal(ai, c.data.view(torch.int32)), f"unit {u}"
            differs |= not torch.equal(ai, d.data.view(torch.int32))
    assert differs, "the stateful update should depend on the call order"


def test_split_into_pieces_covers_the_layout_on_vector_boundaries():
    """The runtime's piece split: contiguous cover of [0, total), at most
    piece_elems + 15 per piece, and every boundary inside a tensor a multiple
    of 16 elements after that tensor's start (zero-size and tiny tensors,
    one tensor larger than several pieces)."""
    import random

    from test1_amd.layer_state import split_into_pieces

    rng = random.Random(11)
    cases = [([4096, 16777216, 4194304, 4194304, 16777216, 58720256, 58720256, 58720256, 4096], 1 << 26),
             ([525336576, 4096], 1 << 26), ([231], 64), ([0, 5, 0, 1000, 17], 100), ([10], 0), ([], 64)]
    cases += [([rng.choice([0, 1, 7, 16, 33, rng.randrange(1, 5000)]) for _ in range(rng.randrange(1, 9))],
               rng.choice([16, 48, 100, 1000])) for _ in range(200)]
    for sizes, pe in cases:
        total = sum(sizes)
        pieces = split_into_pieces(sizes, pe)
        if total == 0:
            assert pieces == []
            continue
        assert pieces[0][0] == 0 and pieces[-1][1] == total
        assert all(b > a for a, b in pieces) and all(pieces[k][1] == pieces[k + 1][0] for k in range(len(pieces) - 1))
        if pe > 0:
            assert max(b - a for a, b in pieces) <= pe + 15
            assert len(pieces) <= -(-total // pe)
        else:
            assert len(pieces) == 1
        starts = [sum(sizes[:i]) for i in range(len(sizes))]
        for a, _ in pieces[1:]:
            inside = [o for o, n in zip(starts, sizes) if o < a < o + n]
            assert all((a - o) % 16 == 0 for o in inside), (sizes, pe, a)


def test_piecewise_update_gives_the_reference_bits():
    """A unit updated piece by piece (as the runtime overlaps its gradient
    copies and its staging with the update) gives the bits of the whole-unit
    update pinned against the reference's compiled cpu_adam above, with the
    reference's first-of-step scalars, over 6 steps; the callbacks run
    before and after each piece in order.  Pieces of 48 and 100 elements
    cut every multi-piece parameter in its vector body and leave the odd
    tails (33 x 7 = 231 elements: tail 7) at the parameter's end."""
    descending = lambda step: [4, 3, 2, 1, 0]  # noqa: E731
    ref_units, ref_opt = _run_layer_adam(descending, reference_order=False)
    for pe in (48, 100, 1 << 20):
        calls = []
        got_units, got_opt = _run_layer_adam(descending, reference_order=True, piece_elems=pe, calls=calls)
        assert any(n > 1 for _, n, _ in calls) == (pe < 1000)
        for _, n, log in calls:
            assert log == [(k, j) for j in range(n) for k in ("before", "after")]
        for u in ref_units:
            for a, b in zip(ref_units[u], got_units[u]):
                assert torch.equal(a.data.view(torch.int32), b.data.view(torch.int32)), (pe, u)
                sa, sb = ref_opt.state[a], got_opt.state[b]
                for k in ("exp_avg", "exp_avg_sq"):
                    assert torch.equal(sa[k].view(torch.int32), sb[k].view(torch.int32)), (pe, u, k)


def test_piecewise_update_rejects_ranges_off_the_vector_boundary():
    """A piece split inside a parameter at a position that is not a multiple
    of 16 would change which elements take the scalar tail: refused."""
    p = torch.nn.Parameter(torch.zeros(100))
    opt = LayerAdam(lr=1e-3, num_layer=1)
    opt.reference_order = True
    opt.add_layer_params(0, [p])
    g = torch.zeros(100, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="16-element boundary"):
        opt.step_with_grad_views(0, {p: g}, pieces=[[(p, 0, 40)], [(p, 40, 100)]])


def test_row_update_split_early_and_late_gives_the_reference_bits():
    """The embedding's update split in two: the rows the batch did not touch
    (zero gradient) first, the batch's rows once their gradient has landed.
    Over 6 steps, in the reference's order and in shuffled orders, the table
    and its moments carry the bits of the whole update pinned against the
    reference's compiled cpu_adam above."""
    import random

    descending = lambda step: [4, 3, 2, 1, 0]  # noqa: E731
    rng = random.Random(5)
    orders = {s: rng.sample(range(5), 5) for s in range(6)}
    ref_units, ref_opt = _run_layer_adam(descending, reference_order=False)
    for order in (descending, lambda s: orders[s]):
        got_units, got_opt = _run_layer_adam(order, reference_order=True, early=True)
        for u in ref_units:
            for a, b in zip(ref_units[u], got_units[u]):
                assert torch.equal(a.data.view(torch.int32), b.data.view(torch.int32)), u
                for k in ("exp_avg", "exp_avg_sq"):
                    assert torch.equal(ref_opt.state[a][k].view(torch.int32), got_opt.state[b][k].view(torch.int32))
        assert got_opt._groups_by_layer[0]["step"] == 6 and not got_opt._early_rows


def test_row_update_skip_marker_and_invalid_markers():
    """``SF_ROW_SKIP`` rows are left exactly as they are, ``SF_ROW_ZERO``
    rows get the zero-gradient update, other negative markers are refused."""
    from test1_amd import _native

    g = torch.Generator().manual_seed(1)
    p = torch.randn(8, 16, generator=g) * 0.02
    m, v = torch.zeros(8, 16), torch.zeros(8, 16)
    p0 = p.clone()
    hp = cpu_adam.hparams_in_reference_order(1, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, True, False)
    slot = torch.tensor([_native.SF_ROW_SKIP, _native.SF_ROW_ZERO] * 4, dtype=torch.int64)
    cpu_adam.adam_step_rows(p, m, v, slot, torch.empty((0, 16), dtype=torch.bfloat16), hp)
    assert torch.equal(p[0::2], p0[0::2]) and not torch.equal(p[1::2], p0[1::2])
    with pytest.raises(RuntimeError):
        cpu_adam.adam_step_rows(p, m, v, torch.full((8,), -3, dtype=torch.int64),
                                torch.empty((0, 16), dtype=torch.bfloat16), hp)
