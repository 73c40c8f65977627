"""Pin the CPU oracle against what the mathematics, library routines and the reference's
own recorded data fix -- never against a retyped copy of its own formula."""
import ctypes
from fractions import Fraction
import json
import math
from pathlib import Path

import numpy as np
import pytest

from exact import HALF, SINGLE, half_value, round_fraction, to_half_bits

GOLDEN = Path(__file__).resolve().parent / 'golden'
LIBM = ctypes.CDLL('libm.so.6')
LIBM.fmaf.argtypes = [ctypes.c_float] * 3
LIBM.fmaf.restype = ctypes.c_float


# ---------------------------------------------------------------------------------------
# fp16 conversions and the fused fp16 multiply-add
# ---------------------------------------------------------------------------------------

def test_half_to_float_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    expected = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.h2f(b) for b in bits], dtype=np.float32)
    finite = np.isfinite(expected)
    assert np.array_equal(got[finite].view(np.uint32), expected[finite].view(np.uint32))
    assert np.isnan(got[~np.isfinite(expected) & np.isnan(expected)]).all()


def test_float_to_half_matches_numpy_at_midpoints(oracle):
    # every finite half, the exact midpoints between neighbours and one fp32 ulp either side
    halves = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (halves[:-1] + halves[1:]) / 2
    candidates = np.concatenate([halves, mids]).astype(np.float32)
    candidates = np.concatenate([candidates, np.nextafter(candidates, np.float32(np.inf)),
                                 np.nextafter(candidates, np.float32(0))])
    candidates = np.concatenate([candidates, -candidates, np.float32([65504, 65519.99, 65520, 1e6])])
    with np.errstate(over='ignore'):   # 65520 and 1e6 round to infinity on purpose
        expected = candidates.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f2h(v) for v in candidates], dtype=np.uint16)
    assert np.array_equal(got, expected)


def _exact_hfma(a, b, c):
    value = half_value(a) * half_value(b) + half_value(c)
    return round_fraction(value, HALF)


def test_hfma_against_exact_rationals(oracle):
    rng = np.random.default_rng(7)
    finite = np.arange(0, 0x7c00, dtype=np.uint16)
    finite = np.concatenate([finite, finite | 0x8000])
    triples = rng.choice(finite, size=(4000, 3))
    # products landing exactly on half midpoints, subnormal results, cancellation
    special = [(0x3c00, 0x0001, 0x0000), (0x3800, 0x0001, 0x0000), (0x3800, 0x0003, 0x0000),
               (0x3c01, 0x3c01, 0x0000), (0x3c00, 0x3c00, 0xbc00), (0x0400, 0x3800, 0x8001),
               (0x3bff, 0x0001, 0x0001), (0x7bff, 0x3c00, 0x7bff)]
    for a, b, c in list(map(tuple, triples)) + special:
        got = oracle.hfma(a, b, c)
        expected = _exact_hfma(a, b, c)
        if isinstance(expected, float):
            assert got in (0x7c00, 0xfc00) and (got == 0x7c00) == (expected > 0)
        else:
            assert half_value(got) == expected, (hex(a), hex(b), hex(c))


# ---------------------------------------------------------------------------------------
# Hash-grid geometry: reference-held layouts
# ---------------------------------------------------------------------------------------

def _goldens():
    return json.loads((GOLDEN / 'layout_goldens.json').read_text())


def test_grid_levels_match_reference_recorded_hashgrid_layout(oracle):
    hash_runs = [v for v in _goldens().values() if v['config'].get('representation') == 'hash_grid']
    assert hash_runs, 'expected HashGrid runs among the reference records'
    for run in hash_runs:
        config = run['config']
        rows, _ = oracle.grid_levels(config['hash_encoding'])
        assert [r[1] for r in rows] == config['resolutions']
        assert [r[2] for r in rows] == config['cell_caps']
        total = sum(r[2] for r in rows) * config['hash_encoding']['n_features_per_level']
        assert total + config['gate_parameters'] + config['decoder_parameters'] == config['allocated_parameters']


def test_grid_levels_single_expert_workload(oracle):
    rows, entries = oracle.grid_levels(dict(n_levels=16, base_resolution=16, log2_hashmap_size=19,
                                            per_level_scale=1.38))
    assert [r[1] for r in rows] == [16, 23, 31, 43, 59, 81, 111, 153, 211, 291, 401, 554, 764, 1054, 1454, 2006]
    assert [r[2] for r in rows][:12] == [256, 536, 968, 1856, 3488, 6568, 12328, 23416, 44528, 84688, 160808, 306920]
    assert [r[4] for r in rows] == [0] * 12 + [1] * 4
    assert entries == 2743512
    rows, entries = oracle.grid_levels(dict(n_levels=16, base_resolution=16, log2_hashmap_size=16,
                                            per_level_scale=1.38))
    assert entries == 552696 and [r[4] for r in rows] == [0] * 9 + [1] * 7


# ---------------------------------------------------------------------------------------
# Hash-grid encode: bilinear interpolation and Instant-NGP Eq. 4 indices
# ---------------------------------------------------------------------------------------

def _exact_corner(scale, x):
    """floor and fraction of fma(scale, x, 0.5) computed exactly (libm fmaf is correctly
    rounded; cross-checked against rational rounding)."""
    p = LIBM.fmaf(scale, x, 0.5)
    exact = round_fraction(Fraction(float(np.float32(scale))) * Fraction(float(np.float32(x))) + Fraction(1, 2), SINGLE)
    assert Fraction(float(np.float32(p))) == exact
    g = math.floor(p)
    return g, np.float32(p) - np.float32(g)


def test_dense_level_reproduces_linear_function(oracle):
    # table T[gx + gy*res] = gx + 1024*gy: bilinear interpolation returns px + 1024*py
    scale = np.float32(21.08)
    res, size = 23, 536
    rows = [(float(scale), res, size, 0, 0)]
    table = np.zeros(size, dtype=np.float32)
    for gy in range(res):
        for gx in range(res):
            if gx + gy * res < size:
                table[gx + gy * res] = gx + 1024 * gy
    rng = np.random.default_rng(3)
    xy = rng.uniform(0, (res - 2.0) / float(scale), size=(2000, 2)).astype(np.float32)
    out = oracle.hash_forward(xy, table, rows, 1)
    px = np.array([LIBM.fmaf(scale, x, 0.5) for x in xy[:, 0]], dtype=np.float64)
    py = np.array([LIBM.fmaf(scale, y, 0.5) for y in xy[:, 1]], dtype=np.float64)
    expected = px + 1024 * py
    assert np.allclose(out[:, 0], expected, rtol=0, atol=1024 * res * 2.0 ** -21)
    # swapping the axes must be visible
    assert not np.allclose(out[:, 0], py + 1024 * px, atol=1.0)


def test_hashed_level_indices_and_weights_brute_force(oracle):
    scale = np.float32(2005.1)
    res, size = 2007, 1 << 12
    rows = [(float(scale), res, size, 0, 1)]
    rng = np.random.default_rng(5)
    xy = rng.random((64, 2), dtype=np.float32)
    for i in range(len(xy)):
        upstream = np.ones((1, 1), dtype=np.float16)
        grad, _ = oracle.hash_backward(xy[i:i + 1], upstream, rows, 1, size)
        gx, fx = _exact_corner(scale, xy[i, 0])
        gy, fy = _exact_corner(scale, xy[i, 1])
        expected = np.zeros(size)
        weights = [(1 - fx) * (1 - fy), fx * (1 - fy), (1 - fx) * fy, fx * fy]
        for k in range(4):
            cx, cy = gx + (k & 1), gy + (k >> 1)
            index = ((cx * 1) ^ ((cy * 2654435761) % 2 ** 32)) % size
            expected[index] += float(np.float32(weights[k]))
        assert np.array_equal(grad, expected)


def test_fp16_chain_against_exact_rounding(oracle):
    rows = [(15.0, 16, 256, 0, 0), (21.08, 23, 536, 256, 0)]
    rng = np.random.default_rng(11)
    table = rng.normal(0, 0.3, size=(792, 2)).astype(np.float16)
    xy = rng.random((40, 2), dtype=np.float32)
    out = oracle.hash_forward(xy, table, rows, 2)
    for i in range(len(xy)):
        for level, (scale, res, size, offset, _) in enumerate(rows):
            gx, fx = _exact_corner(np.float32(scale), xy[i, 0])
            gy, fy = _exact_corner(np.float32(scale), xy[i, 1])
            weights = [np.float32((1 - fx) * (1 - fy)), np.float32(fx * (1 - fy)),
                       np.float32((1 - fx) * fy), np.float32(fx * fy)]
            for c in range(2):
                value = Fraction(0)
                for k in range(4):
                    index = ((gx + (k & 1)) + (gy + (k >> 1)) * res) % size
                    w16 = round_fraction(Fraction(float(weights[k])), HALF)
                    g16 = Fraction(float(table[offset + index, c]))
                    value = round_fraction(w16 * g16 + value, HALF)
                assert Fraction(float(out[i, level * 2 + c])) == value


def test_backward_is_adjoint_of_forward(oracle):
    rows, entries = oracle.grid_levels(dict(n_levels=6, base_resolution=4, log2_hashmap_size=8,
                                            per_level_scale=1.9))
    rng = np.random.default_rng(13)
    table = rng.normal(size=entries * 2).astype(np.float32)
    xy = rng.random((300, 2), dtype=np.float32)
    upstream = rng.normal(size=(300, 12)).astype(np.float32)
    forward = oracle.hash_forward(xy, table, rows, 2).astype(np.float64)
    grad, _ = oracle.hash_backward(xy, upstream, rows, 2, entries * 2)
    left = float((forward * upstream).sum())
    right = float((table.astype(np.float64) * grad).sum())
    assert abs(left - right) <= 1e-5 * (np.abs(forward * upstream).sum())


def test_expert_segments_equal_independent_grids(oracle):
    rows, entries = oracle.grid_levels(dict(n_levels=4, base_resolution=4, log2_hashmap_size=6,
                                            per_level_scale=2.0))
    rng = np.random.default_rng(17)
    experts, params = 3, entries * 2
    table = rng.normal(size=experts * params).astype(np.float16)
    offsets = np.array([0, 50, 50, 120])
    xy = rng.random((120, 2), dtype=np.float32)
    out = oracle.hash_forward(xy, table, rows, 2, offsets=offsets, expert_params=params)
    for e in range(experts):
        part = oracle.hash_forward(xy[offsets[e]:offsets[e + 1]], table[e * params:(e + 1) * params], rows, 2)
        assert np.array_equal(out[offsets[e]:offsets[e + 1]].view(np.uint16), part.view(np.uint16))


# ---------------------------------------------------------------------------------------
# Packed planes: direct layout == dense hash level at integer scale; rank addressing
# ---------------------------------------------------------------------------------------

def _layout(resolutions, supports, dims, caps):
    import torch
    from odie_amd.model import make_layout
    config = dict(resolutions=resolutions, n_levels=len(resolutions), representation='xy_planes', coarse_levels=0,
                  gate_topology='shared', gate_position='feature', initial_active_prefix=0)
    return make_layout(config, [torch.as_tensor(s) for s in supports], dims, caps)


def _numpy_layout(layout):
    return {k: layout[k].numpy() if hasattr(layout[k], 'numpy') else layout[k]
            for k in ('descriptors', 'node_bitmap', 'node_prefix', 'bitmap')}


def test_packed_direct_equals_dense_hash_level(oracle):
    import torch
    resolutions = [5, 9]
    supports = [np.ones(r * r, dtype=bool) for r in resolutions]
    caps = [32, 88]
    layout = _layout(resolutions, supports, [2, 2], caps)
    rng = np.random.default_rng(19)
    grid = rng.normal(0, 0.2, size=layout['params']).astype(np.float32)
    xy = rng.random((500, 2), dtype=np.float32)
    out, vis = oracle.packed_forward(xy, grid, _numpy_layout(layout), 4)
    assert vis.all()
    rows = [(float(r - 1), r, (r * r + 7) // 8 * 8, o, 0) for r, o in zip(resolutions, [0, 32])]
    dense = oracle.hash_forward(xy, grid.astype(np.float16), rows, 2)
    assert np.array_equal(out.view(np.uint16), dense.view(np.uint16))


def test_packed_rank_addressing_brute_force(oracle):
    import torch
    rng = np.random.default_rng(23)
    resolutions = [4, 12, 17]
    supports = [np.ones(16, dtype=bool), rng.random(144) < 0.3, rng.random(289) < 0.15]
    from odie_amd.model import plane_closure
    closures = [plane_closure(torch.as_tensor(s), r).numpy() for s, r in zip(supports, resolutions)]
    caps = [16, (len(closures[1]) + 7) // 8 * 8 + 8, (len(closures[2]) + 7) // 8 * 8]
    layout = _layout(resolutions, supports, [2, 1, 4], caps)
    grid = rng.normal(0, 0.2, size=layout['params']).astype(np.float32)
    xy = rng.random((800, 2), dtype=np.float32)
    out, vis = oracle.packed_forward(xy, grid, _numpy_layout(layout), 7)
    # brute force: expand each plane to a dense node table by searchsorted rank
    offset, dense_rows, dense_tables = 0, [], []
    for level, (r, nodes, dim) in enumerate(zip(resolutions, closures, [2, 1, 4])):
        points = (r * r + 7) // 8 * 8
        plane = np.zeros((points, dim), dtype=np.float32)
        base = layout['levels'][level]['plane_offset']
        plane[nodes] = grid[base:base + len(nodes) * dim].reshape(-1, dim)
        hashed = oracle.hash_forward(xy, plane.astype(np.float16).reshape(-1), [(float(r - 1), r, points, 0, 0)], dim)
        column = layout['levels'][level]['feature_offset']
        cells = oracle_cells(xy, r)
        visible = supports[level][cells]
        assert np.array_equal(vis[:, level], visible)
        expected = np.where(visible[:, None], hashed, np.float16(0))
        assert np.array_equal(out[:, column:column + dim].view(np.uint16), expected.view(np.uint16))


def oracle_cells(xy, r):
    px = np.array([LIBM.fmaf(np.float32(r - 1), x, 0.5) for x in xy[:, 0]])
    py = np.array([LIBM.fmaf(np.float32(r - 1), y, 0.5) for y in xy[:, 1]])
    return np.floor(px).astype(np.int64) + np.floor(py).astype(np.int64) * r


def test_packed_backward_is_adjoint(oracle):
    import torch
    rng = np.random.default_rng(29)
    resolutions = [6, 11]
    supports = [np.ones(36, dtype=bool), rng.random(121) < 0.4]
    from odie_amd.model import plane_closure
    caps = [40, (len(plane_closure(torch.as_tensor(supports[1]), 11)) + 7) // 8 * 8]
    layout = _layout(resolutions, supports, [2, 2], caps)
    grid = rng.normal(size=layout['params']).astype(np.float32).astype(np.float16).astype(np.float32)
    xy = rng.random((400, 2), dtype=np.float32)
    upstream = rng.normal(size=(400, 4)).astype(np.float16)
    grad, _ = oracle.packed_backward(xy, upstream, _numpy_layout(layout), layout['params'])
    out, _ = oracle.packed_forward(xy, grid, _numpy_layout(layout), 4)
    left = float((out.astype(np.float64) * upstream.astype(np.float64)).sum())
    right = float((grid.astype(np.float64) * grad).sum())
    scale = float(np.abs(out.astype(np.float64) * upstream.astype(np.float64)).sum())
    assert abs(left - right) <= 2e-3 * scale     # fp16 forward chain rounding


# ---------------------------------------------------------------------------------------
# Residual, thresholds, selection, ranking, compaction, Adam
# ---------------------------------------------------------------------------------------

def test_native_thresholds_are_exact_boundaries(oracle):
    for resolution in (2, 3, 8, 13, 128, 2048):
        thresholds = oracle.native_thresholds(resolution)
        for region, t in enumerate(thresholds, start=1):
            below = np.nextafter(np.float32(t), np.float32(0))
            assert math.floor(LIBM.fmaf(resolution - 1, t, 0.5)) >= region
            assert math.floor(LIBM.fmaf(resolution - 1, below, 0.5)) < region


def test_residual_matches_bincount_restatement(oracle):
    rng = np.random.default_rng(31)
    shape, resolution = (37, 53), 8
    prediction = rng.random((shape[0] * shape[1], 3), dtype=np.float32)
    target = rng.integers(0, 256, size=(shape[0] * shape[1], 3), dtype=np.uint8)
    thresholds = oracle.native_thresholds(resolution)
    xmap = np.searchsorted(thresholds, np.arange(shape[1], dtype=np.float32) / np.float32(shape[1] - 1), side='right')
    ymap = np.searchsorted(thresholds, np.arange(shape[0], dtype=np.float32) / np.float32(shape[0] - 1), side='right')
    xb = np.searchsorted(xmap, np.arange(resolution + 1)).astype(np.int32)
    yb = np.searchsorted(ymap, np.arange(resolution + 1)).astype(np.int32)
    totals = np.zeros(resolution ** 2)
    # streamed in uneven chunks, as the reference's residual pass runs
    for begin, end in ((0, 700), (700, 701), (701, shape[0] * shape[1])):
        oracle.residual(prediction[begin:end], target[begin:end], shape[1], resolution, xb, yb, begin=begin,
                        totals=totals)
    truth = target.astype(np.float32) / np.float32(255.0)
    squared = (prediction - truth) * (prediction - truth)
    per_pixel = squared.sum(axis=1, dtype=np.float64) / 3.0
    cells = oracle.pixel_cells(shape, resolution)
    expected = np.bincount(cells, weights=per_pixel, minlength=resolution ** 2)
    assert np.array_equal(totals, expected)


def _brute_greedy(scores, resolution, cap):
    cells, points = resolution ** 2, oracle_align8(resolution ** 2)
    selected = np.zeros(cells, dtype=bool)
    nodes = np.zeros(points, dtype=bool)
    used = 0
    order = []
    while True:
        cost = np.array([sum(not nodes[(c + d) % points] for d in (0, 1, resolution, resolution + 1))
                         for c in range(cells)])
        free = [c for c in range(cells) if not selected[c] and cost[c] == 0]
        if free:
            cell = min(free)
        else:
            best = None
            for k in range(1, min(4, cap - used) + 1):
                members = [c for c in range(cells) if not selected[c] and cost[c] == k]
                if not members:
                    continue
                top = max(members, key=lambda c: (scores[c], -c))
                if best is None:
                    best = (scores[top], k, top)
                    continue
                left, right = scores[top] * best[1], best[0] * k
                if left > right or (left == right and top < best[2]):
                    best = (scores[top], k, top)
            if best is None:
                break
            cell = best[2]
        selected[cell] = True
        for d in (0, 1, resolution, resolution + 1):
            if not nodes[(cell + d) % points]:
                nodes[(cell + d) % points] = True
                used += 1
        order.append(cell)
    return selected, nodes, order


def oracle_align8(value):
    return (value + 7) // 8 * 8


@pytest.mark.parametrize('resolution,cap,seed', [(3, 8, 0), (4, 16, 1), (5, 16, 2), (7, 32, 3), (9, 48, 4)])
def test_b2_greedy_matches_brute_force(oracle, resolution, cap, seed):
    rng = np.random.default_rng(seed)
    scores = rng.choice([0.0, 0.25, 0.5, 0.5, 1.0, 3.0], size=resolution ** 2)   # planted ties
    trace = []
    selected, nodes, iterations = oracle.select_benefit_cost(scores, resolution, cap, trace=trace)
    brute_selected, brute_nodes, order = _brute_greedy(scores, resolution, cap)
    assert np.array_equal(selected, brute_selected) and np.array_equal(nodes, brute_nodes)
    assert trace == order and iterations == len(order)
    assert nodes.sum() <= cap


def test_b1_mean_rank_respects_cap_and_order(oracle):
    rng = np.random.default_rng(41)
    scores = rng.choice([0.0, 1.0, 2.0], size=49)
    selected, nodes = oracle.select_mean_rank(scores, 7, 24)
    assert nodes.sum() <= 24
    closure = oracle.closure_nodes(np.flatnonzero(selected), 7)
    assert np.array_equal(closure, np.flatnonzero(nodes))


def _subset_cost(cells, resolution, points):
    """Node slots a set of cells (listed in rank order) spends under B1's count: each cell's four
    corner entries that no earlier cell of the set touched, an entry listed twice counted twice."""
    seen, cost = set(), 0
    for cell in cells:
        entries = [(cell + d) % points for d in (0, 1, resolution, resolution + 1)]
        cost += sum(1 for e in entries if e not in seen)
        seen.update(entries)
    return cost


@pytest.mark.parametrize('resolution,cap,seed', [(1, 0, 0), (1, 8, 1), (2, 8, 2), (3, 8, 3), (3, 16, 4),
                                                 (4, 8, 5), (4, 16, 6), (4, 24, 7)])
def test_b1_mean_rank_is_the_first_feasible_subset_in_rank_order(oracle, resolution, cap, seed):
    """B1 against a brute force over every subset of the cells of tiny grids with planted ties:
    with the ranking (score descending, id ascending) as priority, the admitted set is the
    feasible subset (node slots spent within the cap) whose indicator vector in rank order is
    largest -- the walk's admit-if-it-fits rule, stated without the walk.  Catches a reversed
    ranking, a wrong tie order and a wrong slot count (R = 1 lists corner 1 twice)."""
    rng = np.random.default_rng(seed)
    cells, points = resolution ** 2, oracle_align8(resolution ** 2)
    scores = rng.choice([0.0, 0.5, 0.5, 2.0, 2.0, 3.0], size=cells)
    ranking = sorted(range(cells), key=lambda c: (-scores[c], c))
    best = None
    for mask in range(1 << cells):
        members = [c for c in ranking if mask >> c & 1]
        if _subset_cost(members, resolution, points) > cap:
            continue
        vector = tuple(int(mask >> c & 1) for c in ranking)
        if best is None or vector > best[0]:
            best = (vector, members)
    selected, nodes = oracle.select_mean_rank(scores, resolution, cap)
    assert sorted(np.flatnonzero(selected).tolist()) == sorted(best[1])
    assert np.array_equal(np.flatnonzero(nodes), oracle.closure_nodes(best[1], resolution) if best[1] else [])


def test_topk_and_compaction_against_python_sort(oracle):
    rng = np.random.default_rng(43)
    scores = rng.choice([0.5, 1.5, 2.5, 7.0], size=1000)
    ids = oracle.topk_ids(scores, 37)
    brute = sorted(sorted(range(1000), key=lambda i: (-scores[i], i))[:37])
    assert list(ids) == brute
    expert = rng.integers(0, 9, size=500)
    perm, offsets = oracle.compact(expert, 9)
    brute = sorted(range(500), key=lambda i: (expert[i], i))
    assert list(perm) == brute and offsets[-1] == 500


def test_adam_torch_variant_matches_torch(oracle):
    import torch
    rng = np.random.default_rng(47)
    start = rng.normal(size=64)
    grads = [rng.normal(size=64) * 128 for _ in range(5)]
    param = torch.nn.Parameter(torch.tensor(start))
    optimizer = torch.optim.Adam([param], lr=1e-2, betas=(.9, .999), eps=1e-15, foreach=False)
    p, m, v = start.copy(), np.zeros(64), np.zeros(64)
    steps = np.zeros(64, dtype=np.uint32)
    for t, g in enumerate(grads, start=1):
        param.grad = torch.tensor(g / 128.)
        optimizer.step()
        p = oracle.adam(0, p, g, m, v, steps, t, 1e-2, scale=128.)
    assert np.allclose(p, param.detach().numpy(), rtol=1e-12, atol=1e-15)


def test_adam_tcnn_variant_skips_zero_gradients(oracle):
    p = np.array([1.0, 2.0])
    m, v, steps = np.zeros(2), np.zeros(2), np.zeros(2, dtype=np.uint32)
    p = oracle.adam(1, p, np.array([0.5, 0.0]), m, v, steps, 1, 0.1)
    assert p[1] == 2.0 and steps.tolist() == [1, 0] and m[1] == 0 and v[1] == 0
    # first step of Adam moves by lr * sign(g) (bias-corrected m/sqrt(v) = 1)
    assert abs(p[0] - 0.9) < 1e-12
    p = oracle.adam(1, p, np.array([0.0, 0.5]), m, v, steps, 2, 0.1)
    assert abs(p[1] - 1.9) < 1e-12 and steps.tolist() == [1, 1]


def test_adam_tcnn_dense_variant_never_skips(oracle):
    p = np.array([1.0, 2.0])
    m, v, steps = np.zeros(2), np.zeros(2), np.zeros(2, dtype=np.uint32)
    p = oracle.adam(2, p, np.array([0.5, 0.0]), m, v, steps, 1, 0.1)
    assert steps.tolist() == [1, 1] and p[1] == 2.0 and abs(p[0] - 0.9) < 1e-12
    # a zero gradient after a nonzero one still moves the parameter by its momentum
    p = oracle.adam(2, p, np.array([0.0, 0.0]), m, v, steps, 2, 0.1)
    assert steps.tolist() == [2, 2] and p[0] < 0.9


# Decoder MLP and loss ---------------------------------------------------------------------

def _mlp_case(seed, rows):
    rng = np.random.default_rng(seed)
    x = (rng.normal(size=(rows, 32)) * 0.5).astype(np.float16)
    flat = np.concatenate([(rng.uniform(-1, 1, size=r * c) * np.sqrt(6.0 / (r + c))) for r, c in
                           ((64, 32), (64, 64), (16, 64))]).astype(np.float16)
    return x, flat


def test_mlp_forward_matches_torch_modules(oracle):
    import torch
    x, flat = _mlp_case(3, 200)
    w1, w2, w3 = oracle.mlp_weights(flat)
    net = torch.nn.Sequential(torch.nn.Linear(32, 64, bias=False), torch.nn.ReLU(),
                              torch.nn.Linear(64, 64, bias=False), torch.nn.ReLU(),
                              torch.nn.Linear(64, 16, bias=False)).double()
    h1, h2, y = oracle.mlp_forward(x, flat)
    with torch.no_grad():
        for layer, weight in zip((net[0], net[2], net[4]), (w1, w2, w3)):
            layer.weight.copy_(torch.from_numpy(weight.astype(np.float64)))
        # the same network with fp16 rounding after each layer
        a = torch.from_numpy(x.astype(np.float64))
        a = net[1](net[0](a)).half().double()
        assert np.array_equal(a.numpy().astype(np.float16), h1)
        a = net[3](net[2](a)).half().double()
        assert np.array_equal(a.numpy().astype(np.float16), h2)
        a = net[4](a).half()
        assert np.array_equal(a.numpy(), y)


def test_mlp_backward_matches_autograd(oracle):
    import torch
    x, flat = _mlp_case(5, 96)
    h1, h2, _ = oracle.mlp_forward(x, flat)
    rng = np.random.default_rng(6)
    dy = np.zeros((96, 16), dtype=np.float16)
    dy[:, :3] = rng.normal(size=(96, 3)).astype(np.float16)
    dz, dz_magnitude, dweights, magnitude = oracle.mlp_backward(x, h1, h2, dy, flat)
    # float64 autograd through the same network without fp16 rounding, with the ReLU masks of
    # the fp16 forward held fixed (a pre-activation that rounds to fp16 zero flips a mask); the
    # oracle then differs only by fp16 rounding of activations and gradients
    w = [torch.tensor(v.astype(np.float64), requires_grad=True) for v in oracle.mlp_weights(flat)]
    xt = torch.tensor(x.astype(np.float64), requires_grad=True)
    m1, m2 = (torch.tensor((h > 0).astype(np.float64)) for h in (h1, h2))
    out = (((xt @ w[0].T) * m1) @ w[1].T * m2) @ w[2].T
    (out * torch.tensor(dy.astype(np.float64))).sum().backward()
    expected = torch.cat([v.grad.reshape(-1) for v in w]).numpy()
    assert np.all(np.abs(dweights - expected) <= 2e-2 * magnitude + 1e-12)
    assert np.abs(dweights - expected).max() < 0.05 * np.abs(expected).max()
    got = dz.astype(np.float64) * 128.0
    assert np.all(np.abs(got - xt.grad.numpy()) <= 2e-2 * dz_magnitude * 128.0 + 1e-6)
    # a transposed hidden weight is caught
    wrong = flat.copy()
    wrong[2048:2048 + 4096] = oracle.mlp_weights(flat)[1].T.ravel()
    _, _, bad, _ = oracle.mlp_backward(x, h1, h2, dy, wrong)
    assert not np.all(np.abs(bad - expected) <= 2e-2 * magnitude + 1e-12)


def _round_f32(value):
    """Correct rounding of a Fraction to fp32 (ties to even)."""
    from fractions import Fraction
    guess = np.float32(float(value))
    best = None
    for candidate in (np.nextafter(guess, np.float32(-np.inf)), guess, np.nextafter(guess, np.float32(np.inf))):
        error = abs(Fraction(float(candidate)) - value)
        key = (error, int(np.array(candidate).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, candidate)
    return best[1]


def test_mlp_loss_known_answers(oracle):
    # y = 0.5, byte 255 -> t = 1, d = -0.5; real = 1: 2d/3 * 128 = -42.666.. -> fp16 -42.65625,
    # times 128 = -5460 exactly; squares = 3 * 0.25 / 3 = 0.25
    y = np.full((1, 16), 0.5, dtype=np.float16)
    rgb = np.full((1, 3), 255, dtype=np.uint8)
    t = oracle.mlp_targets(np.array([0]), rgb=rgb, ids=np.array([0]))
    assert t.dtype == np.float32 and np.all(t == np.float32(1.0))
    dy, squares = oracle.mlp_loss(y, t, np.array([0]), 1)
    assert dy[0, :3].tolist() == [-5460.0] * 3 and not dy[0, 3:].any() and squares[0] == np.float32(0.25)
    # padding rows: zero gradient and zero square
    dy, squares = oracle.mlp_loss(y, t, np.array([5]), 5)
    assert not dy.any() and squares[0] == 0
    # the byte scaling multiplies by the fp32 reciprocal (not a division): 1/255 rounded first
    byte = np.array([[7, 0, 0]], dtype=np.uint8)
    t = oracle.mlp_targets(np.array([0]), rgb=byte, ids=np.array([0]))
    assert t[0, 0] == np.float32(np.float32(7.0) * np.float32(1.0 / 255.0))


def test_mlp_loss_squares_are_fused_sums(oracle):
    from fractions import Fraction
    rng = np.random.default_rng(9)
    y = rng.uniform(-2, 2, size=(300, 16)).astype(np.float16)
    t = rng.uniform(0, 1, size=(300, 3)).astype(np.float32)
    _, squares = oracle.mlp_loss(y, t, np.arange(300), 300)
    for row in range(300):
        s = np.float32(0)
        for c in range(3):
            d = np.float32(np.float32(y[row, c]) - t[row, c])
            s = _round_f32(Fraction(float(d)) ** 2 + Fraction(float(s)))
        assert squares[row] == np.float32(s / np.float32(3))


# Router gate ---------------------------------------------------------------------------------

def test_gate_weight_rule_matches_recorded_gates(oracle):
    from pathlib import Path
    data = np.load(Path(__file__).parent / 'golden' / 'gate_support_sample.npz', allow_pickle=False)
    gate, visible, effective = data['gate'], data['visible'], data['effective']
    weighted = oracle.gate_apply(np.ones((len(gate), 32), dtype=np.float16), gate.astype(np.float32), visible)
    assert np.array_equal(weighted[:, 0::2].view(np.uint16), effective.view(np.uint16))
    assert np.array_equal(weighted[:, 1::2].view(np.uint16), effective.view(np.uint16))
    # invisible cells contribute nothing, visible ones their gate
    assert not effective[~visible].any() and np.array_equal(effective[visible], gate[visible])


def test_gate_values_match_torch(oracle):
    import torch
    z = np.concatenate([np.linspace(-30, 30, 4001), [-0.0, 0.0, 19.99, 20.0, 20.01]]).astype(np.float16)
    z = np.tile(z[:, None], (1, 16))
    s = oracle.gate_values(z, 0)
    expected = torch.sigmoid(torch.from_numpy(z.astype(np.float64))).float().numpy()
    assert np.allclose(s, expected, rtol=2.0 ** -23, atol=0)
    soft = oracle.gate_values(z, 0, softplus=True)
    expected = torch.nn.functional.softplus(torch.from_numpy(z.astype(np.float64)), threshold=20).float().numpy()
    assert np.allclose(soft, expected, rtol=2.0 ** -23, atol=0)
    assert (oracle.gate_values(z, 5)[:, :5] == 1).all()


def test_gate_back_matches_exact_rational_arithmetic(oracle):
    from fractions import Fraction
    rng = np.random.default_rng(12)
    x = rng.normal(size=(40, 32)).astype(np.float16)
    value = (rng.normal(size=(40, 32)) * 3).astype(np.float16)
    s = rng.uniform(0, 1, size=(40, 16)).astype(np.float32)
    visible = rng.integers(0, 2, size=(40, 16)).astype(bool)
    direct, da = oracle.gate_back(x, value, s, 3, visible=visible)

    def exact16(q):   # correct rounding of a rational to fp16 (ties to even)
        guess = np.float16(float(q))
        best = None
        for c in (np.nextafter(guess, np.float16(-np.inf)), guess, np.nextafter(guess, np.float16(np.inf))):
            key = (abs(Fraction(float(c)) - q), int(np.array(c).view(np.uint16)) & 1)
            if best is None or key < best[0]:
                best = (key, c)
        return best[1]
    for i in range(40):
        for l in range(16):
            w = exact16(Fraction(float(s[i, l])) * int(visible[i, l]))
            for c in range(2):
                assert direct[i, 2 * l + c] == exact16(Fraction(float(value[i, 2 * l + c])) * Fraction(float(w)))
            p0 = exact16(Fraction(float(value[i, 2 * l])) * Fraction(float(x[i, 2 * l])))
            p1 = exact16(Fraction(float(value[i, 2 * l + 1])) * Fraction(float(x[i, 2 * l + 1])))
            reduced = exact16(Fraction(float(exact16(Fraction(0) + Fraction(float(p0))))) + Fraction(float(p1)))
            if l < 3:
                assert da[i, l] == 0
            else:
                incoming = np.float32(np.float32(reduced) * np.float32(int(visible[i, l])))
                derivative = np.float32(np.float32(incoming * np.float32(np.float32(1) - s[i, l])) * s[i, l])
                assert da[i, l] == exact16(Fraction(float(np.float16(derivative))) * 128)


def test_gate_mlp_backward_matches_autograd(oracle):
    import torch
    rng = np.random.default_rng(13)
    x = (rng.normal(size=(64, 32)) * 0.5).astype(np.float16)
    flat = np.concatenate([rng.uniform(-1, 1, 1024) * np.sqrt(6 / 64), rng.uniform(-1, 1, 512) * np.sqrt(6 / 48)])
    flat = flat.astype(np.float16)
    h, z, _ = oracle.gate_logits(x, flat)
    da = (rng.normal(size=(64, 16)) * 100).astype(np.float16)
    dr, dr_magnitude, dweights, magnitude = oracle.gate_mlp_backward(x, h, da, flat)
    w = [torch.tensor(v.astype(np.float64), requires_grad=True) for v in oracle.gate_weights(flat)]
    xt = torch.tensor(x.astype(np.float64), requires_grad=True)
    mask = torch.tensor((h > 0).astype(np.float64))
    logits = ((xt @ w[0].T) * mask) @ w[1].T
    (logits * torch.tensor(da.astype(np.float64))).sum().backward()
    expected = torch.cat([v.grad.reshape(-1) for v in w]).numpy()
    assert np.all(np.abs(dweights - expected) <= 2e-2 * magnitude + 1e-9)
    assert np.all(np.abs(dr.astype(np.float64) - xt.grad.numpy()) <= 2e-2 * dr_magnitude + 1e-6)


# Stratified sampling ---------------------------------------------------------------------------

def test_stratified_ids_follow_the_strata(oracle):
    """The oracle's ids against exact rational arithmetic: with u in [0, 1) the pixel of slot j
    lies in [floor(s * W / side), ceil((s + 1) * W / side)] of its stratum column s (rows alike;
    the upper end is reachable only through fp32 rounding of u/side + s/side), u = 0 gives
    floor(s * W / side) exactly (truncation, not rounding), and the axes are not swapped
    (W != H)."""
    from fractions import Fraction
    import math
    for width, height, batch in ((97, 61, 16), (1536, 2040, 64), (33, 5, 4), (2048, 1365, 1024)):
        side = int(round(batch ** 0.5))
        rng = np.random.default_rng(width)
        u = rng.random((batch, 2), dtype=np.float32)
        u[1] = np.nextafter(np.float32(1.0), np.float32(0.0))
        ids = oracle.stratified_ids(u, width, height)
        zero = oracle.stratified_ids(np.zeros((batch, 2), dtype=np.float32), width, height)
        for j in range(batch):
            sx, sy = j % side, j // side
            assert zero[j] == math.floor(Fraction(sy * height, side)) * width + math.floor(Fraction(sx * width, side))
            x, y = ids[j] % width, ids[j] // width
            for value, s, size in ((x, sx, width), (y, sy, height)):
                low = math.floor(Fraction(s * size, side))
                high = min(math.ceil(Fraction((s + 1) * size, side)), size - 1)
                assert low <= value <= high, (width, height, batch, j)


# Routing of pixel ids to tile experts --------------------------------------------------------

def _exact_f32(value):
    """Correctly rounded fp32 of a Fraction (ties to even), as a numpy float32."""
    return np.float32(float(round_fraction(value, SINGLE)))


@pytest.mark.parametrize('width,height,regions_x,regions_y', [
    (23, 17, 3, 5),        # non-square image, different tile counts per axis, ragged tiles
    (64, 9, 8, 2),         # tiles of exactly 8 x 4.5 pixels
    (41 * 2 + 2, 13, 2, 1),  # tile width 42: (w-1) * fp32(1/(w-1)) rounds below 1 in fp32
    (7, 5, 2, 2),
])
def test_route_against_per_pixel_brute_force(oracle, width, height, regions_x, regions_y):
    """oracle.route against a brute force over every pixel of the image (and ids past it):
    the tile of a pixel is found by searching the integer bounds ceil(r * size / regions)
    (exact rationals), not by the oracle's floor(x * regions / size); every pixel lies in
    exactly one tile; the local coordinate is the exactly rounded fp32 product
    fp32(x - x0) * fp32(1 / (tile - 1)) of the reference's pixel -> coordinate convention
    (odie/native/runtime.cu:34-36), so 0 at a tile's first pixel, monotone across the tile, and
    within one ulp below 1 at its last (exactly 1 where fp32 allows); x and y are not swapped;
    ids past the image clamp to its last row, ids beyond 2^32 wrap as the 32-bit id does; the
    order is the stable ascending-expert order of a Python sort."""
    def bounds(size, regions):
        return [math.ceil(Fraction(r * size, regions)) for r in range(regions + 1)]
    xb, yb = bounds(width, regions_x), bounds(height, regions_y)
    pixels = width * height
    ids = np.concatenate([np.arange(pixels), pixels + np.arange(3 * width),
                          (1 << 32) + np.arange(5), np.arange(pixels)[::-7]]).astype(np.int64)
    expert, perm, local, offsets = oracle.route(ids, width, height, regions_x, regions_y)
    expected_expert, expected_uv = [], []
    for raw in ids.tolist():
        pixel = raw % (1 << 32)
        x, y = pixel % width, min(pixel // width, height - 1)
        rx = [r for r in range(regions_x) if xb[r] <= x < xb[r + 1]]
        ry = [r for r in range(regions_y) if yb[r] <= y < yb[r + 1]]
        assert len(rx) == 1 and len(ry) == 1
        rx, ry = rx[0], ry[0]
        expected_expert.append(ry * regions_x + rx)
        u = _exact_f32(Fraction(x - xb[rx]) * Fraction(float(_exact_f32(Fraction(1, xb[rx + 1] - xb[rx] - 1)))))
        v = _exact_f32(Fraction(y - yb[ry]) * Fraction(float(_exact_f32(Fraction(1, yb[ry + 1] - yb[ry] - 1)))))
        expected_uv.append((u, v))
    assert expert.tolist() == expected_expert
    order = sorted(range(len(ids)), key=lambda i: expected_expert[i])
    assert list(perm) == order
    uv = np.array(expected_uv, dtype=np.float32)[order]
    assert np.array_equal(local.view(np.uint32), uv.view(np.uint32))
    counts = [expected_expert.count(e) for e in range(regions_x * regions_y)]
    assert list(offsets) == [sum(counts[:e]) for e in range(regions_x * regions_y + 1)]
    # the geometry of each tile: first pixel 0, last pixel 1 or one ulp below, increasing
    slot_of = {int(ids[j]): k for k, j in enumerate(perm) if ids[j] < pixels}
    for ry in range(regions_y):
        for rx in range(regions_x):
            row = [local[slot_of[yb[ry] * width + x]][0] for x in range(xb[rx], xb[rx + 1])]
            column = [local[slot_of[y * width + xb[rx]]][1] for y in range(yb[ry], yb[ry + 1])]
            for values in (row, column):
                assert values[0] == 0.0
                assert 1.0 - 2.0 ** -24 <= values[-1] <= 1.0
                assert all(a < b for a, b in zip(values, values[1:]))
    last = np.float32(41.0) * np.float32(1.0 / 41.0)
    assert last == np.float32(1.0) - np.float32(2.0 ** -24)   # the rounding the third case exercises


@pytest.mark.parametrize('width,height,regions_x,regions_y,slots,experts', [
    (23, 17, 3, 5, [4, -1, 0, 9, 2, 1, -1, 3, 5, 6, -3, 7, 8, 10, 11], 12),   # shuffled, with gaps
    (7, 5, 2, 2, [0, 0, -1, 1], 2),                                          # two tiles share an expert
    (7, 5, 2, 2, [-1, -1, -1, -1], 1),                                       # no tile owns one
])
def test_route_with_slots_against_a_python_sort(oracle, width, height, regions_x, regions_y, slots, experts):
    """oracle.route with a slot map against the plain route (pinned by the per-pixel brute force
    above) and a Python sort: an id's expert is its tile's slot (-1 outside [0, experts)), the
    order is the stable sort by (slot, or experts for none), offsets count the experts and the
    first id without one, and the local coordinates are the tile's, whichever slot it maps to."""
    pixels = width * height
    ids = np.concatenate([np.arange(pixels), np.arange(pixels)[::-3], pixels + np.arange(4)]).astype(np.int64)
    tile, plain_perm, plain_local, _ = oracle.route(ids, width, height, regions_x, regions_y)
    expert, perm, local, offsets = oracle.route(ids, width, height, regions_x, regions_y, slots=slots,
                                                experts=experts)
    owner = [slots[t] if 0 <= slots[t] < experts else -1 for t in tile.tolist()]
    assert expert.tolist() == owner
    key = [e if e >= 0 else experts for e in owner]
    order = sorted(range(len(ids)), key=lambda i: key[i])
    assert list(perm) == order
    assert list(offsets) == [sum(1 for k in key if k < e) for e in range(experts + 1)]
    where = {j: k for k, j in enumerate(plain_perm)}     # slot of each input in the plain route
    assert np.array_equal(local.view(np.uint32), plain_local[[where[j] for j in order]].view(np.uint32))
    tiles = regions_x * regions_y
    identity = oracle.route(ids, width, height, regions_x, regions_y, slots=list(range(tiles)), experts=tiles)
    plain = oracle.route(ids, width, height, regions_x, regions_y)
    for got, want in zip(identity, plain):
        assert np.array_equal(got, want)


def test_gate_upstream_matches_exact_rational_arithmetic(oracle):
    """hash_router_gradient (odie/native/runtime.cu:99-103) in exact arithmetic: the router's input
    gradient is divided by 128 in fp32 (exact: a power of two inside the fp32 range), rounded once
    to fp16 (which loses bits only where the quotient falls below fp16's normal range), then added
    to the direct gradient with one fp16 rounding.  The planted values hit fp16 subnormal
    quotients, ties to even in the sum, overflow to infinity and signed zeros, so dropping the
    intermediate rounding, scaling by another power of two or adding before the division fails."""
    rng = np.random.default_rng(77)
    direct = (rng.normal(size=4000) * rng.choice([1e-6, 1e-3, 1.0, 300.0], size=4000)).astype(np.float16)
    dr = np.clip(rng.normal(size=4000) * rng.choice([1e-3, 1.0, 1e3, 6e4], size=4000), -65504, 65504)
    dr = dr.astype(np.float16)
    planted_direct = np.array([0.0, -0.0, -0.0, 65504.0, 2.0 ** -14, 1.0, 2.0 ** -24, 0.0], dtype=np.float16)
    planted_dr = np.array([-0.0, -0.0, 0.0, 60000.0, 3 * 2.0 ** -17, 2.0 ** -4, 1.5 * 2.0 ** -17, 2.0 ** -10],
                          dtype=np.float16)
    direct = np.concatenate([direct, planted_direct])
    dr = np.concatenate([dr, planted_dr])
    with np.errstate(over='ignore'):
        out = oracle.gate_upstream(direct, dr)
    for a, b, got in zip(direct.tolist(), dr.tolist(), out):
        unscaled = round_fraction(Fraction(b) / 128, HALF)
        if unscaled == 0 and (b < 0 or (b == 0 and math.copysign(1.0, b) < 0)):
            unscaled_sign = -1.0
        else:
            unscaled_sign = 1.0 if unscaled >= 0 else -1.0
        total = Fraction(a) + Fraction(unscaled)
        expected = round_fraction(total, HALF)
        bits = int(np.array([got], dtype=np.float16).view(np.uint16)[0])
        if isinstance(expected, float):                       # overflow
            assert bits == to_half_bits(expected)
        elif expected == 0:
            # IEEE: the sum of two zeros of the same sign keeps it, otherwise +0
            negative = math.copysign(1.0, a) < 0 and unscaled_sign < 0 and Fraction(a) == 0
            assert bits == (0x8000 if negative else 0x0000), (a, b)
        else:
            assert Fraction(float(np.float16(got))) == expected, (a, b)
    assert np.isinf(out[-5]) and out[-5] > 0            # 65504 + 468.75 overflows
