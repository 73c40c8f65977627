"""CPU oracle for the sparse grid-query hot path -- TEST INFRASTRUCTURE ONLY.

Restates the reference's algorithms so the HIP kernels can be checked against them:
the arithmetic-heavy parts in plain C (odie_oracle.c, built by oracle/Makefile into
oracle/_build/libodie_oracle.so), the rest here in numpy / pure Python.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only
as the checker or the timed CPU baseline; the odie_amd package never does.

Pinning status of each function (what fixes it beyond this restatement) is listed in
PINS below and checked by tests/test_oracle_pins.py.
"""
import ctypes as C
import heapq
import math
from pathlib import Path
import struct
import subprocess

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / '_build' / 'libodie_oracle.so'

PINS = {
    'f2h/h2f/hfma': 'exhaustive fp16 round trips vs numpy; hfma vs exact rational arithmetic (fractions)',
    'grid_levels': 'reference-held layouts in results/**/metrics.json (tests/golden/layout_goldens.json)',
    'hash_forward': 'dense level == bilinear interpolation in exact arithmetic; hash index vs '
                    'Instant-NGP Eq. 4 brute force; fp16 chain vs fractions on tiny inputs',
    'hash_backward': 'adjoint identity <fwd(x,g),u> = <g,bwd(x,u)> in fp64; brute force on tiny inputs',
    'packed_forward/backward': 'all-visible direct layout == hash grid dense level with integer scale; '
                               'rank addressing vs brute force; adjoint identity',
    'residual': 'numpy bincount restatement of odie/selection.py:58-73',
    'native_thresholds': 'exact rational fma boundaries brute-forced over fp32 bit patterns',
    'select_benefit_cost': 'O(n^2) brute-force greedy on tiny resolutions with planted ties',
    'select_mean_rank': 'brute force over every subset of tiny grids (R <= 4) with planted ties: the first '
                        'feasible subset in rank order (tests/test_oracle_pins.py)',
    'adam': 'torch.optim.Adam on the CPU (torch-style variant)',
    'compaction/topk': 'numpy.argsort(kind="stable")',
    'mlp': 'torch.nn.functional.linear/relu in float64 on the CPU (same fp16 weights and inputs); '
           'layer outputs rounded once to fp16',
    'mlp_loss': 'closed form of odie/native/runtime.cu:53-63 in IEEE float32/float16 numpy arithmetic; '
                'hand-computed known answers',
    'gate': 'recorded gates of the reference (tests/golden/gate_support_sample.npz: effective = fp16(s*visible)); '
            'torch.sigmoid / softplus; exact fp16 arithmetic of parallel_gate_back checked by fractions; autograd '
            'of the gate MLP',
    'route': 'per-pixel brute force over whole small non-square images: tile found by searching the integer '
             'bounds ceil(r*size/regions), local coordinate as the exactly rounded fp32 product (fractions), '
             'stable order of a Python sort, clamped and wrapped ids',
    'gate_upstream': 'exact rational arithmetic (fractions) with planted subnormal quotients, ties, overflow and '
                     'signed zeros',
    'stratified_ids': 'exact rational arithmetic: each pixel lies in its stratum\'s pixel interval, u = 0 gives '
                      'floor(stratum * size / side), u -> 1 stays below the next stratum; axes distinguished on '
                      'non-square images',
}


def build():
    subprocess.run(['make', '-s', '-C', str(HERE)], check=True)
    return LIBRARY


_lib = None


class Level(C.Structure):
    _fields_ = [('scale', C.c_float), ('res', C.c_uint32), ('size', C.c_uint32),
                ('offset', C.c_uint32), ('hashed', C.c_uint32)]


def lib():
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        handle = C.CDLL(str(LIBRARY))
        P, I, I64 = C.c_void_p, C.c_int, C.c_int64
        handle.ora_h2f.argtypes, handle.ora_h2f.restype = [C.c_uint16], C.c_float
        handle.ora_d2h.argtypes, handle.ora_d2h.restype = [C.c_double], C.c_uint16
        handle.ora_f2h.argtypes, handle.ora_f2h.restype = [C.c_float], C.c_uint16
        handle.ora_hfma.argtypes, handle.ora_hfma.restype = [C.c_uint16] * 3, C.c_uint16
        handle.ora_hash_forward.argtypes = [P, P, I, I64, P, I, P, I, I, I, P, I]
        handle.ora_hash_backward.argtypes = [P, P, I, I64, P, I, P, I, I, I, P, P, P]
        handle.ora_hash_backward_f32.argtypes = [P, P, I, I64, P, P, I, I, I, P, I]
        handle.ora_packed_forward.argtypes = [P, I64, P, P, I, P, P, P, I, P, P, I]
        handle.ora_packed_backward.argtypes = [P, I64, P, I, P, I, P, P, P, P, P, P]
        handle.ora_residual.argtypes = [P, P, I, I64, I64, I, I, P, P, P]
        handle.ora_adam.argtypes = [I, P, P, P, P, P, I64, I64, C.c_double, C.c_double, C.c_double,
                                    C.c_double, C.c_double]
        for name in ('ora_hash_forward', 'ora_hash_backward', 'ora_hash_backward_f32', 'ora_packed_forward',
                     'ora_packed_backward', 'ora_residual', 'ora_adam'):
            getattr(handle, name).restype = None
        _lib = handle
    return _lib


def _p(array):
    return None if array is None else array.ctypes.data


# ---------------------------------------------------------------------------------------
# fp16 scalars
# ---------------------------------------------------------------------------------------

def h2f(bits):
    return lib().ora_h2f(int(bits))


def f2h(value):
    return lib().ora_f2h(float(value))


def hfma(a, b, c):
    return lib().ora_hfma(int(a), int(b), int(c))


# ---------------------------------------------------------------------------------------
# Hash grid geometry (odie/config.py:79-94, restated independently of odie_amd.config)
# ---------------------------------------------------------------------------------------

def _f32(value):
    return struct.unpack('f', struct.pack('f', value))[0]


def grid_levels(encoding):
    """[(scale, res, size, offset, hashed)] and the entry total of one table."""
    levels = int(encoding['n_levels'])
    base = int(encoding['base_resolution'])
    size_limit = 1 << int(encoding['log2_hashmap_size'])
    growth = _f32(encoding['per_level_scale'])
    log_growth = _f32(math.log2(growth))
    rows, offset = [], 0
    for i in range(levels):
        scale = _f32(_f32(_f32(2 ** _f32(i * log_growth)) * base) - 1)
        res = math.ceil(scale) + 1
        size = min((res * res + 7) // 8 * 8, size_limit)
        rows.append((scale, res, size, offset, int(res * res > size)))
        offset += size
    return rows, offset


def _levels(rows):
    array = (Level * len(rows))()
    for i, row in enumerate(rows):
        array[i] = Level(*row)
    return array


def _offsets(offsets, n):
    if offsets is None:
        return np.array([0, n], dtype=np.int64), 1
    offsets = np.ascontiguousarray(offsets, dtype=np.int64)
    return offsets, len(offsets) - 1


def hash_forward(xy, table, rows, features, *, offsets=None, expert_params=None, width=None, threads=1):
    """fp16 table -> fp16 [N, width]; fp32 table -> fp32 [N, width]."""
    xy = np.ascontiguousarray(xy, dtype=np.float32)
    table = np.ascontiguousarray(table)
    offsets, experts = _offsets(offsets, len(xy))
    width = width or len(rows) * features
    half = table.dtype == np.float16
    out = np.zeros((len(xy), width), dtype=np.float16 if half else np.float32)
    expert_params = expert_params or table.size // experts
    lib().ora_hash_forward(_p(xy), _p(offsets), experts, expert_params, _p(table.view(np.uint16) if half else table),
                           1 if half else 0, _levels(rows), len(rows), features, width,
                           _p(out.view(np.uint16) if half else out), threads)
    return out


def hash_backward(xy, upstream, rows, features, total, *, offsets=None, expert_params=None, counts=False):
    """(gradient fp64 [total], magnitude fp64 [total]) -- exact-order-free checker; with counts,
    also the number of contributions of every entry (fp64 [total])."""
    xy = np.ascontiguousarray(xy, dtype=np.float32)
    upstream = np.ascontiguousarray(upstream)
    offsets, experts = _offsets(offsets, len(xy))
    expert_params = expert_params or total // experts
    grad = np.zeros(total, dtype=np.float64)
    magnitude = np.zeros(total, dtype=np.float64)
    count = np.zeros(total, dtype=np.float64) if counts else None
    half = upstream.dtype == np.float16
    values = upstream.view(np.uint16) if half else np.ascontiguousarray(upstream, dtype=np.float32)
    lib().ora_hash_backward(_p(xy), _p(offsets), experts, expert_params, _p(values),
                            1 if half else 0, _levels(rows), len(rows), features, upstream.shape[1],
                            _p(grad), _p(magnitude), _p(count))
    return (grad, magnitude, count) if counts else (grad, magnitude)


def hash_backward_f32(xy, upstream, rows, features, total, *, offsets=None, expert_params=None, threads=1):
    """The CPU-baseline form: fp32 accumulation with atomic adds across threads."""
    xy = np.ascontiguousarray(xy, dtype=np.float32)
    upstream = np.ascontiguousarray(upstream, dtype=np.float16)
    offsets, experts = _offsets(offsets, len(xy))
    expert_params = expert_params or total // experts
    grad = np.zeros(total, dtype=np.float32)
    lib().ora_hash_backward_f32(_p(xy), _p(offsets), experts, expert_params, _p(upstream.view(np.uint16)),
                                _levels(rows), len(rows), features, upstream.shape[1], _p(grad), threads)
    return grad


# ---------------------------------------------------------------------------------------
# Packed xy planes (odie/packed_kernels.cu)
# ---------------------------------------------------------------------------------------

def packed_forward(xy, grid, layout, width, threads=1):
    xy = np.ascontiguousarray(xy, dtype=np.float32)
    desc = np.ascontiguousarray(layout['descriptors'], dtype=np.int32)
    node_bitmap = np.ascontiguousarray(layout['node_bitmap'], dtype=np.uint64)
    prefix = np.ascontiguousarray(layout['node_prefix'], dtype=np.int32)
    bitmap = np.ascontiguousarray(layout['bitmap'], dtype=np.uint8)
    grid = np.ascontiguousarray(grid, dtype=np.float32)
    out = np.zeros((len(xy), width), dtype=np.float16)
    vis = np.zeros((len(xy), len(desc)), dtype=np.uint8)
    lib().ora_packed_forward(_p(xy), len(xy), _p(grid), _p(desc), len(desc), _p(node_bitmap), _p(prefix),
                             _p(bitmap), width, _p(out.view(np.uint16)), _p(vis), threads)
    return out, vis.astype(bool)


def packed_backward(xy, upstream, layout, total, counts=False):
    xy = np.ascontiguousarray(xy, dtype=np.float32)
    upstream = np.ascontiguousarray(upstream, dtype=np.float16)
    desc = np.ascontiguousarray(layout['descriptors'], dtype=np.int32)
    node_bitmap = np.ascontiguousarray(layout['node_bitmap'], dtype=np.uint64)
    prefix = np.ascontiguousarray(layout['node_prefix'], dtype=np.int32)
    bitmap = np.ascontiguousarray(layout['bitmap'], dtype=np.uint8)
    grad = np.zeros(total, dtype=np.float64)
    magnitude = np.zeros(total, dtype=np.float64)
    count = np.zeros(total, dtype=np.float64) if counts else None
    lib().ora_packed_backward(_p(xy), len(xy), _p(upstream.view(np.uint16)), upstream.shape[1], _p(desc),
                              len(desc), _p(node_bitmap), _p(prefix), _p(bitmap), _p(grad), _p(magnitude),
                              _p(count))
    return (grad, magnitude, count) if counts else (grad, magnitude)


# ---------------------------------------------------------------------------------------
# Residual, thresholds, selection (odie/selection.py, odie/residual_cuda.cu)
# ---------------------------------------------------------------------------------------

def residual(prediction, target, width, resolution, xb, yb, begin=0, totals=None):
    prediction = np.ascontiguousarray(prediction, dtype=np.float32)
    target = np.ascontiguousarray(target)
    rgb8 = target.dtype == np.uint8
    if not rgb8:
        target = target.astype(np.float32)
    xb = np.ascontiguousarray(xb, dtype=np.int32)
    yb = np.ascontiguousarray(yb, dtype=np.int32)
    if totals is None:
        totals = np.zeros(resolution * resolution, dtype=np.float64)
    end = begin + prediction.reshape(-1, 3).shape[0]
    lib().ora_residual(_p(prediction), _p(target), int(rgb8), begin, end, width, resolution, _p(xb), _p(yb),
                       _p(totals))
    return totals


def align8(value):
    return (int(value) + 7) // 8 * 8


def _float_from_bits(bits):
    return struct.unpack('<f', struct.pack('<I', bits))[0]


def native_thresholds(resolution):
    """Smallest fp32 x in [0,1] with floor(fma(R-1, x, 0.5)) >= region, per region 1..R-1
    (odie/selection.py:16-42): binary search over fp32 bit patterns against the exact
    rounding boundary of the fused result."""
    scale = resolution - 1
    thresholds = []
    for region in range(1, resolution):
        region_bits = struct.unpack('<I', struct.pack('<f', region))[0]
        below_num, below_den = _float_from_bits(region_bits - 1).as_integer_ratio()
        # fma(scale, x, 0.5) rounds up to `region` once scale*x + 0.5 passes the midpoint
        # between `region` and its fp32 predecessor (ties go to the even neighbour).
        boundary_num = (region - 1) * below_den + below_num
        boundary_den = 2 * below_den
        include_tie = region_bits % 2 == 0
        lower, upper = 0, 0x3F800000
        while lower < upper:
            middle = (lower + upper) // 2
            numerator, denominator = _float_from_bits(middle).as_integer_ratio()
            left, right = scale * numerator * boundary_den, boundary_num * denominator
            if left > right or (left == right and include_tie):
                upper = middle
            else:
                lower = middle + 1
        thresholds.append(_float_from_bits(lower))
    return np.asarray(thresholds, dtype=np.float32)


def pixel_cells(shape, resolution):
    height, width = shape
    thresholds = native_thresholds(resolution)
    x = np.arange(width, dtype=np.float32) / np.float32(width - 1)
    y = np.arange(height, dtype=np.float32) / np.float32(height - 1)
    xb = np.searchsorted(thresholds, x, side='right')
    yb = np.searchsorted(thresholds, y, side='right')
    return (yb[:, None] * resolution + xb[None, :]).reshape(-1)


def closure_nodes(cells, resolution):
    cells = np.asarray(cells, dtype=np.int64)
    return np.unique(np.concatenate([cells, cells + 1, cells + resolution, cells + resolution + 1])
                     % align8(resolution ** 2))


def select_mean_rank(scores, resolution, cap):
    """B1 (odie/selection.py:108-126): stable descending ranking, admit a cell when its new
    closure nodes fit under the cap."""
    scores = np.asarray(scores, dtype=np.float64)
    points = align8(resolution ** 2)
    selected = np.zeros(resolution ** 2, dtype=bool)
    nodes = np.zeros(points, dtype=bool)
    used = 0
    for cell in np.argsort(-scores, kind='stable'):
        corners = (cell + np.array([0, 1, resolution, resolution + 1])) % points
        added = corners[~nodes[corners]]
        if used + len(added) <= cap:
            selected[cell] = True
            nodes[added] = True
            used += len(added)
    return selected, nodes


def select_benefit_cost(scores, resolution, cap, normalize_by_cost=True, trace=None):
    """B2 exact greedy (odie/selection.py:129-207): free cells (no new nodes) first in
    ascending id; otherwise the best score/cost over cost 1..min(4, cap-used), compared by
    cross-multiplication, ties to the lower id.  Returns (selected, nodes, iterations)."""
    scores = np.asarray(scores, dtype=np.float64)
    cells, points = resolution ** 2, align8(resolution ** 2)
    selected = np.zeros(cells, dtype=bool)
    nodes = np.zeros(points, dtype=bool)
    missing = np.full(cells, 4, dtype=np.int64)
    heaps = [[] for _ in range(5)]
    heaps[4] = [(-float(value), cell) for cell, value in enumerate(scores)]
    heapq.heapify(heaps[4])
    used = iterations = 0
    deltas = (0, 1, resolution, resolution + 1)

    def top(cost):
        heap = heaps[cost]
        while heap and (selected[heap[0][1]] or missing[heap[0][1]] != cost):
            heapq.heappop(heap)
        return heap[0] if heap else None

    while True:
        free = top(0)
        if free is not None:
            cell, cost = free[1], 0
        else:
            best = None
            for cost in range(1, min(4, cap - used) + 1):
                candidate = top(cost)
                if candidate is None:
                    continue
                score, cell = -candidate[0], candidate[1]
                if best is None:
                    best = (score, cost, cell)
                    continue
                left, right = ((score * best[1], best[0] * cost) if normalize_by_cost else (score, best[0]))
                if left > right or (left == right and cell < best[2]):
                    best = (score, cost, cell)
            if best is None:
                break
            _, cost, cell = best
        heapq.heappop(heaps[cost])
        selected[cell] = True
        corners = [(cell + d) % points for d in deltas]
        added = [node for node in corners if not nodes[node]]
        assert len(added) == cost, 'stale marginal cost'
        nodes[added] = True
        used += cost
        iterations += 1
        if trace is not None:
            trace.append(cell)
        changed = set()
        for node in added:
            for d in deltas:
                incident = (node - d) % points
                if incident < cells and not selected[incident]:
                    missing[incident] -= 1
                    changed.add(incident)
        for incident in changed:
            now = int(missing[incident])
            heapq.heappush(heaps[now], (incident if now == 0 else -float(scores[incident]), incident))
    return selected, nodes, iterations


def topk_ids(scores, k):
    """Top-k by (score descending, id ascending), returned sorted ascending by id."""
    order = np.argsort(-np.asarray(scores, dtype=np.float64), kind='stable')[:k]
    return np.sort(order)


def compact(expert, experts):
    """Stable counting sort by expert id: (perm, offsets)."""
    expert = np.asarray(expert)
    perm = np.argsort(expert, kind='stable')
    counts = np.bincount(expert, minlength=experts)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    return perm.astype(np.int64), offsets.astype(np.int64)


def adam(variant, param, grad, m, v, steps, step, lr, beta1=0.9, beta2=0.999, eps=1e-15, scale=1.0):
    """In place on float64 arrays (steps: uint32 per-parameter ages for variant 1)."""
    param = np.ascontiguousarray(param, dtype=np.float64)
    grad = np.ascontiguousarray(grad, dtype=np.float64)
    lib().ora_adam(int(variant), _p(param), _p(grad), _p(m), _p(v), _p(steps), param.size, int(step),
                   lr, beta1, beta2, eps, scale)
    return param


def route(ids, width, height, regions_x, regions_y, slots=None, experts=None):
    """Routing spec restated with integer division: expert = (y*RY//H)*RX + x*RX//W, local
    coordinate fp32(x - x0) * fp32(1/(tile-1)); returns (expert, perm, local_xy, offsets)
    with perm the stable ascending-expert order.  With slots (tile -> expert; a value outside
    [0, experts) means none), an id's expert is its tile's slot, the ids of tiles without one
    follow every expert's in input order, offsets has experts + 1 entries (offsets[experts]:
    the first of those) and their expert is -1."""
    ids = np.asarray(ids, dtype=np.int64).astype(np.uint32).astype(np.int64)
    x, y = ids % width, np.minimum(ids // width, height - 1)
    rx, ry = x * regions_x // width, y * regions_y // height
    expert = ry * regions_x + rx
    x0 = -((-rx * width) // regions_x)
    y0 = -((-ry * height) // regions_y)
    x1 = -((-(rx + 1) * width) // regions_x)
    y1 = -((-(ry + 1) * height) // regions_y)
    u = (x - x0).astype(np.float32) * (1.0 / (x1 - x0 - 1).astype(np.float64)).astype(np.float32)
    v = (y - y0).astype(np.float32) * (1.0 / (y1 - y0 - 1).astype(np.float64)).astype(np.float32)
    if slots is None:
        perm, offsets = compact(expert, regions_x * regions_y)
    else:
        slot = np.asarray(slots, dtype=np.int64)[expert]
        owned = (slot >= 0) & (slot < experts)
        perm, offsets = compact(np.where(owned, slot, experts), experts + 1)
        offsets = offsets[:experts + 1]
        expert = np.where(owned, slot, -1)
    local = np.stack([u, v], axis=1).astype(np.float32)[perm]
    return expert.astype(np.int32), perm, local, offsets


# --------------------------------------------------------------------------------------------
# Decoder MLP width -> 64 -> 64 -> 16 (the FullyFusedMLP head, odie/hash_grid.py:32-34, with
# n_input_dims W = align16 of the grid's features, odie/native/runtime.cu:17,190) and the step's
# loss (odie/native/runtime.cu:53-63).  Weights: fp16 [64*W + 5120] = W1 [64][W] | W2 [64][64] |
# W3 [16][64], row-major [out][in] (7168 at W = 32).  Layers are computed in float64 and rounded
# once to fp16; TCNN's own accumulation order is not restated (parity tolerance covers fp32
# accumulation).

MLP_SHAPES = ((64, 32), (64, 64), (16, 64))


def mlp_shapes(width=32):
    return ((64, width), (64, 64), (16, 64))


def mlp_weights(flat16):
    """(W1, W2, W3) of a flat fp16 weight vector; the input width follows from its size."""
    flat16 = np.asarray(flat16, dtype=np.float16)
    width, rest = divmod(flat16.size - 64 * 64 - 16 * 64, 64)
    if rest or width < 1:
        raise ValueError('decoder weights must hold 64*W + 5120 values')
    out, start = [], 0
    for rows, cols in mlp_shapes(width):
        out.append(flat16[start:start + rows * cols].reshape(rows, cols))
        start += rows * cols
    return out


def mlp_layer(inputs16, weight16, relu):
    """fp16 [rows, in] x fp16 [out, in]^T in float64, ReLU, one rounding to fp16; also the
    magnitude sum |inputs| |W|^T that bounds accumulation-order differences."""
    x = np.asarray(inputs16, dtype=np.float64)
    w = np.asarray(weight16, dtype=np.float64)
    acc = x @ w.T
    if relu:
        acc = np.where(acc > 0, acc, 0.0)
    return acc.astype(np.float16), np.abs(x) @ np.abs(w).T


def mlp_forward(x16, flat16):
    w1, w2, w3 = mlp_weights(flat16)
    h1, _ = mlp_layer(x16, w1, True)
    h2, _ = mlp_layer(h1, w2, True)
    y, _ = mlp_layer(h2, w3, False)
    return h1, h2, y


def mlp_targets(rows, rgb=None, ids=None, target=None):
    """fp32 targets [rows, 3]: byte * fp32(1/255) (odie/native/runtime.cu:37,56) or given fp32."""
    if rgb is not None:
        bytes_ = np.asarray(rgb, dtype=np.uint8).reshape(-1, 3)[np.asarray(ids)[rows]]
        return bytes_.astype(np.float32) * (np.float32(1.0) / np.float32(255.0))
    return np.asarray(target, dtype=np.float32).reshape(-1, 3)[rows]


def mlp_loss(y16, targets, inputs, real):
    """dy fp16 [rows, 16] and squares fp32 [rows] of odie/native/runtime.cu:53-63 for output
    rows y16 whose input indices are `inputs`: d = y - t (fp32), dy = fp16(fp16(2d/(3 real) *
    128) * 128) for c < 3, squares = fma(d2, d2, fma(d1, d1, d0*d0)) / 3; zero for inputs >= real."""
    y = np.asarray(y16, dtype=np.float16)[:, :3].astype(np.float32)
    d = (y - np.asarray(targets, dtype=np.float32)).astype(np.float32)
    with np.errstate(over='ignore'):
        scaled = ((np.float32(2.0) * d) / np.float32(3 * real) * np.float32(128.0)).astype(np.float16)
        dy3 = (scaled.astype(np.float32) * np.float32(128.0)).astype(np.float16)
    wide = d.astype(np.longdouble)
    square = np.zeros(len(d), dtype=np.float32)
    for c in range(3):   # fused multiply-add: one rounding of d^2 + s
        square = (wide[:, c] * wide[:, c] + square.astype(np.longdouble)).astype(np.float32)
    squares = (square / np.float32(3.0)).astype(np.float32)
    real_rows = np.asarray(inputs) < real
    dy = np.zeros((len(d), 16), dtype=np.float16)
    dy[:, :3] = np.where(real_rows[:, None], dy3, np.float16(0))
    return dy, np.where(real_rows, squares, np.float32(0))


def mlp_backward(x16, h1, h2, dy16, flat16):
    """Gradients of the decoder from the given activations: dz fp16 [rows, 32] =
    fp16(fp16(dL/dx) / 128), dweights float64 [7168], and magnitude bounds of both."""
    w1, w2, w3 = (w.astype(np.float64) for w in mlp_weights(flat16))
    x, a1, a2, dy = (np.asarray(v, dtype=np.float16).astype(np.float64) for v in (x16, h1, h2, dy16))
    pre2 = dy @ w3
    dh2 = np.where(a2 > 0, pre2, 0.0).astype(np.float16).astype(np.float64)
    m2 = np.where(a2 > 0, np.abs(dy) @ np.abs(w3), 0.0)
    pre1 = dh2 @ w2
    dh1 = np.where(a1 > 0, pre1, 0.0).astype(np.float16).astype(np.float64)
    m1 = np.where(a1 > 0, (np.abs(dh2) + m2) @ np.abs(w2), 0.0)
    dx = (dh1 @ w1).astype(np.float16)
    dz = (dx.astype(np.float32) / np.float32(128.0)).astype(np.float16)
    mx = (np.abs(dh1) + m1) @ np.abs(w1)
    dweights = np.concatenate([(dh1.T @ x).ravel(), (dh2.T @ a1).ravel(), (dy.T @ a2).ravel()])
    magnitude = np.concatenate([((np.abs(dh1) + m1).T @ np.abs(x)).ravel(),
                                ((np.abs(dh2) + m2).T @ np.abs(a1)).ravel(),
                                (np.abs(dy).T @ np.abs(a2)).ravel()])
    return dz, mx / 128.0, dweights, magnitude


def mlp_step_f32(x16, flat16, targets, inputs, real, threads=1):
    """The CPU-baseline form of the decoder stage (forward, loss, backward) in torch-CPU float32
    with fp16 rounding of activations and gradients at the same points as mlp_forward /
    mlp_loss / mlp_backward; returns (dz fp16 [rows, 32], dweights fp32 [7168])."""
    import torch
    torch.set_num_threads(max(1, threads))
    w1, w2, w3 = (torch.from_numpy(w.astype(np.float32)) for w in mlp_weights(flat16))
    x = torch.from_numpy(np.asarray(x16, dtype=np.float16)).float()
    h1 = torch.relu(x @ w1.T).half().float()
    h2 = torch.relu(h1 @ w2.T).half().float()
    y = (h2 @ w3.T).half()
    dy, _ = mlp_loss(y.numpy(), targets, inputs, real)
    g = torch.from_numpy(dy).float()
    dh2 = ((g @ w3) * (h2 > 0)).half().float()
    dh1 = ((dh2 @ w2) * (h1 > 0)).half().float()
    dz = ((dh1 @ w1).half().float() / 128.0).half()
    dweights = torch.cat([(dh1.T @ x).reshape(-1), (dh2.T @ h1).reshape(-1), (g.T @ h2).reshape(-1)])
    return dz.numpy(), dweights.numpy()


# --------------------------------------------------------------------------------------------
# Router gate (odie/native/runtime.cu:64-92,99-103; odie/model.py:17-22): gate MLP W -> 32 -> G
# (ReLU, no bias; G = align16(levels)), s = 1 below `coarse`, else sigmoid / softplus of the fp16
# logit; the `features[l]` columns of level l (in level order) scaled by fp16(s * visible), columns
# past the levels' features set to 1.  Weights fp16 [32*W + 32*G] = Wg1 [32][W] | Wg2 [G][32]
# (1536 for 16 levels of 2 features).

GATE_SHAPES = ((32, 32), (16, 32))


def _levels_of(features):
    return [l for l, f in enumerate(features) for _ in range(f)]


def gate_weights(flat16, levels=16):
    flat16 = np.asarray(flat16, dtype=np.float16)
    outputs = (levels + 15) // 16 * 16
    width, rest = divmod(flat16.size - 32 * outputs, 32)
    if rest or width < 1:
        raise ValueError('gate weights must hold 32*W + 32*align16(levels) values')
    return flat16[:32 * width].reshape(32, width), flat16[32 * width:].reshape(outputs, 32)


def gate_logits(x16, flat16, levels=16):
    """(hidden fp16 [n, 32], logits fp16 [n, G], magnitude bound of the logits)."""
    w1, w2 = gate_weights(flat16, levels)
    h, _ = mlp_layer(x16, w1, True)
    z, magnitude = mlp_layer(h, w2, False)
    return h, z, magnitude


def gate_values(z16, coarse, softplus=False):
    """s fp32 [n, G] from fp16 logits (odie/native/runtime.cu:72); libm exp in float64, rounded."""
    z = np.asarray(z16, dtype=np.float16).astype(np.float64)
    if softplus:
        s = np.where(z > 20.0, z, np.log1p(np.exp(z)))
    else:
        s = 1.0 / (1.0 + np.exp(-z))
    s = s.astype(np.float32)
    s[:, :coarse] = np.float32(1.0)
    return s


def gate_apply(x16, s, visible=None, features=None):
    """weighted fp16 [n, W]: each column of level l times fp16(s_l * visible_l) (one fp16
    rounding), columns past the levels' features 1."""
    features = [2] * 16 if features is None else list(features)
    s = np.asarray(s, dtype=np.float32)[:, :len(features)]
    vis = np.ones_like(s) if visible is None else np.asarray(visible, dtype=np.float32)
    weight = (s * vis).astype(np.float16).astype(np.float64)
    x = np.asarray(x16, dtype=np.float16).astype(np.float64)
    out = np.ones(x.shape, dtype=np.float16)
    columns = len(_levels_of(features))
    out[:, :columns] = (x[:, :columns] * weight[:, _levels_of(features)]).astype(np.float16)
    return out


def gate_back(x16, value16, s, coarse, softplus=False, visible=None, features=None):
    """parallel_gate_back (odie/native/runtime.cu:77-91): direct fp16 [n, W] (0 past the levels'
    features) and da fp16 [n, L] (loss scale 128 x value's scale), every fp16 operation one
    rounding of the exact result; a level's products are summed in column order from 0."""
    features = [2] * 16 if features is None else list(features)
    levels = len(features)
    x = np.asarray(x16, dtype=np.float16).astype(np.float64)
    value = np.asarray(value16, dtype=np.float16).astype(np.float64)
    s = np.asarray(s, dtype=np.float32)[:, :levels]
    vis = np.ones_like(s) if visible is None else np.asarray(visible, dtype=np.float32)
    weight = (s * vis).astype(np.float16).astype(np.float64)
    columns = _levels_of(features)
    direct = np.zeros(x.shape, dtype=np.float16)
    direct[:, :len(columns)] = (value[:, :len(columns)] * weight[:, columns]).astype(np.float16)
    products = (value * x).astype(np.float16).astype(np.float64)
    reduced = np.zeros(s.shape, dtype=np.float64)
    start = 0
    for level, count in enumerate(features):
        for c in range(start, start + count):
            reduced[:, level] = (reduced[:, level] + products[:, c]).astype(np.float16).astype(np.float64)
        start += count
    incoming = reduced.astype(np.float32) * vis
    if softplus:
        derivative = incoming * (-np.expm1(-s.astype(np.float64))).astype(np.float32)
    else:
        derivative = (incoming * (np.float32(1.0) - s)).astype(np.float32) * s
    derivative = derivative.astype(np.float32)
    derivative[:, :coarse] = np.float32(0.0)
    da = (derivative.astype(np.float16).astype(np.float32) * np.float32(128.0)).astype(np.float16)
    return direct, da


def gate_mlp_backward(x16, h16, da16, flat16, levels=16):
    """Gate MLP backward from the given hidden activations and da [n, L] (zero for the logits past
    L): d(raw) fp16 [n, W] with its magnitude bound, weight gradients float64 [32*W + 32*G] with
    theirs."""
    w1, w2 = (w.astype(np.float64) for w in gate_weights(flat16, levels))
    x, h = (np.asarray(v, dtype=np.float16).astype(np.float64) for v in (x16, h16))
    da = np.zeros((x.shape[0], w2.shape[0]))
    given = np.asarray(da16, dtype=np.float16).astype(np.float64)
    da[:, :given.shape[1]] = given
    dh = np.where(h > 0, da @ w2, 0.0).astype(np.float16).astype(np.float64)
    m1 = np.where(h > 0, np.abs(da) @ np.abs(w2), 0.0)
    dr = (dh @ w1).astype(np.float16)
    dr_magnitude = (np.abs(dh) + m1) @ np.abs(w1)
    dweights = np.concatenate([(dh.T @ x).ravel(), (da.T @ h).ravel()])
    magnitude = np.concatenate([((np.abs(dh) + m1).T @ np.abs(x)).ravel(), (np.abs(da).T @ np.abs(h)).ravel()])
    return dr, dr_magnitude, dweights, magnitude


def gate_upstream(direct16, dr16):
    """hash_router_gradient (odie/native/runtime.cu:99-103): fp16(direct + fp16(dr / 128))."""
    unscaled = (np.asarray(dr16, dtype=np.float16).astype(np.float32) / np.float32(128.0)).astype(np.float16)
    return (np.asarray(direct16, dtype=np.float16).astype(np.float64) + unscaled.astype(np.float64)).astype(np.float16)


def stratified_ids(uniforms, width, height):
    """ids of one stratified batch from fp32 uniforms [batch, 2], the expression of
    odie/data.py:73-80 in numpy fp32: uv = u / side + stratum / side, pixel = trunc(uv * (W, H))
    clamped, id = y * W + x."""
    u = np.asarray(uniforms, dtype=np.float32).reshape(-1, 2)
    batch = u.shape[0]
    side = int(round(batch ** 0.5))
    slots = np.arange(batch)
    strata = np.stack((slots % side, slots // side), axis=1).astype(np.float32) / np.float32(side)
    uv = u / np.float32(side) + strata
    xy = (uv * np.array([width, height], dtype=np.float32)).astype(np.int64)
    return np.clip(xy[:, 1], 0, height - 1) * width + np.clip(xy[:, 0], 0, width - 1)
