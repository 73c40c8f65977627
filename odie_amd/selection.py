"""Selection-side geometry and the GPU selectors: the residual's cell bounds, closure checks,
top-k, the B1 mean-rank admission and the B2 exact greedy (odie/selection.py,
odie/gpu_residual.py:75-179).

The cell bounds come from the encode's own geometry evaluated on the device (odie_cell_bounds):
a pixel's cell is floor(fmaf(R-1, x, 0.5)) of its coordinate, as odie/selection.py:16-55 defines
the map through fp32 thresholds.
"""
import numpy as np
import torch

from . import _lib


def align8(value):
    return (int(value) + 7) // 8 * 8


def cell_bounds(shape, resolution, device='cuda'):
    """(xb, yb, ymap): first pixel column/row of every native cell column/row, [R+1] int32 each
    (odie/gpu_residual.py:49-62), and the cell row of every pixel row."""
    height, width = shape
    if type(resolution) is not int or not 2 <= resolution <= 2 ** 23:
        raise ValueError('Resolution must be an integer between 2 and 2^23')
    xb = torch.empty(resolution + 1, dtype=torch.int32, device=device)
    yb = torch.empty(resolution + 1, dtype=torch.int32, device=device)
    _lib.check(_lib.library().odie_cell_bounds(width, height, resolution, xb.data_ptr(), yb.data_ptr(),
                                               _lib.stream_of(xb)))
    xb, yb = xb.cpu().numpy(), yb.cpu().numpy()
    return xb, yb, np.repeat(np.arange(resolution), np.diff(yb))


def closure_nodes(cells, resolution):
    """Sorted unique closure nodes {c, c+1, c+R, c+R+1} mod align8(R^2) (odie/selection.py:76-79)."""
    cells = np.asarray(cells, dtype=np.int64)
    return np.unique(np.concatenate([cells, cells + 1, cells + resolution, cells + resolution + 1])
                     % align8(resolution ** 2))


def selection_record(selected, nodes, resolution, cap, policy, iterations):
    """The closure check and record of odie/selection.py:90-105: raises unless nodes is exactly
    the closure of the selected cells and fits the cap."""
    selected, nodes = np.asarray(selected, dtype=bool), np.asarray(nodes, dtype=bool)
    closure = closure_nodes(np.flatnonzero(selected), resolution)
    if not np.array_equal(closure, np.flatnonzero(nodes)) or len(closure) > cap:
        raise AssertionError('Selection must preserve its complete node closure')
    used = int(nodes.sum())
    return {
        'policy': policy, 'selected_cells': int(selected.sum()),
        'closure_nodes': used, 'node_capacity': cap,
        'unused_allocated_node_slots': int(cap - used),
        'aligned_used_node_slots': align8(used),
        'node_capacity_utilization': float(used / cap) if cap else 0.,
        'aligned_capacity_utilization': float(align8(used) / cap) if cap else 0.,
        'complete_interpolation_closure': True,
        'tie_order': 'descending score, ascending native cell ID',
        'iterations': iterations,
    }


def uniform_bounds(size, tile):
    """Bounds of equal tiles of `tile` pixels (the last one shorter if size % tile)."""
    return np.array(list(range(0, size, tile)) + [size], dtype=np.int32)


def topk_tiles(scores, k):
    """ids (int32, ascending) of the k largest scores, ties to the lower id -- on the GPU."""
    if scores.dtype != torch.float64 or scores.ndim != 1 or not scores.is_cuda:
        raise ValueError('scores must be a CUDA fp64 vector')
    scores = scores.contiguous()
    ids = torch.empty(k, dtype=torch.int32, device=scores.device)
    _lib.check(_lib.library().odie_topk(scores.data_ptr(), scores.numel(), k, ids.data_ptr(),
                                        _lib.stream_of(scores)))
    return ids


class GreedySelection:
    """Device state of the B2 exact greedy selector (odie/gpu_residual.py:75-128): scores stay
    on the device, the host only polls the four stats words between bounded launches."""

    def __init__(self, scores, resolution, cap, normalize_by_cost=True, trace=False, chunk=512):
        if scores.dtype != torch.float64 or scores.ndim != 1 or not scores.is_cuda:
            raise ValueError('scores must be a CUDA fp64 vector')
        n = resolution * resolution
        if scores.numel() != n:
            raise ValueError('scores must hold resolution^2 cells')
        if cap < 0 or cap % 8 or cap > align8(n):
            raise ValueError('cap must be an 8-aligned node count within align8(resolution^2)')
        device = scores.device
        self.scores = scores.contiguous()
        self.n, self.points, self.resolution, self.cap = n, align8(n), resolution, cap
        self.normalize_by_cost, self.chunk = normalize_by_cost, chunk
        lib = _lib.library()
        self.missing = torch.empty(n, dtype=torch.int32, device=device)
        self.chosen = torch.empty(n, dtype=torch.uint8, device=device)
        self.nodes = torch.empty(self.points, dtype=torch.uint8, device=device)
        self.tree = torch.empty(int(lib.odie_selection_tree_ints(n)), dtype=torch.int32, device=device)
        self.stats = torch.empty(4, dtype=torch.int64, device=device)
        self.trace = torch.full((n,), -1, dtype=torch.int32, device=device) if trace else None
        self.launches = 0

    def run(self):
        """Select until done; returns (selected bool [n], nodes bool [points], iterations)."""
        lib, stream = _lib.library(), _lib.stream_of(self.scores)
        _lib.check(lib.selection_init(self.scores.data_ptr(), self.n, self.points, self.missing.data_ptr(),
                                      self.chosen.data_ptr(), self.nodes.data_ptr(), self.tree.data_ptr(),
                                      self.stats.data_ptr(), None, None, 0, stream))
        trace = self.trace.data_ptr() if self.trace is not None else None
        while True:
            _lib.check(lib.selection_chunk(self.scores.data_ptr(), self.n, self.points, self.resolution, self.cap,
                                           self.normalize_by_cost, self.missing.data_ptr(), self.chosen.data_ptr(),
                                           self.nodes.data_ptr(), self.tree.data_ptr(), None, None, 0, self.chunk,
                                           self.stats.data_ptr(), trace, stream))
            self.launches += 1
            stats = self.stats.cpu()
            if stats[3]:
                raise AssertionError('device greedy: exact marginal cost invariant failed')
            if stats[2]:
                break
        used, iterations = int(stats[0]), int(stats[1])
        selected, nodes = self.chosen.bool(), self.nodes.bool()
        if int(nodes.sum()) != used:
            raise AssertionError('device greedy: node count and stats disagree')
        return selected, nodes, iterations


def select_device(scores, resolution, cap, normalize_by_cost=True, trace=False, chunk=512):
    """B2 exact greedy over device-resident fp64 scores (odie/gpu_residual.py:75).  Returns
    (selected, nodes, iterations[, trace int32 [iterations]])."""
    state = GreedySelection(scores, resolution, cap, normalize_by_cost, trace, chunk)
    selected, nodes, iterations = state.run()
    if trace:
        return selected, nodes, iterations, state.trace[:iterations]
    return selected, nodes, iterations


def select_mean_rank(mean, resolution, cap):
    """B1 (odie/selection.py:108-126) on the device: cells ranked by descending score, ties by
    ascending cell id, each admitted when the closure nodes it adds keep the count within the
    node cap (odie_select_mean_rank).  mean: fp64 scores [R^2] (CUDA); the reference's argument
    checks and its record.  Returns (selected bool [R^2] on the device, record)."""
    mean = torch.as_tensor(mean)
    if (mean.dtype != torch.float64 or mean.ndim != 1 or mean.numel() != resolution ** 2
            or not bool(torch.isfinite(mean).all()) or bool((mean < 0).any())):
        raise ValueError('Scores must be a finite nonnegative R^2 vector')
    if type(cap) is not int or cap % 8 or not 0 <= cap <= align8(resolution ** 2):
        raise ValueError('Node cap must be 8-aligned and within the native plane')
    mean = mean.to('cuda' if not mean.is_cuda else mean.device).contiguous()
    lib, device = _lib.library(), mean.device
    need = int(lib.odie_select_mean_rank_workspace(resolution))
    if need < 0:
        raise ValueError('resolution^2 must be within 1..2^24')
    n = resolution * resolution
    workspace = torch.empty(need, dtype=torch.uint8, device=device)
    chosen = torch.empty(n, dtype=torch.uint8, device=device)
    nodes = torch.empty(align8(n), dtype=torch.uint8, device=device)
    stats = torch.empty(2, dtype=torch.int64, device=device)
    _lib.check(lib.odie_select_mean_rank(mean.data_ptr(), resolution, cap, chosen.data_ptr(), nodes.data_ptr(),
                                         stats.data_ptr(), workspace.data_ptr(), need, _lib.stream_of(mean)))
    selected = chosen.bool()
    record = selection_record(selected.cpu().numpy(), nodes.bool().cpu().numpy(), resolution, cap,
                              'B1 live RGB region mean; stable cell ranking adapted to complete node cap',
                              int(stats[1]))
    return selected, record
