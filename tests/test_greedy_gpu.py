"""B2 exact greedy on the device (selection_init / selection_chunk) against the oracle's heap
restatement of odie/selection.py:129-207: chosen cells, closure nodes, iteration count and the
order of choices are bit-exact."""
import numpy as np
import pytest
import torch

import oracle
from odie_amd import synth
from odie_amd.selection import align8, select_device

pytestmark = pytest.mark.gpu


def _scores(seed, cells, ties):
    if ties:
        # few distinct values, signed zeros: exercises every tie rule
        values = synth.integers(seed, 'greedy', cells, 6).astype(np.float64) * 0.5
        values[synth.integers(seed, 'negzero', cells, 4) == 0] = -0.0
    else:
        values = synth.uniform(seed, 'greedy', cells).astype(np.float64) ** 3
    return values


def _check(values, resolution, cap, normalize=True, chunk=512):
    trace = []
    selected, nodes, iterations = oracle.select_benefit_cost(values, resolution, cap, normalize_by_cost=normalize,
                                                             trace=trace)
    got_selected, got_nodes, got_iterations, got_trace = select_device(
        torch.from_numpy(values).cuda(), resolution, cap, normalize_by_cost=normalize, trace=True, chunk=chunk)
    assert got_iterations == iterations
    assert np.array_equal(got_trace.cpu().numpy(), np.asarray(trace, dtype=np.int32))
    assert np.array_equal(got_selected.cpu().numpy(), selected)
    assert np.array_equal(got_nodes.cpu().numpy(), nodes)


@pytest.mark.parametrize('resolution', [2, 3, 5, 8])
@pytest.mark.parametrize('ties', [False, True])
def test_tiny_grids_every_cap(resolution, ties):
    values = _scores(resolution, resolution * resolution, ties)
    for cap in range(0, align8(resolution * resolution) + 1, 8):
        _check(values, resolution, cap)


@pytest.mark.parametrize('resolution,cap,ties,normalize', [
    (64, 1024, False, True),      # two tree levels, all in LDS
    (64, 4096, True, True),       # cap = every node: all cells end selected
    (100, 2000, True, True),      # three levels, ragged last node
    (100, 2000, False, False),    # unnormalized: raw score order under the node cap
    (181, 9000, True, True),
])
def test_medium_grids(resolution, cap, ties, normalize):
    _check(_scores(7, resolution * resolution, ties), resolution, cap, normalize)


def test_chunk_boundaries_do_not_change_the_result():
    values = _scores(11, 48 * 48, True)
    _check(values, 48, 512, chunk=1)
    _check(values, 48, 512, chunk=3)


def test_large_grid_with_device_resident_tree_levels():
    # 448^2 cells: the level-0 nodes exceed the LDS-resident part, so the lowest tree level
    # is repaired in device memory
    _check(_scores(5, 448 * 448, False), 448, 8192)


def test_zero_scores_still_fill_capacity():
    values = np.zeros(32 * 32)
    _check(values, 32, 256)
