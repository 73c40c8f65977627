"""B1 mean-rank admission on the device (odie_select_mean_rank) against the oracle's restatement
of odie/selection.py:108-126 (pinned by a brute force over every subset of tiny grids): chosen
cells, closure nodes and the walk's length bit-exact, with planted ties and signed zeros, caps
that end the walk early, late and never, and grid sizes from one cell to the DIV2K layout's
finest level (1020^2 cells)."""
import numpy as np
import pytest
import torch

import oracle
from odie_amd import synth
from odie_amd.selection import align8, select_mean_rank

pytestmark = pytest.mark.gpu


def _scores(seed, cells, ties):
    if ties:
        values = synth.integers(seed, 'b1', cells, 5).astype(np.float64) * 0.25
        values[synth.integers(seed, 'b1_negzero', cells, 3) == 0] = -0.0
    else:
        values = synth.uniform(seed, 'b1', cells).astype(np.float64) ** 4
    return values


def _check(values, resolution, cap):
    print('B1 on the device: R=%d, cap %d' % (resolution, cap), flush=True)
    want_selected, want_nodes = oracle.select_mean_rank(values, resolution, cap)
    selected, record = select_mean_rank(torch.from_numpy(values).cuda(), resolution, cap)
    assert np.array_equal(selected.cpu().numpy(), want_selected)
    assert record['closure_nodes'] == int(want_nodes.sum()) and record['iterations'] == resolution ** 2
    assert record['selected_cells'] == int(want_selected.sum())


@pytest.mark.parametrize('resolution', [1, 2, 3, 5, 8])
@pytest.mark.parametrize('ties', [False, True])
def test_tiny_grids_every_cap(resolution, ties):
    values = _scores(resolution, resolution ** 2, ties)
    for cap in range(0, align8(resolution ** 2) + 1, 8):
        _check(values, resolution, cap)


@pytest.mark.parametrize('resolution,cap,ties', [
    (33, 256, True), (64, 1024, False), (64, 4096, True),     # the walk ends early, late, never
    (128, 2048, True), (128, 16384, False),                   # the 16384 residual tiles
    (1020, 87968, True), (1020, 87968, False),                # DIV2K L16's finest level and node cap
    (1023, 8, False),                                         # n not a multiple of the tile
])
def test_larger_grids(resolution, cap, ties):
    _check(_scores(resolution + cap, resolution ** 2, ties), resolution, cap)


def test_all_equal_scores_admit_in_id_order():
    values = np.zeros(40 * 40)
    _check(values, 40, 200)


def test_rejects_what_the_reference_rejects():
    with pytest.raises(ValueError, match='finite nonnegative'):
        select_mean_rank(torch.full((16,), -1.0, dtype=torch.float64, device='cuda'), 4, 8)
    with pytest.raises(ValueError, match='finite nonnegative'):
        select_mean_rank(torch.full((16,), float('nan'), dtype=torch.float64, device='cuda'), 4, 8)
    with pytest.raises(ValueError, match='8-aligned'):
        select_mean_rank(torch.zeros(16, dtype=torch.float64, device='cuda'), 4, 12)
