"""GPU residual totals (score_chunk) and top-k against the oracle: bit-exact."""
import numpy as np
import pytest
import torch

import oracle
from odie_amd import synth
from odie_amd.gpu_residual import DeviceScores
from odie_amd.selection import topk_tiles

pytestmark = pytest.mark.gpu


def _image(seed, shape):
    pixels = shape[0] * shape[1]
    prediction = synth.uniform(seed, 'prediction', pixels * 3).reshape(pixels, 3)
    target = synth.integers(seed, 'target', pixels * 3, 256).astype(np.uint8).reshape(pixels, 3)
    return prediction, target


@pytest.mark.parametrize('rgb8', [True, False])
@pytest.mark.parametrize('shape,resolution,tile,chunks', [
    ((137, 211), 16, None, [0, 5000, 5001, 20000, 137 * 211]),     # native cells, ragged chunks
    ((512, 512), None, 64, [0, 512 * 512]),                          # uniform 64x64 tiles
    ((300, 257), 13, None, [0, 300 * 257]),
])
def test_residual_bit_exact(rgb8, shape, resolution, tile, chunks):
    prediction, target = _image(1, shape)
    if not rgb8:
        target = (target.astype(np.float32) / np.float32(255.0)).astype(np.float32)
    scores = DeviceScores(shape, resolution=resolution, tile=tile)
    for begin, end in zip(chunks[:-1], chunks[1:]):
        scores.add(torch.from_numpy(prediction[begin:end]).cuda(), torch.from_numpy(target[begin:end]).cuda(), begin)
    got = scores.totals.cpu().numpy()
    expected = np.zeros(scores.resolution ** 2)
    xb, yb = scores.xb.cpu().numpy(), scores.yb.cpu().numpy()
    for begin, end in zip(chunks[:-1], chunks[1:]):
        oracle.residual(prediction[begin:end], target[begin:end], shape[1], scores.resolution, xb, yb, begin=begin,
                        totals=expected)
    assert np.array_equal(got.view(np.uint64), expected.view(np.uint64))
    assert scores.counts.sum() == shape[0] * shape[1]


@pytest.mark.parametrize('n,k', [(16384, 512), (1000, 1), (1000, 1000), (70000, 4096), (37, 5)])
def test_topk_matches_oracle(n, k):
    values = synth.integers(3, 'scores', n, 50).astype(np.float64) * 0.125   # many ties
    values[::7] = synth.uniform(3, 'fine', len(values[::7])).astype(np.float64)
    values[3] = -0.0
    values[4] = 0.0
    ids = topk_tiles(torch.from_numpy(values).cuda(), k).cpu().numpy()
    assert np.array_equal(ids, oracle.topk_ids(values, k))


@pytest.mark.parametrize('shape,resolution', [((1365, 2048), 8), ((61, 97), 13), ((1000, 1000), 128), ((5, 7), 2),
                                              ((64, 64), 1290), ((2040, 1536), 764)])
def test_cell_bounds_match_the_oracle_thresholds(shape, resolution):
    """odie_cell_bounds (the encode's fmaf geometry on the device) against the oracle's exact fp32
    thresholds (pinned by exact rational arithmetic): the first pixel of every cell column/row."""
    from odie_amd.selection import cell_bounds
    height, width = shape
    xb, yb, ymap = cell_bounds(shape, resolution)
    thresholds = oracle.native_thresholds(resolution)
    def expected(size):
        cells = np.searchsorted(thresholds, np.arange(size, dtype=np.float32) / np.float32(size - 1), side='right')
        return np.searchsorted(cells, np.arange(resolution + 1)).astype(np.int32), cells
    want_x, _ = expected(width)
    want_y, rows = expected(height)
    assert np.array_equal(xb, want_x) and np.array_equal(yb, want_y)
    assert np.array_equal(ymap, rows)
