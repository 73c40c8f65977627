"""Host-side geometry of the selection path and the GPU top-k.

native_thresholds restates odie/selection.py:16-42: for each region 1..R-1 the smallest fp32
x in [0,1] with floor(fma(R-1, x, 0.5)) >= region, found by binary search over fp32 bit
patterns against the exact rational rounding boundary of the fused result.  It is host set-up
(the column/row bounds of the residual's cells), computed once per resolution.
"""
from functools import lru_cache
import struct

import numpy as np
import torch

from . import _lib


def align8(value):
    return (int(value) + 7) // 8 * 8


def _float_from_bits(bits):
    return struct.unpack('<f', struct.pack('<I', bits))[0]


@lru_cache(maxsize=128)
def native_thresholds(resolution):
    if type(resolution) is not int or not 2 <= resolution <= 2 ** 23:
        raise ValueError('Resolution must be an integer between 2 and 2^23')
    scale = resolution - 1
    out = []
    for region in range(1, resolution):
        region_bits = struct.unpack('<I', struct.pack('<f', region))[0]
        # fma rounds up to `region` once scale*x + 0.5 passes the midpoint between `region`
        # and its fp32 predecessor; ties round to the even neighbour.
        below_num, below_den = _float_from_bits(region_bits - 1).as_integer_ratio()
        boundary_num = (region - 1) * below_den + below_num
        boundary_den = 2 * below_den
        even = region_bits % 2 == 0
        lower, upper = 0, 0x3F800000
        while lower < upper:
            middle = (lower + upper) // 2
            numerator, denominator = _float_from_bits(middle).as_integer_ratio()
            left, right = scale * numerator * boundary_den, boundary_num * denominator
            if left > right or (left == right and even):
                upper = middle
            else:
                lower = middle + 1
        out.append(_float_from_bits(lower))
    return tuple(out)


def cell_bounds(shape, resolution):
    """(xb, yb): first pixel column/row of every native cell column/row (odie/gpu_residual.py:49-62)."""
    height, width = shape
    thresholds = np.asarray(native_thresholds(resolution), dtype=np.float32)
    xmap = np.searchsorted(thresholds, np.arange(width, dtype=np.float32) / np.float32(width - 1), side='right')
    ymap = np.searchsorted(thresholds, np.arange(height, dtype=np.float32) / np.float32(height - 1), side='right')
    bounds = np.arange(resolution + 1)
    return (np.searchsorted(xmap, bounds).astype(np.int32), np.searchsorted(ymap, bounds).astype(np.int32), ymap)


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
