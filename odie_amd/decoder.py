"""The decoder head on the GPU: TCNN FullyFusedMLP width -> 64 -> 64 -> 16 (ReLU, no bias, no
output activation, fp16), as configured at odie/hash_grid.py:32-34, odie/model.py:186-195 and
odie/native/runtime.cu:151-162,190, with width = align16 of the grid's feature count (16..80;
odie/config.py:175-176).

Decoder keeps an fp32 master of the 64*width + 5120 weights (W1 [64][width] | W2 [64][64] |
W3 [16][64], row-major [out][in]; 7168 at width 32) and their fp16 copy, which the kernels read.
`train` runs forward, the native step's loss (odie/native/runtime.cu:53-63) and backward in one
launch.
"""
import math

import numpy as np
import torch

from . import _lib, synth

INPUT, HIDDEN, OUTPUT = 32, 64, 16
WIDTHS = (16, 32, 48, 64, 80)
LEVELS = INPUT // 2   # grid levels of 2 features in the 32-wide planes layout


def shapes(width=INPUT):
    return ((HIDDEN, width), (HIDDEN, HIDDEN), (OUTPUT, HIDDEN))


def parameter_count(width=INPUT):
    """64*width + 5120 (odie/config.py:176): 7168 at width 32."""
    return sum(rows * cols for rows, cols in shapes(width))


SHAPES = shapes()
PARAMETERS = parameter_count()


def initial_weights(seed, width=INPUT):
    """fp32 [64*width + 5120]: each layer uniform in +-sqrt(6 / (fan_in + fan_out)) from the
    counter PRNG."""
    parts = []
    for index, (rows, cols) in enumerate(shapes(width)):
        bound = math.sqrt(6.0 / (rows + cols))
        u = synth.uniform(seed, 'decoder%d' % index, rows * cols).astype(np.float64)
        parts.append(((2.0 * u - 1.0) * bound).astype(np.float32))
    return np.concatenate(parts)


class Decoder:
    def __init__(self, weights=None, seed=0, device='cuda', width=INPUT):
        if width not in WIDTHS:
            raise ValueError('decoder width must be one of %s' % (WIDTHS,))
        self.width = width
        count = parameter_count(width)
        values = initial_weights(seed, width) if weights is None else np.asarray(weights, dtype=np.float32)
        if values.shape != (count,):
            raise ValueError('decoder weights must be fp32 [%d]' % count)
        self.params = torch.from_numpy(values.copy()).to(device)
        self.half = self.params.half()
        self.grad = torch.zeros(count, dtype=torch.float32, device=device)

    def sync_weights(self):
        """Refresh the fp16 copy from the fp32 master (odie_sync_weights)."""
        self.half.copy_(self.params)

    def forward(self, x):
        x = _features(x, self.width)
        out = torch.empty((x.shape[0], OUTPUT), dtype=torch.float16, device=x.device)
        _lib.check(_lib.library().odie_mlp_forward(x.data_ptr(), x.shape[0], self.width, self.half.data_ptr(),
                                                   out.data_ptr(), _lib.stream_of(x)))
        return out

    def train(self, x, real=None, *, colors=None, pixels=None, rgb=None, ids=None, target=None, rows=None, out=None,
              hidden=None, squares=None, dz=None):
        """Forward + loss + backward.  Returns dz fp16 [n, width] (the grid's upstream at loss
        scale 128); self.grad receives dL/dW at loss scale 16384.  The target of row j: colors[j]
        (packed RGB8), or the pixel pixels[j] of rgb, or pixel ids[rows[j]] of rgb, or target."""
        x = _features(x, self.width)
        n = x.shape[0]
        real = n if real is None else int(real)
        colors, rgb, ids = _target_source(colors, pixels, rgb, ids, target)
        if dz is None:
            dz = torch.empty((n, self.width), dtype=torch.float16, device=x.device)
        _lib.check(_lib.library().odie_mlp_train(
            x.data_ptr(), n, self.width, real, self.half.data_ptr(), _lib.ptr(colors), _lib.ptr(rgb), _lib.ptr(ids), _lib.ptr(target),
            _lib.ptr(rows), _lib.ptr(out), _lib.ptr(hidden), _lib.ptr(squares), dz.data_ptr(), self.grad.data_ptr(),
            _lib.stream_of(x)))
        return dz

    def train_planes(self, x, real=None, *, colors=None, pixels=None, rgb=None, ids=None, target=None, rows=None,
                     out=None, hidden=None, squares=None, planes=None, blockmax=None):
        """train() with dz written for ExpertGrid.backward_adam_planes: planes int32 [16, n] (the
        fp16 feature pair of each level and row) and blockmax fp32 [ceil(n/128), 32] (max |dz|
        per 128-row record and column: level l, feature f at 2l + f).  Returns (planes, blockmax).
        Width 32 only."""
        if self.width != INPUT:
            raise ValueError('the planes layout is built for width 32 (16 levels x 2 features)')
        x = _features(x, self.width)
        n = x.shape[0]
        real = n if real is None else int(real)
        colors, rgb, ids = _target_source(colors, pixels, rgb, ids, target)
        records = (n + 127) // 128
        if planes is None:
            planes = torch.empty((LEVELS, n), dtype=torch.int32, device=x.device)
        if blockmax is None:
            blockmax = torch.empty((records, 2 * LEVELS), dtype=torch.float32, device=x.device)
        if tuple(planes.shape) != (LEVELS, n) or planes.dtype != torch.int32 or not planes.is_contiguous():
            raise ValueError('planes must be a contiguous int32 [16, n] tensor')
        if (tuple(blockmax.shape) != (records, 2 * LEVELS) or blockmax.dtype != torch.float32
                or not blockmax.is_contiguous()):
            raise ValueError('blockmax must be a contiguous fp32 [ceil(n/128), 32] tensor')
        _lib.check(_lib.library().odie_mlp_train_planes(
            x.data_ptr(), n, real, self.half.data_ptr(), _lib.ptr(colors), _lib.ptr(rgb), _lib.ptr(ids),
            _lib.ptr(target), _lib.ptr(rows), _lib.ptr(out), _lib.ptr(hidden), _lib.ptr(squares), planes.data_ptr(),
            blockmax.data_ptr(), self.grad.data_ptr(), _lib.stream_of(x)))
        return planes, blockmax


def _target_source(colors, pixels, rgb, ids, target):
    """The (colors, rgb, ids) arguments of odie_mlp_train for one target source: packed colors;
    pixel indexes with the image (passed as colors with rgb); rgb with ids; or fp32 target."""
    given = [colors is not None, pixels is not None, ids is not None, target is not None]
    if sum(given) != 1 or (pixels is not None or ids is not None) != (rgb is not None):
        raise ValueError('give colors, pixels with rgb, rgb with ids, or target')
    if pixels is not None:
        return pixels, rgb, None
    return colors, rgb, ids


def _features(x, width):
    if x.dtype != torch.float16 or x.ndim != 2 or x.shape[1] != width or not x.is_cuda:
        raise ValueError('decoder input must be CUDA fp16 [n, %d]' % width)
    return x.contiguous()
