"""The router gate on the GPU: gate MLP width -> 32 -> G (the `gate` head of odie/hash_grid.py:28-30
and odie/model.py:186-195; G = align16(levels)) and the per-level feature gating of the native
step (odie/native/runtime.cu:64-92,99-103).

Gate keeps an fp32 master of its 32*width + 32*G weights (Wg1 [32][width] | Wg2 [G][32],
row-major [out][in]; 1536 for 16 levels of 2 features) and their fp16 copy.  Level l owns
`features[l]` consecutive columns of a row (1, 2 or 4), in level order; width is align16 of their
sum.  forward(raw) gives the decoder's input; backward(raw, value) turns the decoder's input
gradient into the grid's upstream and fills self.grad.
"""
import ctypes
import math

import numpy as np
import torch

from . import _lib, synth

LEVELS, INPUT, HIDDEN = 16, 32, 32


def _align16(value):
    return (int(value) + 15) // 16 * 16


def shapes(width=INPUT, levels=LEVELS):
    return ((HIDDEN, width), (_align16(levels), HIDDEN))


def parameter_count(width=INPUT, levels=LEVELS):
    """32*width + 32*align16(levels) (odie/config.py:176): 1536 at 16 levels of 2 features."""
    return sum(rows * cols for rows, cols in shapes(width, levels))


SHAPES = shapes()
PARAMETERS = parameter_count()


def initial_weights(seed, width=INPUT, levels=LEVELS):
    parts = []
    for index, (rows, cols) in enumerate(shapes(width, levels)):
        bound = math.sqrt(6.0 / (rows + cols))
        u = synth.uniform(seed, 'gate%d' % index, rows * cols).astype(np.float64)
        parts.append(((2.0 * u - 1.0) * bound).astype(np.float32))
    return np.concatenate(parts)


class Gate:
    def __init__(self, weights=None, seed=0, coarse=0, activation='sigmoid', device='cuda', features=None):
        if activation not in ('sigmoid', 'softplus'):
            raise ValueError('activation must be sigmoid or softplus (odie/model.py:17-22)')
        self.features = [2] * LEVELS if features is None else [int(f) for f in features]
        if not 1 <= len(self.features) <= 32 or any(f not in (1, 2, 4) for f in self.features):
            raise ValueError('the gate takes 1..32 levels of 1, 2 or 4 features')
        self.levels = len(self.features)
        self.width = _align16(sum(self.features))
        if self.width > 80:
            raise ValueError('the levels\' features exceed the 80 columns the gate is built for')
        count = parameter_count(self.width, self.levels)
        values = (initial_weights(seed, self.width, self.levels) if weights is None
                  else np.asarray(weights, dtype=np.float32))
        if values.shape != (count,):
            raise ValueError('gate weights must be fp32 [%d]' % count)
        self.params = torch.from_numpy(values.copy()).to(device)
        self.half = self.params.half()
        self.grad = torch.zeros(count, dtype=torch.float32, device=device)
        self.coarse, self.softplus = int(coarse), activation == 'softplus'
        self._table = (ctypes.c_int32 * self.levels)(*self.features)   # host int32 [levels]

    def sync_weights(self):
        self.half.copy_(self.params)

    def forward(self, raw, visible=None, weighted=None, sigmoid=None):
        raw = self._rows(raw)
        n = raw.shape[0]
        weighted = torch.empty_like(raw) if weighted is None else weighted
        sigmoid = torch.empty((n, self.levels), dtype=torch.float32, device=raw.device) if sigmoid is None else sigmoid
        _lib.check(_lib.library().odie_gate_forward(raw.data_ptr(), n, self.width, self.levels, self._table,
                                                    self.half.data_ptr(), _lib.ptr(visible), self.coarse,
                                                    int(self.softplus), weighted.data_ptr(), sigmoid.data_ptr(),
                                                    _lib.stream_of(raw)))
        return weighted, sigmoid

    def backward(self, raw, value, sigmoid, visible=None, upstream=None):
        raw, value = self._rows(raw), self._rows(value)
        upstream = torch.empty_like(raw) if upstream is None else upstream
        _lib.check(_lib.library().odie_gate_backward(raw.data_ptr(), value.data_ptr(), raw.shape[0], self.width,
                                                     self.levels, self._table, self.half.data_ptr(),
                                                     _lib.ptr(visible), sigmoid.data_ptr(), self.coarse,
                                                     int(self.softplus), upstream.data_ptr(), self.grad.data_ptr(),
                                                     _lib.stream_of(raw)))
        return upstream

    def _rows(self, x):
        if x.dtype != torch.float16 or x.ndim != 2 or x.shape[1] != self.width or not x.is_cuda:
            raise ValueError('gate rows must be CUDA fp16 [n, %d]' % self.width)
        return x.contiguous()
