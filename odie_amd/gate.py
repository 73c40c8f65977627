"""The router gate on the GPU: gate MLP 32 -> 32 -> 16 (the `gate` head of odie/hash_grid.py:28-30)
and the per-level feature gating of the native step (odie/native/runtime.cu:64-92,99-103).

Gate keeps an fp32 master of the 1536 weights (Wg1 [32][32] | Wg2 [16][32], row-major
[out][in]) and their fp16 copy.  forward(raw) gives the decoder's input; backward(raw, value)
turns the decoder's input gradient into the grid's upstream and fills self.grad.
"""
import math

import numpy as np
import torch

from . import _lib, synth

LEVELS, INPUT, HIDDEN = 16, 32, 32
SHAPES = ((HIDDEN, INPUT), (LEVELS, HIDDEN))
PARAMETERS = sum(rows * cols for rows, cols in SHAPES)   # 1536 (odie/config.py:176-177)


def initial_weights(seed):
    parts = []
    for index, (rows, cols) in enumerate(SHAPES):
        bound = math.sqrt(6.0 / (rows + cols))
        u = synth.uniform(seed, 'gate%d' % index, rows * cols).astype(np.float64)
        parts.append(((2.0 * u - 1.0) * bound).astype(np.float32))
    return np.concatenate(parts)


class Gate:
    def __init__(self, weights=None, seed=0, coarse=0, activation='sigmoid', device='cuda'):
        if activation not in ('sigmoid', 'softplus'):
            raise ValueError('activation must be sigmoid or softplus (odie/model.py:17-22)')
        values = initial_weights(seed) if weights is None else np.asarray(weights, dtype=np.float32)
        if values.shape != (PARAMETERS,):
            raise ValueError('gate weights must be fp32 [%d]' % PARAMETERS)
        self.params = torch.from_numpy(values.copy()).to(device)
        self.half = self.params.half()
        self.grad = torch.zeros(PARAMETERS, dtype=torch.float32, device=device)
        self.coarse, self.softplus = int(coarse), activation == 'softplus'

    def sync_weights(self):
        self.half.copy_(self.params)

    def forward(self, raw, visible=None, weighted=None, sigmoid=None):
        raw = _rows(raw)
        n = raw.shape[0]
        weighted = torch.empty_like(raw) if weighted is None else weighted
        sigmoid = torch.empty((n, LEVELS), dtype=torch.float32, device=raw.device) if sigmoid is None else sigmoid
        _lib.check(_lib.library().odie_gate_forward(raw.data_ptr(), n, self.half.data_ptr(), _lib.ptr(visible),
                                                    self.coarse, int(self.softplus), weighted.data_ptr(),
                                                    sigmoid.data_ptr(), _lib.stream_of(raw)))
        return weighted, sigmoid

    def backward(self, raw, value, sigmoid, visible=None, upstream=None):
        raw, value = _rows(raw), _rows(value)
        upstream = torch.empty_like(raw) if upstream is None else upstream
        _lib.check(_lib.library().odie_gate_backward(raw.data_ptr(), value.data_ptr(), raw.shape[0], self.half.data_ptr(),
                                                     _lib.ptr(visible), sigmoid.data_ptr(), self.coarse,
                                                     int(self.softplus), upstream.data_ptr(), self.grad.data_ptr(),
                                                     _lib.stream_of(raw)))
        return upstream


def _rows(x):
    if x.dtype != torch.float16 or x.ndim != 2 or x.shape[1] != INPUT or not x.is_cuda:
        raise ValueError('gate rows must be CUDA fp16 [n, %d]' % INPUT)
    return x.contiguous()
