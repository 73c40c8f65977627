"""Streamed per-cell residual totals on the GPU (odie/gpu_residual.py:49-72).

DeviceScores keeps fp64 totals on the device and adds one streamed chunk of predictions at a
time through score_chunk, in raster order, so the totals equal the reference's sequential
CPU rule (odie/selection.py:58-73) bit for bit.
"""
import numpy as np
import torch

from . import _lib
from .selection import cell_bounds, uniform_bounds


class DeviceScores:
    """Cells are the native geometry cells at `resolution` (the reference's convention), or
    equal tiles of `tile` pixels when tile is given."""

    def __init__(self, shape, resolution=None, tile=None, device='cuda'):
        height, width = shape
        self.shape = shape
        if tile is not None:
            xb, yb = uniform_bounds(width, tile), uniform_bounds(height, tile)
            if len(xb) != len(yb):
                raise ValueError('uniform tiles need as many tile columns as rows')
            self.resolution = len(xb) - 1
            self.ymap = np.repeat(np.arange(self.resolution), np.diff(yb))
        else:
            self.resolution = resolution
            xb, yb, self.ymap = cell_bounds(shape, resolution, device=device)
        self.counts = (np.diff(yb).astype(np.int64)[:, None] * np.diff(xb)[None, :]).reshape(-1)
        self.xb = torch.from_numpy(xb).to(device)
        self.yb = torch.from_numpy(yb).to(device)
        self.totals = torch.zeros(self.resolution ** 2, dtype=torch.float64, device=device)

    def add(self, prediction, target, begin):
        prediction, target = prediction.contiguous(), target.contiguous()
        if prediction.dtype != torch.float32 or prediction.shape[-1] != 3:
            raise ValueError('prediction must be fp32 [N, 3]')
        if target.dtype not in (torch.uint8, torch.float32) or target.shape != prediction.shape:
            raise ValueError('target must be uint8 or fp32 of the prediction shape')
        end, width = begin + prediction.shape[0], self.shape[1]
        if end == begin:
            return
        first_y = int(self.ymap[begin // width])
        active = (int(self.ymap[(end - 1) // width]) - first_y + 1) * self.resolution
        _lib.check(_lib.library().score_chunk(
            prediction.data_ptr(), target.data_ptr(), begin, end, width, self.resolution, first_y, active,
            self.xb.data_ptr(), self.yb.data_ptr(), self.totals.data_ptr(), target.dtype == torch.uint8,
            _lib.stream_of(prediction)))
