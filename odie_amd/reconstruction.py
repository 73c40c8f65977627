"""Streamed full-image reconstruction of the multi-expert model and its residual scores on the
GPU: the inference + scoring part of the reference's select_live (odie/gpu_residual.py:130-179)
and evaluate (odie/evaluation.py:12-36), with the encode and the decoder fused in one kernel
(odie_reconstruct) so the features never reach memory.

Pixels are visited in raster order in batches; each batch's prediction is scored into the
per-cell fp64 totals (DeviceScores, score_chunk) in that order, so the totals are the
reference's sequential rule bit for bit, and the mse is the reference's torch expression.
"""
import math

import torch

from . import _lib
from .gpu_residual import DeviceScores


def reconstruct(grid, decoder_half, shape, regions, begin, n, *, slots=None, prediction=None, features=None,
                output=None):
    """Predictions of pixels [begin, begin+n) (raster ids) through `grid` (an ExpertGrid with fp16
    F=2 tables, one expert per tile of a regions = (regions_x, regions_y) grid, or per slot when
    slots maps tiles to table slots) and the decoder's fp16 weights.  Returns prediction fp32
    [n, 3] (allocated when not given); features [n, 32] / output [n, 16] fp16 are filled when
    given."""
    height, width = shape
    regions_x, regions_y = regions
    if grid.table.dtype != torch.float16 or grid.features != 2:
        raise ValueError('the fused reconstruction reads fp16 tables of 2 features per level')
    if slots is not None and (slots.dtype != torch.int32 or slots.numel() != regions_x * regions_y):
        raise ValueError('slots must be int32 [regions_x * regions_y]')
    device = grid.table.device
    if prediction is None and features is None and output is None:
        prediction = torch.empty((n, 3), dtype=torch.float32, device=device)
    for name, tensor, shape_ in (('prediction', prediction, (n, 3)), ('features', features, (n, 32)),
                                 ('output', output, (n, 16))):
        if tensor is not None and (tuple(tensor.shape) != shape_ or not tensor.is_contiguous()):
            raise ValueError('%s must be a contiguous %s tensor' % (name, shape_))
    _lib.check(_lib.library().odie_reconstruct(
        begin, n, width, height, regions_x, regions_y, _lib.ptr(slots), grid.experts, grid.table.data_ptr(),
        grid.expert_params, grid.levels, len(grid.levels), decoder_half.data_ptr(), _lib.ptr(prediction),
        _lib.ptr(features), _lib.ptr(output), _lib.stream_of(grid.table)))
    return prediction


@torch.no_grad()
def score_image(grid, decoder_half, target, shape, regions, *, resolution=None, tile=None, batch=1 << 24,
                slots=None, fused=True, prediction=None):
    """Reconstruct the whole image and score it: returns ({'mse', 'psnr_db'}, DeviceScores).
    target: CUDA uint8 [H*W, 3].  Cells are the native geometry cells at `resolution`, or
    uniform tiles of `tile` pixels (DeviceScores).  fused: one odie_reconstruct_scores launch
    (a wave per cell, no prediction in memory unless `prediction` [H*W, 3] is given); otherwise
    batches of `batch` pixels through odie_reconstruct and score_chunk with the reference's torch
    mse."""
    height, width = shape
    pixels = height * width
    if target.dtype != torch.uint8 or tuple(target.shape) != (pixels, 3):
        raise ValueError('target must be uint8 [H*W, 3]')
    scores = DeviceScores(shape, resolution=resolution, tile=tile, device=target.device)
    if fused:
        if grid.table.dtype != torch.float16 or grid.features != 2:
            raise ValueError('the fused reconstruction reads fp16 tables of 2 features per level')
        if prediction is not None and (tuple(prediction.shape) != (pixels, 3) or prediction.dtype != torch.float32):
            raise ValueError('prediction must be fp32 [H*W, 3]')
        squares = torch.zeros(scores.resolution ** 2, dtype=torch.float64, device=target.device)
        xb, yb = scores.xb.to(torch.int32).contiguous(), scores.yb.to(torch.int32).contiguous()
        _lib.check(_lib.library().odie_reconstruct_scores(
            width, height, regions[0], regions[1], _lib.ptr(slots), grid.experts, grid.table.data_ptr(),
            grid.expert_params, grid.levels, len(grid.levels), decoder_half.data_ptr(), target.data_ptr(),
            scores.resolution, xb.data_ptr(), yb.data_ptr(), scores.totals.data_ptr(), squares.data_ptr(),
            _lib.ptr(prediction), _lib.stream_of(target)))
        total = squares.sum()
    else:
        total = torch.zeros((), dtype=torch.float64, device=target.device)
        buffer = torch.empty((min(batch, pixels), 3), dtype=torch.float32, device=target.device)
        for begin in range(0, pixels, batch):
            n = min(batch, pixels - begin)
            chunk = reconstruct(grid, decoder_half, shape, regions, begin, n, slots=slots, prediction=buffer[:n])
            truth = target[begin:begin + n]
            # the mse of odie/evaluation.py:25 (ByteTarget: bytes / 255. on the device)
            total += (chunk - truth.float() / 255.).square().double().sum()
            scores.add(chunk, truth, begin)
    mse = float(total.item() / target.numel())
    if not math.isfinite(mse) or not bool(torch.isfinite(scores.totals).all()):
        raise FloatingPointError('GPU live RGB residual is nonfinite')
    return {'mse': mse, 'psnr_db': -10 * math.log10(mse) if mse else None}, scores
