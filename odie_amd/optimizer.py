"""Fused Adam on the GPU (odie_adam_step) for flat fp32 parameter buffers.

FusedAdam keeps the moments (and, for the per-parameter-age variant, the ages) next to one
flat fp32 master buffer and updates it -- and an optional fp16 copy -- in one pass per step.
variant 'torch' follows torch.optim.Adam (odie/optimizer.py:33-44); variant 'tcnn' skips zero
gradients and keeps per-parameter ages (the grid, odie/native/runtime.cu:212-215); variant
'tcnn_dense' keeps per-parameter ages without the skip (the MLP heads, :159-160).
"""
import torch

from . import _lib

_VARIANTS = {'torch': 0, 'tcnn': 1, 'tcnn_dense': 2}


class FusedAdam:
    def __init__(self, master, lr, betas=(0.9, 0.999), eps=1e-15, variant='torch', half_copy=None):
        if master.dtype != torch.float32 or not master.is_cuda or not master.is_contiguous():
            raise ValueError('master must be a contiguous CUDA fp32 tensor')
        if variant not in _VARIANTS:
            raise ValueError('variant must be torch, tcnn or tcnn_dense')
        self.master, self.lr, self.betas, self.eps = master, float(lr), betas, float(eps)
        self.variant = variant
        self.variant_code = _VARIANTS[variant]
        self.half_copy = half_copy
        self.m = torch.zeros_like(master)
        self.v = torch.zeros_like(master)
        self.steps = torch.zeros(master.numel(), dtype=torch.int32, device=master.device) if variant != 'torch' else None
        self.step_count = 0

    def step(self, grad, loss_scale=1.0):
        if grad.numel() != self.master.numel() or grad.dtype not in (torch.float32, torch.float16):
            raise ValueError('grad must match the master size, fp32 or fp16')
        grad = grad.contiguous()
        self.step_count += 1
        _lib.check(_lib.library().odie_adam_step(
            self.master.data_ptr(), _lib.ptr(self.half_copy), grad.data_ptr(),
            _lib.F16 if grad.dtype == torch.float16 else _lib.F32, self.m.data_ptr(), self.v.data_ptr(),
            _lib.ptr(self.steps), self.master.numel(), _VARIANTS[self.variant], self.step_count, self.lr,
            self.betas[0], self.betas[1], self.eps, float(loss_scale), _lib.stream_of(self.master)))
