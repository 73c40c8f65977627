"""Hash-grid encode on the GPU: the tcnn.Encoding the reference's HashGrid wraps
(odie/hash_grid.py:27,54), for one grid or for packed experts.

Tables are flat: level l of expert e, entry j, feature c lives at
e*expert_params + (offset_l + j)*F + c (tiny-cuda-nn's layout).  Everything here calls
libodie_amd.so; there is no CPU path.
"""
import torch
from torch import nn

from . import _lib
from .config import grid_levels

_DTYPES = {torch.float32: _lib.F32, torch.float16: _lib.F16}


def _check_coords(coords):
    if coords.dtype != torch.float32 or coords.ndim != 2 or coords.shape[1] != 2 or not coords.is_cuda:
        raise ValueError('coords must be a CUDA fp32 [N, 2] tensor')
    if not coords.is_contiguous():
        raise ValueError('coords must be contiguous')


def _offsets_arg(offsets, experts, n):
    if experts == 1 and offsets is None:
        return None
    if offsets is None or offsets.dtype != torch.int32 or offsets.numel() != experts + 1 or not offsets.is_cuda:
        raise ValueError('offsets must be a CUDA int32 tensor of experts+1 entries')
    return offsets


def grid_handoff_bytes(n, levels, features, *, experts=1, expert_params):
    """Bytes of the handoff that grid_forward(handoff=...) fills for the encode backward of the
    same batch (odie_grid_handoff_bytes; 0 when the backward would take nothing)."""
    size = _lib.library().odie_grid_handoff_bytes(n, experts, expert_params, levels, len(levels), features)
    if size < 0:
        _lib.check(-1)
    return size


def grid_forward(coords, table, levels, features, *, offsets=None, experts=1, expert_params=None,
                 width=None, out=None, handoff=None):
    """Encode coords [N,2] into [N, width] features of the table's dtype.  With handoff (uint8,
    at least grid_handoff_bytes long) the forward also fills the encode backward's handoff
    (odie_grid_forward_handoff: the slice masks or the band lists, by the backward's plan)."""
    _check_coords(coords)
    if table.dtype not in _DTYPES or not table.is_cuda or not table.is_contiguous():
        raise ValueError('table must be a contiguous CUDA fp32 or fp16 tensor')
    n = coords.shape[0]
    width = width or len(levels) * features
    expert_params = expert_params or table.numel() // experts
    if expert_params * experts > table.numel():
        raise ValueError('table holds fewer than experts*expert_params values')
    offsets = _offsets_arg(offsets, experts, n)
    if out is None:
        out = torch.empty((n, width), dtype=table.dtype, device=coords.device)
    elif out.dtype != table.dtype or out.shape != (n, width) or not out.is_contiguous():
        raise ValueError('out must be a contiguous [N, width] tensor of the table dtype')
    if handoff is None:
        _lib.check(_lib.library().odie_grid_forward(
            coords.data_ptr(), n, _lib.ptr(offsets), experts, table.data_ptr(), expert_params,
            _DTYPES[table.dtype], levels, len(levels), features, out.data_ptr(), width,
            _lib.stream_of(coords)))
        return out
    _check_handoff(handoff)
    _lib.check(_lib.library().odie_grid_forward_handoff(
        coords.data_ptr(), n, _lib.ptr(offsets), experts, table.data_ptr(), expert_params,
        _DTYPES[table.dtype], levels, len(levels), features, out.data_ptr(), width,
        handoff.data_ptr(), handoff.numel(), _lib.stream_of(coords)))
    return out


def grid_backward(coords, upstream, levels, features, *, offsets=None, experts=1, expert_params,
                  gradient=None, accumulate=False, handoff=None):
    """Scatter upstream [N, width] into an fp32 gradient of experts*expert_params values.  With
    handoff (filled by grid_forward(handoff=...) on the same coords and offsets, no tuning change
    in between) the backward reads it instead of forming it (odie_grid_backward_handoff)."""
    _check_coords(coords)
    if upstream.dtype not in _DTYPES or upstream.ndim != 2 or upstream.shape[0] != coords.shape[0]:
        raise ValueError('upstream must be fp32 or fp16 [N, width]')
    upstream = upstream.contiguous()
    offsets = _offsets_arg(offsets, experts, coords.shape[0])
    total = experts * expert_params
    if gradient is None:
        gradient = torch.empty(total, dtype=torch.float32, device=coords.device)
        accumulate = False
    elif gradient.dtype != torch.float32 or gradient.numel() < total or not gradient.is_contiguous():
        raise ValueError('gradient must be a contiguous fp32 tensor of experts*expert_params values')
    if handoff is None:
        _lib.check(_lib.library().odie_grid_backward(
            coords.data_ptr(), coords.shape[0], _lib.ptr(offsets), experts, upstream.data_ptr(),
            _DTYPES[upstream.dtype], upstream.shape[1], expert_params, levels, len(levels), features,
            gradient.data_ptr(), 0 if accumulate else 1, _lib.stream_of(coords)))
        return gradient
    _check_handoff(handoff)
    _lib.check(_lib.library().odie_grid_backward_handoff(
        coords.data_ptr(), coords.shape[0], _lib.ptr(offsets), experts, upstream.data_ptr(),
        _DTYPES[upstream.dtype], upstream.shape[1], expert_params, levels, len(levels), features,
        gradient.data_ptr(), 0 if accumulate else 1, handoff.data_ptr(), handoff.numel(), _lib.stream_of(coords)))
    return gradient


def _check_handoff(handoff):
    if handoff.dtype != torch.uint8 or not handoff.is_cuda or not handoff.is_contiguous():
        raise ValueError('handoff must be a contiguous CUDA uint8 tensor')


class _GridEncode(torch.autograd.Function):
    @staticmethod
    def forward(ctx, coords, params, module):
        table = params if module.dtype == torch.float32 else params.to(module.dtype)
        ctx.save_for_backward(coords)
        ctx.module = module
        return grid_forward(coords, table, module.levels, module.features, width=module.n_output_dims,
                            expert_params=module.n_params)

    @staticmethod
    def backward(ctx, grad_output):
        (coords,) = ctx.saved_tensors
        module = ctx.module
        gradient = grid_backward(coords, grad_output.to(module.dtype), module.levels, module.features,
                                 expert_params=module.n_params)
        return None, gradient, None


class GridEncoding(nn.Module):
    """2D multiresolution hash-grid encoding with fp32 master parameters.

    encoding: {'n_levels', 'n_features_per_level', 'log2_hashmap_size', 'base_resolution',
    'per_level_scale'} as in the reference's hash_encoding config (odie/config.py:103-109).
    dtype fp16 runs the fp16 table/fp16 chain path, fp32 the fp32 path.
    """

    def __init__(self, encoding, dtype=torch.float16, device='cuda'):
        super().__init__()
        self.encoding = dict(encoding)
        self.features = int(encoding['n_features_per_level'])
        self.levels, self.n_params_entries = grid_levels(encoding)
        self.n_params = self.n_params_entries * self.features
        self.n_output_dims = len(self.levels) * self.features
        self.dtype = dtype
        self.params = nn.Parameter(torch.zeros(self.n_params, dtype=torch.float32, device=device))

    def forward(self, coords):
        return _GridEncode.apply(coords.contiguous(), self.params, self)
