"""Packed multi-expert hash grid: routing of pixel ids to tile experts, compaction, and
the encode over every expert's table in one launch.

Each expert owns a full multiresolution hash-grid table and fits one tile of the image as
a sub-image; routing and compaction run on the GPU (odie_route), the encode reads the
compacted coordinates with per-expert offsets (odie_grid_forward/backward).
"""
import torch

from . import _lib
from .config import grid_levels
from .encoding import grid_backward, grid_forward, grid_handoff_bytes


def tile_bounds(size, regions):
    """Integer tile starts ceil(r*size/regions), r = 0..regions."""
    return [(r * size + regions - 1) // regions for r in range(regions + 1)]


class Routing:
    """Device buffers of one routed batch: perm, local coords, offsets (and optional
    per-input expert ids and per-slot packed RGB8 targets)."""

    def __init__(self, perm, coords, offsets, expert, colors=None):
        self.perm, self.coords, self.offsets, self.expert = perm, coords, offsets, expert
        self.colors = colors


def route(ids, width, height, regions_x, regions_y, *, with_expert=False, out=None, workspace=None, rgb=None,
          uniforms=None, slots=None, experts=None, pixels=False):
    """Route int64 pixel ids [N] (CUDA) to regions_x*regions_y tile experts and compact.  With
    rgb (CUDA uint8 [H*W*3]) each slot also receives its pixel's packed colour in out.colors;
    with pixels=True (and no rgb) out.colors receives the slot's pixel index instead.  With
    uniforms (CUDA fp32 [N, 2], N a square power of two) and ids None, the ids are those of
    the stratified draw on those uniforms (odie_stratified_ids), computed inside the route.
    With slots (CUDA int32 [regions_x*regions_y], tile -> expert in [0, experts), any other
    value: no expert) the tiles share `experts` experts; ids of tiles without one follow every
    expert's, from offsets[experts] on (odie_route_allocated)."""
    if uniforms is not None:
        if ids is not None:
            raise ValueError('give ids or uniforms, not both')
        if uniforms.dtype != torch.float32 or uniforms.ndim != 2 or uniforms.shape[1] != 2 or not uniforms.is_cuda:
            raise ValueError('uniforms must be a CUDA fp32 [N, 2] tensor')
        ids = uniforms.contiguous()
        entry = 'odie_route_stratified'
    else:
        if ids is None or ids.dtype != torch.int64 or ids.ndim != 1 or not ids.is_cuda:
            raise ValueError('ids must be a CUDA int64 [N] tensor')
        ids = ids.contiguous()
        entry = 'odie_route'
    n, tiles = ids.shape[0], regions_x * regions_y
    if slots is not None:
        if (slots.dtype != torch.int32 or slots.numel() != tiles or not slots.is_cuda
                or not slots.is_contiguous()):
            raise ValueError('slots must be a contiguous CUDA int32 tensor of regions_x * regions_y entries')
        if experts is None or not 1 <= experts < 4096:
            raise ValueError('experts must be within 1..4095 with slots')
    else:
        experts = tiles
    buckets = experts + 1 if slots is not None else experts
    lib = _lib.library()
    need = lib.odie_route_workspace(n, buckets)
    if need < 0:
        raise ValueError('invalid routing size')
    device = ids.device
    if out is None:
        out = Routing(torch.empty(n, dtype=torch.int32, device=device),
                      torch.empty((n, 2), dtype=torch.float32, device=device),
                      torch.empty(experts + 1, dtype=torch.int32, device=device),
                      torch.empty(n, dtype=torch.int32, device=device) if with_expert else None,
                      torch.empty(n, dtype=torch.int32, device=device) if rgb is not None or pixels else None)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 4), dtype=torch.uint8, device=device)
    if pixels and rgb is not None:
        raise ValueError('pixels=True writes pixel indexes in place of the colours of rgb')
    colors = out.colors if rgb is not None or pixels else None
    if slots is not None:
        stratified = entry == 'odie_route_stratified'
        _lib.check(lib.odie_route_allocated(None if stratified else ids.data_ptr(),
                                            ids.data_ptr() if stratified else None, n, width, height, regions_x,
                                            regions_y, slots.data_ptr(), experts, _lib.ptr(out.expert),
                                            out.perm.data_ptr(), out.coords.data_ptr(), out.offsets.data_ptr(),
                                            _lib.ptr(rgb), _lib.ptr(colors), workspace.data_ptr(),
                                            workspace.numel() * workspace.element_size(), _lib.stream_of(ids)))
        return out
    _lib.check(getattr(lib, entry)(ids.data_ptr(), n, width, height, regions_x, regions_y, _lib.ptr(out.expert),
                                   out.perm.data_ptr(), out.coords.data_ptr(), out.offsets.data_ptr(),
                                   _lib.ptr(rgb), _lib.ptr(colors), workspace.data_ptr(),
                                   workspace.numel() * workspace.element_size(), _lib.stream_of(ids)))
    return out


def tile_ranges(image, regions_x, regions_y):
    """RGB8 range of every tile (uint8 image [H, W, 3], on any device): the largest, over the
    three channels, of the channel's largest minus smallest byte in the tile -- 0 exactly for a
    tile of one colour.  int32 [regions_y * regions_x] in tile order, with the route's tile bounds."""
    image = torch.as_tensor(image)
    height, width = image.shape[:2]
    xs, ys = tile_bounds(width, regions_x), tile_bounds(height, regions_y)
    ranges = torch.empty(regions_y * regions_x, dtype=torch.int32)
    for ry in range(regions_y):
        band = image[ys[ry]:ys[ry + 1]]
        top, bottom = band.amax(dim=0).int(), band.amin(dim=0).int()   # [W, 3]: per column and channel
        for rx in range(regions_x):
            spread = top[xs[rx]:xs[rx + 1]].amax(dim=0) - bottom[xs[rx]:xs[rx + 1]].amin(dim=0)
            ranges[ry * regions_x + rx] = int(spread.max())
    return ranges


def allocate_tiles(image, regions_x, regions_y, expert_params, budget_params):
    """Experts for the non-flat tiles (tile_ranges > 0), in tile order, while their parameters
    fit the budget: returns (slots int32 [regions_y * regions_x] with -1 for tiles left without
    an expert, experts).  A flat tile is one colour: the decoder reproduces it from the zero
    features every id without an expert reads, as the reference leaves cells off its supports
    (odie/model.py:226-257)."""
    ranges = tile_ranges(image, regions_x, regions_y)
    most = int(budget_params // expert_params)
    slots = torch.full((regions_x * regions_y,), -1, dtype=torch.int32)
    experts = 0
    for tile in torch.nonzero(ranges > 0).flatten().tolist():
        if experts == most:
            break
        slots[tile] = experts
        experts += 1
    return slots, experts


class ExpertGrid:
    """experts independent hash grids packed in one table of experts*expert_params values."""

    def __init__(self, encoding, experts, dtype=torch.float16, device='cuda'):
        self.encoding = dict(encoding)
        self.features = int(encoding['n_features_per_level'])
        self.levels, entries = grid_levels(encoding)
        self.experts = experts
        self.expert_params = entries * self.features
        self.width = len(self.levels) * self.features
        self.table = torch.zeros(experts * self.expert_params, dtype=dtype, device=device)

    def forward(self, coords, offsets, out=None, handoff=None):
        """Features [N, width]; with handoff (uint8, at least handoff_bytes(N)) also the encode
        backward's handoff, for backward(handoff=...) or backward_adam_planes(handoff=...)."""
        return grid_forward(coords, self.table, self.levels, self.features, offsets=offsets,
                            experts=self.experts, expert_params=self.expert_params, width=self.width, out=out,
                            handoff=handoff)

    def handoff_bytes(self, n):
        """Bytes of the handoff forward(handoff=...) fills for a batch of n coordinates."""
        return grid_handoff_bytes(n, self.levels, self.features, experts=self.experts,
                                  expert_params=self.expert_params)

    def backward(self, coords, offsets, upstream, gradient=None, accumulate=False, handoff=None):
        return grid_backward(coords, upstream, self.levels, self.features, offsets=offsets, experts=self.experts,
                             expert_params=self.expert_params, gradient=gradient, accumulate=accumulate,
                             handoff=handoff)

    def backward_adam(self, coords, offsets, upstream, optimizer, loss_scale=1.0):
        """Encode backward fused with optimizer.step (a FusedAdam over this table's fp32 master,
        typically with half_copy = self.table): the same parameters, moments and ages as
        backward() followed by optimizer.step(gradient, loss_scale), without the gradient."""
        from .encoding import _DTYPES, _check_coords, _offsets_arg
        _check_coords(coords)
        if upstream.dtype not in _DTYPES or upstream.ndim != 2 or upstream.shape[0] != coords.shape[0]:
            raise ValueError('upstream must be fp32 or fp16 [N, width]')
        if optimizer.master.numel() != self.experts * self.expert_params:
            raise ValueError('the optimizer must own this table\'s fp32 master')
        upstream = upstream.contiguous()
        offsets = _offsets_arg(offsets, self.experts, coords.shape[0])
        optimizer.step_count += 1
        _lib.check(_lib.library().odie_grid_backward_adam(
            coords.data_ptr(), coords.shape[0], _lib.ptr(offsets), self.experts, upstream.data_ptr(),
            _DTYPES[upstream.dtype], upstream.shape[1], self.expert_params, self.levels, len(self.levels),
            self.features, optimizer.master.data_ptr(), _lib.ptr(optimizer.half_copy), optimizer.m.data_ptr(),
            optimizer.v.data_ptr(), _lib.ptr(optimizer.steps), optimizer.variant_code, optimizer.step_count,
            optimizer.lr, optimizer.betas[0], optimizer.betas[1], optimizer.eps, float(loss_scale),
            _lib.stream_of(coords)))

    def _check_planes(self, coords, planes, blockmax):
        from .encoding import _check_coords
        _check_coords(coords)
        n = coords.shape[0]
        levels = len(self.levels)
        if tuple(planes.shape) != (levels, n) or planes.dtype != torch.int32 or not planes.is_contiguous():
            raise ValueError('planes must be a contiguous int32 [levels, N] tensor')
        if (tuple(blockmax.shape) != ((n + 127) // 128, 2 * levels) or blockmax.dtype != torch.float32
                or not blockmax.is_contiguous()):
            raise ValueError('blockmax must be a contiguous fp32 [ceil(N/128), 2 levels] tensor')

    def backward_planes(self, coords, offsets, planes, blockmax, gradient=None, accumulate=False):
        """backward() with the fp16 upstream given as Decoder.train_planes writes it (planes int32
        [levels, N], blockmax fp32 [ceil(N/128), 2 levels]): the same gradient, bit for bit."""
        from .encoding import _offsets_arg
        self._check_planes(coords, planes, blockmax)
        total = self.experts * self.expert_params
        if gradient is None:
            gradient = torch.empty(total, dtype=torch.float32, device=coords.device)
            accumulate = False
        elif gradient.dtype != torch.float32 or gradient.numel() != total or not gradient.is_contiguous():
            raise ValueError('gradient must be a contiguous fp32 tensor of experts * expert_params values')
        offsets = _offsets_arg(offsets, self.experts, coords.shape[0])
        _lib.check(_lib.library().odie_grid_backward_planes(
            coords.data_ptr(), coords.shape[0], _lib.ptr(offsets), self.experts, planes.data_ptr(),
            blockmax.data_ptr(), self.expert_params, self.levels, len(self.levels), self.features,
            gradient.data_ptr(), 0 if accumulate else 1, _lib.stream_of(coords)))
        return gradient

    def backward_adam_planes(self, coords, offsets, planes, blockmax, optimizer, loss_scale=1.0, handoff=None):
        """backward_adam with the fp16 upstream given as Decoder.train_planes writes it (planes
        int32 [levels, N], blockmax fp32 [ceil(N/128), 2 levels]): the same update, bit for bit.
        With handoff (filled by forward(handoff=...) on the same coords and offsets, no tuning change
        in between) the backward reads it instead of forming it."""
        from .encoding import _offsets_arg
        self._check_planes(coords, planes, blockmax)
        n = coords.shape[0]
        if optimizer.master.numel() != self.experts * self.expert_params:
            raise ValueError('the optimizer must own this table\'s fp32 master')
        offsets = _offsets_arg(offsets, self.experts, n)
        if handoff is not None and (handoff.dtype != torch.uint8 or not handoff.is_cuda or not handoff.is_contiguous()):
            raise ValueError('handoff must be a contiguous CUDA uint8 tensor')
        optimizer.step_count += 1
        if handoff is None:
            _lib.check(_lib.library().odie_grid_backward_adam_planes(
                coords.data_ptr(), n, _lib.ptr(offsets), self.experts, planes.data_ptr(), blockmax.data_ptr(),
                self.expert_params, self.levels, len(self.levels), self.features, optimizer.master.data_ptr(),
                _lib.ptr(optimizer.half_copy), optimizer.m.data_ptr(), optimizer.v.data_ptr(),
                _lib.ptr(optimizer.steps), optimizer.variant_code, optimizer.step_count, optimizer.lr,
                optimizer.betas[0], optimizer.betas[1], optimizer.eps, float(loss_scale), _lib.stream_of(coords)))
            return
        _lib.check(_lib.library().odie_grid_backward_adam_planes_handoff(
            coords.data_ptr(), n, _lib.ptr(offsets), self.experts, planes.data_ptr(), blockmax.data_ptr(),
            self.expert_params, self.levels, len(self.levels), self.features, optimizer.master.data_ptr(),
            _lib.ptr(optimizer.half_copy), optimizer.m.data_ptr(), optimizer.v.data_ptr(), _lib.ptr(optimizer.steps),
            optimizer.variant_code, optimizer.step_count, optimizer.lr, optimizer.betas[0], optimizer.betas[1],
            optimizer.eps, float(loss_scale), handoff.data_ptr(), handoff.numel(), _lib.stream_of(coords)))
