"""Pixel sampling for the training step (odie/data.py:47-106): the same batch generators, with
the stratified draw's id arithmetic on the GPU (odie_stratified_ids).

The uniforms come from torch.rand on the caller's generator, as in the reference; the ids of a
stratified batch are then one fused kernel instead of the reference's chain of torch ops."""
import torch

from . import _lib


def stratified_ids(uniforms, shape, out=None):
    """ids int64 [batch] of one stratified batch from uniforms fp32 [batch, 2] (CUDA)."""
    height, width = shape
    if uniforms.dtype != torch.float32 or uniforms.ndim != 2 or uniforms.shape[1] != 2 or not uniforms.is_cuda:
        raise ValueError('uniforms must be CUDA fp32 [batch, 2]')
    uniforms = uniforms.contiguous()
    batch = uniforms.shape[0]
    if out is None:
        out = torch.empty(batch, dtype=torch.int64, device=uniforms.device)
    _lib.check(_lib.library().odie_stratified_ids(uniforms.data_ptr(), batch, width, height, out.data_ptr(),
                                                  _lib.stream_of(uniforms)))
    return out


def stratified_batches(shape, batch, generator, device='cuda'):
    """One random pixel per square stratum per step (odie/data.py:63-80): ceil(H*W/batch) batches."""
    height, width = shape
    side = int(batch ** .5)
    if batch < 1 or batch & (batch - 1) or side * side != batch:
        raise ValueError('Stratified sampling requires a square power-of-two batch size')
    for _ in range((height * width + batch - 1) // batch):
        yield stratified_ids(torch.rand((batch, 2), device=device, generator=generator), shape)


# Batch generators of the reference's sampling modes (odie/data.py:47-106).  The torch RNG is
# consumed in the reference's order and sizes (one randperm over the pixels for 'global' and
# 'global_full'; for 'chunked' one over the chunks, then one per chunk as it is visited), so a
# seeded generator yields the same ids.  The permutations are cut into batches by _cut.

def _cut(order, batch, *, base=0, wrap=False, device=None):
    """Consecutive slices of `batch` entries of a 1-D permutation, plus `base`.  With wrap, the
    last slice is completed from the start of the permutation (positions taken modulo its
    length), so every batch is full; with device, slices move there as int64."""
    total = order.numel()
    for first in range(0, total, batch):
        if wrap and first + batch > total:
            ids = order[(first + torch.arange(batch, device=order.device)) % total]
        else:
            ids = order[first:first + batch]
        if device is not None:
            ids = ids.to(device=device, dtype=torch.int64)
        yield ids + base if base else ids


def full_batches(pixels, batch, generator, device='cuda'):
    """Every pixel once in a permutation drawn on the generator's device (CPU for giant images;
    int32 while the ids fit), the last batch completed from its start; each batch moves to
    `device` as int64 on its own (odie/data.py:47-60)."""
    dtype = torch.int32 if pixels < 2 ** 31 else torch.int64
    order = torch.randperm(pixels, dtype=dtype, device=generator.device, generator=generator)
    yield from _cut(order, batch, wrap=True, device=device)


def _chunked(pixels, batch, generator, chunk, device):
    if chunk <= 0 or chunk % batch:
        raise ValueError('Chunk size must be a positive multiple of batch size')
    chunks = -(-pixels // chunk)
    for k in torch.randperm(chunks, device=device, generator=generator).cpu().tolist():
        size = min(chunk, pixels - k * chunk)
        yield from _cut(torch.randperm(size, device=device, generator=generator), batch, base=k * chunk)


def shuffled_batches(pixels, batch, generator, mode='global', chunk=4194304, device='cuda', shape=None):
    """Pixel ids of one epoch in `mode` (odie/data.py:83-106): 'global' (one permutation),
    'global_full' (full_batches), 'chunked' (chunks of `chunk` ids in random order, each
    permuted) or 'stratified' (stratified_batches; `shape` is the image's (H, W))."""
    if mode == 'global':
        yield from _cut(torch.randperm(pixels, device=device, generator=generator), batch)
    elif mode == 'global_full':
        yield from full_batches(pixels, batch, generator, device)
    elif mode == 'chunked':
        yield from _chunked(pixels, batch, generator, chunk, device)
    elif mode == 'stratified':
        if shape is None or len(shape) != 2 or shape[0] * shape[1] != pixels or min(shape) < 2:
            raise ValueError('Stratified sampling requires the matching image shape')
        yield from stratified_batches(shape, batch, generator, device)
    else:
        raise ValueError('sampling must be global, chunked, global_full or stratified')
