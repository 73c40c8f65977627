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


def full_batches(pixels, batch, generator, device='cuda'):
    """A global permutation once, padded with its beginning (odie/data.py:47-60)."""
    dtype = torch.int32 if pixels <= 2 ** 31 - 1 else torch.int64
    order = torch.randperm(pixels, dtype=dtype, device=generator.device, generator=generator)
    for begin in range(0, pixels, batch):
        ids = order[begin:begin + batch]
        if ids.numel() < batch:
            padding = torch.arange(batch - ids.numel(), device=order.device) % pixels
            ids = torch.cat((ids, order[padding]))
        yield ids.to(device=device, dtype=torch.int64)


def shuffled_batches(pixels, batch, generator, mode='global', chunk=4194304, device='cuda', shape=None):
    """The reference's sampling modes (odie/data.py:83-106)."""
    if mode == 'global_full':
        yield from full_batches(pixels, batch, generator, device)
    elif mode == 'stratified':
        if shape is None or len(shape) != 2 or shape[0] * shape[1] != pixels or min(shape) < 2:
            raise ValueError('Stratified sampling requires the matching image shape')
        yield from stratified_batches(shape, batch, generator, device)
    elif mode == 'global':
        permutation = torch.randperm(pixels, device=device, generator=generator)
        for begin in range(0, pixels, batch):
            yield permutation[begin:begin + batch]
    elif mode == 'chunked':
        if chunk <= 0 or chunk % batch:
            raise ValueError('Chunk size must be a positive multiple of batch size')
        count = (pixels + chunk - 1) // chunk
        order = torch.randperm(count, device=device, generator=generator).cpu().tolist()
        for block in order:
            start = block * chunk
            size = min(chunk, pixels - start)
            permutation = torch.randperm(size, device=device, generator=generator)
            for begin in range(0, size, batch):
                yield permutation[begin:begin + batch] + start
    else:
        raise ValueError('sampling must be global, chunked, global_full or stratified')
