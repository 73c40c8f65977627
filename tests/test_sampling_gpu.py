"""Stratified sampling on the GPU (odie_stratified_ids) against the oracle's restatement of
odie/data.py:73-80, bit for bit, on torch.rand draws and on edge draws; the batch generators'
contracts (odie/data.py:47-106)."""
import numpy as np
import pytest
import torch

import oracle
from odie_amd.sampling import shuffled_batches, stratified_ids

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('shape,batch', [((61, 97), 16), ((2040, 1536), 65536), ((5, 33), 4), ((1365, 2048), 1),
                                         ((32768, 32768), 4096)])
def test_stratified_ids_match_the_oracle(shape, batch):
    generator = torch.Generator(device='cuda').manual_seed(batch)
    uniforms = torch.rand((batch, 2), device='cuda', generator=generator)
    uniforms[0] = 0.0
    if batch > 1:
        uniforms[1] = float(np.nextafter(np.float32(1.0), np.float32(0.0)))
    ids = stratified_ids(uniforms, shape).cpu().numpy()
    assert np.array_equal(ids, oracle.stratified_ids(uniforms.cpu().numpy(), shape[1], shape[0]))
    assert ids.min() >= 0 and ids.max() < shape[0] * shape[1]


def test_stratified_ids_clamp_out_of_range_draws():
    """Uniforms outside [0, 1), pixel coordinates beyond the int32 range included: the
    truncation saturates and the clamps put the pixel on the image's border, as the oracle's
    64-bit truncation and clamps do; a NaN lands on 0 in both.  (Coordinates beyond the int64
    range are left out: a float -> int64 conversion out of range differs between platforms.)"""
    shape, batch = (1365, 2048), 64
    uniforms = torch.rand((batch, 2), device='cuda', generator=torch.Generator(device='cuda').manual_seed(5))
    odd = torch.tensor([[-3.0, 2.5], [1e10, -1e10], [-0.4, 0.999], [1e14, -1e14], [float('nan'), 0.5],
                        [0.5, float('nan')], [-1e-30, 1.0]], device='cuda')
    uniforms[:odd.shape[0]] = odd
    ids = stratified_ids(uniforms, shape).cpu().numpy()
    with np.errstate(invalid='ignore'):
        expected = oracle.stratified_ids(uniforms.cpu().numpy(), shape[1], shape[0])
    assert np.array_equal(ids, expected)


def test_stratified_rejects_non_square_batches():
    with pytest.raises(RuntimeError, match='square power-of-two'):
        stratified_ids(torch.rand((8, 2), device='cuda'), (10, 10))


def test_batch_generators():
    pixels, batch = 1000, 64
    g = torch.Generator(device='cuda').manual_seed(1)
    batches = list(shuffled_batches(pixels, batch, g, mode='global'))
    assert sorted(torch.cat(batches).tolist()) == list(range(pixels))
    g = torch.Generator(device='cpu').manual_seed(1)
    full = list(shuffled_batches(pixels, batch, g, mode='global_full'))
    assert all(b.numel() == batch for b in full) and len(full) == (pixels + batch - 1) // batch
    assert set(torch.cat(full).tolist()) == set(range(pixels))
    g = torch.Generator(device='cuda').manual_seed(1)
    chunked = list(shuffled_batches(pixels, batch, g, mode='chunked', chunk=256))
    assert sorted(torch.cat(chunked).tolist()) == list(range(pixels))
    g = torch.Generator(device='cuda').manual_seed(1)
    strat = list(shuffled_batches(40 * 30, 64, g, mode='stratified', shape=(30, 40)))
    assert len(strat) == (1200 + 63) // 64 and all(b.dtype == torch.int64 and b.numel() == 64 for b in strat)
