"""The batch generators of the reference's sampling modes on the CPU (odie/data.py:47-106):
each mode's invariants, and the seeded stream -- the generators draw torch's permutations in the
reference's order and sizes, so a seeded generator's batches are those permutations cut into
batches (the reference's full_batches pads its last batch with the permutation's beginning;
chunked mode permutes the chunk order first, then each chunk as it is visited)."""
import pytest
import torch

from odie_amd.sampling import full_batches, shuffled_batches


def _generator(seed):
    return torch.Generator(device='cpu').manual_seed(seed)


@pytest.mark.parametrize('pixels,batch', [(1000, 64), (1024, 64), (5, 8), (3, 16), (1, 1)])
def test_global_full_is_a_padded_permutation(pixels, batch):
    """Every batch full and int64; the batches, concatenated, are one permutation of the pixels
    followed by its own first entries (wrapping as often as a batch longer than the image needs);
    and the permutation is the generator's first draw of that size."""
    batches = list(full_batches(pixels, batch, _generator(3), device='cpu'))
    assert len(batches) == -(-pixels // batch)
    assert all(b.dtype == torch.int64 and b.numel() == batch for b in batches)
    order = torch.randperm(pixels, dtype=torch.int32, generator=_generator(3)).long()
    stream = torch.cat(batches)
    assert torch.equal(stream[:pixels], order)
    assert torch.equal(stream, order[torch.arange(stream.numel()) % pixels])


@pytest.mark.parametrize('pixels,batch', [(1000, 64), (4096, 256), (7, 3)])
def test_global_visits_every_pixel_once(pixels, batch):
    batches = list(shuffled_batches(pixels, batch, _generator(5), mode='global', device='cpu'))
    assert [b.numel() for b in batches] == [min(batch, pixels - k) for k in range(0, pixels, batch)]
    stream = torch.cat(batches)
    assert torch.equal(stream, torch.randperm(pixels, generator=_generator(5)))
    assert torch.equal(stream.sort().values, torch.arange(pixels))


@pytest.mark.parametrize('pixels,batch,chunk', [(1000, 64, 256), (1024, 64, 256), (300, 10, 100), (9, 3, 30)])
def test_chunked_visits_chunks_in_a_random_order(pixels, batch, chunk):
    """Chunks of `chunk` consecutive ids, visited in the order of a permutation of the chunks;
    within a chunk its ids permuted and cut into batches that never straddle two chunks; every
    pixel once; the draws are the chunk permutation, then one permutation per chunk."""
    batches = list(shuffled_batches(pixels, batch, _generator(7), mode='chunked', chunk=chunk, device='cpu'))
    stream = torch.cat(batches)
    assert torch.equal(stream.sort().values, torch.arange(pixels))
    chunks = -(-pixels // chunk)
    g = _generator(7)
    visit = torch.randperm(chunks, generator=g).tolist()
    expected = []
    for k in visit:
        size = min(chunk, pixels - k * chunk)
        expected.append(torch.randperm(size, generator=g) + k * chunk)
    assert torch.equal(stream, torch.cat(expected))
    for b in batches:
        assert b.numel() <= batch and int(b.min()) // chunk == int(b.max()) // chunk


def test_modes_are_checked():
    with pytest.raises(ValueError, match='multiple of batch'):
        next(shuffled_batches(100, 8, _generator(1), mode='chunked', chunk=12, device='cpu'))
    with pytest.raises(ValueError, match='matching image shape'):
        next(shuffled_batches(100, 16, _generator(1), mode='stratified', shape=(10, 11), device='cpu'))
    with pytest.raises(ValueError, match='sampling must be'):
        next(shuffled_batches(100, 16, _generator(1), mode='tiles', device='cpu'))
