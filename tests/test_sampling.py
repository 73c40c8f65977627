"""The batch generators of the reference's sampling modes on the CPU (odie/data.py:47-106):
each mode's invariants, and the seeded stream -- the generators draw torch's permutations in the
reference's order and sizes, so a seeded generator's batches are those permutations cut into
batches (the reference's full_batches pads its last batch with the permutation's beginning;
chunked mode permutes the chunk order first, then each chunk as it is visited)."""
import numpy as np
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


def test_allocate_tiles_takes_non_flat_tiles_under_the_budget():
    """Flat tiles (one colour) get no expert; the others get experts in tile order until the
    parameter budget is spent; the tile ranges use the route's ceil bounds."""
    from odie_amd.experts import allocate_tiles, tile_bounds, tile_ranges
    rng = np.random.default_rng(3)
    height, width, rx, ry = 50, 70, 4, 3
    image = rng.integers(0, 256, (height, width, 3), dtype=np.uint8)
    xs, ys = tile_bounds(width, rx), tile_bounds(height, ry)
    flat = [1, 6, 7]
    for t in flat:
        image[ys[t // rx]:ys[t // rx + 1], xs[t % rx]:xs[t % rx + 1]] = (12, 200, 12 + t)
    image[ys[2]:ys[3], xs[3]:xs[4]] = (5, 5, 5)                     # tile 11: one colour but for
    image[ys[2]:ys[3], xs[3]:xs[3] + 1, 1] = 6                      # one column a shade off
    ranges = tile_ranges(torch.from_numpy(image), rx, ry)
    assert [int(v) for v in ranges[flat]] == [0, 0, 0]          # one colour each (channels differ)
    assert int(ranges[11]) == 1 and (ranges[[t for t in range(rx * ry) if t not in flat]] > 0).all()
    slots, experts = allocate_tiles(torch.from_numpy(image), rx, ry, expert_params=100, budget_params=10 ** 6)
    assert experts == rx * ry - 3 and [int(slots[t]) for t in flat] == [-1, -1, -1]
    assert [int(v) for v in slots[slots >= 0]] == list(range(experts))
    slots, experts = allocate_tiles(torch.from_numpy(image), rx, ry, expert_params=100, budget_params=450)
    assert experts == 4 and [int(v) for v in slots[:8]] == [0, -1, 1, 2, 3, -1, -1, -1]
