"""GPU routing + compaction against the oracle's integer-division restatement: expert
ids, compaction order (perm), local coordinates and offsets all bit-exact."""
import numpy as np
import pytest
import torch

import oracle
from odie_amd import synth
from odie_amd.experts import route

pytestmark = pytest.mark.gpu


@pytest.fixture(params=[1, 0], ids=['one_scan_launch', 'two_scan_launches'])
def scan_form(request):
    """Both scans of the counts: one launch (each segment adds the sums its predecessors publish;
    the default when there are at most 1024 segments) and the reduce and apply launches."""
    from odie_amd import _lib
    _lib.set_tuning('route_one_scan', request.param)
    yield request.param
    _lib.set_tuning('route_one_scan', 1)


@pytest.mark.parametrize('width,height,rx,ry,n', [
    (2048, 1365, 8, 8, 1 << 20),        # 64 experts over the 2048x1365 image
    (32768, 32768, 32, 32, 1 << 20),    # 1024 tile experts of the gigapixel image
    (100, 37, 3, 5, 4099),              # ragged tiles, n not a multiple of 64
    (64, 64, 1, 1, 777),                # a single expert
    (7, 5, 2, 2, 1),
    (4096, 4096, 60, 60, 1 << 23),      # 3600 experts: too many for the staged scatter's LDS
    (2048, 1365, 8, 8, 1 << 22),        # the training step's batch
])
def test_route_matches_oracle(width, height, rx, ry, n, scan_form):
    ids = synth.integers(17, 'ids', n, width * height)
    result = route(torch.from_numpy(ids).cuda(), width, height, rx, ry, with_expert=True)
    expert, perm, local, offsets = oracle.route(ids, width, height, rx, ry)
    assert np.array_equal(result.expert.cpu().numpy(), expert)
    assert np.array_equal(result.offsets.cpu().numpy(), offsets)
    assert np.array_equal(result.perm.cpu().numpy(), perm)
    assert np.array_equal(result.coords.cpu().numpy().view(np.uint32), local.view(np.uint32))


def test_route_tiles_at_every_bound_of_a_large_image():
    """Tile lookup (an fp32 estimate corrected by exact 64-bit product comparisons) at and around
    every tile bound of a 100003 x 42948 image (4.29e9 pixels, just under 2^32) cut into 60 x 60
    tiles whose bounds fall between pixels: experts, order and local coordinates bit-exact."""
    width, height, rx, ry = 100003, 42948, 60, 60
    xs = np.unique(np.clip([(r * width + rx - 1) // rx + d for r in range(rx + 1) for d in (-1, 0, 1)], 0, width - 1))
    ys = np.unique(np.clip([(r * height + ry - 1) // ry + d for r in range(ry + 1) for d in (-1, 0, 1)], 0, height - 1))
    ids = (ys[:, None].astype(np.int64) * width + xs[None, :]).reshape(-1)
    ids = np.concatenate([ids, synth.integers(29, 'ids', 4096, width * height)])
    result = route(torch.from_numpy(ids).cuda(), width, height, rx, ry, with_expert=True)
    expert, perm, local, offsets = oracle.route(ids, width, height, rx, ry)
    assert np.array_equal(result.expert.cpu().numpy(), expert)
    assert np.array_equal(result.offsets.cpu().numpy(), offsets)
    assert np.array_equal(result.perm.cpu().numpy(), perm)
    assert np.array_equal(result.coords.cpu().numpy().view(np.uint32), local.view(np.uint32))


@pytest.mark.parametrize('width,height,rx,ry', [(2, 2, 1, 1), (3, 1000, 1, 4), (7, 5, 2, 2), (1024, 999, 4, 4),
                                          (65535, 65537, 60, 60), (65536, 65535, 60, 60), (65537, 65535, 60, 60),
                                          (100003, 42948, 60, 60)])
def test_route_splits_ids_at_every_kind_of_row_bound(width, height, rx, ry):
    """id -> (x, y) by one multiply-high with the width's magic number (Granlund and
    Montgomery's division by invariant integers): ids at, just before and just after row bounds,
    the image's last pixel, ids past it (clamped to the last row) up to 2^32 - 1; pixel indexes,
    experts, order and local coordinates bit-exact against integer division."""
    rows = np.unique(np.concatenate([[0, 1, height - 1], synth.integers(31, 'rows', 200, height)]))
    ids = (rows[:, None].astype(np.int64) * width + np.array([0, 1, width - 1, width])[None, :]).reshape(-1)
    top = (1 << 32) - 1
    ids = np.concatenate([ids, [width * height - 1, min(width * height, top), top, top - width]])
    ids = ids[(ids >= 0) & (ids <= top)]
    result = route(torch.from_numpy(ids).cuda(), width, height, rx, ry, with_expert=True, pixels=True)
    expert, perm, local, offsets = oracle.route(ids, width, height, rx, ry)
    x, y = ids % width, np.minimum(ids // width, height - 1)
    assert np.array_equal(result.colors.cpu().numpy().view(np.uint32), (y * width + x)[perm].astype(np.uint32))
    assert np.array_equal(result.expert.cpu().numpy(), expert)
    assert np.array_equal(result.offsets.cpu().numpy(), offsets)
    assert np.array_equal(result.perm.cpu().numpy(), perm)
    assert np.array_equal(result.coords.cpu().numpy().view(np.uint32), local.view(np.uint32))


@pytest.mark.parametrize('width,height,rx,ry,n,offset', [(2048, 1365, 8, 8, 1 << 18, 0), (100, 37, 3, 5, 4099, 0),
                                                          (100, 37, 3, 5, 4099, 1)])
def test_route_gathers_slot_colors(width, height, rx, ry, n, offset, scan_form):
    """Colors are read in 8-byte windows from a 4-byte aligned image, byte by byte at its last
    pixels and from an image that starts off a 4-byte boundary (offset 1)."""
    ids = synth.integers(23, 'ids', n, width * height)
    ids[:5] = width * height + np.arange(5)          # past the image: clamped to the last row
    ids[5:8] = width * height - 1 - np.arange(3)     # the image's last pixels
    image = synth.integers(23, 'image', width * height * 3, 256).astype(np.uint8)
    buffer = torch.zeros(width * height * 3 + offset, dtype=torch.uint8, device='cuda')
    rgb = buffer[offset:]
    rgb.copy_(torch.from_numpy(image))
    assert rgb.data_ptr() % 4 == offset
    result = route(torch.from_numpy(ids).cuda(), width, height, rx, ry, rgb=rgb)
    _, perm, _, _ = oracle.route(ids, width, height, rx, ry)
    clamped = ids.astype(np.uint32).astype(np.int64)
    x, y = clamped % width, np.minimum(clamped // width, height - 1)
    pixel = image.reshape(-1, 3)[(y * width + x)[perm]].astype(np.uint32)
    expected = pixel[:, 0] | (pixel[:, 1] << 8) | (pixel[:, 2] << 16)
    assert np.array_equal(result.colors.cpu().numpy().view(np.uint32), expected)
    assert np.array_equal(result.perm.cpu().numpy(), perm)
    # without the image: each slot's pixel index itself (the decoder gathers the bytes)
    indexes = route(torch.from_numpy(ids).cuda(), width, height, rx, ry, pixels=True)
    assert np.array_equal(indexes.colors.cpu().numpy(), (y * width + x)[perm])
    assert np.array_equal(indexes.perm.cpu().numpy(), perm)


def test_route_clustered_ids_and_empty_experts(scan_form):
    # all ids inside one tile: every other expert is empty
    width, height = 2048, 1365
    xs = synth.integers(19, 'x', 50000, 256)
    ys = synth.integers(19, 'y', 50000, 170)
    ids = (ys + 171) * width + xs + 512
    result = route(torch.from_numpy(ids).cuda(), width, height, 8, 8, with_expert=True)
    expert, perm, local, offsets = oracle.route(ids, width, height, 8, 8)
    assert np.array_equal(result.perm.cpu().numpy(), perm)
    assert np.array_equal(result.offsets.cpu().numpy(), offsets)
    assert np.array_equal(result.coords.cpu().numpy().view(np.uint32), local.view(np.uint32))


def test_route_empty_batch():
    result = route(torch.zeros(0, dtype=torch.int64, device='cuda'), 2048, 1365, 8, 8)
    assert result.offsets.cpu().tolist() == [0] * 65


@pytest.mark.parametrize('width,height,rx,ry,n', [
    (2048, 1365, 8, 8, 1 << 16),        # the native step's batch over the 64-expert image
    (32768, 32768, 32, 32, 1 << 20),    # the gigapixel image's 1024 tiles
    (100, 37, 3, 5, 64),                # ragged tiles, strata larger than pixels
])
def test_route_stratified_fuses_the_draw(width, height, rx, ry, n, scan_form):
    """odie_route_stratified (the stratified draw computed inside the route) equals the route of
    odie_stratified_ids' ids bit for bit: experts, perm, local coordinates, offsets, colours;
    the oracle's stratified ids and route pin both."""
    from odie_amd.sampling import stratified_ids
    uniforms = torch.rand((n, 2), device='cuda', generator=torch.Generator(device='cuda').manual_seed(n))
    uniforms[0] = torch.tensor([0.0, 0.0])
    uniforms[-1] = torch.tensor([float.fromhex('0x1.fffffep-1')] * 2)   # largest fp32 below 1
    image = torch.from_numpy(synth.integers(n, 'image', width * height * 3, 256).astype(np.uint8)).cuda()
    ids = stratified_ids(uniforms, (height, width))
    fused = route(None, width, height, rx, ry, with_expert=True, rgb=image, uniforms=uniforms)
    plain = route(ids, width, height, rx, ry, with_expert=True, rgb=image)
    for name in ('expert', 'perm', 'offsets', 'colors'):
        assert torch.equal(getattr(fused, name), getattr(plain, name)), name
    assert torch.equal(fused.coords.view(torch.int32), plain.coords.view(torch.int32))
    expected = oracle.stratified_ids(uniforms.cpu().numpy(), width, height)
    assert np.array_equal(ids.cpu().numpy(), expected)
    _, perm, local, offsets = oracle.route(expected, width, height, rx, ry)
    assert np.array_equal(fused.perm.cpu().numpy(), perm)
    assert np.array_equal(fused.coords.cpu().numpy().view(np.uint32), local.view(np.uint32))


def _slot_map(seed, tiles, experts):
    """A tile -> expert map over `tiles` tiles: `experts` of them own an expert (shuffled), the
    others hold -1 or a value out of range (both mean none)."""
    rng = np.random.default_rng(seed)
    slots = np.full(tiles, -1, dtype=np.int32)
    owners = rng.permutation(tiles)[:experts]
    slots[owners] = rng.permutation(experts).astype(np.int32)
    spare = np.flatnonzero(slots < 0)
    slots[spare[::3]] = experts + 7
    return slots


@pytest.mark.parametrize('width,height,rx,ry,experts,n', [
    (2048, 1365, 8, 8, 41, 1 << 20),        # 41 of 64 tiles own an expert
    (32768, 32768, 32, 32, 700, 1 << 20),   # 700 of the gigapixel image's 1024 tiles
    (100, 37, 3, 5, 1, 4099),               # one expert, ragged tiles
    (4096, 4096, 60, 60, 3000, 1 << 21),    # too many buckets for the staged scatter's LDS
])
def test_route_allocated_matches_oracle(width, height, rx, ry, experts, n, scan_form):
    """odie_route_allocated: ids grouped by their tile's expert, the ids of tiles without one
    after all experts in input order; experts (-1 for those), perm, local coordinates, offsets
    [experts + 1] and colours bit-exact against the oracle's route with the same slot map, for
    stored ids and for the stratified draw."""
    slots = _slot_map(n, rx * ry, experts)
    ids = synth.integers(19, 'ids', n, width * height)
    image = torch.from_numpy(synth.integers(19, 'image', width * height * 3, 256).astype(np.uint8)).cuda() \
        if width * height <= 1 << 24 else None
    d_slots = torch.from_numpy(slots).cuda()
    result = route(torch.from_numpy(ids).cuda(), width, height, rx, ry, with_expert=True, rgb=image,
                   slots=d_slots, experts=experts)
    expert, perm, local, offsets = oracle.route(ids, width, height, rx, ry, slots=slots, experts=experts)
    assert np.array_equal(result.expert.cpu().numpy(), expert)
    assert np.array_equal(result.offsets.cpu().numpy(), offsets)
    assert np.array_equal(result.perm.cpu().numpy(), perm)
    assert np.array_equal(result.coords.cpu().numpy().view(np.uint32), local.view(np.uint32))
    if image is not None:
        pixel = image.cpu().numpy().reshape(-1, 3)[np.minimum(ids, width * height - 1)[perm]].astype(np.uint32)
        colors = pixel[:, 0] | (pixel[:, 1] << 8) | (pixel[:, 2] << 16)
        assert np.array_equal(result.colors.cpu().numpy().view(np.uint32), colors)
    side = 1 << ((n.bit_length() - 1) // 2)
    if side * side == n:
        uniforms = torch.rand((n, 2), device='cuda', generator=torch.Generator(device='cuda').manual_seed(n))
        fused = route(None, width, height, rx, ry, with_expert=True, uniforms=uniforms, slots=d_slots,
                      experts=experts)
        drawn = oracle.stratified_ids(uniforms.cpu().numpy(), width, height)
        expert, perm, local, offsets = oracle.route(drawn, width, height, rx, ry, slots=slots, experts=experts)
        assert np.array_equal(fused.expert.cpu().numpy(), expert)
        assert np.array_equal(fused.offsets.cpu().numpy(), offsets)
        assert np.array_equal(fused.perm.cpu().numpy(), perm)
        assert np.array_equal(fused.coords.cpu().numpy().view(np.uint32), local.view(np.uint32))


def test_forward_gives_rows_without_an_expert_zero_features():
    """Rows from offsets[experts] on (the ids of tiles without an expert) encode to zero features
    and receive no gradient; the other rows match the oracle's encode bit for bit and its gradient
    within the bar."""
    from odie_amd.config import grid_levels
    from odie_amd.encoding import grid_backward, grid_forward
    from oracle.bounds import check_gradient, hash_quantum
    width, height, rx, ry, experts, n = 640, 480, 4, 4, 9, 50000
    slots = _slot_map(5, rx * ry, experts)
    ids = synth.integers(37, 'ids', n, width * height)
    result = route(torch.from_numpy(ids).cuda(), width, height, rx, ry, slots=torch.from_numpy(slots).cuda(),
                   experts=experts)
    _, perm, local, offsets = oracle.route(ids, width, height, rx, ry, slots=slots, experts=experts)
    owned = int(offsets[experts])
    assert 0 < owned < n
    encoding = dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=12, base_resolution=8, per_level_scale=1.4)
    levels, entries = grid_levels(encoding)
    params = 2 * entries
    table = synth.table(37, experts * params, -1.0, 1.0).astype(np.float16)
    features = grid_forward(result.coords, torch.from_numpy(table).cuda(), levels, 2, offsets=result.offsets,
                            experts=experts, expert_params=params).cpu().numpy()
    rows = [(r.scale, r.resolution, r.size, r.offset, r.hashed) for r in levels]
    expected = oracle.hash_forward(local[:owned], table, rows, 2, offsets=offsets, expert_params=params)
    assert np.array_equal(features[:owned].view(np.uint16), expected.view(np.uint16))
    assert not features[owned:].view(np.uint16).any()
    up = synth.upstream(37, n, 32)
    for mode in (1, 0):   # owner, then the atomics kernel
        from odie_amd import _lib
        _lib.set_tuning('backward_mode', mode)
        try:
            grad = grid_backward(result.coords, torch.from_numpy(up).cuda(), levels, 2, offsets=result.offsets,
                                 experts=experts, expert_params=params).cpu().numpy()
        finally:
            _lib.set_tuning('backward_mode', 1)
        want, magnitude, counts = oracle.hash_backward(local[:owned], up[:owned], rows, 2, experts * params,
                                                       offsets=offsets, expert_params=params, counts=True)
        check_gradient(grad, want, magnitude, counts, hash_quantum(up, rows, 2, experts * params,
                                                                    offsets=offsets, expert_params=params),
                       'rows without an expert, mode %d' % mode)
