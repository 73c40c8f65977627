"""odie_route_noalloc (the route with its scratch in a static device array) against odie_route
(caller workspace): the same expert ids, compaction order, local coordinates, offsets and slot
colours, bit for bit, on two calls in a row -- the second with fewer ids and more experts, so
it runs over what the first left in the shared array -- and the refusal of a size whose scratch
exceeds the array, before anything is queued."""
import numpy as np
import pytest
import torch

from odie_amd import _lib, synth
from odie_amd.experts import route

LIMIT = (4 << 20) + (64 << 10)


def _noalloc(ids, width, height, regions_x, regions_y, rgb):
    lib = _lib.library()
    n, experts = ids.numel(), regions_x * regions_y
    device = ids.device
    expert = torch.full((n,), -7, dtype=torch.int32, device=device)
    perm = torch.full((n,), -7, dtype=torch.int32, device=device)
    coords = torch.full((n, 2), -7.0, dtype=torch.float32, device=device)
    offsets = torch.full((experts + 1,), -7, dtype=torch.int32, device=device)
    colors = torch.full((n,), -7, dtype=torch.int32, device=device)
    _lib.check(lib.odie_route_noalloc(ids.data_ptr(), n, width, height, regions_x, regions_y, expert.data_ptr(),
                                      perm.data_ptr(), coords.data_ptr(), offsets.data_ptr(), rgb.data_ptr(),
                                      colors.data_ptr(), _lib.stream_of(ids)))
    return expert, perm, coords, offsets, colors


def _compare(seed, width, height, regions_x, regions_y, n):
    print(f'noalloc route: seed {seed}, {width}x{height}, {regions_x}x{regions_y} experts, {n} ids', flush=True)
    ids = torch.from_numpy(synth.integers(seed, 'ids', n, width * height)).cuda()
    image = torch.from_numpy(synth.integers(seed, 'image', width * height * 3, 256).astype(np.uint8)).cuda()
    expected = route(ids, width, height, regions_x, regions_y, with_expert=True, rgb=image)
    expert, perm, coords, offsets, colors = _noalloc(ids, width, height, regions_x, regions_y, image)
    torch.cuda.synchronize()
    assert torch.equal(expert, expected.expert)
    assert torch.equal(perm, expected.perm)
    assert torch.equal(coords.view(torch.int32), expected.coords.view(torch.int32))
    assert torch.equal(offsets, expected.offsets)
    assert torch.equal(colors, expected.colors)


@pytest.mark.gpu
def test_noalloc_route_matches_route_twice():
    lib = _lib.library()
    assert lib.odie_route_workspace(1 << 22, 64) <= LIMIT
    _compare(31, 2048, 1365, 8, 8, 1 << 22)          # the 64-expert step's route, 2 MiB + 2 KiB of scratch
    _compare(32, 1000, 999, 16, 16, 300001)          # fewer ids over more (ragged) experts


@pytest.mark.gpu
def test_noalloc_route_under_graph_capture():
    """After one eager call (the capture's warm-up), the route captured in a HIP graph and replayed
    three times, with eager work between the replays that overwrites the outputs and the shared
    scratch (another noalloc route): every replay equals odie_route."""
    width, height, regions, n = 640, 480, 8, 200003
    print(f'noalloc route under graph capture: {width}x{height}, {regions}x{regions} experts, {n} ids', flush=True)
    ids = torch.from_numpy(synth.integers(33, 'ids', n, width * height)).cuda()
    image = torch.from_numpy(synth.integers(33, 'image', width * height * 3, 256).astype(np.uint8)).cuda()
    expected = route(ids, width, height, regions, regions, with_expert=True, rgb=image)
    outputs = _noalloc(ids, width, height, regions, regions, image)       # warm-up, eager
    lib = _lib.library()
    graph = torch.cuda.graph_pool_handle()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, pool=graph, stream=side):
            expert, perm, coords, offsets, colors = outputs
            _lib.check(lib.odie_route_noalloc(ids.data_ptr(), n, width, height, regions, regions, expert.data_ptr(),
                                              perm.data_ptr(), coords.data_ptr(), offsets.data_ptr(),
                                              image.data_ptr(), colors.data_ptr(), _lib.stream_of(ids)))
    torch.cuda.current_stream().wait_stream(side)
    other = torch.from_numpy(synth.integers(34, 'ids', 99991, width * height)).cuda()
    for replay in range(3):
        for tensor in outputs:
            tensor.fill_(-7)
        _noalloc(other, width, height, 16, 16, image)                     # eager: reuses the scratch
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(expert, expected.expert), replay
        assert torch.equal(perm, expected.perm), replay
        assert torch.equal(coords.view(torch.int32), expected.coords.view(torch.int32)), replay
        assert torch.equal(offsets, expected.offsets), replay
        assert torch.equal(colors, expected.colors), replay


def test_noalloc_capacity_at_its_documented_bounds(native):
    """The largest id counts the header documents for each expert count fit the array, one id
    more does not, and 2^24 ids over 64 experts do not."""
    for experts, most, power in ((64, 8510976, 23), (256, 2127360, 21), (1024, 531456, 19), (4096, 132608, 17)):
        assert native.odie_route_workspace(1 << power, experts) <= LIMIT
        assert native.odie_route_workspace(most, experts) <= LIMIT
        assert native.odie_route_workspace(most + 1, experts) > LIMIT
        assert native.odie_route_workspace(2 << power, experts) > LIMIT
    assert native.odie_route_workspace(1 << 24, 64) > LIMIT


def test_noalloc_route_refuses_scratch_beyond_its_array(native):
    # 2^24 ids over 1024 experts need 16 MiB of counts: refused before touching the device
    n, width, height = 1 << 24, 32768, 32768
    assert native.odie_route_workspace(n, 1024) > LIMIT
    code = native.odie_route_noalloc(8, n, width, height, 32, 32, None, 8, 8, 8, None, None, 0)
    assert code == -1
    message = native.odie_error().decode()
    assert 'odie_route_noalloc' in message and 'use odie_route with a workspace' in message
