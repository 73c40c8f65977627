"""GPU parity of the grid encode (HIP via the C-ABI) against the CPU oracle.

Forward: bit-exact (fp16 chain and fp32 chain).  Backward: each gradient entry within
1e-4 of the sum of the absolute values of its contributions (summation order is free), plus
half the fixed-point quantum of its own (level, feature) column per contribution (the owner
backward rounds each contribution once; oracle.bounds states the bar and the quantum).
"""
import numpy as np
import pytest
import torch

import oracle
from oracle.bounds import check_gradient as _check, hash_quantum, packed_quantum
from odie_amd import _lib
from odie_amd.config import grid_levels
from odie_amd.encoding import grid_backward, grid_forward
from odie_amd import synth

pytestmark = pytest.mark.gpu


def rows_of(levels):
    return [(r.scale, r.resolution, r.size, r.offset, r.hashed) for r in levels]


def hash_bar(xy, up, levels, features, total, offsets=None, expert_params=None):
    """The oracle's gradient with each entry's bar: (expected, sum|c|, count, quantum)."""
    rows = rows_of(levels)
    expected, magnitude, counts = oracle.hash_backward(xy, up, rows, features, total, offsets=offsets,
                                                       expert_params=expert_params, counts=True)
    return expected, magnitude, counts, hash_quantum(up, rows, features, total, offsets=offsets,
                                                     expert_params=expert_params)


def packed_bar(xy, up, layout, total):
    expected, magnitude, counts = oracle.packed_backward(xy, up, layout, total, counts=True)
    return expected, magnitude, counts, packed_quantum(up, layout, total)


def check_gradient(gpu, bar, label=''):
    _check(gpu.detach().cpu().numpy(), *bar, label=label)


def encoding(levels=16, base=16, log2=19, scale=1.38, features=2):
    return dict(n_levels=levels, base_resolution=base, log2_hashmap_size=log2, per_level_scale=scale,
                n_features_per_level=features)


@pytest.mark.parametrize('dtype', [torch.float16, torch.float32])
def test_single_grid_forward_bit_exact(dtype):
    enc = encoding()
    levels, entries = grid_levels(enc)
    n = 1 << 16
    xy = synth.coordinates(0, n)
    values = synth.table(0, entries * 2)
    table = values.astype(np.float16) if dtype == torch.float16 else values
    out = grid_forward(torch.from_numpy(xy).cuda(), torch.from_numpy(table).cuda(), levels, 2)
    expected = oracle.hash_forward(xy, table, rows_of(levels), 2, threads=0)
    got = out.cpu().numpy()
    view = np.uint16 if dtype == torch.float16 else np.uint32
    mismatch = got.view(view) != expected.view(view)
    assert not mismatch.any(), 'mismatches at %s' % (np.argwhere(mismatch)[:5],)


@pytest.mark.parametrize('log2', [14, 19])
@pytest.mark.parametrize('mode', [0, 1, 2], ids=['single', 'pairs', 'auto'])
def test_forward_corner_pairs_bit_exact(mode, log2):
    """The fp16 forward's 16-byte corner-pair loads (tuning key paired_loads: off, on, and the
    default, on only for tables past 4 MB) against the oracle, on a table that fits one L2
    (2^14 entries) and one that does not (2^19): the odd corner outside its group of four
    entries takes the single load."""
    enc = encoding(log2=log2)
    levels, entries = grid_levels(enc)
    n = 1 << 15
    xy = synth.coordinates(3, n)
    table = synth.table(3, entries * 2).astype(np.float16)
    out = _tuned('paired_loads', mode, 2, lambda: grid_forward(torch.from_numpy(xy).cuda(),
                                                               torch.from_numpy(table).cuda(), levels, 2))
    expected = oracle.hash_forward(xy, table, rows_of(levels), 2, threads=0)
    mismatch = out.cpu().numpy().view(np.uint16) != expected.view(np.uint16)
    assert not mismatch.any(), 'mismatches at %s' % (np.argwhere(mismatch)[:5],)


@pytest.mark.parametrize('experts', [1, 3])
def test_handoff_band_lists_bit_identical(experts):
    """The forward filling the handoff with the owner's band lists (2^19-entry levels, whose
    passes the owner bands) and walking the coordinates in band order, and the backward reading
    them: features and gradient bit-identical to the plain pair, one expert and three."""
    from odie_amd.encoding import grid_handoff_bytes
    enc = encoding(log2=19)
    levels, entries = grid_levels(enc)
    n = (1 << 17) + 333
    params = entries * 2
    xy = torch.from_numpy(synth.coordinates(5, n)).cuda()
    table = torch.from_numpy(synth.table(5, experts * params).astype(np.float16)).cuda()
    upstream = torch.from_numpy(synth.upstream(5, n, 32)).cuda().half()
    offsets = torch.tensor([k * n // experts for k in range(experts + 1)], dtype=torch.int32).cuda()
    size = grid_handoff_bytes(n, levels, 2, experts=experts, expert_params=params)
    assert size >= 12 * n   # band lists: a 4-byte index and an 8-byte (x, y) per coordinate
    handoff = torch.empty(size, dtype=torch.uint8, device='cuda')
    kw = dict(offsets=offsets, experts=experts, expert_params=params)
    plain = grid_forward(xy, table, levels, 2, **kw)
    walked = grid_forward(xy, table, levels, 2, handoff=handoff, **kw)
    assert np.array_equal(walked.cpu().numpy().view(np.uint16), plain.cpu().numpy().view(np.uint16))
    formed = grid_backward(xy, upstream, levels, 2, **kw)
    read = grid_backward(xy, upstream, levels, 2, handoff=handoff, **kw)
    assert np.array_equal(read.cpu().numpy().view(np.uint32), formed.cpu().numpy().view(np.uint32))


@pytest.fixture(params=[(1, 1), (1, 0), (0, 0)], ids=['owner-banded', 'owner', 'atomics'])
def backward_mode(request):
    mode, banded = request.param
    _lib.set_tuning('backward_mode', mode)
    _lib.set_tuning('banded', banded)
    yield mode
    _lib.set_tuning('backward_mode', 1)
    _lib.set_tuning('banded', 2)


def _tuned(key, value, default, call):
    _lib.set_tuning(key, value)
    try:
        return call()
    finally:
        _lib.set_tuning(key, default)


@pytest.mark.parametrize('lds_bytes', [0, 65536])
def test_single_grid_backward_tolerance(lds_bytes, backward_mode):
    enc = encoding()
    levels, entries = grid_levels(enc)
    n = 1 << 16
    xy = synth.coordinates(0, n)
    up = synth.upstream(0, n, 32)
    _lib.set_tuning('lds_bytes', lds_bytes)
    _lib.set_tuning('owner_lds_bytes', 162816 if lds_bytes else 32768)
    try:
        grad = grid_backward(torch.from_numpy(xy).cuda(), torch.from_numpy(up).cuda(), levels, 2,
                             expert_params=entries * 2)
    finally:
        _lib.set_tuning('lds_bytes', 65536)
        _lib.set_tuning('owner_lds_bytes', 162816)
    check_gradient(grad, hash_bar(xy, up, levels, 2, entries * 2),
                   'single grid lds=%d mode=%d' % (lds_bytes, backward_mode))


def test_owner_backward_is_deterministic():
    levels, entries = grid_levels(encoding(log2=14))
    n = 30000
    xy = torch.from_numpy(synth.coordinates(21, n)).cuda()
    up = torch.from_numpy(synth.upstream(21, n, 32)).cuda()
    first = grid_backward(xy, up, levels, 2, expert_params=entries * 2)
    second = grid_backward(xy, up, levels, 2, expert_params=entries * 2)
    assert torch.equal(first, second)


def test_owner_backward_is_order_independent():
    """Coordinates in row bands, x ascending within a band (the order of a stratified draw), and
    the same rows shuffled within each expert give the same fixed-point sums bit for bit: every
    coordinate is added once whichever lane takes it (dense levels spread a wave over its block,
    hashed levels take consecutive coordinates).  The upstream has one magnitude per level and
    random signs, so every range (an expert's, or a split of one) bounds the same fixed-point
    scale in both orders.  The banded order is also checked against the oracle."""
    levels, entries = grid_levels(encoding(log2=14))
    params, experts, per = entries * 2, 64, 4096
    n = experts * per
    xy = synth.coordinates(31, n)
    rng = np.random.default_rng(31)
    magnitude = 2.0 ** -(np.arange(32) // 2 % 4)
    up = (np.where(rng.random((n, 32)) < 0.5, -1.0, 1.0) * magnitude).astype(np.float16)
    banded, shuffled = [], []
    for e in range(experts):
        rows = np.arange(e * per, (e + 1) * per)
        bands = np.floor(xy[rows, 1] * 64).astype(np.int64)
        banded.append(rows[np.lexsort((xy[rows, 0], bands))])
        shuffled.append(rng.permutation(rows))
    offsets = np.arange(0, n + 1, per, dtype=np.int32)
    d_off = torch.from_numpy(offsets).cuda()
    grads = []
    for order in (np.concatenate(banded), np.concatenate(shuffled)):
        grads.append(grid_backward(torch.from_numpy(xy[order]).cuda(), torch.from_numpy(up[order]).cuda(), levels, 2,
                                   offsets=d_off, experts=experts, expert_params=params))
    assert torch.equal(grads[0], grads[1])
    order = np.concatenate(banded)
    check_gradient(grads[0], hash_bar(xy[order], up[order], levels, 2, experts * params, offsets=offsets,
                                      expert_params=params), 'banded')


def _expert_batch(seed, log2, experts, n, outside=False):
    levels, entries = grid_levels(encoding(log2=log2))
    counts = np.random.default_rng(seed).multinomial(n, np.ones(experts) / experts)
    offsets = torch.from_numpy(np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)).cuda()
    xy = synth.coordinates(seed, n)
    if outside:   # off the unit square: the band lists' last slot, visited by every slice
        xy[::97, 0] = 1.5
        xy[5::101, 1] = -0.25
        xy[7::211] = (-3.0, 2.5)
    up = torch.from_numpy(synth.upstream(seed, n, 32)).cuda()
    return levels, entries * 2, offsets, torch.from_numpy(xy).cuda(), up


@pytest.mark.parametrize('log2,experts,n,outside', [(16, 64, 1 << 20, False), (14, 16, 300000, True),
                                                    (19, 1, 1 << 20, False), (12, 3, 5000, True)])
def test_banded_owner_matches_unbanded(log2, experts, n, outside):
    """The banded fine passes skip only coordinates whose corners cannot reach the slice, and
    every pass bounds its fixed-point scale over the expert's coordinates: where the unbanded
    owner does not split a pass either (64 experts of 16384 coordinates), the gradient is the
    same integer sum bit for bit; otherwise both are within fp32 rounding of each other."""
    levels, params, offsets, xy, up = _expert_batch(log2, log2, experts, n, outside)
    run = lambda: grid_backward(xy, up.half(), levels, 2, offsets=offsets, experts=experts, expert_params=params)
    banded = _tuned('banded', 1, 2, run)
    plain = _tuned('banded', 0, 2, run)
    got, want = banded.cpu().numpy(), plain.cpu().numpy()
    if experts == 64:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    else:
        finite = np.isfinite(want)
        assert np.array_equal(finite, np.isfinite(got))
        assert np.allclose(got[finite], want[finite], rtol=1e-5, atol=1e-6 * np.abs(want[finite]).max())


def test_single_expert_band_order_against_the_oracle():
    """One expert (its offsets dropped: every row is its) with band lists: the backward transposes
    the upstream in band-list order and every pass reads it at the list positions.  Off-square
    coordinates (the lists' last slot) and a ragged last 128-row record; the gradient within the
    oracle's bar, and within fp32 rounding of the index-order (unbanded) owner."""
    levels, entries = grid_levels(encoding(log2=17))
    params, n = entries * 2, 300001
    xy = synth.coordinates(41, n)
    xy[::97, 0] = 1.5
    xy[7::211] = (-3.0, 2.5)
    up = synth.upstream(41, n, 32)
    d_xy, d_up = torch.from_numpy(xy).cuda(), torch.from_numpy(up).cuda().half()
    run = lambda: grid_backward(d_xy, d_up, levels, 2, expert_params=params)
    banded = _tuned('banded', 1, 2, run)
    plain = _tuned('banded', 0, 2, run)
    got, want = banded.cpu().numpy(), plain.cpu().numpy()
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6 * np.abs(want).max())
    check_gradient(banded, hash_bar(xy, up.astype(np.float16), levels, 2, params), 'band order')


@pytest.mark.parametrize('log2,experts,n', [(19, 1, 1 << 20), (14, 16, 300000), (12, 3, 5000)])
def test_banded_splits_are_exact(log2, experts, n):
    """Banded splits write 64-bit partial sums at one scale per pass and are added exactly: the
    gradient is the same bit for bit however finely the passes are split."""
    levels, params, offsets, xy, up = _expert_batch(log2 + 1, log2, experts, n)
    run = lambda: grid_backward(xy, up.half(), levels, 2, offsets=offsets, experts=experts, expert_params=params)
    _lib.set_tuning('banded', 1)
    try:
        auto = run()
        fine = _tuned('split_target', 1024, 0, run)
        whole = _tuned('split_target', 1 << 30, 0, run)
    finally:
        _lib.set_tuning('banded', 2)
    assert torch.equal(auto, fine) and torch.equal(auto, whole)


def test_banded_owner_with_unordered_offsets():
    """Offsets that decrease somewhere make the expert ranges overlap: the band lists are not
    used and the fine passes walk the experts' index ranges, as the unbanded owner does."""
    levels, entries = grid_levels(encoding(log2=14))
    experts, n = 16, 40000
    bounds = np.linspace(0, n, experts + 1).astype(np.int32)
    bounds[5], bounds[6] = bounds[6], bounds[5]
    offsets = torch.from_numpy(bounds).cuda()
    xy = torch.from_numpy(synth.coordinates(41, n)).cuda()
    up = torch.from_numpy(synth.upstream(41, n, 32)).cuda()
    run = lambda: grid_backward(xy, up, levels, 2, offsets=offsets, experts=experts, expert_params=entries * 2)
    assert torch.equal(_tuned('banded', 1, 2, run), _tuned('banded', 0, 2, run))


def test_experts_forward_and_backward(backward_mode):
    enc = encoding(log2=14)
    levels, entries = grid_levels(enc)
    experts, params = 16, entries * 2
    n = 40000
    rng = np.random.default_rng(1)
    counts = rng.multinomial(n, np.r_[np.zeros(2), np.ones(experts - 3), [0.0]] / (experts - 3))
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)   # empty experts 0, 1, 15
    xy = synth.coordinates(3, n)
    table = synth.table(3, experts * params).astype(np.float16)
    up = synth.upstream(3, n, 32)
    d_xy, d_off = torch.from_numpy(xy).cuda(), torch.from_numpy(offsets).cuda()
    out = grid_forward(d_xy, torch.from_numpy(table).cuda(), levels, 2, offsets=d_off, experts=experts,
                       expert_params=params)
    expected = oracle.hash_forward(xy, table, rows_of(levels), 2, offsets=offsets, expert_params=params, threads=0)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), expected.view(np.uint16))
    grad = grid_backward(d_xy, torch.from_numpy(up).cuda(), levels, 2, offsets=d_off, experts=experts,
                         expert_params=params)
    check_gradient(grad, hash_bar(xy, up, levels, 2, experts * params, offsets=offsets, expert_params=params),
                   'experts')


@pytest.mark.parametrize('features,n_levels,width,n', [(1, 5, 5, 1000), (4, 3, 16, 777), (8, 2, 16, 513),
                                                        (2, 20, 40, 3001), (2, 16, 36, 1029), (2, 1, 2, 1)])
def test_shapes_and_padding(features, n_levels, width, n, backward_mode):
    enc = encoding(levels=n_levels, base=3, log2=10, scale=1.7, features=features)
    levels, entries = grid_levels(enc)
    xy = synth.coordinates(5, n)
    xy[0] = (0.0, 0.0)
    if n > 1:
        xy[1] = (1.0, 1.0)
    table = synth.table(5, entries * features, -1.0, 1.0).astype(np.float16)
    out = grid_forward(torch.from_numpy(xy).cuda(), torch.from_numpy(table).cuda(), levels, features, width=width)
    expected = oracle.hash_forward(xy, table, rows_of(levels), features, width=width)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), expected.view(np.uint16))
    up = synth.upstream(5, n, width)
    up[:, ::3] = 0   # zero upstream values are skipped
    grad = grid_backward(torch.from_numpy(xy).cuda(), torch.from_numpy(up).cuda(), levels, features,
                         expert_params=entries * features)
    check_gradient(grad, hash_bar(xy, up, levels, features, entries * features), 'F=%d L=%d' % (features, n_levels))


def test_fp32_upstream_and_accumulate(backward_mode):
    levels, entries = grid_levels(encoding(levels=8, log2=12))
    n = 5000
    xy = synth.coordinates(7, n)
    up = synth.normal(7, 'up32', n * 16).astype(np.float32).reshape(n, 16)
    d_xy = torch.from_numpy(xy).cuda()
    grad = grid_backward(d_xy, torch.from_numpy(up).cuda(), levels, 2, expert_params=entries * 2)
    grad = grid_backward(d_xy, torch.from_numpy(up).cuda(), levels, 2, expert_params=entries * 2, gradient=grad,
                         accumulate=True)
    expected, magnitude, counts, quantum = hash_bar(xy, up, levels, 2, entries * 2)
    check_gradient(grad, (2 * expected, 2 * magnitude, 2 * counts, quantum), 'fp32 upstream x2')


def test_empty_input_and_xcd_order_invariance():
    levels, entries = grid_levels(encoding(levels=4, log2=10))
    empty = torch.zeros((0, 2), device='cuda')
    assert grid_forward(empty, torch.zeros(entries * 2, dtype=torch.float16, device='cuda'), levels, 2).shape == (0, 8)
    grad = grid_backward(empty, torch.zeros((0, 8), dtype=torch.float16, device='cuda'), levels, 2,
                         expert_params=entries * 2)
    assert not grad.any()
    xy = torch.from_numpy(synth.coordinates(9, 3000)).cuda()
    table = torch.from_numpy(synth.table(9, entries * 2).astype(np.float16)).cuda()
    first = grid_forward(xy, table, levels, 2)
    _lib.set_tuning('xcd_remap', 0)
    try:
        second = grid_forward(xy, table, levels, 2)
    finally:
        _lib.set_tuning('xcd_remap', 1)
    assert torch.equal(first, second)


def test_grid_encoding_module_autograd():
    from odie_amd.encoding import GridEncoding
    module = GridEncoding(encoding(levels=6, log2=12), dtype=torch.float16)
    with torch.no_grad():
        module.params.copy_(torch.from_numpy(synth.table(11, module.n_params, -1, 1)))
    xy = torch.from_numpy(synth.coordinates(11, 2048)).cuda()
    out = module(xy)
    weight = torch.from_numpy(synth.upstream(11, 2048, 12)).cuda()
    (out.float() * weight.float()).sum().backward()
    check_gradient(module.params.grad, hash_bar(xy.cpu().numpy(), weight.cpu().numpy(), module.levels, 2,
                                                module.n_params), 'autograd')


def _packed_layout(seed, resolutions=(8, 13, 20, 32, 51, 81), dims=(2, 2, 2, 2, 1, 4), dense=3):
    from odie_amd.model import make_layout, plane_closure
    rng = np.random.default_rng(seed)
    supports, caps = [], []
    for level, r in enumerate(resolutions):
        support = np.ones(r * r, dtype=bool) if level < dense else rng.random(r * r) < 0.3
        nodes = plane_closure(torch.as_tensor(support), r)
        supports.append(torch.as_tensor(support))
        caps.append(min((r * r + 7) // 8 * 8, (nodes.numel() + 7) // 8 * 8 + 8 * level))
    config = dict(resolutions=list(resolutions), n_levels=len(resolutions), representation='xy_planes',
                  coarse_levels=0, gate_topology='shared', gate_position='feature', initial_active_prefix=3)
    return make_layout(config, supports, list(dims), caps)


def _packed_gradient(layout, xy, up, **tuning):
    from odie_amd.model import packed_backward
    dev = {k: layout[k].cuda() for k in ('descriptors', 'node_bitmap', 'node_prefix', 'bitmap')}
    settings = dict(dict(packed_owner=1), **tuning)
    for key, value in settings.items():
        _lib.set_tuning(key, value)
    try:
        return packed_backward(xy, up, dev['descriptors'], dev['node_bitmap'], dev['node_prefix'], dev['bitmap'],
                               layout['params'])
    finally:
        _lib.set_tuning('packed_owner', 0)
        _lib.set_tuning('packed_splits', 0)


# Nine levels of 8..512 cells (the finer ones 30% supported), mixed F1/F2/F4: about 1.4e6
# parameters, so the owner's slices span several levels at the coarse end and split the fine ones.
BIG_PLANES = dict(resolutions=(8, 13, 20, 32, 64, 128, 256, 384, 512), dims=(2, 2, 2, 2, 4, 2, 2, 1, 2), dense=5)


def test_packed_owner_matches_oracle_and_atomics():
    """The owner-computes packed backward against the oracle (multi-slice layout, off-square and
    edge coordinates) and against the global-atomics kernel it replaces (fp32 order only)."""
    layout = _packed_layout(4, **BIG_PLANES)
    n, width = 30000, 32
    xy = synth.coordinates(17, n)
    xy[:4] = [(0, 0), (1, 1), (0, 1), (1, 0)]
    up = synth.upstream(17, n, width)
    d_xy, d_up = torch.from_numpy(xy).cuda(), torch.from_numpy(up).cuda()
    owner = _packed_gradient(layout, d_xy, d_up)
    atomics = _packed_gradient(layout, d_xy, d_up, packed_owner=0)
    host = {k: layout[k].numpy() for k in ('descriptors', 'node_bitmap', 'node_prefix', 'bitmap')}
    bar = packed_bar(xy, up, host, layout['params'])
    check_gradient(owner, bar, 'packed owner')
    check_gradient(atomics, bar, 'packed atomics')


@pytest.mark.parametrize('seed,n', [(5, 30000), (6, 4097), (7, 1)])
def test_packed_owner_splits_are_exact(seed, n):
    """Splits share one fixed-point scale per slice and sum 64-bit partials: the gradient is the
    same bit for bit for any split count, and from run to run."""
    layout = _packed_layout(seed, **BIG_PLANES)
    d_xy = torch.from_numpy(synth.coordinates(seed, n)).cuda()
    d_up = torch.from_numpy(synth.upstream(seed, n, 32)).cuda()
    first = _packed_gradient(layout, d_xy, d_up)
    for splits in (1, 3, 7):
        assert torch.equal(first, _packed_gradient(layout, d_xy, d_up, packed_splits=splits)), splits
    assert torch.equal(first, _packed_gradient(layout, d_xy, d_up))


def test_packed_planes_forward_backward():
    from odie_amd.model import PackedQuery
    layout = _packed_layout(2)
    n, width = 20000, 13
    xy = synth.coordinates(13, n)
    xy[:4] = [(0, 0), (1, 1), (0, 1), (1, 0)]
    grid = synth.table(13, layout['params'], -0.5, 0.5)
    host = {k: layout[k].numpy() for k in ('descriptors', 'node_bitmap', 'node_prefix', 'bitmap')}
    expected, vis = oracle.packed_forward(xy, grid, host, width)
    dev = {k: layout[k].cuda() for k in ('descriptors', 'node_bitmap', 'node_prefix', 'bitmap')}
    d_grid = torch.from_numpy(grid).cuda().requires_grad_(True)
    features, visible = PackedQuery.apply(torch.from_numpy(xy).cuda(), d_grid, dev['descriptors'], dev['node_bitmap'],
                                          dev['node_prefix'], dev['bitmap'], width)
    assert np.array_equal(features.detach().cpu().numpy().view(np.uint16), expected.view(np.uint16))
    assert np.array_equal(visible.cpu().numpy(), vis)
    up = synth.upstream(13, n, width)
    features.backward(torch.from_numpy(up).cuda())
    check_gradient(d_grid.grad, packed_bar(xy, up, host, layout['params']), 'packed')


def test_owner_scale_sees_both_features():
    """Regression: the largest |upstream| of a row block must cover both features of a level.
    Feature 0 carries values ~1e3 while feature 1 is ~1e-3 and largest in a row whose feature 0
    is tiny; a maximum taken over packed 32-bit words follows feature 1 only, picks a scale
    2^40 too fine and saturates the fixed-point contributions of feature 0."""
    levels, entries = grid_levels(encoding(log2=12))
    n = 4096
    xy = synth.coordinates(31, n)
    up = np.empty((n, 32), dtype=np.float32)
    up[:, 0::2] = np.where(synth.uniform(31, 'sign', n * 16).reshape(n, 16) < 0.5, -1000.0, 1000.0)
    up[:, 1::2] = 0.001
    up[7, 1::2] = 0.002
    up[7, 0::2] = 0.0001
    up = up.astype(np.float16)
    grad = grid_backward(torch.from_numpy(xy).cuda(), torch.from_numpy(up).cuda(), levels, 2,
                         expert_params=entries * 2)
    bar = hash_bar(xy, up, levels, 2, entries * 2)
    check_gradient(grad, bar, 'two-scale upstream')
    _check_relative(grad, bar, 'two-scale upstream')


def _check_relative(gpu, bar, label):
    """Every touched entry whose contributions are not all below 10^4 quanta (an entry reached
    only through corner weights of order 1e-5 or less) meets 1e-4 * sum|c| alone, the north
    star's relative bar, with no quantum term; and those exceptions are rare."""
    expected, magnitude, counts, quantum = bar
    got = gpu.detach().cpu().numpy().astype(np.float64)
    touched = counts > 0
    coarse = counts * quantum * 0.5 > 1e-4 * magnitude
    strict = np.abs(got - expected) <= 1e-4 * magnitude
    assert strict[touched & ~coarse].all(), '%s: %d entries miss the relative bar' % (
        label, (touched & ~coarse & ~strict).sum())
    assert (touched & coarse).sum() <= 1e-3 * touched.sum(), '%s: %d of %d entries below 10^4 quanta' % (
        label, (touched & coarse).sum(), touched.sum())


def _level_magnitudes(seed, n, levels, features, magnitude):
    """Upstream [n, levels * features] of random signs, column l * features + c of size
    magnitude[l][c] (1 +- 1/2 per row)."""
    rng = np.random.default_rng(seed)
    scale = np.repeat(np.asarray(magnitude, dtype=np.float64).reshape(1, levels * features), n, axis=0)
    sign = np.where(rng.random((n, levels * features)) < 0.5, -1.0, 1.0)
    return (sign * scale * (0.5 + rng.random((n, levels * features)))).astype(np.float16)


@pytest.mark.parametrize('experts', [1, 16])
def test_owner_scale_per_level_in_the_coarse_group(experts, backward_mode):
    """Levels that share the coarse-group pass carry upstream 10^5 apart (as a router step whose
    coarse gates differ that much can), and the two features of some levels 10^5 apart too.
    Every column has its own fixed-point scale, so the small levels keep their precision: each
    entry within its own bar, and every entry not reached only through tiny corner weights within
    1e-4 of its contribution scale alone."""
    levels, entries = grid_levels(encoding(log2=12))
    n = experts * 6000
    xy = synth.coordinates(43, n)
    magnitude = [[1e3, 1e3] if l % 2 == 0 else [1e-2, 1e-7 if l % 4 == 1 else 1e-2] for l in range(16)]
    up = _level_magnitudes(43, n, 16, 2, magnitude)
    params = entries * 2
    offsets = np.linspace(0, n, experts + 1).astype(np.int32) if experts > 1 else None
    grad = grid_backward(torch.from_numpy(xy).cuda(), torch.from_numpy(up).cuda(), levels, 2,
                         offsets=None if offsets is None else torch.from_numpy(offsets).cuda(), experts=experts,
                         expert_params=params)
    bar = hash_bar(xy, up, levels, 2, experts * params, offsets=offsets, expert_params=params)
    check_gradient(grad, bar, 'levels 10^5 apart, mode %d' % backward_mode)
    _check_relative(grad, bar, 'levels 10^5 apart, mode %d' % backward_mode)


def test_packed_owner_scale_per_level():
    """The packed-plane owner's slices span several coarse levels; their upstream columns are
    10^6 apart (alternating by level, and by feature within the four-feature level): each keeps
    its own scale, for any split count."""
    layout = _packed_layout(8, **BIG_PLANES)
    n, width = 20000, 32
    xy = synth.coordinates(47, n)
    dims = BIG_PLANES['dims']
    magnitude = np.ones(width)
    column = 0
    for level, f in enumerate(dims):
        for c in range(f):
            magnitude[column] = 1e3 if (level + c) % 2 == 0 else 1e-3
            column += 1
    rng = np.random.default_rng(47)
    up = (np.where(rng.random((n, width)) < 0.5, -1.0, 1.0) * magnitude * (0.5 + rng.random((n, width))))
    up = up.astype(np.float16)
    d_xy, d_up = torch.from_numpy(xy).cuda(), torch.from_numpy(up).cuda()
    host = {k: layout[k].numpy() for k in ('descriptors', 'node_bitmap', 'node_prefix', 'bitmap')}
    bar = packed_bar(xy, up, host, layout['params'])
    first = _packed_gradient(layout, d_xy, d_up)
    check_gradient(first, bar, 'packed owner, levels 10^6 apart')
    _check_relative(first, bar, 'packed owner, levels 10^6 apart')
    for splits in (1, 5):
        assert torch.equal(first, _packed_gradient(layout, d_xy, d_up, packed_splits=splits)), splits


@pytest.mark.parametrize('experts,n', [(8, 50000), (1, 4097), (3, 1)])
def test_planes_backward_equals_rows(experts, n):
    """odie_grid_backward_planes on the upstream in the decoder's planes layout (level-major fp16
    pairs and per-column 128-row maxima) gives odie_grid_backward's gradient bit for bit, and
    accumulates into a given gradient."""
    from odie_amd.experts import ExpertGrid
    encoding = dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=12, base_resolution=8, per_level_scale=1.4)
    grid = ExpertGrid(encoding, experts)
    coords = torch.from_numpy(synth.coordinates(51, n)).cuda()
    counts = np.diff(np.linspace(0, n, experts + 1).astype(np.int64))
    offsets = torch.from_numpy(np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)).cuda()
    upstream = torch.from_numpy(synth.upstream(51, n, 32)).cuda()
    planes = upstream.view(torch.int32).t().contiguous()
    records = (n + 127) // 128
    column = torch.zeros((records * 128, 32), dtype=torch.float32, device='cuda')
    column[:n] = upstream.abs().float()
    blockmax = column.view(records, 128, 32).amax(dim=1).contiguous()
    rows = grid.backward(coords, offsets, upstream)
    via_planes = grid.backward_planes(coords, offsets, planes, blockmax)
    assert torch.equal(rows.view(torch.int32), via_planes.view(torch.int32))
    twice = grid.backward_planes(coords, offsets, planes, blockmax, gradient=via_planes.clone(), accumulate=True)
    assert torch.equal(twice, 2 * rows)


@pytest.mark.parametrize('log2,experts,n,outside', [(16, 64, 1 << 20, False), (14, 16, 300000, True),
                                                    (15, 3, 5000, True), (16, 1, 65536, False)])
def test_owner_masks_are_bit_identical(log2, experts, n, outside):
    """Hashed slices that walk only the coordinates whose slice masks reach them form the same
    integer sums as slices that walk every coordinate: the gradient bit for bit (coordinates off
    the unit square included), for 2- to 8-block levels."""
    levels, params, offsets, xy, up = _expert_batch(log2 + 3, log2, experts, n, outside)
    run = lambda: grid_backward(xy, up.half(), levels, 2, offsets=offsets, experts=experts, expert_params=params)
    _lib.set_tuning('banded', 0)
    try:
        masked = _tuned('owner_masks', 1, 1, run)
        plain = _tuned('owner_masks', 0, 1, run)
    finally:
        _lib.set_tuning('banded', 2)
    assert torch.equal(masked.view(torch.int32), plain.view(torch.int32))
