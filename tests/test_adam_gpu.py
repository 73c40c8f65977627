"""Fused Adam against the oracle (fp64 closed form) and torch.optim.Adam."""
import numpy as np
import pytest
import torch

import oracle
from odie_amd import synth
from odie_amd.optimizer import FusedAdam

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('variant,grad_dtype,n', [('torch', torch.float32, 1000003), ('tcnn', torch.float16, 4099),
                                                  ('torch', torch.float16, 17), ('tcnn', torch.float32, 100000),
                                                  ('tcnn_dense', torch.float32, 7168)])
def test_adam_matches_oracle(variant, grad_dtype, n):
    start = synth.normal(5, 'params', n).astype(np.float32)
    master = torch.from_numpy(start).cuda()
    half = torch.empty(n, dtype=torch.float16, device='cuda')
    opt = FusedAdam(master, lr=1e-2, variant=variant, half_copy=half)
    p = start.astype(np.float64)
    m, v = np.zeros(n), np.zeros(n)
    steps = np.zeros(n, dtype=np.uint32)
    for t in range(1, 4):
        g = (synth.normal(5 + t, 'grad', n) * 128).astype(np.float32)
        g[::5] = 0.0
        grad = torch.from_numpy(g).to(grad_dtype)
        opt.step(grad.cuda(), loss_scale=128.0)
        p = oracle.adam({'torch': 0, 'tcnn': 1, 'tcnn_dense': 2}[variant], p, grad.float().numpy().astype(np.float64), m, v, steps, t,
                        1e-2, scale=128.0)
    got = master.cpu().numpy().astype(np.float64)
    assert np.allclose(got, p, rtol=1e-5, atol=1e-6), np.abs(got - p).max()
    assert np.array_equal(half.cpu().numpy().view(np.uint16), master.cpu().numpy().astype(np.float16).view(np.uint16))
    if variant != 'torch':
        assert np.array_equal(opt.steps.cpu().numpy().astype(np.uint32), steps)


def test_adam_matches_torch_optimizer():
    n = 5000
    start = synth.normal(9, 'params', n).astype(np.float32)
    reference = torch.nn.Parameter(torch.from_numpy(start.copy()))
    torch_opt = torch.optim.Adam([reference], lr=1e-3, betas=(.9, .999), eps=1e-15, foreach=False)
    master = torch.from_numpy(start.copy()).cuda()
    opt = FusedAdam(master, lr=1e-3)
    for t in range(5):
        g = torch.from_numpy(synth.normal(20 + t, 'grad', n).astype(np.float32))
        reference.grad = g / 128.0
        torch_opt.step()
        opt.step((g).cuda(), loss_scale=128.0)
    assert torch.allclose(master.cpu(), reference.detach(), rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize('experts,n,variant,up16', [
    (4, 20000, 'tcnn', True),
    (4, 20000, 'torch', True),
    (3, 9000, 'tcnn_dense', False),   # fp32 upstream
    (1, 200000, 'tcnn', True),        # one expert, many coords: the backward splits and reduces
    (2, 0, 'tcnn_dense', True),       # empty batch: every gradient is zero
])
def test_grid_backward_adam_equals_backward_then_adam(experts, n, variant, up16):
    from odie_amd.experts import ExpertGrid
    encoding = dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=12, base_resolution=8, per_level_scale=1.4)
    grids, optimizers = [], []
    for _ in range(2):
        grid = ExpertGrid(encoding, experts, dtype=torch.float16)
        master = torch.from_numpy(synth.table(8, grid.table.numel())).cuda()
        grid.table.copy_(master)
        grids.append(grid)
        optimizers.append(FusedAdam(master, lr=1e-2, variant=variant, half_copy=grid.table))
    coords = torch.from_numpy(synth.coordinates(9, n)).cuda()
    counts = np.diff(np.linspace(0, n, experts + 1).astype(np.int64))
    offsets = torch.from_numpy(np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)).cuda()
    for step in range(2):
        upstream = torch.from_numpy(synth.upstream(10 + step, n, 32)).cuda()
        if not up16:
            upstream = upstream.float()
        grids[0].backward_adam(coords, offsets, upstream, optimizers[0], loss_scale=128.0)
        gradient = grids[1].backward(coords, offsets, upstream)
        optimizers[1].step(gradient, loss_scale=128.0)
    for name in ('master', 'm', 'v'):
        x, y = (getattr(o, name).cpu().numpy() for o in optimizers)
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), name
    assert np.array_equal(grids[0].table.cpu().numpy().view(np.uint16), grids[1].table.cpu().numpy().view(np.uint16))
    if variant != 'torch':
        assert np.array_equal(optimizers[0].steps.cpu().numpy(), optimizers[1].steps.cpu().numpy())


@pytest.mark.parametrize('experts,n,variant', [
    (4, 20000, 'tcnn'),
    (1, 200000, 'tcnn'),        # one expert, many coords: split passes and their reduction
    (3, 1000 + 17, 'torch'),    # ragged last 128-row record
])
def test_grid_backward_adam_planes_equals_rows(experts, n, variant):
    """odie_grid_backward_adam_planes on the upstream's level-major planes and 128-row maxima
    (built here with torch) gives the row-major entry point's update bit for bit."""
    from odie_amd.experts import ExpertGrid
    encoding = dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=12, base_resolution=8, per_level_scale=1.4)
    grids, optimizers = [], []
    for _ in range(2):
        grid = ExpertGrid(encoding, experts, dtype=torch.float16)
        master = torch.from_numpy(synth.table(8, grid.table.numel())).cuda()
        grid.table.copy_(master)
        grids.append(grid)
        optimizers.append(FusedAdam(master, lr=1e-2, variant=variant, half_copy=grid.table))
    coords = torch.from_numpy(synth.coordinates(9, n)).cuda()
    counts = np.diff(np.linspace(0, n, experts + 1).astype(np.int64))
    offsets = torch.from_numpy(np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)).cuda()
    records = (n + 127) // 128
    for step in range(2):
        upstream = torch.from_numpy(synth.upstream(10 + step, n, 32)).cuda()
        planes = upstream.view(torch.int32).t().contiguous()
        column = torch.zeros((records * 128, 32), dtype=torch.float32, device='cuda')
        column[:n] = upstream.abs().view(n, 32).float()
        blockmax = column.view(records, 128, 32).amax(dim=1).contiguous()
        grids[0].backward_adam_planes(coords, offsets, planes, blockmax, optimizers[0], loss_scale=128.0)
        grids[1].backward_adam(coords, offsets, upstream, optimizers[1], loss_scale=128.0)
    for name in ('master', 'm', 'v'):
        x, y = (getattr(o, name).cpu().numpy() for o in optimizers)
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), name
    assert np.array_equal(grids[0].table.cpu().numpy().view(np.uint16), grids[1].table.cpu().numpy().view(np.uint16))


def test_fused_backward_with_split_group_pass():
    """One expert with 2^19-entry tables and 65536 coordinates (the native step's batch): only
    the coarse-group pass is split over the coordinates and summed, with the optimizer applied in
    that sum; the rest flush straight into the optimizer.  Same update as backward + adam."""
    from odie_amd.experts import ExpertGrid
    encoding = dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=19, base_resolution=16,
                    per_level_scale=1.38)
    n = 65536
    grids, optimizers = [], []
    for _ in range(2):
        grid = ExpertGrid(encoding, 1, dtype=torch.float16)
        master = torch.from_numpy(synth.table(12, grid.table.numel())).cuda()
        grid.table.copy_(master)
        grids.append(grid)
        optimizers.append(FusedAdam(master, lr=1e-2, variant='tcnn', half_copy=grid.table))
    coords = torch.from_numpy(synth.coordinates(13, n)).cuda()
    offsets = torch.tensor([0, n], dtype=torch.int32, device='cuda')
    for step in range(2):
        upstream = torch.from_numpy(synth.upstream(14 + step, n, 32)).cuda()
        grids[0].backward_adam(coords, offsets, upstream, optimizers[0], loss_scale=128.0)
        gradient = grids[1].backward(coords, offsets, upstream)
        optimizers[1].step(gradient, loss_scale=128.0)
    for name in ('master', 'm', 'v'):
        x, y = (getattr(o, name).cpu().numpy() for o in optimizers)
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), name
    assert np.array_equal(optimizers[0].steps.cpu().numpy(), optimizers[1].steps.cpu().numpy())


@pytest.mark.parametrize('variant', ['tcnn', 'tcnn_dense'])
def test_fused_flush_with_old_and_recent_ages(variant):
    """Step 300 with per-parameter ages spread over 0..299: the fused flush takes the step size of
    the latest 256 ages from a per-workgroup table and computes older ones directly; the update is
    the unfused optimizer's bit for bit."""
    from odie_amd.experts import ExpertGrid
    encoding = dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=12, base_resolution=8, per_level_scale=1.4)
    n, experts = 20000, 4
    grids, optimizers = [], []
    for _ in range(2):
        grid = ExpertGrid(encoding, experts, dtype=torch.float16)
        master = torch.from_numpy(synth.table(8, grid.table.numel())).cuda()
        grid.table.copy_(master)
        grids.append(grid)
        opt = FusedAdam(master, lr=1e-2, variant=variant, half_copy=grid.table)
        ages = synth.integers(21, 'ages', master.numel(), 300).astype(np.int32)
        opt.steps.copy_(torch.from_numpy(ages).cuda())
        opt.m.copy_(master * 1e-3)
        opt.v.copy_(master * master * 1e-4)
        opt.step_count = 299
        optimizers.append(opt)
    coords = torch.from_numpy(synth.coordinates(9, n)).cuda()
    offsets = torch.from_numpy(np.linspace(0, n, experts + 1).astype(np.int32)).cuda()
    upstream = torch.from_numpy(synth.upstream(23, n, 32)).cuda()
    grids[0].backward_adam(coords, offsets, upstream, optimizers[0], loss_scale=128.0)
    optimizers[1].step(grids[1].backward(coords, offsets, upstream), loss_scale=128.0)
    for name in ('master', 'm', 'v', 'steps'):
        x, y = (getattr(o, name).cpu().numpy() for o in optimizers)
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), name
    assert np.array_equal(grids[0].table.cpu().numpy().view(np.uint16), grids[1].table.cpu().numpy().view(np.uint16))
