"""PackedXYPlanes, the on-demand model (odie/model.py:154-279), and build_model
(odie/model.py:318-321): the constructor's refusals and dispatch (CPU), and the evaluation
forward against the reference's gating formula written out in torch (GPU)."""
import numpy as np
import pytest
import torch

from odie_amd import synth
from odie_amd.hash_grid import HashGrid
from odie_amd.model import PackedXYPlanes, build_model

RESOLUTIONS = [4, 5, 6, 8, 10, 12, 16, 20, 24, 32, 40, 48, 64, 80, 96, 128]


def _config(router=True, coarse=0, **changes):
    config = dict(resolutions=RESOLUTIONS, n_levels=16, representation='xy_planes', coarse_levels=coarse,
                  gate_coarse_levels_K=coarse, gate_topology='shared', gate_position='feature',
                  initial_active_prefix=8, seed=5, feature_init_std=5e-2, router_enabled=router,
                  router_output_activation='sigmoid', decoder_parameters=7168,
                  gate_parameters=1536 if router else 0)
    config.update(changes)
    return config


def _inputs(seed, dims=None):
    supports, caps = [], []
    for level, r in enumerate(RESOLUTIONS):
        supports.append(torch.ones(r * r, dtype=torch.bool) if level < 8 else
                        torch.from_numpy(synth.uniform(seed + level, 'model_support', r * r) < 0.4))
        caps.append((r * r + 7) // 8 * 8)
    return supports, [2] * 16 if dims is None else list(dims), caps


# the reference's DIV2K rows (odie/config.py:129: [2]*15 + [1], 31 columns padded to 32) and a
# row of mixed F1/F2/F4 levels (36 columns padded to 48)
DIV2K_DIMS = [2] * 15 + [1]
MIXED_DIMS = [1, 4, 2, 2, 4, 1, 2, 2, 2, 4, 2, 2, 1, 2, 1, 4]


def _head_sizes(dims):
    width = (sum(dims) + 15) // 16 * 16
    return dict(decoder_parameters=64 * width + 5120, gate_parameters=32 * width + 32 * 16)


@pytest.mark.parametrize('changes,kwargs,error,message', [
    ({}, dict(axis_mode='x'), ValueError, 'axis'),
    ({}, dict(kernel_a=0.5), ValueError, 'axis'),
    (dict(decoder_parameters=1), {}, RuntimeError, 'head allocation'),
    (dict(gate_parameters=0), {}, RuntimeError, 'head allocation'),
    (dict(gate_coarse_levels_K=3), {}, ValueError, 'Gate K'),
])
def test_packed_model_refuses_what_the_reference_refuses(changes, kwargs, error, message):
    supports, dims, caps = _inputs(1)
    with pytest.raises(error, match=message):
        PackedXYPlanes(_config(**changes), supports, dims, caps, device='cpu', **kwargs)


@pytest.mark.parametrize('dims', [DIV2K_DIMS, MIXED_DIMS])
def test_packed_model_takes_mixed_feature_rows(dims):
    supports, dims, caps = _inputs(1, dims)
    model = PackedXYPlanes(_config(**_head_sizes(dims)), supports, dims, caps, device='cpu')
    width = (sum(dims) + 15) // 16 * 16
    assert model.input_width == sum(dims) and model.decoder.width == model.gate.width == width
    assert model.gate.features == dims
    with pytest.raises(RuntimeError, match='head allocation'):
        PackedXYPlanes(_config(), supports, dims, caps, device='cpu') if width != 32 else \
            PackedXYPlanes(_config(decoder_parameters=1), supports, dims, caps, device='cpu')


def test_build_model_dispatches_on_the_representation():
    supports, dims, caps = _inputs(2)
    model = build_model(_config(router=False), supports, dims, caps, device='cpu')
    assert isinstance(model, PackedXYPlanes) and model.gate is None
    stats = model.storage_stats()
    assert stats['grid_params'] == model.grid.numel() and stats['decoder_params'] == 7168
    assert stats['layout_version'] == 'packed-xy-only-native-closure-v1'
    with pytest.raises(ValueError, match='no supports'):
        build_model(dict(_config(), representation='hash_grid'), supports, dims, caps)
    assert HashGrid is not None


@pytest.mark.gpu
@pytest.mark.parametrize('router,coarse,prefix,dims', [(False, 0, 16, None), (True, 0, 16, None), (True, 2, 12, None),
                                                       (True, 3, 3, None), (True, 0, 16, DIV2K_DIMS),
                                                       (True, 2, 14, MIXED_DIMS), (False, 0, 16, MIXED_DIMS)])
def test_packed_model_forward_follows_the_reference_gating(router, coarse, prefix, dims):
    """forward = decoder(rows of raw * fp16(gate * (visible & level < prefix)), padded with ones
    to align16 columns), with raw past the prefix zeroed and the first K gates one
    (odie/model.py:266-279), written here in torch from the gate activations the kernel
    reports."""
    supports, dims, caps = _inputs(3, dims)
    config = _config(router, coarse, **_head_sizes(dims))
    if not router:
        config['gate_parameters'] = 0
    model = PackedXYPlanes(config, supports, dims, caps)
    model.set_active_prefix(prefix)
    xy = torch.from_numpy(synth.coordinates(3, 4000)).cuda()
    rgb = model.forward(xy)
    raw, visible = model.query_features(xy)
    levels = torch.tensor([l for l, f in enumerate(dims) for _ in range(f)], device='cuda')
    active = torch.arange(16, device='cuda') < prefix
    raw = raw * active[levels].half()
    width = model.decoder.width
    rows = torch.ones((4000, width), dtype=torch.float16, device='cuda')
    rows[:, :raw.shape[1]] = raw
    if router:
        _, activation = model.gate.forward(rows)
        gates = torch.cat([torch.ones_like(activation[:, :coarse]), activation[:, coarse:]], dim=1)
        if prefix <= coarse:
            gates = torch.ones_like(gates)
        weights = (gates * (visible & active).float()).half()[:, levels]
        rows[:, :raw.shape[1]] = raw * weights
    want = model.decoder.forward(rows).float()[:, :3]
    assert rgb.shape == (4000, 3)
    assert torch.equal(rgb, want)
    if prefix < 16:
        full = PackedXYPlanes(config, supports, dims, caps)
        full.set_active_prefix(16)
        assert not torch.equal(rgb, full.forward(xy))


@pytest.mark.gpu
def test_native_optimizer_trains_a_packed_model():
    """NativeOptimizer takes PackedXYPlanes itself (its grid, addressing buffers, layout, prefix
    and heads): steps move the grid and both heads, and forward sees the new weights."""
    from odie_amd.native_backend import make_native_optimizer
    width, height = 97, 61
    supports, dims, caps = _inputs(4)
    config = dict(_config(router=True), target_storage='uint8', plane_feature_dimensions=dims, grid_lr=1e-2,
                  gate_lr=1e-3, decoder_lr=1e-3)
    model = PackedXYPlanes(config, supports, dims, caps)
    model.set_active_prefix(16)
    image = torch.from_numpy(synth.image(8, width, height)).cuda().contiguous()
    xy = torch.from_numpy(synth.coordinates(8, 777)).cuda()
    before = model.forward(xy)
    grid, decoder, gate = model.grid.clone(), model.decoder.params.clone(), model.gate.params.clone()
    opt, _ = make_native_optimizer(model, image, (height, width), config)
    for step in range(3):
        opt.step_raw(torch.from_numpy(synth.integers(step, 'packed_model_ids', 4096, width * height)).cuda())
    torch.cuda.synchronize()
    opt.close()
    assert not torch.equal(model.grid, grid)
    assert not torch.equal(model.decoder.params, decoder)
    assert not torch.equal(model.gate.params, gate)
    assert not torch.equal(model.forward(xy), before)
