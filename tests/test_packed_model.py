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


def _inputs(seed):
    supports, caps = [], []
    for level, r in enumerate(RESOLUTIONS):
        supports.append(torch.ones(r * r, dtype=torch.bool) if level < 8 else
                        torch.from_numpy(synth.uniform(seed + level, 'model_support', r * r) < 0.4))
        caps.append((r * r + 7) // 8 * 8)
    return supports, [2] * 16, caps


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


def test_packed_model_refuses_other_feature_widths():
    supports, dims, caps = _inputs(1)
    with pytest.raises(ValueError, match='levels of 2 features'):
        PackedXYPlanes(_config(), supports, [1] + dims[1:], caps, device='cpu')


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
@pytest.mark.parametrize('router,coarse,prefix', [(False, 0, 16), (True, 0, 16), (True, 2, 12), (True, 3, 3)])
def test_packed_model_forward_follows_the_reference_gating(router, coarse, prefix):
    """forward = decoder(raw * fp16(gate * (visible & level < prefix))), with raw past the prefix
    zeroed and the first K gates one (odie/model.py:266-279), written here in torch from the
    gate activations the kernel reports."""
    supports, dims, caps = _inputs(3)
    model = PackedXYPlanes(_config(router, coarse), supports, dims, caps)
    model.set_active_prefix(prefix)
    xy = torch.from_numpy(synth.coordinates(3, 4000)).cuda()
    rgb = model.forward(xy)
    raw, visible = model.query_features(xy)
    active = torch.arange(16, device='cuda') < prefix
    raw = raw * active.repeat_interleave(2).half()
    if router:
        _, activation = model.gate.forward(raw)
        gates = torch.cat([torch.ones_like(activation[:, :coarse]), activation[:, coarse:]], dim=1)
        if prefix <= coarse:
            gates = torch.ones_like(gates)
        weights = (gates * (visible & active).float()).half().repeat_interleave(2, dim=1)
        raw = raw * weights
    want = model.decoder.forward(raw).float()[:, :3]
    assert rgb.shape == (4000, 3)
    assert torch.equal(rgb, want)
    if prefix < 16:
        full = PackedXYPlanes(_config(router, coarse), supports, dims, caps)
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
