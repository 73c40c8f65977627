"""HashGrid, the no-on-demand model (odie/hash_grid.py:8-80): its constructor's refusals (CPU),
its evaluation forward against the composition of the tested entry points, and
NativeOptimizer training it directly (GPU)."""
import numpy as np
import pytest
import torch

from odie_amd import synth
from odie_amd.config import hash_grid_layout
from odie_amd.hash_grid import HashGrid

ENCODING = dict(otype='HashGrid', n_levels=16, n_features_per_level=2, log2_hashmap_size=12, base_resolution=4,
                per_level_scale=1.5)


def _config(router=True, coarse=0, **changes):
    resolutions, _ = hash_grid_layout(ENCODING)
    config = dict(representation='hash_grid', hash_encoding=ENCODING, n_levels=16, initial_active_prefix=16,
                  plane_feature_dimensions=[2] * 16, router_enabled=router, gate_coarse_levels_K=coarse,
                  router_output_activation='sigmoid', seed=3, decoder_parameters=7168,
                  gate_parameters=1536 if router else 0, resolutions=resolutions, target_storage='uint8',
                  grid_lr=1e-2, gate_lr=1e-3, decoder_lr=1e-3)
    config.update(changes)
    return config


def _caps():
    return hash_grid_layout(ENCODING)[1]


@pytest.mark.parametrize('changes,supports,error,message', [
    (dict(initial_active_prefix=12), [], ValueError, 'all levels active'),
    ({}, [torch.ones(16, dtype=torch.bool)], ValueError, 'no supports'),
    (dict(decoder_parameters=7167), [], RuntimeError, 'budget'),
    (dict(gate_parameters=0), [], RuntimeError, 'budget'),
])
def test_hash_grid_refuses_what_the_reference_refuses(changes, supports, error, message):
    with pytest.raises(error, match=message):
        HashGrid(_config(**changes), supports, [2] * 16, _caps(), device='cpu')


def test_hash_grid_refuses_planes_that_differ_from_the_encoding():
    with pytest.raises(ValueError, match='features per level'):
        HashGrid(_config(), [], [2] * 15 + [1], _caps(), device='cpu')


@pytest.mark.parametrize('levels,features', [(8, 2), (12, 4), (20, 1)])
def test_hash_grid_takes_other_shapes(levels, features):
    encoding = dict(ENCODING, n_levels=levels, n_features_per_level=features)
    resolutions, caps = hash_grid_layout(encoding)
    width = (levels * features + 15) // 16 * 16
    config = _config(hash_encoding=encoding, n_levels=levels, initial_active_prefix=levels, resolutions=resolutions,
                     plane_feature_dimensions=[features] * levels, decoder_parameters=64 * width + 5120,
                     gate_parameters=32 * width + 32 * ((levels + 15) // 16 * 16))
    model = HashGrid(config, [], [features] * levels, caps, device='cpu')
    assert model.grid.numel() == features * sum(caps)
    assert model.decoder.width == model.gate.width == width
    assert model.storage_stats()['gate_params'] == config['gate_parameters']


def test_hash_grid_refuses_a_table_that_differs_from_the_caps():
    caps = _caps()
    caps[-1] += 8
    with pytest.raises(RuntimeError, match='budget'):
        HashGrid(_config(), [], [2] * 16, caps, device='cpu')


def test_hash_grid_layout_and_stats_on_the_host():
    model = HashGrid(_config(router=False), [], [2] * 16, _caps(), device='cpu')
    stats = model.storage_stats()
    assert stats['grid_params'] == model.grid.numel() == 2 * sum(_caps())
    assert stats['gate_params'] == 0 and stats['decoder_params'] == 7168
    assert [level['resolution'] for level in stats['levels']] == hash_grid_layout(ENCODING)[0]
    assert float(model.grid.abs().max()) <= 1e-4
    model.set_active_prefix(16)
    with pytest.raises(ValueError):
        model.set_active_prefix(15)


@pytest.mark.gpu
@pytest.mark.parametrize('router,coarse', [(False, 0), (True, 0), (True, 3)])
def test_hash_grid_forward_is_the_composition(router, coarse):
    from odie_amd.encoding import grid_forward
    model = HashGrid(_config(router, coarse), [], [2] * 16, _caps())
    model.grid.copy_(torch.from_numpy((synth.normal(4, 'hash_grid_test', model.grid.numel()) * 0.05)
                                      .astype(np.float32)))
    xy = torch.from_numpy(synth.coordinates(4, 5000)).cuda()
    rgb = model.forward(xy)
    raw = grid_forward(xy, model.grid.half(), model.levels, 2)
    if router:
        raw, _ = model.gate.forward(raw)
    want = model.decoder.forward(raw).float()[:, :3]
    assert rgb.shape == (5000, 3) and rgb.dtype == torch.float32
    assert torch.equal(rgb, want)


@pytest.mark.gpu
def test_native_optimizer_trains_a_hash_grid():
    """NativeOptimizer takes the HashGrid itself, as the reference's takes its model
    (odie/native_backend.py:47-73): a step moves the grid and the heads, and the model's forward
    then sees the new weights."""
    from odie_amd.native_backend import NativeOptimizer
    width, height = 97, 61
    model = HashGrid(_config(router=True), [], [2] * 16, _caps())
    image = torch.from_numpy(synth.image(6, width, height)).cuda().contiguous()
    xy = torch.from_numpy(synth.coordinates(6, 777)).cuda()
    before = model.forward(xy)
    grid, decoder, gate = model.grid.clone(), model.decoder.params.clone(), model.gate.params.clone()
    opt = NativeOptimizer(model, image, (height, width), _config(router=True), [model.grid])
    for step in range(3):
        opt.step_raw(torch.from_numpy(synth.integers(step, 'hash_grid_ids', 4096, width * height)).cuda())
    torch.cuda.synchronize()
    opt.close()
    assert not torch.equal(model.grid, grid)
    assert not torch.equal(model.decoder.params, decoder)
    assert not torch.equal(model.gate.params, gate)
    assert not torch.equal(model.forward(xy), before)
