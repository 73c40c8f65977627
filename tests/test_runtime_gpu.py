"""The native step runtime (odie_create / odie_step / odie_configure / odie_state ..., the
reference's Probe at odie/native/runtime.cu:163-331) against the composition of the separately
tested entry points on the same inputs: the hash-grid step bit for bit (its backward and Adam are
deterministic), the packed-plane step with the grid gradient within the encode-backward
tolerance (fp32 atomics) and every update bit for bit from that gradient; a captured graph
replayed with eager work between replays, bit for bit against eager steps; the optimizer-state
summaries.  Gradients reach the optimizers through fp16 stores as in the reference: the grid's
fp16(g) at loss scale 128, the heads' fp16(fp16(g) / 128) at 128 (odie/native/runtime.cu:
298-309, kernels.cuh:140-143)."""
import json

import numpy as np
import pytest
import torch

from odie_amd import _lib, synth
from odie_amd.config import grid_levels
from odie_amd.decoder import Decoder
from odie_amd.encoding import grid_backward, grid_forward
from odie_amd.gate import Gate
from odie_amd.model import PackedPlanes
from odie_amd.native_backend import NativeModel, NativeOptimizer, make_native_optimizer
from odie_amd.optimizer import FusedAdam

pytestmark = pytest.mark.gpu

HASH = dict(otype='HashGrid', n_levels=16, n_features_per_level=2, log2_hashmap_size=12, base_resolution=4,
            per_level_scale=1.5)
RESOLUTIONS = [4, 5, 6, 8, 10, 12, 16, 20, 24, 32, 40, 48, 64, 80, 96, 128]
# level rows of the reference's own configurations: DIV2K (odie/config.py:129, configs/baselines/
# odie_div2k.json: [2]*15 + [1]) and the level ablations (configs/ablations/div2k_L8/L12/L20.json)
SHAPES = {'16x2': [2] * 16, 'div2k': [2] * 15 + [1], 'L8': [2] * 7 + [1], 'L12': [2] * 11 + [1],
          'L20': [2] * 19 + [1]}


def _resolutions(levels):
    """levels resolutions from 4 to 128, nondecreasing (the 16-level list for 16 levels)."""
    if levels == 16:
        return RESOLUTIONS
    return [int(round(4 * 32 ** (l / (levels - 1)))) for l in range(levels)]


def _config(representation, router, coarse=0, activation='sigmoid', dims=None, encoding=None):
    dims = [2] * 16 if dims is None else dims
    return dict(representation=representation, hash_encoding=encoding or HASH, n_levels=len(dims),
                plane_feature_dimensions=dims, router_enabled=router, target_storage='uint8',
                gate_coarse_levels_K=coarse, router_output_activation=activation, grid_lr=1e-2, gate_lr=2e-3,
                decoder_lr=1e-3)


def _width(dims):
    return (sum(dims) + 15) // 16 * 16


def _stream():
    return torch.cuda.Stream()


def _image(seed, width, height):
    return torch.from_numpy(synth.image(seed, width, height)).cuda().contiguous()


def _planes(seed, dims=None):
    dims = [2] * 16 if dims is None else dims
    resolutions = _resolutions(len(dims))
    full = len(dims) // 2
    supports, caps = [], []
    for level, r in enumerate(resolutions):
        if level < full:
            supports.append(torch.ones(r * r, dtype=torch.bool))
        else:
            supports.append(torch.from_numpy(synth.uniform(seed + level, 'runtime_support', r * r) < 0.35))
        caps.append((r * r + 7) // 8 * 8)
    config = dict(resolutions=resolutions, n_levels=len(dims), representation='xy_planes', coarse_levels=0,
                  gate_topology='shared', gate_position='feature', initial_active_prefix=full, seed=seed,
                  feature_init_std=5e-2)
    planes = PackedPlanes(config, supports, dims, caps)
    planes.set_active_prefix(len(dims))
    return planes


class Composition:
    """The step from the tested entry points, with its own copies of every weight."""

    def __init__(self, grid, decoder, gate, config, width, height, hash_levels=None, planes=None, half=True):
        self.dims = list(config['plane_feature_dimensions'])
        self.row = _width(self.dims)
        self.grid = grid.clone()
        self.decoder = Decoder(weights=decoder.params.cpu().numpy(), width=self.row)
        self.gate = None if gate is None else Gate(weights=gate.params.cpu().numpy(), coarse=gate.coarse,
                                                   activation='softplus' if gate.softplus else 'sigmoid',
                                                   features=self.dims)
        self.levels, self.planes, self.half = hash_levels, planes, half
        self.table = self.grid.half() if hash_levels is not None else None
        self.grid_opt = FusedAdam(self.grid, config['grid_lr'], eps=1e-15, variant='tcnn', half_copy=self.table)
        self.dec_opt = FusedAdam(self.decoder.params, config['decoder_lr'], eps=1e-15, variant='tcnn_dense',
                                 half_copy=self.decoder.half)
        self.gate_opt = None if gate is None else FusedAdam(self.gate.params, config['gate_lr'], eps=1e-15,
                                                            variant='tcnn_dense', half_copy=self.gate.half)
        self.width, self.height = width, height

    def forward(self, ids, active=None):
        w = self.width
        active = len(self.dims) if active is None else active
        rx = torch.tensor(np.float32(1.0 / (w - 1)), device='cuda')
        ry = torch.tensor(np.float32(1.0 / (self.height - 1)), device='cuda')
        xy = torch.stack([(ids % w).float() * rx, (ids // w).float() * ry], dim=1).contiguous()
        if self.levels is not None:
            raw = grid_forward(xy, self.table, self.levels, self.dims[0], width=self.row)
            vis = None
        else:
            raw, vis = _packed_query(self.planes, self.grid, xy, self.row)
            raw[:, sum(self.dims[:active]):] = 0
            vis[:, active:] = 0
        raw[:, sum(self.dims):] = 1.0          # the row's padding columns (odie/native/runtime.cu:51)
        return xy, raw, vis

    def step(self, ids, image, active=None, grid_gradient=None, update=True):
        xy, raw, vis = self.forward(ids, active)
        squares = torch.empty(ids.numel(), dtype=torch.float32, device='cuda')
        features, sigmoid = raw, None
        if self.gate is not None:
            features, sigmoid = self.gate.forward(raw, visible=vis)
        dz = self.decoder.train(features, rgb=image.reshape(-1), ids=ids, squares=squares)
        up = dz if self.gate is None else self.gate.backward(raw, dz, sigmoid, visible=vis)
        if self.levels is not None:
            gradient = grid_backward(xy, up, self.levels, self.dims[0], expert_params=self.grid.numel())
        else:
            gradient = _packed_gradient(self.planes, xy, up, self.grid.numel())
        if update:
            used = gradient if grid_gradient is None else grid_gradient
            self.grid_opt.step(used.half() if self.half else used, loss_scale=128.0)
            for head, opt in ((self.gate, self.gate_opt), (self.decoder, self.dec_opt)):
                if head is not None:
                    opt.step((head.grad.half().float() / 128.0).half(), loss_scale=128.0)
        return raw, squares, gradient


def _packed_query(planes, grid, xy, row):
    n, levels = xy.shape[0], planes.n_levels
    raw = torch.empty((n, row), dtype=torch.float16, device='cuda')
    vis = torch.empty((n, levels), dtype=torch.uint8, device='cuda')
    _lib.check(_lib.library().odie_packed_forward(
        xy.data_ptr(), n, grid.data_ptr(), grid.numel(), planes.descriptors.data_ptr(), levels,
        planes.node_bitmap.data_ptr(), planes.node_prefix.data_ptr(), planes.bitmap.data_ptr(), row, raw.data_ptr(),
        vis.data_ptr(), _lib.stream_of(xy)))
    return raw, vis


def _packed_gradient(planes, xy, up, total):
    gradient = torch.empty(total, dtype=torch.float32, device='cuda')
    _lib.check(_lib.library().odie_packed_backward(
        xy.data_ptr(), xy.shape[0], up.data_ptr(), up.shape[1], planes.descriptors.data_ptr(), planes.n_levels,
        planes.node_bitmap.data_ptr(), planes.node_prefix.data_ptr(), planes.bitmap.data_ptr(), gradient.data_ptr(),
        total, _lib.stream_of(xy)))
    return gradient


def _bits(t):
    return t.detach().cpu().numpy().view(np.uint16 if t.dtype == torch.float16 else np.uint32)


def _hash_model(seed, router, coarse=0, activation='sigmoid', encoding=None):
    encoding = encoding or HASH
    levels, entries = grid_levels(encoding)
    features = int(encoding['n_features_per_level'])
    dims = [features] * int(encoding['n_levels'])
    grid = torch.from_numpy((synth.normal(seed, 'runtime_grid', features * entries) * 0.05).astype(np.float32)).cuda()
    gate = Gate(seed=seed + 1, coarse=coarse, activation=activation, features=dims) if router else None
    return NativeModel(Decoder(seed=seed, width=_width(dims)), gate, grid=grid, active_prefix=len(dims)), levels


@pytest.mark.parametrize('router,coarse,activation,levels,features', [
    (False, 0, 'sigmoid', 16, 2), (True, 2, 'sigmoid', 16, 2), (True, 0, 'softplus', 16, 2),
    (True, 1, 'sigmoid', 8, 2),        # 16 columns
    (True, 0, 'sigmoid', 12, 4),       # 48 columns
    (False, 0, 'sigmoid', 20, 1),      # 20 columns padded to 32, G = 32 gate outputs
])
def test_hash_step_matches_composition(router, coarse, activation, levels, features):
    width, height = 97, 61
    encoding = dict(HASH, n_levels=levels, n_features_per_level=features)
    with torch.cuda.stream(_stream()):
        image = _image(11, width, height)
        config = _config('hash_grid', router, coarse, activation, dims=[features] * levels, encoding=encoding)
        model, grid_levels_ = _hash_model(5, router, coarse, activation, encoding)
        row = _width([features] * levels)
        ref = Composition(model.grid, model.decoder, model.gate, config, width, height, hash_levels=grid_levels_)
        opt = NativeOptimizer(model, image, (height, width), config, [model.grid])
        for step, n in enumerate((3000, 4089, 1, 2048)):
            ids = torch.from_numpy(synth.integers(step, 'runtime_ids', n, width * height)).cuda()
            opt.step_raw(ids)
            raw, squares, _ = ref.step(ids, image)
            torch.cuda.synchronize()
            assert np.array_equal(_bits(opt.copied('raw', (n, row), torch.float16)), _bits(raw)), step
            assert np.array_equal(_bits(opt.copied('squares', (n,), torch.float32)), _bits(squares)), step
            assert np.array_equal(_bits(model.grid), _bits(ref.grid)), step
            assert np.array_equal(_bits(model.decoder.params), _bits(ref.decoder.params)), step
            if router:
                assert np.array_equal(_bits(model.gate.params), _bits(ref.gate.params)), step
        opt.close()


@pytest.mark.parametrize('router,active,half,shape', [(False, 16, True, '16x2'), (True, 16, True, '16x2'),
                                                      (True, 12, True, '16x2'), (False, 9, False, '16x2'),
                                                      (True, 16, True, 'div2k'), (True, 11, True, 'div2k'),
                                                      (True, 8, True, 'L8'), (True, 12, True, 'L12'),
                                                      (True, 20, True, 'L20'), (False, 17, True, 'L20')])
def test_packed_step_matches_composition(router, active, half, shape):
    width, height = 83, 64
    dims = SHAPES[shape]
    with torch.cuda.stream(_stream()):
        image = _image(12, width, height)
        config = _config('xy_planes', router, 1, dims=dims)
        planes = _planes(3, dims)
        planes.set_active_prefix(active)
        row = _width(dims)
        model = NativeModel(Decoder(seed=4, width=row), Gate(seed=6, coarse=1, features=dims) if router else None,
                            planes=planes)
        ref = Composition(model.grid, model.decoder, model.gate, config, width, height, planes=planes, half=half)
        opt, plane_views = make_native_optimizer(model, image, (height, width), config)
        if not half:
            opt.close()
            opt = NativeOptimizer(model, image, (height, width), config, plane_views, half=False)
        for step, n in enumerate((2500, 4096, 7)):
            ids = torch.from_numpy(synth.integers(step + 40, 'runtime_ids', n, width * height)).cuda()
            opt.step_raw(ids)
            gradient = opt.copied('grid_grad', (model.grid.numel(),), torch.float32)
            raw, squares, expected = ref.step(ids, image, active, grid_gradient=gradient)
            torch.cuda.synchronize()
            assert np.array_equal(_bits(opt.copied('raw', (n, row), torch.float16)), _bits(raw)), step
            assert np.array_equal(_bits(opt.copied('squares', (n,), torch.float32)), _bits(squares)), step
            got, want = gradient.double().cpu().numpy(), expected.double().cpu().numpy()
            scale = np.abs(want).max() + 1e-30
            assert np.all(np.abs(got - want) <= 1e-5 * np.abs(want) + 1e-6 * scale), step
            assert np.array_equal(_bits(model.grid), _bits(ref.grid)), step
            assert np.array_equal(_bits(model.decoder.params), _bits(ref.decoder.params)), step
            if router:
                assert np.array_equal(_bits(model.gate.params), _bits(ref.gate.params)), step
        opt.close()


def test_graph_replays_match_eager_steps():
    width, height = 256, 256
    config = _config('hash_grid', True, 2)
    stream = _stream()
    with torch.cuda.stream(stream):
        image = _image(13, width, height)
        graphed, _ = _hash_model(9, True, 2)
        eager, _ = _hash_model(9, True, 2)
        a = NativeOptimizer(graphed, image, (height, width), config, [graphed.grid])
        b = NativeOptimizer(eager, image, (height, width), config, [eager.grid])
        a.prepare_epoch()
        assert a.recaptures == 1 and a.graph is not None
        a.prepare_epoch()                      # same settings: no recapture
        assert a.recaptures == 1
        for step in range(4):
            ids = torch.from_numpy(synth.integers(step, 'graph_ids', 65536, width * height)).cuda()
            loss_a = a.train_batch(ids)
            noise = torch.rand(100000, device='cuda').sum()        # eager work between replays
            b.step_raw(ids)
            squares = b.copied('squares', (65536,), torch.float32)
            torch.cuda.synchronize()
            assert float(noise) > 0
            assert np.array_equal(_bits(a.squares), _bits(squares)), step
            assert float(loss_a) == float(squares.double().mean())
            assert np.array_equal(_bits(graphed.grid), _bits(eager.grid)), step
            assert np.array_equal(_bits(graphed.decoder.params), _bits(eager.decoder.params)), step
            assert np.array_equal(_bits(graphed.gate.params), _bits(eager.gate.params)), step
        assert a.native_state_digest() == b.native_state_digest()
        # a learning-rate change recaptures
        a.param_groups[0]['lr'] = 5e-3
        a.prepare_epoch()
        assert a.recaptures == 2
        a.close()
        b.close()


def test_state_summaries():
    width, height = 64, 64
    with torch.cuda.stream(_stream()):
        image = _image(14, width, height)
        config = _config('xy_planes', False)
        planes = _planes(8)
        model = NativeModel(Decoder(seed=2), None, planes=planes)
        opt, views = make_native_optimizer(model, image, (height, width), config)
        assert all(opt.state.get(view) == {} for view in views)
        assert opt.state.get(torch.zeros(1)) is None
        digest0 = opt.native_state_digest()
        ids = torch.from_numpy(synth.integers(1, 'state_ids', 4096, width * height)).cuda()
        opt.step_raw(ids, update=False)
        assert opt.native_state_digest() == digest0
        assert all(opt.state.get(view) == {} for view in views)
        opt.step_raw(ids)
        assert opt.native_state_digest() != digest0
        assert opt.state.get(views[0]) == {'native_adam_state': True}
        summary = json.loads(opt.native_state_digest())
        assert summary['bytes'] == 12 * (model.grid.numel() + 7168)
        opt.close()


def test_runtime_rejects_invalid_steps():
    width, height = 32, 32
    with torch.cuda.stream(_stream()):
        image = _image(15, width, height)
        config = _config('hash_grid', False)
        model, _ = _hash_model(1, False)
        opt = NativeOptimizer(model, image, (height, width), config, [model.grid])
        with pytest.raises(RuntimeError, match='Invalid native batch size'):
            opt.step_raw(torch.zeros(65537, dtype=torch.int64, device='cuda'))
        with pytest.raises(RuntimeError, match='Invalid active prefix'):
            opt.check(opt.lib.odie_configure(opt.handle, json.dumps(dict(active=1, grid_lr=1.0, decoder_lr=1.0)).encode()))
        with pytest.raises(RuntimeError, match='state range'):
            opt.state_summary(0, model.grid.numel() + 1)
        # ids past the image read its last row instead of memory past it
        opt.step_raw(torch.full((256,), width * height + 5, dtype=torch.int64, device='cuda'), update=False)
        torch.cuda.synchronize()
        assert torch.isfinite(opt.copied('squares', (256,), torch.float32)).all()
        opt.close()
