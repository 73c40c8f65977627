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


def _config(representation, router, coarse=0, activation='sigmoid'):
    return dict(representation=representation, hash_encoding=HASH, n_levels=16, plane_feature_dimensions=[2] * 16,
                router_enabled=router, target_storage='uint8', gate_coarse_levels_K=coarse,
                router_output_activation=activation, grid_lr=1e-2, gate_lr=2e-3, decoder_lr=1e-3)


def _stream():
    return torch.cuda.Stream()


def _image(seed, width, height):
    return torch.from_numpy(synth.image(seed, width, height)).cuda().contiguous()


def _planes(seed):
    supports, caps = [], []
    for level, r in enumerate(RESOLUTIONS):
        if level < 8:
            supports.append(torch.ones(r * r, dtype=torch.bool))
        else:
            supports.append(torch.from_numpy(synth.uniform(seed + level, 'runtime_support', r * r) < 0.35))
        caps.append((r * r + 7) // 8 * 8)
    config = dict(resolutions=RESOLUTIONS, n_levels=16, representation='xy_planes', coarse_levels=0,
                  gate_topology='shared', gate_position='feature', initial_active_prefix=8, seed=seed,
                  feature_init_std=5e-2)
    planes = PackedPlanes(config, supports, [2] * 16, caps)
    planes.set_active_prefix(16)
    return planes


class Composition:
    """The step from the tested entry points, with its own copies of every weight."""

    def __init__(self, grid, decoder, gate, config, width, height, hash_levels=None, planes=None, half=True):
        self.grid = grid.clone()
        self.decoder = Decoder(weights=decoder.params.cpu().numpy())
        self.gate = None if gate is None else Gate(weights=gate.params.cpu().numpy(), coarse=gate.coarse,
                                                   activation='softplus' if gate.softplus else 'sigmoid')
        self.levels, self.planes, self.half = hash_levels, planes, half
        self.table = self.grid.half() if hash_levels is not None else None
        self.grid_opt = FusedAdam(self.grid, config['grid_lr'], eps=1e-15, variant='tcnn', half_copy=self.table)
        self.dec_opt = FusedAdam(self.decoder.params, config['decoder_lr'], eps=1e-15, variant='tcnn_dense',
                                 half_copy=self.decoder.half)
        self.gate_opt = None if gate is None else FusedAdam(self.gate.params, config['gate_lr'], eps=1e-15,
                                                            variant='tcnn_dense', half_copy=self.gate.half)
        self.width, self.height = width, height

    def forward(self, ids, active=16):
        w = self.width
        rx = torch.tensor(np.float32(1.0 / (w - 1)), device='cuda')
        ry = torch.tensor(np.float32(1.0 / (self.height - 1)), device='cuda')
        xy = torch.stack([(ids % w).float() * rx, (ids // w).float() * ry], dim=1).contiguous()
        if self.levels is not None:
            raw = grid_forward(xy, self.table, self.levels, 2, width=32)
            vis = None
        else:
            raw, vis = _packed_query(self.planes, self.grid, xy)
            raw[:, 2 * active:] = 0
            vis[:, active:] = 0
        return xy, raw, vis

    def step(self, ids, image, active=16, grid_gradient=None, update=True):
        xy, raw, vis = self.forward(ids, active)
        squares = torch.empty(ids.numel(), dtype=torch.float32, device='cuda')
        features, sigmoid = raw, None
        if self.gate is not None:
            features, sigmoid = self.gate.forward(raw, visible=vis)
        dz = self.decoder.train(features, rgb=image.reshape(-1), ids=ids, squares=squares)
        up = dz if self.gate is None else self.gate.backward(raw, dz, sigmoid, visible=vis)
        if self.levels is not None:
            gradient = grid_backward(xy, up, self.levels, 2, expert_params=self.grid.numel())
        else:
            gradient = _packed_gradient(self.planes, xy, up, self.grid.numel())
        if update:
            used = gradient if grid_gradient is None else grid_gradient
            self.grid_opt.step(used.half() if self.half else used, loss_scale=128.0)
            for head, opt in ((self.gate, self.gate_opt), (self.decoder, self.dec_opt)):
                if head is not None:
                    opt.step((head.grad.half().float() / 128.0).half(), loss_scale=128.0)
        return raw, squares, gradient


def _packed_query(planes, grid, xy):
    n = xy.shape[0]
    raw = torch.empty((n, 32), dtype=torch.float16, device='cuda')
    vis = torch.empty((n, 16), dtype=torch.uint8, device='cuda')
    _lib.check(_lib.library().odie_packed_forward(
        xy.data_ptr(), n, grid.data_ptr(), grid.numel(), planes.descriptors.data_ptr(), 16,
        planes.node_bitmap.data_ptr(), planes.node_prefix.data_ptr(), planes.bitmap.data_ptr(), 32, raw.data_ptr(),
        vis.data_ptr(), _lib.stream_of(xy)))
    return raw, vis


def _packed_gradient(planes, xy, up, total):
    gradient = torch.empty(total, dtype=torch.float32, device='cuda')
    _lib.check(_lib.library().odie_packed_backward(
        xy.data_ptr(), xy.shape[0], up.data_ptr(), 32, planes.descriptors.data_ptr(), 16,
        planes.node_bitmap.data_ptr(), planes.node_prefix.data_ptr(), planes.bitmap.data_ptr(), gradient.data_ptr(),
        total, _lib.stream_of(xy)))
    return gradient


def _bits(t):
    return t.detach().cpu().numpy().view(np.uint16 if t.dtype == torch.float16 else np.uint32)


def _hash_model(seed, router, coarse=0, activation='sigmoid'):
    levels, entries = grid_levels(HASH)
    grid = torch.from_numpy((synth.normal(seed, 'runtime_grid', 2 * entries) * 0.05).astype(np.float32)).cuda()
    gate = Gate(seed=seed + 1, coarse=coarse, activation=activation) if router else None
    return NativeModel(Decoder(seed=seed), gate, grid=grid), levels


@pytest.mark.parametrize('router,coarse,activation', [(False, 0, 'sigmoid'), (True, 2, 'sigmoid'),
                                                       (True, 0, 'softplus')])
def test_hash_step_matches_composition(router, coarse, activation):
    width, height = 97, 61
    with torch.cuda.stream(_stream()):
        image = _image(11, width, height)
        config = _config('hash_grid', router, coarse, activation)
        model, levels = _hash_model(5, router, coarse, activation)
        ref = Composition(model.grid, model.decoder, model.gate, config, width, height, hash_levels=levels)
        opt = NativeOptimizer(model, image, (height, width), config, [model.grid])
        for step, n in enumerate((3000, 4089, 1, 2048)):
            ids = torch.from_numpy(synth.integers(step, 'runtime_ids', n, width * height)).cuda()
            opt.step_raw(ids)
            raw, squares, _ = ref.step(ids, image)
            torch.cuda.synchronize()
            assert np.array_equal(_bits(opt.copied('raw', (n, 32), torch.float16)), _bits(raw)), step
            assert np.array_equal(_bits(opt.copied('squares', (n,), torch.float32)), _bits(squares)), step
            assert np.array_equal(_bits(model.grid), _bits(ref.grid)), step
            assert np.array_equal(_bits(model.decoder.params), _bits(ref.decoder.params)), step
            if router:
                assert np.array_equal(_bits(model.gate.params), _bits(ref.gate.params)), step
        opt.close()


@pytest.mark.parametrize('router,active,half', [(False, 16, True), (True, 16, True), (True, 12, True),
                                                (False, 9, False)])
def test_packed_step_matches_composition(router, active, half):
    width, height = 83, 64
    with torch.cuda.stream(_stream()):
        image = _image(12, width, height)
        config = _config('xy_planes', router, 1)
        planes = _planes(3)
        planes.set_active_prefix(active)
        model = NativeModel(Decoder(seed=4), Gate(seed=6, coarse=1) if router else None, planes=planes)
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
            assert np.array_equal(_bits(opt.copied('raw', (n, 32), torch.float16)), _bits(raw)), step
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
