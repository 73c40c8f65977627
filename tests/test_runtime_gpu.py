"""The native step runtime (odie_create / odie_step / odie_configure / odie_state ..., the
reference's Probe at odie/native/runtime.cu:163-331) against the composition of the separately
tested entry points on the same inputs: the hash-grid step bit for bit (its backward and Adam are
deterministic), the packed-plane step with the grid gradient within the encode-backward
tolerance (fp32 atomics) and every update bit for bit from that gradient; a captured graph
replayed with eager work between replays, bit for bit against eager steps; the optimizer-state
summaries; and one packed-plane step at the reference's level rows against the oracle, stage by
stage.  Gradients reach the optimizers through fp16 stores as in the reference: the grid's
fp16(g) at loss scale 128, the heads' fp16(fp16(g) / 128) at 128 (odie/native/runtime.cu:
298-309, kernels.cuh:140-143)."""
import json

import numpy as np
import pytest
import torch

import oracle
from oracle.bounds import check_gradient, hash_quantum, packed_quantum
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
          'L20': [2] * 19 + [1], '12x2': [2] * 12}


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
                                                      (True, 20, True, 'L20'), (False, 17, True, 'L20'),
                                                      (True, 12, True, '12x2'), (True, 9, True, '12x2')])
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



def _layer_bound(expected, magnitude):
    """fp16 rounding of a layer's output (2^-10 relative) plus fp32 accumulation order (2^-16 of
    its magnitude sum)."""
    return 2.0 ** -10 * np.abs(expected.astype(np.float64)) + 2.0 ** -16 * magnitude + 2.0 ** -24


def _heads_match_oracle(raw, visible, dims, coarse, gate0, decoder0, image, ids, got):
    """The gate and decoder stages of one runtime step against the oracle, from the runtime's
    features `raw` (fp16 [n, row] on the GPU): the gate's s (from the same launch run again on raw)
    within fp16-logit rounding and the gated features bit-exact given s; the decoder launch run
    again with its hidden layers exported reproduces the runtime's outputs and squares bit for bit,
    its layers within the per-layer bars, squares bit-exact, dz and the decoder gradient within
    the decoder bars; the gate's upstream and gradient within the gate bars.  `got` holds the
    runtime's output, squares, decoder_grad and gate_grad.  Returns the upstream (fp16 [n, row])
    the grid gradient is formed from."""
    n, levels = raw.shape[0], len(dims)
    raw_host, ids_host = raw.cpu().numpy(), ids.cpu().numpy()
    inputs = raw
    if gate0 is not None:
        gate16 = gate0.astype(np.float16)
        probe = Gate(weights=gate0, coarse=coarse, features=dims)
        vis = None if visible is None else torch.from_numpy(visible.astype(np.uint8)).cuda()
        weighted, s = probe.forward(raw, visible=vis)
        s_host = s.cpu().numpy()
        h_gate, z, _ = oracle.gate_logits(raw_host, gate16, levels)
        ref_s, z = oracle.gate_values(z, coarse)[:, :levels], z[:, :levels].astype(np.float64)
        assert np.all(np.abs(s_host - ref_s) <= ref_s * (1 - ref_s) * 2.0 ** -9 * (np.abs(z) + 1) + 2.0 ** -22)
        assert np.array_equal(weighted.cpu().numpy().view(np.uint16),
                              oracle.gate_apply(raw_host, s_host, visible, dims).view(np.uint16))
        inputs = weighted

    decoder16 = decoder0.astype(np.float16)
    out = torch.empty((n, 16), dtype=torch.float16, device='cuda')
    hidden = torch.empty((n, 128), dtype=torch.float16, device='cuda')
    again = torch.empty(n, dtype=torch.float32, device='cuda')
    dz = Decoder(weights=decoder0, width=raw.shape[1]).train(inputs, rgb=image.reshape(-1), ids=ids, out=out,
                                                             hidden=hidden, squares=again)
    x16, h, dz, output = inputs.cpu().numpy(), hidden.cpu().numpy(), dz.cpu().numpy(), got['output']
    assert np.array_equal(out.cpu().numpy().view(np.uint16), output.view(np.uint16))
    assert np.array_equal(again.cpu().numpy(), got['squares'])
    w1, w2, w3 = oracle.mlp_weights(decoder16)
    for value, (want, magnitude) in ((h[:, :64], oracle.mlp_layer(x16, w1, True)),
                                     (h[:, 64:], oracle.mlp_layer(h[:, :64], w2, True)),
                                     (output, oracle.mlp_layer(h[:, 64:], w3, False))):
        assert np.all(np.abs(value.astype(np.float64) - want) <= _layer_bound(want, magnitude))
    slots = np.arange(n)
    targets = oracle.mlp_targets(slots, rgb=image.cpu().numpy().reshape(-1, 3), ids=ids_host)
    dy, ref_squares = oracle.mlp_loss(output, targets, slots, n)
    assert np.array_equal(got['squares'], ref_squares)
    ref_dz, dz_magnitude, ref_dw, dw_magnitude = oracle.mlp_backward(x16, h[:, :64], h[:, 64:], dy, decoder16)
    assert np.all(np.abs(dz.astype(np.float64) - ref_dz) <=
                  2.0 ** -10 * np.abs(ref_dz.astype(np.float64)) + 2.0 ** -10 * dz_magnitude + 2.0 ** -24)
    assert np.all(np.abs(got['decoder_grad'].astype(np.float64) - ref_dw) <= 2.0 ** -9 * dw_magnitude + 1e-6)
    if gate0 is None:
        return dz
    upstream = probe.backward(raw, torch.from_numpy(dz).cuda(), s, visible=vis).cpu().numpy()
    direct, da = oracle.gate_back(raw_host, dz, s_host, coarse, visible=visible, features=dims)
    dr, dr_magnitude, dweights, magnitude = oracle.gate_mlp_backward(raw_host, h_gate, da, gate16, levels)
    want = oracle.gate_upstream(direct, dr).astype(np.float64)
    assert np.all(np.abs(upstream.astype(np.float64) - want) <=
                  2.0 ** -10 * np.abs(want) + 2.0 ** -10 * dr_magnitude / 128 + 2.0 ** -24)
    assert np.all(np.abs(got['gate_grad'].astype(np.float64) - dweights) <= 2.0 ** -9 * magnitude + 1e-6)
    return upstream


def _fetch(opt, n, row, model):
    """The runtime's buffers after a step, on the host."""
    got = dict(output=opt.copied('output', (n, 16), torch.float16),
               squares=opt.copied('squares', (n,), torch.float32),
               grid_grad=opt.copied('grid_grad', (model.grid.numel(),), torch.float32),
               decoder_grad=opt.copied('decoder_grad', (model.decoder.params.numel(),), torch.float32))
    if model.gate is not None:
        got['gate_grad'] = opt.copied('gate_grad', (model.gate.params.numel(),), torch.float32)
    raw = opt.copied('raw', (n, row), torch.float16)
    torch.cuda.synchronize()
    return raw, {k: v.cpu().numpy() for k, v in got.items()}


def _coordinates(ids_host, width, height):
    """The pixel centres' unit coordinates of odie/native/runtime.cu:34-36, in fp32."""
    rx, ry = np.float32(1.0 / (width - 1)), np.float32(1.0 / (height - 1))
    return np.stack([(ids_host % width).astype(np.float32) * rx, (ids_host // width).astype(np.float32) * ry], 1)


def _check_gradient(grid_grad, grad, magnitude, counts, quantum):
    """fp32 atomics or fixed point: order and each entry's quantum only."""
    check_gradient(grid_grad, grad, magnitude, counts, quantum, 'runtime grid gradient')


@pytest.mark.parametrize('shape,router,active', [('div2k', True, 16), ('L20', True, 13), ('16x2', False, 11)])
def test_packed_step_matches_oracle(shape, router, active):
    """One odie_step of the packed-plane runtime at the reference's level rows against the oracle,
    stage by stage, each stage from the runtime's own output of the previous one: the features
    bit-exact (levels past the active prefix zero, padding columns one); the heads as
    _heads_match_oracle checks them; the grid gradient within the encode-backward bar of the
    oracle's gradient of the runtime's upstream; the three Adam updates from the runtime's fp16
    gradients (grid: fp16(g) at loss scale 128; heads: fp16(fp16(g) / 128) at 128) within the
    Adam bar."""
    width, height, n, coarse = 83, 64, 3000, 1
    dims = SHAPES[shape]
    row, columns = _width(dims), sum(dims)
    print('packed runtime step vs oracle: %s, router %s, active %d' % (shape, router, active), flush=True)
    with torch.cuda.stream(_stream()):
        image = _image(16, width, height)
        config = _config('xy_planes', router, coarse, dims=dims)
        planes = _planes(5, dims)
        planes.set_active_prefix(active)
        model = NativeModel(Decoder(seed=7, width=row),
                            Gate(seed=8, coarse=coarse, features=dims) if router else None, planes=planes)
        opt, _ = make_native_optimizer(model, image, (height, width), config)
        grid0 = model.grid.cpu().numpy()
        decoder0 = model.decoder.params.cpu().numpy()
        gate0 = model.gate.params.cpu().numpy() if router else None
        ids_host = synth.integers(60, 'runtime_ids', n, width * height)
        ids = torch.from_numpy(ids_host).cuda()
        opt.step_raw(ids)
        raw, got = _fetch(opt, n, row, model)

        xy = _coordinates(ids_host, width, height)
        layout = {k: getattr(planes, k).cpu().numpy() for k in ('descriptors', 'node_bitmap', 'node_prefix', 'bitmap')}
        expected, visible = oracle.packed_forward(xy, grid0, layout, row)
        expected[:, sum(dims[:active]):] = 0
        expected[:, columns:] = 1.0
        visible[:, active:] = False
        assert np.array_equal(raw.cpu().numpy().view(np.uint16), expected.view(np.uint16))
        up = _heads_match_oracle(raw, visible, dims, coarse, gate0, decoder0, image, ids, got)
        _check_gradient(got['grid_grad'], *oracle.packed_backward(xy, up, layout, grid0.size, counts=True),
                        packed_quantum(up, layout, grid0.size))

        def adam(variant, start, gradient, lr):
            m, v = np.zeros(start.size), np.zeros(start.size)
            steps = np.zeros(start.size, dtype=np.uint32)
            return oracle.adam(variant, start.astype(np.float64), gradient, m, v, steps, 1, lr, scale=128.0)

        def head_gradient(g):
            return (g.astype(np.float16).astype(np.float32) / np.float32(128.0)).astype(np.float16).astype(np.float64)

        updates = [(model.grid, adam(1, grid0, got['grid_grad'].astype(np.float16).astype(np.float64), 1e-2)),
                   (model.decoder.params, adam(2, decoder0, head_gradient(got['decoder_grad']), 1e-3))]
        if router:
            updates.append((model.gate.params, adam(2, gate0, head_gradient(got['gate_grad']), 2e-3)))
        for params, want in updates:
            assert np.allclose(params.cpu().numpy().astype(np.float64), want, rtol=1e-5, atol=1e-7)
        opt.close()


@pytest.mark.parametrize('router,coarse,levels,features', [(True, 2, 16, 2), (False, 0, 20, 1), (True, 0, 12, 4)])
def test_hash_step_matches_oracle(router, coarse, levels, features):
    """One odie_step of the hash-grid runtime without the update (which writes the grid gradient
    out instead of fusing it into Adam) against the oracle: the features of the fp16 table
    bit-exact with padding columns one, the heads as _heads_match_oracle checks them, and the grid
    gradient within the encode-backward bar of the oracle's gradient of the runtime's upstream;
    no parameter moves."""
    width, height, n = 97, 61, 3000
    encoding = dict(HASH, n_levels=levels, n_features_per_level=features)
    dims = [features] * levels
    row = _width(dims)
    print('hash runtime step vs oracle: %d x F%d, router %s' % (levels, features, router), flush=True)
    with torch.cuda.stream(_stream()):
        image = _image(17, width, height)
        config = _config('hash_grid', router, coarse, dims=dims, encoding=encoding)
        model, hash_levels = _hash_model(6, router, coarse, encoding=encoding)
        opt = NativeOptimizer(model, image, (height, width), config, [model.grid])
        grid0 = model.grid.cpu().numpy()
        decoder0 = model.decoder.params.cpu().numpy()
        gate0 = model.gate.params.cpu().numpy() if router else None
        ids_host = synth.integers(61, 'runtime_ids', n, width * height)
        ids = torch.from_numpy(ids_host).cuda()
        opt.step_raw(ids, update=False)
        raw, got = _fetch(opt, n, row, model)

        xy = _coordinates(ids_host, width, height)
        rows = [(r.scale, r.resolution, r.size, r.offset, r.hashed) for r in hash_levels]
        expected = oracle.hash_forward(xy, grid0.astype(np.float16), rows, features, expert_params=grid0.size,
                                       width=row)
        expected[:, levels * features:] = 1.0
        assert np.array_equal(raw.cpu().numpy().view(np.uint16), expected.view(np.uint16))
        up = _heads_match_oracle(raw, None, dims, coarse, gate0, decoder0, image, ids, got)
        _check_gradient(got['grid_grad'], *oracle.hash_backward(xy, up, rows, features, grid0.size,
                                                                expert_params=grid0.size, counts=True),
                        hash_quantum(up, rows, features, grid0.size))
        assert np.array_equal(_bits(model.grid), grid0.view(np.uint32))
        assert np.array_equal(_bits(model.decoder.params), decoder0.view(np.uint32))
        opt.close()
