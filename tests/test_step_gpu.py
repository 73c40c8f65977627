"""One full training step of the packed multi-expert model (odie_amd.trainer.ExpertTrainer)
against the oracle, stage by stage, each stage from the GPU's own output of the previous one:
routing and the encode forward bit-exact; the decoder stage through a re-run with its
hidden activations exported (bit-identical dz) checked as in the decoder tests; the grid
gradient within the encode-backward tolerance; both Adam updates within the Adam tolerance."""
import numpy as np
import pytest
import torch

import oracle
from oracle.bounds import check_gradient, hash_quantum
from odie_amd import synth
from odie_amd.trainer import ExpertTrainer

pytestmark = pytest.mark.gpu

ENCODING = dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=10, base_resolution=4, per_level_scale=1.3)


def rows_of(levels):
    return [(r.scale, r.resolution, r.size, r.offset, r.hashed) for r in levels]


@pytest.mark.parametrize('regions,batch,n,flat', [((2, 2), 4096, 3000, ()), ((3, 2), 2048, 2048, ()),
                                                   ((3, 2), 4096, 4000, (1, 4))])
def test_training_step_matches_oracle(regions, batch, n, flat):
    """flat: tiles painted one colour, left without an expert by allocate_tiles (their ids read
    zero features and train the decoder only)."""
    from odie_amd.experts import allocate_tiles, tile_bounds
    width, height = 96, 70
    image = synth.image(3, width, height)
    xs, ys = tile_bounds(width, regions[0]), tile_bounds(height, regions[1])
    for t in flat:
        image[ys[t // regions[0]]:ys[t // regions[0] + 1], xs[t % regions[0]]:xs[t % regions[0] + 1]] = (40, 90, 7)
    slots, experts = None, None
    if flat:
        from odie_amd.config import grid_levels
        params = 2 * grid_levels(ENCODING)[1]
        slots, experts = allocate_tiles(torch.from_numpy(image), *regions, params, 64 * params)
        assert experts == regions[0] * regions[1] - len(flat)
    trainer = ExpertTrainer(image, ENCODING, *regions, batch, seed=3, fused=False, slots=slots, experts=experts)
    ids_host = synth.integers(3, 'step_ids', n, width * height)
    ids = torch.from_numpy(ids_host).cuda()
    master0 = trainer.master.cpu().numpy().astype(np.float64)
    table0 = trainer.grid.table.cpu().numpy()
    decoder0 = trainer.decoder.params.cpu().numpy().astype(np.float64)
    weights16 = trainer.decoder.half.cpu().numpy()
    squares = trainer.step(ids).cpu().numpy()
    torch.cuda.synchronize()

    # routing and encode forward: bit-exact (ids without an expert last, with zero features)
    _, perm, local, offsets = oracle.route(ids_host, width, height, *regions, slots=slots, experts=experts)
    owned = int(offsets[-1])
    assert (owned < n) == bool(flat)
    assert np.array_equal(trainer.routing.perm[:n].cpu().numpy(), perm)
    assert np.array_equal(trainer.routing.coords[:n].cpu().numpy().view(np.uint32), local.view(np.uint32))
    assert np.array_equal(trainer.routing.offsets.cpu().numpy(), offsets)
    rows = rows_of(trainer.grid.levels)
    raw = np.zeros((n, 32), dtype=np.float16)
    raw[:owned] = oracle.hash_forward(local[:owned], table0, rows, 2, offsets=offsets,
                                      expert_params=trainer.grid.expert_params)
    assert np.array_equal(trainer.raw[:n].cpu().numpy().view(np.uint16), raw.view(np.uint16))

    # decoder: the same launch with hidden activations and outputs exported gives the same dz
    from odie_amd.decoder import Decoder
    probe = Decoder(weights=decoder0.astype(np.float32))
    out = torch.empty((n, 16), dtype=torch.float16, device='cuda')
    hidden = torch.empty((n, 128), dtype=torch.float16, device='cuda')
    again = torch.empty((n,), dtype=torch.float32, device='cuda')
    dz = probe.train(trainer.raw[:n], n, rgb=trainer.rgb, ids=ids, rows=trainer.routing.perm[:n], out=out,
                     hidden=hidden, squares=again).cpu().numpy()
    assert np.array_equal(dz.view(np.uint16), trainer.dz[:n].cpu().numpy().view(np.uint16))
    assert np.array_equal(again.cpu().numpy()[perm], squares)      # the trainer keeps routed order
    h = hidden.cpu().numpy()
    y = out.cpu().numpy()[perm]
    w1, w2, w3 = oracle.mlp_weights(weights16)
    for got, (expected, magnitude) in ((h[:, :64], oracle.mlp_layer(raw, w1, True)),
                                       (h[:, 64:], oracle.mlp_layer(h[:, :64], w2, True)),
                                       (y, oracle.mlp_layer(h[:, 64:], w3, False))):
        assert np.all(np.abs(got.astype(np.float64) - expected) <=
                      2.0 ** -10 * np.abs(expected.astype(np.float64)) + 2.0 ** -16 * magnitude + 2.0 ** -24)
    targets = oracle.mlp_targets(perm, rgb=image.reshape(-1, 3), ids=ids_host)
    dy, ref_squares = oracle.mlp_loss(y, targets, perm, n)
    assert np.array_equal(squares, ref_squares)
    ref_dz, dz_magnitude, ref_dw, dw_magnitude = oracle.mlp_backward(raw, h[:, :64], h[:, 64:], dy, weights16)
    assert np.all(np.abs(dz.astype(np.float64) - ref_dz) <=
                  2.0 ** -10 * np.abs(ref_dz.astype(np.float64)) + 2.0 ** -10 * dz_magnitude + 2.0 ** -24)
    decoder_grad = probe.grad.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(decoder_grad - ref_dw) <= 2.0 ** -9 * dw_magnitude + 1e-6)

    # grid gradient from the GPU's dz (loss scale 128)
    total = trainer.grid.table.numel()
    params = trainer.grid.expert_params
    grad, magnitude, counts = oracle.hash_backward(local[:owned], dz[:owned], rows, 2, total, offsets=offsets,
                                                   expert_params=params, counts=True)
    got = trainer.gradient.cpu().numpy().astype(np.float64)
    check_gradient(got, grad, magnitude, counts, hash_quantum(dz, rows, 2, total, offsets=offsets,
                                                              expert_params=params), 'step')

    # Adam: grid (per-parameter ages, zero gradients skipped, scale 128) and decoder
    # (per-parameter ages, no skip, scale 16384), each from the GPU's gradient
    m, v = np.zeros(total), np.zeros(total)
    steps = np.zeros(total, dtype=np.uint32)
    expected = oracle.adam(1, master0.copy(), got, m, v, steps, 1, 1e-2, scale=128.0)
    master = trainer.master.cpu().numpy().astype(np.float64)
    assert np.allclose(master, expected, rtol=1e-5, atol=1e-7)
    assert np.array_equal(trainer.grid.table.cpu().numpy(), trainer.master.cpu().numpy().astype(np.float16))
    assert np.array_equal(trainer.grid_optimizer.steps.cpu().numpy().astype(np.uint32), steps)
    m, v = np.zeros(decoder0.size), np.zeros(decoder0.size)
    steps = np.zeros(decoder0.size, dtype=np.uint32)
    expected = oracle.adam(2, decoder0.copy(), decoder_grad, m, v, steps, 1, 1e-3, scale=16384.0)
    assert np.allclose(trainer.decoder.params.cpu().numpy(), expected, rtol=1e-5, atol=1e-7)
    assert np.array_equal(trainer.decoder.half.cpu().numpy(), trainer.decoder.params.cpu().numpy().astype(np.float16))


def test_training_reduces_the_loss():
    width, height = 64, 48
    image = synth.image(4, width, height)
    trainer = ExpertTrainer(image, ENCODING, 2, 2, 8192, grid_lr=1e-2, decoder_lr=1e-2, seed=4)
    losses = []
    for step in range(60):
        ids = torch.from_numpy(synth.integers(step, 'train_ids', 8192, width * height)).cuda()
        losses.append(float(trainer.step(ids).double().mean()))
    assert np.isfinite(losses).all()
    assert np.mean(losses[-5:]) < 0.5 * np.mean(losses[:5]), losses[::10]


def test_fused_grid_adam_step_is_bit_identical():
    width, height = 80, 60
    image = synth.image(6, width, height)
    fused = ExpertTrainer(image, ENCODING, 2, 3, 4096, seed=6, fused=True)
    plain = ExpertTrainer(image, ENCODING, 2, 3, 4096, seed=6, fused=False)
    for step in range(3):
        ids = torch.from_numpy(synth.integers(step, 'fused_ids', 4096 - 7 * step, width * height)).cuda()
        a = fused.step(ids).cpu().numpy()
        b = plain.step(ids).cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for name in ('master', 'm', 'v'):
        x = getattr(fused.grid_optimizer, name).cpu().numpy()
        y = getattr(plain.grid_optimizer, name).cpu().numpy()
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), name
    assert np.array_equal(fused.grid_optimizer.steps.cpu().numpy(), plain.grid_optimizer.steps.cpu().numpy())
    assert np.array_equal(fused.grid.table.cpu().numpy().view(np.uint16), plain.grid.table.cpu().numpy().view(np.uint16))
    assert np.array_equal(fused.decoder.params.cpu().numpy(), plain.decoder.params.cpu().numpy())


def test_planes_layout_step_is_bit_identical():
    """The decoder writing the grid's upstream as level-major planes (the default without the
    router) trains exactly as the row-major upstream does."""
    width, height = 96, 70
    image = synth.image(9, width, height)
    planes = ExpertTrainer(image, ENCODING, 3, 2, 5000, seed=9)
    rows = ExpertTrainer(image, ENCODING, 3, 2, 5000, seed=9, planes=False)
    assert planes.planes and not rows.planes
    for step in range(3):
        ids = torch.from_numpy(synth.integers(step, 'planes_ids', 5000 - 11 * step, width * height)).cuda()
        a = planes.step(ids).cpu().numpy()
        b = rows.step(ids).cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for name in ('master', 'm', 'v'):
        x = getattr(planes.grid_optimizer, name).cpu().numpy()
        y = getattr(rows.grid_optimizer, name).cpu().numpy()
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), name
    assert np.array_equal(planes.decoder.params.cpu().numpy(), rows.decoder.params.cpu().numpy())


def test_forward_handoff_step_is_bit_identical():
    """The encode forward filling the backward's handoff (the default with the planes path; here
    its slice masks) trains exactly as the backward forming them itself.  2^15-entry hashed
    levels: each is cut into masked blocks, so the masks are in play."""
    encoding = dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=15, base_resolution=16,
                    per_level_scale=1.38)
    width, height = 256, 200
    image = synth.image(11, width, height)
    batch = 1 << 16
    given = ExpertTrainer(image, encoding, 2, 2, batch, seed=11)
    formed = ExpertTrainer(image, encoding, 2, 2, batch, seed=11, handoff=False)
    assert given.handoff and not formed.handoff
    assert given.grid.handoff_bytes(batch) > 0
    for step in range(3):
        ids = torch.from_numpy(synth.integers(step, 'mask_ids', batch - 13 * step, width * height)).cuda()
        a = given.step(ids).cpu().numpy()
        b = formed.step(ids).cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for name in ('master', 'm', 'v'):
        x = getattr(given.grid_optimizer, name).cpu().numpy()
        y = getattr(formed.grid_optimizer, name).cpu().numpy()
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), name
    assert np.array_equal(given.grid_optimizer.steps.cpu().numpy(), formed.grid_optimizer.steps.cpu().numpy())
    assert np.array_equal(given.grid.table.cpu().numpy().view(np.uint16), formed.grid.table.cpu().numpy().view(np.uint16))
    assert np.array_equal(given.decoder.params.cpu().numpy(), formed.decoder.params.cpu().numpy())


def test_router_step_composes_the_tested_stages():
    from odie_amd.decoder import Decoder
    from odie_amd.gate import Gate
    width, height = 72, 56
    image = synth.image(8, width, height)
    trainer = ExpertTrainer(image, ENCODING, 2, 2, 3000, seed=8, fused=False, router=True, coarse_levels=2)
    gate0 = trainer.gate.params.cpu().numpy()
    decoder0 = trainer.decoder.params.cpu().numpy()
    ids = torch.from_numpy(synth.integers(8, 'router_ids', 3000, width * height)).cuda()
    trainer.step(ids)
    torch.cuda.synchronize()
    gate, decoder = Gate(weights=gate0, coarse=2), Decoder(weights=decoder0)
    raw = trainer.raw[:3000]
    weighted, sigmoid = gate.forward(raw)
    assert np.array_equal(weighted.cpu().numpy().view(np.uint16), trainer.weighted[:3000].cpu().numpy().view(np.uint16))
    dz = decoder.train(weighted, 3000, pixels=trainer.routing.colors[:3000], rgb=trainer.rgb)
    upstream = gate.backward(raw, dz, sigmoid)
    assert np.array_equal(upstream.cpu().numpy().view(np.uint16), trainer.upstream[:3000].cpu().numpy().view(np.uint16))
    gradient = trainer.grid.backward(trainer.routing.coords[:3000], trainer.routing.offsets, upstream)
    assert np.array_equal(gradient.cpu().numpy().view(np.uint32), trainer.gradient.cpu().numpy().view(np.uint32))
    assert np.array_equal(gate.grad.cpu().numpy().view(np.uint32), trainer.gate.grad.cpu().numpy().view(np.uint32))
    # the gate's optimizer ran (per-parameter ages, no skip, scale 16384)
    assert (trainer.gate_optimizer.steps.cpu().numpy() == 1).all()


def test_gigapixel_step_is_deterministic_and_fused_equals_unfused():
    """The 1024-expert configuration at its real size (32x32 tiles of a 32768^2 image, 2^9-entry
    tables, 2^24 ids): two steps of the fused trainer equal two steps of the unfused one bit for
    bit (size-independent property; the oracle covers the same step at small sizes)."""
    from odie_amd import synth as s
    enc = dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=9, base_resolution=16, per_level_scale=1.38)
    side, n = 32768, 1 << 24
    image = s.image_device(1, side, side)
    fused = ExpertTrainer(image, enc, 32, 32, n, seed=1, fused=True)
    plain = ExpertTrainer(image, enc, 32, 32, n, seed=1, fused=False)
    for k in range(2):
        ids = torch.from_numpy(s.integers(k, 'gigapixel_ids', n, side * side)).cuda()
        a = fused.step(ids)
        b = plain.step(ids)
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), k
        assert bool(torch.isfinite(a).all())
    assert torch.equal(fused.master.view(torch.int32), plain.master.view(torch.int32))
    assert torch.equal(fused.decoder.params, plain.decoder.params)
