"""Parity at the benchmarked shapes, against the oracle.

The 64-expert step exactly as bench.py runs it (2048x1365 image of seed 0, 8x8 tile experts,
16 levels x 2 fp16 features, 2^16-entry tables, base 16, scale 1.38; the fused grid Adam with
the decoder writing level-major upstream planes), on 2^18 of the bench's ids, stage by stage,
each stage from the GPU's own output of the previous one:
  route and encode forward bit-exact; the decoder's hidden layers, outputs, loss and dz within
  the decoder bars, with the planes and their 128-row maxima equal to dz bit for bit; the grid
  gradient -- recovered from the first moment the fused update wrote, m = (1 - b1) g / 128 --
  within the encode-backward bar of the oracle's gradient; the grid and decoder Adam updates
  within the Adam bar.
The 1024-expert reconstruction model of the residual + selection pass (2^9-entry tables, base
16, scale 1.38, 32x32 expert tiles) through the fused scoring launch: on a 2048^2 image with
16384 residual cells, every pixel's features bit-exact and its prediction within the decoder
bars, the fp64 totals bit-exact and the top 512 cells equal to the oracle's; and at the full
32768^2 image with 256^2 residual tiles, the top 512 of all 16384 totals equal the oracle's
ranking and eight sampled tiles' totals and predictions match the oracle."""
import numpy as np
import pytest
import torch

import bench
import oracle
from oracle.bounds import gradient_bound, hash_quantum
from odie_amd import synth
from odie_amd.decoder import Decoder
from odie_amd.experts import ExpertGrid
from odie_amd.reconstruction import reconstruct, score_image
from odie_amd.selection import topk_tiles
from odie_amd.trainer import ExpertTrainer

pytestmark = pytest.mark.gpu
THREADS = 16


def rows_of(levels):
    return [(r.scale, r.resolution, r.size, r.offset, r.hashed) for r in levels]


def layer_bound(expected, magnitude):
    """fp16 rounding of the output (2^-10 relative) plus fp32 accumulation order (2^-16 of the
    magnitude sum), the decoder tests' per-layer bar."""
    return 2.0 ** -10 * np.abs(expected.astype(np.float64)) + 2.0 ** -16 * magnitude + 2.0 ** -24


def test_headline_step_matches_oracle():
    n = 1 << 18
    width, height, regions = bench.WIDTH, bench.HEIGHT, bench.REGIONS
    print('headline step: %dx%d, %dx%d experts, %d of the bench ids' % (width, height, regions, regions, n),
          flush=True)
    image = synth.image(0, width, height)
    trainer = ExpertTrainer(image, bench.ENCODING, regions, regions, n, grid_lr=1e-2, decoder_lr=1e-3, seed=0)
    assert trainer.fused and trainer.planes            # the bench's path
    ids_host = synth.integers(0, 'ids', bench.N_COORDS, width * height)[:n]
    ids = torch.from_numpy(ids_host).cuda()
    master0 = trainer.master.cpu().numpy().astype(np.float64)
    table0 = trainer.grid.table.cpu().numpy()
    decoder0 = trainer.decoder.params.cpu().numpy()
    weights16 = trainer.decoder.half.cpu().numpy()
    squares = trainer.step(ids).cpu().numpy()
    torch.cuda.synchronize()

    # route: expert order, local coordinates, offsets and each slot's pixel index
    _, perm, local, offsets = oracle.route(ids_host, width, height, regions, regions)
    assert np.array_equal(trainer.routing.perm[:n].cpu().numpy(), perm)
    assert np.array_equal(trainer.routing.coords[:n].cpu().numpy().view(np.uint32), local.view(np.uint32))
    assert np.array_equal(trainer.routing.offsets.cpu().numpy(), offsets)
    assert np.array_equal(trainer.routing.colors[:n].cpu().numpy(), ids_host[perm])

    # encode forward
    rows, params = rows_of(trainer.grid.levels), trainer.grid.expert_params
    raw = oracle.hash_forward(local, table0, rows, 2, offsets=offsets, expert_params=params, threads=THREADS)
    assert np.array_equal(trainer.raw[:n].cpu().numpy().view(np.uint16), raw.view(np.uint16))

    # decoder: the same launch with its hidden layers exported (row-major dz) equals the planes
    probe = Decoder(weights=decoder0)
    out = torch.empty((n, 16), dtype=torch.float16, device='cuda')
    hidden = torch.empty((n, 128), dtype=torch.float16, device='cuda')
    again = torch.empty(n, dtype=torch.float32, device='cuda')
    dz = probe.train(trainer.raw[:n], n, pixels=trainer.routing.colors[:n], rgb=trainer.rgb, out=out, hidden=hidden,
                     squares=again).cpu().numpy()
    planes = trainer.plane_buffer[:16 * n].view(16, n).cpu().numpy().view(np.uint32)
    assert np.array_equal(planes, np.ascontiguousarray(dz).view(np.uint32).T)
    peaks = np.abs(dz.astype(np.float32)).reshape(-1, 128, 32).max(axis=1)
    assert np.array_equal(trainer.max_buffer[:32 * (n // 128)].view(-1, 32).cpu().numpy(), peaks)
    assert np.array_equal(again.cpu().numpy(), squares)
    h, y = hidden.cpu().numpy(), out.cpu().numpy()
    w1, w2, w3 = oracle.mlp_weights(weights16)
    for got, (expected, magnitude) in ((h[:, :64], oracle.mlp_layer(raw, w1, True)),
                                       (h[:, 64:], oracle.mlp_layer(h[:, :64], w2, True)),
                                       (y, oracle.mlp_layer(h[:, 64:], w3, False))):
        assert np.all(np.abs(got.astype(np.float64) - expected) <= layer_bound(expected, magnitude))
    slots = np.arange(n)
    targets = oracle.mlp_targets(slots, rgb=image.reshape(-1, 3), ids=ids_host[perm])
    dy, ref_squares = oracle.mlp_loss(y, targets, slots, n)
    assert np.array_equal(squares, ref_squares)
    ref_dz, dz_magnitude, ref_dw, dw_magnitude = oracle.mlp_backward(raw, h[:, :64], h[:, 64:], dy, weights16)
    assert np.all(np.abs(dz.astype(np.float64) - ref_dz) <=
                  2.0 ** -10 * np.abs(ref_dz.astype(np.float64)) + 2.0 ** -10 * dz_magnitude + 2.0 ** -24)
    decoder_grad = probe.grad.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(decoder_grad - ref_dw) <= 2.0 ** -9 * dw_magnitude + 1e-6)

    # grid: the fused update's first moment is m = (1 - b1) * g / 128 (fp32), so it gives back the
    # gradient the backward formed; checked against the oracle's gradient of the GPU's dz
    total = trainer.grid.table.numel()
    grad, magnitude, counts = oracle.hash_backward(local, dz, rows, 2, total, offsets=offsets, expert_params=params,
                                                   counts=True)
    own = gradient_bound(magnitude, counts, hash_quantum(dz, rows, 2, total, offsets=offsets, expert_params=params))
    del counts
    m = trainer.grid_optimizer.m.cpu().numpy().astype(np.float64)
    one_minus_b1 = float(np.float32(1.0) - np.float32(0.9))
    recovered = m / one_minus_b1 * 128.0
    bound = own + 2.0 ** -22 * np.abs(recovered)   # plus the rounding of m = (1 - b1) g / 128 in fp32
    bad = np.abs(recovered - grad) > bound
    assert not bad.any(), '%d/%d gradient entries out of tolerance' % (bad.sum(), bad.size)
    touched = np.abs(grad) > own
    ages = trainer.grid_optimizer.steps.cpu().numpy().astype(np.uint32)
    assert (ages[touched] == 1).all() and (ages[magnitude == 0] == 0).all()
    mm, vv = np.zeros(total), np.zeros(total)
    steps = np.zeros(total, dtype=np.uint32)
    expected = oracle.adam(1, master0.copy(), recovered, mm, vv, steps, 1, 1e-2, scale=128.0)
    assert np.array_equal(ages, steps)
    master = trainer.master.cpu().numpy()
    assert np.allclose(master.astype(np.float64), expected, rtol=1e-5, atol=1e-7)
    assert np.array_equal(trainer.grid.table.cpu().numpy(), master.astype(np.float16))
    del grad, magnitude, own, m, recovered, bound, mm, vv, expected, master

    # decoder Adam (per-parameter ages, no skip, loss scale 16384)
    mm, vv = np.zeros(decoder0.size), np.zeros(decoder0.size)
    steps = np.zeros(decoder0.size, dtype=np.uint32)
    expected = oracle.adam(2, decoder0.astype(np.float64), decoder_grad, mm, vv, steps, 1, 1e-3, scale=16384.0)
    assert np.allclose(trainer.decoder.params.cpu().numpy(), expected, rtol=1e-5, atol=1e-7)


def _c5_model():
    grid = ExpertGrid(bench.C5_ENCODING, bench.C5_TILES * bench.C5_TILES)
    table = synth.table(1, grid.table.numel(), -1.0, 1.0, name='c5_table').astype(np.float16)
    grid.table.copy_(torch.from_numpy(table))
    return grid, table, Decoder(seed=1)


def _check_prediction(features16, prediction, raw16, weights16):
    """features bit-exact; prediction = the decoder's first three outputs within the per-layer
    bars carried through the layers (each layer's error bound passed on through |W|)."""
    assert np.array_equal(features16.view(np.uint16), raw16.view(np.uint16))
    w1, w2, w3 = oracle.mlp_weights(weights16)
    h1, m1 = oracle.mlp_layer(raw16, w1, True)
    e1 = layer_bound(h1, m1)
    h2, m2 = oracle.mlp_layer(h1, w2, True)
    e2 = layer_bound(h2, m2) + e1 @ np.abs(w2.astype(np.float64)).T
    y, m3 = oracle.mlp_layer(h2, w3, False)
    e3 = layer_bound(y, m3) + e2 @ np.abs(w3.astype(np.float64)).T
    assert np.all(np.abs(prediction.astype(np.float64) - y[:, :3]) <= e3[:, :3])


def test_c5_model_on_a_downsized_image_matches_oracle():
    side, cell = 2048, 16                      # 128 x 128 = 16384 residual cells, as at full size
    tiles, top = bench.C5_TILES, bench.C5_TOP
    print('c5 model: %d^2 image, %dx%d experts, %d^2 residual cells' % (side, tiles, tiles, cell), flush=True)
    grid, table, decoder = _c5_model()
    image = synth.image(1, side, side).reshape(-1, 3)
    target = torch.from_numpy(image).cuda()
    n = side * side
    image_out = torch.full((n, 3), float('nan'), dtype=torch.float32, device='cuda')
    metrics, scores = score_image(grid, decoder.half, target, (side, side), (tiles, tiles), tile=cell, fused=True,
                                  prediction=image_out)
    assert scores.resolution ** 2 == 16384
    features = torch.empty((n, 32), dtype=torch.float16, device='cuda')
    reconstruct(grid, decoder.half, (side, side), (tiles, tiles), 0, n, features=features)
    prediction = image_out.cpu().numpy()
    _, perm, local, offsets = oracle.route(np.arange(n), side, side, tiles, tiles)
    raw = oracle.hash_forward(local, table, rows_of(grid.levels), 2, offsets=offsets,
                              expert_params=grid.expert_params, threads=THREADS)
    raster = np.empty_like(raw)
    raster[perm] = raw
    _check_prediction(features.cpu().numpy(), prediction, raster, decoder.half.cpu().numpy())
    expected = oracle.residual(prediction, image, side, scores.resolution, scores.xb.cpu().numpy(),
                               scores.yb.cpu().numpy())
    assert np.array_equal(scores.totals.cpu().numpy().view(np.uint64), expected.view(np.uint64))
    means = expected / scores.counts
    ids = topk_tiles(scores.totals / torch.from_numpy(scores.counts).cuda(), top).cpu().numpy()
    assert np.array_equal(ids, oracle.topk_ids(means, top))
    assert np.isfinite(metrics['mse'])


def test_c5_full_size_selection_and_sampled_tiles_match_oracle():
    side, cell = bench.C5_SIDE, bench.C5_RESIDUAL_TILE
    tiles, top = bench.C5_TILES, bench.C5_TOP
    print('c5 full size: %d^2 image, %d^2 residual tiles, top %d' % (side, cell, top), flush=True)
    grid, table, decoder = _c5_model()
    target = synth.image_device(1, side, side).reshape(-1, 3)
    metrics, scores = score_image(grid, decoder.half, target, (side, side), (tiles, tiles), tile=cell, fused=True)
    totals = scores.totals.cpu().numpy()
    ids = topk_tiles(scores.totals / torch.from_numpy(scores.counts).cuda(), top).cpu().numpy()
    assert np.array_equal(ids, oracle.topk_ids(totals / scores.counts, top))
    resolution = scores.resolution
    xb, yb = scores.xb.cpu().numpy(), scores.yb.cpu().numpy()
    weights16 = decoder.half.cpu().numpy()
    rng = np.random.default_rng(5)
    sample = np.concatenate([[0, resolution * resolution - 1], ids[:2], rng.integers(0, resolution ** 2, 4)])
    for c in sample.tolist():
        cx, cy = c % resolution, c // resolution
        y0, y1, x0, x1 = int(yb[cy]), int(yb[cy + 1]), int(xb[cx]), int(xb[cx + 1])
        begin, count = y0 * side, (y1 - y0) * side
        print('  tile %d: rows %d..%d, columns %d..%d' % (c, y0, y1, x0, x1), flush=True)
        features = torch.empty((count, 32), dtype=torch.float16, device='cuda')
        rows_prediction = torch.empty((count, 3), dtype=torch.float32, device='cuda')
        reconstruct(grid, decoder.half, (side, side), (tiles, tiles), begin, count, prediction=rows_prediction,
                    features=features)
        truth = target[begin:begin + count].cpu().numpy()
        fold = oracle.residual(rows_prediction.cpu().numpy(), truth, side, resolution, xb, yb, begin=begin)
        assert fold[c] == totals[c], c
        # the tile's own pixels against the oracle's encode and decoder
        inside = (slice(None), slice(x0, x1))
        tile_features = features.view(y1 - y0, side, 32)[inside].reshape(-1, 32).cpu().numpy()
        tile_prediction = rows_prediction.view(y1 - y0, side, 3)[inside].reshape(-1, 3).cpu().numpy()
        del features, rows_prediction
        px = (np.arange(y0, y1)[:, None] * side + np.arange(x0, x1)[None, :]).ravel()
        _, perm, local, offsets = oracle.route(px, side, side, tiles, tiles)
        raw = oracle.hash_forward(local, table, rows_of(grid.levels), 2, offsets=offsets,
                                  expert_params=grid.expert_params, threads=THREADS)
        raster = np.empty_like(raw)
        raster[perm] = raw
        _check_prediction(tile_features, tile_prediction, raster, weights16)
    assert np.isfinite(metrics['mse'])
