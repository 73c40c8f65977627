"""Fused reconstruction (odie_reconstruct) against the composition of the tested entry points:
route the raster ids, encode the compacted coordinates (odie_grid_forward), run the decoder
(odie_mlp_forward) and put the rows back in raster order -- features, decoder outputs and
predictions bit for bit, over ragged ranges and with tiles that have no expert.  Then the
scoring pipeline (score_image): per-cell totals bit-exact against the oracle's residual of the
fused predictions, the top tiles against the oracle's ranking, the mse against torch's expression;
both the streamed form (odie_reconstruct + score_chunk) and the fused one (odie_reconstruct_scores,
a wave per cell)."""
import numpy as np
import pytest
import torch

import oracle
from odie_amd import synth
from odie_amd.decoder import Decoder
from odie_amd.experts import ExpertGrid, route
from odie_amd.reconstruction import reconstruct, score_image
from odie_amd.selection import topk_tiles

pytestmark = pytest.mark.gpu

ENCODING = dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=10, base_resolution=4, per_level_scale=1.3)


def _model(seed, experts):
    grid = ExpertGrid(ENCODING, experts)
    values = synth.normal(seed, 'recon_table', grid.table.numel()) * 0.5
    grid.table.copy_(torch.from_numpy(values.astype(np.float16)))
    return grid, Decoder(seed=seed)


def _composed(grid, decoder, shape, regions, begin, n, slots=None):
    height, width = shape
    ids = torch.arange(begin, begin + n, dtype=torch.int64, device='cuda')
    routing = route(ids, width, height, *regions)
    features_c = grid.forward(routing.coords, routing.offsets) if slots is None else None
    if slots is not None:
        # tiles without an expert read zero features; others read their slot's table
        table = grid.table.view(grid.experts, -1)
        regrouped = ExpertGrid(ENCODING, regions[0] * regions[1])
        for tile, slot in enumerate(slots.tolist()):
            if 0 <= slot < grid.experts:
                regrouped.table.view(regrouped.experts, -1)[tile].copy_(table[slot])
        features_c = regrouped.forward(routing.coords, routing.offsets)
    output_c = decoder.forward(features_c)
    perm = routing.perm.long()
    features = torch.empty_like(features_c)
    features[perm] = features_c
    output = torch.empty_like(output_c)
    output[perm] = output_c
    return features, output


def _bits(t):
    return t.cpu().numpy().view(np.uint16 if t.dtype == torch.float16 else np.uint32)


@pytest.mark.parametrize('shape,regions,begin,n', [((96, 130), (3, 2), 0, 96 * 130),
                                                   ((96, 130), (3, 2), 1001, 5000 - 7),
                                                   ((200, 64), (2, 5), 12345, 1)])
def test_reconstruction_equals_route_encode_decoder(shape, regions, begin, n):
    grid, decoder = _model(2, regions[0] * regions[1])
    features = torch.empty((n, 32), dtype=torch.float16, device='cuda')
    output = torch.empty((n, 16), dtype=torch.float16, device='cuda')
    prediction = reconstruct(grid, decoder.half, shape, regions, begin, n, prediction=torch.empty(
        (n, 3), dtype=torch.float32, device='cuda'), features=features, output=output)
    want_features, want_output = _composed(grid, decoder, shape, regions, begin, n)
    assert np.array_equal(_bits(features), _bits(want_features))
    assert np.array_equal(_bits(output), _bits(want_output))
    assert np.array_equal(_bits(prediction), _bits(want_output[:, :3].float()))


def test_tiles_without_an_expert_predict_zero():
    shape, regions = (120, 90), (3, 3)
    grid, decoder = _model(3, 5)
    slots = torch.tensor([4, -1, 0, 2, 9, 1, -1, 3, 0], dtype=torch.int32, device='cuda')   # 9 >= experts: none
    n = shape[0] * shape[1]
    features = torch.empty((n, 32), dtype=torch.float16, device='cuda')
    output = torch.empty((n, 16), dtype=torch.float16, device='cuda')
    reconstruct(grid, decoder.half, shape, regions, 0, n, slots=slots, features=features, output=output)
    want_features, want_output = _composed(grid, decoder, shape, regions, 0, n, slots=slots.cpu())
    assert np.array_equal(_bits(features), _bits(want_features))
    assert np.array_equal(_bits(output), _bits(want_output))
    empty = (want_features == 0).all(dim=1)
    assert bool(empty.any()) and bool((output[empty] == 0).all())


@pytest.mark.parametrize('fused', [True, False])
@pytest.mark.parametrize('shape,resolution,tile,batch', [((128, 160), 8, None, 4096), ((128, 128), None, 32, 10000),
                                                         ((90, 77), 5, None, 1000)])
def test_scoring_pipeline_matches_the_oracle(shape, resolution, tile, batch, fused):
    regions = (4, 4) if shape[0] >= 128 else (3, 2)
    grid, decoder = _model(4, regions[0] * regions[1])
    image = synth.image(5, shape[1], shape[0]).reshape(-1, 3)
    target = torch.from_numpy(image).cuda()
    n = shape[0] * shape[1]
    image_out = torch.full((n, 3), float('nan'), dtype=torch.float32, device='cuda') if fused else None
    metrics, scores = score_image(grid, decoder.half, target, shape, regions, resolution=resolution, tile=tile,
                                  batch=batch, fused=fused, prediction=image_out)
    prediction = reconstruct(grid, decoder.half, shape, regions, 0, n).cpu().numpy()
    if fused:
        assert np.array_equal(image_out.cpu().numpy().view(np.uint32), prediction.view(np.uint32))
    expected = oracle.residual(prediction, image, shape[1], scores.resolution, scores.xb.cpu().numpy(),
                               scores.yb.cpu().numpy())
    assert np.array_equal(scores.totals.cpu().numpy().view(np.uint64), expected.view(np.uint64))
    truth = torch.from_numpy(image).cuda().float() / 255.
    reference = ((torch.from_numpy(prediction).cuda() - truth).square().double().sum() / image.size).item()
    assert metrics['mse'] == pytest.approx(reference, rel=1e-12)   # summation order only
    k = scores.resolution ** 2 // 4
    ids = topk_tiles(scores.totals / torch.from_numpy(scores.counts).cuda(), k).cpu().numpy()
    means = expected / scores.counts
    assert np.array_equal(ids, oracle.topk_ids(means, k))


def test_device_image_on_the_gpu_equals_numpy():
    expected = synth.image(7, 300, 170)
    got = synth.image_device(7, 300, 170, device='cuda', rows=64).cpu().numpy()
    assert np.array_equal(got, expected)
