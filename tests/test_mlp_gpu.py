"""Decoder MLP on MFMA (odie_mlp_forward / odie_mlp_train) against the oracle, stage by stage.

Each layer is checked from the GPU's own input to that layer (its exported hidden
activations), so a ReLU mask that flips on a pre-activation within rounding of zero cannot
cascade.  Tolerance for fp16 results: 2^-10 relative plus 2^-16 of the magnitude sum
sum |a||b| (fp32 accumulation in a different order); the loss (dy, squares) is checked
through the rows' outputs bit-exactly, and the weight gradients within 2^-9 of their
magnitude sums.
"""
import numpy as np
import pytest
import torch

import oracle
from odie_amd import synth
from odie_amd.decoder import Decoder, PARAMETERS

pytestmark = pytest.mark.gpu


def _inputs(seed, n, width=32):
    x = (synth.normal(seed, 'mlp_x', n * width).reshape(n, width) * 0.5).astype(np.float16)
    decoder = Decoder(seed=seed, width=width)
    return x, decoder


def _close16(got, expected, magnitude):
    got = got.astype(np.float64)
    expected = expected.astype(np.float64)
    tolerance = 2.0 ** -10 * np.abs(expected) + 2.0 ** -16 * magnitude + 2.0 ** -24
    bad = np.abs(got - expected) > tolerance
    assert not bad.any(), (np.flatnonzero(bad)[:8], got.ravel()[np.flatnonzero(bad)[:4]],
                           expected.ravel()[np.flatnonzero(bad)[:4]])


@pytest.mark.parametrize('n,width', [(1, 32), (31, 32), (1000, 32), (4096, 32), (1000, 16), (777, 48), (3000, 64),
                                     (2049, 80)])
def test_forward_matches_oracle(n, width):
    x, decoder = _inputs(1, n, width)
    out = decoder.forward(torch.from_numpy(x).cuda()).cpu().numpy()
    flat = decoder.half.cpu().numpy()
    w1, w2, w3 = (w.astype(np.float64) for w in oracle.mlp_weights(flat))
    h1, h2, y = oracle.mlp_forward(x, flat)
    # end to end: a hidden value that differs by rounding (or a mask flipped by a pre-activation
    # within rounding of zero) moves the output by at most its magnitude chain
    m1 = np.abs(x.astype(np.float64)) @ np.abs(w1).T
    m2 = (np.abs(h1.astype(np.float64)) + m1) @ np.abs(w2).T
    m3 = (np.abs(h2.astype(np.float64)) + m2) @ np.abs(w3).T
    _close16(out, y, 2.0 ** 4 * m3)


def _train_case(seed, n, *, rgb8=True, permute=True, real=None, width=32):
    x, decoder = _inputs(seed, n, width)
    real = n if real is None else real
    rows = synth.integers(seed, 'rows', n, 1 << 30).argsort(kind='stable').astype(np.int32) if permute \
        else np.arange(n, dtype=np.int32)
    pixels = 5000
    image = synth.integers(seed, 'image', pixels * 3, 256).astype(np.uint8)
    ids = synth.integers(seed, 'ids', n, pixels).astype(np.int64)
    target = synth.uniform(seed, 'target', n * 3).reshape(n, 3)
    device = dict(device='cuda')
    xd = torch.from_numpy(x).cuda()
    out = torch.full((n, 16), float('nan'), dtype=torch.float16, **device)
    hidden = torch.empty((n, 128), dtype=torch.float16, **device)
    squares = torch.full((n,), float('nan'), dtype=torch.float32, **device)
    kwargs = dict(rows=torch.from_numpy(rows).cuda(), out=out, hidden=hidden, squares=squares)
    if rgb8 == 'colors':
        pixel = image.reshape(-1, 3)[ids[rows]].astype(np.uint32)
        packed = (pixel[:, 0] | (pixel[:, 1] << 8) | (pixel[:, 2] << 16)).astype(np.uint32).view(np.int32)
        kwargs.update(colors=torch.from_numpy(packed).cuda())
    elif rgb8 == 'pixels':   # each tile row's pixel index, the target's bytes read by the decoder
        kwargs.update(pixels=torch.from_numpy(ids[rows].astype(np.int32)).cuda(), rgb=torch.from_numpy(image).cuda())
    elif rgb8:
        kwargs.update(rgb=torch.from_numpy(image).cuda(), ids=torch.from_numpy(ids).cuda())
    else:
        kwargs.update(target=torch.from_numpy(target).cuda())
    dz = decoder.train(xd, real, **kwargs).cpu().numpy()
    got = dict(out=out.cpu().numpy(), hidden=hidden.cpu().numpy(), squares=squares.cpu().numpy(), dz=dz,
               dweights=decoder.grad.cpu().numpy())
    return x, decoder.half.cpu().numpy(), rows, image, ids, target, real, got


@pytest.mark.parametrize('n,rgb8,permute,real,width', [
    (4096, True, True, None, 32),
    (1000, False, False, None, 32),     # ragged last tile, fp32 targets, identity rows
    (2048, True, True, 1500, 32),       # inputs >= real are padding rows
    (1 << 17, True, True, None, 32),    # every workgroup runs several tiles
    ((1 << 20) + 4133, True, True, None, 32),   # whole 128-row records per wave, ragged last record
    (5000, 'colors', True, 4000, 32),   # packed per-row targets (as odie_route writes them)
    (5000, 'pixels', True, 4000, 32),   # per-row pixel indexes into the image
    ((1 << 20) + 99, 'pixels', True, None, 32),
    (4096, True, True, None, 16),       # the input widths of the other level rows: 8 levels (16),
    (3001, True, False, 2500, 48),      # 20 levels of F2/F1 (48), F4 rows (64, 80)
    (1 << 16, 'colors', True, None, 64),
    (5000, False, True, None, 80),
])
def test_train_matches_oracle_stagewise(n, rgb8, permute, real, width):
    x, flat, rows, image, ids, target, real, got = _train_case(7, n, rgb8=rgb8, permute=permute, real=real,
                                                               width=width)
    w1, w2, w3 = oracle.mlp_weights(flat)
    xs = x  # tile row j reads x[j]
    h1 = got['hidden'][:, :64]
    h2 = got['hidden'][:, 64:]
    ref_h1, m1 = oracle.mlp_layer(xs, w1, True)
    _close16(h1, ref_h1, m1)
    ref_h2, m2 = oracle.mlp_layer(h1, w2, True)
    _close16(h2, ref_h2, m2)
    ref_y, m3 = oracle.mlp_layer(h2, w3, False)
    y = got['out'][rows]                      # outputs are stored at the input row
    _close16(y, ref_y, m3)
    # loss through the GPU's own outputs: bit-exact
    targets = oracle.mlp_targets(rows, rgb=image if rgb8 else None, ids=ids, target=None if rgb8 else target)
    dy, squares = oracle.mlp_loss(y, targets, rows, real)
    assert np.array_equal(got['squares'][rows], squares)
    dz, dz_magnitude, dweights, magnitude = oracle.mlp_backward(xs, h1, h2, dy, flat)
    _close16(got['dz'], dz, 2.0 ** 6 * dz_magnitude)
    bad = np.abs(got['dweights'] - dweights) > 2.0 ** -9 * magnitude + 1e-6
    assert not bad.any(), np.flatnonzero(bad)[:8]


def test_train_is_deterministic_and_forward_agrees():
    first = _train_case(11, 3000)[-1]
    second = _train_case(11, 3000)[-1]
    for key in ('out', 'dz', 'dweights', 'squares'):
        assert np.array_equal(first[key].view(np.uint8), second[key].view(np.uint8)), key
    x, decoder = _inputs(11, 3000)
    rows = synth.integers(11, 'rows', 3000, 1 << 30).argsort(kind='stable')
    forward = decoder.forward(torch.from_numpy(x).cuda()).cpu().numpy()
    assert np.array_equal(forward.view(np.uint16), first['out'][rows].view(np.uint16))


def test_empty_batch_zeroes_weight_gradient():
    decoder = Decoder(seed=2)
    decoder.grad.fill_(1.0)
    decoder.train(torch.empty((0, 32), dtype=torch.float16, device='cuda'), 1,
                  target=torch.zeros((0, 3), device='cuda'))
    torch.cuda.synchronize()
    assert decoder.grad.shape == (PARAMETERS,) and not decoder.grad.any()


def _record_maxima(dz):
    """max |dz| per 128-row record and column (torch's amax keeps NaN), fp32 [ceil(n/128), 32]."""
    n = dz.shape[0]
    records = (n + 127) // 128
    column = dz.abs().view(n, 32).float()
    padded = torch.zeros((records * 128, 32), dtype=torch.float32, device=dz.device)
    padded[:n] = column
    return padded.view(records, 128, 32).amax(dim=1)


@pytest.mark.parametrize('n,poison', [(1, False), (1000, False), (4096 + 37, False), (1 << 17, False), (3000, True),
                                     ((1 << 20) + 37, False)])
def test_train_planes_equals_rows(n, poison):
    """odie_mlp_train_planes writes odie_mlp_train's dz, bit for bit, as level-major planes with
    exact 128-row maxima (NaN where a row of the record is NaN); outputs and gradients agree."""
    x, decoder = _inputs(13, n)
    xd = torch.from_numpy(x).cuda()
    if poison:
        # a NaN target makes its row's dz NaN (a NaN input would not: the ReLU on bit patterns
        # turns a negative-signed NaN into +0)
        target = torch.from_numpy(synth.normal(13, 'target', n * 3).reshape(n, 3).astype(np.float32)).cuda()
        target[1234, 1] = float('nan')
        source = dict(target=target)
    else:
        image = synth.image(13, 64, 48)
        source = dict(rgb=torch.from_numpy(image).cuda(), ids=torch.from_numpy(synth.integers(13, 'ids', n, 64 * 48)).cuda())
    squares = [torch.full((n,), float('nan'), device='cuda') for _ in range(2)]
    dz = decoder.train(xd, squares=squares[0], **source)
    rows_grad = decoder.grad.clone()
    planes, blockmax = decoder.train_planes(xd, squares=squares[1], **source)
    want = dz.view(torch.int32).view(n, 16).t().contiguous()
    assert torch.equal(planes, want)
    expected = _record_maxima(dz)
    assert np.array_equal(blockmax.cpu().numpy(), expected.cpu().numpy(), equal_nan=True)
    assert bool(blockmax.isnan().any()) == poison
    assert torch.equal(squares[0].view(torch.int32), squares[1].view(torch.int32))
    assert torch.equal(decoder.grad.view(torch.int32), rows_grad.view(torch.int32))
