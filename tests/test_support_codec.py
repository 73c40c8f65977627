"""The on-disk support codec and fp16 artifact (odie/support_codec.py, odie/train.py:207-232):
round trips, the smallest-stream rule, the reference's validation errors, the legacy bitmap
form, and the per-layer storage records of the reference's own runs (results/**/metrics.json)."""
import json
from pathlib import Path
import zlib

import numpy as np
import pytest
import torch

from odie_amd import synth
from odie_amd.decoder import Decoder
from odie_amd.gate import Gate
from odie_amd.model import PackedPlanes
from odie_amd.support_codec import (compress_checkpoint, decode_support, decode_supports, encode_support,
                                    encode_supports, read_artifact, support_storage_statistics, write_artifact)

GOLDEN = Path(__file__).parent / 'golden'


def _mask(resolution, fraction, seed, blocky=False):
    if blocky:   # one rectangle: compresses well
        m = np.zeros((resolution, resolution), dtype=bool)
        m[resolution // 4:resolution // 2, resolution // 3:] = True
        return torch.from_numpy(m.reshape(-1))
    return torch.from_numpy(synth.uniform(seed, 'mask', resolution * resolution) < fraction)


@pytest.mark.parametrize('resolution,fraction,blocky,encoding', [
    (8, 1.0, False, 'all'), (8, 0.0, False, 'none'), (64, 0.5, False, 'bitmap'),
    (256, 0.0, True, 'bitmap_deflate'), (13, 0.3, False, None), (1, 1.0, False, 'all')])
def test_round_trip_and_smallest_stream(resolution, fraction, blocky, encoding):
    support = _mask(resolution, fraction, resolution, blocky)
    record = encode_support(support)
    assert torch.equal(decode_support(record), support)
    assert record['num_cells'] == resolution ** 2 and record['selected_count'] == int(support.sum())
    if encoding is not None:
        assert record['encoding'] == encoding
    if 'data' in record:
        bitmap = np.packbits(support.numpy(), bitorder='little').tobytes()
        deflated = zlib.compressobj(9, zlib.DEFLATED, -15)
        deflated = deflated.compress(bitmap) + deflated.flush()
        assert record['data'].numel() == min(len(bitmap), len(deflated))   # the raw bitmap wins ties


def test_decoder_rejects_corrupt_records():
    support = _mask(16, 0.5, 3)
    good = encode_support(support)
    bad = dict(good, selected_count=good['selected_count'] + 1)
    with pytest.raises(ValueError, match='selected count mismatch'):
        decode_support(bad)
    padded = dict(good, num_cells=15 * 15, resolution=15)
    with pytest.raises(ValueError, match='padding mismatch|count'):
        decode_support(padded)
    with pytest.raises(ValueError, match='Invalid support geometry'):
        decode_support(dict(good, resolution=5))
    with pytest.raises(ValueError, match='Unknown support encoding'):
        decode_support(dict(good, encoding='png'))
    with pytest.raises(RuntimeError, match='libjbig'):
        decode_support(dict(good, encoding='jbig1'))
    with pytest.raises(ValueError, match='Constant mask count mismatch'):
        decode_support(dict(num_cells=4, resolution=2, selected_count=3, encoding='all'))
    blocky = encode_support(_mask(256, 0, 0, True))
    trailing = dict(blocky, data=torch.cat([blocky['data'], torch.tensor([7], dtype=torch.uint8)]))
    with pytest.raises(ValueError, match='trailing DEFLATE'):
        decode_support(trailing)
    with pytest.raises(ValueError, match='nonempty flat CPU bool'):
        encode_support(torch.zeros(0, dtype=torch.bool))
    with pytest.raises(ValueError, match='square grid'):
        encode_support(torch.ones(10, dtype=torch.bool))


def test_legacy_bitmaps_and_layer_checks():
    supports = [_mask(r, 0.4, r) for r in (4, 9, 16)]
    configuration = dict(representation='xy_planes', resolutions=[4, 9, 16])
    legacy = dict(configuration=configuration, support_num_cells=[16, 81, 256],
                  support_bitmaps=[torch.from_numpy(np.packbits(s.numpy(), bitorder='little')) for s in supports])
    assert all(torch.equal(a, b) for a, b in zip(decode_supports(legacy), supports))
    modern = dict(configuration=configuration, support_num_cells=[16, 81, 256],
                  support_storage_version='layerwise-bitmap-deflate-jbig-v1', support_encodings=encode_supports(supports))
    assert all(torch.equal(a, b) for a, b in zip(decode_supports(modern), supports))
    with pytest.raises(ValueError, match='storage version'):
        decode_supports(dict(modern, support_storage_version='v0'))
    with pytest.raises(ValueError, match='model configuration'):
        decode_supports(dict(modern, configuration=dict(configuration, resolutions=[4, 9, 15])))


def test_reference_run_storage_records_are_consistent():
    """Every support_storage layer recorded by the reference's runs obeys the codec's invariants:
    bitmap_bytes = ceil(R^2 / 8), constant masks carry no payload and name 'all' exactly when every
    cell is selected, and no stream is larger than the raw bitmap."""
    records = json.loads((GOLDEN / 'support_storage_records.json').read_text())
    assert len(records) >= 10
    for run in records:
        for layer in run['layers']:
            cells = layer['resolution'] ** 2
            assert layer['bitmap_bytes'] == (cells + 7) // 8
            if layer['encoding'] in ('all', 'none'):
                assert layer['payload_bytes'] == 0
                assert layer['selected_count'] == (cells if layer['encoding'] == 'all' else 0)
            else:
                assert 0 < layer['selected_count'] < cells
                assert 0 < layer['payload_bytes'] <= layer['bitmap_bytes']
                if layer['encoding'] == 'bitmap':
                    assert layer['payload_bytes'] == layer['bitmap_bytes']
        assert run['bitmap_bytes'] == sum(layer['bitmap_bytes'] for layer in run['layers'])
        assert run['payload_bytes'] == sum(layer['payload_bytes'] for layer in run['layers'])


def test_artifact_round_trip(tmp_path):
    resolutions = [4, 6, 9, 13, 20]
    supports = [torch.ones(r * r, dtype=torch.bool) if i < 3 else _mask(r, 0.3, i) for i, r in enumerate(resolutions)]
    caps = [(r * r + 7) // 8 * 8 for r in resolutions]
    configuration = dict(resolutions=resolutions, n_levels=5, representation='xy_planes', coarse_levels=1,
                         gate_topology='shared', gate_position='feature', initial_active_prefix=3, seed=4,
                         feature_init_std=1e-2, plane_feature_dimensions=[2] * 5, cell_caps=caps,
                         gate_coarse_levels_K=1, router_output_activation='sigmoid')
    planes = PackedPlanes(configuration, supports, [2] * 5, caps, device='cpu')
    decoder, gate = Decoder(seed=1, device="cpu", width=16), Gate(seed=2, coarse=1, device="cpu", features=[2] * 5)
    path = tmp_path / 'model_latest_fp16.pt'
    storage = write_artifact(path, configuration, planes, decoder, gate, epoch=3, optimizer_steps=30,
                             metrics={'mse': 0.01})
    assert storage == support_storage_statistics(encode_supports(planes.supports))
    artifact, planes2, decoder2, gate2 = read_artifact(path, device='cpu')
    assert artifact['version'] == 'packed-capacity-control-v1' and artifact['epoch'] == 3
    assert all(torch.equal(a, b) for a, b in zip(planes.supports, planes2.supports))
    assert torch.equal(planes2.grid, planes.grid.half().float())
    assert torch.equal(decoder2.params, decoder.params.half().float())
    assert torch.equal(gate2.params, gate.params.half().float()) and gate2.coarse == 1
    assert set(artifact['parameters']) == {'grid', 'gate.params', 'decoder.params'}
    out = tmp_path / 'repacked.pt'
    summary = compress_checkpoint(path, out)
    assert summary['roundtrip_verified'] and out.exists()
    with pytest.raises(FileExistsError):
        compress_checkpoint(path, out)
