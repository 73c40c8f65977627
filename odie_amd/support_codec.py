"""The on-disk form of a trained model: lossless layerwise support storage and the fp16
artifact (odie/support_codec.py:1-188, odie/train.py:197-232), so that artifacts written by the
reference load here and the other way round.

A support (a flat bool mask of one level's R x R cells) is stored as the smallest of: nothing
('all' / 'none'), the raw LSB-first bitmap, its raw DEFLATE stream (zlib level 9, window 15, no
header) or a JBIG1 stream; the raw bitmap wins ties.  JBIG1 needs libjbig, which this image does
not have: as in the reference without it, masks are written as bitmap / DEFLATE, and reading a
JBIG1 mask raises.
"""
import math
from pathlib import Path
import warnings
import zlib

import numpy as np
import torch

STORAGE_VERSION = 'layerwise-bitmap-deflate-jbig-v1'
ARTIFACT_VERSION = 'packed-capacity-control-v1'


def jbig_tool():
    """The JBIG1 bridge of the reference needs g++ with libjbig; it is absent here."""
    warnings.warn('JBIG unavailable: libjbig headers/library are required; exporting bitmap/DEFLATE masks.')
    return None


def encode_support(support):
    """Record of one support: num_cells, resolution, selected_count, encoding and, unless the
    mask is constant, data (flat uint8 tensor) (odie/support_codec.py:51-74)."""
    if support.device.type != 'cpu' or support.dtype != torch.bool or support.ndim != 1 or support.numel() < 1:
        raise ValueError('Support must be a nonempty flat CPU bool tensor')
    values = support.numpy()
    total, count = values.size, int(values.sum())
    resolution = math.isqrt(total)
    if resolution ** 2 != total:
        raise ValueError('Support must describe a square grid')
    record = dict(num_cells=total, resolution=resolution, selected_count=count)
    if count in (0, total):
        return dict(record, encoding='all' if count else 'none')
    bitmap = np.packbits(values, bitorder='little').tobytes()
    compressor = zlib.compressobj(9, zlib.DEFLATED, -15)
    candidates = {'bitmap': bitmap, 'bitmap_deflate': compressor.compress(bitmap) + compressor.flush()}
    # the raw bitmap is first, so ties keep the simplest representation
    encoding, data = min(candidates.items(), key=lambda item: len(item[1]))
    record.update(encoding=encoding, data=torch.from_numpy(np.frombuffer(data, dtype=np.uint8).copy()))
    if not torch.equal(decode_support(record), support):
        raise AssertionError('Selected mask codec changed support membership')
    return record


def decode_support(record):
    """The flat bool mask of a record, with the reference's validation (odie/support_codec.py:77-117)."""
    total, resolution, count = record['num_cells'], record['resolution'], record['selected_count']
    if (type(total) is not int or total < 1 or type(resolution) is not int or resolution < 1 or resolution ** 2 != total
            or type(count) is not int or not 0 <= count <= total):
        raise ValueError('Invalid support geometry or selected count')
    encoding = record['encoding']
    if encoding in ('all', 'none'):
        if count != (total if encoding == 'all' else 0):
            raise ValueError('Constant mask count mismatch')
        return torch.full((total,), encoding == 'all', dtype=torch.bool)
    payload = record['data']
    if not isinstance(payload, torch.Tensor) or payload.dtype != torch.uint8 or payload.ndim != 1:
        raise ValueError('Mask payload must be a flat uint8 tensor')
    data = payload.detach().cpu().numpy().tobytes()
    if encoding == 'jbig1':
        raise RuntimeError('Reading this JBIG checkpoint requires g++ and libjbig headers/library')
    if encoding not in ('bitmap', 'bitmap_deflate'):
        raise ValueError('Unknown support encoding: ' + str(encoding))
    if encoding == 'bitmap_deflate':
        decoder = zlib.decompressobj(-15)
        try:
            data = decoder.decompress(data, (total + 7) // 8 + 1)
        except zlib.error as error:
            raise ValueError('Invalid DEFLATE mask') from error
        if not decoder.eof or decoder.unused_data or decoder.unconsumed_tail:
            raise ValueError('Incomplete or trailing DEFLATE data')
    if len(data) != (total + 7) // 8 or (total % 8 and data[-1] >> (total % 8)):
        raise ValueError('Bitmap length or padding mismatch')
    values = np.unpackbits(np.frombuffer(data, dtype=np.uint8), bitorder='little', count=total)
    if int(values.sum()) != count:
        raise ValueError('Decoded selected count mismatch')
    return torch.from_numpy(values.astype(bool))


def encode_supports(supports):
    return [encode_support(support) for support in supports]


def decode_supports(artifact):
    """Supports of an artifact: the layerwise records, or the legacy packed bitmaps
    (odie/support_codec.py:124-148)."""
    counts = artifact['support_num_cells']
    if 'support_encodings' in artifact:
        if artifact.get('support_storage_version') != STORAGE_VERSION:
            raise ValueError('Unsupported support storage version')
        if len(artifact['support_encodings']) != len(counts):
            raise ValueError('Encoded layer count mismatch')
        supports = [decode_support(record) for record in artifact['support_encodings']]
    else:
        bitmaps = artifact['support_bitmaps']
        if len(bitmaps) != len(counts):
            raise ValueError('Legacy bitmap layer count mismatch')
        supports = []
        for bits, count in zip(bitmaps, counts):
            if (type(count) is not int or count < 1 or bits.dtype != torch.uint8 or bits.ndim != 1
                    or bits.numel() != (count + 7) // 8):
                raise ValueError('Invalid legacy bitmap')
            supports.append(torch.from_numpy(np.unpackbits(bits.detach().cpu().numpy(), bitorder='little',
                                                           count=count).astype(bool)))
    if [support.numel() for support in supports] != counts:
        raise ValueError('Support sizes differ from checkpoint geometry')
    configuration = artifact['configuration']
    resolutions = configuration.get('resolutions')
    expected = [] if configuration['representation'] == 'hash_grid' else \
        [r * r for r in resolutions] if resolutions is not None else None
    if expected is not None and counts != expected:
        raise ValueError('Support sizes differ from model configuration')
    return supports


def restore_support_record(artifact):
    return dict(artifact['support_payload'], supports=decode_supports(artifact))


def support_storage_statistics(encodings):
    """Per-layer storage record (the `support_storage` block of the reference's metrics)."""
    layers = [dict(level=i, resolution=record['resolution'], selected_count=record['selected_count'],
                   encoding=record['encoding'], bitmap_bytes=(record['num_cells'] + 7) // 8,
                   payload_bytes=record['data'].numel() if 'data' in record else 0)
              for i, record in enumerate(encodings)]
    return dict(version=STORAGE_VERSION, selection_rule='smallest available serialized stream; raw bitmap wins ties',
                layers=layers, bitmap_bytes=sum(row['bitmap_bytes'] for row in layers),
                payload_bytes=sum(row['payload_bytes'] for row in layers))


def compress_checkpoint(source, destination):
    """Repack an artifact's supports into the layerwise form without touching its weights
    (odie/support_codec.py:161-188)."""
    source, destination = Path(source), Path(destination)
    if destination.exists():
        raise FileExistsError(destination)
    artifact = torch.load(source, map_location='cpu', weights_only=True)
    supports = decode_supports(artifact)
    encodings = encode_supports(supports)
    compact = {key: value for key, value in artifact.items()
               if key not in ('support_bitmaps', 'support_encodings', 'support_storage_version')}
    compact.update(support_storage_version=STORAGE_VERSION, support_encodings=encodings)
    destination.parent.mkdir(parents=True, exist_ok=True)
    with destination.open('xb') as stream:
        torch.save(compact, stream)
    restored = torch.load(destination, map_location='cpu', weights_only=True)
    if not all(torch.equal(a, b) for a, b in zip(supports, decode_supports(restored))):
        raise AssertionError('Repacked checkpoint changed supports')
    if not all(torch.equal(value.contiguous().view(torch.uint8), restored['parameters'][name].contiguous().view(torch.uint8))
               for name, value in artifact['parameters'].items()):
        raise AssertionError('Repacked checkpoint changed weights')
    return dict(source=str(source), output=str(destination), source_bytes=source.stat().st_size,
                checkpoint_bytes=destination.stat().st_size,
                fp16_parameter_payload_bytes=sum(p.numel() * p.element_size() for p in restored['parameters'].values()),
                support_storage=support_storage_statistics(encodings), roundtrip_verified=True)


def model_parameters(planes, decoder, gate=None):
    """fp16 CPU copies of the model's parameters under the reference module's names
    (grid, gate.params, decoder.params; odie/train.py:199)."""
    state = {'grid': planes.grid.detach().to('cpu', torch.float16)}
    if gate is not None:
        state['gate.params'] = gate.params.detach().to('cpu', torch.float16)
    state['decoder.params'] = decoder.params.detach().to('cpu', torch.float16)
    return state


def write_artifact(path, configuration, planes, decoder, gate=None, *, settings=None, support_payload=None,
                   support_metadata=None, epoch=0, optimizer_steps=0, metrics=None):
    """The reference's model_latest_fp16.pt (odie/train.py:207-215): configuration, the layerwise
    supports, the fp16 parameters and the run's counters, verified by reloading."""
    encodings = encode_supports(planes.supports)
    artifact = {'version': ARTIFACT_VERSION, 'configuration': configuration, 'settings': settings or {},
                'support_storage_version': STORAGE_VERSION, 'support_encodings': encodings,
                'support_num_cells': [s.numel() for s in planes.supports],
                'support_payload': support_payload or {}, 'support_metadata': support_metadata or {},
                'parameters': model_parameters(planes, decoder, gate), 'checkpoint': 'latest',
                'epoch': epoch, 'optimizer_steps': optimizer_steps, 'metrics': metrics or {}}
    torch.save(artifact, path)
    reloaded = torch.load(path, map_location='cpu', weights_only=True)
    if reloaded['configuration'] != configuration:
        raise AssertionError('Saved configuration changed during round trip')
    if not all(torch.equal(a, b) for a, b in zip(planes.supports, decode_supports(reloaded))):
        raise AssertionError('Saved supports changed during round trip')
    return support_storage_statistics(encodings)


def read_artifact(path, device='cuda', plane_dims=None, plane_node_caps=None):
    """Model of an artifact: PackedPlanes from its configuration (plane_feature_dimensions and
    cell_caps unless given) and supports with the stored fp16 grid, and the fp16 head weights (as
    fp32 masters)."""
    from .decoder import Decoder
    from .gate import Gate
    from .model import PackedPlanes
    artifact = torch.load(path, map_location='cpu', weights_only=True)
    configuration = dict(artifact['configuration'])
    supports = decode_supports(artifact)
    plane_dims = configuration['plane_feature_dimensions'] if plane_dims is None else plane_dims
    plane_node_caps = configuration['cell_caps'] if plane_node_caps is None else plane_node_caps
    planes = PackedPlanes(dict(configuration, initial_active_prefix=0), supports, plane_dims, plane_node_caps,
                          device=device)
    parameters = artifact['parameters']
    if parameters['grid'].numel() != planes.grid.numel():
        raise ValueError('Saved grid size differs from the layout of its supports')
    planes.grid.copy_(parameters['grid'].to(device=planes.grid.device, dtype=torch.float32))
    planes.set_active_prefix(int(configuration['n_levels']))
    decoder = Decoder(weights=parameters['decoder.params'].float().numpy(), device=device)
    gate = None
    if 'gate.params' in parameters:
        gate = Gate(weights=parameters['gate.params'].float().numpy(), coarse=int(configuration.get(
            'gate_coarse_levels_K', 0)), activation=configuration.get('router_output_activation', 'sigmoid'),
            device=device)
    return artifact, planes, decoder, gate
