"""The on-disk form of a trained model: lossless layerwise support storage and the fp16 artifact
(the format of odie/support_codec.py:1-188 and odie/train.py:197-232), so that artifacts written
by the reference load here and the other way round.

A support (a flat bool mask of one level's R x R cells) is stored as a record with num_cells,
resolution, selected_count and encoding: 'all' / 'none' for constant masks (no payload), else
the shortest payload among the available codecs -- 'bitmap' (LSB-first bits), 'bitmap_deflate'
(that bitmap as raw DEFLATE: zlib level 9, window 15, no header) and 'jbig1' -- tried in that
order, so the plain bitmap wins ties.  JBIG1 needs libjbig, which this image does not have: as in
the reference without it, masks are written with the other codecs and reading a JBIG1 mask
raises.
"""
import math
from pathlib import Path
import warnings
import zlib

import numpy as np
import torch

STORAGE_VERSION = 'layerwise-bitmap-deflate-jbig-v1'
ARTIFACT_VERSION = 'packed-capacity-control-v1'
SELECTION_RULE = 'smallest available serialized stream; raw bitmap wins ties'


def jbig_tool():
    """The JBIG1 bridge needs g++ with libjbig; it is absent here."""
    warnings.warn('JBIG unavailable: libjbig headers/library are required; exporting bitmap/DEFLATE masks.')
    return None


def _bitmap_bytes(total):
    return (total + 7) // 8


class _Bitmap:
    name = 'bitmap'

    def pack(self, mask):
        return np.packbits(mask, bitorder='little').tobytes()

    def unpack(self, data, total):
        if len(data) != _bitmap_bytes(total) or (total % 8 and data[-1] >> (total % 8)):
            raise ValueError('Bitmap length or padding mismatch')
        return np.unpackbits(np.frombuffer(data, dtype=np.uint8), bitorder='little', count=total)


class _Deflate(_Bitmap):
    name = 'bitmap_deflate'

    def pack(self, mask):
        stream = zlib.compressobj(9, zlib.DEFLATED, -15)
        return stream.compress(super().pack(mask)) + stream.flush()

    def unpack(self, data, total):
        stream = zlib.decompressobj(-15)
        try:
            raw = stream.decompress(data, _bitmap_bytes(total) + 1)
        except zlib.error as error:
            raise ValueError('Invalid DEFLATE mask') from error
        if not stream.eof or stream.unused_data or stream.unconsumed_tail:
            raise ValueError('Incomplete or trailing DEFLATE data')
        return super().unpack(raw, total)


class _Jbig:
    name = 'jbig1'

    def pack(self, mask):
        jbig_tool()          # warns: without libjbig there is no JBIG1 stream to compare
        return None

    def unpack(self, data, total):
        raise RuntimeError('Reading this JBIG checkpoint requires g++ and libjbig headers/library')


CODECS = (_Bitmap(), _Deflate(), _Jbig())
_BY_NAME = {codec.name: codec for codec in CODECS}


def _geometry(record):
    total, resolution, count = record['num_cells'], record['resolution'], record['selected_count']
    valid = (type(total) is int and total >= 1 and type(resolution) is int and resolution >= 1
             and resolution ** 2 == total and type(count) is int and 0 <= count <= total)
    if not valid:
        raise ValueError('Invalid support geometry or selected count')
    return total, count


def encode_support(support):
    """Record of one flat CPU bool support (odie/support_codec.py:51-74)."""
    if support.device.type != 'cpu' or support.dtype != torch.bool or support.ndim != 1 or support.numel() < 1:
        raise ValueError('Support must be a nonempty flat CPU bool tensor')
    mask = support.numpy()
    total = mask.size
    resolution = math.isqrt(total)
    if resolution * resolution != total:
        raise ValueError('Support must describe a square grid')
    count = int(mask.sum())
    record = dict(num_cells=total, resolution=resolution, selected_count=count)
    if count == total or count == 0:
        record['encoding'] = 'all' if count else 'none'
        return record
    best = None
    for codec in CODECS:
        payload = codec.pack(mask)
        if payload is not None and (best is None or len(payload) < len(best[1])):
            best = (codec.name, payload)
    record['encoding'] = best[0]
    record['data'] = torch.from_numpy(np.frombuffer(best[1], dtype=np.uint8).copy())
    if not torch.equal(decode_support(record), support):
        raise AssertionError('Selected mask codec changed support membership')
    return record


def decode_support(record):
    """The flat bool mask of a record, validated (odie/support_codec.py:77-117)."""
    total, count = _geometry(record)
    encoding = record['encoding']
    if encoding in ('all', 'none'):
        full = encoding == 'all'
        if count != (total if full else 0):
            raise ValueError('Constant mask count mismatch')
        return torch.full((total,), full, dtype=torch.bool)
    payload = record['data']
    if not isinstance(payload, torch.Tensor) or payload.dtype != torch.uint8 or payload.ndim != 1:
        raise ValueError('Mask payload must be a flat uint8 tensor')
    codec = _BY_NAME.get(encoding)
    if codec is None:
        raise ValueError('Unknown support encoding: ' + str(encoding))
    mask = codec.unpack(payload.detach().cpu().numpy().tobytes(), total)
    if int(mask.sum()) != count:
        raise ValueError('Decoded selected count mismatch')
    return torch.from_numpy(mask.astype(bool))


def encode_supports(supports):
    return list(map(encode_support, supports))


def _legacy_supports(artifact, counts):
    bitmaps = artifact['support_bitmaps']
    if len(bitmaps) != len(counts):
        raise ValueError('Legacy bitmap layer count mismatch')
    masks = []
    for bits, count in zip(bitmaps, counts):
        if (type(count) is not int or count < 1 or bits.dtype != torch.uint8 or bits.ndim != 1
                or bits.numel() != _bitmap_bytes(count)):
            raise ValueError('Invalid legacy bitmap')
        values = np.unpackbits(bits.detach().cpu().numpy(), bitorder='little', count=count)
        masks.append(torch.from_numpy(values.astype(bool)))
    return masks


def _layerwise_supports(artifact, counts):
    if artifact.get('support_storage_version') != STORAGE_VERSION:
        raise ValueError('Unsupported support storage version')
    records = artifact['support_encodings']
    if len(records) != len(counts):
        raise ValueError('Encoded layer count mismatch')
    return [decode_support(record) for record in records]


def decode_supports(artifact):
    """Supports of an artifact: its layerwise records, or the legacy packed bitmaps, checked
    against the stored cell counts and the configuration's resolutions
    (odie/support_codec.py:124-148)."""
    counts = artifact['support_num_cells']
    layerwise = 'support_encodings' in artifact
    supports = (_layerwise_supports if layerwise else _legacy_supports)(artifact, counts)
    if [support.numel() for support in supports] != counts:
        raise ValueError('Support sizes differ from checkpoint geometry')
    configuration = artifact['configuration']
    if configuration['representation'] == 'hash_grid':
        expected = []
    else:
        resolutions = configuration.get('resolutions')
        expected = None if resolutions is None else [r * r for r in resolutions]
    if expected is not None and counts != expected:
        raise ValueError('Support sizes differ from model configuration')
    return supports


def restore_support_record(artifact):
    return dict(artifact['support_payload'], supports=decode_supports(artifact))


def support_storage_statistics(encodings):
    """Per-layer storage record (the `support_storage` block of the run's metrics)."""
    layers = []
    for level, record in enumerate(encodings):
        layers.append(dict(level=level, resolution=record['resolution'], selected_count=record['selected_count'],
                           encoding=record['encoding'], bitmap_bytes=_bitmap_bytes(record['num_cells']),
                           payload_bytes=record['data'].numel() if 'data' in record else 0))
    totals = {key: sum(layer[key] for layer in layers) for key in ('bitmap_bytes', 'payload_bytes')}
    return dict(version=STORAGE_VERSION, selection_rule=SELECTION_RULE, layers=layers, **totals)


def _same_bytes(a, b):
    return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


# Entries of an artifact that hold its supports, in either storage (legacy bitmaps or records).
_SUPPORT_ENTRIES = ('support_bitmaps', 'support_encodings', 'support_storage_version')


def _reload_checked(path, supports, *, configuration=None, parameters=None):
    """Loads an artifact just written and checks that nothing changed on the way: its supports
    decode to `supports`, and (when given) its configuration and the bytes of every named
    parameter are the ones written.  Returns the reloaded artifact."""
    reloaded = torch.load(path, map_location='cpu', weights_only=True)
    if configuration is not None and reloaded['configuration'] != configuration:
        raise AssertionError('Saved configuration changed during round trip')
    decoded = decode_supports(reloaded)
    if len(decoded) != len(supports) or not all(torch.equal(a, b) for a, b in zip(supports, decoded)):
        raise AssertionError('Saved supports changed during round trip')
    if parameters is not None:
        stored = reloaded['parameters']
        changed = [name for name, value in parameters.items() if name not in stored or not _same_bytes(value, stored[name])]
        if changed:
            raise AssertionError('Saved weights changed during round trip: ' + ', '.join(changed))
    return reloaded


def compress_checkpoint(source, destination):
    """Rewrite an artifact with its supports as layerwise records (the smallest stream per
    level) and every other entry as it was; the copy is reloaded and checked before the record
    of the rewrite is returned (the keys of odie/support_codec.py:161-188).  Never overwrites."""
    source, destination = Path(source), Path(destination)
    if destination.exists():
        raise FileExistsError(destination)
    artifact = torch.load(source, map_location='cpu', weights_only=True)
    supports = decode_supports(artifact)
    records = encode_supports(supports)
    rewritten = {key: value for key, value in artifact.items() if key not in _SUPPORT_ENTRIES}
    rewritten.update(support_storage_version=STORAGE_VERSION, support_encodings=records)
    destination.parent.mkdir(parents=True, exist_ok=True)
    with destination.open('xb') as stream:        # exclusive: a file that appeared meanwhile is kept
        torch.save(rewritten, stream)
    weights = _reload_checked(destination, supports, parameters=artifact['parameters'])['parameters']
    return {'source': str(source), 'output': str(destination), 'source_bytes': source.stat().st_size,
            'checkpoint_bytes': destination.stat().st_size,
            'fp16_parameter_payload_bytes': sum(w.numel() * w.element_size() for w in weights.values()),
            'support_storage': support_storage_statistics(records), 'roundtrip_verified': True}


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
    """The fp16 model artifact (odie/train.py:207-215): configuration, the layerwise supports,
    the fp16 parameters and the run's counters, verified by reloading."""
    encodings = encode_supports(planes.supports)
    artifact = {'version': ARTIFACT_VERSION, 'configuration': configuration, 'settings': settings or {},
                'support_storage_version': STORAGE_VERSION, 'support_encodings': encodings,
                'support_num_cells': [s.numel() for s in planes.supports],
                'support_payload': support_payload or {}, 'support_metadata': support_metadata or {},
                'parameters': model_parameters(planes, decoder, gate), 'checkpoint': 'latest',
                'epoch': epoch, 'optimizer_steps': optimizer_steps, 'metrics': metrics or {}}
    torch.save(artifact, path)
    _reload_checked(path, planes.supports, configuration=configuration, parameters=artifact['parameters'])
    return support_storage_statistics(encodings)


def read_artifact(path, device='cuda', plane_dims=None, plane_node_caps=None):
    """Model of an artifact: PackedPlanes from its configuration (plane_feature_dimensions and
    cell_caps unless given) and supports with the stored fp16 grid, and the fp16 head weights (as
    fp32 masters) for rows of align16(sum F) columns."""
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
    width = (sum(plane_dims) + 15) // 16 * 16
    decoder = Decoder(weights=parameters['decoder.params'].float().numpy(), device=device, width=width)
    gate = None
    if 'gate.params' in parameters:
        gate = Gate(weights=parameters['gate.params'].float().numpy(), coarse=int(configuration.get(
            'gate_coarse_levels_K', 0)), activation=configuration.get('router_output_activation', 'sigmoid'),
            device=device, features=plane_dims)
    return artifact, planes, decoder, gate
