"""Extract layout goldens from the reference's own run records.

Reads results/**/metrics.json under the reference checkout (default /root/reference) and
writes tests/golden/layout_goldens.json: for every run, the resolved configuration numbers
(resolutions, per-level node caps, feature dims, head parameter counts, HashGrid encoding)
and the per-level storage layout the reference recorded (plane offsets, native plane
points, node-index words, direct addressing).  Data only; no reference code is copied.
"""
import json
from pathlib import Path
import sys

ROOT = Path(sys.argv[1] if len(sys.argv) > 1 else '/root/reference')
OUT = Path(__file__).resolve().parent / 'layout_goldens.json'
CONFIG_KEYS = ('representation', 'n_levels', 'base_resolution', 'max_resolution', 'resolutions', 'cell_caps',
               'plane_feature_dimensions', 'gate_parameters', 'decoder_parameters', 'allocated_parameters',
               'parameter_budget', 'router_enabled', 'full_cover_coarse_layers', 'hash_encoding')
LEVEL_KEYS = ('level', 'resolution', 'plane_dim', 'allowed_cells', 'plane_retained_nodes', 'plane_node_capacity',
              'native_plane_points', 'plane_offset', 'feature_offset', 'node_index_words', 'direct_node_access')
STORAGE_KEYS = ('grid_params', 'gate_params', 'decoder_params', 'node_bitmap_bytes', 'node_prefix_bytes',
                'bitmap_bytes', 'descriptor_bytes', 'input_width')

runs = {}
for path in sorted((ROOT / 'results').rglob('metrics.json')):
    record = json.loads(path.read_text())
    training = record.get('training', {})
    config = training.get('configuration')
    if not config:
        continue
    entry = {'config': {k: config[k] for k in CONFIG_KEYS if k in config},
             'source': str(path.relative_to(ROOT))}
    storage = training.get('storage')
    if storage and 'levels' in storage:
        entry['storage'] = {k: storage[k] for k in STORAGE_KEYS if k in storage}
        entry['levels'] = [{k: level[k] for k in LEVEL_KEYS if k in level} for level in storage['levels']]
    runs[str(path.parent.relative_to(ROOT / 'results'))] = entry
OUT.write_text(json.dumps(runs, sort_keys=True))
print('wrote', OUT, len(runs), 'runs')
