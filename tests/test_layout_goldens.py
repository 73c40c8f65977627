"""make_layout and the head sizes against the packed layouts the reference recorded for its own
runs (tests/golden/layout_goldens.json: 57 xy_planes runs of results/**/metrics.json -- DIV2K at
16 levels of [2]*15+[1], the 8 / 12 / 20-level ablations, the gigapixel and no-router runs).

Supports are not recorded, only what they lead to; a level the reference addressed directly gets
a full support here, any other a one-cell support, which give the same addressing mode.  Every
field that follows from the resolutions, cell caps and feature dimensions is compared:
plane_offset, feature_offset, native_plane_points, plane_node_capacity, node_index_words,
direct_node_access, the descriptor rows, the storage byte counts of the addressing buffers, the
input width, the grid parameters, and the gate and decoder sizes of the heads (which together
with the grid equal the allocated parameters)."""
import json
from pathlib import Path

import pytest
import torch

from odie_amd.model import DESCRIPTOR_COLUMNS, make_heads, make_layout

RUNS = json.loads((Path(__file__).resolve().parent / 'golden' / 'layout_goldens.json').read_text())
PACKED = sorted(name for name, run in RUNS.items() if run['config'].get('representation') == 'xy_planes')


def test_fixture_holds_the_packed_runs():
    assert len(PACKED) == 57
    assert {len(RUNS[name]['config']['plane_feature_dimensions']) for name in PACKED} == {8, 12, 16, 20}


@pytest.mark.parametrize('name', PACKED)
def test_layout_matches_the_recorded_run(name):
    run = RUNS[name]
    config, recorded = run['config'], run['levels']
    dims, caps, resolutions = config['plane_feature_dimensions'], config['cell_caps'], config['resolutions']
    supports = []
    for level, r in zip(recorded, resolutions):
        support = torch.zeros(r * r, dtype=torch.bool)
        if level['direct_node_access']:
            support[:] = True
        else:
            support[0] = True
        supports.append(support)
    layout_config = dict(config, coarse_levels=0, gate_topology='shared', gate_position='feature',
                         initial_active_prefix=0)
    layout = make_layout(layout_config, supports, dims, caps)
    fields = ('level', 'resolution', 'plane_dim', 'plane_node_capacity', 'native_plane_points', 'plane_offset',
              'feature_offset', 'node_index_words', 'direct_node_access')
    for got, want in zip(layout['levels'], recorded):
        assert {k: got[k] for k in fields} == {k: want[k] for k in fields}, (name, want['level'])
    rows = layout['descriptors'].tolist()
    column = {key: i for i, key in enumerate(DESCRIPTOR_COLUMNS)}
    for row, want in zip(rows, recorded):
        assert row[column['resolution']] == want['resolution'] and row[column['points']] == want['native_plane_points']
        assert row[column['plane_offset']] == want['plane_offset'] and row[column['features']] == want['plane_dim']
        assert row[column['feature_offset']] == want['feature_offset']
        assert row[column['direct']] == int(want['direct_node_access'])
        assert (row[column['node_word_offset']] == -1) == want['direct_node_access']
    storage = run['storage']
    size = lambda t: t.numel() * t.element_size()
    assert size(layout['node_bitmap']) == storage['node_bitmap_bytes']
    assert size(layout['node_prefix']) == storage['node_prefix_bytes']
    assert size(layout['bitmap']) == storage['bitmap_bytes']
    assert size(layout['descriptors']) == storage['descriptor_bytes']
    assert layout['input_width'] == storage['input_width'] and layout['params'] == storage['grid_params']
    gate, decoder = make_heads(dict(config, seed=0), dims, config['router_enabled'], 0, 'cpu')
    gate_size = gate.params.numel() if gate is not None else 0
    assert gate_size == config['gate_parameters'] == storage['gate_params']
    assert decoder.params.numel() == config['decoder_parameters'] == storage['decoder_params']
    assert layout['params'] + gate_size + decoder.params.numel() == config['allocated_parameters']
