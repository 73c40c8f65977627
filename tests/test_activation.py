"""Support activation (odie/model.py:226-262) and the selection closure check
(odie/selection.py:76-105) on the host, and a query through the activated plane on the GPU."""
import numpy as np
import pytest
import torch

import oracle
from odie_amd import synth
from odie_amd.model import PackedPlanes, plane_closure
from odie_amd.selection import closure_nodes, selection_record

RESOLUTIONS = [8, 13, 20, 32, 51]


def _planes(device):
    supports = [torch.ones(r * r, dtype=torch.bool) if level < 3 else torch.zeros(r * r, dtype=torch.bool)
                for level, r in enumerate(RESOLUTIONS)]
    caps = [(r * r + 7) // 8 * 8 for r in RESOLUTIONS]
    caps[4] = 400
    config = dict(resolutions=RESOLUTIONS, n_levels=5, representation='xy_planes', coarse_levels=0,
                  gate_topology='shared', gate_position='feature', initial_active_prefix=3, seed=7,
                  feature_init_std=1e-2)
    return PackedPlanes(config, supports, [2, 2, 2, 1, 4], caps, device=device)


def _support(r, fraction, seed):
    return torch.from_numpy(synth.uniform(seed, 'support', r * r) < fraction)


def test_activation_checks_and_record():
    planes = _planes('cpu')
    assert planes.initialized_planes == [True, True, True, False, False]
    with pytest.raises(ValueError, match='next unopened plane'):
        planes.activate_support(4, _support(51, 0.1, 1))
    with pytest.raises(ValueError, match='flat CPU bool'):
        planes.activate_support(3, torch.zeros(31 * 31, dtype=torch.bool))
    with pytest.raises(ValueError, match='nonempty complete closure'):
        planes.activate_support(3, torch.zeros(32 * 32, dtype=torch.bool))
    before = planes.grid.data_ptr()
    support = _support(32, 0.2, 2)
    record = planes.activate_support(3, support)
    assert record['level'] == 3 and record['initialized_once'] and record['grid_storage_unchanged']
    assert record['selected_nodes'] == plane_closure(support, 32).numel()
    assert record['native_dense_draw_shape'] == [1024, 2]
    assert planes.grid.data_ptr() == before
    assert planes.layout['levels'][3]['plane_retained_nodes'] == record['selected_nodes']
    with pytest.raises(RuntimeError, match='cannot be replaced'):
        planes.set_active_prefix(3)
        planes.activate_support(3, support)
    planes.set_active_prefix(4)
    with pytest.raises(ValueError, match='within its cap'):
        planes.activate_support(4, torch.ones(51 * 51, dtype=torch.bool))   # closure 2608 > cap 400
    with pytest.raises(ValueError, match='Active prefix'):
        planes.set_active_prefix(6)


def test_selection_record_checks_closure():
    selected = np.zeros(64, dtype=bool)
    selected[[0, 9, 63]] = True
    nodes = np.zeros(64, dtype=bool)
    nodes[closure_nodes(np.flatnonzero(selected), 8)] = True
    record = selection_record(selected, nodes, 8, 16, 'B2', 3)
    assert record['closure_nodes'] == int(nodes.sum()) and record['selected_cells'] == 3
    assert np.array_equal(closure_nodes([63], 8), oracle.closure_nodes([63], 8))
    nodes[5] = not nodes[5]
    with pytest.raises(AssertionError, match='closure'):
        selection_record(selected, nodes, 8, 16, 'B2', 3)


@pytest.mark.gpu
def test_activated_plane_queries_match_oracle():
    planes = _planes('cuda')
    planes.activate_support(3, _support(32, 0.25, 3))
    xy = synth.coordinates(21, 5000)
    features, visible = planes.query_features(torch.from_numpy(xy).cuda())
    host = {k: planes.layout[k].numpy() for k in ('descriptors', 'node_bitmap', 'node_prefix', 'bitmap')}
    expected, vis = oracle.packed_forward(xy, planes.grid.cpu().numpy(), host, planes.input_width)
    assert np.array_equal(features.cpu().numpy().view(np.uint16), expected.view(np.uint16))
    assert np.array_equal(visible.cpu().numpy(), vis)
    assert vis[:, 3].any() and not vis[:, 3].all() and not vis[:, 4].any()
