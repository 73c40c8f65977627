"""The no-on-demand model (odie/hash_grid.py:8-80): every level of a 2D hash grid trained, with
the decoder and, when the router is on, the gate head, on this library's kernels.

HashGrid takes the reference's constructor arguments and refuses what it refuses.  Its table
`grid` is the fp32 master of all levels (tiny-cuda-nn keeps fp32 parameters and queries an fp16
copy), laid out as the encoding's levels of n_features_per_level values per entry; `gate` /
`decoder` are Gate / Decoder with fp32 masters in `params`, so NativeOptimizer reads this model
through the attributes the reference's optimizer reads.  forward(coordinates) is the evaluation
path (odie/hash_grid.py:52-61): encode, pad the feature row with ones to align16 columns, gate
the levels, decode, first 3 outputs as fp32 -- without autograd; training goes through
NativeOptimizer or ExpertTrainer.
"""
from copy import deepcopy

import numpy as np
import torch

from . import synth
from .config import grid_levels
from .encoding import grid_forward
from .model import decode_rows, head_storage, heads_match, make_heads


class HashGrid:
    def __init__(self, config, supports, plane_dims, plane_node_caps, device='cuda'):
        if supports or config['initial_active_prefix'] != config['n_levels']:
            raise ValueError('HashGrid requires no supports and all levels active')
        self.config = deepcopy(config)
        encoding = config['hash_encoding']
        self.router_enabled = bool(config['router_enabled'])
        self.n_levels = self.active_prefix = int(config['n_levels'])
        self.gate_coarse_levels_K = int(config['gate_coarse_levels_K'])
        self.features_per_level = int(encoding.get('n_features_per_level', 2))
        self.plane_dims, self.plane_node_caps = list(plane_dims), list(plane_node_caps)
        self.input_width = sum(self.plane_dims)
        self.supports = []
        if self.plane_dims != [self.features_per_level] * self.n_levels or int(encoding['n_levels']) != self.n_levels:
            raise ValueError('HashGrid levels must carry the encoding\'s features per level')
        self.levels, entries = grid_levels(encoding)
        # the per-level view the optimizer slices (plane_offset / capacity / dim), in table order
        offsets = np.concatenate([[0], np.cumsum(np.multiply(self.plane_dims, self.plane_node_caps))])
        self.layout = dict(levels=[dict(plane_offset=int(start), plane_node_capacity=cap, plane_dim=dim)
                                   for start, cap, dim in zip(offsets, self.plane_node_caps, self.plane_dims)])
        self.gate, self.decoder = make_heads(config, self.plane_dims, self.router_enabled,
                                             self.gate_coarse_levels_K, device)
        if self.features_per_level * entries != int(offsets[-1]) or not heads_match(config, self.gate, self.decoder):
            raise RuntimeError('Actual TCNN allocation differs from the reference HashGrid budget')
        # tiny-cuda-nn's grid initialisation: uniform in +-1e-4, here from the counter PRNG
        u = synth.uniform(int(config['seed']), 'hash_grid', int(offsets[-1])).astype(np.float64)
        self.grid = torch.from_numpy(((2.0 * u - 1.0) * 1e-4).astype(np.float32)).to(device)

    def set_active_prefix(self, prefix):
        if prefix != self.n_levels:
            raise ValueError('The no-on-demand model always trains every level')

    def forward(self, coordinates):
        """RGB fp32 [n, 3] at coordinates fp32 [n, 2] in [0, 1]^2, from the current fp32 masters
        (each call rounds them to fp16 as tiny-cuda-nn's modules do)."""
        with torch.no_grad():
            raw = grid_forward(coordinates, self.grid.half(), self.levels, self.features_per_level)
            return decode_rows(raw, self.gate, self.decoder)

    __call__ = forward

    def storage_stats(self):
        counts, bytes_ = head_storage(self.grid.numel(), self.gate, self.decoder)
        stats = dict(counts, router_enabled=self.router_enabled, axis_params=0, plane_params=counts['grid_params'],
                     plane_caps=self.plane_node_caps, **bytes_, full_gradient_bytes=2 * counts['actual_params'],
                     index_bytes=0, node_bitmap_bytes=0, node_prefix_bytes=0, bitmap_bytes=0,
                     runtime_index_bytes=None, input_width=self.input_width,
                     active_layers_from_update1=self.n_levels, active_prefix=self.n_levels,
                     full_cover_coarse_layers=list(range(self.n_levels)), plane_dims=self.plane_dims,
                     coordinate_version='unit-endpoints-v1', layout_version='official-tcnn-hash-grid-v1',
                     addressing_version='official-tcnn-hash-grid',
                     initialization='TCNN distributions from a counter PRNG (grid uniform +-1e-4)')
        stats['levels'] = [dict(level=level, resolution=resolution, **item) for level, (resolution, item)
                           in enumerate(zip(self.config['resolutions'], self.layout['levels']))]
        return stats
