"""The no-on-demand model (odie/hash_grid.py:8-80): every level of a 2D hash grid trained, the
decoder and, with a router, the gate head, on this library's kernels.

HashGrid takes the reference's constructor arguments and refuses what it refuses
(odie/hash_grid.py:10-11,41-43).  `grid` is the fp32 master table (tiny-cuda-nn keeps its
parameters in fp32 and queries an fp16 copy of them), `gate` / `decoder` are Gate / Decoder
with fp32 masters in `params`, so NativeOptimizer reads the model through the attributes the
reference's optimizer reads.  forward(coordinates) is the reference's evaluation path
(odie/hash_grid.py:52-61): encode, gate the levels, decode, first 3 outputs as fp32.  It runs the
kernels without autograd: training goes through NativeOptimizer (or ExpertTrainer).
"""
from copy import deepcopy

import numpy as np
import torch

from . import synth
from .config import grid_levels
from .decoder import Decoder, LEVELS, PARAMETERS as DECODER_PARAMETERS
from .encoding import grid_forward
from .gate import Gate, PARAMETERS as GATE_PARAMETERS

# tiny-cuda-nn's seeds for the two heads (odie/hash_grid.py:28,33)
GATE_SEED, DECODER_SEED = 2000003, 4000037


class HashGrid:
    def __init__(self, config, supports, plane_dims, plane_node_caps, device='cuda'):
        if supports or config['initial_active_prefix'] != config['n_levels']:
            raise ValueError('HashGrid requires no supports and all levels active')
        self.config = deepcopy(config)
        self.router_enabled = bool(config['router_enabled'])
        self.n_levels = self.active_prefix = int(config['n_levels'])
        self.gate_coarse_levels_K = int(config['gate_coarse_levels_K'])
        self.input_width = sum(plane_dims)
        self.plane_dims, self.plane_node_caps = list(plane_dims), list(plane_node_caps)
        self.supports = []
        encoding = config['hash_encoding']
        if (int(encoding.get('n_features_per_level', 2)) != 2 or self.n_levels != LEVELS or
                list(plane_dims) != [2] * LEVELS):
            raise ValueError('HashGrid runs %d levels of 2 features (the width of the heads)' % LEVELS)
        self.levels, entries = grid_levels(encoding)
        offset, levels = 0, []
        for dim, cap in zip(plane_dims, plane_node_caps):
            levels.append(dict(plane_offset=offset, plane_node_capacity=cap, plane_dim=dim))
            offset += dim * cap
        self.layout = dict(levels=levels)
        gate = GATE_PARAMETERS if self.router_enabled else 0
        if (2 * entries != offset or DECODER_PARAMETERS != config['decoder_parameters'] or
                gate != config['gate_parameters']):
            raise RuntimeError('Actual TCNN allocation differs from the reference HashGrid budget')
        seed = int(config['seed'])
        # tiny-cuda-nn's grid initialisation: uniform in +-1e-4
        table = (synth.uniform(seed, 'hash_grid', 2 * entries).astype(np.float64) * 2.0 - 1.0) * 1e-4
        self.grid = torch.from_numpy(table.astype(np.float32)).to(device)
        self.gate = (Gate(seed=(seed + GATE_SEED) % 2 ** 31, coarse=self.gate_coarse_levels_K,
                          activation=config['router_output_activation'], device=device)
                     if self.router_enabled else None)
        self.decoder = Decoder(seed=(seed + DECODER_SEED) % 2 ** 31, device=device)

    def set_active_prefix(self, prefix):
        if prefix != self.n_levels:
            raise ValueError('The no-on-demand model always trains every level')

    def forward(self, coordinates):
        """RGB fp32 [n, 3] at coordinates fp32 [n, 2] in [0, 1]^2, from the current fp32 masters
        (each call rounds them to fp16 as tiny-cuda-nn's modules do)."""
        with torch.no_grad():
            raw = grid_forward(coordinates, self.grid.half(), self.levels, 2)
            if self.gate is not None:
                self.gate.sync_weights()
                raw, _ = self.gate.forward(raw)
            self.decoder.sync_weights()
            return self.decoder.forward(raw).float()[:, :3]

    __call__ = forward

    def storage_stats(self):
        grid, decoder = self.grid.numel(), self.decoder.params.numel()
        gate = self.gate.params.numel() if self.gate is not None else 0
        heads = gate + decoder
        return dict(actual_params=grid + heads, grid_params=grid, head_params=heads,
                    gate_params=gate, decoder_params=decoder, router_enabled=self.router_enabled,
                    axis_params=0, plane_params=grid, plane_caps=self.plane_node_caps,
                    fp16_parameter_payload_bytes=2 * (grid + heads), fp32_master_bytes=4 * (grid + heads),
                    adam_moment_bytes=8 * (grid + heads), full_gradient_bytes=2 * (grid + heads),
                    index_bytes=0, node_bitmap_bytes=0, node_prefix_bytes=0, bitmap_bytes=0,
                    runtime_index_bytes=None, input_width=self.input_width,
                    active_layers_from_update1=self.n_levels, active_prefix=self.n_levels,
                    full_cover_coarse_layers=list(range(self.n_levels)), plane_dims=self.plane_dims,
                    coordinate_version='unit-endpoints-v1', layout_version='official-tcnn-hash-grid-v1',
                    addressing_version='official-tcnn-hash-grid',
                    initialization='TCNN distributions from a counter PRNG (grid uniform +-1e-4)',
                    levels=[dict(level=i, resolution=r, **item) for i, (r, item) in
                            enumerate(zip(self.config['resolutions'], self.layout['levels']))])
