"""Packed xy-plane layout and the PackedQuery op (odie/model.py).

make_layout / plane_closure / make_node_index follow odie/model.py:33-118: each level's
retained nodes are the closure {c, c+1, c+R, c+R+1} mod align8(R^2) of its support; a
level whose closure is every node is addressed directly, otherwise through a bitmap of
present nodes (64 per uint64 word, LSB first) and an int32 exclusive per-word prefix of
present-node counts.  Descriptor row: R, points, plane offset, node-word offset (-1 when
direct), cell-bitmap byte offset, F, output feature offset, direct.

The layout is host bookkeeping done at initialization and at each plane activation;
PackedQuery runs the encode on the GPU through libodie_amd.so.
"""
import numpy as np
import torch

from . import _lib

COORDINATE_VERSION = 'unit-endpoints-native-fmaf-half-cell-align8-modulo-v1'
LAYOUT_VERSION = 'packed-xy-only-native-closure-v1'
ADDRESSING_VERSION = 'node-bitmap64-exclusive-prefix32-v1'
INT32_MAX = 2 ** 31 - 1


def align8(value):
    return (int(value) + 7) // 8 * 8


def router_weights(logits, activation):
    if activation == 'sigmoid':
        return torch.sigmoid(logits)
    if activation == 'softplus':
        return torch.nn.functional.softplus(logits, beta=1., threshold=20.)
    raise ValueError('Unknown router activation: ' + activation)


def gate_coarse_levels(config):
    count = int(config.get('gate_coarse_levels_K', config['coarse_levels']))
    if not 0 <= count <= int(config['n_levels']) or int(config['coarse_levels']) != count:
        raise ValueError('Gate K must agree with coarse_levels and remain within declared level count')
    return count


def plane_closure(support, resolution):
    """Sorted unique closure nodes of a flat bool support of R^2 cells (int64)."""
    support = torch.as_tensor(support)
    cells = support.nonzero(as_tuple=True)[0]
    nodes = torch.cat([cells, cells + 1, cells + resolution, cells + resolution + 1])
    return torch.unique(nodes.remainder(align8(resolution ** 2)), sorted=True)


def make_node_index(nodes, points):
    """(uint64 presence bitmap, int32 exclusive per-word prefix) of sorted unique nodes."""
    if not isinstance(points, int) or points <= 0 or points > INT32_MAX:
        raise ValueError('Native node universe must fit positive int32 addressing')
    if nodes.device.type != 'cpu' or nodes.dtype != torch.int64 or nodes.ndim != 1:
        raise ValueError('Nodes must be a flat CPU int64 tensor')
    values = nodes.numpy()
    if values.size and (values[0] < 0 or values[-1] >= points or bool((np.diff(values) <= 0).any())):
        raise ValueError('Nodes must be sorted, unique and inside the native universe')
    words = (points + 63) // 64
    present = np.zeros(words * 64, dtype=np.uint8)
    present[values] = 1
    packed = np.packbits(present.reshape(words, 64), axis=1, bitorder='little')
    bitmap = packed.view('<u8').reshape(words).copy()
    counts = present.reshape(words, 64).sum(1, dtype=np.int64)
    prefix = (np.cumsum(counts) - counts).astype(np.int32)
    return torch.from_numpy(bitmap.view(np.int64)).view(torch.uint64), torch.from_numpy(prefix)


def _cell_bitmap(support, points):
    padded = np.zeros(points, dtype=np.uint8)
    padded[:support.numel()] = support.numpy().astype(np.uint8)
    return torch.from_numpy(np.packbits(padded.reshape(-1, 8), axis=1, bitorder='little').reshape(-1))


def make_layout(config, supports, plane_dims, plane_node_caps):
    resolutions = list(config['resolutions'])
    if not (len(resolutions) == len(supports) == len(plane_dims) == len(plane_node_caps) == int(config['n_levels'])) \
            or not all(f in (1, 2, 4) for f in plane_dims):
        raise ValueError('Require aligned level descriptors and F1/F2/F4 features')
    if config['representation'] != 'xy_planes':
        raise ValueError('XY-only representation is required')
    gate_coarse_levels(config)
    if config['gate_topology'] != 'shared' or config['gate_position'] != 'feature':
        raise ValueError('Preserve the shared feature gate')
    node_bitmaps, prefixes, bitmaps, descriptors, levels, clean = [], [], [], [], [], []
    params = feature_offset = node_word_offset = bitmap_offset = 0
    for level, (resolution, support, dim, cap) in enumerate(zip(resolutions, supports, plane_dims, plane_node_caps)):
        if support.device.type != 'cpu' or support.dtype != torch.bool or support.shape != (resolution ** 2,):
            raise ValueError('Support must be a flat CPU bool R^2 tensor')
        if level < int(config['initial_active_prefix']) and not bool(support.all()):
            raise ValueError('Declared initial full-cover supports must remain full')
        support = support.clone()
        points = align8(resolution ** 2)
        nodes = plane_closure(support, resolution)
        if cap % 8 or not nodes.numel() <= cap <= points:
            raise ValueError('Aligned node capacity must contain the complete interpolation closure')
        if points > INT32_MAX or params + cap * dim > INT32_MAX:
            raise ValueError('Native points and packed offsets must fit int32 addressing')
        direct = nodes.numel() == points
        if direct:
            index_offset, words = -1, 0
        else:
            node_bitmap, prefix = make_node_index(nodes, points)
            index_offset, words = node_word_offset, node_bitmap.numel()
            node_bitmaps.append(node_bitmap)
            prefixes.append(prefix)
            node_word_offset += words
        bitmap = _cell_bitmap(support, points)
        descriptors.append([resolution, points, params, index_offset, bitmap_offset, dim, feature_offset, int(direct)])
        levels.append({'level': level, 'resolution': resolution, 'plane_dim': dim,
                       'allowed_cells': int(support.sum()), 'plane_retained_nodes': nodes.numel(),
                       'plane_node_capacity': cap, 'plane_unused_slots': cap - nodes.numel(),
                       'native_plane_points': points, 'plane_offset': params,
                       'feature_offset': feature_offset, 'nodes': nodes,
                       'node_index_words': words, 'direct_node_access': direct})
        bitmaps.append(bitmap)
        clean.append(support)
        params += cap * dim
        feature_offset += dim
        bitmap_offset += bitmap.numel()
    return {'descriptors': torch.tensor(descriptors, dtype=torch.int32),
            'node_bitmap': torch.cat(node_bitmaps) if node_bitmaps else torch.empty(0, dtype=torch.uint64),
            'node_prefix': torch.cat(prefixes) if prefixes else torch.empty(0, dtype=torch.int32),
            'bitmap': torch.cat(bitmaps), 'levels': levels, 'supports': clean,
            'params': params, 'input_width': feature_offset}


def _device_layout(tensor):
    return tensor if tensor.numel() else torch.zeros(1, dtype=tensor.dtype, device=tensor.device)


def packed_forward(coordinates, grid, descriptors, node_bitmap, node_prefix, bitmap, width):
    """(features fp16 [N, width], visibility bool [N, L]) -- odie/packed_kernels.cu:107-125."""
    if coordinates.dtype != torch.float32 or coordinates.ndim != 2 or coordinates.shape[1] != 2:
        raise ValueError('coordinates must be CUDA contiguous FP32 Nx2')
    if grid.dtype != torch.float32 or grid.ndim != 1:
        raise ValueError('grid must be flat CUDA FP32')
    coordinates, grid = coordinates.contiguous(), grid.contiguous()
    n, levels = coordinates.shape[0], descriptors.shape[0]
    features = torch.empty((n, width), dtype=torch.float16, device=coordinates.device)
    visibility = torch.empty((n, levels), dtype=torch.bool, device=coordinates.device)
    _lib.check(_lib.library().odie_packed_forward(
        coordinates.data_ptr(), n, grid.data_ptr(), grid.numel(), descriptors.data_ptr(), levels,
        _device_layout(node_bitmap).data_ptr(), _device_layout(node_prefix).data_ptr(), bitmap.data_ptr(), width,
        features.data_ptr(), visibility.data_ptr(), _lib.stream_of(coordinates)))
    return features, visibility


def packed_backward(coordinates, upstream, descriptors, node_bitmap, node_prefix, bitmap, parameter_count):
    """fp32 gradient [parameter_count] -- odie/packed_kernels.cu:127-145."""
    if upstream.dtype != torch.float16 or upstream.ndim != 2 or upstream.shape[0] != coordinates.shape[0]:
        raise ValueError('upstream must be CUDA contiguous FP16 NxF')
    upstream = upstream.contiguous()
    gradient = torch.empty(parameter_count, dtype=torch.float32, device=coordinates.device)
    _lib.check(_lib.library().odie_packed_backward(
        coordinates.data_ptr(), coordinates.shape[0], upstream.data_ptr(), upstream.shape[1],
        descriptors.data_ptr(), descriptors.shape[0], _device_layout(node_bitmap).data_ptr(),
        _device_layout(node_prefix).data_ptr(), bitmap.data_ptr(), gradient.data_ptr(), parameter_count,
        _lib.stream_of(coordinates)))
    return gradient


class PackedQuery(torch.autograd.Function):
    """Same contract as odie/model.py:137-151."""

    @staticmethod
    def forward(ctx, coordinates, grid, descriptors, node_bitmap, node_prefix, bitmap, width):
        features, visible = packed_forward(coordinates, grid, descriptors, node_bitmap, node_prefix, bitmap, width)
        ctx.save_for_backward(coordinates, descriptors, node_bitmap, node_prefix, bitmap)
        ctx.param_count = grid.numel()
        ctx.mark_non_differentiable(visible)
        return features, visible

    @staticmethod
    def backward(ctx, feature_gradient, visibility_gradient):
        coordinates, descriptors, node_bitmap, node_prefix, bitmap = ctx.saved_tensors
        gradient = packed_backward(coordinates, feature_gradient.contiguous(), descriptors, node_bitmap,
                                   node_prefix, bitmap, ctx.param_count)
        return None, gradient, None, None, None, None, None


class PackedPlanes:
    """The packed xy-plane grid of PackedXYPlanes (odie/model.py:154-262) without its TCNN heads:
    fp32 master `grid` in packed storage, the layout's addressing buffers on the device, the
    active prefix, and the activation of the next plane's support.

    Plane values are inputs of the path (odie/model.py:208-224 draws them from a CUDA generator
    stream); here a plane's native nodes draw N(0, feature_init_std) from the counter PRNG of
    odie_amd.synth under the same per-level seed, so a plane is initialized exactly once and
    identically on every machine.
    """

    def __init__(self, config, supports, plane_dims, plane_node_caps, device='cuda'):
        self.config = dict(config)
        self.layout = make_layout(self.config, supports, plane_dims, plane_node_caps)
        self.supports = self.layout['supports']
        self.plane_dims, self.plane_node_caps = list(plane_dims), list(plane_node_caps)
        self.n_levels = int(self.config['n_levels'])
        self.input_width = self.layout['input_width']
        self.device = torch.device(device)
        self.grid = torch.zeros(self.layout['params'], dtype=torch.float32, device=self.device)
        self.initialized_planes = [False] * self.n_levels
        for level, item in enumerate(self.layout['levels']):
            if item['nodes'].numel():
                self._initialize_plane(level)
        self._upload(self.layout)
        self.active_prefix = int(self.config.get('initial_active_prefix', self.n_levels))

    def _upload(self, layout):
        for name in ('descriptors', 'node_bitmap', 'node_prefix', 'bitmap'):
            setattr(self, name, _device_layout(layout[name]).to(self.device))

    @torch.no_grad()
    def _initialize_plane(self, level):
        from . import synth
        if self.initialized_planes[level]:
            raise RuntimeError('Each plane must be initialized exactly once')
        item = self.layout['levels'][level]
        level_seed = (self.config['seed'] + 1000003 * (level + 1)) % (2 ** 31)
        branch_seed = (level_seed + 104729 * 3) % (2 ** 31)
        width = max(2, item['plane_dim'])
        draws = synth.normal(branch_seed, 'plane', item['native_plane_points'] * width).reshape(-1, width)
        nodes = item['nodes'].numpy()
        values = (draws[nodes, :item['plane_dim']] * float(self.config['feature_init_std'])).astype(np.float32)
        offset = item['plane_offset']
        self.grid[offset:offset + values.size].copy_(torch.from_numpy(values.reshape(-1)))
        self.initialized_planes[level] = True

    @torch.no_grad()
    def activate_support(self, level, support):
        """Add only the next unopened plane, retaining packed storage and offsets
        (odie/model.py:226-257): same checks, same record."""
        if level != self.active_prefix or not 2 <= level < self.n_levels:
            raise ValueError('Select the next unopened plane before advancing the prefix')
        if self.initialized_planes[level] or bool(self.supports[level].any()):
            raise RuntimeError('An opened support cannot be replaced or initialized again')
        resolution = self.config['resolutions'][level]
        if support.device.type != 'cpu' or support.dtype != torch.bool or support.shape != (resolution ** 2,):
            raise ValueError('New support must be a flat CPU bool R^2 tensor')
        nodes = plane_closure(support, resolution)
        cap = self.plane_node_caps[level]
        if not 0 < nodes.numel() <= cap:
            raise ValueError('New support requires a nonempty complete closure within its cap')
        storage_pointer = self.grid.data_ptr()
        updated = list(self.supports)
        updated[level] = support.clone()
        layout = make_layout(self.config, updated, self.plane_dims, self.plane_node_caps)
        self._upload(layout)
        self.layout, self.supports = layout, layout['supports']
        points = layout['levels'][level]['native_plane_points']
        self._initialize_plane(level)
        if self.grid.data_ptr() != storage_pointer:
            raise AssertionError('Packed storage changed during plane activation')
        return {'level': level, 'initialized_once': True, 'grid_storage_unchanged': True,
                'original_dense_f2_seed': (self.config['seed'] + 1000003 * (level + 1) + 104729 * 3) % (2 ** 31),
                'native_dense_draw_shape': [points, max(2, self.plane_dims[level])], 'selected_nodes': nodes.numel()}

    def set_active_prefix(self, prefix):
        if not isinstance(prefix, int) or not 2 <= prefix <= self.n_levels:
            raise ValueError('Active prefix must be an integer between 2 and declared level count')
        self.active_prefix = prefix

    def query_features(self, coordinates):
        """(features fp16 [N, input_width], visibility bool [N, L]) through PackedQuery."""
        if coordinates.dtype != torch.float32 or coordinates.ndim != 2 or coordinates.shape[1] != 2 \
                or coordinates.requires_grad:
            raise ValueError('Coordinates must be FP32 Nx2, without coordinate gradients')
        return PackedQuery.apply(coordinates.contiguous(), self.grid, self.descriptors, self.node_bitmap,
                                 self.node_prefix, self.bitmap, self.input_width)


# tiny-cuda-nn's seeds for the two heads (odie/model.py:191-193)
GATE_SEED, DECODER_SEED = 2000003, 4000037


class PackedXYPlanes(PackedPlanes):
    """The on-demand model (odie/model.py:154-262): the packed planes with the router gate and the
    decoder (Gate / Decoder, fp32 masters in `params`), 16 levels of 2 features (the width this
    library's heads and runtime are built for).  forward(coordinates) is the reference's
    evaluation path (odie/model.py:266-279): query, mask the levels past the active prefix, gate
    by level with visibility, decode, first 3 outputs as fp32; it runs without autograd, training
    goes through NativeOptimizer."""

    def __init__(self, config, supports, plane_dims, plane_node_caps, axis_mode='none', kernel_a=0.,
                 kernel_omega=1.5 * np.pi, device='cuda'):
        if axis_mode != 'none' or kernel_a != 0.:
            raise ValueError('No axis branches or non-linear interpolation kernel in this ablation')
        from .decoder import Decoder, LEVELS, PARAMETERS as DECODER_PARAMETERS
        if list(plane_dims) != [2] * LEVELS or int(config['n_levels']) != LEVELS:
            raise ValueError('PackedXYPlanes runs %d levels of 2 features (the width of the heads)' % LEVELS)
        super().__init__(config, supports, plane_dims, plane_node_caps, device=device)
        from .gate import Gate, PARAMETERS as GATE_PARAMETERS
        self.router_enabled = bool(config.get('router_enabled', True))
        self.gate_coarse_levels_K = gate_coarse_levels(config)
        seed = int(config['seed'])
        if ((GATE_PARAMETERS if self.router_enabled else 0) != config['gate_parameters'] or
                DECODER_PARAMETERS != config['decoder_parameters']):
            raise RuntimeError('Unexpected TCNN head allocation for the configured input width')
        self.gate = (Gate(seed=(seed + GATE_SEED) % 2 ** 31, coarse=self.gate_coarse_levels_K,
                          activation=config.get('router_output_activation', 'sigmoid'), device=device)
                     if self.router_enabled else None)
        self.decoder = Decoder(seed=(seed + DECODER_SEED) % 2 ** 31, device=device)

    def forward(self, coordinates):
        with torch.no_grad():
            raw, visible = self.query_features(coordinates)
            level = torch.arange(self.n_levels, device=raw.device)
            active = level < self.active_prefix
            raw = raw * active.repeat_interleave(2).to(raw.dtype)
            self.decoder.sync_weights()
            if self.gate is None:
                return self.decoder.forward(raw).float()[:, :3]
            self.gate.sync_weights()
            # levels at or below K keep a gate of one; a prefix within them gates nothing else
            weighted, _ = self.gate.forward(raw, visible=(visible & active).to(torch.uint8).contiguous())
            return self.decoder.forward(weighted).float()[:, :3]

    __call__ = forward

    def storage_stats(self):
        grid = self.grid.numel()
        gate = self.gate.params.numel() if self.gate is not None else 0
        heads = gate + self.decoder.params.numel()
        size = lambda t: t.numel() * t.element_size()
        node_bitmaps, prefixes, bitmaps = size(self.node_bitmap), size(self.node_prefix), size(self.bitmap)
        descriptors = size(self.descriptors)
        gate_index = self.input_width * 8                     # the int64 feature -> level index
        active_flags = self.n_levels + 2 * self.input_width   # bool per level, fp16 per feature
        return {'actual_params': grid + heads, 'grid_params': grid, 'head_params': heads,
                'gate_params': gate, 'decoder_params': self.decoder.params.numel(),
                'router_enabled': self.router_enabled, 'axis_params': 0, 'plane_params': grid,
                'plane_caps': self.plane_node_caps, 'fp16_parameter_payload_bytes': 2 * (grid + heads),
                'fp32_master_bytes': 4 * (grid + heads), 'adam_moment_bytes': 8 * (grid + heads),
                'full_gradient_bytes': 4 * (grid + heads), 'index_bytes': node_bitmaps + prefixes,
                'node_bitmap_bytes': node_bitmaps, 'node_prefix_bytes': prefixes, 'bitmap_bytes': bitmaps,
                'descriptor_bytes': descriptors,
                'runtime_index_bytes': node_bitmaps + prefixes + bitmaps + descriptors + gate_index + active_flags,
                'active_flag_bytes': active_flags, 'input_width': self.input_width,
                'native_input_padding': (self.input_width + 15) // 16 * 16, 'axis_mode': 'none',
                'active_layers_from_update1': int(self.config.get('initial_active_prefix', 2)),
                'active_prefix': self.active_prefix, 'gate_coarse_levels_K': self.gate_coarse_levels_K,
                'full_cover_coarse_layers': self.config.get('full_cover_coarse_layers', [0, 1]),
                'plane_dims': self.plane_dims,
                'coordinate_version': COORDINATE_VERSION, 'layout_version': LAYOUT_VERSION,
                'addressing_version': ADDRESSING_VERSION, 'query_cuda_launches': 1, 'backward_cuda_launches': 1,
                'forward_precision': 'P01 FP32 geometry and FP16 interpolation chain',
                'gradient_precision': 'FP16 feature gradient, FP32 interpolation weights and atomicAdd',
                'levels': [{key: value for key, value in level.items() if key != 'nodes'}
                           for level in self.layout['levels']]}


def build_model(config, supports, plane_dims, plane_node_caps, **kwargs):
    """The model of config['representation'] (odie/model.py:318-321)."""
    if config['representation'] == 'hash_grid':
        from .hash_grid import HashGrid
        return HashGrid(config, supports, plane_dims, plane_node_caps)
    return PackedXYPlanes(config, supports, plane_dims, plane_node_caps, **kwargs)
