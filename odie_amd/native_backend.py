"""The persistent native optimizer: the reference's NativeOptimizer (odie/native_backend.py:23-136)
over this library's odie_* runtime (include/odie_amd.h), with a HIP graph recaptured whenever
the active prefix or a learning rate changes.

The model is read as the reference reads it (odie/native_backend.py:47-73): `grid` (fp32
master), `decoder.params` and `gate.params` (fp32 masters, gate None without a router),
`active_prefix`, and for packed planes `descriptors`, `node_bitmap`, `node_prefix`, `bitmap`
and `layout`.  NativeModel assembles such a model from PackedPlanes (or a hash-grid table),
a Decoder and a Gate.  What the reference fixes when it compiles its library (level count,
feature width, router, target storage, K, activation; odie/build.py:26-30) is passed as
settings instead.
"""
import json

import torch

from . import _lib

BATCH = 65536


class PlaneState:
    """Per-plane view of the grid's Adam state: {} while pristine (odie/native_backend.py:7-20)."""

    def __init__(self, backend, planes):
        self.backend = backend
        self.ranges = {}
        offset = 0
        for plane in planes:
            self.ranges[plane] = (offset, offset + plane.numel())
            offset += plane.numel()

    def get(self, plane, default=None):
        if plane not in self.ranges:
            return default
        value = self.backend.state_summary(*self.ranges[plane])
        return {} if value['pristine'] else {'native_adam_state': True}


class NativeModel:
    """The attributes NativeOptimizer reads.  planes: a PackedPlanes (its packed storage, layout
    and prefix are read live, so activate_support / set_active_prefix show through), or None with
    `grid` an fp32 hash-grid table."""

    def __init__(self, decoder, gate=None, planes=None, grid=None, active_prefix=16):
        if (planes is None) == (grid is None):
            raise ValueError('give packed planes or a hash-grid table')
        self.decoder, self.gate, self.planes = decoder, gate, planes
        self._grid, self._active = grid, int(active_prefix)

    def __getattr__(self, name):
        planes = self.__dict__.get('planes')
        if planes is not None and name in ('descriptors', 'node_bitmap', 'node_prefix', 'bitmap', 'layout'):
            return getattr(planes, name)
        raise AttributeError(name)

    @property
    def grid(self):
        return self.planes.grid if self.planes is not None else self._grid

    @property
    def active_prefix(self):
        return self.planes.active_prefix if self.planes is not None else self._active


def compile_settings(config):
    """The reference's build definitions (odie/build.py:26-30) as runtime settings."""
    levels = int(config['n_levels'])
    raw = int(sum(config['plane_feature_dimensions'])) if 'plane_feature_dimensions' in config else 2 * levels
    return dict(levels=levels, raw_width=raw, rgb8=int(config.get('target_storage', 'uint8') == 'uint8'),
                gate_coarse_levels=int(config.get('gate_coarse_levels_K', 0)),
                router_activation=config.get('router_output_activation', 'sigmoid'))


class NativeOptimizer:
    def __init__(self, model, target, shape, config, planes, half=True):
        self.lib = lib = _lib.library()
        self.build_manifest = dict(definitions=compile_settings(config), library=str(_lib.LIBRARY))
        self.model, self.target, self.config = model, target, config
        self.half = half
        self.graph = self.key = None
        self.recaptures = 0
        self.stream = torch.cuda.current_stream()
        self.param_groups = [dict(name='grid', params=planes, lr=config['grid_lr'])]
        if model.gate is not None:
            self.param_groups.append(dict(name='gate', params=[model.gate.params], lr=config['gate_lr']))
        self.param_groups.append(dict(name='decoder', params=[model.decoder.params], lr=config['decoder_lr']))
        if target.dtype != (torch.uint8 if self.build_manifest['definitions']['rgb8'] else torch.float32) \
                or tuple(target.shape) != (shape[0], shape[1], 3) or not target.is_contiguous():
            raise ValueError('target must be a contiguous [H, W, 3] image of the configured storage')
        settings = dict(stream=self.stream.cuda_stream, total=model.grid.numel(),
                        width=shape[1], height=shape[0], mode=20 if half else 16, warp_limit=128,
                        rgb=target.data_ptr(), grid=model.grid.data_ptr(),
                        decoder=model.decoder.params.data_ptr(),
                        **self.build_manifest['definitions'], **self.current_settings())
        if model.gate is not None:
            settings['gate'] = model.gate.params.data_ptr()
        if config['representation'] == 'hash_grid':
            settings['hash_encoding'] = config['hash_encoding']
        self.handle = lib.odie_create(json.dumps(settings).encode())
        if not self.handle:
            raise RuntimeError(lib.odie_error().decode())
        self.pointers = json.loads(lib.odie_pointers(self.handle))
        self.fixed = torch.zeros(BATCH, device='cuda', dtype=torch.int64)
        self.squares = torch.empty(BATCH, device='cuda', dtype=torch.float32)
        self.state = PlaneState(self, planes)
        self.warmed = False

    def current_settings(self):
        lrs = {g['name'] + '_lr': float(g['lr']) for g in self.param_groups}
        if self.config['representation'] == 'hash_grid':
            return dict(active=self.model.active_prefix, **lrs)
        return dict(active=self.model.active_prefix,
                    **{k: getattr(self.model, k).data_ptr() for k in ('descriptors', 'node_bitmap', 'node_prefix', 'bitmap')},
                    **lrs)

    def check(self, code):
        if code:
            raise RuntimeError(self.lib.odie_error().decode())

    def step_raw(self, ids, update=True):
        if ids.dtype != torch.int64 or not ids.is_cuda or not ids.is_contiguous():
            raise ValueError('ids must be a contiguous CUDA int64 tensor')
        self.check(self.lib.odie_step(self.handle, ids.data_ptr(), ids.numel(), int(update)))

    def copied(self, name, shape, dtype):
        result = torch.empty(shape, device='cuda', dtype=dtype)
        self.check(self.lib.odie_copy(result.data_ptr(), self.pointers[name], result.numel() * result.element_size(),
                                      self.stream.cuda_stream))
        return result

    def release_graph(self):
        torch.cuda.synchronize()
        self.graph = self.key = None
        self.lib.odie_release_contexts(self.handle)

    def prepare_epoch(self):
        """Configure the handle for the current prefix and learning rates and capture one
        65536-id step in a graph (odie/native_backend.py:95-113).  Three dry runs without the
        optimizer size the library's workspace before capture."""
        settings = self.current_settings()
        key = tuple(settings.items())
        if key == self.key:
            return
        self.release_graph()
        self.check(self.lib.odie_configure(self.handle, json.dumps(settings).encode()))
        with torch.cuda.stream(self.stream):
            for _ in range(3):
                self.step_raw(self.fixed, update=False)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=self.stream):
            self.step_raw(self.fixed)
            self.check(self.lib.odie_copy(self.squares.data_ptr(), self.pointers['squares'], BATCH * 4,
                                          self.stream.cuda_stream))
        self.lib.odie_pin_contexts(self.handle)
        self.graph, self.key = graph, key
        self.recaptures += 1

    def train_batch(self, ids):
        """One step; returns the batch's mean squared error (float64 tensor).  A full batch
        replays the captured graph; the mean is taken eagerly after the replay."""
        if ids.numel() == BATCH and self.graph is not None:
            self.fixed.copy_(ids)
            self.graph.replay()
            return self.squares.double().mean()
        self.step_raw(ids)
        self.check(self.lib.odie_copy(self.squares.data_ptr(), self.pointers['squares'], ids.numel() * 4,
                                      self.stream.cuda_stream))
        return self.squares[:ids.numel()].double().mean()

    def sync_weights(self):
        self.check(self.lib.odie_sync_weights(self.handle))

    def state_summary(self, begin=-1, end=-1):
        data = self.lib.odie_state(self.handle, begin, end)
        if data is None:
            raise RuntimeError(self.lib.odie_error().decode())
        return json.loads(data)

    def native_state_digest(self):
        return json.dumps(self.state_summary(), sort_keys=True)

    def close(self):
        if self.handle:
            self.release_graph()
            self.lib.odie_destroy(self.handle)
            self.handle = None


def make_native_optimizer(model, target, shape, config):
    """Per-level plane views of the packed grid and the optimizer over them
    (odie/native_backend.py:139-142)."""
    planes = [torch.nn.Parameter(model.grid[level['plane_offset']:level['plane_offset'] +
              level['plane_node_capacity'] * level['plane_dim']].detach()) for level in model.layout['levels']]
    return NativeOptimizer(model, target, shape, config, planes), planes
