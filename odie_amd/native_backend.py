"""The persistent native optimizer over this library's odie_* runtime (include/odie_amd.h), with
the interface of the reference's NativeOptimizer (odie/native_backend.py:23-142): the same
constructor, settings keys, graph recapture on a change of prefix or learning rate, per-plane
state view and state digest.

Structure: _Runtime owns one odie_* handle and turns its -1 / odie_error() convention into
exceptions; NativeOptimizer keeps the settings the handle was configured with and one captured
HIP graph of a full 65536-id step for them; PlaneState answers "has this plane's Adam state
been touched" per plane.  What the reference fixes when it compiles its runtime (level count,
feature width, router, target storage, K, activation; odie/build.py:26-30) is passed to the
handle as settings instead (compile_settings).

The model is read through the attributes the reference reads: `grid`, `decoder.params`,
`gate.params` (gate None without a router), `active_prefix`, and for packed planes
`descriptors`, `node_bitmap`, `node_prefix`, `bitmap` and `layout`.  NativeModel assembles
such a model from PackedPlanes (or a hash-grid table), a Decoder and a Gate.
"""
from itertools import accumulate
import json

import torch

from . import _lib

BATCH = 65536
PACKED_BUFFERS = ('descriptors', 'node_bitmap', 'node_prefix', 'bitmap')


class _Runtime:
    """One odie_* handle; every failing call raises RuntimeError with odie_error()."""

    def __init__(self, lib, settings):
        self.lib = lib
        self.handle = lib.odie_create(json.dumps(settings).encode())
        if not self.handle:
            raise RuntimeError(self.message())

    def message(self):
        return self.lib.odie_error().decode()

    def check(self, code):
        if code:
            raise RuntimeError(self.message())

    def step(self, ids, update):
        self.check(self.lib.odie_step(self.handle, ids.data_ptr(), ids.numel(), int(update)))

    def configure(self, settings):
        self.check(self.lib.odie_configure(self.handle, json.dumps(settings).encode()))

    def pointers(self):
        return json.loads(self.lib.odie_pointers(self.handle))

    def state(self, begin, end):
        reply = self.lib.odie_state(self.handle, begin, end)
        if reply is None:
            raise RuntimeError(self.message())
        return json.loads(reply)

    def copy(self, destination, source, count, stream):
        self.check(self.lib.odie_copy(destination, source, count, stream))

    def destroy(self):
        if self.handle:
            self.lib.odie_destroy(self.handle)
            self.handle = None


class PlaneState:
    """Adam state of each grid plane as the training loop reads it (odie/native_backend.py:7-20):
    get(plane) is {} while the runtime's moments and ages over the plane's parameters are all
    zero, {'native_adam_state': True} once any is not; planes it does not hold give `default`."""

    def __init__(self, backend, planes):
        self.backend = backend
        self._planes = list(planes)
        ends = list(accumulate(plane.numel() for plane in self._planes))
        self._bounds = list(zip([0] + ends[:-1], ends))

    @property
    def ranges(self):
        return dict(zip(self._planes, self._bounds))

    def get(self, plane, default=None):
        found = [bounds for candidate, bounds in zip(self._planes, self._bounds) if candidate is plane]
        if not found:
            return default
        return {'native_adam_state': True} if not self.backend.state_summary(*found[0])['pristine'] else {}


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
        if planes is not None and name in PACKED_BUFFERS + ('layout',):
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
    dims = config.get('plane_feature_dimensions')
    return dict(levels=levels, raw_width=int(sum(dims)) if dims is not None else 2 * levels,
                rgb8=int(config.get('target_storage', 'uint8') == 'uint8'),
                gate_coarse_levels=int(config.get('gate_coarse_levels_K', 0)),
                router_activation=config.get('router_output_activation', 'sigmoid'))


class NativeOptimizer:
    def __init__(self, model, target, shape, config, planes, half=True):
        self.lib = _lib.library()
        definitions = compile_settings(config)
        self.build_manifest = dict(definitions=definitions, library=str(_lib.LIBRARY))
        self.model, self.target, self.config, self.half = model, target, config, half
        self.graph = self.key = None
        self.recaptures = 0
        self.warmed = False
        self.stream = torch.cuda.current_stream()
        groups = [('grid', planes)]
        if model.gate is not None:
            groups.append(('gate', [model.gate.params]))
        groups.append(('decoder', [model.decoder.params]))
        self.param_groups = [dict(name=name, params=params, lr=config[name + '_lr']) for name, params in groups]
        storage = torch.uint8 if definitions['rgb8'] else torch.float32
        if target.dtype != storage or tuple(target.shape) != (shape[0], shape[1], 3) or not target.is_contiguous():
            raise ValueError('target must be a contiguous [H, W, 3] image of the configured storage')
        settings = dict(stream=self.stream.cuda_stream, total=model.grid.numel(), width=shape[1], height=shape[0],
                        mode=20 if half else 16, warp_limit=128, rgb=target.data_ptr(), grid=model.grid.data_ptr(),
                        decoder=model.decoder.params.data_ptr(), **definitions, **self.current_settings())
        if model.gate is not None:
            settings['gate'] = model.gate.params.data_ptr()
        if config['representation'] == 'hash_grid':
            settings['hash_encoding'] = config['hash_encoding']
        self.runtime = _Runtime(self.lib, settings)
        self.handle = self.runtime.handle
        self.pointers = self.runtime.pointers()
        self.fixed = torch.zeros(BATCH, device='cuda', dtype=torch.int64)
        self.squares = torch.empty(BATCH, device='cuda', dtype=torch.float32)
        self.state = PlaneState(self, planes)

    def current_settings(self):
        """What odie_configure takes: the active prefix, the learning rates and, for packed planes,
        the addresses of the live layout buffers."""
        settings = dict(active=self.model.active_prefix)
        if self.config['representation'] != 'hash_grid':
            settings.update((name, getattr(self.model, name).data_ptr()) for name in PACKED_BUFFERS)
        settings.update((group['name'] + '_lr', float(group['lr'])) for group in self.param_groups)
        return settings

    def check(self, code):
        self.runtime.check(code)

    def step_raw(self, ids, update=True):
        if ids.dtype != torch.int64 or not ids.is_cuda or not ids.is_contiguous():
            raise ValueError('ids must be a contiguous CUDA int64 tensor')
        self.runtime.step(ids, update)

    def copied(self, name, shape, dtype):
        """A copy of one of the handle's buffers (odie_pointers) as a new tensor."""
        result = torch.empty(shape, device='cuda', dtype=dtype)
        self.runtime.copy(result.data_ptr(), self.pointers[name], result.numel() * result.element_size(),
                          self.stream.cuda_stream)
        return result

    def _fetch_squares(self, count):
        self.runtime.copy(self.squares.data_ptr(), self.pointers['squares'], count * 4, self.stream.cuda_stream)

    def release_graph(self):
        torch.cuda.synchronize()
        self.graph = self.key = None
        self.lib.odie_release_contexts(self.handle)

    def prepare_epoch(self):
        """Configure the handle for the current prefix and learning rates, then capture one
        65536-id step in a graph (odie/native_backend.py:95-113); nothing happens when they are
        unchanged.  Three dry runs without the optimizer size the library's workspace first."""
        settings = self.current_settings()
        key = tuple(sorted(settings.items()))
        if key == self.key:
            return
        self.release_graph()
        self.runtime.configure(settings)
        with torch.cuda.stream(self.stream):
            for _ in range(3):
                self.step_raw(self.fixed, update=False)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=self.stream):
            self.step_raw(self.fixed)
            self._fetch_squares(BATCH)
        self.lib.odie_pin_contexts(self.handle)
        self.graph, self.key = graph, key
        self.recaptures += 1

    def train_batch(self, ids):
        """One step; returns the batch's mean squared error (float64 tensor).  A full batch
        replays the captured graph; the mean is taken eagerly after it."""
        count = ids.numel()
        if count == BATCH and self.graph is not None:
            self.fixed.copy_(ids)
            self.graph.replay()
        else:
            self.step_raw(ids)
            self._fetch_squares(count)
        return self.squares[:count].double().mean()

    def sync_weights(self):
        self.check(self.lib.odie_sync_weights(self.handle))

    def state_summary(self, begin=-1, end=-1):
        return self.runtime.state(begin, end)

    def native_state_digest(self):
        return json.dumps(self.state_summary(), sort_keys=True)

    def close(self):
        if self.runtime.handle:
            self.release_graph()
            self.runtime.destroy()
            self.handle = None


def make_native_optimizer(model, target, shape, config):
    """Per-level views of the packed grid (each plane's capacity times its features) and the
    optimizer over them (odie/native_backend.py:139-142)."""
    def view(level):
        start = level['plane_offset']
        return torch.nn.Parameter(model.grid[start:start + level['plane_node_capacity'] * level['plane_dim']].detach())
    planes = [view(level) for level in model.layout['levels']]
    return NativeOptimizer(model, target, shape, config, planes), planes
