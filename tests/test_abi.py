"""The C-ABI library loads, exports every declared symbol, and rejects bad arguments
before queuing any device work (these calls never reach the GPU)."""
import ctypes as C
import json
import subprocess

import pytest

from odie_amd import _lib
from odie_amd.config import grid_levels


HIP_ERROR_INVALID_VALUE = 1   # hipErrorInvalidValue


def test_every_declared_symbol_is_exported(native):
    declared = _lib.declared_symbols()
    assert 'odie_grid_forward' in declared and 'odie_error' in declared
    exported = subprocess.run(['nm', '-D', '--defined-only', str(_lib.LIBRARY)], capture_output=True, text=True,
                              check=True).stdout
    names = {line.split()[-1] for line in exported.splitlines() if line.strip()}
    missing = [name for name in declared if name not in names]
    assert not missing, missing
    for name in declared:
        getattr(native, name)


def test_bindings_cover_declarations():
    assert set(_lib.declared_symbols()) <= set(_lib.SIGNATURES), \
        set(_lib.declared_symbols()) - set(_lib.SIGNATURES)


def _levels():
    return grid_levels(dict(n_levels=4, base_resolution=4, log2_hashmap_size=8, per_level_scale=2.0))


@pytest.mark.parametrize('change,message', [
    (dict(n=-1), 'n must be'),
    (dict(experts=0), 'experts must be'),
    (dict(experts=2), 'offsets are required'),
    (dict(n_levels=0), 'n_levels must be'),
    (dict(n_levels=33), 'n_levels must be'),
    (dict(features=3), 'features per level'),
    (dict(dtype=7), 'param_dtype'),
    (dict(width=3), 'out_width'),
    (dict(expert_params=10), 'expert_params'),
])
def test_grid_forward_rejects_bad_arguments(native, change, message):
    levels, entries = _levels()
    args = dict(n=16, experts=1, n_levels=4, features=2, dtype=1, width=8, expert_params=entries * 2)
    args.update(change)
    code = native.odie_grid_forward(8, args['n'], None, args['experts'], 8, args['expert_params'], args['dtype'],
                                    levels, args['n_levels'], args['features'], 16, args['width'], 0)
    assert code == -1
    assert message in native.odie_error().decode()


def test_grid_handoff_bytes_follows_the_owner_plan(native):
    """odie_grid_handoff_bytes plans on the host.  Slice masks (whole planes of n rounded up to 256
    bytes) for 64 experts of 2^16-entry levels, whose hashed levels the owner cuts into masked
    blocks; band lists (starts, then a 4-byte index and an 8-byte (x, y) per coordinate) for one
    expert of 2^19-entry levels, whose passes the owner bands; nothing for tables that fit one
    slice.  A forward given fewer bytes refuses before launching."""
    levels, entries = grid_levels(dict(n_levels=16, base_resolution=16, log2_hashmap_size=16, per_level_scale=1.38))
    n = (1 << 22) - 5
    stride = (n + 255) // 256 * 256
    size = native.odie_grid_handoff_bytes(n, 64, entries * 2, levels, 16, 2)
    assert size > 0 and size % stride == 0 and size // stride <= 16
    assert native.odie_grid_handoff_bytes(0, 64, entries * 2, levels, 16, 2) == 0
    big, big_entries = grid_levels(dict(n_levels=16, base_resolution=16, log2_hashmap_size=19, per_level_scale=1.38))
    lists = native.odie_grid_handoff_bytes(n, 1, big_entries * 2, big, 16, 2)
    assert 12 * n <= lists < 12 * n + 64 * 1024
    small, small_entries = _levels()
    assert native.odie_grid_handoff_bytes(4096, 1, small_entries * 2, small, 4, 2) == 0
    assert native.odie_grid_handoff_bytes(16, 1, small_entries * 2, small, 4, 3) == -1
    assert 'features per level' in native.odie_error().decode()
    code = native.odie_grid_forward_handoff(8, n, 8, 64, 8, entries * 2, 1, levels, 16, 2, 16, 32, 8, size - 1, 0)
    assert code == -1
    assert 'shorter than odie_grid_handoff_bytes' in native.odie_error().decode()


def test_levels_must_be_contiguous(native):
    levels, entries = _levels()
    levels[2].offset += 8
    assert native.odie_grid_backward(8, 16, None, 1, 8, 1, 8, entries * 2 + 64, levels, 4, 2, 16, 1, 0) == -1
    assert 'contiguous' in native.odie_error().decode()


def test_packed_rejects_bad_arguments(native):
    assert native.odie_packed_forward(8, 4, 8, 100, 8, 1, 8, 8, 8, 4, 8, 8, 0) == -1
    assert '2..32 levels' in native.odie_error().decode()
    assert native.odie_packed_forward(8, 4, 8, 100, 8, 4, 8, 8, 8, 200, 8, 8, 0) == -1
    assert 'width' in native.odie_error().decode()


def test_tuning_rejects_unknown_keys(native):
    assert native.odie_set_tuning(b'nonsense', 1) == -1
    assert native.odie_set_tuning(b'lds_bytes', 10 ** 9) == -1


def test_route_tuning_keys_take_their_ranges(native):
    """The routes' keys (no GPU work: a setting only changes how later calls launch)."""
    for value in (0, 1):
        assert native.odie_set_tuning(b'route_one_scan', value) == 0
    assert native.odie_set_tuning(b'route_one_scan', 2) == -1
    assert native.odie_set_tuning(b'route_part', 512) == 0
    assert native.odie_set_tuning(b'route_part', 500) == -1      # not a power of two
    assert native.odie_set_tuning(b'route_part', 1 << 17) == -1  # past 65536
    assert 'route_part' in native.odie_error().decode()
    assert native.odie_set_tuning(b'route_one_scan', 1) == 0


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setattr(_lib, 'LIBRARY', tmp_path / 'libodie_amd.so')
    monkeypatch.setattr(_lib, '_handle', None)
    with pytest.raises(_lib.NativeError, match='no CPU fallback'):
        _lib.library()


def test_route_rejects_bad_arguments(native):
    assert native.odie_route(8, 16, 2048, 1365, 65, 8, None, 8, 8, 8, None, None, 8, 1 << 20, 0) == -1
    assert 'regions per axis' in native.odie_error().decode()
    assert native.odie_route(8, 16, 10, 10, 8, 8, None, 8, 8, 8, None, None, 8, 1 << 20, 0) == -1
    assert 'two pixels' in native.odie_error().decode()
    assert native.odie_route(8, 16, 2048, 1365, 8, 8, None, 8, 8, 8, None, None, 8, 4, 0) == -1
    assert 'workspace' in native.odie_error().decode()
    # 2^22 ids in 8192 sub-chunks of 512: 64 x 8192 counts, then one sum per 1024 of them
    assert native.odie_route_workspace(1 << 22, 64) == 64 * 8192 * 4 + 512 * 4
    assert native.odie_route_workspace(1 << 24, 4096) > 0
    for n, experts in ((5, 4097), (5, 0), (-1, 4), (1 << 31, 4)):   # outside [0, 2^31-1] x [1, 64*64]
        assert native.odie_route_workspace(n, experts) == -1


def test_selection_entry_points_reject_bad_arguments(native):
    assert native.score_chunk(8, 8, 5, 3, 10, 4, 0, 4, 8, 8, 8, True, 0) == HIP_ERROR_INVALID_VALUE
    assert 'begin' in native.odie_error().decode()
    assert native.odie_topk(8, 10, 11, 8, 0) == -1
    assert 'k must be' in native.odie_error().decode()
    assert native.odie_adam_step(8, None, 8, 0, 8, 8, None, 10, 3, 1, 0.1, 0.9, 0.999, 1e-15, 1.0, 0) == -1
    assert 'variant' in native.odie_error().decode()
    assert native.odie_adam_step(16, None, 16, 0, 16, 16, None, 10, 2, 1, 0.1, 0.9, 0.999, 1e-15, 1.0, 0) == -1
    assert 'null' in native.odie_error().decode()     # variants 1 and 2 need the ages
    # decoder MLP: alignment, targets
    assert native.odie_mlp_forward(8, 10, 32, 16, 16, 0) == -1 and 'aligned' in native.odie_error().decode()
    assert native.odie_mlp_forward(16, 10, 24, 16, 16, 0) == -1 and 'width' in native.odie_error().decode()
    assert native.odie_mlp_forward(16, 10, 96, 16, 16, 0) == -1 and 'width' in native.odie_error().decode()
    assert native.odie_mlp_train(16, 10, 32, 10, 16, None, None, None, None, None, None, None, None, 16, 16, 0) == -1
    assert 'target' in native.odie_error().decode()
    assert native.odie_mlp_train(16, 10, 32, 0, 16, None, None, None, 16, None, None, None, None, 16, 16, 0) == -1
    assert 'real' in native.odie_error().decode()
    assert native.odie_mlp_train(16, 1 << 26, 80, 1, 16, 16, None, None, None, None, None, None, None, 16, 16, 0) == -1
    assert '2^31' in native.odie_error().decode()
    assert native.odie_mlp_train_planes(16, 10, 10, 16, 16, None, None, None, None, None, None, None, None, 16, 16,
                                        0) == -1
    assert 'planes is null' in native.odie_error().decode()
    assert native.odie_mlp_train_planes(16, 10, 10, 16, 16, None, None, None, None, None, None, None, 16, None, 16,
                                        0) == -1
    assert 'null' in native.odie_error().decode()
    assert native.odie_mlp_train_planes(16, 10, 10, 16, 16, None, None, None, None, None, None, None, 18, 16, 16,
                                        0) == -1
    assert 'aligned' in native.odie_error().decode()
    # encode backward on planes: two features per level, both buffers
    from odie_amd.config import grid_levels
    levels, entries = grid_levels(dict(n_levels=16, base_resolution=8, log2_hashmap_size=10, per_level_scale=1.4))
    adam = [16, None, 16, 16, 16, 1, 1, 0.01, 0.9, 0.99, 1e-15, 128.0, 0]
    assert native.odie_grid_backward_adam_planes(16, 10, None, 1, 16, None, entries * 2, levels, 16, 2, *adam) == -1
    assert 'planes and blockmax must be' in native.odie_error().decode()
    assert native.odie_grid_backward_adam_planes(16, 10, None, 1, 16, 16, entries, levels, 16, 1, *adam) == -1
    assert '2 fp16 features' in native.odie_error().decode()
    # router gate: coarse range, alignment, feature layout
    assert native.odie_gate_forward(16, 10, 32, 16, None, 16, None, 17, 0, 16, 16, 0) == -1
    assert 'coarse' in native.odie_error().decode()
    assert native.odie_gate_forward(8, 10, 32, 16, None, 16, None, 0, 0, 16, 16, 0) == -1
    assert 'aligned' in native.odie_error().decode()
    assert native.odie_gate_backward(16, 16, 10, 32, 16, None, 16, None, 16, 0, 0, 16, None, 0) == -1
    assert 'null' in native.odie_error().decode()
    three = (C.c_int32 * 16)(*([2] * 15 + [3]))
    assert native.odie_gate_forward(16, 10, 48, 16, three, 16, None, 0, 0, 16, 16, 0) == -1
    assert '1, 2 or 4' in native.odie_error().decode()
    f31 = (C.c_int32 * 16)(*([2] * 15 + [1]))
    assert native.odie_gate_forward(16, 10, 48, 16, f31, 16, None, 0, 0, 16, 16, 0) == -1
    assert 'align16' in native.odie_error().decode()
    assert native.odie_gate_forward(16, 10, 32, 33, None, 16, None, 0, 0, 16, 16, 0) == -1
    assert 'levels' in native.odie_error().decode()
    # cell bounds: sizes
    assert native.odie_cell_bounds(1, 8, 4, 16, 16, 0) == -1 and 'at least 2' in native.odie_error().decode()
    assert native.odie_cell_bounds(8, 8, 1, 16, 16, 0) == -1 and 'resolution' in native.odie_error().decode()
    assert native.odie_adam_step(8, None, 8, 0, 8, 8, None, 10, 0, 0, 0.1, 0.9, 0.999, 1e-15, 1.0, 0) == -1
    assert 'step' in native.odie_error().decode()
    # greedy selector: n must be resolution^2, cap 8-aligned, chunk positive, tree large enough
    args = [8, 4096, 4096, 63, 256, True, 8, 8, 8, 8, None, None, 0, 512, 8, None, 0]
    refused = HIP_ERROR_INVALID_VALUE
    assert native.selection_chunk(*args) == refused and 'resolution^2' in native.odie_error().decode()
    args[3], args[4] = 64, 100
    assert native.selection_chunk(*args) == refused and 'cap' in native.odie_error().decode()
    args[4], args[13] = 256, 0
    assert native.selection_chunk(*args) == refused and 'chunk' in native.odie_error().decode()
    offsets, sizes = (C.c_int * 1)(0), (C.c_int * 1)(10)
    assert native.selection_init(8, 4096, 4096, 8, 8, 8, 8, 8, offsets, sizes, 1, 0) == refused
    assert 'too small' in native.odie_error().decode()
    assert native.selection_init(8, 4096, 4100, 8, 8, 8, 8, 8, None, None, 0, 0) == refused
    assert 'points' in native.odie_error().decode()


def test_reference_check_of_the_runtime_code(native):
    """selection_init, selection_chunk and score_chunk fail as the reference's do, with the
    runtime's error code (odie/native/selection_cuda.cu:217,229, odie/residual_cuda.cu:51:
    `return int(cudaGetLastError())`), so the reference's unchanged check -- a nonzero result
    raises RuntimeError with the runtime's string for it (odie/selection_cuda.py:49-51) -- run on
    the HIP runtime raises with that string, and odie_error() keeps this library's message."""
    runtime = C.CDLL('libamdhip64.so')
    runtime.hipGetErrorString.argtypes = [C.c_int]
    runtime.hipGetErrorString.restype = C.c_char_p

    def check(result):   # the reference's Cuda.check, with the HIP runtime's error string
        if result:
            raise RuntimeError(runtime.hipGetErrorString(result).decode())

    check(native.score_chunk(None, None, 0, 0, 8, 4, 0, 0, None, None, None, True, 0))   # nothing to do
    calls = [
        (lambda: native.score_chunk(8, 8, 5, 3, 10, 4, 0, 4, 8, 8, 8, True, 0), 'score_chunk: need 0 <= begin'),
        (lambda: native.selection_init(8, 4096, 4100, 8, 8, 8, 8, 8, None, None, 0, 0), 'selection_init: points'),
        (lambda: native.selection_chunk(8, 4096, 4096, 63, 256, True, 8, 8, 8, 8, None, None, 0, 512, 8, None, 0),
         'selection_chunk: n must be resolution^2'),
    ]
    for call, message in calls:
        with pytest.raises(RuntimeError, match='invalid argument'):
            check(call())
        assert native.odie_error().decode().startswith(message)


def test_selection_tree_fits_the_callers_fan32_allocation(native):
    # the reference sizes the tree buffer as 5 ints per node of a fan-32 tree
    # (odie/gpu_residual.py:77-88); the fan-64, 4-category tree must never need more
    def fan32_ints(n):
        total, children = 0, n
        while True:
            parents = (children + 31) // 32
            total += parents * 5
            if parents == 1:
                return total
            children = parents
    assert native.odie_selection_tree_ints(4096) == (64 + 1) * 4
    assert native.odie_selection_tree_ints(200704) == (3136 + 49 + 1) * 4
    for n in (4, 9, 64, 65, 4096, 4097, 10 ** 6, 2 ** 24, 2 ** 31 - 1):
        assert 0 < native.odie_selection_tree_ints(n) <= fan32_ints(n)
    assert native.odie_selection_tree_ints(0) == -1


def _settings(**change):
    settings = dict(stream=0, total=1024, width=64, height=64, mode=20, rgb=4096, grid=4096, decoder=4096,
                    descriptors=4096, node_bitmap=4096, node_prefix=4096, bitmap=4096, active=16, grid_lr=1e-2,
                    decoder_lr=1e-3, levels=16)
    settings.update(change)
    return json.dumps({k: v for k, v in settings.items() if v is not None}).encode()


@pytest.mark.parametrize('settings,message', [
    (b'not json', 'settings JSON'),
    (b'[1, 2]', 'expected an object'),
    (b'{"stream": 0} trailing', 'trailing'),
    (_settings(total=None), 'missing setting: total'),
    (_settings(total=0), 'invalid total'),
    (_settings(grid=0), 'null rgb or grid'),
    (_settings(grid=4100), '16-byte aligned'),
    (_settings(levels=21), 'levels must be within 2..20'),
    (_settings(levels=1), 'levels must be within 2..20'),
    (_settings(levels=None), 'levels is required'),
    (_settings(raw_width=96), 'raw_width must be within'),
    (_settings(router_activation='tanh'), 'router_activation'),
    (_settings(gate_coarse_levels=17), 'gate_coarse_levels'),
    (_settings(gate=4096, mode=4), 'parallel gate'),
    (_settings(gate=4096, mode=21), 'mode bit 1'),
    (_settings(hash_encoding=dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=12, base_resolution=4,
                                  per_level_scale=1.5), mode=16), 'half gradients'),
    (_settings(hash_encoding=dict(n_levels=21, n_features_per_level=2, log2_hashmap_size=12, base_resolution=4,
                                  per_level_scale=1.5), levels=None), 'levels must be within 2..20'),
    (_settings(hash_encoding=dict(n_levels=8, n_features_per_level=3, log2_hashmap_size=12, base_resolution=4,
                                  per_level_scale=1.5), levels=None), '1, 2 or 4'),
    (_settings(hash_encoding=dict(n_levels=8, n_features_per_level=2, log2_hashmap_size=12, base_resolution=4,
                                  per_level_scale=1.5)), 'levels differs'),
    (_settings(hash_encoding=dict(n_levels=16, n_features_per_level=2, log2_hashmap_size=12, base_resolution=4,
                                  per_level_scale=1.5)), 'allocation differs'),
])
def test_runtime_rejects_settings_before_touching_the_device(native, settings, message):
    assert native.odie_create(settings) is None
    assert message in native.odie_error().decode()


def test_runtime_entry_points_reject_a_null_handle(native):
    assert native.odie_step(None, 8, 16, 1) == -1
    assert 'null handle' in native.odie_error().decode()
    assert native.odie_configure(None, b'{}') == -1
    assert native.odie_sync_weights(None) == -1
    assert native.odie_pointers(None) is None
    assert native.odie_state(None, -1, -1) is None
    native.odie_pin_contexts(None)
    native.odie_release_contexts(None)
    native.odie_destroy(None)


def test_reconstruct_rejects_bad_arguments(native):
    levels, entries = grid_levels(dict(n_levels=16, base_resolution=4, log2_hashmap_size=8, per_level_scale=1.3))
    params = entries * 2
    call = lambda **k: native.odie_reconstruct(
        k.get('begin', 0), k.get('n', 64), k.get('width', 64), k.get('height', 64), k.get('rx', 2), k.get('ry', 2),
        None, k.get('experts', 4), 4096, k.get('params', params), levels, k.get('levels', 16), 4096, 4096, None,
        None, 0)
    for change, message in [(dict(n=-1), 'nonnegative'), (dict(rx=65), 'regions per axis'),
                            (dict(width=3), 'two pixels'), (dict(begin=64 * 64 - 10, n=11), 'past the image'),
                            (dict(levels=8), '16 levels'), (dict(experts=0), 'experts'),
                            (dict(params=params - 1), 'expert_params')]:
        assert call(**change) == -1, change
        assert message in native.odie_error().decode(), (change, native.odie_error())
    assert call(n=0) == 0


def test_reconstruct_scores_rejects_bad_arguments(native):
    levels, entries = grid_levels(dict(n_levels=16, base_resolution=4, log2_hashmap_size=8, per_level_scale=1.3))
    call = lambda resolution=8, experts=4, target=4096: native.odie_reconstruct_scores(
        64, 64, 2, 2, None, experts, 4096, entries * 2, levels, 16, 4096, target, resolution, 4096, 4096, 4096, None,
        None, 0)
    for kwargs, message in [(dict(resolution=0), 'resolution'), (dict(experts=0), 'experts'),
                            (dict(target=None), 'null pointer')]:
        assert call(**kwargs) == -1
        assert message in native.odie_error().decode()


def test_route_stratified_rejects_bad_arguments(native):
    args = lambda uniforms, n: (uniforms, n, 2048, 1365, 8, 8, None, 8, 8, 8, None, None, 8, 1 << 20, 0)
    assert native.odie_route_stratified(*args(8, 8)) == -1          # not a square
    assert 'square power-of-two' in native.odie_error().decode()
    assert native.odie_route_stratified(*args(8, 12)) == -1
    assert native.odie_route_stratified(*args(12, 16)) == -1        # misaligned uniforms
    assert 'aligned' in native.odie_error().decode()
    assert native.odie_route_stratified(*args(None, 16)) == -1
    assert native.odie_route_stratified(8, 16, 2048, 1365, 8, 8, None, 8, 8, 8, None, None, 8, 4, 0) == -1
    assert 'workspace' in native.odie_error().decode()


def test_stratified_ids_reject_bad_arguments(native):
    assert native.odie_stratified_ids(8, 8, 10, 10, 8, 0) == -1
    assert 'square power-of-two' in native.odie_error().decode()
    assert native.odie_stratified_ids(8, 12, 10, 10, 8, 0) == -1
    assert native.odie_stratified_ids(None, 16, 10, 10, 8, 0) == -1


def test_route_allocated_rejects_bad_arguments(native):
    # every call below fails a check before anything is queued (the pointers are never used)
    args = [8, None, 100, 640, 480, 4, 4, 8, 9, None, 8, 8, 8, None, None, 8, 1 << 20, 0]
    bad = list(args)
    bad[1] = 8                                             # ids and uniforms both given
    assert native.odie_route_allocated(*bad) == -1 and 'exactly one' in native.odie_error().decode()
    bad = list(args)
    bad[8] = 4096                                          # experts + 1 buckets above 4096
    assert native.odie_route_allocated(*bad) == -1 and '1..4095' in native.odie_error().decode()
    bad = list(args)
    bad[7] = None                                          # no slot map
    assert native.odie_route_allocated(*bad) == -1 and 'slots is null' in native.odie_error().decode()
    bad = list(args)
    bad[16] = native.odie_route_workspace(100, 9) - 4       # workspace sized for the experts alone
    assert native.odie_route_workspace(100, 10) > native.odie_route_workspace(100, 9) - 4
    assert native.odie_route_allocated(*bad) == -1 and 'experts + 1' in native.odie_error().decode()
