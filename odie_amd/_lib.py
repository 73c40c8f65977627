"""ctypes binding of libodie_amd.so, the only compute path of this package.

There is no CPU fallback: if the library is missing, importing a compute entry point
raises immediately.  Device buffers are passed as raw addresses (torch tensors'
data_ptr()), streams as hipStream_t values (torch.cuda.current_stream().cuda_stream).
"""
import ctypes as C
from pathlib import Path
import re

LIBRARY = Path(__file__).resolve().parent / 'libodie_amd.so'
HEADER = Path(__file__).resolve().parent.parent / 'include' / 'odie_amd.h'

F32, F16 = 0, 1


class GridLevel(C.Structure):
    """Mirror of odie_grid_level (include/odie_amd.h)."""
    _fields_ = [('scale', C.c_float), ('resolution', C.c_uint32), ('size', C.c_uint32),
                ('offset', C.c_uint32), ('hashed', C.c_uint32)]


_P, _I, _I64, _U64 = C.c_void_p, C.c_int, C.c_int64, C.c_uint64

SIGNATURES = {
    'odie_error': ([], C.c_char_p),
    'odie_copy': ([_U64, _U64, _U64, _U64], _I),
    'odie_grid_backward_adam': ([_P, _I64, _P, _I, _P, _I, _I, _I64, _P, _I, _I, _P, _P, _P, _P, _P, _I, _I64,
                                 C.c_float, C.c_float, C.c_float, C.c_float, C.c_float, _U64], _I),
    'odie_grid_backward_adam_planes': ([_P, _I64, _P, _I, _P, _P, _I64, _P, _I, _I, _P, _P, _P, _P, _P, _I, _I64,
                                        C.c_float, C.c_float, C.c_float, C.c_float, C.c_float, _U64], _I),
    'odie_grid_backward_planes': ([_P, _I64, _P, _I, _P, _P, _I64, _P, _I, _I, _P, _I, _U64], _I),
    'odie_set_tuning': ([C.c_char_p, _I], _I),
    'odie_grid_forward': ([_P, _I64, _P, _I, _P, _I64, _I, _P, _I, _I, _P, _I, _U64], _I),
    'odie_grid_handoff_bytes': ([_I64, _I, _I64, _P, _I, _I], _I64),
    'odie_grid_forward_handoff': ([_P, _I64, _P, _I, _P, _I64, _I, _P, _I, _I, _P, _I, _P, _I64, _U64], _I),
    'odie_grid_backward_handoff': ([_P, _I64, _P, _I, _P, _I, _I, _I64, _P, _I, _I, _P, _I, _P, _I64, _U64], _I),
    'odie_grid_backward_adam_planes_handoff': ([_P, _I64, _P, _I, _P, _P, _I64, _P, _I, _I, _P, _P, _P, _P, _P,
                                                _I, _I64, C.c_float, C.c_float, C.c_float, C.c_float, C.c_float,
                                                _P, _I64, _U64], _I),
    'odie_grid_backward': ([_P, _I64, _P, _I, _P, _I, _I, _I64, _P, _I, _I, _P, _I, _U64], _I),
    'odie_packed_forward': ([_P, _I64, _P, _I64, _P, _I, _P, _P, _P, _I, _P, _P, _U64], _I),
    'odie_packed_backward': ([_P, _I64, _P, _I, _P, _I, _P, _P, _P, _P, _I64, _U64], _I),
    'odie_route_workspace': ([_I64, _I], _I64),
    'odie_route': ([_P, _I64, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _I64, _U64], _I),
    'odie_select_mean_rank_workspace': ([_I], _I64),
    'odie_select_mean_rank': ([_P, _I, _I, _P, _P, _P, _P, _I64, _U64], _I),
    'odie_route_allocated': ([_P, _P, _I64, _I, _I, _I, _I, _P, _I, _P, _P, _P, _P, _P, _P, _P, _I64, _U64], _I),
    'odie_route_noalloc': ([_P, _I64, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _U64], _I),
    'odie_route_stratified': ([_P, _I64, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _I64, _U64], _I),
    'score_chunk': ([_P, _P, _I64, _I64, _I, _I, _I, _I, _P, _P, _P, C.c_bool, _U64], _I),
    'odie_topk': ([_P, _I64, _I64, _P, _U64], _I),
    'odie_cell_bounds': ([_I, _I, _I, _P, _P, _U64], _I),
    'odie_selection_tree_ints': ([_I], _I64),
    'selection_init': ([_P, _I, _I, _P, _P, _P, _P, _P, _P, _P, _I, _U64], _I),
    'selection_chunk': ([_P, _I, _I, _I, _I, C.c_bool, _P, _P, _P, _P, _P, _P, _I, _I, _P, _P, _U64], _I),
    'odie_mlp_forward': ([_P, _I64, _I, _P, _P, _U64], _I),
    'odie_mlp_train': ([_P, _I64, _I, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _U64], _I),
    'odie_mlp_train_planes': ([_P, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _U64], _I),
    'odie_gate_forward': ([_P, _I64, _I, _I, _P, _P, _P, _I, _I, _P, _P, _U64], _I),
    'odie_gate_backward': ([_P, _P, _I64, _I, _I, _P, _P, _P, _P, _I, _I, _P, _P, _U64], _I),
    'odie_adam_step': ([_P, _P, _P, _I, _P, _P, _P, _I64, _I, _I64, C.c_float, C.c_float, C.c_float,
                        C.c_float, C.c_float, _U64], _I),
    'odie_reconstruct': ([_I64, _I64, _I, _I, _I, _I, _P, _I, _P, _I64, _P, _I, _P, _P, _P, _P, _U64], _I),
    'odie_reconstruct_scores': ([_I, _I, _I, _I, _P, _I, _P, _I64, _P, _I, _P, _P, _I, _P, _P, _P, _P, _P, _U64],
                                _I),
    'odie_stratified_ids': ([_P, _I, _I, _I, _P, _U64], _I),
    'odie_create': ([C.c_char_p], _P),
    'odie_step': ([_P, _U64, _I, _I], _I),
    'odie_configure': ([_P, C.c_char_p], _I),
    'odie_pointers': ([_P], C.c_char_p),
    'odie_state': ([_P, _I, _I], C.c_char_p),
    'odie_sync_weights': ([_P], _I),
    'odie_pin_contexts': ([_P], None),
    'odie_release_contexts': ([_P], None),
    'odie_destroy': ([_P], None),
}

_handle = None


class NativeError(RuntimeError):
    pass


def library():
    """Load libodie_amd.so once; raise if it has not been built."""
    global _handle
    if _handle is None:
        if not LIBRARY.exists():
            raise NativeError('libodie_amd.so is not built (run __graft_entry__.build() or '
                              'python -m odie_amd.build); there is no CPU fallback')
        lib = C.CDLL(str(LIBRARY))
        for name, (arguments, result) in SIGNATURES.items():
            function = getattr(lib, name)
            function.argtypes = arguments
            function.restype = result
        _handle = lib
    return _handle


def check(code):
    if code:
        raise NativeError(library().odie_error().decode())


def declared_symbols():
    """Function names declared in include/odie_amd.h."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r'^\s*(?:const\s+)?[\w\s\*]*?\b(odie_\w+|selection_\w+|score_\w+)\s*\(',
                                 text, flags=re.M)))


def ptr(tensor):
    return None if tensor is None else tensor.data_ptr()


def stream_of(tensor=None):
    import torch
    device = tensor.device if tensor is not None else None
    return torch.cuda.current_stream(device).cuda_stream


def set_tuning(key, value):
    check(library().odie_set_tuning(key.encode(), int(value)))
