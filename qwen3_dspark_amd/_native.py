"""ctypes binding of the C ABI declared in include/dspark_amd.h.

Loading never falls back: a missing library raises, and every non-zero
return code is raised as NativeError with the library's message.
"""
import ctypes
import os
import threading

from .build import LIB_PATH, TIMELINE_LIB_PATH

_lock = threading.Lock()
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
_D = ctypes.c_double
_PP = ctypes.POINTER(ctypes.c_void_p)   # host array of device pointers

# name -> (restype, argtypes); mirrors include/dspark_amd.h exactly.
SIGNATURES = {
    'dspark_last_error': (ctypes.c_char_p, []),
    'dspark_abi_version': (_I, []),
    'dspark_stream_read': (_I, [_P, _L, _I, _I, _P, _P]),
    'dspark_xcd_read_stamps': (_I, [_P, _L, _I, _P, _P]),
    'dspark_attn_workspace_bytes': (_L, [_I, _L, _I, _I]),
    'dspark_varlen_attn_fwd': (_I, [_P, _P, _P, _P, _P, _I, _L, _L, _I, _I, _F, _I, _P, _I, _I, _P, _P, _L, _P]),
    'dspark_verify_attn_fwd': (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _L, _L, _L, _L, _I, _F, _I, _P, _I, _I,
                                    _P, _P, _L, _P]),
    'dspark_noalloc_scratch_bytes': (_L, []),
    'dspark_verify_attn_fwd_noalloc': (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _L, _L, _L, _L, _I, _F, _I, _P, _I,
                                            _I, _P, _P]),
    'dspark_verify_attn_staged_fwd': (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _L, _L, _L, _L, _I, _F, _I,
                                           _P, _I, _I, _P, _P, _L, _P]),
    'dspark_draft_attn_fwd': (_I, [_P, _I, _P, _P, _I, _P, _P, _P, _L, _L, _P, _P, _P, _P, _I, _L, _I, _F, _I, _P,
                                   _I, _I, _I, _I, _P, _P, _P, _P, _L, _P]),
    'dspark_txn_metadata': (_I, [_P, _I, _L, _L, _L, _P, _P, _P, _P, _P, _P, _P, _P]),
    'dspark_kv_stage': (_I, [_P, _P, _P, _P, _L, _L, _P]),
    'dspark_kv_commit': (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _L, _L, _L, _L, _L, _I, _L, _L, _P]),
    'dspark_kv_gather': (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _L, _L, _L, _L, _L, _L, _I, _L, _L, _P, _P, _P]),
    'dspark_layout_workspace_bytes': (_L, [_L, _L, _I]),
    'dspark_layout_build': (_I, [_P, _P, _L, _P, _P, _L, _I, _P, _P, _P, _P, _P, _L, _P]),
    'dspark_pool_gather': (_I, [_P, _P, _L, _L, _L, _I, _L, _P, _L, _P, _P, _P]),
    'dspark_pool_append': (_I, [_P, _P, _L, _L, _L, _L, _L, _I, _L, _I, _I, _PP, _PP, _L, _L, _L, _P, _I, _P, _P]),
    'dspark_qkv_prologue': (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _F, _P, _P, _P, _L, _P]),
    'dspark_rope_table': (_I, [_P, _P, _I, _P, _P]),
    'dspark_draft_kv_project': (_I, [_P, _I, _I, _P, _P, _I, _P, _P, _I, _F, _F, _P, _P, _L, _L, _L, _P, _P]),
    'dspark_draft_kv_epilogue': (_I, [_P, _I, _L, _P, _I, _I, _I, _P, _I, _P, _P, _I, _F, _F, _P, _P, _L, _L, _L,
                                      _P, _P]),
    'dspark_row_stats_bytes': (_L, [_I, _I]),
    'dspark_logit_row_stats': (_I, [_P, _I, _I, _I, _L, _D, _P, _P, _P]),
    'dspark_draw_workspace_bytes': (_L, [_I]),
    'dspark_spec_verify': (_I, [_P, _I, _L, _I, _D, _P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _P, _P, _P, _L, _P]),
    'dspark_logits_to_probs': (_I, [_P, _I, _I, _I, _L, _D, _P, _P, _P]),
    'dspark_sample_rows': (_I, [_P, _I, _I, _P, _P, _P, _L, _P]),
    'dspark_crop_plan_workspace_bytes': (_L, [_L]),
    'dspark_crop_plan': (_I, [_P, _P, _L, _L, _L, _P, _P, _P, _P, _L, _P]),
    'dspark_rows_rebuild': (_I, [_PP, _PP, _PP, _I, _I, _L, _L, _L, _P, _L, _P]),
}

ABI_VERSION = 7


class NativeError(RuntimeError):
    """A C-ABI call returned a non-zero status."""


# Extra entry points of the timeline (profiling) build.
TIMELINE_SIGNATURES = {
    'dspark_timeline_bytes': (_L, []),
    'dspark_timeline_fetch': (_I, [_P, _L]),
    'dspark_timeline_fetch_wg': (_I, [_P, _L]),
    'dspark_timeline_fetch_verify': (_I, [_P, _L]),
}


def timeline_build():
    """True when this process uses the timeline build (DSPARK_AMD_TIMELINE set)."""
    return bool(os.environ.get('DSPARK_AMD_TIMELINE'))


def load():
    """Load (once) and return the HIP extension; raise if it is not built."""
    global _lib
    with _lock:
        if _lib is None:
            path = TIMELINE_LIB_PATH if timeline_build() else LIB_PATH
            if not os.path.exists(path):
                raise RuntimeError(f'HIP extension not built ({path}); run __graft_entry__.build(). '
                                   'There is no CPU or fallback implementation.')
            lib = ctypes.CDLL(path)
            table = dict(SIGNATURES, **(TIMELINE_SIGNATURES if timeline_build() else {}))
            for name, (res, args) in table.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.dspark_abi_version() != ABI_VERSION:
                raise RuntimeError('HIP extension ABI version mismatch; rebuild it')
            _lib = lib
    return _lib


def call(name, *args):
    """Invoke an entry point and raise NativeError on a non-zero status."""
    lib = _lib or load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        raise NativeError(f'{name}: {lib.dspark_last_error().decode(errors="replace")}')
    return rc


def pointer_array(tensors):
    """Host array of device pointers (for entry points taking one per layer);
    None entries become NULL."""
    return (ctypes.c_void_p * len(tensors))(*(None if t is None else t.data_ptr() for t in tensors))


def ptr(t):
    """Device address of a tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()


def stream_handle(device):
    import torch
    return torch.cuda.current_stream(device).cuda_stream
