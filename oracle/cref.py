"""ctypes loader for oracle/attn_ref.c (test infrastructure only).

All arrays are numpy: bf16 inputs as uint16 bit patterns, outputs float32.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, '_build', 'liboracle.so')
_lib = None


def build():
    subprocess.run(['make', '-C', HERE], check=True, capture_output=True)
    return LIB


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f'{LIB} missing: run make -C oracle')
        lib = ctypes.CDLL(LIB)
        P, I, L, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
        lib.oracle_varlen_attn.argtypes = [P, P, P, P, P, I, I, F, P, I]
        lib.oracle_verify_attn.argtypes = [P, P, P, P, P, P, P, P, I, L, F, P, I]
        lib.oracle_draft_attn.argtypes = [P, P, P, P, P, P, P, P, P, I, F, P, I]
        lib.oracle_max_threads.restype = I
        for f in (lib.oracle_varlen_attn, lib.oracle_verify_attn, lib.oracle_draft_attn):
            f.restype = None
        _lib = lib
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _u16(a):
    a = np.ascontiguousarray(a)
    assert a.dtype == np.uint16
    return a


def _i32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def varlen_attention(q, k, v, cu_q, cu_k, *, causal, scale, threads=0):
    q, k, v = _u16(q), _u16(k), _u16(v)
    cu_q, cu_k = _i32(cu_q), _i32(cu_k)
    out = np.zeros(q.shape, np.float32)
    load().oracle_varlen_attn(_p(q), _p(k), _p(v), _p(cu_q), _p(cu_k), len(cu_q) - 1, int(causal),
                              float(scale), _p(out), int(threads))
    return out


def verify_attention(q, k_res, v_res, k_scr, v_scr, slots, contexts, cu_q, *, scale, threads=0):
    """k_res/v_res: one resident layer [slots, cap, 8, 128] (uint16)."""
    q, k_res, v_res, k_scr, v_scr = map(_u16, (q, k_res, v_res, k_scr, v_scr))
    slots, contexts, cu_q = _i32(slots), _i32(contexts), _i32(cu_q)
    out = np.zeros(q.shape, np.float32)
    load().oracle_verify_attn(_p(q), _p(k_res), _p(v_res), _p(k_scr), _p(v_scr), _p(slots), _p(contexts),
                              _p(cu_q), len(slots), k_res.shape[1], float(scale), _p(out), int(threads))
    return out


def draft_attention(q, k_ctx, v_ctx, ctx_off, ctx_len, k_blk, v_blk, cu_b, anchors, *, scale, threads=0):
    q, k_ctx, v_ctx, k_blk, v_blk = map(_u16, (q, k_ctx, v_ctx, k_blk, v_blk))
    ctx_off = np.ascontiguousarray(np.asarray(ctx_off, dtype=np.int64))
    ctx_len, cu_b, anchors = _i32(ctx_len), _i32(cu_b), _i32(anchors)
    out = np.zeros(q.shape, np.float32)
    load().oracle_draft_attn(_p(q), _p(k_ctx), _p(v_ctx), _p(ctx_off), _p(ctx_len), _p(k_blk), _p(v_blk),
                             _p(cu_b), _p(anchors), len(ctx_len), float(scale), _p(out), int(threads))
    return out


def max_threads():
    return load().oracle_max_threads()
