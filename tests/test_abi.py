"""The C-ABI library loads and exports exactly what include/dspark_amd.h
declares; argument validation runs on the host (no GPU work is launched)."""
import ctypes
import os
import re
import subprocess

import pytest

from qwen3_dspark_amd import _native
from qwen3_dspark_amd.build import LIB_PATH

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, 'include', 'dspark_amd.h')).read()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(dspark_[a-z0-9_]+)\s*\(', text)))


def header_arity():
    text = open(os.path.join(ROOT, 'include', 'dspark_amd.h')).read()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    out = {}
    for name, params in re.findall(r'\b(dspark_[a-z0-9_]+)\s*\(([^)]*)\)\s*;', text):
        params = params.strip()
        out[name] = 0 if params in ('', 'void') else params.count(',') + 1
    return out


def test_header_and_binding_agree():
    assert header_functions() == sorted(_native.SIGNATURES)
    arity = header_arity()
    assert sorted(arity) == header_functions()
    for name, (_, args) in _native.SIGNATURES.items():
        assert arity[name] == len(args), name


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB_PATH), 'run __graft_entry__.build() first'
    out = subprocess.run(['nm', '-D', '--defined-only', LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r'\sT\s(dspark_[a-z0-9_]+)', out))
    assert set(header_functions()) <= exported
    lib = _native.load()
    for name in header_functions():
        assert getattr(lib, name) is not None
    assert lib.dspark_abi_version() == _native.ABI_VERSION


def test_workspace_size_formula():
    lib = _native.load()
    # (ceil(rows/chunk) + n_req) items * 8 KV heads * tiles * 16 rows * (128 + 2) floats
    assert lib.dspark_attn_workspace_bytes(4, 1000, 1, 512) == (2 + 4) * 8 * 1 * 16 * 130 * 4
    assert lib.dspark_attn_workspace_bytes(64, 524288 + 448, 1, 512) == (1025 + 64) * 8 * 16 * 130 * 4
    assert lib.dspark_attn_workspace_bytes(0, 10, 1, 512) == -1
    # a call with a work list of n segments needs n partial slots: (n, 0, ...)
    assert lib.dspark_attn_workspace_bytes(127, 0, 1, 1024) == 127 * 8 * 16 * 130 * 4


@pytest.mark.parametrize('name', ['dspark_varlen_attn_fwd', 'dspark_verify_attn_fwd', 'dspark_verify_attn_staged_fwd',
                                  'dspark_verify_attn_fwd_noalloc',
                                  'dspark_draft_attn_fwd',
                                  'dspark_txn_metadata', 'dspark_kv_stage', 'dspark_kv_commit', 'dspark_kv_gather',
                                  'dspark_layout_build', 'dspark_pool_gather', 'dspark_pool_append',
                                  'dspark_crop_plan', 'dspark_rows_rebuild', 'dspark_qkv_prologue', 'dspark_rope_table',
                                  'dspark_draft_kv_project', 'dspark_draft_kv_epilogue', 'dspark_logit_row_stats',
                                  'dspark_spec_verify',
                                  'dspark_logits_to_probs', 'dspark_sample_rows'])
def test_null_arguments_are_rejected_before_any_launch(name):
    lib = _native.load()
    fn = getattr(lib, name)
    args = []
    for t in fn.argtypes:
        args.append(None if t is ctypes.c_void_p or issubclass(t, ctypes._Pointer) else 1)
    rc = fn(*args)
    assert rc == -1
    assert 'null pointer' in lib.dspark_last_error().decode()


def test_invalid_sizes_are_rejected_before_any_launch():
    lib = _native.load()
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: validation fails first
    rc = lib.dspark_varlen_attn_fwd(fake, fake, fake, fake, fake, 0, 8, 8, 1, 1, 0.088, 512, None, 0, 0, fake, fake,
                                    1 << 20, None)
    assert rc == -1 and 'n_req' in lib.dspark_last_error().decode()
    rc = lib.dspark_varlen_attn_fwd(fake, fake, fake, fake, fake, 2, 8, 8, 1, 1, 0.088, 500, None, 0, 0, fake, fake,
                                    1 << 20, None)
    assert rc == -1 and 'chunk' in lib.dspark_last_error().decode()
    rc = lib.dspark_varlen_attn_fwd(fake, fake, fake, fake, fake, 2, 8, 8, 1, 1, 0.088, 512, None, 0, 0, fake, fake,
                                    16, None)
    assert rc == -1 and 'workspace too small' in lib.dspark_last_error().decode()
    rc = lib.dspark_varlen_attn_fwd(fake, fake, fake, fake, fake, 2, 8, 8, 1, 1, 0.088, 512, fake, 0, 1, fake, fake,
                                    1 << 20, None)
    assert rc == -1 and 'n_work' in lib.dspark_last_error().decode()
    rc = lib.dspark_varlen_attn_fwd(fake, fake, fake, fake, fake, 2, 8, 8, 1, 1, 0.088, 512, fake, 3, 12, fake, fake,
                                    1 << 20, None)
    assert rc == -1 and 'multiple of 8' in lib.dspark_last_error().decode()
    rc = lib.dspark_draft_attn_fwd(fake, 0, fake, fake, 0, None, fake, fake, 1024, 128, fake, fake, fake, fake,
                                   2, 100, 9, 0.088, 512, None, 0, 0, 0, 1, None, None, fake, fake, 1 << 24, None)
    assert rc == -1 and 'max_blocks' in lib.dspark_last_error().decode()
    rc = lib.dspark_draft_attn_fwd(fake, 0, fake, fake, 2, None, fake, fake, 1024, 128, fake, fake, fake, fake,
                                   2, 100, 8, 0.088, 512, None, 0, 0, 0, 1, None, None, fake, fake, 1 << 24, None)
    assert rc == -1 and 'k_dtype' in lib.dspark_last_error().decode()
    for wgs, queues, queue, anc in ((256, 1, None, fake), (256, 3, fake, fake), (250, 8, fake, fake),
                                    (256, 1, fake, None)):
        rc = lib.dspark_draft_attn_fwd(fake, 0, fake, fake, 0, None, fake, fake, 1024, 128, fake, fake, fake, fake,
                                       2, 100, 8, 0.088, 512, fake, 2, 2, wgs, queues, queue, anc, fake, fake,
                                       1 << 24, None)
        assert rc == -1 and 'persistent mode' in lib.dspark_last_error().decode()
    rc = lib.dspark_verify_attn_fwd(fake, fake, fake, fake, fake, fake, fake, fake, 2, 1 << 20, 100, 128, 1000, 7,
                                    0.088, 512, None, 0, 0, fake, fake, 1 << 24, None)
    assert rc == -1 and 'strides' in lib.dspark_last_error().decode()
    rc = lib.dspark_kv_stage(fake, fake, fake, fake, 4, 24, None)
    assert rc == -1 and 'multiple of 16' in lib.dspark_last_error().decode()
    rc = lib.dspark_kv_commit(fake, fake, fake, fake, fake, fake, fake, 2, 7, 1, 1 << 20, 1 << 16, 1 << 12, 24, 16,
                              8, 256, 14, None)
    assert rc == -1 and '16 bytes' in lib.dspark_last_error().decode()
    assert lib.dspark_layout_workspace_bytes(10, 10, 8193) == -1
    assert lib.dspark_layout_workspace_bytes(0, 10, 1) == -1
    rc = lib.dspark_layout_build(fake, fake, 4, fake, fake, 4, 9000, fake, fake, fake, fake, fake, 1 << 20, None)
    assert rc == -1 and 'max_req' in lib.dspark_last_error().decode()
    rc = lib.dspark_layout_build(fake, fake, 4, fake, fake, 4, 4, fake, fake, fake, fake, fake, 16, None)
    assert rc == -1 and 'workspace too small' in lib.dspark_last_error().decode()
    rc = lib.dspark_pool_gather(fake, fake, 8, 4096, 256, 8, 24, fake, 4, fake, fake, None)
    assert rc == -1 and 'multiples of 16' in lib.dspark_last_error().decode()
