"""The allocation-free verification entry point.

dspark_verify_attn_fwd_noalloc keeps its split-K partials in the library's
static device scratch instead of a caller workspace.  It runs the same
kernels on the same arguments as dspark_verify_attn_fwd, so its outputs must
be bit-identical: checked on two calls in a row through the C ABI, the
second on a smaller transaction (fewer requests, shorter contexts, another
work list) so that stale contents of the shared scratch would show.  A call
whose partials exceed the static maximum is refused before any launch.
"""
import numpy as np
import pytest
import torch

from helpers import SCALE, SEED, randn_bf16

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope='module')
def dev():
    from qwen3_dspark_amd._device import require_gfx950
    return require_gfx950('cuda')


def transaction(dev, store, names, contexts, gen):
    """Admit requests with random committed rows and begin a 7-row round."""
    from qwen3_dspark_amd.persistent_kv import Bucket
    handles = []
    for name, c in zip(names, contexts):
        h = store.add_request(name)
        kv = randn_bf16(gen, 2, 1, c, 8, 128).to(dev)
        store.load_prefix(h, kv[0], kv[1])
        handles.append(h)
    bucket = Bucket((7,) * len(names), tuple(max(contexts) for _ in names), f'no-alloc test, {len(names)} requests')
    store.register_bucket(bucket)
    tx = store.begin(handles, bucket)
    q = sum(tx.query_lengths)
    store.stage_layer(tx, 0, randn_bf16(gen, q, 8, 128).to(dev), randn_bf16(gen, q, 8, 128).to(dev))
    return tx, randn_bf16(gen, q, 16, 128).to(dev)


def launch_args(store, tx, query, out):
    """The argument list dspark_verify_attn_fwd takes for layer 0, without
    the trailing (workspace, workspace bytes, stream)."""
    from qwen3_dspark_amd import _native
    ws = store.workspace(tx.bucket)
    k, v, sk, sv = store.kv_device.layer_pointers[0]
    C, bucket = store.context_capacity, tx.bucket
    n_work, runs = store.kv_device.launch_shape(bucket)
    return [query.data_ptr(), k, v, sk, sv, ws.cu_query.data_ptr(), ws.cu_key.data_ptr(), ws.req.data_ptr(),
            bucket.request_count, 8 * C * 128, 128, C * 128, bucket.key_capacity, bucket.maximum_query_length,
            SCALE, store.chunk, ws.work.data_ptr(), n_work, runs, _native.ptr(out)], ws


def test_noalloc_matches_workspace_entry_point_on_two_calls(dev):
    from qwen3_dspark_amd import _native
    from qwen3_dspark_amd.persistent_kv import PersistentTargetKV
    lib = _native.load()
    stream = _native.stream_handle(dev)
    assert lib.dspark_noalloc_scratch_bytes() == 32 << 20
    gen = torch.Generator().manual_seed(SEED)
    rng = np.random.default_rng(SEED)
    store = PersistentTargetKV(layers=1, slots=64, context_capacity=4096, max_query_tokens=448, heads=8, dim=128,
                               device=dev)
    big = [int(x) for x in rng.integers(256, 4089, size=48)]
    small = [int(x) for x in rng.integers(16, 600, size=6)]
    for label, names, contexts in (('48 requests', [f'a{i}' for i in range(48)], big),
                                   ('6 requests (smaller)', [f'b{i}' for i in range(6)], small)):
        say(f'[no-alloc] {label}: contexts {min(contexts)}..{max(contexts)}')
        tx, query = transaction(dev, store, names, contexts, gen)
        ref = torch.full_like(query, float('nan'))
        got = torch.full_like(query, float('nan'))
        args, ws = launch_args(store, tx, query, ref)
        _native.call('dspark_verify_attn_fwd', *args, ws.attn.data_ptr(), ws.attn.numel(), stream)
        args, _ = launch_args(store, tx, query, got)
        _native.call('dspark_verify_attn_fwd_noalloc', *args, stream)
        torch.cuda.synchronize(dev)
        assert torch.isfinite(ref.float()).all()
        assert torch.equal(ref.view(torch.int16), got.view(torch.int16)), label
        store.abort(tx)
        for h in tx.slots:
            store.remove_request(h)


def test_noalloc_refuses_partials_beyond_the_static_scratch(dev):
    from qwen3_dspark_amd import _native
    from qwen3_dspark_amd.persistent_kv import PersistentTargetKV
    lib = _native.load()
    gen = torch.Generator().manual_seed(SEED + 1)
    store = PersistentTargetKV(layers=1, slots=4, context_capacity=512, max_query_tokens=28, heads=8, dim=128,
                               device=dev)
    tx, query = transaction(dev, store, ['r0', 'r1', 'r2', 'r3'], [100, 200, 300, 400], gen)
    out = torch.zeros_like(query)
    args, _ = launch_args(store, tx, query, out)
    # No work list and a key bound of 2^20 rows in 1024-row chunks: about
    # 1,028 partial slots of 66,560 bytes, more than the 32 MiB maximum.
    args[12], args[15], args[16], args[17], args[18] = 1 << 20, 1024, None, 0, 0
    need = lib.dspark_attn_workspace_bytes(4, 1 << 20, 1, 1024)
    assert need > lib.dspark_noalloc_scratch_bytes()
    rc = lib.dspark_verify_attn_fwd_noalloc(*args, _native.stream_handle(dev))
    assert rc == -1
    assert 'static scratch' in lib.dspark_last_error().decode()
    torch.cuda.synchronize(dev)
    assert int(torch.count_nonzero(out.view(torch.int16))) == 0
    store.abort(tx)
