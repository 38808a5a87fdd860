"""GPU tests of the persistent KV transaction store: the reference's store
tests (tests/test_persistent_target_kv.py, tests/test_query_family.py) on the
HIP store, bit-exact metadata/gather/commit against the oracle, and the fused
verification attention against the oracle and the materialised path."""
import copy
from types import SimpleNamespace
from unittest.mock import patch

import numpy as np
import pytest
import torch

from helpers import SCALE, SEED, attention_gate, bits, f64, randn_bf16, segments
from oracle import cref, semantics

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope='module')
def dev():
    from qwen3_dspark_amd._device import require_gfx950
    return require_gfx950('cuda')


def small_pool(dev, **kw):
    from qwen3_dspark_amd.persistent_kv import PersistentTargetKV
    args = dict(layers=2, slots=3, context_capacity=24, max_query_tokens=8, heads=2, dim=4, dtype=torch.float32)
    args.update(kw)
    return PersistentTargetKV(device=dev, **args)


def prefix(pool, handle, n, offset):
    x = torch.arange(pool.layers * n * pool.heads * pool.dim, dtype=pool.dtype,
                     device=pool.device).reshape(pool.layers, n, pool.heads, pool.dim) + offset
    pool.load_prefix(handle, x, x + 0.25)
    return x, x + 0.25


def stage(pool, tx):
    q = sum(tx.query_lengths)
    x = torch.arange(pool.layers * q * pool.heads * pool.dim, dtype=pool.dtype,
                     device=pool.device).reshape(pool.layers, q, pool.heads, pool.dim) + 10000
    for layer in range(pool.layers):
        pool.stage_layer(tx, layer, x[layer], x[layer] + 0.5)
    return x, x + 0.5


def test_growing_context_stable_buffers_exact_q_and_independent_scratch(dev, golden):
    from qwen3_dspark_amd.persistent_kv import Bucket
    say('[kv] growing context (reference golden)')
    g = golden['txn_growing_context']
    pool = small_pool(dev)
    a, b, idle = pool.add_request('A'), pool.add_request('B'), pool.add_request('idle')
    ak, av = prefix(pool, a, 3, 100)
    bk, bv = prefix(pool, b, 5, 500)
    ik, _ = prefix(pool, idle, 9, 900)
    bucket = Bucket(tuple(g['bucket'][0]), tuple(g['bucket'][1]), 'GPU fixture')
    pool.register_bucket(bucket)
    pointers = pool.pointers(bucket)
    before = pool.keys.clone()
    tx = pool.begin([a, b], bucket)
    sk, sv = stage(pool, tx)
    assert torch.equal(before, pool.keys)
    for layer in range(pool.layers):
        k, v, cq, ck, pos = pool.prepare_attention(tx, layer)
        assert torch.equal(k[:13], torch.cat((ak[layer], sk[layer, :2], bk[layer], sk[layer, 2:])))
        assert torch.equal(v[:13], torch.cat((av[layer], sv[layer, :2], bv[layer], sv[layer, 2:])))
        assert torch.equal(k[13:], torch.zeros_like(k[13:]))
        assert cq.tolist() == g['cu_query'] and ck.tolist() == g['cu_key'] and pos.tolist() == g['positions']
    work = pool.work(tx)
    assert work['inactive_resident_key_tokens'] == g['inactive_resident_key_tokens']
    assert work['physical_key_capacity'] == g['physical_key_capacity']
    assert work['padded_key_capacity'] == g['padded_key_capacity']
    pool.commit(tx, {a: 1, b: 2})
    assert torch.equal(pool.request_kv(a)[0], torch.cat((ak, sk[:, :1]), dim=1))
    assert torch.equal(pool.request_kv(b)[0], torch.cat((bk, sk[:, 2:4]), dim=1))
    assert torch.equal(pool.request_kv(idle)[0], ik)
    assert pool.pointers(bucket) == pointers
    second = pool.begin([a, b], bucket)
    stage(pool, second)
    _, _, _, ck, pos = pool.prepare_attention(second, 0)
    assert ck.tolist() == g['second_cu_key'] and pos.tolist() == g['second_positions']
    assert pool.pointers(bucket) == pointers
    pool.abort(second)


def test_abort_slot_reuse_and_invalid_commits(dev, golden):
    from qwen3_dspark_amd.persistent_kv import Bucket, Slot
    say('[kv] abort / slot reuse / invalid commits')
    pool = small_pool(dev)
    old = pool.add_request('same')
    prefix(pool, old, 7, 77)
    bucket = Bucket((1,), (10,), 'GPU fixture')
    pool.register_bucket(bucket)
    before = pool.keys.clone()
    tx = pool.begin([old], bucket)
    stage(pool, tx)
    pool.abort(tx)
    assert torch.equal(before, pool.keys) and pool.length(old) == 7
    pool.remove_request(old)
    fresh = pool.add_request('same')
    assert old.index == fresh.index and old.incarnation != fresh.incarnation
    for stale in (old, copy.copy(fresh), Slot(fresh.request, fresh.index, fresh.incarnation)):
        with pytest.raises(ValueError):
            pool.length(stale)
    tx = pool.begin([fresh], bucket)
    sk, _ = stage(pool, tx)
    k, _, _, ck, pos = pool.prepare_attention(tx, 0)
    assert ck.tolist() == golden['txn_slot_reuse']['cu_key'] and pos.tolist() == golden['txn_slot_reuse']['positions']
    assert torch.equal(k[:1], sk[0]) and int(torch.count_nonzero(k[1:])) == 0
    pool.commit(tx, {fresh: 1})
    assert pool.length(fresh) == 1
    # invalid commits fail before any resident write
    pool = small_pool(dev)
    a = pool.add_request('A')
    prefix(pool, a, 2, 1)
    bucket = Bucket((2,), (4,), 'GPU fixture')
    pool.register_bucket(bucket)
    before = pool.keys.clone()
    tx = pool.begin([a], bucket)
    for call in (lambda: pool.remove_request(a), lambda: pool.add_request('B'), lambda: pool.begin([a], bucket)):
        with pytest.raises(RuntimeError):
            call()
    with pytest.raises(ValueError):
        pool.prepare_attention(tx, 0)
    with pytest.raises(ValueError):
        pool.commit(tx, {a: 1})
    stage(pool, tx)
    for bad in golden['txn_invalid_commit']['invalid_counts']:
        with pytest.raises(ValueError):
            pool.commit(tx, {a: bad})
    with pytest.raises(ValueError):
        pool.commit(copy.copy(tx), {a: 1})
    assert torch.equal(before, pool.keys)
    pool.commit(tx, {a: 0})
    assert torch.equal(before, pool.keys)
    with pytest.raises(ValueError):
        pool.abort(tx)


def test_failed_metadata_launch_never_publishes_transaction(dev, golden):
    from qwen3_dspark_amd import _native
    from qwen3_dspark_amd.persistent_kv import Bucket
    say('[kv] failed metadata preparation')
    pool = small_pool(dev)
    a = pool.add_request('A')
    prefix(pool, a, 3, 3)
    bucket = Bucket((2,), (8,), 'GPU fixture')
    pool.register_bucket(bucket)
    old = pool.begin([a], bucket)
    pool.abort(old)
    before = pool.keys.clone()

    def fail(name, *args):
        raise _native.NativeError(f'{name}: injected metadata failure')
    with patch.object(_native, 'call', side_effect=fail), pytest.raises(_native.NativeError, match='injected'):
        pool.begin([a], bucket)
    assert pool.open_transaction is None and torch.equal(pool.keys, before)
    with pytest.raises(ValueError):
        pool.abort(old)
    tx = pool.begin([a], bucket)
    stage(pool, tx)
    _, _, cq, ck, pos = pool.prepare_attention(tx, 0)
    g = golden['txn_retry_metadata']
    assert cq.tolist() == g['cu_query'] and ck.tolist() == g['cu_key'] and pos.tolist() == g['positions']
    pool.abort(tx)


def test_ordered_shape_bounds_and_active_subset(dev, golden):
    from qwen3_dspark_amd.persistent_kv import Bucket
    say('[kv] ordered bounds / reordered subset')
    g = golden['txn_reordered_subset']
    pool = small_pool(dev)
    a, b = pool.add_request('A'), pool.add_request('B')
    prefix(pool, a, 8, 0)
    prefix(pool, b, 4, 0)
    small = Bucket((1,), (7,), 'GPU fixture')
    pool.register_bucket(small)
    with pytest.raises(ValueError):
        pool.begin([a], small)
    pair = Bucket((2, 1), (8, 8), 'GPU fixture')
    pool.register_bucket(pair)
    for handles in ([a, a], [a]):
        with pytest.raises(ValueError):
            pool.begin(handles, pair)
    tx = pool.begin([b, a], pair)
    stage(pool, tx)
    _, _, cq, ck, pos = pool.prepare_attention(tx, 1)
    assert cq.tolist() == g['cu_query'] and ck.tolist() == g['cu_key'] and pos.tolist() == g['positions']
    pool.abort(tx)
    tx = pool.begin([b], small)
    stage(pool, tx)
    assert pool.work(tx)['inactive_resident_key_tokens'] == g['inactive_with_B_small']
    pool.abort(tx)
    with pytest.raises(ValueError):
        pool.register_bucket(Bucket((8, 8), (8, 8), 'fixture'))


def test_query_families_shared_arena(dev):
    from qwen3_dspark_amd.persistent_kv import QueryFamily
    say('[kv] query families on a shared arena')
    pool = small_pool(dev, layers=1, slots=3, context_capacity=16, max_query_tokens=6, heads=1, dim=4)
    small, large = QueryFamily(2, 3, 2, 24, 16, 'small actual B'), QueryFamily(2, 6, 6, 32, 16, 'varying actual Q')
    pool.register_families((small, large))
    handles = [pool.add_request(r) for r in ('a', 'b', 'idle')]
    for i, h in enumerate(handles):
        x = torch.full((1, i + 1, 1, 4), float(i), device=dev)
        pool.load_prefix(h, x, x)
    pointers = {f: pool.pointers(f) for f in (small, large)}
    assert pointers[small] == pointers[large]
    before = pool.keys.clone()
    for queries in ((0, 6), (2, 3), (1, 6), (True, 5), (1, 1, 4)):
        with pytest.raises(ValueError):
            pool.begin(handles[:2], large, query_lengths=queries)
        assert pool.open_transaction is None
    with pytest.raises(ValueError):
        pool.begin(handles[:2], large)
    with pytest.raises(ValueError):
        pool.register_families((small,))
    assert torch.equal(before, pool.keys)
    for family, queries, active in ((small, (1, 2), handles[:2]), (large, (5, 1), handles[1::-1]),
                                    (small, (2, 1), handles[:2])):
        contexts = tuple(pool.length(h) for h in active)
        tx = pool.begin(active, family, query_lengths=queries)
        values = torch.arange(family.query_tokens * 4, dtype=torch.float32, device=dev).reshape(-1, 1, 4) + 20
        pool.stage_layer(tx, 0, values, values + 1)
        _, _, cuq, cuk, pos = pool.prepare_attention(tx, 0)
        assert cuq.tolist() == [0, queries[0], sum(queries)]
        assert cuk.tolist() == [0, contexts[0] + queries[0], sum(contexts) + sum(queries)]
        assert pos.tolist() == [i for c, q in zip(contexts, queries) for i in range(c, c + q)]
        old = {h: pool.request_kv(h)[0] for h in active}
        counts = {h: min(q, 2) for h, q in zip(active, queries)}
        pool.commit(tx, counts)
        offset = 0
        for h, q in zip(active, queries):
            expected = torch.cat((old[h], values[offset:offset + counts[h]][None]), dim=1)
            assert torch.equal(pool.request_kv(h)[0], expected)
            offset += q
        assert pool.pointers(family) == pointers[family]
    assert torch.equal(pool.request_kv(handles[2])[0], before[:, 2, :3])


def test_metadata_gather_commit_bit_exact_against_oracle(dev):
    """Random transactions at Qwen3 row width (bf16 [8,128]): all seven
    metadata arrays, the materialised K/V and the committed resident bytes
    equal the oracle bit for bit."""
    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV
    rng = np.random.default_rng(SEED)
    gen = torch.Generator().manual_seed(SEED)
    L, S, C, Q = 3, 6, 96, 40
    pool = PersistentTargetKV(layers=L, slots=S, context_capacity=C, max_query_tokens=Q, heads=8, dim=128, device=dev)
    handles = [pool.add_request(f'r{i}') for i in range(S)]
    lens = rng.integers(0, 40, size=S)
    for h, n in zip(handles, lens):
        kv = randn_bf16(gen, 2, L, int(n), 8, 128).to(dev)
        pool.load_prefix(h, kv[0], kv[1])
    for trial in range(4):
        active = list(rng.permutation(S)[:int(rng.integers(1, S + 1))])
        queries = tuple(int(x) for x in rng.integers(1, 8, size=len(active)))
        ceilings = tuple(int(C - q - rng.integers(0, 5)) for q in queries)
        bucket = Bucket(queries, ceilings, f'random trial {trial}')
        pool.register_bucket(bucket)
        say(f'[kv] oracle trial {trial}: active={active} q={queries}')
        hs = [handles[i] for i in active]
        ctx = [pool.length(h) for h in hs]
        tx = pool.begin(hs, bucket)
        new_k = randn_bf16(gen, L, sum(queries), 8, 128).to(dev)
        new_v = randn_bf16(gen, L, sum(queries), 8, 128).to(dev)
        for layer in range(L):
            pool.stage_layer(tx, layer, new_k[layer], new_v[layer])
        ws = pool.workspace(bucket)
        meta = semantics.txn_metadata(active, ctx, queries, C, bucket.key_capacity)
        k, v, cq, ck, pos = pool.prepare_attention(tx, 1)
        assert np.array_equal(ws.committed_indices.cpu().numpy(), meta['committed_indices'])
        assert np.array_equal(ws.scratch_indices.cpu().numpy(), meta['scratch_indices'])
        assert np.array_equal(ws.from_scratch.cpu().numpy().ravel(), meta['from_scratch'])
        assert np.array_equal(ws.valid.cpu().numpy().ravel(), meta['valid'])
        assert np.array_equal(pos.cpu().numpy(), meta['positions'])
        assert np.array_equal(cq.cpu().numpy(), meta['cu_query']) and np.array_equal(ck.cpu().numpy(), meta['cu_key'])
        res = bits(pool.keys[1])
        scr = bits(pool.scratch_keys[1])
        assert np.array_equal(bits(k), semantics.materialize(res, scr, meta))
        assert np.array_equal(bits(v), semantics.materialize(bits(pool.values[1]), bits(pool.scratch_values[1]), meta))
        counts = [int(rng.integers(0, q + 1)) for q in queries]
        expect, _ = semantics.commit(bits(pool.keys), bits(pool.scratch_keys), active, ctx, queries, counts, C)
        expect_v, _ = semantics.commit(bits(pool.values), bits(pool.scratch_values), active, ctx, queries, counts, C)
        pool.commit(tx, dict(zip(hs, counts)))
        assert np.array_equal(bits(pool.keys), expect) and np.array_equal(bits(pool.values), expect_v)
        assert [pool.length(h) for h in hs] == [c + n for c, n in zip(ctx, counts)]


def test_fused_verify_attention_parity_commit_and_second_round(dev):
    """Config: 4 requests, cached contexts U[64,512], 7 appended rows, 1 layer
    (plus a second layer), seeded accepted prefix 0..7 committed, rest
    rolled back; the next round attends over the committed rows with the
    staging fused into the attention launch."""
    from qwen3_dspark_amd.kernels import HipCapacityKernel, HipVarlenKernel
    from qwen3_dspark_amd.layout import PersistentAttentionLayout
    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV
    rng = np.random.default_rng(SEED)
    gen = torch.Generator().manual_seed(SEED)
    L, B, C = 2, 4, 1024
    pool = PersistentTargetKV(layers=L, slots=B + 1, context_capacity=C, max_query_tokens=7 * B, heads=8, dim=128, device=dev)
    handles = [pool.add_request(f'r{i}') for i in range(B + 1)]
    for h in handles:
        n = int(rng.integers(64, 513))
        kv = randn_bf16(gen, 2, L, n, 8, 128).to(dev)
        pool.load_prefix(h, kv[0], kv[1])
    # Poison every resident row that no request may read (beyond each length).
    for i, h in enumerate(handles):
        pool.keys[:, i, pool.length(h):] = float('nan')
        pool.values[:, i, pool.length(h):] = float('nan')
    active = handles[:B]
    bucket = Bucket((7,) * B, (C - 7 - 7,) * B, 'config #2 shape')
    pool.register_bucket(bucket)
    cap_kernel = HipCapacityKernel(dev)
    exact_kernel = HipVarlenKernel(dev)
    for rnd in range(2):
        ctx = [pool.length(h) for h in active]
        say(f'[verify] round {rnd} contexts={ctx}')
        tx = pool.begin(active, bucket)
        q = randn_bf16(gen, L, 7 * B, 16, 128).to(dev)
        nk = randn_bf16(gen, L, 7 * B, 8, 128).to(dev)
        nv = randn_bf16(gen, L, 7 * B, 8, 128).to(dev)
        for layer in range(L):
            if rnd == 0:
                pool.stage_layer(tx, layer, nk[layer], nv[layer])
                out = pool.attend(tx, layer, q[layer])
            else:   # staging fused into the attention launch
                out = pool.attend(tx, layer, q[layer], keys=nk[layer], values=nv[layer])
                with pytest.raises(ValueError, match='exactly once'):
                    pool.attend(tx, layer, q[layer], keys=nk[layer], values=nv[layer])
            torch.cuda.synchronize()
            assert torch.equal(pool.scratch_keys[layer, :7 * B], nk[layer])
            assert torch.equal(pool.scratch_values[layer, :7 * B], nv[layer])
            cu_q = list(range(0, 7 * B + 1, 7))
            ref = cref.verify_attention(bits(q[layer]), bits(pool.keys[layer]), bits(pool.values[layer]),
                                        bits(pool.scratch_keys[layer]), bits(pool.scratch_values[layer]),
                                        [h.index for h in active], ctx, cu_q, scale=SCALE)
            attention_gate(f64(out), ref, segments(cu_q))
            # The fused path equals exact-K attention over the materialised
            # gather bit for bit (same key lengths, so the same segment plan);
            # the capacity kernel's fixed chunks merge in another order.
            k, v, cq, ck, _ = pool.prepare_attention(tx, layer)
            keys = tuple(c + 7 for c in ctx)
            exact = SimpleNamespace(query_lengths=tx.query_lengths, key_lengths=keys, cu_query=cq, cu_key=ck,
                                    request_markers=tuple(range(B)))
            assert torch.equal(exact_kernel(q[layer], k[:sum(keys)], v[:sum(keys)], exact, scale=SCALE), out)
            layout = PersistentAttentionLayout(tx.query_lengths, keys, cq, ck,
                                               bucket.key_capacity, bucket.maximum_key_length, bucket.maximum_query_length)
            cap = cap_kernel(q[layer], k, v, layout, scale=SCALE)
            attention_gate(f64(cap), ref, segments(cu_q))
            assert float((cap.float() - out.float()).abs().max()) <= 2e-2
        counts = {h: int(rng.integers(0, 8)) for h in active}
        before = [pool.request_kv(h) for h in active]
        pool.commit(tx, counts)
        for i, h in enumerate(active):
            n = counts[h]
            got_k, got_v = pool.request_kv(h)
            assert torch.equal(got_k, torch.cat((before[i][0], nk[:, 7 * i:7 * i + n]), dim=1))
            assert torch.equal(got_v, torch.cat((before[i][1], nv[:, 7 * i:7 * i + n]), dim=1))
            # rolled-back rows never reach resident memory
            assert torch.isnan(pool.keys[:, h.index, ctx[i] + n:]).all()


def test_xcd_calibration_and_skewed_plans_meet_the_oracle(dev):
    """XCD-balanced plans (no reference counterpart): calibrate_xcd on a
    real store gives 8 speeds of mean 1 within 1 +- 0.25, and with strongly
    skewed speeds (runs of one XCD carrying 2.5x the cost of another's) the
    fused verification attention still meets the oracle; the work list's
    cuts move, the cover stays exact."""
    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV
    rng = np.random.default_rng(SEED + 3)
    gen = torch.Generator().manual_seed(SEED + 3)
    B, C = 6, 4096
    pool = PersistentTargetKV(layers=1, slots=B, context_capacity=C, max_query_tokens=7 * B, heads=8, dim=128,
                              device=dev)
    handles = [pool.add_request(f'r{i}') for i in range(B)]
    for h in handles:
        n = int(rng.integers(256, C - 7))
        kv = randn_bf16(gen, 2, 1, n, 8, 128).to(dev)
        pool.load_prefix(h, kv[0], kv[1])
    speed = pool.calibrate_xcd()
    say(f'[xcd] calibrated speeds {[round(x, 3) for x in speed]}')
    assert len(speed) == 8 and abs(sum(speed) / 8 - 1) < 1e-9 and all(0.75 <= x <= 1.25 for x in speed)
    bucket = Bucket((7,) * B, (C - 7,) * B, 'xcd plans')
    pool.register_bucket(bucket)
    ctx = [pool.length(h) for h in handles]
    cu_q = list(range(0, 7 * B + 1, 7))
    lists = []
    for skew in (None, (2.0, 0.8, 1.4, 1.0, 1.2, 0.9, 1.1, 1.0)):
        pool.set_xcd_speed(skew)
        tx = pool.begin(handles, bucket)
        lists.append(pool.workspace(bucket).work.clone())
        q = randn_bf16(gen, 7 * B, 16, 128).to(dev)
        nk = randn_bf16(gen, 7 * B, 8, 128).to(dev)
        nv = randn_bf16(gen, 7 * B, 8, 128).to(dev)
        out = pool.attend(tx, 0, q, keys=nk, values=nv)
        torch.cuda.synchronize()
        ref = cref.verify_attention(bits(q), bits(pool.keys[0]), bits(pool.values[0]), bits(pool.scratch_keys[0]),
                                    bits(pool.scratch_values[0]), [h.index for h in handles], ctx, cu_q, scale=SCALE)
        attention_gate(f64(out), ref, segments(cu_q))
        pool.abort(tx)
    assert not torch.equal(lists[0], lists[1])      # the skewed speeds moved the cuts


def test_verify_rows_without_visible_keys_in_a_tile(dev):
    """Contexts whose last key tile holds new rows visible to the later
    query rows only (c + 7 just past a 32-key or chunk boundary): every
    output stays finite and meets the oracle, fused staging or not."""
    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV
    gen = torch.Generator().manual_seed(SEED + 5)
    contexts = [26, 31, 61, 90, 1050, 1051, 2045, 300]
    B, C = len(contexts), 2112
    say(f'[verify] partial-tile visibility contexts={contexts}')
    pool = PersistentTargetKV(layers=1, slots=B, context_capacity=C, max_query_tokens=7 * B, heads=8, dim=128,
                              device=dev)
    handles = [pool.add_request(f'r{i}') for i in range(B)]
    for h, c in zip(handles, contexts):
        kv = randn_bf16(gen, 2, 1, c, 8, 128).to(dev)
        pool.load_prefix(h, kv[0], kv[1])
    bucket = Bucket((7,) * B, (C - 7,) * B, 'partial tiles')
    pool.register_bucket(bucket)
    cu_q = list(range(0, 7 * B + 1, 7))
    for fused in (False, True):
        tx = pool.begin(handles, bucket)
        q = randn_bf16(gen, 7 * B, 16, 128).to(dev)
        nk, nv = randn_bf16(gen, 7 * B, 8, 128).to(dev), randn_bf16(gen, 7 * B, 8, 128).to(dev)
        if fused:
            out = pool.attend(tx, 0, q, keys=nk, values=nv)
        else:
            pool.stage_layer(tx, 0, nk, nv)
            out = pool.attend(tx, 0, q)
        torch.cuda.synchronize()
        assert torch.isfinite(out.float()).all()
        ref = cref.verify_attention(bits(q), bits(pool.keys[0]), bits(pool.values[0]), bits(pool.scratch_keys[0]),
                                    bits(pool.scratch_values[0]), [h.index for h in handles], contexts, cu_q,
                                    scale=SCALE)
        attention_gate(f64(out), ref, segments(cu_q))
        pool.abort(tx)


def test_fused_attention_contract(dev):
    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV
    say('[verify] contract errors')
    pool = PersistentTargetKV(layers=1, slots=2, context_capacity=64, max_query_tokens=8, heads=8, dim=128, device=dev)
    a = pool.add_request('a')
    bucket = Bucket((3,), (10,), 'contract')
    pool.register_bucket(bucket)
    tx = pool.begin([a], bucket)
    q = torch.zeros(3, 16, 128, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match='scratch missing'):
        pool.attend(tx, 0, q)
    kv = torch.zeros(3, 8, 128, dtype=torch.bfloat16, device=dev)
    pool.stage_layer(tx, 0, kv, kv)
    for bad in (q.float(), q[:2], q.cpu()):
        with pytest.raises(ValueError):
            pool.attend(tx, 0, bad)
    with pytest.raises(ValueError):
        pool.attend(tx, 0, q, scale=1.0)
    out = pool.attend(tx, 0, q)
    assert torch.equal(out, torch.zeros_like(out))
    pool.abort(tx)
