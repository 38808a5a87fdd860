"""The persistent KV store's host state machine on the CPU: the reference's
store, family and external-writer tests (tests/test_persistent_target_kv.py,
tests/test_query_family.py:26-69, tests/test_persistent_qwen_graph.py:28-106)
run against PersistentTargetKV with the CPU stand-in of its device half
(tests/kv_fake.py), plus the phase/transition table and poisoning.  The GPU
versions of the same cases (tests/test_gpu_kv.py) run the HIP device half."""
import copy
import itertools

import pytest
import torch

from kv_fake import store
from qwen3_dspark_amd.persistent_kv import (_REFUSALS, _TRANSITIONS, Bucket, Phase, QueryFamily, Slot,
                                            PersistentTargetKV)


def prefix(pool, handle, n, offset):
    x = torch.arange(pool.layers * n * pool.heads * pool.dim, dtype=pool.dtype).reshape(
        pool.layers, n, pool.heads, pool.dim) + offset
    pool.load_prefix(handle, x, x + 0.25)
    return x, x + 0.25


def stage(pool, tx):
    q = sum(tx.query_lengths)
    x = torch.arange(pool.layers * q * pool.heads * pool.dim, dtype=pool.dtype).reshape(
        pool.layers, q, pool.heads, pool.dim) + 10000
    for layer in range(pool.layers):
        pool.stage_layer(tx, layer, x[layer], x[layer] + 0.5)
    return x, x + 0.5


def test_growing_context_stable_buffers_exact_q_and_independent_scratch(golden):
    g = golden['txn_growing_context']
    pool = store()
    a, b, idle = pool.add_request('A'), pool.add_request('B'), pool.add_request('idle')
    ak, av = prefix(pool, a, 3, 100)
    bk, _ = prefix(pool, b, 5, 500)
    ik, _ = prefix(pool, idle, 9, 900)
    bucket = Bucket(tuple(g['bucket'][0]), tuple(g['bucket'][1]), 'CPU fixture')
    pool.register_bucket(bucket)
    pointers = pool.pointers(bucket)
    before = pool.keys.clone()
    tx = pool.begin([a, b], bucket)
    sk, sv = stage(pool, tx)
    assert torch.equal(before, pool.keys)
    for layer in range(pool.layers):
        k, v, cq, ck, pos = pool.prepare_attention(tx, layer)
        assert torch.equal(k[:13], torch.cat((ak[layer], sk[layer, :2], bk[layer], sk[layer, 2:])))
        assert torch.equal(k[13:], torch.zeros_like(k[13:]))
        assert cq.tolist() == g['cu_query'] and ck.tolist() == g['cu_key'] and pos.tolist() == g['positions']
    work = pool.work(tx)
    assert work['logical_query_tokens'] == work['physical_query_tokens']
    assert work['inactive_resident_key_tokens'] == g['inactive_resident_key_tokens']
    assert (work['physical_key_capacity'], work['padded_key_capacity']) == (g['physical_key_capacity'],
                                                                            g['padded_key_capacity'])
    assert pool.commit(tx, {a: 1, b: 2}) == dict(committed_tokens=3, copied_kv_bytes=2 * 2 * 2 * 4 * 4 * 3)
    assert torch.equal(pool.request_kv(a)[0], torch.cat((ak, sk[:, :1]), dim=1))
    assert torch.equal(pool.request_kv(b)[0], torch.cat((bk, sk[:, 2:4]), dim=1))
    assert torch.equal(pool.request_kv(idle)[0], ik)
    second = pool.begin([a, b], bucket)
    stage(pool, second)
    _, _, _, ck, pos = pool.prepare_attention(second, 0)
    assert ck.tolist() == g['second_cu_key'] and pos.tolist() == g['second_positions']
    assert pool.pointers(bucket) == pointers
    pool.abort(second)
    assert pool.phase is Phase.IDLE


def test_abort_no_commit_and_slot_reuse_cannot_read_old_bytes(golden):
    pool = store()
    old = pool.add_request('same')
    prefix(pool, old, 7, 77)
    bucket = Bucket((1,), (10,), 'CPU fixture')
    pool.register_bucket(bucket)
    before = pool.keys.clone()
    tx = pool.begin([old], bucket)
    stage(pool, tx)
    pool.abort(tx)
    assert torch.equal(before, pool.keys) and pool.length(old) == 7
    pool.remove_request(old)
    fresh = pool.add_request('same')
    assert old.index == fresh.index and old.incarnation != fresh.incarnation
    foreign = store().add_request('same')
    for stale in (old, copy.copy(fresh), Slot(fresh.request, fresh.index, fresh.incarnation), foreign):
        with pytest.raises(ValueError, match='Stale or foreign'):
            pool.length(stale)
    tx = pool.begin([fresh], bucket)
    sk, _ = stage(pool, tx)
    k, _, _, ck, pos = pool.prepare_attention(tx, 0)
    assert ck.tolist() == golden['txn_slot_reuse']['cu_key'] and pos.tolist() == golden['txn_slot_reuse']['positions']
    assert torch.equal(k[:1], sk[0]) and int(torch.count_nonzero(k[1:])) == 0
    pool.commit(tx, {fresh: 1})
    assert pool.length(fresh) == 1


def test_lowest_vacant_slot_is_reused_and_capacity_is_finite():
    pool = store()
    handles = [pool.add_request(r) for r in 'abc']
    assert [h.index for h in handles] == [0, 1, 2]
    with pytest.raises(ValueError, match='capacity exhausted'):
        pool.add_request('d')
    for bad in ('', None, 'b'):
        with pytest.raises(ValueError, match='New nonempty'):
            pool.add_request(bad)
    pool.remove_request(handles[2])
    pool.remove_request(handles[0])
    again = pool.add_request('e')
    assert (again.index, again.incarnation) == (0, 2)
    assert pool.add_request('a').index == 2


def test_invalid_transaction_and_commit_fail_before_resident_mutation(golden):
    pool = store()
    a = pool.add_request('A')
    prefix(pool, a, 2, 1)
    bucket = Bucket((2,), (4,), 'CPU fixture')
    pool.register_bucket(bucket)
    before = pool.keys.clone()
    tx = pool.begin([a], bucket)
    for call in (lambda: pool.remove_request(a), lambda: pool.add_request('B'), lambda: pool.begin([a], bucket),
                 lambda: pool.register_bucket(bucket), lambda: pool.load_prefix(a, before[:, 0], before[:, 0])):
        with pytest.raises(RuntimeError, match='Outstanding'):
            call()
    with pytest.raises(ValueError, match='Layer scratch missing'):
        pool.prepare_attention(tx, 0)
    with pytest.raises(ValueError, match='Complete layer scratch'):
        pool.commit(tx, {a: 1})
    stage(pool, tx)
    for bad in golden['txn_invalid_commit']['invalid_counts'] + [True]:
        with pytest.raises(ValueError, match='valid verified prefix'):
            pool.commit(tx, {a: bad})
    with pytest.raises(ValueError, match='Stale, copied or foreign transaction'):
        pool.commit(copy.copy(tx), {a: 1})
    assert torch.equal(before, pool.keys) and 'commit' not in pool.kv_device.calls
    pool.commit(tx, {a: 0})
    assert torch.equal(before, pool.keys)
    with pytest.raises(ValueError, match='Stale'):
        pool.abort(tx)


def test_failed_metadata_preparation_never_publishes_or_revives_transaction(golden):
    pool = store()
    a = pool.add_request('A')
    prefix(pool, a, 3, 3)
    bucket = Bucket((2,), (8,), 'CPU fixture')
    pool.register_bucket(bucket)
    old = pool.begin([a], bucket)
    pool.abort(old)
    before = pool.keys.clone()
    pool.kv_device.fail = 'build_metadata'
    with pytest.raises(RuntimeError, match='injected'):
        pool.begin([a], bucket)
    assert pool.open_transaction is None and pool.phase is Phase.IDLE and not pool.failed
    assert torch.equal(pool.keys, before)
    with pytest.raises(ValueError):
        pool.abort(old)
    tx = pool.begin([a], bucket)
    stage(pool, tx)
    _, _, cq, ck, pos = pool.prepare_attention(tx, 0)
    g = golden['txn_retry_metadata']
    assert cq.tolist() == g['cu_query'] and ck.tolist() == g['cu_key'] and pos.tolist() == g['positions']
    pool.abort(tx)


def test_ordered_shape_bounds_and_active_subset(golden):
    g = golden['txn_reordered_subset']
    pool = store()
    a, b = pool.add_request('A'), pool.add_request('B')
    prefix(pool, a, 8, 0)
    prefix(pool, b, 4, 0)
    small = Bucket((1,), (7,), 'CPU fixture')
    pool.register_bucket(small)
    with pytest.raises(ValueError, match='applicability'):
        pool.begin([a], small)
    pair = Bucket((2, 1), (8, 8), 'CPU fixture')
    pool.register_bucket(pair)
    with pytest.raises(ValueError, match='unique'):
        pool.begin([a, a], pair)
    with pytest.raises(ValueError, match='Registered exact-query bucket'):
        pool.begin([a], pair)
    tx = pool.begin([b, a], pair)
    stage(pool, tx)
    _, _, cq, ck, pos = pool.prepare_attention(tx, 1)
    assert cq.tolist() == g['cu_query'] and ck.tolist() == g['cu_key'] and pos.tolist() == g['positions']
    pool.abort(tx)
    tx = pool.begin([b], small)
    stage(pool, tx)
    assert pool.work(tx)['inactive_resident_key_tokens'] == g['inactive_with_B_small']
    pool.abort(tx)
    with pytest.raises(ValueError, match='capacity'):
        pool.register_bucket(Bucket((8, 8), (8, 8), 'fixture'))


def test_xcd_speeds_are_validated_normalised_clipped_and_admin_only():
    """XCD-balanced plans (no reference counterpart): explicit speeds are
    checked and normalised to mean 1, calibration clips the measured
    speeds to 1 +- clip, and neither may change during a transaction."""
    pool = store()
    assert pool.xcd_speed is None
    pool.set_xcd_speed([2.0, 2.0, 2.0, 2.0, 4.0, 4.0, 4.0, 4.0])
    assert pool.xcd_speed == (2 / 3,) * 4 + (4 / 3,) * 4
    for bad in ([1.0] * 7, [1.0] * 7 + [0.0], [1.0] * 7 + [float('nan')], [1.0] * 7 + [-1.0]):
        with pytest.raises(ValueError, match='8 positive finite'):
            pool.set_xcd_speed(bad)
    pool.set_xcd_speed(None)
    assert pool.xcd_speed is None
    got = pool.calibrate_xcd(clip=0.1)                       # the stand-in measures 1.3, 0.7, 1, ...
    assert pool.kv_device.calls[-1] == 'measure_xcd_speed'
    assert got == pytest.approx([1.1, 0.9, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0])
    h = pool.add_request('a')
    bucket = Bucket((1,), (4,), 'xcd')
    pool.register_bucket(bucket)
    tx = pool.begin([h], bucket)
    with pytest.raises(RuntimeError, match='Outstanding verification transaction'):
        pool.set_xcd_speed(None)
    with pytest.raises(RuntimeError, match='Outstanding verification transaction'):
        pool.calibrate_xcd()
    with pytest.raises(RuntimeError, match='Outstanding verification transaction'):
        pool.set_slot_balance(False)
    pool.abort(tx)
    # the second-slot share: on by default, a bool, admin-only
    assert pool.slot_balance is True
    pool.set_slot_balance(False)
    assert pool.slot_balance is False and pool.kv_device.slot_balance is False
    with pytest.raises(ValueError, match='True or False'):
        pool.set_slot_balance(1)


def test_attention_staging_matches_independent_variable_prefix_sdpa():
    """tests/test_persistent_target_kv.py:133-147: each request's slice of the
    materialised K/V gives exactly the attention over its true rows."""
    pool = store(heads=2, dim=4)
    a, b = pool.add_request('A'), pool.add_request('B')
    ak, av = prefix(pool, a, 3, 0)
    bk, bv = prefix(pool, b, 5, 1)
    bucket = Bucket((2, 1), (10, 10), 'CPU fixture')
    pool.register_bucket(bucket)
    tx = pool.begin([a, b], bucket)
    sk, sv = stage(pool, tx)
    queries = torch.randn(3, 4, 4, generator=torch.Generator().manual_seed(1))
    k, v, _, ck, _ = pool.prepare_attention(tx, 0)
    for i, (pk, pv, off, n) in enumerate(((ak[0], av[0], 0, 2), (bk[0], bv[0], 2, 1))):
        true_k, true_v = torch.cat((pk, sk[0, off:off + n])), torch.cat((pv, sv[0, off:off + n]))
        q = queries[off:off + n].transpose(0, 1)[None]
        visible = torch.arange(len(true_k))[None, :] <= torch.arange(len(pk), len(pk) + n)[:, None]

        def attention(kk, vv):
            return torch.nn.functional.scaled_dot_product_attention(
                q, kk.transpose(0, 1)[None], vv.transpose(0, 1)[None], attn_mask=visible[None, None], enable_gqa=True)
        assert torch.equal(attention(k[ck[i]:ck[i + 1]], v[ck[i]:ck[i + 1]]), attention(true_k, true_v))
    pool.abort(tx)


def test_query_families_share_one_arena_and_bound_actual_shapes():
    """tests/test_query_family.py:26-69."""
    p = store(layers=1, slots=3, context_capacity=16, max_query_tokens=6, heads=1, dim=4)
    small, large = QueryFamily(2, 3, 2, 24, 16, 'small actual B'), QueryFamily(2, 6, 6, 32, 16, 'varying Q')
    p.register_families((small, large))
    handles = [p.add_request(r) for r in ('a', 'b', 'idle')]
    for i, h in enumerate(handles):
        x = torch.full((1, i + 1, 1, 4), float(i))
        p.load_prefix(h, x, x)
    pointers = {f: p.pointers(f) for f in (small, large)}
    assert pointers[small] == pointers[large]
    before = p.keys.clone()
    for queries in ((0, 6), (2, 3), (1, 6), (True, 5), (1, 1, 4)):
        with pytest.raises(ValueError):
            p.begin(handles[:2], large, query_lengths=queries)
        assert p.open_transaction is None
    with pytest.raises(ValueError, match='actual ordered query lengths'):
        p.begin(handles[:2], large)
    with pytest.raises(ValueError, match='no dynamic extension'):
        p.register_families((small,))
    with pytest.raises(ValueError, match='shared arena'):
        p.register_bucket(QueryFamily(1, 1, 1, 4, 4, 'undeclared'))
    assert torch.equal(before, p.keys)
    for family, queries, active in ((small, (1, 2), handles[:2]), (large, (5, 1), handles[1::-1]),
                                    (small, (2, 1), handles[:2])):
        contexts = tuple(p.length(h) for h in active)
        tx = p.begin(active, family, query_lengths=queries)
        assert tx.query_lengths == queries
        values = torch.arange(family.query_tokens * 4, dtype=torch.float32).reshape(-1, 1, 4) + 20
        p.stage_layer(tx, 0, values, values + 1)
        _, _, cuq, cuk, pos = p.prepare_attention(tx, 0)
        assert cuq.tolist() == [0, queries[0], sum(queries)]
        assert cuk.tolist() == [0, contexts[0] + queries[0], sum(contexts) + sum(queries)]
        assert pos.tolist() == [i for c, q in zip(contexts, queries) for i in range(c, c + q)]
        work = p.work(tx)
        assert work['physical_query_tokens'] == work['logical_query_tokens'] == sum(queries)
        assert work['workspace_is_shared']
        assert work['shared_arena_allocated_bytes'] == p.workspace_bytes(p.family_arena_shape((small, large)))
        old = {h: p.request_kv(h)[0] for h in active}
        counts = {h: min(q, 2) for h, q in zip(active, queries)}
        p.commit(tx, counts)
        offset = 0
        for h, q in zip(active, queries):
            assert torch.equal(p.request_kv(h)[0], torch.cat((old[h], values[offset:offset + counts[h]][None]), dim=1))
            offset += q
        assert p.pointers(family) == pointers[family]
    assert torch.equal(p.request_kv(handles[2])[0], before[:, 2, :3])
    old = handles[0]
    p.remove_request(old)
    fresh = p.add_request('a')
    with pytest.raises(ValueError):
        p.begin((old, handles[1]), small, query_lengths=(1, 2))
    tx = p.begin((fresh, handles[1]), small, query_lengths=(1, 2))
    assert tx.context_lengths[0] == 0
    p.abort(tx)


class Writer:
    """A minimal external writer: an event object per submission that
    becomes observable once `ready` is set (CPUReplayEmulator's role in
    tests/test_persistent_qwen_graph.py)."""

    def __init__(self):
        self.ready, self.raises, self.events = False, False, []

    def submit(self, receipt):
        event = object()
        self.events.append((event, receipt))
        return event

    def complete(self, event, receipt):
        if self.raises:
            raise RuntimeError('injected completion failure')
        return self.ready and any(e is event and r is receipt for e, r in self.events)


def test_exact_program_transaction_generation_event_and_complete_layers():
    """tests/test_persistent_qwen_graph.py:63-91."""
    p = store(layers=2, slots=1, context_capacity=8, max_query_tokens=2, heads=1, dim=2)
    h = p.add_request('a')
    b = Bucket((2,), (4,), 'receipt test')
    p.register_bucket(b)
    backend = Writer()
    writer = p.register_external_writer(b, (0, 1), backend.complete)
    with pytest.raises(ValueError, match='complete ordered layer signature'):
        p.register_external_writer(b, (0,), backend.complete)
    tx = p.begin([h], b)
    with pytest.raises(ValueError, match='exact registered external writer'):
        p.prepare_external_write(tx, copy.copy(writer))
    receipt = p.prepare_external_write(tx, writer)
    assert p.phase is Phase.PREPARED
    with pytest.raises(ValueError, match='unpublished'):
        p.complete_external_write(receipt)
    with pytest.raises(ValueError, match='Cannot mix'):
        p.stage_layer(tx, 0, torch.ones(2, 1, 2), torch.ones(2, 1, 2))
    event = backend.submit(receipt)
    p.submit_external_write(receipt, event)
    with pytest.raises(ValueError, match='exactly once'):
        p.submit_external_write(receipt, event)
    with pytest.raises(RuntimeError, match='not been observed'):
        p.complete_external_write(receipt)
    with pytest.raises(RuntimeError, match='unfinished external write'):
        p.abort(tx)
    with pytest.raises(ValueError, match='Complete layer scratch'):
        p.commit(tx, {h: 1})
    backend.ready = True
    with pytest.raises(ValueError, match='receipt'):
        p.complete_external_write(copy.copy(receipt))
    p.scratch_keys.fill_(2)
    p.scratch_values.fill_(3)
    p.complete_external_write(receipt)
    assert p.phase is Phase.PUBLISHED and p.staged_layers() == 2
    p.commit(tx, {h: 1})
    assert torch.equal(p.request_kv(h)[0], torch.full((2, 1, 1, 2), 2.))
    tx2 = p.begin([h], b)
    r2 = p.prepare_external_write(tx2, writer)
    assert r2.generation > receipt.generation
    with pytest.raises(ValueError, match='receipt'):
        p.complete_external_write(receipt)
    p.submit_external_write(r2, event)
    with pytest.raises(RuntimeError, match='not been observed'):
        p.complete_external_write(r2)
    p.invalidate()
    with pytest.raises(RuntimeError, match='invalidated'):
        p.commit(tx2, {h: 0})


def test_stale_scratch_address_and_foreign_receipts_fail_closed():
    """tests/test_persistent_qwen_graph.py:93-106, plus a completion checker
    that raises and a changed workspace view."""
    def make():
        p = store(layers=1, slots=1, context_capacity=4, max_query_tokens=1, heads=1, dim=2)
        h = p.add_request('a')
        b = Bucket((1,), (2,), 'fixture')
        p.register_bucket(b)
        backend = Writer()
        writer = p.register_external_writer(b, (0,), backend.complete)
        tx = p.begin([h], b)
        return p, backend, tx, p.prepare_external_write(tx, writer)
    p, _, _, r = make()
    other, _, _, foreign = make()
    with pytest.raises(ValueError, match='foreign external write receipt'):
        p.submit_external_write(foreign, None)
    p.scratch_keys = p.scratch_keys.clone()
    with pytest.raises(RuntimeError, match='allocation changed'):
        p.submit_external_write(r, None)
    assert p.failed and p.phase is Phase.POISONED
    other.abort(foreign.transaction)
    p, _, tx, r = make()
    ws = p.workspace(tx.bucket)
    ws.keys = ws.keys.transpose(1, 2)
    with pytest.raises(RuntimeError, match='view/layout changed'):
        p.submit_external_write(r, None)
    assert p.failed
    p, backend, tx, r = make()
    p.submit_external_write(r, backend.submit(r))
    backend.raises = True
    with pytest.raises(RuntimeError, match='injected completion'):
        p.abort(tx)
    assert p.failed


def test_device_failures_poison_the_store():
    """A failed resident write (prefix bootstrap or commit) poisons the store:
    every later call fails closed with the same error."""
    p = store()
    a = p.add_request('A')
    p.kv_device.fail = 'write_prefix'
    with pytest.raises(RuntimeError, match='injected'):
        prefix(p, a, 2, 0)
    assert p.failed
    for call in (lambda: p.add_request('B'), lambda: p.length(a), lambda: p.request_kv(a),
                 lambda: p.register_bucket(Bucket((1,), (2,), 'x'))):
        with pytest.raises(RuntimeError, match='invalidated'):
            call()
    p = store()
    a = p.add_request('A')
    prefix(p, a, 2, 0)
    b = Bucket((2,), (4,), 'fixture')
    p.register_bucket(b)
    tx = p.begin([a], b)
    stage(p, tx)
    p.kv_device.fail = 'commit'
    with pytest.raises(RuntimeError, match='injected'):
        p.commit(tx, {a: 1})
    assert p.failed and p.open_transaction is tx
    with pytest.raises(RuntimeError, match='invalidated'):
        p.abort(tx)


def test_transition_table_admits_exactly_the_listed_events():
    """Every (phase, event) pair: the table's next phase, or the event's
    refusal with its class and message; a poisoned store refuses all."""
    events = sorted(_REFUSALS)
    for phase, event in itertools.product(Phase, events):
        p = store()
        p._phase = phase
        if phase is Phase.POISONED:
            with pytest.raises(RuntimeError, match='invalidated'):
                p._permit(event)
            continue
        nxt = _TRANSITIONS[phase].get(event)
        if nxt is not None:
            assert p._permit(event) is nxt
        else:
            cls, message = _REFUSALS[event]
            with pytest.raises(cls) as info:
                p._permit(event)
            assert type(info.value) is cls and str(info.value) == message
    assert set(_TRANSITIONS) == set(Phase) - {Phase.POISONED}
    assert all(set(row) <= set(events) for row in _TRANSITIONS.values())


def test_hip_device_half_refuses_without_a_gpu():
    with pytest.raises(RuntimeError, match='gfx950'):
        PersistentTargetKV(layers=1, slots=1, context_capacity=4, max_query_tokens=1, heads=8, dim=128, device='cpu')
    with pytest.raises(ValueError, match='16 bytes'):
        PersistentTargetKV(layers=1, slots=1, context_capacity=4, max_query_tokens=1, heads=1, dim=2,
                           dtype=torch.float32, device='cpu')


def test_real_tiny_qwen_kv_commit_matches_independent_prefix_forward():
    """tests/test_persistent_target_kv.py:149-184: KV from a real tiny HF
    Qwen3 staged and committed through the store equals the KV of a forward
    over the committed prefix."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    torch.manual_seed(340)
    config = Qwen3Config(vocab_size=64, hidden_size=32, intermediate_size=48, num_hidden_layers=2,
                         num_attention_heads=4, num_key_value_heads=2, head_dim=8, max_position_embeddings=128,
                         attention_dropout=0.)
    config._attn_implementation = 'sdpa'
    model = Qwen3ForCausalLM(config).eval()
    pool = store(layers=2, slots=2, context_capacity=24, max_query_tokens=5, heads=2, dim=8)
    handles = (pool.add_request('A'), pool.add_request('B'))
    prefixes = (torch.tensor([[1, 2, 3]]), torch.tensor([[4, 5, 6, 7, 8]]))
    chunks = (torch.tensor([[9, 10]]), torch.tensor([[11, 12, 13]]))
    old, new = [], []

    def extract(cache):
        return tuple(torch.stack([getattr(layer, n)[0].transpose(0, 1) for layer in cache.layers])
                     for n in ('keys', 'values'))
    with torch.no_grad():
        for h, prompt, chunk in zip(handles, prefixes, chunks):
            out = model(prompt, use_cache=True)
            k, v = extract(out.past_key_values)
            old.append((k.clone(), v.clone()))
            pool.load_prefix(h, k, v)
            verified = model(chunk, past_key_values=out.past_key_values, use_cache=True)
            k, v = extract(verified.past_key_values)
            new.append((k[:, prompt.shape[1]:], v[:, prompt.shape[1]:]))
        bucket = Bucket((2, 3), (12, 12), 'tiny Qwen CPU fixture')
        pool.register_bucket(bucket)
        tx = pool.begin(handles, bucket)
        snapshot = pool.keys.clone()
        for layer in range(pool.layers):
            pool.stage_layer(tx, layer, torch.cat([x[0][layer] for x in new]), torch.cat([x[1][layer] for x in new]))
            k, _, _, ck, _ = pool.prepare_attention(tx, layer)
            for i in range(2):
                assert torch.equal(k[ck[i]:ck[i + 1]], torch.cat((old[i][0][layer], new[i][0][layer])))
        assert torch.equal(snapshot, pool.keys)
        pool.commit(tx, dict(zip(handles, (1, 2))))
        for h, prompt, chunk, n in zip(handles, prefixes, chunks, (1, 2)):
            expected = model(torch.cat((prompt, chunk[:, :n]), dim=1), use_cache=True)
            ek, ev = extract(expected.past_key_values)
            actual = pool.request_kv(h)
            torch.testing.assert_close(actual[0], ek, rtol=1e-5, atol=1e-6)
            torch.testing.assert_close(actual[1], ev, rtol=1e-5, atol=1e-6)
