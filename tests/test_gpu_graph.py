"""Captured verification rounds (VerificationGraph) and the capacity-tail
kernel under graph capture, replayed several times with eager work and
synchronisations between replays; every replay is checked against the
eager result of the same inputs (bit for bit) and against the oracle
(persistent_qwen_graph.py:97-275; scripts/probe_native_capacity_graph.py
protocol for the capacity kernel)."""
import numpy as np
import pytest
import torch

from helpers import SCALE, SEED, attention_gate, bits, f64, randn_bf16, segments
from oracle import attention, cref

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda:0')


def say(*a):
    print(*a, flush=True)


def test_verification_graph_replays_equal_eager_rounds():
    """6 requests, contexts U[64, 900], 7 new rows each, 3 layers; four
    rounds: eager attention (then abort), the same inputs through the graph,
    commit of a seeded accepted prefix, so every replay sees new lengths."""
    from qwen3_dspark_amd.graph import VerificationGraph
    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV
    rng = np.random.default_rng(SEED)
    gen = torch.Generator().manual_seed(SEED)
    L, B, C = 3, 6, 1024
    pool = PersistentTargetKV(layers=L, slots=B, context_capacity=C, max_query_tokens=7 * B, heads=8, dim=128,
                              device=DEV)
    handles = [pool.add_request(f'r{i}') for i in range(B)]
    for h in handles:
        n = int(rng.integers(64, 901))
        kv = randn_bf16(gen, 2, L, n, 8, 128).to(DEV)
        pool.load_prefix(h, kv[0], kv[1])
    bucket = Bucket((7,) * B, (C - 7 * 5,) * B, 'graph test')
    pool.register_bucket(bucket)
    graph = VerificationGraph(pool, bucket).capture()
    for rnd in range(4):
        ctx = [pool.length(h) for h in handles]
        say(f'[graph] round {rnd} contexts={ctx}')
        q = randn_bf16(gen, L, 7 * B, 16, 128).to(DEV)
        nk = randn_bf16(gen, L, 7 * B, 8, 128).to(DEV)
        nv = randn_bf16(gen, L, 7 * B, 8, 128).to(DEV)
        tx = pool.begin(handles, bucket)
        eager = [pool.attend(tx, l, q[l], keys=nk[l], values=nv[l]) for l in range(L)]
        pool.abort(tx)
        torch.cuda.synchronize()
        tx = pool.begin(handles, bucket)
        graph.query.copy_(q)
        graph.keys.copy_(nk)
        graph.values.copy_(nv)
        done = graph.submit(tx)
        with pytest.raises(ValueError):
            pool.commit(tx, {h: 0 for h in handles})      # scratch not published yet
        out = graph.wait(done)
        for l in range(L):
            assert torch.equal(out[l], eager[l]), f'layer {l} replay differs from eager'
            assert torch.equal(pool.scratch_keys[l, :7 * B], nk[l])
            assert torch.equal(pool.scratch_values[l, :7 * B], nv[l])
        cu_q = list(range(0, 7 * B + 1, 7))
        ref = cref.verify_attention(bits(q[rnd % L]), bits(pool.keys[rnd % L]), bits(pool.values[rnd % L]),
                                    bits(pool.scratch_keys[rnd % L]), bits(pool.scratch_values[rnd % L]),
                                    [h.index for h in handles], ctx, cu_q, scale=SCALE)
        attention_gate(f64(out[rnd % L]), ref, segments(cu_q))
        counts = {h: int(rng.integers(0, 8)) for h in handles}
        before = [pool.request_kv(h) for h in handles]
        pool.commit(tx, counts)
        for i, h in enumerate(handles):
            got_k, _ = pool.request_kv(h)
            assert torch.equal(got_k, torch.cat((before[i][0], nk[:, 7 * i:7 * i + counts[h]]), dim=1))


def test_verification_graph_protocol_errors():
    from qwen3_dspark_amd.graph import VerificationGraph
    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV
    pool = PersistentTargetKV(layers=2, slots=3, context_capacity=256, max_query_tokens=8, heads=8, dim=128,
                              device=DEV)
    hs = [pool.add_request(f'r{i}') for i in range(2)]
    for h in hs:
        kv = torch.zeros(2, 2, 16, 8, 128, dtype=torch.bfloat16, device=DEV)
        pool.load_prefix(h, kv[0], kv[1])
    bucket, other = Bucket((3, 4), (100, 100), 'graph'), Bucket((7,), (100,), 'other')
    pool.register_bucket(bucket)
    pool.register_bucket(other)
    graph = VerificationGraph(pool, bucket)
    tx = pool.begin(hs, bucket)
    with pytest.raises(RuntimeError, match='capture'):
        graph.submit(tx)
    pool.abort(tx)
    graph.capture()
    with pytest.raises(ValueError, match='already'):
        graph.capture()
    tx = pool.begin(hs[:1], other)
    with pytest.raises(ValueError):
        graph.submit(tx)                                    # transaction of another bucket
    pool.abort(tx)
    tx = pool.begin(hs, bucket)
    pool.stage_layer(tx, 0, torch.zeros(7, 8, 128, dtype=torch.bfloat16, device=DEV),
                     torch.zeros(7, 8, 128, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(ValueError):
        graph.submit(tx)                                    # eager staging already started
    pool.abort(tx)
    tx = pool.begin(hs, bucket)
    done = graph.submit(tx)
    with pytest.raises(ValueError):
        graph.submit(tx)                                    # one replay per transaction
    graph.wait(done)
    with pytest.raises(ValueError):
        graph.wait(done)                                    # already published
    pool.commit(tx, {hs[0]: 3, hs[1]: 4})
    assert [pool.length(h) for h in hs] == [19, 20]


def test_capacity_kernel_graph_replay():
    """The reference's capacity-tail graph probe: Q=(1,4), ceilings 144,
    capacity 293, fixed maximum K 148; one capture, replays at contexts
    (128,128), (129,131), (130,135) with new queries and K/V written in
    place, each replay bit-identical to the eager zero-tail call and
    unaffected by finite or NaN tails."""
    from qwen3_dspark_amd.kernels import HipCapacityKernel
    from qwen3_dspark_amd.layout import PersistentAttentionLayout
    gen = torch.Generator().manual_seed(SEED + 5)
    kernel = HipCapacityKernel(DEV)
    q_lens, kcap = (1, 4), 293
    cu_q = torch.tensor([0, 1, 5], dtype=torch.int32, device=DEV)
    cu_k = torch.tensor([0, 129, 261], dtype=torch.int32, device=DEV)
    q = torch.zeros(5, 16, 128, dtype=torch.bfloat16, device=DEV)
    k = torch.zeros(kcap, 8, 128, dtype=torch.bfloat16, device=DEV)
    v = torch.zeros_like(k)
    layout = PersistentAttentionLayout(q_lens, (129, 132), cu_q, cu_k, kcap, 148, 4)
    kernel(q, k, v, layout, scale=SCALE)                  # eager warm-up: validation and workspace
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=DEV)
    stream.wait_stream(torch.cuda.current_stream(DEV))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        static_out = kernel(q, k, v, layout, scale=SCALE)
    torch.cuda.current_stream(DEV).wait_stream(stream)
    for contexts in ([128, 128], [129, 131], [130, 135]):
        k_lens = [c + n for c, n in zip(contexts, q_lens)]
        say(f'[capacity graph] contexts={contexts}')
        qq = randn_bf16(gen, 5, 16, 128)
        kk, vv = randn_bf16(gen, kcap, 8, 128), randn_bf16(gen, kcap, 8, 128)
        eager_layout = PersistentAttentionLayout(q_lens, tuple(k_lens),
                                                 torch.tensor([0, 1, 5], dtype=torch.int32, device=DEV),
                                                 torch.tensor([0, k_lens[0], sum(k_lens)], dtype=torch.int32,
                                                              device=DEV), kcap, 148, 4)
        tail = slice(sum(k_lens), kcap)
        kz, vz = kk.clone(), vv.clone()
        kz[tail], vz[tail] = 0.0, 0.0
        eager = kernel(qq.to(DEV), kz.to(DEV), vz.to(DEV), eager_layout, scale=SCALE)
        for fill in ((0.0, 0.0), (100.0, -100.0), (float('nan'), float('nan'))):
            kt, vt = kk.clone(), vv.clone()
            kt[tail], vt[tail] = fill
            q.copy_(qq.to(DEV))
            k.copy_(kt.to(DEV))
            v.copy_(vt.to(DEV))
            cu_k.copy_(torch.tensor([0, k_lens[0], sum(k_lens)], dtype=torch.int32))
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(static_out, eager), f'replay differs from eager (tail {fill})'
        ref = attention.varlen_attention(f64(qq), f64(kz), f64(vz), [0, 1, 5], [0, k_lens[0], sum(k_lens)],
                                         causal=True, scale=SCALE)
        attention_gate(f64(static_out), ref, segments([0, 1, 5]))
