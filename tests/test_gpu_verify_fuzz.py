"""Seeded random verification transactions against the oracle
(persistent_target_kv.py:369-499 transaction, persistent_qwen_target.py:30-42
bottom-right attention): request counts, context lengths (empty included),
per-request query lengths 1..8, idle slots, plans with random XCD speeds and
the second-slot share on or off, two rounds with the new rows staged by the
attention launch and a random accepted prefix committed in between.  Each
layer meets the oracle gate, the scratch holds the new rows bit for bit,
commits append exactly the accepted rows, and rows past every length (NaN)
are never read."""
import numpy as np
import pytest
import torch

from helpers import SCALE, SEED, attention_gate, bits, f64, randn_bf16, segments
from oracle import cref

pytestmark = pytest.mark.gpu

CASES = 12


@pytest.fixture(scope='module')
def dev():
    from qwen3_dspark_amd._device import require_gfx950
    return require_gfx950('cuda')


@pytest.mark.parametrize('case', range(CASES))
def test_random_verification_transactions(dev, case):
    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV
    rng = np.random.default_rng(SEED + 9000 + case)
    gen = torch.Generator().manual_seed(SEED + 9000 + case)
    L, C = 2, 2048
    n_act = int(rng.integers(1, 13))
    n_idle = int(rng.integers(0, 3))
    qls = [int(rng.integers(1, 9)) for _ in range(n_act)]
    pool = PersistentTargetKV(layers=L, slots=n_act + n_idle, context_capacity=C, max_query_tokens=sum(qls),
                              heads=8, dim=128, device=dev)
    handles = [pool.add_request(f'r{i}') for i in range(n_act + n_idle)]
    lengths = []
    for h in handles:
        n = int(rng.choice([0, 1, 31, 32, 33])) if rng.random() < 0.3 else int(rng.integers(0, C - 40))
        lengths.append(n)
        if n:
            kv = randn_bf16(gen, 2, L, n, 8, 128).to(dev)
            pool.load_prefix(h, kv[0], kv[1])
    for i, h in enumerate(handles):
        pool.keys[:, i, pool.length(h):] = float('nan')
        pool.values[:, i, pool.length(h):] = float('nan')
    order = [int(x) for x in rng.permutation(n_act + n_idle)[:n_act]]
    active = [handles[i] for i in order]
    bucket = Bucket(tuple(qls), (C - 2 * 8,) * n_act, 'random verification shape')
    pool.register_bucket(bucket)
    speed = None if case % 3 == 0 else [float(x) for x in rng.uniform(0.8, 1.2, size=8)]
    pool.set_xcd_speed(speed)
    pool.set_slot_balance(case % 2 == 0)
    print(f'[verify fuzz] case {case}: contexts={[pool.length(h) for h in active]} queries={qls} '
          f'idle={n_idle} xcd_speed={speed is not None} slot_balance={case % 2 == 0}', flush=True)
    cu_q = [0]
    for q in qls:
        cu_q.append(cu_q[-1] + q)
    for rnd in range(2):
        ctx = [pool.length(h) for h in active]
        tx = pool.begin(active, bucket)
        q = randn_bf16(gen, L, cu_q[-1], 16, 128).to(dev)
        nk = randn_bf16(gen, L, cu_q[-1], 8, 128).to(dev)
        nv = randn_bf16(gen, L, cu_q[-1], 8, 128).to(dev)
        for layer in range(L):
            out = pool.attend(tx, layer, q[layer], keys=nk[layer], values=nv[layer])
            torch.cuda.synchronize()
            assert torch.equal(pool.scratch_keys[layer, :cu_q[-1]], nk[layer])
            assert torch.equal(pool.scratch_values[layer, :cu_q[-1]], nv[layer])
            ref = cref.verify_attention(bits(q[layer]), bits(pool.keys[layer]), bits(pool.values[layer]),
                                        bits(pool.scratch_keys[layer]), bits(pool.scratch_values[layer]),
                                        [h.index for h in active], ctx, cu_q, scale=SCALE)
            attention_gate(f64(out), ref, segments(cu_q))
        counts = {h: int(rng.integers(0, ql + 1)) for h, ql in zip(active, qls)}
        before = [pool.request_kv(h) for h in active]
        pool.commit(tx, counts)
        for i, h in enumerate(active):
            n = counts[h]
            got_k, got_v = pool.request_kv(h)
            assert torch.equal(got_k, torch.cat((before[i][0], nk[:, cu_q[i]:cu_q[i] + n]), dim=1))
            assert torch.equal(got_v, torch.cat((before[i][1], nv[:, cu_q[i]:cu_q[i] + n]), dim=1))
            assert torch.isnan(pool.keys[:, h.index, ctx[i] + n:]).all()
