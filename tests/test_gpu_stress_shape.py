"""The 64-request stress workload at its full size, one verification layer and
one draft layer, against the C oracle (oracle/attn_ref.c):

* 64 requests with contexts floor(exp(U(ln 256, ln 8192))) (seeded), the
  resident store at its fixed capacity of 8,192 rows per request, 7 new rows
  per request staged into scratch by the attention launch itself
  (persistent_target_kv.py:427-438, persistent_qwen_target.py:30-42);
* 1..8 draft blocks of 7 rows per request, one of them at the full context,
  the others at seeded anchors, over a slotted context pool of the same
  capacity (packed_draft.py:35-47, model.py:41-61).

Every resident or pool row past a request's length holds NaN, so a read
beyond the lengths would fail the gate.  Beyond the attention tolerance,
an exact size-independent property: doubling V (resident, staged and pool
rows alike) doubles every output bit for bit (power-of-two scaling is exact
through the softmax weights, the FP32 partials, their merge and the bf16
rounding), with the same segment plan.
"""
import math
import os

import numpy as np
import pytest
import torch

from helpers import SEED, attention_gate, f64, segments

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda:0')
B, Q, CAP = 64, 7, 8192


def say(*a):
    print(*a, flush=True)


def bits(t):
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def workload():
    rng = np.random.default_rng(SEED)
    ctx = np.floor(np.exp(rng.uniform(math.log(256), math.log(8192), size=B))).astype(int)
    ctx = [int(c) for c in np.minimum(ctx, CAP - 2 * Q)]
    anchors = []
    for c in ctx:
        n = int(rng.integers(1, 9))
        anchors.append([c] + [int(x) for x in rng.integers(0, c + 1, size=n - 1)])
    return ctx, anchors


def threads():
    return max(1, min(16, os.cpu_count() or 1))


@torch.no_grad()
def test_verify_layer_at_the_stress_shape():
    from oracle import cref
    from qwen3_dspark_amd.kernels import SCALE
    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV
    ctx, _ = workload()
    say(f'[stress verify] {B} requests, contexts sum={sum(ctx)} max={max(ctx)}, capacity {CAP}')
    gen = torch.Generator(device=DEV).manual_seed(SEED)
    pool = PersistentTargetKV(layers=1, slots=B, context_capacity=CAP, max_query_tokens=B * Q, heads=8, dim=128,
                              device=DEV)
    handles = [pool.add_request(f'r{i}') for i in range(B)]
    pool.keys.normal_(generator=gen)
    pool.values.normal_(generator=gen)
    for h, c in zip(handles, ctx):
        pool.load_prefix(h, pool.keys[:, h.index, :c], pool.values[:, h.index, :c])
        pool.keys[:, h.index, c:] = float('nan')
        pool.values[:, h.index, c:] = float('nan')
    bucket = Bucket((Q,) * B, (CAP - Q,) * B, 'stress shape')
    pool.register_bucket(bucket)
    q = torch.randn(B * Q, 16, 128, generator=gen, device=DEV).to(torch.bfloat16)
    kn = torch.randn(B * Q, 8, 128, generator=gen, device=DEV).to(torch.bfloat16)
    vn = torch.randn(B * Q, 8, 128, generator=gen, device=DEV).to(torch.bfloat16)

    tx = pool.begin(handles, bucket)
    out = pool.attend(tx, 0, q, keys=kn, values=vn)
    torch.cuda.synchronize()
    assert torch.equal(pool.scratch_keys[0][:B * Q], kn) and torch.equal(pool.scratch_values[0][:B * Q], vn)
    pool.abort(tx)
    say('[stress verify] kernel done; running the C oracle')
    cmax = max(ctx)
    cu_q = [Q * i for i in range(B + 1)]
    ref = cref.verify_attention(bits(q), bits(pool.keys[0, :, :cmax]), bits(pool.values[0, :, :cmax]), bits(kn),
                                bits(vn), [h.index for h in handles], ctx, cu_q, scale=SCALE, threads=threads())
    stats = attention_gate(f64(out), ref, segments(cu_q))
    say(f'[stress verify] max |d| {stats[0]["max_abs"]:.2e}, mean |d| {stats[0]["mean_abs"]:.2e}')

    pool.values.mul_(2)
    tx = pool.begin(handles, bucket)
    out2 = pool.attend(tx, 0, q, keys=kn, values=2 * vn)
    pool.abort(tx)
    assert torch.equal(out2, 2 * out)


@torch.no_grad()
def test_draft_layer_at_the_stress_shape():
    from oracle import cref
    from qwen3_dspark_amd.draft import DraftBatch, HipDraftAttention
    from qwen3_dspark_amd.kernels import SCALE
    ctx, anchors = workload()
    n_blocks = sum(len(a) for a in anchors)
    say(f'[stress draft] {B} requests, {n_blocks} blocks, contexts sum={sum(ctx)}')
    gen = torch.Generator(device=DEV).manual_seed(SEED + 1)
    ck = torch.randn(B, 8, CAP, 128, generator=gen, device=DEV).to(torch.bfloat16)
    cv = torch.randn(B, 8, CAP, 128, generator=gen, device=DEV).to(torch.bfloat16)
    for r, c in enumerate(ctx):
        ck[r, :, c:] = float('nan')
        cv[r, :, c:] = float('nan')
    nq = 7 * n_blocks
    q = torch.randn(nq, 16, 128, generator=gen, device=DEV).to(torch.bfloat16)
    bk = torch.randn(nq, 8, 128, generator=gen, device=DEV).to(torch.bfloat16)
    bv = torch.randn(nq, 8, 128, generator=gen, device=DEV).to(torch.bfloat16)
    offsets = [r * CAP for r in range(B)]      # slot * capacity + first position
    batch = DraftBatch(DEV, offsets, ctx, anchors)
    draft = HipDraftAttention(DEV)
    out = draft(q, bk, bv, ck, cv, batch, scale=SCALE)
    torch.cuda.synchronize()
    say('[stress draft] kernel done; running the C oracle')
    # token-major host copies of each request's context rows
    hk = bits(torch.cat([ck[r, :, :c].transpose(0, 1) for r, c in enumerate(ctx)]))
    hv = bits(torch.cat([cv[r, :, :c].transpose(0, 1) for r, c in enumerate(ctx)]))
    offs = np.concatenate([[0], np.cumsum(ctx)[:-1]]).tolist()
    cu_b = np.cumsum([0] + [len(a) for a in anchors])
    flat = [x for a in anchors for x in a]
    ref = cref.draft_attention(bits(q), hk, hv, offs, ctx, bits(bk), bits(bv), cu_b, flat, scale=SCALE,
                               threads=threads())
    stats = attention_gate(f64(out), ref, [(7 * cu_b[i], 7 * cu_b[i + 1]) for i in range(B)])
    say(f'[stress draft] max |d| {stats[0]["max_abs"]:.2e}, mean |d| {stats[0]["mean_abs"]:.2e}')

    out2 = draft(q, bk, 2 * bv, ck, 2 * cv, batch, scale=SCALE)
    assert torch.equal(out2, 2 * out)
