"""Verify-layer prologue (dspark_qkv_prologue) against the oracle
restatement of Qwen3's q/k/v projection, q/k RMSNorm and RoPE
(oracle/qkv.py, itself pinned to transformers' modules), and its use as
stage_layer's replacement in a PersistentTargetKV transaction."""
import numpy as np
import pytest
import torch

from helpers import SCALE, SEED, attention_gate, bits, f64, randn_bf16, segments
from oracle import cref, qkv

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda:0')
HIDDEN = 1024


def say(*a):
    print(*a, flush=True)


def weights(gen, hidden=HIDDEN):
    s = hidden ** -0.5
    w = [(randn_bf16(gen, n, hidden).float() * s).to(torch.bfloat16) for n in (2048, 1024, 1024)]
    norms = [(0.5 + torch.rand(128, generator=gen)).to(torch.bfloat16) for _ in range(2)]
    return w + norms


def gate(out, ref):
    """bf16 outputs of O(1) magnitude against float64: |d| <= .02 + .02|ref|,
    mean-abs <= 2e-3."""
    o = f64(out)
    d = np.abs(o - ref)
    assert np.isfinite(o).all()
    assert (d <= 0.02 + 0.02 * np.abs(ref)).all(), float(d.max())
    assert d.mean() <= 2e-3, float(d.mean())
    return float(d.max())


@pytest.mark.parametrize('tokens', [448, 5, 100, 1])
def test_prologue_against_oracle(tokens):
    from qwen3_dspark_amd.prologue import QKVPrologue
    gen = torch.Generator().manual_seed(SEED + tokens)
    wq, wk, wv, qn, kn = weights(gen)
    x = randn_bf16(gen, tokens, HIDDEN)
    pos = torch.randint(0, 9000, (tokens,), generator=gen)
    pro = QKVPrologue(*(t.to(DEV) for t in (wq, wk, wv, qn, kn)), eps=1e-6, theta=1e6)
    q, k, v = pro(x.to(DEV), pos.to(DEV))
    torch.cuda.synchronize()
    rq, rk, rv = qkv.qkv_prologue(f64(x), f64(wq), f64(wk), f64(wv), f64(qn), f64(kn), pos.numpy())
    errs = [gate(a, b) for a, b in ((q, rq), (k, rk), (v, rv))]
    say(f'[prologue] T={tokens} max-abs q/k/v {errs}')


@pytest.mark.parametrize('tokens', [448, 5])
def test_rope_table_gives_the_same_bits(tokens):
    """rope_table: cos/sin of the float32 angle positions * inv_freq to
    float32 accuracy, and the prologue fed with it writes the same bits as
    the prologue forming the angles itself."""
    from qwen3_dspark_amd.prologue import QKVPrologue
    gen = torch.Generator().manual_seed(SEED + 31 + tokens)
    pro = QKVPrologue(*(t.to(DEV) for t in weights(gen)), eps=1e-6, theta=1e6)
    x = randn_bf16(gen, tokens, HIDDEN).to(DEV)
    pos = torch.randint(0, 40000, (tokens,), generator=gen)
    table = pro.rope_table(pos.to(DEV))
    plain = pro(x, pos.to(DEV))
    fed = pro(x, pos.to(DEV), rope=table)
    torch.cuda.synchronize()
    angle = (pos.numpy().astype(np.float32)[:, None] * pro.inv_freq.cpu().numpy()[None, :]).astype(np.float64)
    ref = np.concatenate([np.cos(angle), np.sin(angle)], axis=1)
    assert np.abs(table.cpu().numpy().astype(np.float64) - ref).max() <= 2e-6
    for a, b in zip(plain, fed):
        assert torch.equal(a, b)
    with pytest.raises(ValueError, match='Rotary table'):
        pro(x, pos.to(DEV), rope=table[:, :64].contiguous())
    say(f'[prologue] T={tokens} rope table bit-identical')


def test_prologue_writes_scratch_and_feeds_attention():
    """stage_projected writes exactly the prologue's K/V into scratch (bit
    for bit), at the transaction's absolute positions, and the fused
    attention over it meets the oracle."""
    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV
    from qwen3_dspark_amd.prologue import QKVPrologue
    gen = torch.Generator().manual_seed(SEED + 9)
    contexts = [37, 300, 1024, 5]
    B = len(contexts)
    pool = PersistentTargetKV(layers=2, slots=B, context_capacity=1100, max_query_tokens=7 * B, heads=8, dim=128,
                              device=DEV)
    hs = [pool.add_request(f'r{i}') for i in range(B)]
    for h, c in zip(hs, contexts):
        kv = randn_bf16(gen, 2, 2, c, 8, 128).to(DEV)
        pool.load_prefix(h, kv[0], kv[1])
    bucket = Bucket((7,) * B, (1093,) * B, 'prologue')
    pool.register_bucket(bucket)
    pro = QKVPrologue(*(t.to(DEV) for t in weights(gen)))
    tx = pool.begin(hs, bucket)
    x = randn_bf16(gen, 7 * B, HIDDEN).to(DEV)
    q = pool.stage_projected(tx, 0, x, pro)
    positions = torch.tensor([c + i for c in contexts for i in range(7)], device=DEV)
    q2, k2, v2 = pro(x, positions)
    torch.cuda.synchronize()
    assert torch.equal(q, q2)
    assert torch.equal(pool.scratch_keys[0, :7 * B], k2) and torch.equal(pool.scratch_values[0, :7 * B], v2)
    with pytest.raises(ValueError, match='exactly once'):
        pool.stage_projected(tx, 0, x, pro)
    out = pool.attend(tx, 0, q)
    cu_q = list(range(0, 7 * B + 1, 7))
    ref = cref.verify_attention(bits(q), bits(pool.keys[0]), bits(pool.values[0]), bits(pool.scratch_keys[0]),
                                bits(pool.scratch_values[0]), [h.index for h in hs], contexts, cu_q, scale=SCALE)
    attention_gate(f64(out), ref, segments(cu_q))
    pool.abort(tx)


def test_prologue_contract():
    from qwen3_dspark_amd.prologue import QKVPrologue
    gen = torch.Generator().manual_seed(1)
    w = [t.to(DEV) for t in weights(gen)]
    with pytest.raises(ValueError, match='bf16'):
        QKVPrologue(w[0].float(), *w[1:])
    with pytest.raises(ValueError, match='bf16'):
        QKVPrologue(w[0][:, :512], *w[1:])
    pro = QKVPrologue(*w)
    x = torch.zeros(3, HIDDEN, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match='Positions'):
        pro(x, torch.zeros(3, dtype=torch.int32, device=DEV))
    with pytest.raises(ValueError, match='Hidden'):
        pro(x[:, :512], torch.zeros(3, dtype=torch.long, device=DEV))
