"""Pin the CPU oracle: reference golden vectors, closed forms, brute force,
torch SDPA on explicit masks, and agreement of the C and numpy restatements."""
import math

import numpy as np
import pytest
import torch

from helpers import SCALE, bits, randn_bf16
from oracle import attention, cref, semantics


def test_layout_golden_vector(golden):
    g = golden['layout_basic']
    L = semantics.layout_from_metadata(g['query_requests'], g['query_positions'], g['key_requests'], g['key_positions'])
    assert list(L['query_lengths']) == g['query_lengths']
    assert list(L['key_lengths']) == g['key_lengths']
    assert L['cu_query'] == g['cu_query'] and L['cu_key'] == g['cu_key']
    assert L['gather_indices'] == g['gather_indices']
    assert L['pair_domain'] == g['pair_domain']
    # Zero Q gives uniform attention over the visible keys (values = physical index).
    phys = np.arange(9, dtype=np.float64)
    kv = phys[L['gather_indices']].reshape(-1, 1, 1)
    out = attention.varlen_attention(np.zeros((3, 1, 1)), kv, kv, L['cu_query'], L['cu_key'], causal=True, scale=1.0)
    np.testing.assert_allclose(out.ravel(), g['uniform_causal_output'], atol=1e-12)


def test_layout_invalid_cases_raise(golden):
    for case in golden['layout_invalid']['cases']:
        with pytest.raises(semantics.OracleValueError):
            semantics.layout_from_metadata(*case)


def test_noncausal_uniform_closed_form(golden):
    g = golden['noncausal_uniform']
    L = semantics.layout_from_metadata(g['query_requests'], g['query_positions'], g['key_requests'], g['key_positions'])
    v = np.broadcast_to(np.arange(5.0).reshape(5, 1, 1), (5, 2, 8)).copy()
    out = attention.varlen_attention(np.zeros((3, 4, 8)), np.zeros((5, 2, 8)), v, L['cu_query'], L['cu_key'],
                                     causal=False, scale=8 ** -0.5)
    assert np.array_equal(out, np.full((3, 4, 8), g['expected']))


def test_draft_backbone_layout_counters(golden):
    g = golden['draft_backbone_layout']
    L = semantics.layout_from_metadata(g['query_requests'], g['query_positions'], g['key_requests'], g['key_positions'])
    assert sum(L['query_lengths']) == g['query_rows']
    assert sum(L['key_lengths']) == g['gathered_key_rows']
    assert L['pair_domain'] == g['pair_domain']
    assert [k - q for q, k in zip(L['query_lengths'], L['key_lengths'])] == g['context_lengths']


def _prefix(layers, n, heads, dim, offset):
    x = np.arange(layers * n * heads * dim, dtype=np.float32).reshape(layers, n, heads, dim) + offset
    return x, x + 0.25


def test_txn_growing_context_golden(golden):
    g = golden['txn_growing_context']
    p = g['pool']
    L, S, C, Q, H, D = p['layers'], p['slots'], p['context_capacity'], p['max_query_tokens'], p['heads'], p['dim']
    keys = np.zeros((L, S, C, H, D), np.float32)
    values = np.zeros_like(keys)
    lengths = {}
    pre = {}
    for slot, (name, n, off) in enumerate(g['prefixes']):
        k, v = _prefix(L, n, H, D, off)
        keys[:, slot, :n], values[:, slot, :n] = k, v
        lengths[name] = n
        pre[name] = (k, v)
    slot_of = {name: i for i, (name, _, _) in enumerate(g['prefixes'])}
    qls, ceil = g['bucket']
    kcap = sum(qls) + sum(ceil)
    active = g['active']
    ctx = [lengths[a] for a in active]
    meta = semantics.txn_metadata([slot_of[a] for a in active], ctx, qls, C, kcap)
    assert meta['cu_query'].tolist() == g['cu_query']
    assert meta['cu_key'].tolist() == g['cu_key']
    assert meta['positions'].tolist() == g['positions']
    w = semantics.work_counters(ctx, qls, kcap, sum(lengths.values()))
    assert w['inactive_resident_key_tokens'] == g['inactive_resident_key_tokens']
    assert w['physical_key_capacity'] == g['physical_key_capacity']
    assert w['padded_key_capacity'] == g['padded_key_capacity']
    sk = np.arange(L * 5 * H * D, dtype=np.float32).reshape(L, 5, H, D) + 10000
    scratch = np.zeros((L, Q, H, D), np.float32)
    scratch[:, :5] = sk
    for layer in range(L):
        got = semantics.materialize(keys[layer], scratch[layer], meta)
        ak, bk = pre['A'][0][layer], pre['B'][0][layer]
        expect = np.concatenate((ak, sk[layer, :2], bk, sk[layer, 2:]))
        assert np.array_equal(got[:13], expect)
        assert not got[13:].any()
    counts = [g['commit'][a] for a in active]
    new_keys, new_len = semantics.commit(keys, scratch, [slot_of[a] for a in active], ctx, qls, counts, C)
    assert np.array_equal(new_keys[:, slot_of['A'], :4], np.concatenate((pre['A'][0], sk[:, :1]), axis=1))
    assert np.array_equal(new_keys[:, slot_of['B'], :7], np.concatenate((pre['B'][0], sk[:, 2:4]), axis=1))
    assert np.array_equal(new_keys[:, slot_of['idle']], keys[:, slot_of['idle']])
    meta2 = semantics.txn_metadata([slot_of[a] for a in active], new_len, qls, C, kcap)
    assert meta2['cu_key'].tolist() == g['second_cu_key']
    assert meta2['positions'].tolist() == g['second_positions']


def test_txn_small_cases_golden(golden):
    g = golden['txn_slot_reuse']
    meta = semantics.txn_metadata([0], [0], g['bucket'][0], 24, sum(g['bucket'][0]) + sum(g['bucket'][1]))
    assert meta['cu_key'].tolist() == g['cu_key'] and meta['positions'].tolist() == g['positions']
    g = golden['txn_retry_metadata']
    meta = semantics.txn_metadata([0], [g['prefix']], g['bucket'][0], 24, 10)
    assert meta['cu_query'].tolist() == g['cu_query'] and meta['cu_key'].tolist() == g['cu_key']
    assert meta['positions'].tolist() == g['positions']
    g = golden['txn_reordered_subset']
    lens = dict((n, c) for n, c in g['prefixes'])
    slot = {n: i for i, (n, _) in enumerate(g['prefixes'])}
    meta = semantics.txn_metadata([slot[a] for a in g['active']], [lens[a] for a in g['active']],
                                  g['pair'][0], 24, sum(g['pair'][0]) + sum(g['pair'][1]))
    assert meta['cu_query'].tolist() == g['cu_query'] and meta['cu_key'].tolist() == g['cu_key']
    assert meta['positions'].tolist() == g['positions']
    w = semantics.work_counters([lens['B']], [1], 8, sum(lens.values()))
    assert w['inactive_resident_key_tokens'] == g['inactive_with_B_small']
    g = golden['txn_invalid_commit']
    keys = np.random.default_rng(1).standard_normal((1, 1, 24, 1, 16)).astype(np.float32)
    for n in g['invalid_counts']:
        with pytest.raises(semantics.OracleValueError):
            semantics.commit(keys, keys[:, 0], [0], [g['prefix']], g['bucket'][0], [n], 24)
    same, _ = semantics.commit(keys, keys[:, 0, :8], [0], [g['prefix']], g['bucket'][0], [g['valid_noop']], 24)
    assert np.array_equal(same, keys)


def test_block_mask_truth_table_and_dflash_equality(golden):
    g = golden['block_mask_truth_table']
    m = semantics.block_mask(g['anchors'], g['block_size'], g['context_length'])
    assert np.nonzero(m[0])[0].tolist() == g['row0_visible']
    assert np.nonzero(m[4])[0].tolist() == g['row4_visible']
    g = golden['block_mask_equals_dflash']
    a = semantics.block_mask(g['anchors'], g['block_size'], g['context_length'])
    b = semantics.dflash_sdpa_mask(g['anchors'], [True] * len(g['anchors']), g['context_length'], g['block_size'])
    assert np.array_equal(a, b)


def _top_left_oracle(q, k, v, cu_q, cu_k, scale):
    """A deliberately wrong (upper-left aligned) variant, used only to show
    that the ramp sentinel distinguishes alignments."""
    out = np.zeros(q.shape)
    for r in range(len(cu_q) - 1):
        nq, nk = cu_q[r + 1] - cu_q[r], cu_k[r + 1] - cu_k[r]
        vis = np.arange(nk)[None, :] <= np.arange(nq)[:, None]
        out[cu_q[r]:cu_q[r + 1]] = attention._attend(q[cu_q[r]:cu_q[r + 1]], k[cu_k[r]:cu_k[r + 1]],
                                                     v[cu_k[r]:cu_k[r + 1]], vis, scale)
    return out


def test_ramp_sentinel_is_bottom_right_and_discriminates(golden):
    proto = golden['probe_varlen_protocol']
    for case in proto['cases']:
        ql, kl = case['q'], case['k']
        cq, ck = np.cumsum([0] + ql), np.cumsum([0] + kl)
        v = np.concatenate([np.arange(n) / 32.0 for n in kl]).reshape(-1, 1, 1) * np.ones((1, 8, 128))
        zq = np.zeros((cq[-1], 16, 128))
        out = attention.varlen_attention(zq, np.zeros_like(v), v, cq, ck, causal=True, scale=SCALE)
        expect = np.concatenate([[(k - q + i) / proto['ramp_divisor'] for i in range(q)] for q, k in zip(ql, kl)])
        np.testing.assert_allclose(out[:, 0, 0], expect, atol=1e-12)
        wrong = _top_left_oracle(zq, np.zeros_like(v), v, cq, ck, SCALE)
        assert np.abs(wrong[:, 0, 0] - expect).max() > 1e-3 or all(q == k for q, k in zip(ql, kl))
        full = attention.varlen_attention(zq, np.zeros_like(v), v, cq, ck, causal=False, scale=SCALE)
        np.testing.assert_allclose(full[:, 0, 0], np.concatenate([[(k - 1) / 64] * q for q, k in zip(ql, kl)]), atol=1e-12)


def test_brute_force_tiny_softmax():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((2, 16, 128))
    k = rng.standard_normal((3, 8, 128))
    v = rng.standard_normal((3, 8, 128))
    out = attention.varlen_attention(q, k, v, [0, 2], [0, 3], causal=True, scale=SCALE)
    for i in range(2):
        for h in range(16):
            lim = 3 - 2 + i + 1
            s = [sum(q[i, h, d] * k[j, h // 2, d] for d in range(128)) * SCALE for j in range(lim)]
            mx = max(s)
            e = [math.exp(x - mx) for x in s]
            o = [sum(e[j] * v[j, h // 2, d] for j in range(lim)) / sum(e) for d in range(128)]
            np.testing.assert_allclose(out[i, h], o, rtol=1e-10, atol=1e-12)


def _sdpa(q, k, v, mask, scale):
    """torch SDPA (CPU, float64) on explicit masks; q [nq,Hq,D] numpy."""
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).double().transpose(0, 1)[None]
    out = torch.nn.functional.scaled_dot_product_attention(t(q), t(k), t(v), attn_mask=torch.from_numpy(mask)[None, None],
                                                           scale=scale, enable_gqa=True)
    return out[0].transpose(0, 1).numpy()


def test_oracle_matches_torch_sdpa_on_explicit_masks():
    rng = np.random.default_rng(7)
    ql, kl = [1, 7, 3], [17, 40, 3]
    cq, ck = np.cumsum([0] + ql), np.cumsum([0] + kl)
    q = rng.standard_normal((cq[-1], 16, 128))
    k = rng.standard_normal((ck[-1], 8, 128))
    v = rng.standard_normal((ck[-1], 8, 128))
    for causal in (True, False):
        out = attention.varlen_attention(q, k, v, cq, ck, causal=causal, scale=SCALE)
        for r in range(3):
            nq, nk = ql[r], kl[r]
            mask = (np.arange(nk)[None] <= np.arange(nk - nq, nk)[:, None]) if causal else np.ones((nq, nk), bool)
            ref = _sdpa(q[cq[r]:cq[r + 1]], k[ck[r]:ck[r + 1]], v[ck[r]:ck[r + 1]], mask, SCALE)
            np.testing.assert_allclose(out[cq[r]:cq[r + 1]], ref, atol=1e-12, rtol=1e-10)
    # draft blocks against SDPA with the reference block mask
    anchors, c = [0, 5, 12], 12
    qd = rng.standard_normal((21, 16, 128))
    ck_, cv_ = rng.standard_normal((c, 8, 128)), rng.standard_normal((c, 8, 128))
    bk, bv = rng.standard_normal((21, 8, 128)), rng.standard_normal((21, 8, 128))
    out = attention.draft_attention(qd, ck_, cv_, bk, bv, anchors, scale=SCALE)
    mask = semantics.block_mask(anchors, 7, c)
    ref = _sdpa(qd, np.concatenate((ck_, bk)), np.concatenate((cv_, bv)), mask, SCALE)
    np.testing.assert_allclose(out, ref, atol=1e-12, rtol=1e-10)


def test_verify_oracle_equals_materialised_varlen():
    rng = np.random.default_rng(9)
    S, C, Q = 4, 40, 16
    res_k, res_v = rng.standard_normal((S, C, 8, 128)), rng.standard_normal((S, C, 8, 128))
    scr_k, scr_v = rng.standard_normal((Q, 8, 128)), rng.standard_normal((Q, 8, 128))
    slots, ctx, qs = [2, 0, 3], [33, 0, 12], [7, 2, 5]
    q = rng.standard_normal((sum(qs), 16, 128))
    out = attention.verify_attention(q, res_k, res_v, scr_k, scr_v, slots, ctx, qs, scale=SCALE)
    kcap = sum(ctx) + sum(qs) + 9
    meta = semantics.txn_metadata(slots, ctx, qs, C, kcap)
    k = semantics.materialize(res_k, scr_k, meta)
    v = semantics.materialize(res_v, scr_v, meta)
    k[meta['cu_key'][-1]:] = np.nan  # the capacity tail is never read
    v[meta['cu_key'][-1]:] = np.nan
    ref = attention.varlen_attention(q, k, v, meta['cu_query'], meta['cu_key'], causal=True, scale=SCALE)
    np.testing.assert_allclose(out, ref, atol=1e-13)
    assert np.isfinite(ref).all()


def test_c_oracle_matches_numpy_oracle():
    gen = torch.Generator().manual_seed(11)
    S, C, Q = 3, 70, 24
    rk, rv = randn_bf16(gen, S, C, 8, 128), randn_bf16(gen, S, C, 8, 128)
    sk, sv = randn_bf16(gen, Q, 8, 128), randn_bf16(gen, Q, 8, 128)
    slots, ctx, qs = [1, 2, 0], [64, 0, 9], [7, 7, 3]
    q = randn_bf16(gen, sum(qs), 16, 128)
    cu_q = np.cumsum([0] + qs)
    a = cref.verify_attention(bits(q), bits(rk), bits(rv), bits(sk), bits(sv), slots, ctx, cu_q, scale=SCALE)
    b = attention.verify_attention(q.double().numpy(), rk.double().numpy(), rv.double().numpy(),
                                   sk.double().numpy(), sv.double().numpy(), slots, ctx, qs, scale=SCALE)
    assert np.abs(a - b).max() < 1e-5
    # draft: 2 requests, ctx in a row store with offsets
    ctx_rows = randn_bf16(gen, 100, 8, 128), randn_bf16(gen, 100, 8, 128)
    offs, lens, anchors = [10, 50], [30, 41], [[30, 3], [0, 41, 17]]
    nb = sum(len(a_) for a_ in anchors)
    qd = randn_bf16(gen, 7 * nb, 16, 128)
    bk, bv = randn_bf16(gen, 7 * nb, 8, 128), randn_bf16(gen, 7 * nb, 8, 128)
    cu_b = np.cumsum([0] + [len(a_) for a_ in anchors])
    flat = [x for a_ in anchors for x in a_]
    a = cref.draft_attention(bits(qd), bits(ctx_rows[0]), bits(ctx_rows[1]), offs, lens, bits(bk), bits(bv),
                             cu_b, flat, scale=SCALE)
    for r in range(2):
        rows = slice(7 * cu_b[r], 7 * cu_b[r + 1])
        b = attention.draft_attention(qd[rows].double().numpy(),
                                      ctx_rows[0][offs[r]:offs[r] + lens[r]].double().numpy(),
                                      ctx_rows[1][offs[r]:offs[r] + lens[r]].double().numpy(),
                                      bk[rows].double().numpy(), bv[rows].double().numpy(), anchors[r], scale=SCALE)
        assert np.abs(a[rows] - b).max() < 1e-5


def test_qkv_prologue_oracle_matches_transformers_qwen3_modules():
    """The prologue oracle against transformers' own Qwen3 projection, q/k
    RMSNorm and rotary modules (float32, CPU): a library routine pins the
    formula, including the rotate-half pairing and the inverse frequencies."""
    from transformers import Qwen3Config
    from transformers.models.qwen3 import modeling_qwen3 as mq

    from oracle import qkv
    cfg = Qwen3Config(vocab_size=64, hidden_size=256, intermediate_size=256, num_hidden_layers=1,
                      num_attention_heads=16, num_key_value_heads=8, head_dim=128, rope_theta=1e6)
    torch.manual_seed(7)
    attn = mq.Qwen3Attention(cfg, layer_idx=0).eval()
    with torch.no_grad():
        attn.q_norm.weight.uniform_(0.5, 1.5)
        attn.k_norm.weight.uniform_(0.5, 1.5)
    rot = mq.Qwen3RotaryEmbedding(cfg)
    t = 13
    x = torch.randn(1, t, 256)
    pos = torch.tensor([[0, 1, 2, 7, 100, 511, 4095, 8191, 3, 3, 9000, 17, 6000]])
    with torch.no_grad():
        q = attn.q_norm(attn.q_proj(x).view(1, t, -1, 128)).transpose(1, 2)
        k = attn.k_norm(attn.k_proj(x).view(1, t, -1, 128)).transpose(1, 2)
        v = attn.v_proj(x).view(1, t, -1, 128)
        cos, sin = rot(x, pos)
        q, k = mq.apply_rotary_pos_emb(q, k, cos, sin)
    w = {n: p.detach().numpy() for n, p in attn.named_parameters()}
    oq, ok, ov = qkv.qkv_prologue(x[0].numpy(), w['q_proj.weight'], w['k_proj.weight'], w['v_proj.weight'],
                                  w['q_norm.weight'], w['k_norm.weight'], pos[0].numpy(), eps=cfg.rms_norm_eps)
    np.testing.assert_allclose(oq, q[0].transpose(0, 1).numpy(), rtol=1e-4, atol=2e-4)
    np.testing.assert_allclose(ok, k[0].transpose(0, 1).numpy(), rtol=1e-4, atol=2e-4)
    np.testing.assert_allclose(ov, v[0].numpy(), rtol=1e-5, atol=1e-5)
    # Planted mistakes must fail: unrotated pairing and a missing norm weight.
    bad = qkv.rope(qkv.rms_norm((x[0].numpy() @ w['q_proj.weight'].T).reshape(t, 16, 128),
                                np.ones(128), cfg.rms_norm_eps), pos[0].numpy(), qkv.inv_freq())
    assert not np.allclose(bad, q[0].transpose(0, 1).numpy(), atol=1e-3)
    assert np.allclose(qkv.inv_freq(), rot.inv_freq.numpy(), rtol=0, atol=0)


def test_draft_projection_oracle_matches_transformers_qwen3_modules():
    """The draft context projection oracle against torch's nn.Linear and
    transformers' Qwen3RMSNorm / Qwen3RotaryEmbedding / apply_rotary_pos_emb
    (the modules dspark_qwen/model.py builds DSparkDraft from; its rotate is
    the rotate-half form), float32 on the CPU, 2 draft layers."""
    from torch import nn
    from transformers import Qwen3Config
    from transformers.models.qwen3 import modeling_qwen3 as mq

    from oracle import draft_proj, qkv
    hidden, feats, t = 256, 5 * 256, 11
    cfg = Qwen3Config(vocab_size=64, hidden_size=hidden, intermediate_size=256, num_hidden_layers=1,
                      num_attention_heads=16, num_key_value_heads=8, head_dim=128, rope_theta=1e6)
    torch.manual_seed(3)
    fc = nn.Linear(feats, hidden, bias=False)
    cnorm = mq.Qwen3RMSNorm(hidden, eps=cfg.rms_norm_eps)
    layers = [(nn.Linear(hidden, 1024, bias=False), mq.Qwen3RMSNorm(128, eps=cfg.rms_norm_eps),
               nn.Linear(hidden, 1024, bias=False)) for _ in range(2)]
    with torch.no_grad():
        cnorm.weight.uniform_(0.5, 1.5)
        for _, kn, _ in layers:
            kn.weight.uniform_(0.5, 1.5)
    rot = mq.Qwen3RotaryEmbedding(cfg)
    x = torch.randn(1, t, feats)
    pos = torch.tensor([[5, 6, 7, 0, 1, 2, 3, 4000, 4001, 8190, 8191]])
    with torch.no_grad():
        ctx = cnorm(fc(x))
        cos, sin = rot(ctx, pos)
        expect = []
        for kp, kn, vp in layers:
            k = kn(kp(ctx).view(1, t, 8, 128)).transpose(1, 2)
            k, _ = mq.apply_rotary_pos_emb(k, k, cos, sin)
            expect.append((k[0].transpose(0, 1).numpy(), vp(ctx).view(t, 8, 128).numpy()))
    got = draft_proj.project_context_kv(x[0].numpy(), fc.weight.detach().numpy(), cnorm.weight.detach().numpy(),
                                        [(kp.weight.detach().numpy(), kn.weight.detach().numpy(),
                                          vp.weight.detach().numpy()) for kp, kn, vp in layers],
                                        pos[0].numpy(), eps=cfg.rms_norm_eps)
    for (ok, ov), (ek, ev) in zip(got, expect):
        np.testing.assert_allclose(ok, ek, rtol=1e-4, atol=2e-4)
        np.testing.assert_allclose(ov, ev, rtol=1e-4, atol=2e-4)
    # Planted mistakes must fail: the context norm left out, and the norm
    # taken per 128-dim head instead of over the hidden size.
    f = x[0].numpy().astype(np.float64) @ fc.weight.detach().numpy().T
    for wrong_ctx in (f, qkv.rms_norm(f.reshape(t, 2, 128), np.ones(128), 1e-6).reshape(t, hidden)):
        v_bad = (wrong_ctx @ layers[0][2].weight.detach().numpy().T).reshape(t, 8, 128)
        assert not np.allclose(v_bad, expect[0][1], atol=1e-3)


def test_draft_backbone_oracle_matches_transformers_modules_and_closed_forms():
    """The draft backbone oracle (oracle/draft_model.py) against an
    independent float32 evaluation: transformers' Qwen3RMSNorm, Qwen3MLP,
    Qwen3RotaryEmbedding + apply_rotary_pos_emb and torch's SDPA on the
    block mask of oracle.semantics.block_mask (itself pinned to the
    reference's truth table above), 2 layers with 3 blocks over a 40-row
    context.  Closed forms: with o_proj and the MLP's down projection zero a
    layer is the identity (residuals), so the output is the final RMSNorm of
    the block embeddings; a planted mistake (the MLP residual dropped) fails."""
    from torch import nn
    from transformers import Qwen3Config
    from transformers.models.qwen3 import modeling_qwen3 as mq

    from oracle import draft_model, semantics
    hidden, c, anchors = 256, 40, [40, 0, 17]
    cfg = Qwen3Config(vocab_size=64, hidden_size=hidden, intermediate_size=384, num_hidden_layers=1,
                      num_attention_heads=16, num_key_value_heads=8, head_dim=128, rope_theta=1e6)
    torch.manual_seed(11)
    eps = cfg.rms_norm_eps

    def norm(n):
        m = mq.Qwen3RMSNorm(n, eps=eps)
        with torch.no_grad():
            m.weight.uniform_(0.5, 1.5)
        return m
    layers = []
    for _ in range(2):
        layers.append(dict(input_norm=norm(hidden), q=nn.Linear(hidden, 2048, bias=False),
                           k=nn.Linear(hidden, 1024, bias=False), v=nn.Linear(hidden, 1024, bias=False),
                           o=nn.Linear(2048, hidden, bias=False), q_norm=norm(128), k_norm=norm(128),
                           post_norm=norm(hidden), mlp=mq.Qwen3MLP(cfg)))
    final = norm(hidden)
    rot = mq.Qwen3RotaryEmbedding(cfg)
    z0 = torch.randn(1, 21, hidden)
    ctx_kv = [(torch.randn(1, 8, c, 128), torch.randn(1, 8, c, 128)) for _ in layers]
    pos = (torch.tensor(anchors)[:, None] + torch.arange(7)).reshape(1, -1)
    visible = torch.from_numpy(np.asarray(semantics.block_mask(anchors, 7, c))).reshape(21, c + 21)

    def reference(mods, zero=False):
        z = z0
        cos, sin = rot(z, pos)
        with torch.no_grad():
            for m, (ck, cv) in zip(mods, ctx_kv):
                x = m['input_norm'](z)
                q = m['q_norm'](m['q'](x).view(1, 21, 16, 128)).transpose(1, 2)
                k = m['k_norm'](m['k'](x).view(1, 21, 8, 128)).transpose(1, 2)
                v = m['v'](x).view(1, 21, 8, 128).transpose(1, 2)
                q, k = mq.apply_rotary_pos_emb(q, k, cos, sin)
                kk = torch.cat((ck, k), 2).repeat_interleave(2, 1)
                vv = torch.cat((cv, v), 2).repeat_interleave(2, 1)
                o = torch.nn.functional.scaled_dot_product_attention(q, kk, vv, attn_mask=visible)
                z = z + m['o'](o.transpose(1, 2).reshape(1, 21, -1))
                z = z + m['mlp'](m['post_norm'](z))
            return final(z)[0].numpy()

    def weights(m):
        w = lambda mod: mod.weight.detach().numpy()
        return dict(input_norm=w(m['input_norm']), q_proj=w(m['q']), k_proj=w(m['k']), v_proj=w(m['v']),
                    o_proj=w(m['o']), q_norm=w(m['q_norm']), k_norm=w(m['k_norm']), post_norm=w(m['post_norm']),
                    gate=w(m['mlp'].gate_proj), up=w(m['mlp'].up_proj), down=w(m['mlp'].down_proj))
    kv = [(k[0].transpose(0, 1).numpy(), v[0].transpose(0, 1).numpy()) for k, v in ctx_kv]
    out = draft_model.draft_backbone(z0[0].numpy(), [weights(m) for m in layers], kv, anchors,
                                     final.weight.detach().numpy(), eps=eps)
    np.testing.assert_allclose(out, reference(layers), rtol=2e-4, atol=2e-4)
    # closed form: zero o_proj and down projection -> the identity per layer
    with torch.no_grad():
        for m in layers:
            m['o'].weight.zero_()
            m['mlp'].down_proj.weight.zero_()
    out = draft_model.draft_backbone(z0[0].numpy(), [weights(m) for m in layers], kv, anchors,
                                     final.weight.detach().numpy(), eps=eps)
    z = z0[0].double().numpy()
    closed = final.weight.detach().double().numpy() * z / np.sqrt((z * z).mean(-1, keepdims=True) + eps)
    np.testing.assert_allclose(out, closed, rtol=1e-12, atol=1e-12)
    # a planted mistake in a copy of the layer (MLP residual dropped) fails the library check
    torch.manual_seed(12)
    fresh = [dict(m, mlp=mq.Qwen3MLP(cfg), o=nn.Linear(2048, hidden, bias=False)) for m in layers]
    w = [weights(m) for m in fresh]
    good = draft_model.draft_backbone(z0[0].numpy(), w, kv, anchors, final.weight.detach().numpy(), eps=eps)
    ref = reference(fresh)
    np.testing.assert_allclose(good, ref, rtol=2e-4, atol=2e-4)
    real_mlp = draft_model.mlp
    try:
        draft_model.mlp = lambda y, gate, up, down: np.zeros((y.shape[0], np.asarray(down).shape[0]))
        bad = draft_model.draft_backbone(z0[0].numpy(), w, kv, anchors, final.weight.detach().numpy(), eps=eps)
    finally:
        draft_model.mlp = real_mlp
    assert not np.allclose(bad, ref, atol=1e-2)
