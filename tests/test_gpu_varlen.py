"""GPU parity of the packed varlen kernels (causal, noncausal, capacity tail)
against the CPU oracle, plus the reference probe sentinels and isolation
checks (scripts/probe_varlen.py:179-235,
scripts/probe_native_capacity_graph.py:23-35,156-189)."""
import numpy as np
import pytest
import torch

from helpers import SCALE, SEED, attention_gate, bits, f64, randn_bf16, segments
from oracle import attention, cref

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope='module')
def dev():
    from qwen3_dspark_amd._device import require_gfx950
    return require_gfx950('cuda')


@pytest.fixture(scope='module')
def kernels(dev):
    from qwen3_dspark_amd.kernels import HipCapacityKernel, HipDraftVarlenKernel, HipVarlenKernel
    return HipVarlenKernel(dev), HipDraftVarlenKernel(dev), HipCapacityKernel(dev)


def probe_inputs(dev):
    """The physical interleaved cache and the three probe cases of
    scripts/probe_varlen.py (seed 20261009; K, V drawn before Q)."""
    from qwen3_dspark_amd.layout import PackedLayout
    gen = torch.Generator().manual_seed(SEED)
    pairs = [(m, p) for p in range(29) for m, n in [(1, 17), (2, 29), (3, 13)] if p < n]
    kr = torch.tensor([m for m, _ in pairs])
    kp = torch.tensor([p for _, p in pairs])
    key = randn_bf16(gen, 1, 8, len(pairs), 128)
    value = randn_bf16(gen, 1, 8, len(pairs), 128)
    cases = [dict(name='interleaved_cached_tail', markers=[1, 2], q=[1, 8], k=[17, 29], inactive=13),
             dict(name='crop_exit_readd', markers=[1, 2, 4], q=[3, 2, 1], k=[11, 5, 1], inactive=0),
             dict(name='crop_zero_then_append', markers=[1], q=[2], k=[2], inactive=6)]
    out = []
    for index, case in enumerate(cases):
        if index:
            if index == 1:
                keep = ((kr == 1) & (kp < 8)) | ((kr == 2) & (kp < 3))
                added = [(1, p) for p in range(8, 11)] + [(2, p) for p in range(3, 5)] + [(4, 0)]
            else:
                keep = kr != 1
                added = [(1, 0), (1, 1)]
            key, value = key[:, :, keep], value[:, :, keep]
            kr, kp = kr[keep], kp[keep]
            key = torch.cat([key, randn_bf16(gen, 1, 8, len(added), 128)], dim=2)
            value = torch.cat([value, randn_bf16(gen, 1, 8, len(added), 128)], dim=2)
            kr = torch.cat([kr, torch.tensor([m for m, _ in added])])
            kp = torch.cat([kp, torch.tensor([p for _, p in added])])
        qr = torch.tensor([m for m, nq in zip(case['markers'], case['q']) for _ in range(nq)])
        qp = torch.tensor([p for nq, nk in zip(case['q'], case['k']) for p in range(nk - nq, nk)])
        layout = PackedLayout.from_metadata(qr.to(dev), qp.to(dev), kr.to(dev), kp.to(dev))
        assert list(layout.query_lengths) == case['q'] and list(layout.key_lengths) == case['k']
        assert layout.physical_key_tokens - layout.gathered_key_tokens == case['inactive']
        q = randn_bf16(gen, sum(case['q']), 16, 128)
        out.append(dict(case=case, layout=layout, q=q, key=key.clone(), value=value.clone(),
                        kr=kr.clone(), kp=kp.clone(), qr=qr, qp=qp))
    return out


@pytest.mark.parametrize('causal', [True, False])
def test_probe_cases_parity_ramp_and_isolation(dev, kernels, causal):
    kernel = kernels[0] if causal else kernels[1]
    for item in probe_inputs(dev):
        case, layout = item['case'], item['layout']
        say(f"[varlen causal={causal}] case {case['name']} q={case['q']} k={case['k']}")
        key, value = item['key'].to(dev), item['value'].to(dev)
        k, v = layout.gather_kv(key, value)
        q = item['q'].to(dev)
        out = kernel(q, k, v, layout, scale=SCALE)
        torch.cuda.synchronize()
        cu_q, cu_k = layout.cu_query.tolist(), layout.cu_key.tolist()
        ref = attention.varlen_attention(f64(q), f64(k), f64(v), cu_q, cu_k, causal=causal, scale=SCALE)
        attention_gate(f64(out), ref, segments(cu_q))
        # Zero-Q position ramp: bottom-right (k-q+i)/64, noncausal (k-1)/64, exact in bf16.
        ramp = (item['kp'].float() / 32)[None, None, :, None].expand_as(item['value']).to(torch.bfloat16)
        _, rv = layout.gather_kv(key, ramp.to(dev))
        sentinel = kernel(torch.zeros_like(q), k, rv.contiguous(), layout, scale=SCALE)
        if causal:
            expect = torch.cat([torch.arange(kk - qq, kk, dtype=torch.float64) / 64 for qq, kk in zip(case['q'], case['k'])])
        else:
            expect = torch.cat([torch.full((qq,), (kk - 1) / 64, dtype=torch.float64) for qq, kk in zip(case['q'], case['k'])])
        want = expect[:, None, None].expand(-1, 16, 128).to(torch.bfloat16)
        assert torch.equal(sentinel.cpu(), want), 'position-ramp sentinel differs'
        # Poison other requests (K/V 100/-100, Q 100): first request bit-identical.
        first = item['case']['markers'][0]
        pk, pv, pq = item['key'].clone(), item['value'].clone(), item['q'].clone()
        pk[:, :, item['kr'] != first] = 100
        pv[:, :, item['kr'] != first] = -100
        pq[item['qr'] != first] = 100
        pk2, pv2 = layout.gather_kv(pk.to(dev), pv.to(dev))
        changed = kernel(pq.to(dev), pk2, pv2, layout, scale=SCALE)
        n0 = case['q'][0]
        assert torch.equal(changed[:n0], out[:n0])
        if case['inactive']:
            inactive = ~torch.isin(item['kr'], torch.tensor(case['markers']))
            pk, pv = item['key'].clone(), item['value'].clone()
            pk[:, :, inactive] = 100
            pv[:, :, inactive] = -100
            pk2, pv2 = layout.gather_kv(pk.to(dev), pv.to(dev))
            assert torch.equal(kernel(q, pk2, pv2, layout, scale=SCALE), out)


def make_packed(gen, q_lens, k_lens):
    from qwen3_dspark_amd.layout import PackedLayout
    qr = torch.cat([torch.full((n,), i) for i, n in enumerate(q_lens)])
    qp = torch.cat([torch.arange(k - n, k) for n, k in zip(q_lens, k_lens)])
    kr = torch.cat([torch.full((k,), i) for i, k in enumerate(k_lens)])
    kp = torch.cat([torch.arange(k) for k in k_lens])
    q = randn_bf16(gen, sum(q_lens), 16, 128)
    k = randn_bf16(gen, sum(k_lens), 8, 128)
    v = randn_bf16(gen, sum(k_lens), 8, 128)
    return (qr, qp, kr, kp), q, k, v


@pytest.mark.parametrize('name,q_lens,k_lens', [
    ('verify_b4_ragged', [7, 7, 7, 7], [71, 519, 300, 64]),
    ('split_k_long', [7, 7, 3], [3000, 1537, 513]),
    ('multi_tile_q20', [20, 9, 1], [700, 9, 1]),
    ('single_key', [1, 1], [1, 2]),
    ('chunk_boundary', [7, 7], [512, 1031]),
    # the last 32-key tile of a wave is visible to some query rows only
    ('partial_tile_visibility', [7] * 8, [33, 38, 68, 97, 129, 1057, 1058, 2081]),
])
@pytest.mark.parametrize('causal', [True, False])
def test_packed_shapes_against_oracle(dev, kernels, name, q_lens, k_lens, causal):
    from qwen3_dspark_amd.layout import PackedLayout
    say(f'[varlen causal={causal}] {name} q={q_lens} k={k_lens}')
    gen = torch.Generator().manual_seed(SEED + sum(k_lens))
    meta, q, k, v = make_packed(gen, q_lens, k_lens)
    layout = PackedLayout.from_metadata(*(m.to(dev) for m in meta))
    kernel = kernels[0] if causal else kernels[1]
    out = kernel(q.to(dev), k.to(dev), v.to(dev), layout, scale=SCALE)
    torch.cuda.synchronize()
    cu_q, cu_k = layout.cu_query.tolist(), layout.cu_key.tolist()
    ref = cref.varlen_attention(bits(q), bits(k), bits(v), cu_q, cu_k, causal=causal, scale=SCALE)
    attention_gate(f64(out), ref, segments(cu_q))
    # Linearity: doubling V doubles the output exactly (power-of-two scaling).
    out2 = kernel(q.to(dev), k.to(dev), (2 * v).to(dev), layout, scale=SCALE)
    assert torch.equal(out2, 2 * out)


def test_request_order_invariance(dev, kernels):
    """A request-local split plan makes every request's output independent of
    the batch (bit-exact under permutation); the balanced plan moves its cuts
    with the batch, so its outputs agree to the attention tolerance."""
    from qwen3_dspark_amd.kernels import HipVarlenKernel
    from qwen3_dspark_amd.layout import PackedLayout
    say('[varlen] request permutation invariance')
    gen = torch.Generator().manual_seed(SEED + 1)
    q_lens, k_lens = [7, 3, 7, 5], [900, 40, 2100, 7]
    meta, q, k, v = make_packed(gen, q_lens, k_lens)
    layout = PackedLayout.from_metadata(*(m.to(dev) for m in meta))
    perm = [2, 0, 3, 1]
    cq, ck = layout.cu_query.tolist(), layout.cu_key.tolist()
    q2 = torch.cat([q[cq[i]:cq[i + 1]] for i in perm])
    k2 = torch.cat([k[ck[i]:ck[i + 1]] for i in perm])
    v2 = torch.cat([v[ck[i]:ck[i + 1]] for i in perm])
    meta2, _, _, _ = make_packed(torch.Generator().manual_seed(0), [q_lens[i] for i in perm], [k_lens[i] for i in perm])
    layout2 = PackedLayout.from_metadata(*(m.to(dev) for m in meta2))
    cq2 = layout2.cu_query.tolist()
    ref = cref.varlen_attention(bits(q), bits(k), bits(v), cq, ck, causal=True, scale=SCALE)
    for kernel in (HipVarlenKernel(dev, split='request', chunk=512), kernels[0]):
        out = kernel(q.to(dev), k.to(dev), v.to(dev), layout, scale=SCALE)
        out2 = kernel(q2.to(dev), k2.to(dev), v2.to(dev), layout2, scale=SCALE)
        attention_gate(f64(out), ref, segments(cq))
        for j, i in enumerate(perm):
            a, b = out2[cq2[j]:cq2[j + 1]], out[cq[i]:cq[i + 1]]
            if kernel.split == 'request':
                assert torch.equal(a, b)
            else:
                assert float((a.float() - b.float()).abs().max()) <= 2e-2


def test_capacity_tail_zero_finite_nan_bit_identical(dev, kernels):
    """scripts/probe_native_capacity_graph.py protocol: Q=(1,4), ceilings 144,
    three growing contexts; zero/finite/NaN tails give identical outputs."""
    from qwen3_dspark_amd.layout import PersistentAttentionLayout
    cap_kernel = kernels[2]
    gen = torch.Generator().manual_seed(SEED)
    q_lens, kcap = (1, 4), 293
    for contexts in ([128, 128], [129, 131], [130, 135]):
        say(f'[capacity] contexts={contexts}')
        k_lens = [c + q for c, q in zip(contexts, q_lens)]
        cu_q = torch.tensor([0, 1, 5], dtype=torch.int32)
        cu_k = torch.tensor([0, k_lens[0], sum(k_lens)], dtype=torch.int32)
        layout = PersistentAttentionLayout(q_lens, tuple(k_lens), cu_q.to(dev), cu_k.to(dev), kcap, 148, 4)
        q = randn_bf16(gen, 5, 16, 128).to(dev)
        k = randn_bf16(gen, kcap, 8, 128)
        v = randn_bf16(gen, kcap, 8, 128)
        outs = []
        for tail in ('zero', 'finite', 'nan'):
            kk, vv = k.clone(), v.clone()
            fill = {'zero': (0.0, 0.0), 'finite': (100.0, -100.0), 'nan': (float('nan'), float('nan'))}[tail]
            kk[sum(k_lens):] = fill[0]
            vv[sum(k_lens):] = fill[1]
            outs.append(cap_kernel(q, kk.to(dev), vv.to(dev), layout, scale=SCALE))
        assert torch.isfinite(outs[2]).all()
        assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
        ref = attention.varlen_attention(f64(q), f64(k), f64(v), cu_q.tolist(), cu_k.tolist(), causal=True, scale=SCALE)
        attention_gate(f64(outs[0]), ref, segments(cu_q.tolist()))


def test_contract_errors_before_device_work(dev, kernels):
    say('[varlen] contract errors')
    gen = torch.Generator().manual_seed(3)
    from qwen3_dspark_amd.layout import PackedLayout
    meta, q, k, v = make_packed(gen, [1, 8], [17, 29])
    layout = PackedLayout.from_metadata(*(m.to(dev) for m in meta))
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    kernel = kernels[0]
    bad = [
        (q.float(), k, v, SCALE), (q[:, :8].contiguous(), k, v, SCALE), (q, k, v, 1.0),
        (torch.zeros(9, 16, 256, dtype=torch.bfloat16, device=dev)[:, :, ::2], k, v, SCALE),
        (q[:1], k, v, SCALE), (q, k[:-1], v[:-1], SCALE), (q.cpu(), k, v, SCALE),
    ]
    for qq, kk, vv, sc in bad:
        with pytest.raises(ValueError):
            kernel(qq, kk, vv, layout, scale=sc)
    layout.cu_query[1] = 2
    with pytest.raises(ValueError, match='Cumulative'):
        kernel(q, k, v, layout, scale=SCALE)
