"""The reference's mixed-precision draft pool under bf16 autocast: K in FP32
(its k_norm runs in FP32), V in BF16, with Q, K and V cast to bf16 at the
kernel boundary (dspark_qwen/packed_draft.py:222-235; the dtype trail is
pinned by tests/test_packed_draft.py:175-199).  The fused kernel reads the
FP32 K rows in place and rounds them to bf16 in registers, so an FP32-K pool
must give the same output bits as a bf16 pool holding the rounded values,
and meet the oracle gate on those values."""
import numpy as np
import pytest
import torch

from helpers import SCALE, SEED, attention_gate, f64, randn_bf16
from test_gpu_draft import draft_case, oracle, run

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope='module')
def dev():
    from qwen3_dspark_amd._device import require_gfx950
    return require_gfx950('cuda')


def amp_pair(gen, rng, contexts, blocks):
    """The same case twice: FP32 Q, context K and block K (values that bf16
    cannot hold), and their bf16-rounded copies (torch's round to nearest
    even, the reference's .to(dtype))."""
    c = draft_case(gen, rng, contexts, blocks)
    k32 = torch.randn(c['ctx_k'].shape, generator=gen)
    q32 = torch.randn(c['q'].shape, generator=gen)
    bk32 = torch.randn(c['bk'].shape, generator=gen)
    assert not torch.equal(k32, k32.to(torch.bfloat16).float())
    c32 = dict(c, ctx_k=k32, q=q32, bk=bk32)
    c16 = dict(c, ctx_k=k32.to(torch.bfloat16), q=q32.to(torch.bfloat16), bk=bk32.to(torch.bfloat16))
    return c32, c16


@pytest.mark.parametrize('name,contexts,blocks', [
    ('two_requests', [128, 96], [1, 1]),
    ('one_to_eight_blocks', [2000, 57, 0, 1, 513, 64], [8, 1, 1, 2, 3, 7]),
    ('long_split', [3100, 4100], [5, 8]),
])
def test_fp32_k_equals_rounded_bf16_pool(dev, name, contexts, blocks):
    from qwen3_dspark_amd.draft import HipDraftAttention
    say(f'[draft amp] {name} contexts={contexts} blocks={blocks}')
    rng = np.random.default_rng(SEED + 31 + len(name))
    gen = torch.Generator().manual_seed(SEED + 31 + sum(contexts))
    c32, c16 = amp_pair(gen, rng, contexts, blocks)
    ref, cu_b = oracle(c16)
    for kernel in (HipDraftAttention(dev), HipDraftAttention(dev, chunk=1024)):
        out16 = run(dev, kernel, c16)
        out32 = run(dev, kernel, c32)
        assert out32.dtype == torch.bfloat16
        assert torch.equal(out32.view(torch.int16), out16.view(torch.int16))
        attention_gate(f64(out32), ref, [(7 * cu_b[i], 7 * cu_b[i + 1]) for i in range(len(cu_b) - 1)])
        # Only K in FP32 (Q already bf16): the same bits again.
        out_k = run(dev, kernel, dict(c32, q=c16['q']))
        assert torch.equal(out_k.view(torch.int16), out16.view(torch.int16))


def test_fp32_k_pool_forms(dev):
    """The reference's append-order pool layer [1, 8, N, 128] (interleaved
    requests, gather indices) and a head-major slotted pool (NaN outside the
    used rows) with FP32 K give the bits of the bf16 row store."""
    from qwen3_dspark_amd.draft import HipDraftAttention
    say('[draft amp] pool forms')
    rng = np.random.default_rng(SEED + 41)
    gen = torch.Generator().manual_seed(SEED + 41)
    contexts, blocks = [300, 41, 900], [3, 2, 6]
    c32, c16 = amp_pair(gen, rng, contexts, blocks)
    kernel = HipDraftAttention(dev)
    rows_out = run(dev, kernel, c16)
    n = sum(contexts)
    owner = np.concatenate([np.full(l, r) for r, l in enumerate(contexts)])
    rng.shuffle(owner)
    pool_k = torch.zeros(1, 8, n, 128)
    pool_v = torch.zeros(1, 8, n, 128, dtype=torch.bfloat16)
    indices, offs = [], []
    for r, (o, l) in enumerate(zip(c32['offs'], c32['lens'])):
        offs.append(len(indices))
        idx = list(np.nonzero(owner == r)[0])
        indices += idx
        pool_k[0, :, idx] = c32['ctx_k'][o:o + l].transpose(0, 1)
        pool_v[0, :, idx] = c32['ctx_v'][o:o + l].transpose(0, 1)
    idx_t = torch.tensor(indices, dtype=torch.long, device=dev)
    out = run(dev, kernel, c32, ctx_k=pool_k, ctx_v=pool_v, indices=idx_t, offs=offs)
    assert torch.equal(out.view(torch.int16), rows_out.view(torch.int16))
    cap = 1000
    slot_k = torch.full((3, 8, cap, 128), float('nan'))
    slot_v = torch.full((3, 8, cap, 128), float('nan'), dtype=torch.bfloat16)
    soffs = []
    for r, (o, l) in enumerate(zip(c32['offs'], c32['lens'])):
        slot = 2 - r
        slot_k[slot, :, 5:5 + l] = c32['ctx_k'][o:o + l].transpose(0, 1)
        slot_v[slot, :, 5:5 + l] = c32['ctx_v'][o:o + l].transpose(0, 1)
        soffs.append(slot * cap + 5)
    out = run(dev, kernel, c32, ctx_k=slot_k, ctx_v=slot_v, offs=soffs)
    assert torch.equal(out.view(torch.int16), rows_out.view(torch.int16))


def test_mixed_precision_draft_pool(dev):
    """DraftKVPool(key_dtype=float32, value_dtype=bfloat16): appends keep the
    FP32 K and BF16 V rows exactly; attention over it equals attention over a
    bf16 pool fed the rounded K; precision changes are refused."""
    from qwen3_dspark_amd.draft import DraftKVPool
    say('[draft amp] mixed-precision pool')
    gen = torch.Generator().manual_seed(SEED + 51)
    layers = 2
    amp = DraftKVPool(layers=layers, slots=3, capacity=256, key_dtype=torch.float32, value_dtype=torch.bfloat16,
                      device=dev)
    plain = DraftKVPool(layers=layers, slots=3, capacity=256, device=dev)
    assert amp.keys.dtype == torch.float32 and amp.values.dtype == torch.bfloat16 and amp.dtype is None
    for p in (amp, plain):
        for r in ('A', 'B'):
            p.add_request(r)
    chunks = {'A': 37, 'B': 150}
    rows = sum(chunks.values())
    k32 = [torch.randn(rows, 8, 128, generator=gen).to(dev) for _ in range(layers)]
    v16 = [randn_bf16(gen, rows, 8, 128).to(dev) for _ in range(layers)]
    work = amp.append_projected(chunks, list(zip(k32, v16)))
    assert work['append_launches'] == 2
    plain.append_projected(chunks, [(k.to(torch.bfloat16), v) for k, v in zip(k32, v16)])
    kv = amp.request_kv('B')
    for layer in range(layers):
        assert torch.equal(kv[layer][0][0].transpose(0, 1), k32[layer][37:])
        assert torch.equal(kv[layer][1][0].transpose(0, 1), v16[layer][37:])
    anchors = {'B': [150, 3, 77], 'A': [37]}
    nq = 7 * 4
    q32 = torch.randn(nq, 16, 128, generator=gen).to(dev)
    bk32 = torch.randn(nq, 8, 128, generator=gen).to(dev)
    bv = randn_bf16(gen, nq, 8, 128).to(dev)
    for layer in range(layers):
        a = amp.attention(layer, q32, bk32, bv, amp.batch(anchors))
        b = plain.attention(layer, q32.to(torch.bfloat16), bk32.to(torch.bfloat16), bv, plain.batch(anchors))
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    with pytest.raises(ValueError, match='precision'):
        amp.append_projected({'A': 1}, [(k[:1].to(torch.bfloat16), v[:1]) for k, v in zip(k32, v16)])
    with pytest.raises(ValueError, match='precision'):
        amp.attention(0, q32, bk32.to(torch.bfloat16), bv, amp.batch(anchors))
    assert amp.lengths == {'A': 37, 'B': 150}
