"""GPU parity of the fused multi-block draft attention against the oracle
(dspark_qwen/model.py:12-19 block mask), its equivalence with the packed
noncausal path for one block per request (dspark_qwen/packed_draft.py:205-236),
the indexed append-order pool form and isolation under poisoning."""
import numpy as np
import pytest
import torch

from helpers import SCALE, SEED, attention_gate, bits, f64, randn_bf16
from oracle import attention, cref

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope='module')
def dev():
    from qwen3_dspark_amd._device import require_gfx950
    return require_gfx950('cuda')


def draft_case(gen, rng, contexts, blocks, spare=32):
    """Row-store context: request r occupies rows off_r .. off_r + c_r with
    `spare` unused rows between requests; anchors include 0 and c_r."""
    offs, cursor = [], spare
    for c in contexts:
        offs.append(cursor)
        cursor += c + spare
    rows = cursor
    anchors = []
    for c, n in zip(contexts, blocks):
        a = [c] + [int(x) for x in rng.integers(0, c + 1, size=n - 1)]
        if n > 2:
            a[1] = 0
        anchors.append(a)
    nb = sum(blocks)
    return dict(offs=offs, lens=list(contexts), anchors=anchors,
                ctx_k=randn_bf16(gen, rows, 8, 128), ctx_v=randn_bf16(gen, rows, 8, 128),
                q=randn_bf16(gen, 7 * nb, 16, 128), bk=randn_bf16(gen, 7 * nb, 8, 128),
                bv=randn_bf16(gen, 7 * nb, 8, 128))


def run(dev, kernel, c, ctx_k=None, ctx_v=None, indices=None, offs=None):
    from qwen3_dspark_amd.draft import DraftBatch
    batch = DraftBatch(dev, offs or c['offs'], c['lens'], c['anchors'], context_indices=indices)
    out = kernel(c['q'].to(dev), c['bk'].to(dev), c['bv'].to(dev),
                 (c['ctx_k'] if ctx_k is None else ctx_k).to(dev),
                 (c['ctx_v'] if ctx_v is None else ctx_v).to(dev), batch, scale=SCALE)
    torch.cuda.synchronize()
    return out


def oracle(c):
    cu_b = np.cumsum([0] + [len(a) for a in c['anchors']])
    flat = [x for a in c['anchors'] for x in a]
    return cref.draft_attention(bits(c['q']), bits(c['ctx_k']), bits(c['ctx_v']), c['offs'], c['lens'],
                                bits(c['bk']), bits(c['bv']), cu_b, flat, scale=SCALE), cu_b


@pytest.mark.parametrize('name,contexts,blocks', [
    ('config1_fp32_shapes', [128, 96], [1, 1]),
    ('config3_like', [700, 130, 1024, 333], [4, 4, 4, 4]),
    ('one_to_eight_blocks', [2000, 57, 0, 1, 513, 64], [8, 1, 1, 2, 3, 7]),
    ('long_split', [3100, 4100], [5, 8]),
])
def test_multi_block_against_oracle(dev, name, contexts, blocks):
    from qwen3_dspark_amd.draft import HipDraftAttention
    say(f'[draft] {name} contexts={contexts} blocks={blocks}')
    rng = np.random.default_rng(SEED + len(name))
    gen = torch.Generator().manual_seed(SEED + sum(contexts))
    c = draft_case(gen, rng, contexts, blocks)
    ref, cu_b = oracle(c)
    # default chunking, and 1024-key chunks (more split-K partials and merges)
    for kernel in (HipDraftAttention(dev), HipDraftAttention(dev, chunk=1024)):
        out = run(dev, kernel, c)
        attention_gate(f64(out), ref, [(7 * cu_b[i], 7 * cu_b[i + 1]) for i in range(len(cu_b) - 1)])
        # Linearity in V (context and block values together) is exact.
        c2 = dict(c, ctx_v=2 * c['ctx_v'], bv=2 * c['bv'])
        assert torch.equal(run(dev, kernel, c2), 2 * out)


def test_more_than_eight_blocks_per_request(dev):
    """A request with more blocks than one pass of the kernel holds (8) is
    planned as consecutive views over the same context (DSparkDraft.backbone
    takes any number of anchors, model.py:101-119): 11 + 3 blocks meet the
    oracle, and equal bit for bit the same blocks given as separate requests
    of at most 8 blocks over the same context rows."""
    from qwen3_dspark_amd.draft import DraftBatch, HipDraftAttention
    say('[draft] 11 + 3 blocks')
    rng = np.random.default_rng(SEED + 811)
    gen = torch.Generator().manual_seed(SEED + 811)
    c = draft_case(gen, rng, [3000, 200], [11, 3])
    ref, cu_b = oracle(c)
    batch = DraftBatch(dev, c['offs'], c['lens'], c['anchors'])
    assert batch.requests == 2 and batch.views == ((0, 0), (0, 8), (1, 0)) and batch.max_blocks == 8
    split = dict(c, offs=[c['offs'][0], c['offs'][0], c['offs'][1]], lens=[3000, 3000, 200],
                 anchors=[c['anchors'][0][:8], c['anchors'][0][8:], c['anchors'][1]])
    for kernel in (HipDraftAttention(dev), HipDraftAttention(dev, chunk=1024)):
        out = run(dev, kernel, c)
        attention_gate(f64(out), ref, [(7 * cu_b[i], 7 * cu_b[i + 1]) for i in range(len(cu_b) - 1)])
        assert torch.equal(run(dev, kernel, split), out)


def test_single_block_equals_packed_noncausal_path(dev):
    """One block per request at anchor = c: the fused kernel and the packed
    noncausal varlen kernel over ctx ++ block both meet the oracle."""
    from qwen3_dspark_amd.draft import HipDraftAttention
    from qwen3_dspark_amd.kernels import HipDraftVarlenKernel
    from qwen3_dspark_amd.layout import PackedLayout
    say('[draft] single block vs packed noncausal')
    rng = np.random.default_rng(SEED)
    gen = torch.Generator().manual_seed(SEED)
    contexts = [128, 96, 1500]
    c = draft_case(gen, rng, contexts, [1, 1, 1])
    fused = run(dev, HipDraftAttention(dev), c)
    ks, vs, qr, qp, kr, kp = [], [], [], [], [], []
    for r, (o, n) in enumerate(zip(c['offs'], c['lens'])):
        ks += [c['ctx_k'][o:o + n], c['bk'][7 * r:7 * r + 7]]
        vs += [c['ctx_v'][o:o + n], c['bv'][7 * r:7 * r + 7]]
        qr += [r] * 7
        qp += list(range(n, n + 7))
        kr += [r] * (n + 7)
        kp += list(range(n + 7))
    layout = PackedLayout.from_metadata(*(torch.tensor(x, device=dev) for x in (qr, qp, kr, kp)))
    packed = HipDraftVarlenKernel(dev)(c['q'].to(dev), torch.cat(ks).to(dev), torch.cat(vs).to(dev), layout, scale=SCALE)
    ref = attention.varlen_attention(f64(c['q']), f64(torch.cat(ks)), f64(torch.cat(vs)), layout.cu_query.tolist(),
                                     layout.cu_key.tolist(), causal=False, scale=SCALE)
    seg = [(7 * r, 7 * r + 7) for r in range(3)]
    attention_gate(f64(fused), ref, seg)
    attention_gate(f64(packed), ref, seg)


def test_pool_forms_are_bit_identical(dev):
    """The reference pool layout [1,8,N,128] with interleaved requests and
    per-request physical indices, and a head-major slotted pool with NaN
    outside the used rows, give the same bits as the row store."""
    from qwen3_dspark_amd.draft import HipDraftAttention
    say('[draft] pool forms')
    rng = np.random.default_rng(SEED + 5)
    gen = torch.Generator().manual_seed(SEED + 5)
    contexts, blocks = [300, 41, 900], [3, 2, 6]
    c = draft_case(gen, rng, contexts, blocks, spare=0)
    kernel = HipDraftAttention(dev)
    rows_out = run(dev, kernel, c)
    n = sum(contexts)
    owner = np.concatenate([np.full(l, r) for r, l in enumerate(contexts)])
    rng.shuffle(owner)  # interleaved append order
    phys_of = {r: list(np.nonzero(owner == r)[0]) for r in range(3)}
    pool_k = torch.zeros(1, 8, n, 128, dtype=torch.bfloat16)
    pool_v = torch.zeros_like(pool_k)
    indices, offs = [], []
    for r, (o, l) in enumerate(zip(c['offs'], c['lens'])):
        offs.append(len(indices))
        idx = phys_of[r]
        indices += idx
        pool_k[0, :, idx] = c['ctx_k'][o:o + l].transpose(0, 1)
        pool_v[0, :, idx] = c['ctx_v'][o:o + l].transpose(0, 1)
    idx_t = torch.tensor(indices, dtype=torch.long, device=dev)
    out = run(dev, kernel, c, ctx_k=pool_k, ctx_v=pool_v, indices=idx_t, offs=offs)
    assert torch.equal(out, rows_out)
    # Head-major slotted pool [slots, 8, capacity, 128]: request r in slot
    # 2-r at position 5 (offset = slot * capacity + position).
    cap = 1000
    slot_k = torch.full((3, 8, cap, 128), float('nan'), dtype=torch.bfloat16)
    slot_v = torch.full_like(slot_k, float('nan'))
    soffs = []
    for r, (o, l) in enumerate(zip(c['offs'], c['lens'])):
        slot = 2 - r
        slot_k[slot, :, 5:5 + l] = c['ctx_k'][o:o + l].transpose(0, 1)
        slot_v[slot, :, 5:5 + l] = c['ctx_v'][o:o + l].transpose(0, 1)
        soffs.append(slot * cap + 5)
    out = run(dev, kernel, c, ctx_k=slot_k, ctx_v=slot_v, offs=soffs)
    assert torch.equal(out, rows_out)


def test_indexed_pool_long_contexts_every_mode(dev):
    """The append-order pool [1,8,N,128] read through gather indices over
    many ring stages (contexts up to 4100 rows, split-K chunks, an empty and
    a one-row context), with NaN in every pool row no index addresses, for
    a bf16 and an fp32 K pool and every scheduling mode: bit for bit the
    row store's output under the same kernel settings, which meets the
    oracle."""
    from qwen3_dspark_amd.draft import HipDraftAttention
    say('[draft] indexed pool, long contexts, every mode')
    rng = np.random.default_rng(SEED + 41)
    gen = torch.Generator().manual_seed(SEED + 41)
    contexts, blocks = [3100, 700, 4100, 1, 0], [5, 8, 3, 1, 2]
    c = draft_case(gen, rng, contexts, blocks, spare=0)
    ref, cu_b = oracle(c)
    n = sum(contexts) + 777
    perm = rng.permutation(n)
    indices, offs, cursor = [], [], 0
    pool_k = torch.full((1, 8, n, 128), float('nan'), dtype=torch.bfloat16)
    pool_v = torch.full_like(pool_k, float('nan'))
    for o, l in zip(c['offs'], c['lens']):
        offs.append(len(indices))
        idx = perm[cursor:cursor + l]
        cursor += l
        indices += [int(x) for x in idx]
        pool_k[0, :, idx] = c['ctx_k'][o:o + l].transpose(0, 1)
        pool_v[0, :, idx] = c['ctx_v'][o:o + l].transpose(0, 1)
    idx_t = torch.tensor(indices, dtype=torch.long, device=dev)
    kernels = (HipDraftAttention(dev), HipDraftAttention(dev, chunk=1024), HipDraftAttention(dev, persistent=None),
               HipDraftAttention(dev, persistent=8))
    for kernel in kernels:
        rows_out = run(dev, kernel, c)
        attention_gate(f64(rows_out), ref, [(7 * cu_b[i], 7 * cu_b[i + 1]) for i in range(len(cu_b) - 1)])
        for key_pool in (pool_k, pool_k.float()):
            # an fp32 K pool takes fp32 block K (its values here are bf16-exact)
            cc = dict(c, bk=c['bk'].to(key_pool.dtype))
            out = run(dev, kernel, cc, ctx_k=key_pool, ctx_v=pool_v, indices=idx_t, offs=offs)
            assert torch.equal(out, rows_out), (key_pool.dtype, kernel.persistent, kernel.chunk)
    # The kernel reads 32-bit indices: a larger one is refused before launch.
    bad = idx_t.clone()
    bad[0] = 2 ** 31
    with pytest.raises(ValueError, match='below 2'):
        run(dev, kernels[0], c, ctx_k=pool_k, ctx_v=pool_v, indices=bad, offs=offs)


def test_poison_isolation_and_contract(dev):
    from qwen3_dspark_amd.draft import DraftBatch, HipDraftAttention
    say('[draft] poison isolation')
    rng = np.random.default_rng(SEED + 9)
    gen = torch.Generator().manual_seed(SEED + 9)
    c = draft_case(gen, rng, [400, 250], [3, 4])
    kernel = HipDraftAttention(dev)
    out = run(dev, kernel, c)
    # NaN everywhere outside request 0's context rows, and in request 1's
    # Q/blocks: request 0 is bit-identical.
    pk, pv = c['ctx_k'].clone(), c['ctx_v'].clone()
    o0, l0 = c['offs'][0], c['lens'][0]
    mask = torch.ones(pk.shape[0], dtype=torch.bool)
    mask[o0:o0 + l0] = False
    pk[mask] = float('nan')
    pv[mask] = float('nan')
    pq, pbk, pbv = c['q'].clone(), c['bk'].clone(), c['bv'].clone()
    pq[21:] = 100
    pbk[21:] = float('nan')
    pbv[21:] = float('nan')
    changed = run(dev, kernel, dict(c, q=pq, bk=pbk, bv=pbv), ctx_k=pk, ctx_v=pv)
    assert torch.equal(changed[:21], out[:21])
    # Block 1 of request 0 has anchor 0: no context row is visible to it.
    assert c['anchors'][0][1] == 0
    pk, pv = c['ctx_k'].clone(), c['ctx_v'].clone()
    pk[o0:o0 + l0] = 100
    pv[o0:o0 + l0] = -100
    assert torch.equal(run(dev, kernel, c, ctx_k=pk, ctx_v=pv)[7:14], out[7:14])
    with pytest.raises(ValueError):
        DraftBatch(dev, [0], [5], [[6]])
    with pytest.raises(ValueError):
        DraftBatch(dev, [0], [5], [[]])            # a request needs a block (more than 8 are fine)
    batch = DraftBatch(dev, c['offs'], c['lens'], c['anchors'])
    with pytest.raises(ValueError):
        kernel(c['q'].to(dev)[:7], c['bk'].to(dev), c['bv'].to(dev), c['ctx_k'].to(dev), c['ctx_v'].to(dev), batch, scale=SCALE)
    with pytest.raises(ValueError):
        kernel(c['q'].to(dev), c['bk'].to(dev), c['bv'].to(dev), c['ctx_k'][:10].to(dev), c['ctx_v'][:10].to(dev),
               batch, scale=SCALE)


def test_config1_fp32_with_rope_at_absolute_positions(dev):
    """The single-layer fp32 workload as specified: 2 requests with contexts
    128 and 96, one 7-row block each at anchor = context length, 16/8 heads,
    d128.  Seeded CPU FP32 N(0,1) draws in the order K, V, Q
    (scripts/probe_varlen.py:105-110), RoPE theta 1e6 applied to K at
    positions 0 .. c+6 and to Q at the block's positions c .. c+6
    (model.py:22-24 rotate; float32 angles as the model forms them).  Q and
    K go to the kernel in fp32 (rounded to bf16 as it loads them, the
    reference's cast at the kernel boundary), V in bf16 as the kernel takes
    it; the oracle sees the fp32 values."""
    from oracle import qkv
    from qwen3_dspark_amd.draft import DraftBatch, HipDraftAttention
    contexts = [128, 96]
    gen = torch.Generator().manual_seed(SEED)
    freqs = qkv.inv_freq()
    ks, vs, qs = [], [], []
    for c in contexts:
        k = torch.randn(c + 7, 8, 128, generator=gen)
        v = torch.randn(c + 7, 8, 128, generator=gen)
        q = torch.randn(7, 16, 128, generator=gen)
        ks.append(torch.from_numpy(qkv.rope(k.numpy(), np.arange(c + 7), freqs)).float())
        vs.append(v)
        qs.append(torch.from_numpy(qkv.rope(q.numpy(), np.arange(c, c + 7), freqs)).float())
    ctx_k = torch.cat([k[:c] for k, c in zip(ks, contexts)])
    ctx_v = torch.cat([v[:c] for v, c in zip(vs, contexts)]).to(torch.bfloat16)
    bk = torch.cat([k[c:] for k, c in zip(ks, contexts)])
    bv = torch.cat([v[c:] for v, c in zip(vs, contexts)]).to(torch.bfloat16)
    q = torch.cat(qs)
    batch = DraftBatch(dev, [0, contexts[0]], contexts, [[c] for c in contexts])
    out = HipDraftAttention(dev)(q.to(dev), bk.to(dev), bv.to(dev), ctx_k.to(dev), ctx_v.to(dev), batch,
                                 scale=SCALE)
    torch.cuda.synchronize()
    ref = np.concatenate([attention.draft_attention(qs[r].double().numpy(), ks[r][:c].double().numpy(),
                                                    vs[r][:c].double().numpy(), ks[r][c:].double().numpy(),
                                                    vs[r][c:].double().numpy(), [c], scale=SCALE)
                          for r, c in enumerate(contexts)])
    stats = attention_gate(f64(out), ref, [(0, 7), (7, 14)])
    say(f'[draft config1 rope] max |d| {stats[0]["max_abs"]:.2e} mean {stats[0]["mean_abs"]:.2e}')
