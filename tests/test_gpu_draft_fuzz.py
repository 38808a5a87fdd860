"""Seeded random draft batches against the oracle (dspark_qwen/model.py:12-19
block mask over packed_draft.py:205-236's key lists): request counts, context
lengths (empty, one row, stage edges, several chunks), 1..11 blocks per
request with random anchors, draft chunk sizes, the three scheduling modes,
the three pool forms (row store, head-major slotted pool, append-order pool
read through gather indices) with NaN in every row no request owns, and fp32
Q/K.  Each case: the row-store run meets the oracle gate; every other pool
form, and fp32 Q/K holding the same bf16 values, give the same bits."""
import numpy as np
import pytest
import torch

from helpers import SEED, attention_gate, f64
from test_gpu_draft import draft_case, oracle, run

pytestmark = pytest.mark.gpu

CASES = 18
EDGES = (0, 1, 63, 64, 65, 127, 300, 1000, 2047, 2500, 4097)


@pytest.fixture(scope='module')
def dev():
    from qwen3_dspark_amd._device import require_gfx950
    return require_gfx950('cuda')


def random_anchors(rng, c, n):
    return [c] + [int(x) for x in rng.integers(0, c + 1, size=n - 1)]


@pytest.mark.parametrize('case', range(CASES))
def test_random_draft_batch(dev, case):
    from qwen3_dspark_amd.draft import HipDraftAttention
    rng = np.random.default_rng(SEED + 7000 + case)
    gen = torch.Generator().manual_seed(SEED + 7000 + case)
    n_req = int(rng.integers(1, 9))
    contexts = [int(rng.choice(EDGES)) if rng.random() < 0.5 else int(rng.integers(0, 3000)) for _ in range(n_req)]
    blocks = [int(rng.integers(1, 12)) for _ in range(n_req)]
    chunk = (None, 256, 1024)[case % 3]
    persistent = (1, None, 8)[(case // 3) % 3]
    print(f'[draft fuzz] case {case}: contexts={contexts} blocks={blocks} chunk={chunk} persistent={persistent}',
          flush=True)
    c = draft_case(gen, rng, contexts, blocks, spare=5)
    c['anchors'] = [random_anchors(rng, ctx, n) for ctx, n in zip(contexts, blocks)]
    # NaN in the spare rows between requests: no request may read them
    owned = torch.zeros(c['ctx_k'].shape[0], dtype=torch.bool)
    for o, l in zip(c['offs'], c['lens']):
        owned[o:o + l] = True
    c['ctx_k'][~owned] = float('nan')
    c['ctx_v'][~owned] = float('nan')
    ref, cu_b = oracle(c)
    kernel = HipDraftAttention(dev, chunk=chunk, persistent=persistent)
    rows_out = run(dev, kernel, c)
    attention_gate(f64(rows_out), ref, [(7 * cu_b[i], 7 * cu_b[i + 1]) for i in range(len(cu_b) - 1)])
    # head-major slotted pool, requests in shuffled slots at an offset, NaN elsewhere
    cap = max(contexts) + 9
    order = rng.permutation(n_req)
    slot_k = torch.full((n_req, 8, cap, 128), float('nan'), dtype=torch.bfloat16)
    slot_v = torch.full_like(slot_k, float('nan'))
    soffs = []
    for r, (o, l) in enumerate(zip(c['offs'], c['lens'])):
        s = int(order[r])
        slot_k[s, :, 3:3 + l] = c['ctx_k'][o:o + l].transpose(0, 1)
        slot_v[s, :, 3:3 + l] = c['ctx_v'][o:o + l].transpose(0, 1)
        soffs.append(s * cap + 3)
    assert torch.equal(run(dev, kernel, c, ctx_k=slot_k, ctx_v=slot_v, offs=soffs), rows_out)
    # append-order pool [1, 8, N, 128] through gather indices, NaN in unowned rows
    n = sum(contexts) + 11
    perm = rng.permutation(n)
    pool_k = torch.full((1, 8, n, 128), float('nan'), dtype=torch.bfloat16)
    pool_v = torch.full_like(pool_k, float('nan'))
    indices, ioffs, cursor = [], [], 0
    for o, l in zip(c['offs'], c['lens']):
        ioffs.append(len(indices))
        idx = perm[cursor:cursor + l]
        cursor += l
        indices += [int(x) for x in idx]
        pool_k[0, :, idx] = c['ctx_k'][o:o + l].transpose(0, 1)
        pool_v[0, :, idx] = c['ctx_v'][o:o + l].transpose(0, 1)
    idx_t = torch.tensor(indices or [0], dtype=torch.long, device=dev)
    assert torch.equal(run(dev, kernel, c, ctx_k=pool_k, ctx_v=pool_v, indices=idx_t, offs=ioffs), rows_out)
    # fp32 Q and K (context and block) holding the same bf16 values
    if case % 2 == 0:
        c32 = dict(c, q=c['q'].float(), bk=c['bk'].float())
        assert torch.equal(run(dev, kernel, c32, ctx_k=c['ctx_k'].float()), rows_out)
