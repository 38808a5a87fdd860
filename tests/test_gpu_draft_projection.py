"""Draft context projection on the GPU: DraftContextProjector and
DraftKVPool.append_committed (hipBLASLt fc + dspark_draft_kv_project, or for
long appends hipBLASLt k/v GEMM + dspark_draft_kv_epilogue) against
the float64 oracle (oracle/draft_proj.py, itself pinned to transformers'
Qwen3 modules), its transactional contract (packed_draft.py:130-168), and
the full 5-layer draft context path of the 16-request workload feeding draft
attention."""
import numpy as np
import pytest
import torch

from helpers import SCALE, SEED, attention_gate, bits, f64, randn_bf16
from oracle import cref, draft_proj

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda:0')
HIDDEN, FEATS, LAYERS = 1024, 5 * 1024, 5


def say(*a):
    print(*a, flush=True)


def make_weights(gen, layers=LAYERS):
    """Random-init bf16 draft weights scaled so that every stage is O(1)."""
    fc = (randn_bf16(gen, HIDDEN, FEATS).float() * FEATS ** -0.5).to(torch.bfloat16)
    cn = (0.5 + torch.rand(HIDDEN, generator=gen)).to(torch.bfloat16)
    per = []
    for _ in range(layers):
        kp = (randn_bf16(gen, 1024, HIDDEN).float() * HIDDEN ** -0.5).to(torch.bfloat16)
        kn = (0.5 + torch.rand(128, generator=gen)).to(torch.bfloat16)
        vp = (randn_bf16(gen, 1024, HIDDEN).float() * HIDDEN ** -0.5).to(torch.bfloat16)
        per.append((kp, kn, vp))
    return fc, cn, per


def projector(fc, cn, per):
    from qwen3_dspark_amd.draft_projection import DraftContextProjector
    return DraftContextProjector(fc.to(DEV), cn.to(DEV), [tuple(t.to(DEV) for t in l) for l in per])


def gate(out, ref, mean_abs=2e-3):
    """bf16 rows of O(1) magnitude against float64: |d| <= .02 + .02|ref|,
    mean-abs <= 2e-3.  From the float64 fc (whole chain) the bar on the mean
    is 4e-3: the fc output is rounded to bf16 once, as the draft's autocast
    linear does, which adds ~2^-9 relative error to every O(1) row."""
    o = np.asarray(out, np.float64)
    d = np.abs(o - ref)
    assert np.isfinite(o).all()
    assert (d <= 0.02 + 0.02 * np.abs(ref)).all(), float(d.max())
    assert d.mean() <= mean_abs, float(d.mean())
    return float(d.max())


def pool_rows(pool, layer, request, start, n):
    """[n, 8, 128] float64 K and V rows of a request from the head-major pool."""
    s = pool.slot(request)
    k = pool.keys[layer, s, :, start:start + n].transpose(0, 1)
    v = pool.values[layer, s, :, start:start + n].transpose(0, 1)
    return f64(k), f64(v)


@pytest.mark.parametrize('path', ['auto', 'gemm', 'gemm_chunked'])
@pytest.mark.parametrize('counts', [[7] * 64, [1], [60, 3, 37], [2, 3]])
def test_append_committed_against_oracle(counts, path, monkeypatch):
    """Rows of one append (request token counts `counts`, after a first
    append that gives the requests different starting positions) against
    the oracle, with the fc output taken from the device (the kernel's input)
    and, for the whole chain, from the float64 fc.  `gemm` forces the
    library-GEMM + dspark_draft_kv_epilogue path at these sizes, and
    `gemm_chunked` also cuts it into GEMMs of 64 tokens (token0 offsets)."""
    from qwen3_dspark_amd import draft_projection
    from qwen3_dspark_amd.draft import DraftKVPool
    if path != 'auto':
        monkeypatch.setattr(draft_projection, 'GEMM_MIN_TOKENS', 1)
    if path == 'gemm_chunked':
        monkeypatch.setattr(draft_projection, 'GEMM_CHUNK', 64)
    gen = torch.Generator().manual_seed(SEED + len(counts) + sum(counts))
    fc, cn, per = make_weights(gen)
    proj = projector(fc, cn, per)
    names = [f'r{i}' for i in range(len(counts))]
    pool = DraftKVPool(layers=LAYERS, slots=len(counts) + 1, capacity=4096, device=DEV, projector=proj)
    for r in names:
        pool.add_request(r)
    first = {r: 1 + 37 * i % 300 for i, r in enumerate(names)}
    pool.append_committed({r: randn_bf16(gen, 1, n, FEATS).to(DEV) for r, n in first.items()})
    chunks = {r: randn_bf16(gen, 1, n, FEATS) for r, n in zip(names, counts)}
    work = pool.append_committed({r: x.to(DEV) for r, x in chunks.items()})
    torch.cuda.synchronize()
    assert work['new_context_tokens'] == sum(counts) and work['kv_projection_calls'] == LAYERS
    assert pool.lengths == {r: first[r] + n for r, n in zip(names, counts)}
    # Both paths keep the projection in FP32 to the end (the GEMM path's
    # library GEMM writes FP32) and round each output once.
    bar = 2e-3
    x = torch.cat([v[0] for v in chunks.values()])
    pos = np.concatenate([np.arange(first[r], first[r] + n) for r, n in zip(names, counts)])
    fc_dev = proj.fc_forward(x.to(DEV))
    weights = [(f64(kp), f64(kn), f64(vp)) for kp, kn, vp in per]
    ref_dev = draft_proj.project_context_kv(None, None, f64(cn), weights, pos, fc_out=f64(fc_dev))
    ref_full = draft_proj.project_context_kv(f64(x), f64(fc), f64(cn), weights, pos)
    errs = []
    for layer in range(LAYERS):
        got_k, got_v = [], []
        for r, n in zip(names, counts):
            k, v = pool_rows(pool, layer, r, first[r], n)
            got_k.append(k)
            got_v.append(v)
        got_k, got_v = np.concatenate(got_k), np.concatenate(got_v)
        errs.append((gate(got_k, ref_dev[layer][0], bar), gate(got_v, ref_dev[layer][1], bar)))
        gate(got_k, ref_full[layer][0], mean_abs=4e-3)
        gate(got_v, ref_full[layer][1], mean_abs=4e-3)
    say(f'[draft proj] {path} counts={counts[:4]}.. max-abs per layer (k, v) {errs}')


def test_fused_and_gemm_paths_round_alike():
    """The same append through the fused tiles and through the library GEMM
    + epilogue: both keep the projection in FP32 through the norms and RoPE
    and round each output once, so they differ only by FP32 accumulation
    order.  Almost every element is bitwise equal (measured: 99.98 %); the
    rest differ by one or two bf16 ulps of the larger value, or by a small
    absolute amount where RoPE's difference of products cancels.  (An extra
    bf16 rounding of the GEMM output on one path, as before, leaves a large
    fraction of the elements one ulp apart.)"""
    from qwen3_dspark_amd.draft import DraftKVPool
    gen = torch.Generator().manual_seed(SEED + 91)
    fc, cn, per = make_weights(gen)
    proj = projector(fc, cn, per)
    counts = [300, 7, 129, 64]
    chunks = {f'r{i}': randn_bf16(gen, 1, n, FEATS).to(DEV) for i, n in enumerate(counts)}
    rows = {}
    for path in ('fused', 'gemm'):
        pool = DraftKVPool(layers=LAYERS, slots=len(counts), capacity=512, device=DEV, projector=proj)
        for r in chunks:
            pool.add_request(r)
        x = torch.cat([v[0] for v in chunks.values()])
        records = torch.tensor([[pool.slot(r), 0, sum(counts[:i]), n] for i, (r, n) in enumerate(zip(chunks, counts))],
                               dtype=torch.int32, device=DEV)
        proj.project_into(proj.fc_forward(x), records, len(counts), pool.keys, pool.values, path=path)
        torch.cuda.synchronize()
        rows[path] = np.concatenate([np.concatenate([pool.keys[:, pool.slot(r), :, :n].float().cpu().numpy().ravel(),
                                                     pool.values[:, pool.slot(r), :, :n].float().cpu().numpy().ravel()])
                                     for r, n in zip(chunks, counts)]).astype(np.float64)
    a, b = rows['fused'], rows['gemm']
    d = np.abs(a - b)
    bound = 2.0 ** -6 * np.maximum(np.abs(a), np.abs(b)) + 2.0 ** -12     # two bf16 ulps, plus a floor near zero
    differing = float((d > 0).mean())
    say(f'[draft proj] fused vs gemm over {a.size} elements: {differing:.2e} of them differ, max |d| {d.max():.3g}, '
        f'max |d| / bound {float((d / bound).max()):.3g}')
    assert (d <= bound).all(), float((d / bound).max())
    assert differing <= 1e-3, differing


def test_refused_appends_leave_the_pool_unchanged():
    from qwen3_dspark_amd.draft import DraftKVPool
    gen = torch.Generator().manual_seed(SEED + 77)
    fc, cn, per = make_weights(gen, layers=2)
    pool = DraftKVPool(layers=2, slots=3, capacity=64, device=DEV, projector=projector(fc, cn, per))
    pool.add_request('a')
    pool.add_request('b')
    pool.append_committed({'a': randn_bf16(gen, 1, 10, FEATS).to(DEV), 'b': randn_bf16(gen, 1, 4, FEATS).to(DEV)})
    keys, values = pool.keys.clone(), pool.values.clone()

    def unchanged():
        assert pool.lengths == {'a': 10, 'b': 4}
        for l in range(2):
            for r, n in (('a', 10), ('b', 4)):
                s = pool.slot(r)
                assert torch.equal(pool.keys[l, s, :, :n], keys[l, s, :, :n])
                assert torch.equal(pool.values[l, s, :, :n], values[l, s, :, :n])

    bad = randn_bf16(gen, 1, 5, FEATS)
    bad[0, 3, 17] = float('nan')
    with pytest.raises(ValueError, match='finite'):
        pool.append_committed({'a': randn_bf16(gen, 1, 2, FEATS).to(DEV), 'b': bad.to(DEV)})
    unchanged()
    with pytest.raises(ValueError, match='capacity'):
        pool.append_committed({'a': randn_bf16(gen, 1, 55, FEATS).to(DEV)})
    with pytest.raises(ValueError, match='target_features'):
        pool.append_committed({'a': randn_bf16(gen, 1, 2, FEATS - 64).to(DEV)})
    with pytest.raises(KeyError):
        pool.append_committed({'zz': randn_bf16(gen, 1, 2, FEATS).to(DEV)})
    with pytest.raises(ValueError, match='at least one'):
        pool.append_committed({})
    unchanged()
    # a non-finite projection (an infinite weight) is refused after the launch
    kp = per[1][0].clone()
    kp[5, 9] = float('inf')
    pool.projector = projector(fc, cn, [per[0], (kp, per[1][1], per[1][2])])
    with pytest.raises(RuntimeError, match='Nonfinite projected'):
        pool.append_committed({'b': randn_bf16(gen, 1, 3, FEATS).to(DEV)})
    unchanged()


def test_full_draft_context_path_feeds_draft_attention():
    """The 16-request draft workload (contexts U[128, 1024], 4 blocks of 7 at
    seeded anchors): features of the five tapped target layers
    ([T, 1024] ~ N(0,1) each, concatenated to [T, 5120]) projected into the
    pool in two appends per request, then draft attention of every layer
    over the pool against the oracle."""
    from qwen3_dspark_amd.draft import DraftKVPool
    gen = torch.Generator().manual_seed(SEED + 3)
    rng = np.random.default_rng(SEED + 3)
    fc, cn, per = make_weights(gen)
    proj = projector(fc, cn, per)
    ctx = [int(c) for c in rng.integers(128, 1025, size=16)]
    names = [f'req{i}' for i in range(16)]
    pool = DraftKVPool(layers=LAYERS, slots=16, capacity=1024, device=DEV, projector=proj)
    for r in names:
        pool.add_request(r)
    taps = {r: torch.cat([randn_bf16(gen, 1, c, HIDDEN) for _ in range(5)], dim=-1) for r, c in zip(names, ctx)}
    split = {r: int(rng.integers(1, c)) for r, c in zip(names, ctx)}
    pool.append_committed({r: taps[r][:, :split[r]].to(DEV) for r in names})
    pool.append_committed({r: taps[r][:, split[r]:].to(DEV) for r in reversed(names)})
    assert pool.lengths == dict(zip(names, ctx))
    # every projected row against the oracle (device fc output as input)
    x = torch.cat([taps[r][0] for r in names])
    fc_dev = f64(proj.fc_forward(x.to(DEV)))
    pos = np.concatenate([np.arange(c) for c in ctx])
    weights = [(f64(kp), f64(kn), f64(vp)) for kp, kn, vp in per]
    ref = draft_proj.project_context_kv(None, None, f64(cn), weights, pos, fc_out=fc_dev)
    # both appends hold thousands of tokens, so they take the GEMM path and
    # its bar (see test_append_committed_against_oracle)
    for layer in range(LAYERS):
        got = [pool_rows(pool, layer, r, 0, c) for r, c in zip(names, ctx)]
        gate(np.concatenate([k for k, _ in got]), ref[layer][0], 4e-3)
        gate(np.concatenate([v for _, v in got]), ref[layer][1], 4e-3)
    anchors = {r: sorted(int(a) for a in rng.choice(c + 1, size=4, replace=False)) for r, c in zip(names, ctx)}
    batch = pool.batch(anchors)
    nb = 4 * 16
    offs = np.concatenate([[0], np.cumsum(ctx)[:-1]]).tolist()
    cu_b = list(range(0, nb + 1, 4))
    flat = [a for r in names for a in anchors[r]]
    for layer in range(LAYERS):
        q, bk, bv = randn_bf16(gen, 7 * nb, 16, 128), randn_bf16(gen, 7 * nb, 8, 128), randn_bf16(gen, 7 * nb, 8, 128)
        out = pool.attention(layer, q.to(DEV), bk.to(DEV), bv.to(DEV), batch)
        s = [pool.slot(r) for r in names]
        ck = np.concatenate([bits(pool.keys[layer, i, :, :c].transpose(0, 1)) for i, c in zip(s, ctx)])
        cv = np.concatenate([bits(pool.values[layer, i, :, :c].transpose(0, 1)) for i, c in zip(s, ctx)])
        ref_o = cref.draft_attention(bits(q), ck, cv, offs, ctx, bits(bk), bits(bv), cu_b, flat, scale=SCALE)
        attention_gate(out.float().cpu().numpy(), ref_o)
    say(f'[draft proj] 16-request path ok, contexts sum {sum(ctx)}')
