"""The fused paths behind the reference's own constructors and pool.

* The paired benchmark's construction (scripts/benchmark_paired_r1.py:171-172):
  PersistentQwenTarget(m, ids, native_backend=..., graph_backend=TorchGraphBackend(),
  slots=..., context_capacity=..., max_query_tokens=..., max_buckets=...,
  max_graph_buckets=..., graph_byte_budget=..., workspace_byte_budget=...)
  and PackedDraft(d, native_backend=...), with only the backend names
  swapped for this build's, running a speculative round: prefill, draft
  context append, draft backbone, captured-graph verification, commit,
  append of the accepted features, a second draft backbone.  Gates: every
  draft layer's attention launch against the float64 oracle on its own
  inputs, the draft hidden rows against a float32-attention control and the
  float64 forward, the target logits against the CPU float32 model.
* The growable draft pool (no slots/capacity given): growth keeps every
  committed row bit for bit, and a grown pool's backbone equals a fixed
  pool's bit for bit.
* The reference's append-order pool ([1, 8, N, 128] per layer with the
  PackedLayout of its backbone call) through the multi-block kernel
  (HipDraftAttention.over_append_order_pool, the backbone edit shown in the
  integration notes): against the oracle's noncausal attention over the
  layout's gather, in bf16 and in the AMP form (FP32 K pool and Q/K, BF16 V),
  and before the first append (no pool yet).
"""
import copy

import numpy as np
import pytest
import torch

from helpers import SCALE, SEED, attention_gate, f64, segments
from oracle import draft_model, draft_proj
from oracle.attention import draft_attention, varlen_attention
from test_gpu_draft_backbone import MASK_TOKEN, control_backbone, draft_module, layer_weights, rel
from test_gpu_hf_hooks import close

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda:0')
HIDDEN = 1024
TARGET_LAYERS = 6
FEATURE_LAYERS = (1, 2, 3, 4, 5)
VOCAB = 4096


def say(*a):
    print(*a, flush=True)


def bf(t):
    return t.to(torch.bfloat16)


# ---------------------------------------------------------------------------
# the reference's append-order pool through the multi-block kernel
# ---------------------------------------------------------------------------

def append_order_state(contexts, gen):
    """Per-request context rows appended in three interleaved rounds, as the
    reference's PackedDraft.append_committed leaves key_requests /
    key_positions (markers 10, 11, ...)."""
    req, pos, done = [], [], [0] * len(contexts)
    for part in range(3):
        for r, c in enumerate(contexts):
            n = c // 3 + (c % 3 if part == 2 else 0)
            req += [10 + r] * n
            pos += range(done[r], done[r] + n)
            done[r] += n
    assert done == list(contexts)
    return torch.tensor(req, dtype=torch.long), torch.tensor(pos, dtype=torch.long)


@torch.no_grad()
@pytest.mark.parametrize('form', ['bf16', 'amp', 'no_pool'])
def test_reference_append_order_pool_through_blocks_kernel(form):
    from qwen3_dspark_amd.draft import HipDraftAttention
    from qwen3_dspark_amd.layout import PackedLayout
    gen = torch.Generator().manual_seed(SEED)
    contexts = [0, 0, 0] if form == 'no_pool' else [0, 77, 301, 1500]
    n = len(contexts)
    kreq, kpos = append_order_state(contexts, gen)
    N = kreq.numel()
    qreq = torch.tensor([10 + r for r in range(n) for _ in range(7)])
    qpos = torch.tensor([c + i for c in contexts for i in range(7)])
    layout = PackedLayout.from_metadata(qreq.to(DEV), qpos.to(DEV), torch.cat((kreq, qreq)).to(DEV),
                                        torch.cat((kpos, qpos)).to(DEV))
    kdt = torch.float32 if form == 'amp' else torch.bfloat16
    # fp32 K / Q hold values off the bf16 grid: the kernel rounds them as it loads
    q = torch.randn(7 * n, 16, 128, generator=gen).to(kdt)
    kb = torch.randn(1, 8, 7 * n, 128, generator=gen).to(kdt)
    vb = bf(torch.randn(1, 8, 7 * n, 128, generator=gen))
    pool_k = torch.randn(1, 8, max(N, 1), 128, generator=gen).to(kdt)
    pool_v = bf(torch.randn(1, 8, max(N, 1), 128, generator=gen))
    attn = HipDraftAttention(DEV)
    args = (None, None) if form == 'no_pool' else (pool_k.to(DEV), pool_v.to(DEV))
    out = attn.over_append_order_pool(q.to(DEV), kb.to(DEV), vb.to(DEV), *args, layout, scale=SCALE)
    torch.cuda.synchronize()
    # the reference's path: cat(pool, block), index_select by the layout's
    # gather indices, cast to bf16, noncausal attention per request
    kk = torch.cat((pool_k[:, :, :N], kb), dim=2)[0].transpose(0, 1)
    vv = torch.cat((pool_v[:, :, :N], vb), dim=2)[0].transpose(0, 1)
    idx = layout.gather_indices.cpu()
    ref = varlen_attention(f64(bf(q)), f64(bf(kk[idx])), f64(vv[idx]), layout.cu_query.tolist(),
                           layout.cu_key.tolist(), causal=False, scale=SCALE)
    stats = attention_gate(f64(out), ref, segments(layout.cu_query.tolist()))
    say(f'[append-order {form}] max |d| {stats[0]["max_abs"]:.2e} mean {stats[0]["mean_abs"]:.2e}')
    if form == 'amp':
        again = attn.over_append_order_pool(bf(q).to(DEV), bf(kb).to(DEV), vb.to(DEV), bf(pool_k).to(DEV),
                                            pool_v.to(DEV), layout, scale=SCALE)
        assert torch.equal(out, again), 'fp32 inputs must give the bits of their bf16 rounding'


# ---------------------------------------------------------------------------
# growable pool
# ---------------------------------------------------------------------------

@torch.no_grad()
def test_growable_pool_keeps_rows_and_matches_a_fixed_pool():
    from qwen3_dspark_amd import backends
    from qwen3_dspark_amd.draft_backbone import PackedDraft
    draft = draft_module(SEED + 5)
    grow = PackedDraft(draft, native_backend=backends.DRAFT_BLOCKS_BACKEND)
    fixed = PackedDraft(draft, native_backend=backends.DRAFT_BLOCKS_BACKEND, slots=16, capacity=2560)
    assert (grow.pool.slot_capacity, grow.pool.capacity) == (PackedDraft.INITIAL_SLOTS, PackedDraft.INITIAL_CAPACITY)
    gen = torch.Generator().manual_seed(SEED + 5)
    names = [f'g{i}' for i in range(10)]
    first = [40 + 97 * i for i in range(10)]
    for n in names:
        grow.add_request(n)
        fixed.add_request(n)
    assert grow.pool.slot_capacity == 16 and grow.pool.resizes == 1
    feats = {n: bf(torch.randn(1, c, 5 * HIDDEN, generator=gen)).to(DEV) for n, c in zip(names, first)}
    for pd in (grow, fixed):
        pd.append_committed(feats)
    before = {n: grow.request_kv(n) for n in names}
    more = {n: bf(torch.randn(1, 700 + 50 * i, 5 * HIDDEN, generator=gen)).to(DEV)
            for i, n in enumerate(names[5:])}
    for pd in (grow, fixed):
        pd.append_committed(more)
    assert grow.pool.capacity >= max(grow.lengths.values()) > PackedDraft.INITIAL_CAPACITY
    say(f'[grow] slots {grow.pool.slot_capacity}, capacity {grow.pool.capacity}, resizes {grow.pool.resizes}')
    assert grow.lengths == fixed.lengths
    for n in names:
        for (k0, v0), (k1, v1), (kf, vf) in zip(before[n], grow.request_kv(n), fixed.request_kv(n)):
            c = k0.shape[2]
            assert torch.equal(k1[:, :, :c], k0) and torch.equal(v1[:, :, :c], v0)
            assert torch.equal(k1, kf) and torch.equal(v1, vf)
    anchors = {n: torch.tensor([[int(t)]], device=DEV) for n, t in zip(names, range(100, 110))}
    a, b = grow.backbone(anchors), fixed.backbone(anchors)
    assert torch.equal(a.hidden, b.hidden)
    grow.remove_request('g3')
    grow.add_request('late')           # reuses the freed slot, no growth
    assert grow.pool.slot_capacity == 16 and grow.lengths['late'] == 0


# ---------------------------------------------------------------------------
# the paired construction and one speculative round
# ---------------------------------------------------------------------------

def target_models():
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=VOCAB, hidden_size=HIDDEN, intermediate_size=3072, num_hidden_layers=TARGET_LAYERS,
                      num_attention_heads=16, num_key_value_heads=8, head_dim=128, max_position_embeddings=8192,
                      rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=False)
    cfg._attn_implementation = 'sdpa'
    torch.manual_seed(SEED)
    cpu = Qwen3ForCausalLM(cfg).eval().to(torch.bfloat16).float()
    gpu = Qwen3ForCausalLM(copy.deepcopy(cfg)).eval()
    gpu.load_state_dict(cpu.state_dict())
    return cpu, gpu.to(torch.bfloat16).to(DEV)


def gate_draft_round(pd, draft, calls, blocks, feats, features_by_request):
    """Each recorded attention launch against the oracle; the hidden rows
    against the float32-attention control and the float64 forward."""
    names = list(blocks)
    row0 = np.cumsum([0] + [7 * len(blocks[n][1]) for n in names])
    for layer, q, kb, vb, out in calls:
        ref = np.zeros(out.shape)
        for r, n in enumerate(names):
            s, c = pd.pool.slot(n), pd.lengths[n]
            ck = f64(pd.pool.keys[layer, s, :, :c].transpose(0, 1))
            cv = f64(pd.pool.values[layer, s, :, :c].transpose(0, 1))
            lo, hi = row0[r], row0[r + 1]
            ref[lo:hi] = draft_attention(f64(q[lo:hi]), ck, cv, f64(kb[lo:hi]), f64(vb[lo:hi]), blocks[n][1],
                                         scale=SCALE)
        attention_gate(f64(out), ref)
    control = f64(control_backbone(draft, pd, blocks))
    hidden = f64(feats.hidden)
    weights = [layer_weights(l) for l in draft.layers]
    proj = [(w['k_proj'], w['k_norm'], w['v_proj']) for w in weights]
    for r, n in enumerate(names):
        x = torch.cat(features_by_request[n], dim=1)[0]
        c = x.shape[0]
        fc_out = f64(pd.projector.fc_forward(bf(x).contiguous()))
        kv = draft_proj.project_context_kv(None, f64(draft.fc.weight), f64(draft.context_norm.weight), proj,
                                           np.arange(c), fc_out=fc_out)
        toks = torch.full((len(blocks[n][1]), 7), MASK_TOKEN, device=DEV)
        toks[:, 0] = blocks[n][0][0]
        z0 = f64(draft.embedding(toks.reshape(1, -1))[0])
        ref = draft_model.draft_backbone(z0, weights, kv, blocks[n][1], f64(draft.norm.weight))
        lo, hi = row0[r], row0[r + 1]
        err, drift, ctl = rel(hidden[lo:hi], control[lo:hi]), rel(hidden[lo:hi], ref), rel(control[lo:hi], ref)
        assert err < 3e-2, (n, err)
        assert drift <= 1.1 * ctl + 5e-3, (n, drift, ctl)


@torch.no_grad()
def test_paired_construction_runs_a_speculative_round():
    from qwen3_dspark_amd import backends
    from qwen3_dspark_amd.draft_backbone import PackedDraft
    from qwen3_dspark_amd.graph import TorchGraphBackend
    from qwen3_dspark_amd.persistent_kv import Bucket
    from qwen3_dspark_amd.persistent_target import PersistentQwenTarget
    BACKEND, DRAFT_BACKEND = backends.CAPACITY_BACKEND, backends.DRAFT_BLOCKS_BACKEND
    protocol = dict(slots=4, context_capacity=640, max_query_tokens=640, max_buckets=4, max_graph_buckets=1,
                    graph_byte_budget=1 << 32, workspace_byte_budget=1 << 30)
    cpu, model = target_models()
    d = draft_module(SEED + 7)
    # scripts/benchmark_paired_r1.py:171-172 and :177-179, backend names swapped
    target_builder = lambda m, ids, **kw: PersistentQwenTarget(m, ids, native_backend=BACKEND, **kw)
    draft_builder = lambda d: PackedDraft(d, native_backend=DRAFT_BACKEND)
    target = target_builder(model, FEATURE_LAYERS, graph_backend=TorchGraphBackend(), **protocol)
    pd = draft_builder(d)
    backends.check_session_backends(target, pd)
    rng = np.random.default_rng(SEED)
    names = ['r0', 'r1', 'r2', 'r3']
    seqs = [rng.integers(0, VOCAB, size=n).tolist() for n in (50, 211, 13, 333)]
    t = lambda x: torch.tensor([x], device=DEV)
    for n in names:
        target.add_request(n)
        pd.add_request(n)
    pre = Bucket(tuple(len(s) for s in seqs), (0,) * 4, 'prefill')
    target.register_bucket(pre)
    f = target.prefill({n: t(s) for n, s in zip(names, seqs)}, bucket=pre)
    history = {n: [f.for_request(n).context] for n in names}
    pd.append_committed({n: history[n][0] for n in names})
    target.release_features(f)
    assert pd.lengths == target.lengths == {n: len(s) for n, s in zip(names, seqs)}
    say('[paired] prefilled and projected the draft context')

    def draft_round():
        calls, attention = [], pd.pool.attention

        def record(layer, q, kb, vb, batch, *, scale):
            out = attention(layer, q, kb, vb, batch, scale=scale)
            calls.append((layer, q.clone(), kb.clone(), vb.clone(), out.clone()))
            return out
        anchors = {n: t([s[-1]]) for n, s in zip(names, seqs)}
        pd.pool.attention = record
        try:
            feats = pd.backbone(anchors)
        finally:
            pd.pool.attention = attention
        blocks = {n: (anchors[n], (pd.lengths[n],)) for n in names}
        gate_draft_round(pd, d, calls, blocks, feats, history)
        return feats

    draft_round()
    say('[paired] draft round 1 meets the oracle gate')
    step = Bucket((7,) * 4, (640 - 7,) * 4, 'paired verify')
    target.register_graph_bucket(step, reserve_bytes=256 << 20)
    target.capture_graph({n: t(rng.integers(0, VOCAB, size=7).tolist()) for n in names}, bucket=step)
    new = [[s[-1]] + rng.integers(0, VOCAB, size=6).tolist() for s in seqs]
    g = target.verify({n: t(x) for n, x in zip(names, new)}, bucket=step)
    assert g.work['execution_kind'] == TorchGraphBackend.kind
    logits = target.predict(g)
    for r, n in enumerate(names):
        ref = cpu(input_ids=torch.tensor([seqs[r] + new[r]]), use_cache=False).logits[0, -7:].numpy()
        close(logits[n][0].float().cpu().numpy(), ref, (n, 'graph logits'))
    accepted = dict(zip(names, (7, 0, 3, 5)))
    target.commit(g, accepted)
    # the accepted rows' features go to the draft before the lease ends
    kept = {n: g.for_request(n).context[:, :a].clone() for n, a in accepted.items() if a}
    pd.append_committed(kept)
    target.release_features(g)
    for n, x in kept.items():
        history[n].append(x)
    seqs = [s + x[:accepted[n]] for n, s, x in zip(names, seqs, new)]
    assert pd.lengths == target.lengths == {n: len(s) for n, s in zip(names, seqs)}
    draft_round()
    say('[paired] verify round committed; draft round 2 meets the oracle gate')
    target.close()


@torch.no_grad()
def test_backbone_refusals_follow_the_native_contract():
    """A float32 draft run without autocast is refused as the reference's
    native kernel refuses non-BF16 tensors (rocm_varlen.py:65-70); a
    non-finite attention output raises the per-layer message of
    packed_draft.py:237-239 before the hidden check; neither changes the pool."""
    from qwen3_dspark_amd import backends
    from qwen3_dspark_amd.draft_backbone import PackedDraft
    draft = draft_module(SEED + 9)
    pd = PackedDraft(draft, native_backend=backends.DRAFT_BLOCKS_BACKEND)
    gen = torch.Generator().manual_seed(SEED + 9)
    for n, c in (('a', 60), ('b', 200)):
        pd.add_request(n)
        pd.append_committed({n: bf(torch.randn(1, c, 5 * HIDDEN, generator=gen)).to(DEV)})
    anchors = {'a': torch.tensor([[5]], device=DEV), 'b': torch.tensor([[6]], device=DEV)}
    with pytest.raises(ValueError, match='CPU-only test injection'):
        PackedDraft(draft, native_backend=backends.DRAFT_BLOCKS_BACKEND, test_kernel=object())
    with pytest.raises(ValueError, match='both slots and capacity'):
        PackedDraft(draft, native_backend=backends.DRAFT_BLOCKS_BACKEND, slots=4)
    ok = pd.backbone(anchors)
    for m in (draft.layers, draft.norm, draft.embedding):
        m.float()
    with pytest.raises(ValueError, match='BF16 THD tensors'):
        pd.backbone(anchors)
    for m in (draft.layers, draft.norm, draft.embedding):
        m.to(torch.bfloat16)
    assert torch.equal(pd.backbone(anchors).hidden, ok.hidden)
    slot = pd.pool.slot('b')
    saved = pd.pool.values[2, slot, :, 17].clone()
    pd.pool.values[2, slot, :, 17] = float('nan')
    with pytest.raises(RuntimeError, match='^Invalid packed draft attention output$'):
        pd.backbone(anchors)
    pd.pool.values[2, slot, :, 17] = saved
    assert torch.equal(pd.backbone(anchors).hidden, ok.hidden)
