"""The full 5-layer DSpark draft forward on the GPU: PackedDraft
(qwen3_dspark_amd/draft_backbone.py, the drop-in for
dspark_qwen/packed_draft.py:63-249) over a random-init bf16 draft of
Qwen3-0.6B geometry (hidden 1024, 16/8 heads, head dim 128, MLP 3072).

The 16-request workload: contexts drawn uniformly from [128, 1024], target
features from five layers, each [T, 1024] ~ N(0,1), concatenated to
[T, 5120]; append_committed projects them (fc, RMSNorm, per-layer k_proj /
k_norm / RoPE / v_proj) into the pool; then 4 packed 7-token blocks per
request at seeded anchors run through every draft layer.  Checks:
  * every layer's attention launch against the float64 oracle on the exact
    Q, block K/V and pool rows it was given (the attention tolerance gate);
  * the final hidden rows against a control that runs the same bf16 modules
    with float32 dense attention over the same pool (isolates the kernel
    inside the whole forward), and against the float64 oracle of the whole
    forward (oracle/draft_model.py): the HIP path must not drift from it
    further than the control does;
  * the reference's one-block backbone (anchor = committed length) equals
    the multi-block call with those anchors, with the reference's work keys.
"""
import numpy as np
import pytest
import torch
from torch import nn

from helpers import SCALE, SEED, attention_gate, f64
from oracle import draft_model, draft_proj
from oracle.attention import draft_attention

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda:0')
HIDDEN, LAYERS, REQUESTS, BLOCKS = 1024, 5, 16, 4
MASK_TOKEN = 151669


def say(*a):
    print(*a, flush=True)


def rotate(x, cos, sin):
    left, right = x.chunk(2, dim=-1)
    return x * cos[:, None] + torch.cat((-right, left), -1) * sin[:, None]


def draft_module(seed):
    """A DSparkDraft-shaped module (the attribute names PackedDraft reads,
    dspark_qwen/model.py:27-98) with random bf16 weights."""
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3MLP, Qwen3RMSNorm, Qwen3RotaryEmbedding
    cfg = Qwen3Config(vocab_size=151936, hidden_size=HIDDEN, intermediate_size=3072, num_hidden_layers=28,
                      num_attention_heads=16, num_key_value_heads=8, head_dim=128, rope_theta=1e6,
                      rms_norm_eps=1e-6, max_position_embeddings=40960, attention_bias=False)

    class Attention(nn.Module):
        heads, kv_heads, dim = 16, 8, 128

        def __init__(self):
            super().__init__()
            self.q_proj = nn.Linear(HIDDEN, 2048, bias=False)
            self.k_proj = nn.Linear(HIDDEN, 1024, bias=False)
            self.v_proj = nn.Linear(HIDDEN, 1024, bias=False)
            self.o_proj = nn.Linear(2048, HIDDEN, bias=False)
            self.q_norm = Qwen3RMSNorm(128, eps=1e-6)
            self.k_norm = Qwen3RMSNorm(128, eps=1e-6)

        def project_kv(self, states, cos, sin):
            b = states.shape[0]
            k = self.k_norm(self.k_proj(states).view(b, -1, 8, 128)).transpose(1, 2)
            v = self.v_proj(states).view(b, -1, 8, 128).transpose(1, 2)
            return rotate(k, cos, sin), v

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.input_norm = Qwen3RMSNorm(HIDDEN, eps=1e-6)
            self.attention = Attention()
            self.post_norm = Qwen3RMSNorm(HIDDEN, eps=1e-6)
            self.mlp = Qwen3MLP(cfg)

    class Spec:
        block_size, mask_token_id = 7, MASK_TOKEN

    class Draft(nn.Module):
        def __init__(self):
            super().__init__()
            self.spec = Spec()
            self.fc = nn.Linear(5 * HIDDEN, HIDDEN, bias=False)
            self.context_norm = Qwen3RMSNorm(HIDDEN, eps=1e-6)
            self.layers = nn.ModuleList([Block() for _ in range(LAYERS)])
            self.norm = Qwen3RMSNorm(HIDDEN, eps=1e-6)
            self.rotary = Qwen3RotaryEmbedding(cfg)
            self.embedding = nn.Embedding(cfg.vocab_size, HIDDEN)

    torch.manual_seed(seed)
    with torch.device(DEV):
        d = Draft()
    with torch.no_grad():
        for name, p in d.named_parameters():
            if 'norm' in name:
                p.uniform_(0.5, 1.5)
    for m in (d.fc, d.context_norm, d.layers, d.norm, d.embedding):
        m.to(torch.bfloat16)          # the rotary's float32 inverse frequencies stay float32
    return d.eval()


def layer_weights(layer):
    a = layer.attention
    w = lambda m: f64(m.weight)
    return dict(input_norm=w(layer.input_norm), q_proj=w(a.q_proj), k_proj=w(a.k_proj), v_proj=w(a.v_proj),
                o_proj=w(a.o_proj), q_norm=w(a.q_norm), k_norm=w(a.k_norm), post_norm=w(layer.post_norm),
                gate=w(layer.mlp.gate_proj), up=w(layer.mlp.up_proj), down=w(layer.mlp.down_proj))


def workload(rng):
    contexts = [int(c) for c in rng.integers(128, 1025, size=REQUESTS)]
    anchors = []
    for c in contexts:
        rest = rng.choice(np.arange(c), size=BLOCKS - 1, replace=False)
        anchors.append([c] + sorted(int(a) for a in rest))
    return contexts, anchors


@torch.no_grad()
def control_backbone(draft, pd, blocks):
    """The same bf16 modules as PackedDraft, attention in float32 dense over
    the pool rows with the block mask (the control)."""
    outs = []
    for request, (tokens, anchors) in blocks.items():
        n, c = len(anchors), pd.lengths[request]
        toks = tokens.new_full((n, 7), MASK_TOKEN)
        toks[:, 0] = tokens[0]
        pos = (torch.tensor(anchors, device=DEV)[:, None] + torch.arange(7, device=DEV)).reshape(-1)
        z = draft.embedding(toks.reshape(1, -1))
        cos, sin = draft.rotary(z, pos[None])
        visible = torch.zeros(7 * n, c + 7 * n, dtype=torch.bool, device=DEV)
        for b, a in enumerate(anchors):
            visible[7 * b:7 * b + 7, :a] = True
            visible[7 * b:7 * b + 7, c + 7 * b:c + 7 * b + 7] = True
        slot = pd.pool.slot(request)
        for index, layer in enumerate(draft.layers):
            att = layer.attention
            x = layer.input_norm(z)
            q = rotate(att.q_norm(att.q_proj(x).view(1, -1, 16, 128)).transpose(1, 2), cos, sin)
            kb, vb = att.project_kv(x, cos, sin)
            with torch.autocast('cuda', enabled=False):      # float32 attention also under autocast
                k = torch.cat((pd.pool.keys[index, slot, :, :c][None], kb.to(torch.bfloat16)), dim=2).float()
                v = torch.cat((pd.pool.values[index, slot, :, :c][None], vb.to(torch.bfloat16)), dim=2).float()
                k = k.repeat_interleave(2, dim=1)
                v = v.repeat_interleave(2, dim=1).contiguous()
                s = torch.matmul(q.to(torch.bfloat16).float(), k.transpose(-1, -2).contiguous()) * SCALE
                o = torch.matmul(s.masked_fill(~visible, float('-inf')).softmax(-1), v)
                o = o.transpose(1, 2).reshape(1, 7 * n, -1).to(torch.bfloat16)
            z = z + att.o_proj(o)
            z = z + layer.mlp(layer.post_norm(z))
        outs.append(draft.norm(z)[0])
    return torch.cat(outs)


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@torch.no_grad()
def test_config3_full_draft_forward():
    from qwen3_dspark_amd import backends
    from qwen3_dspark_amd.draft_backbone import PackedDraft
    draft = draft_module(SEED)
    rng = np.random.default_rng(SEED)
    contexts, anchors = workload(rng)
    names = [f'r{i}' for i in range(REQUESTS)]
    gen = torch.Generator().manual_seed(SEED)
    features = [torch.randn(1, c, 5 * HIDDEN, generator=gen).to(torch.bfloat16).to(DEV) for c in contexts]
    pd = PackedDraft(draft, native_backend=backends.DRAFT_BLOCKS_BACKEND, slots=REQUESTS, capacity=1024)
    for n in names:
        pd.add_request(n)
    work = pd.append_committed(dict(zip(names, features)))
    assert work['new_context_tokens'] == sum(contexts) and pd.lengths == dict(zip(names, contexts))
    say(f'[config3] appended {sum(contexts)} context rows for {REQUESTS} requests')

    tokens = {n: torch.tensor([rng.integers(0, 151936, size=BLOCKS).tolist()], device=DEV) for n in names}
    blocks = {n: (tokens[n], a) for n, a in zip(names, anchors)}
    calls = []
    attention = pd.pool.attention

    def record(layer, q, kb, vb, batch, *, scale):
        out = attention(layer, q, kb, vb, batch, scale=scale)
        calls.append((layer, q.clone(), kb.clone(), vb.clone(), out.clone()))
        return out
    pd.pool.attention = record
    feats = pd.backbone_blocks(blocks)
    pd.pool.attention = attention
    torch.cuda.synchronize()
    assert feats.hidden.shape == (REQUESTS * BLOCKS * 7, HIDDEN) and feats.blocks == (BLOCKS,) * REQUESTS
    assert feats.work['attention_calls'] == LAYERS and feats.work['mlp_calls'] == LAYERS
    assert feats.work['query_rows'] == 7 * BLOCKS * REQUESTS
    assert feats.work['attention_pair_domain'] == sum(7 * (a + 7) for row in anchors for a in row)
    assert len(calls) == LAYERS

    # every layer's attention launch against the oracle on its own inputs
    row0 = np.cumsum([0] + [7 * BLOCKS] * REQUESTS)
    for layer, q, kb, vb, out in calls:
        ref = np.zeros(out.shape)
        for r, n in enumerate(names):
            s = pd.pool.slot(n)
            ck = f64(pd.pool.keys[layer, s, :, :contexts[r]].transpose(0, 1))
            cv = f64(pd.pool.values[layer, s, :, :contexts[r]].transpose(0, 1))
            lo, hi = row0[r], row0[r + 1]
            ref[lo:hi] = draft_attention(f64(q[lo:hi]), ck, cv, f64(kb[lo:hi]), f64(vb[lo:hi]), anchors[r],
                                         scale=SCALE)
        stats = attention_gate(f64(out), ref)
        say(f'[config3] layer {layer} attention max |d| {stats[0]["max_abs"]:.2e} mean {stats[0]["mean_abs"]:.2e}')

    # whole forward: control and float64 oracle
    control = f64(control_backbone(draft, pd, blocks))
    hidden = f64(feats.hidden)
    fc_out = f64(pd.projector.fc_forward(torch.cat([f[0] for f in features])))
    weights = [layer_weights(l) for l in draft.layers]
    proj = [(w['k_proj'], w['k_norm'], w['v_proj']) for w in weights]
    worst = 0.0
    first = 0
    for r, n in enumerate(names):
        c = contexts[r]
        kv = draft_proj.project_context_kv(None, f64(draft.fc.weight), f64(draft.context_norm.weight), proj,
                                           np.arange(c), fc_out=fc_out[first:first + c])
        first += c
        toks = torch.full((BLOCKS, 7), MASK_TOKEN, device=DEV)
        toks[:, 0] = tokens[n][0]
        z0 = f64(draft.embedding(toks.reshape(1, -1))[0])
        ref = draft_model.draft_backbone(z0, weights, kv, anchors[r], f64(draft.norm.weight))
        lo, hi = row0[r], row0[r + 1]
        err, drift, ctl_drift = rel(hidden[lo:hi], control[lo:hi]), rel(hidden[lo:hi], ref), rel(control[lo:hi], ref)
        worst = max(worst, err)
        assert err < 3e-2, (n, err)
        assert drift <= 1.1 * ctl_drift + 5e-3, (n, drift, ctl_drift)
        assert np.allclose(f64(feats.for_request(n)), hidden[lo:hi])
    say(f'[config3] hidden: worst rel err vs the float32-attention control {worst:.2e}; '
        f'last drift vs float64 {drift:.2e} (control {ctl_drift:.2e})')


@torch.no_grad()
def test_one_block_backbone_and_contract():
    from qwen3_dspark_amd import backends
    from qwen3_dspark_amd.draft_backbone import PackedDraft
    draft = draft_module(SEED + 1)
    names = ['a', 'b', 'c']
    lengths = [300, 41, 777]
    gen = torch.Generator().manual_seed(7)
    with pytest.raises(ValueError, match='explicit noncausal draft backend'):
        PackedDraft(draft, native_backend=backends.REFERENCE_DRAFT_BACKEND, slots=4, capacity=1024)
    pd = PackedDraft(draft, native_backend=backends.DRAFT_BLOCKS_BACKEND, slots=4, capacity=1024)
    assert pd.kernel.backend_name == backends.DRAFT_BLOCKS_BACKEND
    for n, c in zip(names, lengths):
        pd.add_request(n)
        pd.append_committed({n: torch.randn(1, c, 5 * HIDDEN, generator=gen).to(torch.bfloat16).to(DEV)})
    anchors = {n: torch.tensor([[int(t)]], device=DEV) for n, t in zip(names, (11, 151935, 0))}
    one = pd.backbone(anchors)
    multi = pd.backbone_blocks({n: (anchors[n], (pd.lengths[n],)) for n in names})
    assert torch.equal(one.hidden, multi.hidden)
    assert one.context_lengths == tuple(lengths) and one.requests == tuple(names)
    assert torch.equal(one.for_request('b'), one.hidden[7:14])
    keys = {'requests', 'query_rows', 'gathered_key_rows', 'physical_context_rows', 'attention_pair_domain',
            'attention_calls', 'context_block_concatenation_kv_elements', 'context_block_concatenation_kv_bytes',
            'gathered_kv_elements', 'gathered_kv_bytes', 'attention_cast_elements', 'attention_cast_output_bytes',
            'mlp_calls', 'scope'}
    assert keys <= set(one.work)
    assert one.work['gathered_key_rows'] == sum(lengths) + 21 and one.work['query_rows'] == 21
    # reference errors (packed_draft.py:187-203)
    with pytest.raises(ValueError, match='Require active anchor requests'):
        pd.backbone({})
    with pytest.raises(ValueError, match='valid'):
        pd.backbone({'a': torch.tensor([[151936]], device=DEV)})
    with pytest.raises(KeyError):
        pd.backbone({'zz': anchors['a']})
    with pytest.raises(ValueError, match='anchor'):
        pd.backbone_blocks({'b': (torch.tensor([[1]], device=DEV), (42,))})
    # a crop moves the one-block anchor: the block now sees 100 rows of 'c'
    pd.crop('c', 100)
    cropped = pd.backbone({'c': anchors['c']})
    assert cropped.context_lengths == (100,)
    again = pd.backbone_blocks({'c': (anchors['c'], (100,))})
    assert torch.equal(cropped.hidden, again.hidden)
    draft.train()
    with pytest.raises(ValueError, match='inference-only'):
        pd.backbone(anchors)
    draft.eval()


@torch.no_grad()
def test_backbone_under_autocast_with_float32_draft():
    """The reference's own precision form (model.py:111: float32 trainable
    weights under bf16 autocast): Q and block K reach the kernel in fp32
    (q_norm / k_norm run in fp32) and are rounded as it loads them, V in
    bf16; the context projection runs on bf16 snapshots of the weights.
    Checked against the float32-attention control under the same autocast,
    and against the float64 oracle of the whole forward on the float32
    weights."""
    from qwen3_dspark_amd import backends
    from qwen3_dspark_amd.draft_backbone import PackedDraft
    draft = draft_module(SEED + 2)
    for m in (draft.fc, draft.context_norm, draft.layers, draft.norm, draft.embedding):
        m.float()
    names, lengths = ['a', 'b', 'c', 'd'], [200, 1024, 37, 513]
    rng = np.random.default_rng(SEED + 2)
    gen = torch.Generator().manual_seed(SEED + 2)
    pd = PackedDraft(draft, native_backend=backends.DRAFT_BLOCKS_BACKEND, slots=4, capacity=1024)
    features = [torch.randn(1, c, 5 * HIDDEN, generator=gen).to(DEV) for c in lengths]
    for n in names:
        pd.add_request(n)
    pd.append_committed(dict(zip(names, features)))
    anchors = [[c] + sorted(int(a) for a in rng.choice(np.arange(c), size=2, replace=False)) for c in lengths]
    tokens = {n: torch.tensor([rng.integers(0, 151936, size=3).tolist()], device=DEV) for n in names}
    blocks = {n: (tokens[n], a) for n, a in zip(names, anchors)}
    with torch.autocast('cuda', dtype=torch.bfloat16):
        feats = pd.backbone_blocks(blocks)
        control = f64(control_backbone(draft, pd, blocks))
    hidden = f64(feats.hidden)
    assert np.isfinite(hidden).all()
    fc_out = f64(pd.projector.fc_forward(torch.cat([f[0] for f in features]).to(torch.bfloat16)))
    weights = [layer_weights(l) for l in draft.layers]
    proj = [(w['k_proj'], w['k_norm'], w['v_proj']) for w in weights]
    first = 0
    for r, n in enumerate(names):
        c = lengths[r]
        kv = draft_proj.project_context_kv(None, f64(draft.fc.weight), f64(draft.context_norm.weight), proj,
                                           np.arange(c), fc_out=fc_out[first:first + c])
        first += c
        toks = torch.full((3, 7), MASK_TOKEN, device=DEV)
        toks[:, 0] = tokens[n][0]
        z0 = f64(draft.embedding(toks.reshape(1, -1))[0])
        ref = draft_model.draft_backbone(z0, weights, kv, anchors[r], f64(draft.norm.weight))
        lo, hi = 21 * r, 21 * (r + 1)
        err, drift, ctl_drift = rel(hidden[lo:hi], control[lo:hi]), rel(hidden[lo:hi], ref), rel(control[lo:hi], ref)
        say(f'[autocast] {n}: rel err vs control {err:.2e}, drift vs float64 {drift:.2e} (control {ctl_drift:.2e})')
        assert err < 3e-2, (n, err)
        assert drift <= 1.1 * ctl_drift + 5e-3, (n, drift, ctl_drift)
