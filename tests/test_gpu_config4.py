"""The full verification round at its real shape: a 28-layer Qwen3-0.6B-shaped
target (hidden 1024, 16/8 heads, head dim 128, vocab 151,936, random-init
bf16 weights), 32 requests with cached contexts drawn uniformly from
[256, 2048] and prefilled through the fused path, then 7 appended tokens per
request (ids uniform over the vocabulary) verified with all-layer stage,
gather and attention, a seeded accepted prefix of 0..7 committed and the rest
rolled back, and a second verification over the committed rows
(persistent_qwen_target.py:396-457 over persistent_target_kv.py).

The logits of every verified row are checked, per request, against two
references over the request's full token sequence (the reference's dense
oracle, persistent_qwen_target.py:30-42, at model level):
* the same bf16 model with plain-torch float32 causal attention (a
  registered attention function): same rounding points everywhere except
  inside attention, so it isolates the HIP path, gated at a relative
  Frobenius error of 3e-2;
* the same weights run entirely in float32: through 28 layers of bf16
  activations the bf16 model itself drifts by ~4-7 % from it, so the HIP
  path must not drift further than the float32-attention control does.
"""
import numpy as np
import pytest
import torch

from helpers import SEED

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda:0')
NEW = 7
REQUESTS = 32
LO, HI = 256, 2048
REL_TOL = 3e-2


def say(*a):
    print(*a, flush=True)


def fp32_causal_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """[1, Hq, Q, D] x [1, Hkv, K, D] bottom-right causal attention in float32
    (no cache: Q == K here); returns [1, Q, Hq, D] in the query dtype."""
    q, k, v = query.float(), key.float(), value.float()
    rep = q.shape[1] // k.shape[1]
    k = k.repeat_interleave(rep, dim=1)
    v = v.repeat_interleave(rep, dim=1).contiguous()
    s = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scaling
    n_q, n_k = s.shape[-2:]
    visible = torch.ones(n_q, n_k, dtype=torch.bool, device=s.device).tril(n_k - n_q)
    out = torch.matmul(s.masked_fill(~visible, float('-inf')).softmax(-1), v)
    return out.transpose(1, 2).contiguous().to(query.dtype), None


def qwen3_06b_models():
    """(float32 model, bf16 model with float32 attention, bf16 model for the
    HIP path), all with the same bf16-representable random weights."""
    from transformers import AttentionInterface, Qwen3Config, Qwen3ForCausalLM
    AttentionInterface.register('dspark_test_fp32', fp32_causal_attention)
    kw = dict(vocab_size=151936, hidden_size=1024, intermediate_size=3072, num_hidden_layers=28,
              num_attention_heads=16, num_key_value_heads=8, head_dim=128, max_position_embeddings=40960,
              rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)
    ref_cfg = Qwen3Config(**kw)
    ref_cfg._attn_implementation = 'eager'
    torch.manual_seed(SEED)
    with torch.device(DEV):
        ref = Qwen3ForCausalLM(ref_cfg).eval()
    with torch.no_grad():
        for p in ref.parameters():
            p.copy_(p.to(torch.bfloat16).float())      # bf16-representable weights
    models = []
    for impl in ('dspark_test_fp32', 'sdpa'):          # the verifier rebinds the second one's attention
        cfg = Qwen3Config(**kw)
        cfg._attn_implementation = impl
        with torch.device(DEV):
            m = Qwen3ForCausalLM(cfg).eval()
        m.load_state_dict(ref.state_dict())
        models.append(m.to(torch.bfloat16))
    return ref, models[0], models[1]


def rel_err(got, want):
    got = got.double()
    want = want.double()
    return float(torch.linalg.vector_norm(got - want) / torch.linalg.vector_norm(want))


@torch.no_grad()
def test_config4_verification_round_full_size():
    from qwen3_dspark_amd import backends
    from qwen3_dspark_amd.persistent_target import PersistentQwenTarget
    from qwen3_dspark_amd.persistent_kv import Bucket
    ref, control, model = qwen3_06b_models()
    rng = np.random.default_rng(SEED)
    lengths = [int(n) for n in rng.integers(LO, HI + 1, size=REQUESTS)]
    seqs = [rng.integers(0, 151936, size=n).tolist() for n in lengths]
    names = [f'r{i}' for i in range(REQUESTS)]
    capacity = HI + 2 * NEW
    target = PersistentQwenTarget(model, native_backend=backends.CAPACITY_BACKEND, slots=REQUESTS, context_capacity=capacity, max_query_tokens=sum(lengths),
                                  workspace_byte_budget=1 << 31)
    for n in names:
        target.add_request(n)
    t = lambda ids: torch.tensor([ids], device=DEV)
    pre = Bucket(tuple(lengths), (0,) * REQUESTS, 'prefill')
    target.register_bucket(pre)
    target.prefill({n: t(s) for n, s in zip(names, seqs)}, bucket=pre)
    assert target.lengths == dict(zip(names, lengths))
    say(f'[config4] prefilled {REQUESTS} requests, {sum(lengths)} tokens')
    step = Bucket((NEW,) * REQUESTS, (capacity - NEW,) * REQUESTS, 'verify')
    target.register_bucket(step)
    worst = 0.0
    for rnd in range(2):
        new = [rng.integers(0, 151936, size=NEW).tolist() for _ in seqs]
        feats = target.verify({n: t(x) for n, x in zip(names, new)}, bucket=step)
        logits = target.predict(feats)
        for r, n in enumerate(names):
            full = t(seqs[r] + new[r])
            f32 = ref(input_ids=full, use_cache=False).logits[0, -NEW:]
            ctl = control(input_ids=full, use_cache=False).logits[0, -NEW:]
            err = rel_err(logits[n][0], ctl)
            drift, ctl_drift = rel_err(logits[n][0], f32), rel_err(ctl, f32)
            worst = max(worst, err)
            assert err < REL_TOL, (rnd, n, len(seqs[r]), err)
            assert drift <= 1.1 * ctl_drift + 5e-3, (rnd, n, drift, ctl_drift)
        accepted = [int(a) for a in rng.integers(0, NEW + 1, size=REQUESTS)]
        before = {n: target.request_kv(n) for n in names[:4]}
        target.commit(feats, dict(zip(names, accepted)))
        seqs = [s + x[:a] for s, x, a in zip(seqs, new, accepted)]
        assert target.lengths == {n: len(s) for n, s in zip(names, seqs)}
        for r, n in enumerate(names[:4]):
            # the committed prefix is appended; earlier rows are untouched
            after = target.request_kv(n)
            for (k0, v0), (k1, v1) in zip(before[n], after):
                assert k1.shape[2] == k0.shape[2] + accepted[r]
                assert torch.equal(k1[:, :, :k0.shape[2]], k0) and torch.equal(v1[:, :, :v0.shape[2]], v0)
        say(f'[config4] round {rnd}: accepted {sum(accepted)}, worst rel err vs the float32-attention model '
            f'{worst:.2e}')
