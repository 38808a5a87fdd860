"""HF transformers hooks on the fused verification path
(dspark_qwen/persistent_qwen_target.py:45-95; varlen_target.py:115-129).

A 2-layer Qwen3-shaped model (16 query heads, 8 KV heads, head dim 128,
random init, bf16 on the GPU) verifies 7 new tokens per request over a
PersistentTargetKV prefix, commits an accepted prefix and verifies again.
The logits must match the same weights run in float32 on the CPU over each
request's full token sequence (prefix + accepted + new) with HF's own
attention.  The GPU runs no torch attention: only GEMMs, norms and the HIP
kernels behind the hooks.
"""
import copy

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda:0')
NEW = 7


def tiny_qwen3():
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=16, num_key_value_heads=8, head_dim=128, max_position_embeddings=4096,
                      rope_theta=1e6, tie_word_embeddings=False)
    cfg._attn_implementation = 'sdpa'
    torch.manual_seed(20261009)
    cpu = Qwen3ForCausalLM(cfg).eval().to(torch.bfloat16).float()   # bf16-representable weights
    gpu = Qwen3ForCausalLM(copy.deepcopy(cfg)).eval()   # own config: the verifier rebinds its attention
    gpu.load_state_dict(cpu.state_dict())
    return cpu, gpu.to(torch.bfloat16).to(DEV)


@torch.no_grad()
def cpu_logits(model, seq):
    return model(input_ids=torch.tensor([seq]), use_cache=False).logits[0, -NEW:].numpy()


@torch.no_grad()
def cpu_prefix_kv(model, seq):
    """float32 CPU prefill K/V per layer -> bf16 [L, c, 8, 128]."""
    pkv = model(input_ids=torch.tensor([seq]), use_cache=True).past_key_values
    k = torch.stack([layer.keys[0].transpose(0, 1) for layer in pkv.layers])
    v = torch.stack([layer.values[0].transpose(0, 1) for layer in pkv.layers])
    return k.to(torch.bfloat16), v.to(torch.bfloat16)


def close(gpu, ref, what):
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    rel = np.linalg.norm(gpu - ref) / np.linalg.norm(ref)
    assert rel < 3e-2, (what, rel)
    return rel


def test_fused_hooks_two_rounds_match_cpu_model():
    from qwen3_dspark_amd.hf_hooks import FusedVerifier
    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV
    cpu, gpu = tiny_qwen3()
    rng = np.random.default_rng(5)
    prefixes = [rng.integers(0, 512, size=c).tolist() for c in (37, 150, 300)]
    store = PersistentTargetKV(layers=2, slots=3, context_capacity=512, max_query_tokens=3 * NEW, heads=8,
                               dim=128, device=DEV)
    handles = [store.add_request(f'r{i}') for i in range(3)]
    for h, p in zip(handles, prefixes):
        k, v = cpu_prefix_kv(cpu, p)
        store.load_prefix(h, k.to(DEV), v.to(DEV))
    bucket = Bucket((NEW,) * 3, (512 - NEW,) * 3, 'hf hooks')
    store.register_bucket(bucket)
    verifier = FusedVerifier(gpu, store)
    seqs = [list(p) for p in prefixes]
    for rnd, accepted in enumerate(([3, 0, 7], [1, 7, 2])):
        new = [rng.integers(0, 512, size=NEW).tolist() for _ in seqs]
        ids = torch.tensor([[t for n in new for t in n]], device=DEV)
        pos = torch.tensor([[len(s) + i for s in seqs for i in range(NEW)]], device=DEV)
        with verifier.transaction_for(handles, bucket) as tx:
            logits = verifier.forward(ids, pos).logits[0].float().cpu().numpy()
            store.commit(tx, dict(zip(handles, accepted)))
        for r, s in enumerate(seqs):
            rel = close(logits[r * NEW:(r + 1) * NEW], cpu_logits(cpu, s + new[r]), (rnd, r))
            print(f'round {rnd} request {r}: relative logit error {rel:.2e}', flush=True)
        seqs = [s + n[:a] for s, n, a in zip(seqs, new, accepted)]
        assert [store.length(h) for h in handles] == [len(s) for s in seqs]


def test_varlen_callback_matches_fused_path():
    """varlen_attention_forward over a PackedLayout with interleaved
    physical rows equals a direct kernel call on the gathered K/V bit for
    bit, and meets the attention gate against the oracle."""
    from qwen3_dspark_amd.hf_hooks import varlen_attention_forward
    from qwen3_dspark_amd.kernels import HipVarlenKernel
    from qwen3_dspark_amd.layout import PackedLayout
    gen = torch.Generator().manual_seed(3)
    contexts = [12, 40]
    n = sum(contexts)
    key = torch.randn(1, 8, n, 128, generator=gen).to(torch.bfloat16).to(DEV)
    value = torch.randn(1, 8, n, 128, generator=gen).to(torch.bfloat16).to(DEV)
    # physical order interleaves the two requests
    owner = [0] * contexts[0] + [1] * contexts[1]
    perm = np.random.default_rng(1).permutation(n)
    owner = [owner[i] for i in perm]
    kr, kp, seen = [], [], [0, 0]
    for o in owner:
        kr.append(o + 10)
        kp.append(seen[o])
        seen[o] += 1
    qr = [10] * 3 + [11] * 5
    qp = [contexts[0] - 3 + i for i in range(3)] + [contexts[1] - 5 + i for i in range(5)]
    t = lambda x: torch.tensor(x, dtype=torch.long, device=DEV)
    layout = PackedLayout.from_metadata(t(qr), t(qp), t(kr), t(kp))
    query = torch.randn(1, 16, 8, 128, generator=gen).to(torch.bfloat16).to(DEV)
    kernel = HipVarlenKernel(DEV)
    out, _ = varlen_attention_forward(None, query, key, value, None, scaling=128 ** -0.5,
                                      packed_layout=layout, packed_varlen_kernel=kernel)
    k, v = layout.gather_kv(key, value)
    direct = kernel(query[0].transpose(0, 1).contiguous(), k, v, layout, scale=128 ** -0.5)
    assert torch.equal(out[0], direct)
    # and against the oracle: gather by the reference's physical indices
    # (varlen_target.py:74-82), bottom-right causal attention per request
    # (varlen_target.py:98-112)
    from helpers import attention_gate, f64, segments
    from oracle import attention as oracle_attention
    idx = layout.gather_indices.cpu().numpy()
    kk, vv = f64(key[0].transpose(0, 1))[idx], f64(value[0].transpose(0, 1))[idx]
    cu_q, cu_k = layout.cu_query.tolist(), layout.cu_key.tolist()
    ref = oracle_attention.varlen_attention(f64(query[0].transpose(0, 1)), kk, vv, cu_q, cu_k, causal=True,
                                            scale=128 ** -0.5)
    attention_gate(f64(out[0]), ref, segments(cu_q))
    with pytest.raises(ValueError, match='metadata-only'):
        varlen_attention_forward(None, query, key, value, torch.ones(1), packed_layout=layout,
                                 packed_varlen_kernel=kernel)


def test_persistent_qwen_target_prefill_verify_commit_features():
    """The full-model adapter (persistent_qwen_target.py:100-472 API):
    prefill ragged prompts, verify 7 tokens per request, commit a prefix,
    verify again; logits via predict() and captured layer features match the
    CPU float32 model over each request's full sequence."""
    from qwen3_dspark_amd import backends
    from qwen3_dspark_amd.persistent_kv import Bucket
    from qwen3_dspark_amd.persistent_target import PersistentQwenTarget
    cpu, gpu = tiny_qwen3()
    rng = np.random.default_rng(11)
    prompts = [rng.integers(0, 512, size=n).tolist() for n in (20, 65, 9)]
    target = PersistentQwenTarget(gpu, layer_ids=(0, 1), native_backend=backends.CAPACITY_BACKEND, slots=3,
                                  context_capacity=256, max_query_tokens=128)
    names = ['a', 'b', 'c']
    for n in names:
        target.add_request(n)
    pre = Bucket(tuple(len(p) for p in prompts), (0, 0, 0), 'prefill')
    target.register_bucket(pre)
    t = lambda ids: torch.tensor([ids], device=DEV)
    target.prefill({n: t(p) for n, p in zip(names, prompts)}, bucket=pre)
    assert target.lengths == {n: len(p) for n, p in zip(names, prompts)}
    with pytest.raises(ValueError, match='newly admitted'):
        target.prefill({'a': t([1])}, bucket=pre)
    step = Bucket((NEW,) * 3, (256 - NEW,) * 3, 'verify')
    target.register_bucket(step)
    seqs = [list(p) for p in prompts]
    for accepted in ([7, 2, 0], [4, 4, 4]):
        new = [rng.integers(0, 512, size=NEW).tolist() for _ in seqs]
        feats = target.verify({n: t(x) for n, x in zip(names, new)}, bucket=step)
        logits = target.predict(feats)
        outs = {}
        hooks = [cpu.model.layers[i].register_forward_hook(
            lambda m, a, o, i=i: outs.__setitem__(i, o[0] if isinstance(o, tuple) else o)) for i in (0, 1)]
        try:
            with torch.no_grad():
                for r, (n, s) in enumerate(zip(names, seqs)):
                    ref = cpu(input_ids=torch.tensor([s + new[r]]), use_cache=False)
                    close(logits[n][0].float().cpu().numpy(), ref.logits[0, -NEW:].numpy(), (n, 'logits'))
                    f = feats.for_request(n)
                    assert f.start == len(s) and f.last.shape[1] == NEW
                    want = torch.cat([outs[0][0, -NEW:], outs[1][0, -NEW:]], dim=-1)
                    close(f.context[0].float().cpu().numpy(), want.numpy(), (n, 'features'))
        finally:
            for h in hooks:
                h.remove()
        target.commit(feats, dict(zip(names, accepted)))
        seqs = [s + x[:a] for s, x, a in zip(seqs, new, accepted)]
        assert target.lengths == {n: len(s) for n, s in zip(names, seqs)}
    k, v = target.request_kv('b')[0]
    assert k.shape == (1, 8, len(seqs[1]), 128)


def test_one_attention_launch_per_layer_in_the_trace():
    """The device trace of one verification forward through the fused hooks
    (the tracing check of scripts/probe_varlen.py:126-136, which counts one
    aten::_flash_attention_forward per native call and layer): per layer one
    fused attention chunk launch and one split-K merge, no separate staging
    or gather launch, and no torch attention or softmax kernel."""
    from torch.profiler import ProfilerActivity, profile

    from qwen3_dspark_amd.hf_hooks import FusedVerifier
    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV
    cpu, gpu = tiny_qwen3()
    rng = np.random.default_rng(9)
    store = PersistentTargetKV(layers=2, slots=2, context_capacity=512, max_query_tokens=2 * NEW, heads=8,
                               dim=128, device=DEV)
    handles = [store.add_request(f'r{i}') for i in range(2)]
    for h, c in zip(handles, (90, 200)):
        k, v = cpu_prefix_kv(cpu, rng.integers(0, 512, size=c).tolist())
        store.load_prefix(h, k.to(DEV), v.to(DEV))
    bucket = Bucket((NEW,) * 2, (512 - NEW,) * 2, 'trace')
    store.register_bucket(bucket)
    verifier = FusedVerifier(gpu, store)
    ids = torch.tensor([rng.integers(0, 512, size=2 * NEW).tolist()], device=DEV)
    pos = torch.tensor([[90 + i for i in range(NEW)] + [200 + i for i in range(NEW)]], device=DEV)
    for attempt in range(2):          # the first forward warms up the libraries outside the trace
        with verifier.transaction_for(handles, bucket) as tx:
            if attempt == 0:
                verifier.forward(ids, pos)
                store.abort(tx)
                continue
            with profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA]) as prof:
                verifier.forward(ids, pos)
                torch.cuda.synchronize()
            store.abort(tx)
    names = [e.name for e in prof.events() if e.device_type.name == 'CUDA']
    count = lambda key: sum(key in n for n in names)
    assert names, 'the profiler recorded no device activity'
    assert count('varlen_attn_kernel') == 2, names
    assert count('merge_kernel') == 2, names
    assert count('kv_stage_kernel') == 0 and count('kv_gather_kernel') == 0, names
    assert not any('softmax' in n.lower() or 'flash' in n.lower() or 'attention' in n.lower() for n in names), names
