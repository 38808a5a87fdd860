"""VarlenPackedTarget on the GPU: the reference's append-order adapter tests
(tests/test_varlen_target.py:33-119) on a 2-layer Qwen3-shaped model (16
query heads, 8 KV heads, head dim 128, random init, bf16).  Logits and
captured layer features of every append must match the same weights run in
float32 on the CPU over each request's full token sequence; the work
counters must equal the reference's fixture values."""
import pytest
import torch

from test_gpu_hf_hooks import close, tiny_qwen3

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda:0')


def say(*a):
    print(*a, flush=True)


class Mirror:
    """The target plus each request's committed token sequence."""

    def __init__(self, cpu, target):
        self.cpu, self.target, self.seqs = cpu, target, {}

    def add(self, name):
        self.target.add_request(name)
        self.seqs[name] = []

    def crop(self, name, n):
        self.target.crop(name, n)
        self.seqs[name] = self.seqs[name][:n]

    @torch.no_grad()
    def append(self, chunks):
        say(f'[varlen target] append {chunks}')
        feats = self.target.append({r: torch.tensor([ids], device=DEV) for r, ids in chunks.items()})
        logits = self.target.predict(feats)
        outs = {}
        hooks = [self.cpu.model.layers[i].register_forward_hook(
            lambda m, a, o, i=i: outs.__setitem__(i, o[0] if isinstance(o, tuple) else o)) for i in (0, 1)]
        try:
            for r, ids in chunks.items():
                full = self.seqs[r] + list(ids)
                ref = self.cpu(input_ids=torch.tensor([full]), use_cache=False)
                n = len(ids)
                close(logits[r][0].float().cpu().numpy(), ref.logits[0, -n:].numpy(), (r, 'logits'))
                f = feats.for_request(r)
                assert f.start == len(self.seqs[r]) and f.last.shape[1] == n
                want = torch.cat([outs[0][0, -n:], outs[1][0, -n:]], dim=-1)
                close(f.context[0].float().cpu().numpy(), want.numpy(), (r, 'features'))
                self.seqs[r] = full
        finally:
            for h in hooks:
                h.remove()
        assert self.target.lengths == {r: len(s) for r, s in self.seqs.items()}
        w = feats.work
        assert w['physical_query_tokens'] == w['logical_query_tokens'] == sum(len(x) for x in chunks.values())
        assert w['mask_bytes'] == 0 and w['mask_shape'] is None
        assert w['native_varlen_calls_per_layer'] == 1 and w['attention_adapter_calls_per_layer'] == 1
        assert w['attention_backend'] == 'mi355x_hip_varlen_causal_v1'
        active = sum(len(self.seqs[r]) for r in chunks)
        assert w['active_kv_gather_tokens'] == active
        assert w['kv_gather_payload_bytes_per_layer'] == active * 2 * 8 * 128 * 2
        return feats


def test_varlen_packed_target_mixed_queries_inactive_kv_and_lifecycle():
    from qwen3_dspark_amd.hf_hooks import VarlenPackedTarget
    cpu, gpu = tiny_qwen3()
    m = Mirror(cpu, VarlenPackedTarget(gpu, layer_ids=(0, 1)))
    for name in ('a', 'b', 'idle'):
        m.add(name)
    m.append({'a': [1, 2, 3], 'b': [4], 'idle': [5, 6]})
    batch = m.append({'b': [7, 8, 9], 'a': [10]})
    # reference fixture (tests/test_varlen_target.py:84-87)
    assert batch.work['inactive_kv_tokens_excluded'] == 2
    assert batch.work['active_kv_gather_tokens'] == 8
    assert batch.work['varlen_pair_domain_per_head_layer'] == 16
    m.crop('a', 3)
    m.crop('b', 2)
    m.target.remove_request('idle')
    del m.seqs['idle']
    m.add('idle')
    m.append({'idle': [20], 'a': [21], 'b': [22, 23]})
    m.crop('a', 0)
    m.append({'a': [31, 32]})
    # committed KV of every request equals the CPU model's prefill KV of its sequence
    for r, seq in m.seqs.items():
        if not seq:
            continue
        with torch.no_grad():
            pkv = cpu(input_ids=torch.tensor([seq]), use_cache=True).past_key_values
        for layer, (k, v) in enumerate(m.target.request_kv(r)):
            close(k[0].float().cpu().numpy(), pkv.layers[layer].keys[0].numpy(), (r, layer, 'keys'))
            close(v[0].float().cpu().numpy(), pkv.layers[layer].values[0].numpy(), (r, layer, 'values'))


def test_varlen_packed_target_other_requests_rows_never_attended():
    """tests/test_varlen_target.py:96-105: poisoning another request's rows
    changes nothing for the active request, bit for bit."""
    from qwen3_dspark_amd.hf_hooks import VarlenPackedTarget
    cpu, gpu = tiny_qwen3()
    m = Mirror(cpu, VarlenPackedTarget(gpu, layer_ids=(0, 1)))
    for name in ('a', 'b'):
        m.add(name)
    m.append({'a': [1, 2], 'b': [3, 4]})
    clean = m.target.append({'a': torch.tensor([[5]], device=DEV)})
    m.target.crop('a', 2)
    selected = m.target.kv.key_requests == m.target.kv.marker('b')
    for k, v in m.target.kv.kv:
        k[:, :, selected] = 1000
        v[:, :, selected] = -1000
    poisoned = m.target.append({'a': torch.tensor([[5]], device=DEV)})
    assert torch.equal(clean.last, poisoned.last)
    assert poisoned.work['inactive_kv_tokens_excluded'] == 2


def test_varlen_packed_target_failed_kernel_resets_and_inputs_fail_first():
    """tests/test_varlen_target.py:107-119 and packed_target.py:149-158:
    invalid inputs fail before any mutation; a failing kernel resets every
    request (the layers may have grown unevenly)."""
    from qwen3_dspark_amd.hf_hooks import VarlenPackedTarget
    _, gpu = tiny_qwen3()
    target = VarlenPackedTarget(gpu)
    with pytest.raises(ValueError, match='Unknown explicit native varlen backend'):
        VarlenPackedTarget(gpu, native_backend='rocm_aten_no_window_pinned_v1')
    target.add_request('a')
    target.append({'a': torch.tensor([[1, 2]], device=DEV)})
    for bad in ({}, {'zz': torch.tensor([[1]], device=DEV)}, {'a': torch.tensor([[1]])},
                {'a': torch.tensor([[512]], device=DEV)}, {'a': torch.tensor([[1.0]], device=DEV)}):
        with pytest.raises(ValueError):
            target.append(bad)
    assert target.lengths == {'a': 2}

    def fail(*args, **kwargs):
        raise RuntimeError('unsupported kernel fixture')
    target._varlen_kernel = fail
    with pytest.raises(RuntimeError, match='unsupported kernel fixture'):
        target.append({'a': torch.tensor([[3]], device=DEV)})
    assert target.lengths == {}
    assert all(k.shape[2] == 0 for k, _ in target.kv.kv)
