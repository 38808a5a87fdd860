"""AppendOrderKV: the append-order cache of PackedTarget
(dspark_qwen/packed_target.py:30-122).  A numpy simulation of the
reference's cat / keep-mask gather follows random append, crop and remove
sequences; markers, positions and every layer's K/V must match it bit for
bit after each step, and layouts over the cache must equal the oracle's."""
import numpy as np
import pytest
import torch

from helpers import SEED, randn_bf16
from oracle import semantics

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda:0')
LAYERS = 3


def u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


def test_random_sequences_match_reference_semantics():
    from qwen3_dspark_amd.packed_kv import AppendOrderKV
    gen = torch.Generator().manual_seed(SEED)
    rng = np.random.default_rng(21)
    cache = AppendOrderKV(layers=LAYERS, device=DEV)
    # mirror: markers, positions, per layer K/V rows [H, N, D] as int16 bits
    m_kr = np.zeros(0, np.int64)
    m_kp = np.zeros(0, np.int64)
    m_k = [np.zeros((8, 0, 128), np.int16) for _ in range(LAYERS)]
    m_v = [np.zeros((8, 0, 128), np.int16) for _ in range(LAYERS)]
    lengths, names = {}, iter(f'req{i}' for i in range(1000))
    for step in range(45):
        op = rng.choice(['add', 'append', 'append', 'append', 'crop', 'remove'])
        if op == 'add' and len(lengths) < 5:
            r = next(names)
            cache.add_request(r)
            lengths[r] = 0
        elif op == 'append' and lengths:
            chunks = {r: int(rng.integers(1, 40)) for r in lengths if rng.random() < 0.7} or \
                {next(iter(lengths)): 3}
            n = sum(chunks.values())
            proj = [(randn_bf16(gen, 1, 8, n, 128), randn_bf16(gen, 1, 8, n, 128)) for _ in range(LAYERS)]
            cache.append(chunks, [(k.to(DEV), v.to(DEV)) for k, v in proj])
            for r, c in chunks.items():
                m_kr = np.concatenate([m_kr, np.full(c, cache.marker(r))])
                m_kp = np.concatenate([m_kp, np.arange(lengths[r], lengths[r] + c)])
                lengths[r] += c
            for l, (k, v) in enumerate(proj):
                m_k[l] = np.concatenate([m_k[l], u16(k[0])], axis=1)
                m_v[l] = np.concatenate([m_v[l], u16(v[0])], axis=1)
        elif op in ('crop', 'remove') and lengths:
            r = list(lengths)[int(rng.integers(0, len(lengths)))]
            n = 0 if op == 'remove' else int(rng.integers(0, lengths[r] + 1))
            keep = (m_kr != cache.marker(r)) | (m_kp < n)
            if op == 'remove':
                cache.remove_request(r)
                del lengths[r]
            else:
                cache.crop(r, n)
                lengths[r] = n
            m_kr, m_kp = m_kr[keep], m_kp[keep]
            m_k = [x[:, keep] for x in m_k]
            m_v = [x[:, keep] for x in m_v]
        assert cache.lengths == lengths
        assert np.array_equal(cache.key_requests.cpu().numpy(), m_kr)
        assert np.array_equal(cache.key_positions.cpu().numpy(), m_kp)
        for l, (k, v) in enumerate(cache.kv):
            assert np.array_equal(u16(k[0]), m_k[l]) and np.array_equal(u16(v[0]), m_v[l])
        cache.validate_cache(deep=True)
        for r in lengths:
            rows = np.nonzero(m_kr == cache.marker(r))[0]
            for l, (k, v) in enumerate(cache.request_kv(r)):
                assert np.array_equal(u16(k[0]), m_k[l][:, rows]) and np.array_equal(u16(v[0]), m_v[l][:, rows])
        # layout of one forward: the last q rows of every nonempty request
        active = [r for r in lengths if lengths[r]]
        if active:
            qr, qp = [], []
            for r in active:
                q = int(rng.integers(1, lengths[r] + 1))
                qr += [cache.marker(r)] * q
                qp += list(range(lengths[r] - q, lengths[r]))
            L = cache.layout(torch.tensor(qr, device=DEV), torch.tensor(qp, device=DEV))
            o = semantics.layout_from_metadata(qr, qp, m_kr.tolist(), m_kp.tolist())
            assert L.cu_key.tolist() == list(o['cu_key']) and L.gather_indices.tolist() == list(o['gather_indices'])


def test_errors_and_noop_crop():
    from qwen3_dspark_amd.packed_kv import AppendOrderKV
    cache = AppendOrderKV(layers=1, device=DEV)
    cache.add_request('a')
    with pytest.raises(ValueError, match='new nonempty'):
        cache.add_request('a')
    with pytest.raises(ValueError, match='Unknown'):
        cache.crop('b', 0)
    k = torch.zeros(1, 8, 4, 128, dtype=torch.bfloat16, device=DEV)
    cache.append({'a': 4}, [(k, k)])
    with pytest.raises(ValueError, match='Crop length'):
        cache.crop('a', 5)
    before = cache.kv[0][0]
    cache.crop('a', 4)                      # no-op keeps the same tensors
    assert cache.kv[0][0] is before
    with pytest.raises(ValueError, match='contiguous'):
        cache.append({'a': 2}, [(k, k)])
    cache.remove_request('a')
    assert cache.rows == 0 and cache.lengths == {}
