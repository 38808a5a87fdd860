"""Device-built PackedLayout (dspark_layout_build) and gather_kv
(dspark_pool_gather) against the oracle restatement of
dspark_qwen/varlen_target.py:28-82: bit-exact lengths, cumulative lengths
and gather lists, the reference's error messages and their precedence."""
import numpy as np
import pytest
import torch

from oracle import semantics
from qwen3_dspark_amd.layout import MAX_LAYOUT_REQUESTS, PackedLayout

pytestmark = pytest.mark.gpu
DEV = torch.device('cuda:0')


def _t(x):
    return torch.tensor(x, dtype=torch.long, device=DEV)


def _oracle(qr, qp, kr, kp):
    try:
        return semantics.layout_from_metadata(qr, qp, kr, kp), None
    except semantics.OracleValueError as e:
        return None, str(e)


def _product(qr, qp, kr, kp):
    try:
        return PackedLayout.from_metadata(_t(qr), _t(qp), _t(kr), _t(kp)), None
    except ValueError as e:
        return None, str(e)


def _same(L, o):
    assert L.request_markers == tuple(o['markers'])
    assert L.query_lengths == tuple(o['query_lengths']) and L.key_lengths == tuple(o['key_lengths'])
    assert L.cu_query.dtype == torch.int32 and L.cu_key.dtype == torch.int32
    assert L.cu_query.tolist() == list(o['cu_query']) and L.cu_key.tolist() == list(o['cu_key'])
    assert L.gather_indices.dtype == torch.long and L.gather_indices.tolist() == list(o['gather_indices'])
    assert L.physical_key_tokens == o['physical_key_tokens']


def test_golden_vector_and_invalid_cases(golden):
    g = golden['layout_basic']
    L = PackedLayout.from_metadata(*(_t(g[k]) for k in ('query_requests', 'query_positions',
                                                         'key_requests', 'key_positions')))
    assert list(L.query_lengths) == g['query_lengths'] and list(L.key_lengths) == g['key_lengths']
    assert L.cu_query.tolist() == g['cu_query'] and L.cu_key.tolist() == g['cu_key']
    assert L.gather_indices.tolist() == g['gather_indices'] and L.pair_domain == g['pair_domain']
    for case in golden['layout_invalid']['cases']:
        _, expected = _oracle(*case)
        _, got = _product(*case)
        assert expected is not None and got == expected


def _random_layout(rng, n_req, inactive, max_len=30):
    """Interleaved physical cache of active+inactive requests; queries are the
    terminal suffix of each active request."""
    markers = rng.permutation(10 * (n_req + inactive) + 10)[:n_req + inactive] - 5
    lengths = rng.integers(1, max_len, size=n_req + inactive)
    owner = np.repeat(np.arange(n_req + inactive), lengths)
    rng.shuffle(owner)
    pos = np.zeros(n_req + inactive, dtype=np.int64)
    kr, kp = [], []
    for o in owner:
        kr.append(int(markers[o]))
        kp.append(int(pos[o]))
        pos[o] += 1
    active = rng.permutation(n_req)
    qr, qp = [], []
    for i in active:
        n = int(lengths[i])
        q = int(rng.integers(1, n + 1))
        qr += [int(markers[i])] * q
        qp += list(range(n - q, n))
    return qr, qp, kr, kp


def _mutations(rng, qr, qp, kr, kp):
    """Single-element corruptions covering every error class."""
    out = []
    i = int(rng.integers(0, len(kp)))
    out.append((qr, qp, kr, kp[:i] + [kp[i] + 1] + kp[i + 1:]))            # position gap / duplicate
    out.append((qr, qp, kr, kp[:i] + [-1] + kp[i + 1:]))                   # negative position
    j = int(rng.integers(0, len(kp)))
    sw = list(kp)
    sw[i], sw[j] = sw[j], sw[i]
    out.append((qr, qp, kr, sw))                                           # physical order broken
    k = int(rng.integers(0, len(qp)))
    out.append((qr, qp[:k] + [qp[k] - 1] + qp[k + 1:], kr, kp))            # not the terminal suffix
    if len(set(qr)) > 1:
        out.append((qr + [qr[0]], qp + [qp[0]], kr, kp))                   # a request split in two runs
    out.append((qr, qp, [m for m in kr if m != qr[-1]], [p for m, p in zip(kr, kp) if m != qr[-1]]))  # k < q
    return out


def test_random_interleavings_and_mutations_match_oracle():
    rng = np.random.default_rng(3)
    for trial in range(60):
        case = _random_layout(rng, int(rng.integers(1, 7)), int(rng.integers(0, 3)))
        o, _ = _oracle(*case)
        L, err = _product(*case)
        assert err is None, (trial, err)
        _same(L, o)
        for bad in _mutations(rng, *case):
            o_bad, expected = _oracle(*bad)
            L_bad, got = _product(*bad)
            assert got == expected, (trial, got, expected)
            if expected is None:
                _same(L_bad, o_bad)


def test_large_layout_and_edges():
    rng = np.random.default_rng(11)
    # 64 requests with long interleaved histories plus inactive keys.
    case = _random_layout(rng, 64, 8, max_len=3000)
    o, _ = _oracle(*case)
    L, err = _product(*case)
    assert err is None
    _same(L, o)
    # No keys at all: every request's prefix is incomplete.
    _, got = _product([1, 1], [0, 1], [], [])
    assert got == 'Active keys must be a complete request-local prefix'
    # Zero-length suffix edge: q == k (queries cover the whole prefix).
    L, err = _product([7, 7, 7], [0, 1, 2], [7, 7, 7], [0, 1, 2])
    assert err is None and L.key_lengths == (3,) and L.gather_indices.tolist() == [0, 1, 2]
    # More requests than the device build supports.
    n = MAX_LAYOUT_REQUESTS + 1
    with pytest.raises(ValueError, match='At most'):
        PackedLayout.from_metadata(_t(list(range(n))), _t([0] * n), _t(list(range(n))), _t([0] * n))


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_gather_kv_bit_exact(dtype):
    rng = np.random.default_rng(5)
    qr, qp, kr, kp = _random_layout(rng, 5, 2, max_len=200)
    L = PackedLayout.from_metadata(_t(qr), _t(qp), _t(kr), _t(kp))
    n = len(kr)
    g = torch.Generator().manual_seed(9)
    key = torch.randn(1, 8, n, 128, generator=g).to(dtype)
    value = torch.randn(1, 8, n, 128, generator=g).to(dtype)
    k, v = L.gather_kv(key.to(DEV), value.to(DEV))
    idx = np.array(L.gather_indices.tolist())
    for got, src in ((k, key), (v, value)):
        want = src[0].numpy()[:, idx].transpose(1, 0, 2) if dtype == torch.float32 else \
            src[0].view(torch.int16).numpy()[:, idx].transpose(1, 0, 2)
        have = got.cpu().numpy() if dtype == torch.float32 else got.cpu().view(torch.int16).numpy()
        assert have.shape == (len(idx), 8, 128) and np.array_equal(have, want)
    with pytest.raises(ValueError, match='matching'):
        L.gather_kv(key.to(DEV)[:, :, :-1], value.to(DEV)[:, :, :-1])
