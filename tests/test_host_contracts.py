"""Host-side contracts that need no GPU: dataclass validation, layout
construction against the oracle, and refusal of any CPU execution path."""
import numpy as np
import pytest
import torch

from oracle import semantics
from qwen3_dspark_amd.layout import PackedLayout
from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV, QueryFamily


def test_bucket_and_family_validation(golden):
    with pytest.raises(ValueError):
        Bucket((1,), (8,), '')
    with pytest.raises(ValueError):
        Bucket([1], [8], 'lists are not immutable')
    b = Bucket((2, 3), (12, 12), 'fixture')
    assert (b.key_capacity, b.maximum_key_length, b.maximum_query_length) == (29, 15, 3)
    assert b.accepts((2, 3), (3, 5)) and not b.accepts((2, 3), (13, 0)) and not b.accepts((3, 2), (0, 0))
    g = golden['family_bounds']
    tight = QueryFamily(*g['tight'], 'context bounds')
    for queries, contexts in g['rejects']:
        assert not tight.accepts(tuple(queries), tuple(contexts))
    for args in g['invalid_args']:
        with pytest.raises(ValueError):
            QueryFamily(*args, 'invalid')
    with pytest.raises(ValueError):
        QueryFamily(True, 6, 6, 8, 8, 'bool is not an int')


def test_layout_golden_and_invalid(golden):
    g = golden['layout_basic']
    L = PackedLayout.from_metadata(*(torch.tensor(g[k]) for k in ('query_requests', 'query_positions',
                                                                    'key_requests', 'key_positions')))
    assert list(L.query_lengths) == g['query_lengths'] and list(L.key_lengths) == g['key_lengths']
    assert L.cu_query.tolist() == g['cu_query'] and L.cu_key.tolist() == g['cu_key']
    assert L.cu_query.dtype == torch.int32 and L.cu_key.dtype == torch.int32
    assert L.gather_indices.tolist() == g['gather_indices'] and L.pair_domain == g['pair_domain']
    for case in golden['layout_invalid']['cases']:
        with pytest.raises(ValueError):
            PackedLayout.from_metadata(*(torch.tensor(x, dtype=torch.long) for x in case))


def _random_layout(rng, n_req, inactive):
    """Interleaved physical cache of active+inactive requests; queries are the
    terminal suffix of each active request."""
    markers = rng.permutation(1000)[:n_req + inactive]
    lengths = rng.integers(1, 30, size=n_req + inactive)
    pairs = []
    cursor = {m: 0 for m in markers}
    remaining = {m: int(n) for m, n in zip(markers, lengths)}
    while any(remaining.values()):
        m = rng.choice([m for m in markers if remaining[m]])
        pairs.append((int(m), cursor[m]))
        cursor[m] += 1
        remaining[m] -= 1
    active = list(rng.permutation(markers[:n_req]))
    qr, qp = [], []
    for m in active:
        n = int(lengths[list(markers).index(m)])
        q = int(rng.integers(1, n + 1))
        qr += [int(m)] * q
        qp += list(range(n - q, n))
    return qr, qp, [m for m, _ in pairs], [p for _, p in pairs]


def test_layout_matches_oracle_on_random_interleavings():
    rng = np.random.default_rng(3)
    for _ in range(40):
        qr, qp, kr, kp = _random_layout(rng, int(rng.integers(1, 6)), int(rng.integers(0, 3)))
        L = PackedLayout.from_metadata(*(torch.tensor(x, dtype=torch.long) for x in (qr, qp, kr, kp)))
        o = semantics.layout_from_metadata(qr, qp, kr, kp)
        assert L.request_markers == o['markers']
        assert L.query_lengths == o['query_lengths'] and L.key_lengths == o['key_lengths']
        assert L.cu_query.tolist() == o['cu_query'] and L.cu_key.tolist() == o['cu_key']
        assert L.gather_indices.tolist() == o['gather_indices']
        assert L.physical_key_tokens == o['physical_key_tokens']
        # Break one key position: product and oracle must agree on whether
        # (and with which message) the layout is rejected; inactive
        # requests' keys are not validated by either.
        if len(kp) > 1:
            bad = list(kp)
            bad[int(rng.integers(0, len(bad)))] += 1
            try:
                semantics.layout_from_metadata(qr, qp, kr, bad)
                expected = None
            except semantics.OracleValueError as e:
                expected = str(e)
            try:
                PackedLayout.from_metadata(*(torch.tensor(x, dtype=torch.long) for x in (qr, qp, kr, bad)))
                got = None
            except ValueError as e:
                got = str(e)
            assert got == expected


def test_no_cpu_execution_path():
    from qwen3_dspark_amd.draft import HipDraftAttention
    from qwen3_dspark_amd.kernels import HipCapacityKernel, HipDraftVarlenKernel, HipVarlenKernel
    for cls in (HipVarlenKernel, HipDraftVarlenKernel, HipCapacityKernel, HipDraftAttention):
        with pytest.raises(RuntimeError, match='gfx950'):
            cls('cpu')
    with pytest.raises(RuntimeError, match='gfx950'):
        PersistentTargetKV(layers=1, slots=1, context_capacity=4, max_query_tokens=1, heads=8, dim=128, device='cpu')
