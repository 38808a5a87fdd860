"""Host-side contracts that need no GPU: dataclass validation, argument
checks, and refusal of any CPU execution path."""
import pytest
import torch

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


def test_layout_argument_checks_then_no_cpu_path(golden):
    """Malformed arguments raise the reference's ValueError; well-formed
    metadata on the CPU is refused (the layout is built on the GPU only)."""
    g = golden['layout_basic']
    args = [torch.tensor(g[k]) for k in ('query_requests', 'query_positions', 'key_requests', 'key_positions')]
    with pytest.raises(ValueError, match='flat long'):
        PackedLayout.from_metadata(args[0].int(), *args[1:])
    with pytest.raises(ValueError, match='Nonempty'):
        PackedLayout.from_metadata(args[0][:0], args[1][:0], *args[2:])
    with pytest.raises(ValueError, match='matching'):
        PackedLayout.from_metadata(args[0], args[1], args[2], args[3][:-1])
    with pytest.raises(RuntimeError, match='gfx950'):
        PackedLayout.from_metadata(*args)


def test_no_cpu_execution_path():
    from qwen3_dspark_amd.draft import HipDraftAttention
    from qwen3_dspark_amd.kernels import HipCapacityKernel, HipDraftVarlenKernel, HipVarlenKernel
    for cls in (HipVarlenKernel, HipDraftVarlenKernel, HipCapacityKernel, HipDraftAttention):
        with pytest.raises(RuntimeError, match='gfx950'):
            cls('cpu')
    with pytest.raises(RuntimeError, match='gfx950'):
        PersistentTargetKV(layers=1, slots=1, context_capacity=4, max_query_tokens=1, heads=8, dim=128, device='cpu')
