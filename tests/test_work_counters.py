"""Work counters of the draft attention path (packed_draft.py:245-249), on
the CPU: the reference's own backbone numbers, and the dense block mask of
the oracle (model.py:12-19) counted directly for multi-block requests."""
import numpy as np

from oracle import semantics
from qwen3_dspark_amd.draft import draft_work_counters


def test_reference_backbone_counters():
    """tests/test_packed_draft.py:57-67: block size 3, requests with 2 and 4
    context rows, one block each at anchor = context length."""
    w = draft_work_counters([2, 4], [[2], [4]], block_size=3, layers=2)
    assert (w['query_rows'], w['gathered_key_rows'], w['attention_pair_domain']) == (6, 12, 36)
    assert w['attention_calls'] == 2 and w['requests'] == 2
    # the copies the reference counts do not exist on the fused path
    for key in ('context_block_concatenation_kv_elements', 'gathered_kv_elements', 'attention_cast_elements'):
        assert w[key] == 0


def test_multi_block_counters_equal_the_dense_block_mask():
    rng = np.random.default_rng(7)
    contexts, anchors = [], []
    for _ in range(6):
        c = int(rng.integers(0, 40))
        contexts.append(c)
        anchors.append([int(a) for a in rng.integers(0, c + 1, size=int(rng.integers(1, 9)))])
    w = draft_work_counters(contexts, anchors, physical_context_rows=1000, key_element_bytes=4)
    pairs = rows = keys = 0
    for c, a in zip(contexts, anchors):
        mask = semantics.block_mask(a, 7, c)
        pairs += int(mask.sum())
        rows += mask.shape[0]
        keys += int(mask.any(axis=0).sum())   # key columns some row of the request sees
    assert w['attention_pair_domain'] == pairs
    assert w['query_rows'] == rows
    assert w['gathered_key_rows'] == keys
    assert w['kv_bytes_read_per_layer'] == keys * 8 * 128 * (4 + 2)
    assert w['physical_context_rows'] == 1000 and w['draft_blocks'] == sum(len(a) for a in anchors)
