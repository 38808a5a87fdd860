"""Write tests/golden/reference_vectors.json.

Every vector below is a literal input/expected-output pair asserted by the
reference's own tests or probe protocol (cited per entry); entries marked
"derived" reconstruct the inputs a reference test builds internally and keep
only the values that test asserts.  No reference code is imported or run.

    python tests/golden/make_golden.py
"""
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))

VECTORS = {
    'layout_basic': {
        'source': 'tests/test_varlen_target.py:65-80',
        'query_requests': [2, 2, 1], 'query_positions': [2, 3, 2],
        'key_requests': [1, 1, 2, 2, 3, 3, 1, 2, 2], 'key_positions': [0, 1, 0, 1, 0, 1, 2, 2, 3],
        'query_lengths': [2, 1], 'key_lengths': [4, 3], 'cu_query': [0, 2, 3], 'cu_key': [0, 4, 7],
        'gather_indices': [2, 3, 7, 8, 0, 1, 6], 'pair_domain': 11,
        # zero Q, scale 1, K=V=physical index, bottom-right causal
        'uniform_causal_output': [4.0, 5.0, 7.0 / 3.0],
    },
    'layout_invalid': {
        'source': 'tests/test_varlen_target.py:121-125',
        'cases': [
            [[1, 2, 1], [0, 0, 1], [1, 1, 2], [0, 1, 0]],
            [[1], [0], [1, 1], [0, 1]],
            [[1], [1], [1, 1], [0, 2]],
            [[], [], [], []],
        ],
    },
    'noncausal_uniform': {
        'source': 'tests/test_packed_draft.py:109-112',
        'query_requests': [0, 0, 0], 'query_positions': [2, 3, 4],
        'key_requests': [0, 0, 0, 0, 0], 'key_positions': [0, 1, 2, 3, 4],
        # zero Q, V[j] = j for every head/dim, scale 8**-0.5: every output is 2.0
        'expected': 2.0,
    },
    'draft_backbone_layout': {
        'source': 'tests/test_packed_draft.py:29-33,57-67 (derived inputs; asserted values only)',
        'query_requests': [1, 1, 1, 0, 0, 0], 'query_positions': [2, 3, 4, 4, 5, 6],
        'key_requests': [0, 0, 0, 0, 1, 1, 2, 1, 1, 1, 0, 0, 0],
        'key_positions': [0, 1, 2, 3, 0, 1, 0, 2, 3, 4, 4, 5, 6],
        'query_rows': 6, 'gathered_key_rows': 12, 'pair_domain': 36, 'context_lengths': [2, 4],
    },
    'txn_growing_context': {
        'source': 'tests/test_persistent_target_kv.py:37-64',
        'pool': {'layers': 2, 'slots': 3, 'context_capacity': 24, 'max_query_tokens': 8, 'heads': 2, 'dim': 4},
        'prefixes': [['A', 3, 100], ['B', 5, 500], ['idle', 9, 900]],
        'bucket': [[2, 3], [12, 12]],
        'active': ['A', 'B'],
        'cu_query': [0, 2, 5], 'cu_key': [0, 5, 13], 'positions': [3, 4, 5, 6, 7],
        'inactive_resident_key_tokens': 9, 'physical_key_capacity': 29, 'padded_key_capacity': 16,
        'commit': {'A': 1, 'B': 2},
        'second_cu_key': [0, 6, 16], 'second_positions': [4, 5, 7, 8, 9],
    },
    'txn_slot_reuse': {
        'source': 'tests/test_persistent_target_kv.py:66-81',
        'prefix': 7, 'bucket': [[1], [10]], 'cu_key': [0, 1], 'positions': [0], 'commit': 1,
    },
    'txn_invalid_commit': {
        'source': 'tests/test_persistent_target_kv.py:83-98',
        'prefix': 2, 'bucket': [[2], [4]], 'invalid_counts': [3, True], 'valid_noop': 0,
    },
    'txn_retry_metadata': {
        'source': 'tests/test_persistent_target_kv.py:100-116',
        'prefix': 3, 'bucket': [[2], [8]], 'cu_query': [0, 2], 'cu_key': [0, 5], 'positions': [3, 4],
    },
    'txn_reordered_subset': {
        'source': 'tests/test_persistent_target_kv.py:118-131',
        'prefixes': [['A', 8], ['B', 4]], 'small': [[1], [7]], 'pair': [[2, 1], [8, 8]],
        'active': ['B', 'A'], 'cu_query': [0, 2, 3], 'cu_key': [0, 6, 15], 'positions': [4, 5, 8],
        'inactive_with_B_small': 8,
    },
    'family_bounds': {
        'source': 'tests/test_query_family.py:65-69',
        'tight': [2, 6, 6, 7, 6], 'rejects': [[[3, 3], [2, 0]], [[5, 1], [2, 0]]],
        'invalid_args': [[2, 1, 1, 8, 8], [2, 6, 2, 8, 8], [2, 6, 6, 5, 8], [2, 6, 6, 8, 5]],
    },
    'block_mask_truth_table': {
        'source': 'tests/test_core.py:39-42',
        'anchors': [2, 4], 'block_size': 3, 'context_length': 7,
        'row0_visible': [0, 1, 7, 8, 9], 'row4_visible': [0, 1, 2, 3, 10, 11, 12],
    },
    'block_mask_equals_dflash': {
        'source': 'tests/test_core.py:47-55',
        'anchors': [0, 2, 6], 'block_size': 3, 'context_length': 7,
    },
    'probe_varlen_protocol': {
        'source': 'scripts/probe_varlen.py:20-41,179-216',
        'seed': 20261009, 'atol': 0.02, 'rtol': 0.02, 'max_rms_error': 0.005,
        'cases': [
            {'name': 'interleaved_cached_tail', 'markers': [1, 2], 'q': [1, 8], 'k': [17, 29], 'inactive_k': 13},
            {'name': 'crop_exit_readd', 'markers': [1, 2, 4], 'q': [3, 2, 1], 'k': [11, 5, 1], 'inactive_k': 0},
            {'name': 'crop_zero_then_append', 'markers': [1], 'q': [2], 'k': [2], 'inactive_k': 6},
        ],
        # zero Q, V = local position / 32: bottom-right mean (k-q+i)/64
        'ramp_divisor': 64,
    },
    'capacity_protocol': {
        'source': 'scripts/probe_native_capacity_graph.py:23-35',
        'query_lengths': [1, 4], 'context_ceilings': [144, 144],
        'contexts': [[128, 128], [129, 131], [130, 135]],
        'committed_query_rows': [[1, 3], [1, 4], [0, 0]],
        'physical_key_capacity': 293, 'maximum_query_length': 4, 'maximum_key_length': 148,
        'tail_finite_keys': 100.0, 'tail_finite_values': -100.0,
    },
}


def main():
    path = os.path.join(HERE, 'reference_vectors.json')
    with open(path, 'w') as f:
        json.dump(VECTORS, f, indent=1, sort_keys=True)
        f.write('\n')
    print(path)


if __name__ == '__main__':
    main()
