"""Integer / index semantics of the hot path, restated for the CPU oracle.

Test infrastructure only (see oracle/__init__.py).  Plain Python loops over
small inputs; numpy for arrays.
"""
import numpy as np


class OracleValueError(ValueError):
    """Raised where the reference raises ValueError."""


def layout_from_metadata(query_requests, query_positions, key_requests, key_positions):
    """dspark_qwen/varlen_target.py:28-60 (PackedLayout.from_metadata).

    Returns dict(markers, query_lengths, key_lengths, cu_query, cu_key,
    gather_indices, physical_key_tokens) or raises OracleValueError with the
    reference's message.
    """
    qr = [int(x) for x in query_requests]
    qp = [int(x) for x in query_positions]
    kr = [int(x) for x in key_requests]
    kp = [int(x) for x in key_positions]
    if not qr or len(qr) != len(qp) or len(kr) != len(kp):
        raise OracleValueError('Nonempty queries and matching marker/position lengths required')
    markers, counts = [], []
    for m in qr:
        if markers and markers[-1] == m:
            counts[-1] += 1
        else:
            markers.append(m)
            counts.append(1)
    if len(set(markers)) != len(markers):
        raise OracleValueError('Each request query must form one contiguous chunk')
    gathers, k_lengths = [], []
    offset = 0
    for m, count in zip(markers, counts):
        idx = [i for i, x in enumerate(kr) if x == m]
        length = len(idx)
        if length < count or [kp[i] for i in idx] != list(range(length)):
            raise OracleValueError('Active keys must be a complete request-local prefix')
        if qp[offset:offset + count] != list(range(length - count, length)):
            raise OracleValueError('Queries must be the terminal suffix of their own key prefix')
        gathers.extend(idx)
        k_lengths.append(length)
        offset += count

    def cumulative(lengths):
        ends = [0]
        for n in lengths:
            ends.append(ends[-1] + n)
        if ends[-1] >= 2 ** 31:
            raise OracleValueError('Varlen cumulative lengths exceed int32')
        return ends
    return dict(markers=tuple(markers), query_lengths=tuple(counts), key_lengths=tuple(k_lengths),
                cu_query=cumulative(counts), cu_key=cumulative(k_lengths),
                gather_indices=gathers, physical_key_tokens=len(kr),
                pair_domain=sum(q * k for q, k in zip(counts, k_lengths)))


def txn_metadata(slots, contexts, queries, context_capacity, key_capacity):
    """dspark_qwen/persistent_target_kv.py:392-411 (PersistentTargetKV.begin lists)."""
    old, new, choose, positions, cq, ck = [], [], [], [], [0], [0]
    qo = 0
    for i, c, q in zip(slots, contexts, queries):
        old.extend(i * context_capacity + j for j in range(c))
        old.extend([0] * q)
        new.extend([0] * c)
        new.extend(range(qo, qo + q))
        choose.extend([False] * c + [True] * q)
        positions.extend(range(c, c + q))
        qo += q
        cq.append(qo)
        ck.append(ck[-1] + c + q)
    logical = len(old)
    tail = key_capacity - logical
    if tail < 0:
        raise OracleValueError('Actual context exceeds declared bucket applicability')
    old.extend([0] * tail)
    new.extend([0] * tail)
    choose.extend([False] * tail)
    valid = [True] * logical + [False] * tail
    return dict(committed_indices=np.array(old, np.int64), scratch_indices=np.array(new, np.int64),
                from_scratch=np.array(choose, bool), valid=np.array(valid, bool),
                positions=np.array(positions, np.int64), cu_query=np.array(cq, np.int32),
                cu_key=np.array(ck, np.int32))


def materialize(resident_layer, scratch_layer, meta):
    """dspark_qwen/persistent_target_kv.py:452-459 for one tensor (K or V).

    resident_layer [slots, cap, H, D], scratch_layer [max_q, H, D] (any dtype
    numpy array, compared bitwise by the caller).
    """
    flat = resident_layer.reshape(-1, *resident_layer.shape[2:])
    old = flat[meta['committed_indices']]
    new = scratch_layer[meta['scratch_indices']]
    out = np.where(meta['from_scratch'][:, None, None], new, old)
    out = np.where(meta['valid'][:, None, None], out, np.zeros_like(out))
    return out


def commit(resident, scratch, slots, contexts, queries, counts, context_capacity):
    """dspark_qwen/persistent_target_kv.py:470-485 on numpy arrays.

    resident [L, slots, cap, H, D] and scratch [L, max_q, H, D]; returns the
    new resident array and new per-request lengths.  Validation first, as in
    the reference (no write on any invalid count).
    """
    for c, q, n in zip(contexts, queries, counts):
        if type(n) is not int or not 0 <= n <= q or c + n > context_capacity:
            raise OracleValueError('Commit must be a valid verified prefix')
    out = resident.copy()
    qo = 0
    for s, c, q, n in zip(slots, contexts, queries, counts):
        out[:, s, c:c + n] = scratch[:, qo:qo + n]
        qo += q
    return out, [c + n for c, n in zip(contexts, counts)]


def work_counters(contexts, queries, key_capacity, resident_total, **_):
    """The integer counters of dspark_qwen/persistent_target_kv.py:511-523."""
    q = sum(queries)
    actual_k = sum(contexts) + q
    return dict(logical_query_tokens=q, physical_query_tokens=q, logical_active_key_tokens=actual_k,
                physical_key_capacity=key_capacity, padded_key_capacity=key_capacity - actual_k,
                inactive_resident_key_tokens=resident_total - sum(contexts),
                gather_rows_per_kv_per_layer=2 * key_capacity,
                staging_output_rows_per_layer=key_capacity,
                allowed_causal_pairs=sum(c * n + n * (n + 1) // 2 for c, n in zip(contexts, queries)))


def block_mask(anchors, block_size, context_length):
    """dspark_qwen/model.py:12-19: True = visible.  Rows are n*block queries,
    columns context_length context keys then n*block block keys."""
    anchors = [int(a) for a in anchors]
    n = len(anchors)
    rows = n * block_size
    mask = np.zeros((rows, context_length + rows), bool)
    for r in range(rows):
        b = r // block_size
        for j in range(context_length):
            mask[r, j] = j < anchors[b]
        for j in range(rows):
            mask[r, context_length + j] = (j // block_size) == b
    return mask


def dflash_sdpa_mask(anchors, keep, ctx_len, block_size, causal=False):
    """references/nemo-2d365eda/dflash_mask.py:103-153 (single sample, no
    document ids, no sliding window): True = attended."""
    n = len(anchors)
    rows = n * block_size
    out = np.zeros((rows, ctx_len + rows), bool)
    for qi in range(rows):
        qb, qo = divmod(qi, block_size)
        for kv in range(ctx_len + rows):
            if kv < ctx_len:
                vis = kv < anchors[qb] and bool(keep[qb])
            else:
                kb, ko = divmod(kv - ctx_len, block_size)
                vis = kb == qb and (not causal or ko <= qo)
            out[qi, kv] = vis
    return out
