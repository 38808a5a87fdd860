"""Split-K work lists.

Every request's keys are cut into chunks of `chunk` rows (at least one chunk
per request) and each (request, chunk) pair is one work item per KV head.
Items are dispatched longest first so that the short tail chunks of ragged
requests fill the end of the grid (greedy longest-processing-time order);
the partial-result slot of an item stays its request-major index, so the
dispatch order does not affect results.

A work list is int32: one record of WORK_INTS per item in dispatch order,
then one record of REQ_INTS per request (for the split-K merge).  The
records carry everything a workgroup needs to start streaming keys, so a
kernel reads one record instead of walking the cumulative arrays.

  varlen / verify item: request, chunk, chunk base, query start, query
                        length, key length, key start (varlen) or resident
                        slot (verify), chunk count
  draft item:           request, chunk, chunk base, context length, first
                        block, block count, largest anchor, chunk count
  request:              chunk base, chunk count, first query row (varlen) or
                        first block (draft), query length or block count
"""
from ._device import upload

DEFAULT_CHUNK = 1024          # verification / varlen: one query tile per item
# Draft items carry up to 8 blocks of FP32 partials each, so they are cut
# more coarsely: only contexts longer than this are split.
DRAFT_CHUNK = 4096
WORK_INTS = 8
REQ_INTS = 4


def n_chunks(n, chunk):
    return max(1, -(-int(n) // chunk))


def chunk_items(lengths, chunk):
    """[(request, chunk_index)] for all items, longest chunk first (stable)."""
    items = []
    for r, n in enumerate(lengths):
        n = int(n)
        for c in range(n_chunks(n, chunk)):
            items.append((min(chunk, n - c * chunk) if n > 0 else 0, r, c))
    items.sort(key=lambda x: -x[0])
    return [(r, c) for _, r, c in items]


def chunk_bound(n_req, rows_bound, chunk):
    """Upper bound on the number of items for n_req requests totalling at
    most rows_bound key rows (the C ABI's grid bound)."""
    return -(-int(rows_bound) // chunk) + int(n_req)


def _bases(lengths, chunk):
    first, acc = [], 0
    for n in lengths:
        first.append(acc)
        acc += n_chunks(n, chunk)
    return first


def varlen_work(query_lengths, key_lengths, starts, chunk):
    """(flat int32 list, item count) for varlen (starts = first key row of
    each request) or verify (starts = resident slot of each request)."""
    first = _bases(key_lengths, chunk)
    q0, acc = [], 0
    for q in query_lengths:
        q0.append(acc)
        acc += q
    rec = []
    items = chunk_items(key_lengths, chunk)
    for r, c in items:
        rec += (r, c, first[r], q0[r], query_lengths[r], key_lengths[r], starts[r], n_chunks(key_lengths[r], chunk))
    for r, k in enumerate(key_lengths):
        rec += (first[r], n_chunks(k, chunk), q0[r], query_lengths[r])
    return rec, len(items)


def draft_work(context_lengths, cu_blocks, anchors, chunk):
    """(flat int32 list, item count) for draft attention; anchors is the
    flat per-block list, cu_blocks the block offsets per request."""
    first = _bases(context_lengths, chunk)
    rec = []
    items = chunk_items(context_lengths, chunk)
    for r, c in items:
        b0, b1 = cu_blocks[r], cu_blocks[r + 1]
        rec += (r, c, first[r], context_lengths[r], b0, b1 - b0, max(anchors[b0:b1]),
                n_chunks(context_lengths[r], chunk))
    for r, n in enumerate(context_lengths):
        rec += (first[r], n_chunks(n, chunk), cu_blocks[r], cu_blocks[r + 1] - cu_blocks[r])
    return rec, len(items)


def upload_work(records, device):
    """int32 device copy of a work list via the pinned staging ring."""
    return upload(device, records)
