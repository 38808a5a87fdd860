"""Split-K work lists.

Varlen / verification attention: balanced key segments.  The keys of all
requests, laid end to end in request order, are cut into `groups` runs of
(nearly) equal length, each cut moved to a 32-key tile boundary of the
request it falls in; workgroup (w, KV head g) streams run w.  A run may end
inside one request and start inside the next, so a request is held by one
or more segments (one per run it meets).  Every workgroup therefore reads
the same number of key rows, whatever the mix of context lengths, and a
request cut into several segments writes one set of FP32 partials per
segment for the split-K merge.  Segment partial slots are request-major, so
results do not depend on the cut points beyond the floating-point order of
the merge.

  list = [segment records, WORK_INTS each, grouped by run]
         [run ranges: groups + 1 record indices]
         [request records, REQ_INTS each]
  segment: request, first key, end key, partial slot (-1: the request has a
           single segment and writes its output), first query row, query
           length, key length, first key row (varlen) or resident slot (verify)
  request: first partial slot, segment count, first query row, query length

Draft attention: fixed chunks.  Every request's context is cut into chunks
of `chunk` rows (at least one chunk per request) and each (request, chunk)
pair is one work item per KV head, dispatched longest first so that the
short tail chunks of ragged requests fill the end of the grid (greedy
longest-processing-time order); the partial slot of an item stays its
request-major index, so the dispatch order does not affect results.

  draft item: request, chunk, chunk base, context length, first block,
              block count, largest anchor, chunk count
  request:    chunk base, chunk count, first block, block count
"""
from ._device import upload

DEFAULT_CHUNK = 1024          # verification / varlen: fixed chunks when no list is given
TILE = 32                     # segment cuts fall on multiples of this many keys
MIN_SEGMENT = 256             # fewest keys a run is given (tiny calls use fewer runs)
RESIDENT_PER_CU = 2           # varlen/verify workgroups resident per CU (register budget)
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


def run_count(total_keys, n_cu, row_tiles=1):
    """Runs for a balanced list: one workgroup per CU slot and KV head when
    there is enough work, never fewer than MIN_SEGMENT keys per run."""
    slots = max(1, (int(n_cu) * RESIDENT_PER_CU) // (8 * max(1, int(row_tiles))))
    return max(1, min(slots, -(-int(total_keys) // MIN_SEGMENT)))


def _segment_list(query_lengths, key_lengths, starts, per_run):
    """Flatten per-run [(request, k0, k1)] segment lists into the int32 list
    format, giving split requests consecutive request-major partial slots in
    key order.  Returns (list, segment count, run count)."""
    n = len(key_lengths)
    count = [0] * n
    for run in per_run:
        for r, _, _ in run:
            count[r] += 1
    first, slot = [], 0
    for c in count:
        first.append(slot if c > 1 else -1)
        slot += c if c > 1 else 0
    q0, acc = [], 0
    for q in query_lengths:
        q0.append(acc)
        acc += int(q)
    keyed = {}
    # partial slot of a segment = first slot of its request + its key-order rank
    for run in per_run:
        for r, k0, _ in run:
            keyed.setdefault(r, []).append(k0)
    rank = {r: {k0: i for i, k0 in enumerate(sorted(v))} for r, v in keyed.items()}
    out, ranges = [], [0]
    for run in per_run:
        for r, k0, k1 in run:
            slot = first[r] + rank[r][k0] if first[r] >= 0 else -1
            out += (r, k0, k1, slot, q0[r], int(query_lengths[r]), int(key_lengths[r]), int(starts[r]))
        ranges.append(ranges[-1] + len(run))
    out += ranges
    for r in range(n):
        out += (max(first[r], 0), count[r], q0[r], int(query_lengths[r]))
    return out, ranges[-1], len(per_run)


def varlen_work(query_lengths, key_lengths, starts, groups):
    """Balanced plan: (flat int32 list, segment count, run count) for varlen (starts =
    first key row of each request) or verify (starts = resident slot of each
    request); groups = number of runs (workgroups per KV head).  The cut
    points depend on every request's length, so a request's output can
    differ in the last bits between batches; request_work keeps them apart."""
    n = len(key_lengths)
    groups = max(1, int(groups))
    begin, total = [], 0
    for k in key_lengths:
        begin.append(total)
        total += int(k)
    # Run boundaries in the concatenated key stream, each moved down to a
    # tile boundary of the request holding it; monotone by construction.
    cuts, r = [0], 0
    for w in range(1, groups):
        x = (w * total) // groups
        while r + 1 < n and begin[r + 1] <= x:
            r += 1
        cuts.append(max(cuts[-1], begin[r] + ((x - begin[r]) // TILE) * TILE))
    cuts.append(total)
    per_run = [[] for _ in range(groups)]
    w = 0
    for r in range(n):
        a, kl = begin[r], int(key_lengths[r])
        while w + 1 < groups and cuts[w + 1] <= a:   # the run holding key position a
            w += 1
        if kl == 0:
            per_run[w].append((r, 0, 0))
            continue
        v = w
        while True:
            lo, hi = max(cuts[v], a), min(cuts[v + 1], a + kl)
            if hi > lo:
                per_run[v].append((r, lo - a, hi - a))
            if cuts[v + 1] >= a + kl or v + 1 == groups:
                break
            v += 1
    return _segment_list(query_lengths, key_lengths, starts, per_run)


def request_work(query_lengths, key_lengths, starts, chunk, groups):
    """Request-local plan: every request is cut at multiples of `chunk` of
    its own keys (at least one segment), so its output never depends on the
    other requests of the batch.  Segments go to the least-loaded of `groups`
    runs, longest first."""
    import heapq
    segs = []
    for r, kl in enumerate(key_lengths):
        kl = int(kl)
        for c in range(n_chunks(kl, chunk)):
            k0 = c * chunk
            segs.append((min(chunk, kl - k0) if kl > 0 else 0, r, k0, min(kl, k0 + chunk)))
    segs.sort(key=lambda x: (-x[0], x[1], x[2]))
    groups = max(1, min(int(groups), len(segs)))
    heap = [(0, w) for w in range(groups)]
    per_run = [[] for _ in range(groups)]
    for size, r, k0, k1 in segs:
        load, w = heapq.heappop(heap)
        per_run[w].append((r, k0, k1))
        heapq.heappush(heap, (load + size + TILE, w))
    return _segment_list(query_lengths, key_lengths, starts, per_run)


def varlen_list_bound(n_req, groups, rows_bound=0, chunk=None):
    """Most segment records a list over n_req requests holding at most
    rows_bound keys can have: n_req + groups - 1 for a balanced plan (each
    interior cut splits at most one request), ceil(rows_bound / chunk) +
    n_req for a request-local plan."""
    if chunk is None:
        return int(n_req) + int(groups) - 1
    return chunk_bound(n_req, rows_bound, chunk)


SPLITS = ('balanced', 'request')


def segment_plan(split, query_lengths, key_lengths, starts, groups, chunk, capacity=None):
    """(flat int32 list, segment count, run count) of the named plan; the
    launch must pass the returned counts (n_work, n_groups).

    capacity = (segments, runs) lays the list out in regions of fixed size:
    the records padded to `segments`, the run ranges to `runs` (trailing runs
    empty).  Every transaction of a bucket then launches with the same
    arguments and grid, which a captured graph replays."""
    if split == 'balanced':
        out, n_seg, runs = varlen_work(query_lengths, key_lengths, starts, groups)
    elif split == 'request':
        out, n_seg, runs = request_work(query_lengths, key_lengths, starts, chunk, groups)
    else:
        raise ValueError(f'split must be one of {SPLITS}')
    if capacity is None:
        return out, n_seg, runs
    seg_cap, run_cap = capacity
    if n_seg > seg_cap or runs > run_cap:
        raise ValueError('Segment plan exceeds its fixed capacity')
    base = WORK_INTS * n_seg
    ranges = out[base:base + runs + 1]
    padded = out[:base] + [0] * (WORK_INTS * (seg_cap - n_seg)) + ranges + [ranges[-1]] * (run_cap - runs)
    return padded + out[base + runs + 1:], seg_cap, run_cap


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
