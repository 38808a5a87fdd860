"""Split-K work lists.

Varlen / verification attention: balanced key segments.  The keys of all
requests, laid end to end in request order, are cut into `groups` runs of
(nearly) equal length, each cut moved to a 32-key tile boundary of the
request it falls in; the 8 workgroups of run w (one per KV head) run on
XCD w mod 8 (see XCDS).  A run may end
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

With measured per-XCD speeds (xcd_speed), run w's share of the cost is
proportional to the speed of its XCD, so that the XCDs finish together.
With two resident workgroups per CU, the runs dispatched second onto their
CUs get SECOND_SLOT_SHARE of that share (run_shares).

Draft attention: the same balanced segments over the context rows each
request streams (up to its largest anchor), one run per (workgroup, KV
head), cuts on 64-row ring-stage boundaries (draft_work).

Without a list, both kernels walk fixed chunks of `chunk` rows in request
order over a grid sized from the row bound.
"""
from ._device import upload

DEFAULT_CHUNK = 1024          # verification / varlen: fixed chunks when no list is given
TILE = 32                     # segment cuts fall on multiples of this many keys
MIN_SEGMENT = 256             # fewest keys a run is given (tiny calls use fewer runs)
RESIDENT_PER_CU = 2           # varlen/verify workgroups resident per CU (register budget)
XCDS = 8                      # MI355X: workgroup b runs on XCD b mod 8; varlen runs come in whole rounds of 8
SEGMENT_COST = 96             # keys' worth of fixed work per segment in balanced varlen plans (measured)
# Cost share of a balanced varlen run whose workgroups are dispatched after
# every CU already holds one: two resident workgroups share a CU, and the
# later one's waves lose issue arbitration to the older ones, so it streams
# ~15 % slower (measured; 0.6-0.9 all gain about the same).
SECOND_SLOT_SHARE = 0.75
DRAFT_TILE = 64               # draft cuts fall on multiples of the ring stage
DRAFT_SEGMENT_COST = 512      # balanced draft plans: fixed cost of a segment, in context rows (measured)
DRAFT_BLOCK_WEIGHT = 0.055    # balanced draft plans: extra cost of a row per block beyond the first (measured)
MIN_DRAFT_SEGMENT = 1024      # fewest context rows a draft run is given
# Fixed draft chunks when no list is given (a chunk carries up to 8 blocks
# of FP32 partials, so draft chunks are coarser).
DRAFT_CHUNK = 4096
MIN_DRAFT_CHUNK = 256         # the batch-sized draft chunk never falls below this many rows
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
    there is enough work, about MIN_SEGMENT keys per run at least, in whole
    rounds of XCDS runs (run w executes on XCD w mod XCDS)."""
    slots = max(XCDS, (int(n_cu) * RESIDENT_PER_CU) // (8 * max(1, int(row_tiles))) // XCDS * XCDS)
    runs = max(1, min(slots, -(-int(total_keys) // MIN_SEGMENT)))
    return -(-runs // XCDS) * XCDS


def _flatten(n, per_run, record, request):
    """Flatten per-run [(request, k0, k1)] segment lists into the int32 list
    format, giving split requests consecutive request-major partial slots in
    key order.  record(r, k0, k1, slot) and request(r, first, count) give the
    8 and 4 ints of a segment and a request.  Returns (list, segment count,
    run count)."""
    count = [0] * n
    for run in per_run:
        for r, _, _ in run:
            count[r] += 1
    first, slot = [], 0
    for c in count:
        first.append(slot if c > 1 else -1)
        slot += c if c > 1 else 0
    keyed = {}
    # partial slot of a segment = first slot of its request + its key-order rank
    for run in per_run:
        for r, k0, _ in run:
            keyed.setdefault(r, []).append(k0)
    rank = {r: {k0: i for i, k0 in enumerate(sorted(v))} for r, v in keyed.items()}
    out, ranges = [], [0]
    for run in per_run:
        for r, k0, k1 in run:
            out += record(r, k0, k1, first[r] + rank[r][k0] if first[r] >= 0 else -1)
        ranges.append(ranges[-1] + len(run))
    out += ranges
    for r in range(n):
        out += request(r, max(first[r], 0), count[r])
    return out, ranges[-1], len(per_run)


def _segment_list(query_lengths, key_lengths, starts, per_run):
    """Varlen/verify records: request, k0, k1, slot, first query row, query
    length, key length, start; request records: first slot, count, first
    query row, query length."""
    q0, acc = [], 0
    for q in query_lengths:
        q0.append(acc)
        acc += int(q)
    return _flatten(len(key_lengths), per_run,
                    lambda r, k0, k1, slot: (r, k0, k1, slot, q0[r], int(query_lengths[r]), int(key_lengths[r]),
                                             int(starts[r])),
                    lambda r, first, count: (first, count, q0[r], int(query_lengths[r])))


def _balanced_runs(key_lengths, groups, tile, seg_cost=0, weights=None, shares=None):
    """Per-run [(request, k0, k1)] lists: the keys of all requests end to end,
    cut into `groups` runs of (nearly) equal cost, each cut moved down to a
    `tile` boundary of the request holding it.  A request costs seg_cost
    (the fixed work of starting a segment, in keys) plus its keys, each
    weighted by weights[r] (default 1), so runs that hold more request
    starts or heavier keys get fewer keys.  shares (one positive number per
    run) makes run w's cost proportional to shares[w] instead of equal."""
    n = len(key_lengths)
    groups = max(1, int(groups))
    if shares is None:
        bound = [w / groups for w in range(groups + 1)]
    else:
        if len(shares) != groups or min(shares) <= 0:
            raise ValueError('shares must give one positive number per run')
        bound, acc, tot = [0.0], 0.0, float(sum(shares))
        for x in shares:
            acc += float(x)
            bound.append(acc / tot)
    seg_cost = max(0.0, float(seg_cost))
    wt = [1.0] * n if weights is None else [max(1e-3, float(x)) for x in weights]
    begin, vbegin, total, vtotal = [], [], 0, 0.0
    for k, w in zip(key_lengths, wt):
        begin.append(total)
        vbegin.append(vtotal)
        total += int(k)
        vtotal += seg_cost + w * int(k)
    cuts, r = [0], 0
    for w in range(1, groups):
        x = bound[w] * vtotal                         # cut in cost space
        while r + 1 < n and vbegin[r + 1] <= x:
            r += 1
        into = int(max(0.0, (x - vbegin[r] - seg_cost) / wt[r]))   # keys of request r before the cut
        cuts.append(max(cuts[-1], begin[r] + (min(into, int(key_lengths[r])) // tile) * tile))
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
    return per_run


def xcd_shares(groups, xcd_speed):
    """Cost share of each of `groups` runs: the speed of the XCD it runs on
    (run w on XCD w mod XCDS), or None for equal runs."""
    if xcd_speed is None:
        return None
    speed = [float(x) for x in xcd_speed]
    if len(speed) != XCDS or min(speed) <= 0:
        raise ValueError(f'xcd_speed must give {XCDS} positive relative speeds')
    return [speed[w % XCDS] for w in range(int(groups))]


def second_slot_runs(groups, n_cu):
    """Runs whose workgroups are the second resident on their CUs, or an
    empty set.  Run w's workgroups are blockIdx.x = 8 (8 (w / 8) + g) + w mod
    8 (g = KV head); the dispatcher deals ids 0 .. n_cu - 1 one per CU first,
    so with exactly RESIDENT_PER_CU = 2 workgroups per CU (8 groups = 2 n_cu)
    and n_cu a multiple of 64 the runs w >= n_cu / 8 are the second ones.
    Any other launch shape gets no distinction."""
    groups = int(groups)
    if n_cu is None or int(n_cu) % 64 or 8 * groups != RESIDENT_PER_CU * int(n_cu):
        return frozenset()
    return frozenset(range(int(n_cu) // 8, groups))


def run_shares(groups, xcd_speed=None, n_cu=None):
    """Cost share of each of `groups` runs: its XCD's speed (xcd_shares;
    equal without xcd_speed), times SECOND_SLOT_SHARE for the runs of
    second_slot_runs(groups, n_cu); None when every share is equal."""
    shares = xcd_shares(groups, xcd_speed)
    second = second_slot_runs(groups, n_cu)
    if not second:
        return shares
    shares = shares or [1.0] * int(groups)
    return [x * (SECOND_SLOT_SHARE if w in second else 1.0) for w, x in enumerate(shares)]


def varlen_work(query_lengths, key_lengths, starts, groups, seg_cost=None, xcd_speed=None, n_cu=None):
    """Balanced plan: (flat int32 list, segment count, run count) for varlen (starts =
    first key row of each request) or verify (starts = resident slot of each
    request); groups = number of runs (workgroups per KV head); seg_cost
    (default SEGMENT_COST) the fixed cost of a segment in keys; xcd_speed
    (8 relative speeds) weights each run by the speed of its XCD; n_cu (the
    device's CU count) gives the second resident workgroups of each CU
    SECOND_SLOT_SHARE of a run's cost (run_shares).  The cut points depend
    on every request's length (and on xcd_speed), so a request's output can
    differ in the last bits between batches; request_work keeps them
    apart."""
    cost = SEGMENT_COST if seg_cost is None else seg_cost
    return _segment_list(query_lengths, key_lengths, starts,
                         _balanced_runs(key_lengths, groups, TILE, cost, shares=run_shares(groups, xcd_speed, n_cu)))


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
    groups = -(-max(1, min(int(groups), len(segs))) // XCDS) * XCDS     # whole rounds over the XCDs
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


def segment_plan(split, query_lengths, key_lengths, starts, groups, chunk, capacity=None, xcd_speed=None,
                 n_cu=None):
    """(flat int32 list, segment count, run count) of the named plan; the
    launch must pass the returned counts (n_work, n_groups).  xcd_speed,
    n_cu: see varlen_work (balanced plans only).

    capacity = (segments, runs) lays the list out in regions of fixed size:
    the records padded to `segments`, the run ranges to `runs` (trailing runs
    empty).  Every transaction of a bucket then launches with the same
    arguments and grid, which a captured graph replays."""
    if split == 'balanced':
        out, n_seg, runs = varlen_work(query_lengths, key_lengths, starts, groups, xcd_speed=xcd_speed, n_cu=n_cu)
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


def draft_work(context_lengths, cu_blocks, anchors, groups=None, *, chunk=None, offsets=None):
    """Draft plan: (flat int32 list, segment count, run count).  Request r
    streams its context up to its largest anchor (the rows any of its blocks
    sees), and the segment ending a request also attends its blocks' own rows.
      * chunk given (the default plan): every request is cut at multiples of
        `chunk` of its own rows, one segment per run (workgroup), longest
        first, so the hardware dispatcher balances the ragged tail (each
        workgroup's 128 KiB ring fills a CU's LDS, one resident per CU);
      * else: the rows of all requests, end to end, are cut into `groups` runs
        of equal cost at DRAFT_TILE boundaries: a request costs
        DRAFT_SEGMENT_COST plus its rows weighted by 1 + DRAFT_BLOCK_WEIGHT
        per block beyond the first (more blocks, more MFMA and LDS work per
        row).

      segment: request, k0, k1, partial slot (-1: one segment), first block,
               block count, largest anchor, 1 + offsets[r] (0 without
               offsets, or when it does not fit in 31 bits: the kernel then
               reads ctx_off[r] itself)
      request: first partial slot, segment count, first block, block count
    """
    amax = [max(anchors[cu_blocks[r]:cu_blocks[r + 1]]) for r in range(len(context_lengths))]
    off1 = [0] * len(amax) if offsets is None else [int(o) + 1 if 0 <= int(o) < 2 ** 31 - 1 else 0 for o in offsets]
    if any(not 0 <= a <= int(c) for a, c in zip(amax, context_lengths)):
        raise ValueError('Anchors must lie in [0, context length]')
    if chunk is not None:
        segs = []
        for r, n in enumerate(amax):
            for c in range(n_chunks(n, chunk)):
                segs.append((min(chunk, n - c * chunk) if n > 0 else 0, r, c * chunk, min(n, c * chunk + chunk)))
        segs.sort(key=lambda x: (-x[0], x[1], x[2]))
        per_run = [[(r, k0, k1)] for _, r, k0, k1 in segs]
    else:
        nb = [cu_blocks[r + 1] - cu_blocks[r] for r in range(len(amax))]
        per_run = _balanced_runs(amax, groups, DRAFT_TILE, DRAFT_SEGMENT_COST,
                                 [1.0 + DRAFT_BLOCK_WEIGHT * (b - 1) for b in nb])
    return _flatten(len(amax), per_run,
                    lambda r, k0, k1, slot: (r, k0, k1, slot, cu_blocks[r], cu_blocks[r + 1] - cu_blocks[r], amax[r],
                                             off1[r]),
                    lambda r, first, count: (first, count, cu_blocks[r], cu_blocks[r + 1] - cu_blocks[r]))


def draft_chunk_for(visible_rows, n_cu):
    """Fixed draft chunk sized to a batch: its visible context rows (each
    request's largest anchor, summed) cut into about one (chunk, KV head)
    item per CU, in multiples of DRAFT_TILE rows, between MIN_DRAFT_CHUNK
    and DRAFT_CHUNK.  A batch that fills the CUs at DRAFT_CHUNK keeps it; a
    small one is cut finer, so that its few requests still spread over every
    CU (at the price of split-K partials and their merge)."""
    per_head = max(1, int(n_cu) // 8)
    rows = -(-max(1, int(visible_rows)) // per_head)
    rows = -(-rows // DRAFT_TILE) * DRAFT_TILE
    return max(MIN_DRAFT_CHUNK, min(DRAFT_CHUNK, rows))


def draft_run_count(total_rows, n_cu):
    """Draft runs per KV head: one workgroup per CU (its 128 KiB ring fills
    the CU's LDS), never fewer than MIN_DRAFT_SEGMENT rows per run."""
    return max(1, min(max(1, int(n_cu) // 8), -(-int(total_rows) // MIN_DRAFT_SEGMENT)))


def upload_work(records, device):
    """int32 device copy of a work list via the pinned staging ring."""
    return upload(device, records)
