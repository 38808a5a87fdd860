"""Host-side work lists (CPU): balanced key segments for varlen/verification
attention.  The kernels trust these records, so their invariants are checked
here: every key of every request is covered exactly once, cuts fall on
32-key tile boundaries, runs carry (nearly) equal cost (keys, plus a fixed
cost per request starting in the run), and the merge records name exactly
the partial slots the segments write."""
import numpy as np
import pytest

from qwen3_dspark_amd.schedule import (MIN_SEGMENT, REQ_INTS, SEGMENT_COST, TILE, WORK_INTS, request_work,
                                       run_count, varlen_list_bound, varlen_work)


def decode(out, n_seg, groups, n_req):
    rec = [tuple(out[WORK_INTS * i:WORK_INTS * (i + 1)]) for i in range(n_seg)]
    base = WORK_INTS * n_seg
    ranges = out[base:base + groups + 1]
    reqs = [tuple(out[base + groups + 1 + REQ_INTS * r:base + groups + 1 + REQ_INTS * (r + 1)]) for r in range(n_req)]
    assert len(out) == base + groups + 1 + REQ_INTS * n_req
    return rec, ranges, reqs


def check(query_lengths, key_lengths, starts, groups, chunk=None, seg_cost=None, xcd_speed=None, n_cu=None):
    if chunk is None:
        out, n_seg, runs = varlen_work(query_lengths, key_lengths, starts, groups, seg_cost, xcd_speed=xcd_speed,
                                       n_cu=n_cu)
        assert runs == groups
    else:
        out, n_seg, runs = request_work(query_lengths, key_lengths, starts, chunk, groups)
        assert runs == -(-max(1, min(groups, n_seg)) // 8) * 8 and runs % 8 == 0
        groups = runs
    n = len(key_lengths)
    rec, ranges, reqs = decode(out, n_seg, groups, n)
    assert ranges[0] == 0 and ranges[-1] == n_seg and all(a <= b for a, b in zip(ranges, ranges[1:]))
    assert n_seg <= varlen_list_bound(n, groups, sum(key_lengths), chunk)
    q0 = np.concatenate([[0], np.cumsum(query_lengths)[:-1]])
    by_req = {}
    for i, (r, k0, k1, slot, qs, ql, kl, st) in enumerate(rec):
        assert (qs, ql, kl, st) == (q0[r], query_lengths[r], key_lengths[r], starts[r])
        by_req.setdefault(r, []).append((k0, k1, slot))
    loads = []
    for w in range(groups):
        loads.append(sum(rec[i][2] - rec[i][1] for i in range(ranges[w], ranges[w + 1])))
    check.starts = [sum(1 for i in range(ranges[w], ranges[w + 1]) if rec[i][1] == 0) for w in range(groups)]
    segments_of = {}
    for r, kl in enumerate(key_lengths):
        segs = sorted(by_req[r])
        segments_of[r] = [(a, b) for a, b, _ in segs]
        first, count, qs, ql = reqs[r]
        assert count == len(segs) and (qs, ql) == (q0[r], query_lengths[r])
        # exact cover of [0, kl), cuts on tile boundaries
        assert segs[0][0] == 0 and segs[-1][1] == kl
        for (a0, a1, _), (b0, _, _) in zip(segs, segs[1:]):
            assert a1 == b0 and a1 % (TILE if chunk is None else chunk) == 0 and a1 > a0
        if count == 1:
            assert segs[0][2] == -1
        else:
            assert [s for _, _, s in segs] == list(range(first, first + count))
    slots = sorted(s for _, _, s in (x for v in by_req.values() for x in v) if s >= 0)
    assert slots == list(range(len(slots)))       # dense, request-major partial slots
    return loads, segments_of


def test_balanced_runs_at_the_64_request_stress_shape():
    rng = np.random.default_rng(20261009)
    ctx = np.floor(np.exp(rng.uniform(np.log(256), np.log(8192), size=64))).astype(int)
    kl = [int(c) + 7 for c in ctx]
    groups = run_count(sum(kl), 256)
    assert groups == 64
    # keys only: every run within a tile or two of the mean
    loads, _ = check([7] * 64, kl, list(range(64)), groups, seg_cost=0)
    assert max(loads) - min(loads) <= 2 * TILE
    assert sum(loads) == sum(kl)
    # with the fixed cost of a segment: keys + cost x (requests starting in
    # the run) balanced instead; runs holding more starts get fewer keys
    loads, _ = check([7] * 64, kl, list(range(64)), groups)
    # each of a run's two cuts moves its cost by at most a tile plus one
    # segment cost (a cut inside a request's start cost lands at its start)
    cost = [k + SEGMENT_COST * n for k, n in zip(loads, check.starts)]
    assert max(cost) - min(cost) <= 2 * (TILE + SEGMENT_COST)
    assert sum(loads) == sum(kl)
    starts = np.array(check.starts)
    assert np.mean([k for k, n in zip(loads, starts) if n == starts.max()]) < np.mean(loads)


@pytest.mark.parametrize('kl,groups', [([5], 1), ([40], 4), ([0, 5], 3), ([1, 1, 1], 8), ([31, 33, 64, 65], 3),
                                       ([1000, 0, 0, 7, 2048], 5), ([8192] * 3 + [7] * 10, 16)])
def test_edge_shapes(kl, groups):
    ql = [max(1, min(k, 7)) for k in kl]
    check(ql, kl, [3 * i for i in range(len(kl))], groups)


def test_run_count_bounds():
    # whole rounds of 8 runs (run w executes on XCD w mod 8)
    assert run_count(10, 256) == 8
    assert run_count(MIN_SEGMENT * 3, 256) == 8
    assert run_count(MIN_SEGMENT * 12, 256) == 16
    assert run_count(10 ** 7, 256) == 64
    assert run_count(10 ** 7, 256, row_tiles=2) == 32
    assert run_count(10 ** 7, 304) == 72
    assert run_count(10 ** 7, 8, row_tiles=4) == 8


def test_random_shapes_cover_exactly():
    rng = np.random.default_rng(7)
    for _ in range(200):
        n = int(rng.integers(1, 40))
        kl = [int(x) for x in rng.integers(0, 3000, size=n)]
        ql = [max(1, min(k, int(rng.integers(1, 9)))) for k in kl]
        check(ql, kl, list(range(n)), int(rng.integers(1, 70)))


def test_request_plan_cuts_depend_only_on_the_request():
    rng = np.random.default_rng(11)
    for _ in range(50):
        n = int(rng.integers(2, 30))
        kl = [int(x) for x in rng.integers(1, 5000, size=n)]
        ql = [min(k, 7) for k in kl]
        chunk = int(rng.choice([256, 1024]))
        _, segs = check(ql, kl, list(range(n)), int(rng.integers(1, 70)), chunk=chunk)
        perm = rng.permutation(n)
        _, segs2 = check([ql[i] for i in perm], [kl[i] for i in perm], list(range(n)), int(rng.integers(1, 70)),
                         chunk=chunk)
        for j, i in enumerate(perm):
            assert segs2[j] == segs[i] == [(c, min(c + chunk, kl[i])) for c in range(0, kl[i], chunk)]


def test_fixed_capacity_layout_keeps_the_plan():
    from qwen3_dspark_amd.schedule import segment_plan
    rng = np.random.default_rng(5)
    for split in ('balanced', 'request'):
        for _ in range(30):
            n = int(rng.integers(1, 20))
            kl = [int(x) for x in rng.integers(1, 4000, size=n)]
            ql = [min(k, 7) for k in kl]
            runs = int(rng.integers(1, 40))
            out, n_seg, g = segment_plan(split, ql, kl, list(range(n)), runs, 512)
            cap = (n_seg + int(rng.integers(0, 50)), g + int(rng.integers(0, 9)))
            pad, n_work, groups = segment_plan(split, ql, kl, list(range(n)), runs, 512, cap)
            assert (n_work, groups) == cap
            assert pad[:WORK_INTS * n_seg] == out[:WORK_INTS * n_seg]
            ranges = pad[WORK_INTS * n_work:WORK_INTS * n_work + groups + 1]
            assert ranges[:g + 1] == out[WORK_INTS * n_seg:WORK_INTS * n_seg + g + 1]
            assert all(r == n_seg for r in ranges[g:])
            assert pad[WORK_INTS * n_work + groups + 1:] == out[WORK_INTS * n_seg + g + 1:]
            with pytest.raises(ValueError, match='capacity'):
                segment_plan(split, ql, kl, list(range(n)), runs, 512, (n_seg - 1, g) if n_seg > 1 else (0, g))


def test_draft_plan_covers_each_streamed_context_once():
    """Draft segments cover [0, largest anchor) of every request exactly once,
    cut on 64-row boundaries, runs balanced; requests whose anchors are all 0
    still get the one (empty) segment that attends their own blocks."""
    from qwen3_dspark_amd.schedule import DRAFT_TILE, draft_work
    rng = np.random.default_rng(9)
    for _ in range(60):
        n = int(rng.integers(1, 40))
        ctx = [int(x) for x in rng.integers(0, 9000, size=n)]
        anchors, cu = [], [0]
        for c in ctx:
            k = int(rng.integers(1, 9))
            row = [int(x) for x in rng.integers(0, c + 1, size=k)]
            if rng.random() < 0.5:
                row[0] = c
            anchors += row
            cu.append(cu[-1] + k)
        groups = int(rng.integers(1, 40))
        chunked = rng.random() < 0.3
        if chunked:
            out, n_seg, runs = draft_work(ctx, cu, anchors, chunk=1024)
            groups = runs
            assert runs == n_seg                                        # one segment per run
        else:
            out, n_seg, runs = draft_work(ctx, cu, anchors, groups)
            assert runs == groups
        rec = [tuple(out[WORK_INTS * i:WORK_INTS * (i + 1)]) for i in range(n_seg)]
        ranges = out[WORK_INTS * n_seg:WORK_INTS * n_seg + groups + 1]
        reqs = [tuple(out[WORK_INTS * n_seg + groups + 1 + REQ_INTS * r:][:REQ_INTS]) for r in range(n)]
        by_req = {}
        for r, k0, k1, slot, b0, nb, amax, zero in rec:
            assert (b0, nb, amax, zero) == (cu[r], cu[r + 1] - cu[r], max(anchors[cu[r]:cu[r + 1]]), 0)
            by_req.setdefault(r, []).append((k0, k1, slot))
        for r in range(n):
            amax = max(anchors[cu[r]:cu[r + 1]])
            segs = sorted(by_req[r])
            assert segs[0][0] == 0 and segs[-1][1] == amax
            assert sum(1 for s in segs if s[1] >= amax) == 1       # exactly one segment attends the blocks
            for (a0, a1, _), (b0_, _, _) in zip(segs, segs[1:]):
                assert a1 == b0_ and a1 % DRAFT_TILE == 0
            first, count, b0, nb = reqs[r]
            assert count == len(segs) and (b0, nb) == (cu[r], cu[r + 1] - cu[r])
            assert [s for _, _, s in segs] == ([-1] if count == 1 else list(range(first, first + count)))
        loads = [sum(rec[i][2] - rec[i][1] for i in range(ranges[w], ranges[w + 1])) for w in range(groups)]
        total = sum(max(anchors[cu[r]:cu[r + 1]]) for r in range(n))
        assert sum(loads) == total
        if not chunked:
            # balanced in cost: a segment start costs DRAFT_SEGMENT_COST, a row
            # 1 + DRAFT_BLOCK_WEIGHT per block beyond the first; each of a
            # run's two cuts moves its cost by at most a tile of the heaviest
            # rows plus one segment cost
            from qwen3_dspark_amd.schedule import DRAFT_BLOCK_WEIGHT, DRAFT_SEGMENT_COST
            weight = lambda r: 1 + DRAFT_BLOCK_WEIGHT * (cu[r + 1] - cu[r] - 1)
            cost = [sum(weight(rec[i][0]) * (rec[i][2] - rec[i][1]) + DRAFT_SEGMENT_COST * (rec[i][1] == 0)
                        for i in range(ranges[w], ranges[w + 1])) for w in range(groups)]
            assert max(cost) - min(cost) <= 2 * (DRAFT_TILE * (1 + 7 * DRAFT_BLOCK_WEIGHT) + DRAFT_SEGMENT_COST) + 1
        else:
            assert loads == sorted(loads, reverse=True) and max(loads) <= 1024   # longest first


def test_xcd_speeds_size_the_runs_of_each_xcd():
    """Run w executes on XCD w mod 8: with measured XCD speeds, each XCD's
    runs carry cost in proportion to its speed (the cover stays exact)."""
    rng = np.random.default_rng(20261009)
    ctx = np.floor(np.exp(rng.uniform(np.log(256), np.log(8192), size=64))).astype(int)
    kl = [int(c) + 7 for c in ctx]
    groups = run_count(sum(kl), 256)
    speed = [1.05, 0.95, 1.03, 0.97, 1.04, 0.96, 1.02, 0.98]
    loads, _ = check([7] * 64, kl, list(range(64)), groups, xcd_speed=speed)
    cost = [k + SEGMENT_COST * n for k, n in zip(loads, check.starts)]
    total = sum(cost)
    for w in range(groups):   # every run within two cuts' rounding of its share
        assert abs(cost[w] - total * speed[w % 8] / (sum(speed) * groups / 8)) <= 2 * (TILE + SEGMENT_COST)
    per_xcd = [sum(cost[w] for w in range(x, groups, 8)) for x in range(8)]
    ratios = [c / v for c, v in zip(per_xcd, speed)]
    assert max(ratios) / min(ratios) < 1.02
    assert sum(loads) == sum(kl)
    # equal speeds give the equal plan
    assert varlen_work([7] * 64, kl, list(range(64)), groups, xcd_speed=[2.0] * 8) == \
        varlen_work([7] * 64, kl, list(range(64)), groups)
    with pytest.raises(ValueError, match='8 positive'):
        varlen_work([7] * 64, kl, list(range(64)), groups, xcd_speed=[1.0] * 7)


def test_batch_sized_draft_chunk():
    """About one (chunk, KV head) item per CU, multiples of 64 rows, clamped
    to [256, 4096]: the 64-request stress batch keeps 4096, a 16-request
    batch of short contexts is cut finer."""
    from qwen3_dspark_amd.schedule import DRAFT_CHUNK, MIN_DRAFT_CHUNK, draft_chunk_for
    assert draft_chunk_for(157046, 256) == DRAFT_CHUNK
    assert draft_chunk_for(9216, 256) == 320                  # 9216 rows over 32 CUs per KV head: 288 -> 320
    assert draft_chunk_for(224, 256) == MIN_DRAFT_CHUNK
    assert draft_chunk_for(0, 256) == MIN_DRAFT_CHUNK
    for rows in (1, 63, 64, 65, 5000, 70000, 10 ** 7):
        for cus in (8, 80, 256, 304):
            c = draft_chunk_for(rows, cus)
            assert c % 64 == 0 and MIN_DRAFT_CHUNK <= c <= DRAFT_CHUNK
            # at or above the floor and below the cap, chunks of this size give at most one item per CU per head
            if MIN_DRAFT_CHUNK < c < DRAFT_CHUNK:
                assert -(-rows // c) <= max(1, cus // 8)


def test_second_slot_runs_get_a_smaller_share():
    """With two resident workgroups per CU (8 x 64 runs on 256 CUs), the
    runs whose workgroups are dispatched after every CU holds one (w >= 32:
    blockIdx.x = 8 (8 (w / 8) + g) + w mod 8 >= 256 for every KV head g)
    carry SECOND_SLOT_SHARE of the cost of the others; any other shape, or
    no CU count, leaves the plan as it was."""
    from qwen3_dspark_amd.schedule import (SECOND_SLOT_SHARE, run_shares, second_slot_runs, varlen_work,
                                           xcd_shares)
    second = second_slot_runs(64, 256)
    assert second == frozenset(range(32, 64))
    for w in range(64):
        ids = [8 * (8 * (w // 8) + g) + w % 8 for g in range(8)]
        assert all((i >= 256) == (w in second) for i in ids)
    assert second_slot_runs(32, 256) == frozenset()          # one workgroup per CU
    assert second_slot_runs(64, None) == frozenset()
    assert second_slot_runs(8, 32) == frozenset()            # 32 CUs: not a multiple of 64
    speed = [1.05, 0.95, 1.03, 0.97, 1.04, 0.96, 1.02, 0.98]
    shares = run_shares(64, speed, 256)
    base = xcd_shares(64, speed)
    assert shares == [x * (SECOND_SLOT_SHARE if w >= 32 else 1.0) for w, x in enumerate(base)]
    assert run_shares(64, None, None) is None and run_shares(64, speed, None) == base
    # the plan: per-run cost (keys + SEGMENT_COST per segment) follows the shares
    rng = np.random.default_rng(3)
    kl = [int(x) for x in np.exp(rng.uniform(np.log(263), np.log(8199), size=64))]
    loads, _ = check([7] * 64, kl, list(range(64)), 64, xcd_speed=speed, n_cu=256)
    cost = [k + SEGMENT_COST * n for k, n in zip(loads, check.starts)]
    total, norm = sum(cost), sum(shares)
    for w in range(64):
        assert abs(cost[w] - total * shares[w] / norm) <= 2 * (TILE + SEGMENT_COST)
    assert sum(loads) == sum(kl)
    assert varlen_work([7] * 64, kl, list(range(64)), 32, n_cu=256) == varlen_work([7] * 64, kl, list(range(64)), 32)
