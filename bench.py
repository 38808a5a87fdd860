#!/usr/bin/env python3
"""Benchmark of the DSpark attention hot path on one MI355X.

Workload (64-request stress shape, Qwen3-0.6B attention geometry: 16 query
heads, 8 KV heads, head dim 128, bf16):
  * 64 requests, committed contexts c = floor(exp(U(ln 256, ln 8192))),
    KV cache preallocated at capacity 8192 rows per request (28 layers);
  * draft: 5 layers, 1..8 blocks of 7 rows per request, one block anchored
    at c and the others at U[0, c], context streamed from a slotted pool;
  * verify: 7 appended rows per request (448 query tokens), 28 layers.
One step = one speculative round of the hot path:
  draft attention x5 -> begin (transaction metadata) ->
  28 x (verification attention with the new K/V staged in the same
  launch) -> commit of a
  seeded accepted prefix 0..7 per request (the rest rolled back).
Inputs are seeded N(0,1) bf16 already resident in HBM; the timed region
contains only the rounds themselves.

value = verified tokens per second = 448 / round time (wall clock between
two device synchronisations around the K timed rounds).

Per-call durations come from HIP events recorded on the launch stream
inside the timed rounds: one pair around the 28 verification-attention calls
and one around the 5 draft-attention calls of every round (each call is a
split-K chunk kernel followed by its merge kernel), divided by the number of
calls.  The spans contain the gaps between launches but no per-call marker
work (an event pair around a single call adds ~3-4 us to it).

    python bench.py [--gpus 1] [--steps 20] [--warmup 5]
"""
import argparse
import gc
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = 'attn tokens/s + HBM GB/s (% roofline), 64 ragged reqs, Qwen3-0.6B shapes'
SEED = 20261009
B, Q_LEN, CAPACITY = 64, 7, 8192
VERIFY_LAYERS, DRAFT_LAYERS, BLOCK = 28, 5, 7
ROW_BYTES = 8 * 128 * 2            # one K (or V) token row, all 8 KV heads
Q_ROW_BYTES = 16 * 128 * 2         # one Q (or O) token row, all 16 query heads
HBM_PEAK_GBS = 8000.0              # MI355X HBM3E, published


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=5)
    ap.add_argument('--chunk', type=int, default=None, help='keys per split-K verification work item')
    ap.add_argument('--draft-chunk', type=int, default=None, help='keys per split-K draft work item')
    ap.add_argument('--draft-persistent', type=int, default=None, choices=(0, 1, 8),
                    help='draft scheduling: 0 one workgroup per (chunk, KV head), 1 or 8 persistent workgroups '
                         'taking items from one queue or one queue per KV head (default: the library default)')
    ap.add_argument('--draft-ab', action='store_true',
                    help='only compare the draft scheduling modes on one pool (alternating rounds of the '
                         "workload's 5 draft layers), with outputs checked bitwise equal across modes")
    ap.add_argument('--no-cpu-baseline', action='store_true', help='skip the CPU oracle leg (profiling runs)')
    ap.add_argument('--equal-runs', action='store_true',
                    help='verification plans with equal runs on every XCD (no XCD speed calibration)')
    ap.add_argument('--traffic-summary', nargs=2, metavar=('FETCH_DIR', 'WRITE_DIR'),
                    help='turn the FETCH_SIZE and WRITE_SIZE passes of --traffic-probe into profiles/*_traffic.json')
    ap.add_argument('--trace-merge', nargs='+', metavar='JSON',
                    help='merge --trace-summary outputs of separate sets of processes (same kernel sources) into '
                         'profiles/attn_64req_kernel_trace.json, each process tagged with its set')
    ap.add_argument('--trace-summary', nargs='+', metavar='DIR:LOG',
                    help='turn rocprofv3 --kernel-trace runs of the plain bench command (each a trace directory and '
                         'the bench line its process printed) into profiles/attn_64req_kernel_trace.json')
    ap.add_argument('--layer-summary', nargs='+', metavar='DIR:LOG',
                    help='per-layer verification kernel durations from rocprofv3 --kernel-trace runs of the plain '
                         'bench command (each a trace directory and the bench line its process printed)')
    ap.add_argument('--traffic-probe', action='store_true',
                    help='untimed run for hardware-counter passes: 3 verification-attention and 3 draft-attention '
                         'layers of the workload, then a 1 GiB device-to-device copy as the counter calibration')
    ap.add_argument('--stream-probe', action='store_true',
                    help='only measure the streaming-read ceiling (dspark_stream_read over 16 GiB, default and '
                         'non-temporal loads, 512-2048 workgroups)')
    ap.add_argument('--xcd-ab', action='store_true',
                    help='only compare verification plans with equal runs and with XCD-calibrated runs on one store '
                         '(alternating transactions of 28 layers), and report the measured XCD speeds')
    ap.add_argument('--timeline', action='store_true',
                    help='per-workgroup phase timeline of the draft attention on the workload, from the timeline '
                         'build of the library (clock stamps per segment: start, first loads issued, first stage '
                         'landed, stream end, merge + write end), summarised per call')
    ap.add_argument('--skew-sweep', action='store_true',
                    help='only time the draft attention of the workload with V placed at increasing distances '
                         'after K in one allocation (the kv_pair skew), alternating rounds on one pool')
    ap.add_argument('--verify-timeline', action='store_true',
                    help='per-workgroup start and end of the verification attention on the workload (timeline '
                         'build), for the XCD-calibrated and the equal-run plan: the spread of workgroup end times '
                         'that bounds the call, per XCD and per workgroup stream rate')
    ap.add_argument('--graph-ab', action='store_true',
                    help='only compare the captured 28-layer verification round with the same 28 eager calls on one '
                         'store: alternating blocks, each behind the same queued GPU work, outputs bitwise equal')
    ap.add_argument('--mfma-probe', action='store_true',
                    help='only run the draft kernels for a rocprofv3 --pmc MfmaUtil MfmaFlopsBF16 pass')
    ap.add_argument('--cpu-verify-layers', type=int, default=VERIFY_LAYERS, help='verify layers in the CPU sample')
    ap.add_argument('--cpu-draft-layers', type=int, default=DRAFT_LAYERS, help='draft layers in the CPU sample')
    return ap.parse_args()


def workload(steps_total):
    """Seeded integer draws: contexts, draft blocks/anchors, accepted prefixes."""
    import numpy as np
    rng = np.random.default_rng(SEED)
    contexts = np.floor(np.exp(rng.uniform(math.log(256), math.log(8192), size=B))).astype(int)
    # leave room for every round's commit (<= 7 rows per round)
    contexts = np.minimum(contexts, CAPACITY - Q_LEN * (steps_total + 1))
    blocks = rng.integers(1, 9, size=B)
    anchors = []
    for c, n in zip(contexts, blocks):
        a = [int(c)] + [int(x) for x in rng.integers(0, c + 1, size=n - 1)]
        anchors.append(a)
    accepted = rng.integers(0, Q_LEN + 1, size=(steps_total, B))
    return [int(c) for c in contexts], anchors, accepted


def grown_contexts(contexts, accepted):
    """Context lengths after every round of `accepted` has committed: those
    the instrumented rounds (and so the per-call figures) run at."""
    return [int(c) + int(n) for c, n in zip(contexts, accepted.sum(axis=0))]


def verify_bytes(contexts):
    """Algorithmic HBM bytes of one verification-attention layer: every key
    row (committed + staged) read once, Q read once, O written once."""
    return sum(c + Q_LEN for c in contexts) * 2 * ROW_BYTES + 2 * B * Q_LEN * Q_ROW_BYTES


def verify_store(args, dev, layers=VERIFY_LAYERS, calibrate=True):
    """The workload's resident store (seeded N(0,1) K/V, every request at
    its context length), its bucket and the round's Q and new K/V rows."""
    import torch

    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV
    contexts, _, _ = workload(args.warmup + args.steps)
    gen = torch.Generator(device=dev).manual_seed(SEED)
    pool = PersistentTargetKV(layers=layers, slots=B, context_capacity=CAPACITY, max_query_tokens=B * Q_LEN,
                              heads=8, dim=128, device=dev)
    handles = [pool.add_request(f'req{i}') for i in range(B)]
    for layer in range(layers):
        pool.keys[layer].normal_(generator=gen)
        pool.values[layer].normal_(generator=gen)
    for h, c in zip(handles, contexts):
        pool.load_prefix(h, pool.keys[:, h.index, :c], pool.values[:, h.index, :c])
    bucket = Bucket((Q_LEN,) * B, (CAPACITY - Q_LEN,) * B, '64-request stress shape')
    pool.register_bucket(bucket)
    if calibrate and not args.equal_runs:
        pool.calibrate_xcd()
    qv = torch.randn(layers, B * Q_LEN, 16, 128, generator=gen, device=dev).to(torch.bfloat16)
    kn = torch.randn(layers, B * Q_LEN, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
    vn = torch.randn(layers, B * Q_LEN, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
    return pool, handles, bucket, contexts, qv, kn, vn


def plan_ab(pool, handles, bucket, qv, kn, vn, speed, rounds=8):
    """Verification calls under three plans on the same store, alternating
    rounds of 28 calls; median per call.  The timed rounds use
    `xcd_calibrated` (what `roofline` reports): runs sized to the calibrated
    XCD speeds, the second resident workgroup of each CU given
    schedule.SECOND_SLOT_SHARE of a run's cost.  `equal_runs` drops the XCD
    speeds, `no_slot_share` the second-slot share."""
    import numpy as np
    import torch
    out = torch.empty_like(qv)
    plans = {'equal_runs': (None, True), 'xcd_calibrated': (speed, True), 'no_slot_share': (speed, False)}
    if speed is None:
        plans = {'xcd_calibrated': (None, True), 'no_slot_share': (None, False)}
    times = {n: [] for n in plans}
    names = list(plans)
    for r in range(rounds + 1):
        for name in (names if r % 2 == 0 else names[::-1]):
            pool.set_xcd_speed(plans[name][0])
            pool.set_slot_balance(plans[name][1])
            tx = pool.begin(handles, bucket)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for layer in range(VERIFY_LAYERS):
                pool.attend(tx, layer, qv[layer], keys=kn[layer], values=vn[layer], out=out[layer])
            e1.record()
            pool.abort(tx)
            if r >= 1:
                times[name].append((e0, e1))
    torch.cuda.synchronize()
    pool.set_xcd_speed(speed)
    pool.set_slot_balance(True)
    return {n + '_call_ms': round(float(np.median([a.elapsed_time(b) for a, b in t])) / VERIFY_LAYERS, 5)
            for n, t in times.items()}


def graph_vs_eager(pool, handles, bucket, contexts, qv, kn, vn, rounds=14):
    """The captured verification round (VerificationGraph: 28 fused layers in
    one HIP graph) against the same 28 eager calls on one store and one
    transaction plan: blocks alternate, each behind the same queued GPU work
    (a 64 MiB copy, so the host's submission never shows), event-timed on
    the launch stream; median per layer.  Replay outputs must equal the
    eager outputs bit for bit."""
    import numpy as np
    import torch

    from qwen3_dspark_amd.graph import VerificationGraph
    dev = pool.device
    graph = VerificationGraph(pool, bucket).capture()
    graph.query.copy_(qv)
    graph.keys.copy_(kn)
    graph.values.copy_(vn)
    out = torch.empty_like(qv)
    pad = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    pad_src = torch.empty_like(pad)
    times = {'eager': [], 'graph': []}
    same = True
    for r in range(rounds + 2):
        for kind in (('eager', 'graph') if r % 2 == 0 else ('graph', 'eager')):
            tx = pool.begin(handles, bucket)
            pad.copy_(pad_src)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            if kind == 'eager':
                for layer in range(VERIFY_LAYERS):
                    pool.attend(tx, layer, qv[layer], keys=kn[layer], values=vn[layer], out=out[layer])
                e1.record()
                e1.synchronize()
            else:
                done = graph.submit(tx)
                e1.record()
                graph.wait(done)
                same = same and torch.equal(graph.output, out)
            pool.abort(tx)
            if r >= 2:
                times[kind].append(e0.elapsed_time(e1) / VERIFY_LAYERS)
    res = {'layers': VERIFY_LAYERS, 'rounds': rounds, 'bit_identical_to_eager': bool(same)}
    for kind, t in times.items():
        ms = float(np.median(t))
        res[kind] = {'per_layer_ms': round(ms, 5), 'p10_ms': round(float(np.percentile(t, 10)), 5),
                     'p90_ms': round(float(np.percentile(t, 90)), 5),
                     'gbs': round(verify_bytes(contexts) / ms / 1e6, 1)}
        log(f'[graph-ab] {kind}: {ms * 1e3:.1f} us per layer')
    res['replay_over_eager'] = round(res['graph']['per_layer_ms'] / res['eager']['per_layer_ms'], 4)
    return res


def graph_ab(args):
    """--graph-ab: graph_vs_eager on the workload's first round (run it
    under a kernel trace to compare the kernels' durations and gaps)."""
    import torch
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    pool, handles, bucket, contexts, qv, kn, vn = verify_store(args, dev)
    print(json.dumps({'graph_ab': graph_vs_eager(pool, handles, bucket, contexts, qv, kn, vn)}), flush=True)


def xcd_ab(args, rounds=14):
    """Verification attention of the first round of the workload on one
    28-layer store: transactions planned with equal runs and with runs sized
    to the XCD speeds calibrate_xcd measures, alternating, median per call."""
    import numpy as np
    import torch

    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    contexts, _, _ = workload(args.warmup + args.steps)
    gen = torch.Generator(device=dev).manual_seed(SEED)
    pool = PersistentTargetKV(layers=VERIFY_LAYERS, slots=B, context_capacity=CAPACITY, max_query_tokens=B * Q_LEN,
                              heads=8, dim=128, device=dev)
    handles = [pool.add_request(f'req{i}') for i in range(B)]
    for layer in range(VERIFY_LAYERS):
        pool.keys[layer].normal_(generator=gen)
        pool.values[layer].normal_(generator=gen)
    for h, c in zip(handles, contexts):
        pool.load_prefix(h, pool.keys[:, h.index, :c], pool.values[:, h.index, :c])
    bucket = Bucket((Q_LEN,) * B, (CAPACITY - Q_LEN,) * B, '64-request stress shape')
    pool.register_bucket(bucket)
    speed = pool.calibrate_xcd()
    qv = torch.randn(VERIFY_LAYERS, B * Q_LEN, 16, 128, generator=gen, device=dev).to(torch.bfloat16)
    kn = torch.randn(VERIFY_LAYERS, B * Q_LEN, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
    vn = torch.randn(VERIFY_LAYERS, B * Q_LEN, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
    out = torch.empty_like(qv)
    plans = {'equal': None, 'calibrated': speed}
    times = {n: [] for n in plans}
    for r in range(rounds):
        for name in (('equal', 'calibrated') if r % 2 == 0 else ('calibrated', 'equal')):
            pool.set_xcd_speed(plans[name])
            tx = pool.begin(handles, bucket)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for layer in range(VERIFY_LAYERS):
                pool.attend(tx, layer, qv[layer], keys=kn[layer], values=vn[layer], out=out[layer])
            e1.record()
            pool.abort(tx)
            if r >= 2:
                times[name].append((e0, e1))
    torch.cuda.synchronize()
    res = {'xcd_speed': [round(x, 4) for x in speed], 'rounds': rounds - 2, 'calls_per_round': VERIFY_LAYERS}
    for name in plans:
        us = np.array([a.elapsed_time(b) / VERIFY_LAYERS for a, b in times[name]]) * 1e3
        res[name] = {'median_us': round(float(np.median(us)), 2), 'p10_us': round(float(np.percentile(us, 10)), 2),
                     'p90_us': round(float(np.percentile(us, 90)), 2)}
    print(json.dumps({'xcd_ab': res}), flush=True)


def draft_bytes(anchors):
    """Algorithmic bytes of one draft-attention layer: context rows up to the
    largest anchor read once per request, block K/V, Q and O."""
    rows = sum(max(a) for a in anchors)
    q = BLOCK * sum(len(a) for a in anchors)
    return rows * 2 * ROW_BYTES + q * 2 * ROW_BYTES + 2 * q * Q_ROW_BYTES


def main():
    args = parse()
    world = int(os.environ.get('WORLD_SIZE', '1'))
    if args.gpus != 1 or world != 1:
        print(json.dumps({'error': 'bench.py measures one GPU only; the attention path has no cross-GPU '
                                   'exchange (requests would shard across GPUs); run with --gpus 1'}))
        sys.exit(2)
    if args.traffic_summary:
        return traffic_summary(args, *args.traffic_summary)
    if args.trace_summary:
        return trace_summary(args.trace_summary)
    if args.trace_merge:
        return trace_merge(args.trace_merge)
    if args.layer_summary:
        return layer_summary(args.layer_summary)
    if args.traffic_probe:
        return traffic_probe(args)
    if args.mfma_probe:
        return mfma_probe(args)
    if args.timeline:
        return timeline_probe(args)
    if args.verify_timeline:
        return verify_timeline_probe(args)
    if args.skew_sweep:
        return skew_sweep(args)
    if args.draft_ab:
        return draft_ab(args)
    if args.graph_ab:
        return graph_ab(args)
    if args.xcd_ab:
        return xcd_ab(args)
    if args.stream_probe:
        return stream_probe()
    import numpy as np
    import torch

    from qwen3_dspark_amd.draft import DraftBatch, HipDraftAttention
    from qwen3_dspark_amd.kernels import DEFAULT_CHUNK, SCALE
    from qwen3_dspark_amd.schedule import DRAFT_CHUNK
    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV

    chunk = args.chunk or DEFAULT_CHUNK
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    steps_total = args.warmup + args.steps
    contexts, anchors, accepted = workload(steps_total)
    log(f'[bench] contexts sum={sum(contexts)} min={min(contexts)} max={max(contexts)}; '
        f'draft blocks={sum(len(a) for a in anchors)}')

    gen = torch.Generator(device=dev).manual_seed(SEED)
    # -- target store: resident [28, 64, 8192, 8, 128] K and V --------------
    pool = PersistentTargetKV(layers=VERIFY_LAYERS, slots=B, context_capacity=CAPACITY,
                              max_query_tokens=B * Q_LEN, heads=8, dim=128, device=dev, chunk=chunk)
    handles = [pool.add_request(f'req{i}') for i in range(B)]
    for layer in range(VERIFY_LAYERS):
        pool.keys[layer].normal_(generator=gen)
        pool.values[layer].normal_(generator=gen)
    for h, c in zip(handles, contexts):
        # the resident rows already hold the seeded prefix; adopt them in place
        pool.load_prefix(h, pool.keys[:, h.index, :c], pool.values[:, h.index, :c])
    bucket = Bucket((Q_LEN,) * B, (CAPACITY - Q_LEN,) * B, '64-request stress shape')
    pool.register_bucket(bucket)
    # XCD-balanced plans: measure once, at set-up, how fast each XCD reads the
    # store (as a server would at start-up); later plans size each XCD's runs.
    xcd_speed = pool.calibrate_xcd() if not args.equal_runs else None
    log(f'[bench] XCD speeds: {None if xcd_speed is None else [round(x, 3) for x in xcd_speed]}')
    qv = torch.randn(VERIFY_LAYERS, B * Q_LEN, 16, 128, generator=gen, device=dev).to(torch.bfloat16)
    kn = torch.randn(VERIFY_LAYERS, B * Q_LEN, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
    vn = torch.randn(VERIFY_LAYERS, B * Q_LEN, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
    # -- draft: head-major slotted context pool [5, 64, 8, 8192, 128] ----
    from qwen3_dspark_amd._device import kv_pair
    # one allocation, V 32 MiB after K, as DraftKVPool lays its pool out (kv_pair)
    dctx_k, dctx_v = kv_pair((DRAFT_LAYERS, B, 8, CAPACITY, 128), torch.bfloat16, torch.bfloat16, dev)
    for layer in range(DRAFT_LAYERS):
        dctx_k[layer].normal_(generator=gen)
        dctx_v[layer].normal_(generator=gen)
    nq_d = BLOCK * sum(len(a) for a in anchors)
    qd = torch.randn(DRAFT_LAYERS, nq_d, 16, 128, generator=gen, device=dev).to(torch.bfloat16)
    bkd = torch.randn(DRAFT_LAYERS, nq_d, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
    bvd = torch.randn(DRAFT_LAYERS, nq_d, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
    draft = HipDraftAttention(dev, chunk=args.draft_chunk or DRAFT_CHUNK, **draft_modes(args.draft_persistent))
    draft_offsets = [h.index * CAPACITY for h in handles]   # slot * capacity + first position
    torch.cuda.synchronize()

    ev_v = []
    ev_d = []
    step_stats = []

    def events():
        return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def round_(step, instrument=False):
        """One speculative round.  Plain rounds commit the round's accepted
        prefixes.  Instrumented rounds (the per-phase breakdown) put event
        pairs around the draft calls and around the verification calls and
        roll back instead of committing, so that the contexts stay those the
        timed rounds reached: every event marker costs the launch stream a
        few us, so the timed rounds carry none."""
        ctx_now = [pool.length(h) for h in handles]
        batch = DraftBatch(dev, draft_offsets, contexts, anchors)
        draft.plan(batch, dctx_k[0])      # the round's draft plan, prepared like begin() for verification
        outs = []
        if instrument:
            d0, d1 = events()
            d0.record()
        for layer in range(DRAFT_LAYERS):
            outs.append(draft(qd[layer], bkd[layer], bvd[layer], dctx_k[layer], dctx_v[layer], batch, scale=SCALE))
        if instrument:
            d1.record()
            ev_d.append((d0, d1))
        tx = pool.begin(handles, bucket)
        if instrument:
            v0, v1 = events()
            v0.record()
        for layer in range(VERIFY_LAYERS):
            # stage_layer fused into the attention launch (scratch is written
            # by the kernel that reads the new rows)
            outs.append(pool.attend(tx, layer, qv[layer], keys=kn[layer], values=vn[layer]))
        if instrument:
            v1.record()
            ev_v.append((v0, v1, verify_bytes(ctx_now)))
            pool.abort(tx)
            return outs
        counts = [int(x) for x in accepted[step]]
        pool.commit(tx, dict(zip(handles, counts)))
        step_stats.append((ctx_now, counts))
        return outs

    # Like a long-running server after start-up: move the set-up objects
    # out of the cyclic collector's reach, so that a full collection during
    # the rounds (tens of ms over torch/numpy internals) does not stall the
    # launch stream.  The collector stays enabled.
    gc.collect()
    gc.freeze()
    log(f'[bench] warmup {args.warmup} steps')
    for s in range(args.warmup):
        round_(s)
    torch.cuda.synchronize()
    log(f'[bench] timing {args.steps} steps')
    step_stats.clear()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.warmup, steps_total):
        round_(s)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_step = 1e3 * elapsed / args.steps
    log(f'[bench] {args.steps} instrumented steps (per-phase events, rolled back)')
    for s in range(args.steps):
        round_(s, instrument=True)
    torch.cuda.synchronize()

    v_ms = np.array([a.elapsed_time(b) / VERIFY_LAYERS for a, b, _ in ev_v])
    v_bytes = np.array([n for _, _, n in ev_v], dtype=np.float64)
    d_ms = np.array([a.elapsed_time(b) / DRAFT_LAYERS for a, b in ev_d])
    v_avg_ms = float(v_ms.mean())
    v_avg_bytes = float(v_bytes.mean())
    d_avg_ms = float(d_ms.mean())

    def pct(x, calls):
        # percentiles over rounds of the per-call average of each round
        return {'p10': round(float(np.percentile(x, 10)), 5), 'median': round(float(np.median(x)), 5),
                'p90': round(float(np.percentile(x, 90)), 5), 'rounds': int(len(x)), 'calls_per_round': calls}
    d_b = draft_bytes(anchors)
    v_gbs = v_avg_bytes / (v_avg_ms * 1e-3) / 1e9
    d_gbs = d_b / (d_avg_ms * 1e-3) / 1e9
    round_bytes = sum(VERIFY_LAYERS * verify_bytes(c) + DRAFT_LAYERS * d_b
                      + VERIFY_LAYERS * 2 * B * Q_LEN * ROW_BYTES         # stage: scratch write of new K/V rows
                      + VERIFY_LAYERS * 2 * sum(n) * ROW_BYTES * 2       # commit: read + write accepted rows
                      for c, n in step_stats) / len(step_stats)
    round_gbs = round_bytes / (ms_step * 1e-3) / 1e9
    value = B * Q_LEN / (ms_step * 1e-3)

    # HBM bytes per call from the two counter passes of --traffic-probe
    # (FETCH_SIZE, WRITE_SIZE, calibrated against a plain 1 GiB copy), for
    # the first round of this workload; summarised in profiles/.
    # Figures measured on older kernel sources are withheld (None) and flagged.
    def counted(name):
        tpath = os.path.join(ROOT, 'profiles', name)
        if not os.path.exists(tpath):
            return None, None, None
        with open(tpath) as f:
            tj = json.load(f)
        if tj.get('kernel_source_sha256') != kernel_source_hash():
            return None, None, 'stale: measured on other kernel sources'
        return tj.get('hbm_bytes_per_launch'), tj.get('ratio'), tj.get('algorithmic_bytes_per_launch')
    traffic, traffic_ratio, traffic_round = counted('verify_attn_traffic.json')
    profiled = None
    tpath = os.path.join(ROOT, 'profiles', 'attn_64req_kernel_trace.json')
    if os.path.exists(tpath):
        with open(tpath) as f:
            tj = json.load(f)
        profiled = ({'source': 'profiles/attn_64req_kernel_trace.json', 'processes': len(tj['processes']),
                     'verify_frac_from_kernels_range': tj['verify_frac_from_kernels_range'],
                     'draft_frac_from_kernels_range': tj['draft_frac_from_kernels_range']}
                    if tj.get('kernel_source_sha256') == kernel_source_hash()
                    else 'stale: traced on other kernel sources')
    d_traffic, d_traffic_ratio, d_traffic_round = counted('draft_attn_traffic.json')

    result = {
        'metric': METRIC, 'value': round(value, 1), 'unit': 'tokens/s', 'n_gpus': 1,
        'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': round(ms_step, 4),
        'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'bf16',
        'data': 'synthetic (seeded N(0,1) bf16 Q/K/V resident in HBM)',
        'config': {
            'workload': 'one speculative round: 5 draft attention layers + 28 verify attention layers '
                        '(stage + KV gather + attention fused in one kernel) + commit/rollback, 64 ragged requests, '
                        'contexts log-uniform [256, 8192], KV capacity 8192 per request, 16q/8kv heads, d128',
            'requests': B, 'query_rows_per_request': Q_LEN, 'verify_layers': VERIFY_LAYERS,
            'draft_layers': DRAFT_LAYERS, 'draft_blocks': sum(len(a) for a in anchors),
            'context_rows': sum(contexts), 'chunk': chunk, 'draft_chunk': draft.chunk,
        },
        'roofline': {
            'bound': 'hbm', 'achieved': round(v_gbs, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
            'frac': round(v_gbs / HBM_PEAK_GBS, 4), 'traffic': traffic, 'traffic_per_algorithmic_byte': traffic_ratio,
            'traffic_round_algorithmic_bytes': traffic_round,
            'kernel': 'fused verification attention: varlen_attn_kernel<true> + merge_kernel',
            'avg_launch_ms': round(v_avg_ms, 5), 'algorithmic_bytes_per_launch': int(v_avg_bytes),
            'profiled': profiled,
        },
        'breakdown': {
            'per_call_timing': f'{args.steps} instrumented rounds after the timed ones (event pairs around the '
                               'draft and the verification calls, rolled back); the timed rounds carry no events',
            'verify_layer_ms': round(v_avg_ms, 5), 'verify_call_ms': pct(v_ms, VERIFY_LAYERS), 'verify_gbs': round(v_gbs, 1),
            'verify_attn_tokens_per_s': round(B * Q_LEN / (float(np.median(v_ms)) * 1e-3), 1),
            'draft_layer_ms': round(d_avg_ms, 5), 'draft_call_ms': pct(d_ms, DRAFT_LAYERS), 'draft_gbs': round(d_gbs, 1),
            'draft_frac': round(d_gbs / HBM_PEAK_GBS, 4),
            'draft_algorithmic_bytes_per_launch': int(d_b), 'draft_traffic': d_traffic,
            'draft_traffic_per_algorithmic_byte': d_traffic_ratio, 'draft_traffic_round_algorithmic_bytes': d_traffic_round,
            'draft_attn_tokens_per_s': round(nq_d / (float(np.median(d_ms)) * 1e-3), 1),
            'round_algorithmic_bytes': int(round_bytes), 'round_gbs': round(round_gbs, 1),
            'round_frac': round(round_gbs / HBM_PEAK_GBS, 4),
            'xcd_speed': None if xcd_speed is None else [round(x, 4) for x in xcd_speed],
        },
    }

    result['breakdown']['verify_plans'] = plan_ab(pool, handles, bucket, qv, kn, vn, xcd_speed)
    result['next'] = {'verify_graph': graph_vs_eager(pool, handles, bucket, [pool.length(h) for h in handles],
                                                     qv, kn, vn),
                      'qkv_prologue': prologue_leg(dev, B * Q_LEN),
                      'draft_context_projection': [draft_projection_leg(dev, B, Q_LEN),
                                                   draft_projection_leg(dev, 16, None)],
                      'lm_head_and_verification': sampling_leg(dev, args.no_cpu_baseline)}
    result['gpu_configs'] = gpu_configs(dev)

    if not args.no_cpu_baseline:
        result['cpu_baseline'], result['parity'] = cpu_leg(args, pool, bucket, handles, contexts, anchors, qv, qd,
                                                           bkd, bvd, dctx_k, dctx_v, draft, draft_offsets)
        result['cpu_configs'] = cpu_configs(result['cpu_baseline']['cores'])
    print(json.dumps(result), flush=True)


_PAD = {}


def queue_ahead(dev, copies=8):
    """Queue `copies` 1 GiB device copies (~0.4 ms each) on the current
    stream, so that the host enqueues the launches that follow while the GPU
    is still busy and then runs them back to back, as inside a round: a
    kernel launched onto an idle GPU runs several microseconds longer
    (measured: +6 us for a 10 us kernel), which per-call host timing loops
    would otherwise add to every launch."""
    import torch
    if dev not in _PAD:
        _PAD[dev] = (torch.empty(1 << 30, dtype=torch.uint8, device=dev), torch.empty(1 << 30, dtype=torch.uint8,
                                                                                     device=dev))
    dst, src = _PAD[dev]
    for _ in range(copies):
        dst.copy_(src)


def prologue_leg(dev, tokens, reps=50):
    """The verify-layer prologue (q/k/v projection + q/k RMSNorm + RoPE, K/V
    written token-major as into scratch) for one layer of the round's
    tokens, Qwen3-0.6B sizes (hidden 1024), random-init weights, fed the
    transaction's rotary table as PersistentTargetKV.stage_projected does
    (one dspark_rope_table launch per transaction, shared by the 28 layers;
    timed on its own).  Medians of `reps` event-timed launches, queued back
    to back behind GPU work."""
    import numpy as np
    import torch

    from qwen3_dspark_amd.prologue import QKVPrologue
    g = torch.Generator(device=dev).manual_seed(SEED + 7)
    w = [(torch.randn(n, 1024, generator=g, device=dev) * 0.03).to(torch.bfloat16) for n in (2048, 1024, 1024)]
    norms = [torch.ones(128, device=dev, dtype=torch.bfloat16) for _ in range(2)]
    pro = QKVPrologue(*w, *norms)
    x = torch.randn(tokens, 1024, generator=g, device=dev).to(torch.bfloat16)
    pos = torch.arange(tokens, device=dev, dtype=torch.long) * 13
    table = pro.rope_table(pos)
    for _ in range(5):
        pro(x, pos, rope=table)

    def timed(fn):
        times = []
        queue_ahead(dev)
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            times.append((e0, e1))
        torch.cuda.synchronize()
        return float(np.median([a.elapsed_time(b) for a, b in times]))

    ms = timed(lambda: pro(x, pos, rope=table))
    table_ms = timed(lambda: pro.rope_table(pos))
    nbytes = (4096 * 1024 + tokens * 1024 + tokens * 4096) * 2
    flops = 2 * tokens * 1024 * 4096
    return {'tokens': tokens, 'median_ms': round(ms, 5), 'bytes': nbytes, 'gbs': round(nbytes / ms / 1e6, 1),
            'tflops': round(flops / ms / 1e9, 2), 'rope_table_ms_per_transaction': round(table_ms, 5)}


def sampling_leg(dev, skip_cpu, reps=10):
    """The consumer of a verification round: the LM head over each request's
    7 + 1 verified rows (hidden 1024, vocab 151,936, random-init bf16,
    hipBLASLt), then float64 speculative verification of 7 proposed tokens
    per request against draft laws (temperature 0.8): row statistics + one
    verification launch.  Median of `reps` event-timed rounds; the float64
    numpy oracle on the host timed on the same logits (one round) unless
    skipped, and every integer outcome compared with it."""
    import numpy as np
    import torch

    from oracle import sampling as oracle
    from qwen3_dspark_amd.sampling import TargetHead, logits_to_probabilities, sample_categorical, verify_proposals
    V, H, R, N, T = 151936, 1024, B, Q_LEN, 0.8
    g = torch.Generator(device=dev).manual_seed(SEED + 21)
    head = TargetHead((torch.randn(V, H, generator=g, device=dev) * 0.05).to(torch.bfloat16))
    hidden = torch.randn(R * (N + 1), H, generator=g, device=dev).to(torch.bfloat16)
    logits = head(hidden)
    rows = torch.arange(R * (N + 1), device=dev).reshape(R, N + 1)[:, :N].reshape(-1)
    q = logits_to_probabilities(logits[rows].float() + torch.randn(R * N, V, generator=g, device=dev), T)
    tokens = sample_categorical(q, torch.rand(R * N, generator=g, device=dev, dtype=torch.float64))
    uniforms = torch.rand(R * (N + 1), generator=g, device=dev, dtype=torch.float64)
    budgets = [64] * R
    for _ in range(2):
        verify_proposals(head(hidden), tokens, q, uniforms, counts=[N] * R, temperature=T, max_new_tokens=budgets)
    t_head, t_ver = [], []
    for _ in range(reps):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record()
        logits = head(hidden)
        e[1].record()
        got = verify_proposals(logits, tokens, q, uniforms, counts=[N] * R, temperature=T, max_new_tokens=budgets)
        e[2].record()
        torch.cuda.synchronize()
        t_head.append(e[0].elapsed_time(e[1]))
        t_ver.append(e[1].elapsed_time(e[2]))
    ms_head, ms_ver = float(np.median(t_head)), float(np.median(t_ver))
    out = {'requests': R, 'rows': R * (N + 1), 'vocab': V,
           'lm_head_ms': round(ms_head, 4), 'lm_head_tflops': round(2 * R * (N + 1) * H * V / ms_head / 1e9, 1),
           'verify_ms': round(ms_ver, 4),
           'verify_logit_gbs': round(logits.numel() * 2 / ms_ver / 1e6, 1),
           'accepted_draft_tokens': sum(r.accepted_draft_tokens for r in got),
           'emitted_tokens': sum(int(r.tokens.numel()) for r in got),
           'rounds_per_s': round(1e3 / (ms_head + ms_ver), 1)}
    if not skip_cpu:
        p_in = logits.float().cpu().numpy()
        q_h, t_h, u_h = q.cpu().numpy(), tokens.cpu().numpy(), uniforms.cpu().numpy()
        t0 = time.perf_counter()
        p_h = oracle.logits_to_probabilities(p_in, T)
        ref = [oracle.verify_proposal(t_h[N * r:N * r + N], q_h[N * r:N * r + N], p_h[(N + 1) * r:(N + 1) * (r + 1)],
                                      u_h[(N + 1) * r:(N + 1) * (r + 1)], max_new_tokens=64) for r in range(R)]
        cpu_s = time.perf_counter() - t0
        same = all((tuple(x.tokens.tolist()), x.accepted_draft_tokens, x.rejected_index, x.extra_token_kind,
                    x.stop_reason, x.draws) == (y.tokens, y.accepted_draft_tokens, y.rejected_index,
                                                y.extra_token_kind, y.stop_reason, y.draws) for x, y in zip(got, ref))
        out.update(cpu_oracle_verify_ms=round(cpu_s * 1e3, 1), identical_to_oracle=bool(same))
    return out


def draft_projection_leg(dev, n_req, per_request, reps=20):
    """Draft context projection (fc on hipBLASLt, then for 5 draft layers the
    context norm / k_proj / k_norm / RoPE / v_proj written into a slotted
    pool: one fused launch for short appends, a hipBLASLt GEMM plus the
    epilogue launch from GEMM_MIN_TOKENS rows on) for one append: n_req
    requests of `per_request` rows each
    (a round's committed rows), or, with per_request None, the 16-request
    prefill of contexts U[128, 1024].  Random-init bf16 weights (hidden
    1024, features 5 x 1024).  Median of `reps` event-timed appends of each
    part, queued back to back behind GPU work on the pool's stream."""
    import numpy as np
    import torch

    from qwen3_dspark_amd.draft_projection import GEMM_MIN_TOKENS, DraftContextProjector
    from qwen3_dspark_amd._device import upload
    g = torch.Generator(device=dev).manual_seed(SEED + 11)
    h, f = 1024, 5 * 1024
    fc = (torch.randn(h, f, generator=g, device=dev) * f ** -0.5).to(torch.bfloat16)
    cn = torch.ones(h, device=dev, dtype=torch.bfloat16)
    layers = [((torch.randn(1024, h, generator=g, device=dev) * h ** -0.5).to(torch.bfloat16),
               torch.ones(128, device=dev, dtype=torch.bfloat16),
               (torch.randn(1024, h, generator=g, device=dev) * h ** -0.5).to(torch.bfloat16)) for _ in range(5)]
    proj = DraftContextProjector(fc, cn, layers)
    rng = np.random.default_rng(SEED + 11)
    counts = [per_request] * n_req if per_request else [int(c) for c in rng.integers(128, 1025, size=n_req)]
    cap = max(counts) + 1
    keys = torch.empty(5, n_req, 8, cap, 128, dtype=torch.bfloat16, device=dev)
    values = torch.empty_like(keys)
    rec, first = [], 0
    for i, n in enumerate(counts):
        rec += (i, 0, first, n)
        first += n
    records = upload(dev, rec)
    x = torch.randn(first, f, generator=g, device=dev).to(torch.bfloat16)
    fc_out = proj.fc_forward(x)
    for _ in range(3):
        proj.project_into(proj.fc_forward(x), records, n_req, keys, values)
    t_fc, t_kv = [], []
    queue_ahead(dev)
    for _ in range(reps):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record()
        fc_out = proj.fc_forward(x)
        e[1].record()
        proj.project_into(fc_out, records, n_req, keys, values)
        e[2].record()
        t_fc.append((e[0], e[1]))
        t_kv.append((e[1], e[2]))
    torch.cuda.synchronize()
    ms_fc = float(np.median([a.elapsed_time(b) for a, b in t_fc]))
    ms_kv = float(np.median([a.elapsed_time(b) for a, b in t_kv]))
    fc_bytes = (h * f + first * f + first * h) * 2
    fc_flops = 2 * first * f * h
    kv_bytes = (5 * 2 * 1024 * h + first * h + 5 * 2 * first * 1024) * 2
    kv_flops = 2 * first * h * 5 * 2 * 1024
    return {'tokens': first, 'requests': n_req,
            'kv_path': 'hipblaslt_gemm+epilogue' if first >= GEMM_MIN_TOKENS else 'fused',
            'fc_hipblaslt_ms': round(ms_fc, 5), 'fc_tflops': round(fc_flops / ms_fc / 1e9, 1),
            'kv_project_ms': round(ms_kv, 5), 'kv_project_tflops': round(kv_flops / ms_kv / 1e9, 1),
            'kv_project_gbs': round(kv_bytes / ms_kv / 1e6, 1),
            'append_tokens_per_s': round(first / ((ms_fc + ms_kv) * 1e-3), 1)}


def traffic_probe(args):
    """Kernels for `rocprofv3 --pmc FETCH_SIZE` / `--pmc WRITE_SIZE` passes:
    3 verification-attention launches of the workload at the contexts of the
    instrumented rounds (after the warm-up and timed rounds' commits),
    staging fused in as in the rounds, then 3 draft-attention launches
    (store and pool contents are irrelevant to the bytes moved, so they stay
    zero-filled),
    then a plain copy of exactly 2**30 bytes whose counter reading
    calibrates the counters to bytes."""
    import torch

    from qwen3_dspark_amd.draft import DraftBatch, HipDraftAttention
    from qwen3_dspark_amd.kernels import DEFAULT_CHUNK, SCALE
    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV

    dev = torch.device('cuda:0')
    contexts, anchors, accepted = workload(args.warmup + args.steps)
    grown = grown_contexts(contexts, accepted)
    pool = PersistentTargetKV(layers=3, slots=B, context_capacity=CAPACITY, max_query_tokens=B * Q_LEN,
                              heads=8, dim=128, device=dev, chunk=args.chunk or DEFAULT_CHUNK)
    handles = [pool.add_request(f'req{i}') for i in range(B)]
    for h, c in zip(handles, grown):
        pool.load_prefix(h, pool.keys[:, h.index, :c], pool.values[:, h.index, :c])
    bucket = Bucket((Q_LEN,) * B, (CAPACITY - Q_LEN,) * B, '64-request stress shape')
    pool.register_bucket(bucket)
    if not args.equal_runs:
        pool.calibrate_xcd()          # the plan of the timed rounds
    q = torch.zeros(B * Q_LEN, 16, 128, dtype=torch.bfloat16, device=dev)
    kn = torch.zeros(B * Q_LEN, 8, 128, dtype=torch.bfloat16, device=dev)
    tx = pool.begin(handles, bucket)
    for layer in range(3):
        pool.attend(tx, layer, q, keys=kn, values=kn)
    pool.abort(tx)
    torch.cuda.synchronize()
    del pool
    from qwen3_dspark_amd._device import kv_pair
    ctx_k, ctx_v = kv_pair((B, 8, CAPACITY, 128), torch.bfloat16, torch.bfloat16, dev)
    n_rows = BLOCK * sum(len(a) for a in anchors)
    qd = torch.zeros(n_rows, 16, 128, dtype=torch.bfloat16, device=dev)
    kd = torch.zeros(n_rows, 8, 128, dtype=torch.bfloat16, device=dev)
    batch = DraftBatch(dev, [i * CAPACITY for i in range(B)], contexts, anchors)
    draft = HipDraftAttention(dev)
    for _ in range(3):
        draft(qd, kd, kd, ctx_k, ctx_v, batch, scale=SCALE)
    src = torch.ones(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del ctx_k, ctx_v
    print(json.dumps({'traffic_probe': 'done', 'verify_algorithmic_bytes_per_launch': verify_bytes(grown),
                      'draft_algorithmic_bytes_per_launch': draft_bytes(anchors),
                      'context_rows': sum(grown),
                      'calibration_copy_bytes': 1 << 30,
                      'streaming_reference': streaming_reference(dev, src, dst)}), flush=True)


def draft_modes(arg):
    """HipDraftAttention keyword for the --draft-persistent choice."""
    return {} if arg is None else {'persistent': None if arg == 0 else arg}


def draft_ab(args, rounds=16):
    """The workload's 5 draft layers per round on one pool, rounds
    alternating between the scheduling modes (one workgroup per item
    dispatched by the hardware; persistent workgroups on one queue; on one
    queue per KV head), event-timed on the launch stream; median per call.
    Every mode's outputs must be bitwise equal to the first mode's."""
    import numpy as np
    import torch

    from qwen3_dspark_amd.draft import DraftBatch, HipDraftAttention
    from qwen3_dspark_amd.kernels import SCALE
    from qwen3_dspark_amd.schedule import DRAFT_CHUNK
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    contexts, anchors, _ = workload(args.warmup + args.steps)
    gen = torch.Generator(device=dev).manual_seed(SEED)
    from qwen3_dspark_amd._device import kv_pair
    # one allocation, V 32 MiB after K, as DraftKVPool lays its pool out (kv_pair)
    ctx_k, ctx_v = kv_pair((DRAFT_LAYERS, B, 8, CAPACITY, 128), torch.bfloat16, torch.bfloat16, dev)
    for layer in range(DRAFT_LAYERS):
        ctx_k[layer].normal_(generator=gen)
        ctx_v[layer].normal_(generator=gen)
    nq = BLOCK * sum(len(a) for a in anchors)
    qd = torch.randn(DRAFT_LAYERS, nq, 16, 128, generator=gen, device=dev).to(torch.bfloat16)
    bk = torch.randn(DRAFT_LAYERS, nq, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
    bv = torch.randn(DRAFT_LAYERS, nq, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
    batch = DraftBatch(dev, [i * CAPACITY for i in range(B)], contexts, anchors)
    modes = {'hardware dispatch': None, 'persistent, one queue': 1, 'persistent, queue per KV head': 8}
    kernels = {m: HipDraftAttention(dev, chunk=args.draft_chunk or DRAFT_CHUNK, persistent=p)
               for m, p in modes.items()}
    times = {m: [] for m in modes}
    ref = None
    for r in range(rounds + 2):
        for m, k in kernels.items():
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            outs = [k(qd[l], bk[l], bv[l], ctx_k[l], ctx_v[l], batch, scale=SCALE) for l in range(DRAFT_LAYERS)]
            b.record()
            b.synchronize()
            if r >= 2:
                times[m].append(a.elapsed_time(b) / DRAFT_LAYERS)
            if ref is None:
                ref = [o.clone() for o in outs]
            elif not all(torch.equal(o, x) for o, x in zip(outs, ref)):
                raise AssertionError(f'draft outputs differ under {m}')
    d_b = draft_bytes(anchors)
    res = {}
    for m, t in times.items():
        ms = float(np.median(t))
        res[m] = {'median_ms': round(ms, 5), 'p10_ms': round(float(np.percentile(t, 10)), 5),
                  'p90_ms': round(float(np.percentile(t, 90)), 5), 'gbs': round(d_b / ms / 1e6, 1),
                  'frac_of_8tbs': round(d_b / ms / 1e6 / HBM_PEAK_GBS, 4)}
        log(f'[draft-ab] {m}: {ms * 1e3:.1f} us per call ({res[m]["frac_of_8tbs"]:.3f} of 8 TB/s)')
    print(json.dumps({'draft_ab': res, 'rounds': rounds, 'calls_per_round': DRAFT_LAYERS,
                      'outputs_bitwise_equal': True, 'draft_chunk': args.draft_chunk or DRAFT_CHUNK}), flush=True)


def timeline_probe(args, calls=5, samples=6):
    """Per-workgroup timeline of the draft attention (DSPARK_TIMELINE build
    of the library): the workload's draft layers run back to back, `calls`
    per sample as in a round; the stamps of a sample's last call are read
    after it.  Per call: span from the first segment start to the last
    segment end; per segment the phases start -> first loads issued (record
    and scalar metadata), -> first stage landed (the ring's first HBM
    latency), -> stream end, -> half merge and output written; per CU the
    idle time between one segment's end and the next one's start there, and
    the tail (time from the median to the last segment end).  Medians over
    `samples` samples."""
    os.environ['DSPARK_AMD_TIMELINE'] = '1'
    import numpy as np
    import torch

    from qwen3_dspark_amd import _native
    from qwen3_dspark_amd.draft import DraftBatch, HipDraftAttention
    from qwen3_dspark_amd.kernels import SCALE
    from qwen3_dspark_amd.schedule import DRAFT_CHUNK
    lib = _native.load()
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    contexts, anchors, _ = workload(args.warmup + args.steps)
    gen = torch.Generator(device=dev).manual_seed(SEED)
    from qwen3_dspark_amd._device import kv_pair
    # one allocation, V 32 MiB after K, as DraftKVPool lays its pool out (kv_pair)
    ctx_k, ctx_v = kv_pair((DRAFT_LAYERS, B, 8, CAPACITY, 128), torch.bfloat16, torch.bfloat16, dev)
    for layer in range(DRAFT_LAYERS):
        ctx_k[layer].normal_(generator=gen)
        ctx_v[layer].normal_(generator=gen)
    nq = BLOCK * sum(len(a) for a in anchors)
    qd = torch.randn(nq, 16, 128, generator=gen, device=dev).to(torch.bfloat16)
    bk = torch.randn(nq, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
    bv = torch.randn(nq, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
    draft = HipDraftAttention(dev, chunk=args.draft_chunk or DRAFT_CHUNK, **draft_modes(args.draft_persistent))
    batch = DraftBatch(dev, [i * CAPACITY for i in range(B)], contexts, anchors)
    nbytes = int(lib.dspark_timeline_bytes())
    host = np.zeros(nbytes // 8, dtype=np.uint64)
    tick_us = 0.01                               # the 100 MHz constant clock
    rows = []
    for sample in range(samples + 1):
        for layer in range(calls):
            draft(qd, bk, bv, ctx_k[layer], ctx_v[layer], batch, scale=SCALE)
        _native.call('dspark_timeline_fetch', host.ctypes.data, nbytes)
        wg = np.zeros(8192 * 4, dtype=np.uint64)
        _native.call('dspark_timeline_fetch_wg', wg.ctypes.data, wg.nbytes)
        if sample == 0:
            continue                             # warm-up
        rec = host.reshape(-1, 8)
        slot = np.arange(len(rec)) % 16                     # segment index within its workgroup
        valid = (rec[:, 5] >> np.uint64(63)) == 1
        # Every workgroup's first segment of the last call overwrote slot 0;
        # later slots may still hold segments of earlier calls of the sample.
        start = rec[valid & (slot == 0), 0].min()
        rec = rec[valid & (rec[:, 0] >= start)]
        t = rec[:, :5].astype(np.float64)
        t0 = t[:, 0].min()
        t = (t - t0) * tick_us
        where = (rec[:, 5] & np.uint64(0xffffffff)).astype(np.int64)
        xcc = ((rec[:, 5] >> np.uint64(32)) & np.uint64(15)).astype(np.int64)
        cu = xcc * 1000 + ((where >> 8) & 0xff)           # XCC and the CU/SH/SE bits of HW_ID
        keys = ((rec[:, 6] >> np.uint64(32)) & np.uint64(0xffffffff)).astype(np.int64)
        span = float(t[:, 4].max())
        meta, first, stream, merge = (t[:, 1] - t[:, 0], t[:, 2] - t[:, 1], t[:, 3] - t[:, 2], t[:, 4] - t[:, 3])
        gaps, busy, stream_gaps = [], [], []
        for c in np.unique(cu):
            sel = np.argsort(t[cu == c, 0])
            tc = t[cu == c][sel]
            gaps += list(tc[1:, 0] - tc[:-1, 4])
            # between streams: one segment's stream end to the next one's first stage landed
            stream_gaps += list(tc[1:, 2] - tc[:-1, 3])
            covered, end = 0.0, -np.inf          # union of the CU's [start, written] intervals (they may overlap)
            for a0, a1 in zip(tc[:, 0], tc[:, 4]):
                covered += max(0.0, a1 - max(a0, end))
                end = max(end, a1)
            busy.append(float(covered))
        stream_gbs = keys * 2 * 128 * 2 / np.maximum(stream, 1e-3) * 1e-3     # one KV head: K + V rows
        wg = wg.reshape(-1, 4)
        wg = wg[(wg[:, 3] >> np.uint64(63)) == 1]
        persistent = {}
        if len(wg):
            w = (wg & np.uint64((1 << 63) - 1)).astype(np.float64)
            w = (w - t0) * tick_us
            persistent = dict(wg_entry_min_us=float(w[:, 0].min()), wg_entry_max_us=float(w[:, 0].max()),
                              first_ticket_p50_us=float(np.median(w[:, 1] - w[:, 0])),
                              first_ticket_max_us=float((w[:, 1] - w[:, 0]).max()),
                              loop_left_max_us=float(w[:, 2].max()),
                              exit_protocol_p50_us=float(np.median(w[:, 3] - w[:, 2])),
                              exit_protocol_max_us=float((w[:, 3] - w[:, 2]).max()), exit_max_us=float(w[:, 3].max()))
            log(f'[timeline]   workgroups: entry {persistent["wg_entry_min_us"]:.1f}..{persistent["wg_entry_max_us"]:.1f} us, '
                f'first ticket p50 {persistent["first_ticket_p50_us"]:.2f} max {persistent["first_ticket_max_us"]:.2f} us, '
                f'exit protocol p50 {persistent["exit_protocol_p50_us"]:.2f} max {persistent["exit_protocol_max_us"]:.2f} us, '
                f'last exit {persistent["exit_max_us"]:.1f} us')
        rows.append(dict(
            span_us=span, segments=int(len(t)), cus=int(len(np.unique(cu))),
            segments_per_cu=float(len(t) / len(np.unique(cu))),
            start_to_issue_us=float(np.median(meta)), issue_to_first_stage_us=float(np.median(first)),
            stream_us=float(np.median(stream)), merge_write_us=float(np.median(merge)),
            overhead_per_segment_us=float(np.median(meta + first + merge)),
            cu_gap_median_us=float(np.median(gaps)) if gaps else 0.0,
            stream_gap_median_us=float(np.median(stream_gaps)) if stream_gaps else 0.0,
            stream_gap_p90_us=float(np.percentile(stream_gaps, 90)) if stream_gaps else 0.0,
            cu_gap_p90_us=float(np.percentile(gaps, 90)) if gaps else 0.0,
            cu_busy_frac=float(np.sum(busy) / (span * len(busy))),
            end_p50_us=float(np.median(t[:, 4])), end_p90_us=float(np.percentile(t[:, 4], 90)),
            tail_us=float(span - np.percentile(t[:, 4], 90)),
            first_start_spread_us=float(np.sort(t[:, 0])[min(len(t) - 1, 255)]),
            stream_gbs_per_workgroup_p50=float(np.median(stream_gbs[keys >= 1024])) if (keys >= 1024).any() else 0.0,
            **persistent))
        log(f'[timeline] sample {sample}: span {span:.1f} us, {len(t)} segments on {rows[-1]["cus"]} CUs; '
            f'per segment: issue {rows[-1]["start_to_issue_us"]:.2f}, first stage {rows[-1]["issue_to_first_stage_us"]:.2f}, '
            f'merge+write {rows[-1]["merge_write_us"]:.2f} us; CU gap {rows[-1]["cu_gap_median_us"]:.2f} us; '
            f'stream end to next first stage {rows[-1]["stream_gap_median_us"]:.2f} us; '
            f'busy {rows[-1]["cu_busy_frac"]:.3f}; tail {rows[-1]["tail_us"]:.1f} us')
    summary = {k: round(float(np.median([r[k] for r in rows])), 3) for k in rows[0] if all(k in r for r in rows)}
    print(json.dumps({'timeline': 'draft attention', 'workload': '64 requests, contexts log-uniform [256, 8192], '
                      '1..8 blocks each, 5 draft layers back to back', 'draft_chunk': draft.chunk,
                      'persistent': draft.persistent,
                      'samples': samples, 'median': summary, 'per_sample': rows}), flush=True)


def skew_sweep(args, rounds=14, skews_mib=(0, 2, 4, 6, 8, 12, 16, 20, 24, 28, 32, 40, 48, 64, 96)):
    """Draft attention of the workload (one layer's [64, 8, 8192, 128]
    pool, 5 calls per round) with K fixed at the start of one allocation and
    V placed `skew` MiB after K's end, every skew on the same allocation
    (V rewritten before each skew's calls), rounds alternating in order;
    median per call.  The outputs must be bitwise equal for every skew."""
    import numpy as np
    import torch

    from qwen3_dspark_amd.draft import DraftBatch, HipDraftAttention
    from qwen3_dspark_amd.kernels import SCALE
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    contexts, anchors, _ = workload(args.warmup + args.steps)
    shape = (B, 8, CAPACITY, 128)
    n = B * 8 * CAPACITY * 128
    mib = 1 << 19                                        # bf16 elements per MiB
    gen = torch.Generator(device=dev).manual_seed(SEED)
    flat = torch.empty(2 * n + (max(skews_mib) + 2) * mib, dtype=torch.bfloat16, device=dev)
    k = flat[:n].view(shape)
    k.normal_(generator=gen)
    src_v = torch.empty(shape, dtype=torch.bfloat16, device=dev)
    src_v.normal_(generator=gen)
    nq = BLOCK * sum(len(a) for a in anchors)
    qd = torch.randn(nq, 16, 128, generator=gen, device=dev).to(torch.bfloat16)
    bk = torch.randn(nq, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
    bv = torch.randn(nq, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
    batch = DraftBatch(dev, [i * CAPACITY for i in range(B)], contexts, anchors)
    kernel = HipDraftAttention(dev)
    times = {m: [] for m in skews_mib}
    ref = None
    for r in range(rounds):
        for m in (skews_mib if r % 2 == 0 else skews_mib[::-1]):
            v = flat[n + m * mib:2 * n + m * mib].view(shape)
            v.copy_(src_v)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(DRAFT_LAYERS):
                out = kernel(qd, bk, bv, k, v, batch, scale=SCALE)
            e1.record()
            e1.synchronize()
            if ref is None:
                ref = out.clone()
            elif not torch.equal(out, ref):
                raise AssertionError(f'draft output differs at skew {m} MiB')
            if r >= 2:
                times[m].append(e0.elapsed_time(e1) / DRAFT_LAYERS * 1e3)
    res = {f'{m}_mib_us': round(float(np.median(t)), 2) for m, t in times.items()}
    log('[skew-sweep] ' + ', '.join(f'{m} MiB {res[f"{m}_mib_us"]:.1f}' for m in skews_mib))
    print(json.dumps({'skew_sweep': res, 'rounds': rounds - 2, 'calls_per_round': DRAFT_LAYERS,
                      'k_base_mod_1gib': int(flat.data_ptr() % (1 << 30))}), flush=True)


def verify_timeline_probe(args, samples=6):
    """Per-workgroup timeline of the verification attention (DSPARK_TIMELINE
    build): transactions of the workload's 28 layers on one store, rotating
    over the plans of plan_ab (XCD-calibrated with the second-slot share,
    without that share, equal runs with it); after each, the start and end
    stamps of the last layer's workgroups.  Per call: span from the first
    start to the last end, workgroup end times (p10, p50, p90, last), the
    mean end of the workgroups dispatched first and second onto their CUs
    (blockIdx.x below / at or above the CU count) and per XCD, the
    per-workgroup stream rate (keys x 512 B over its own start-to-end time)
    and `balanced_us`, the span a perfect balance of the same work at each
    workgroup's own rate would give.  Medians over `samples` samples per
    plan."""
    os.environ['DSPARK_AMD_TIMELINE'] = '1'
    import numpy as np
    import torch

    from qwen3_dspark_amd import _native
    from qwen3_dspark_amd._device import cu_count
    _native.load()
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    n_cu = cu_count(dev)
    pool, handles, bucket, contexts, qv, kn, vn = verify_store(args, dev)
    speed = pool.xcd_speed
    out = torch.empty_like(qv)
    host = np.zeros(8192 * 4, dtype=np.uint64)
    tick_us = 0.01
    plans = {'xcd_calibrated': (speed, True), 'no_slot_share': (speed, False), 'equal_runs': (None, True)}
    rows = {n: [] for n in plans}
    last = {}                 # per plan: the previous sample's rates by workgroup id and by CU
    names = list(plans)
    for sample in range(len(names) * (samples + 1)):
        name = names[sample % len(names)]
        pool.set_xcd_speed(plans[name][0])
        pool.set_slot_balance(plans[name][1])
        tx = pool.begin(handles, bucket)
        for layer in range(VERIFY_LAYERS):
            pool.attend(tx, layer, qv[layer], keys=kn[layer], values=vn[layer], out=out[layer])
        pool.abort(tx)
        _native.call('dspark_timeline_fetch_verify', host.ctypes.data, host.nbytes)
        if sample < len(names):
            continue                             # warm-up, one per plan
        rec = host.reshape(-1, 4)
        wid = np.nonzero((rec[:, 2] >> np.uint64(63)) == 1)[0]
        rec = rec[wid]
        t0 = float(rec[:, 0].min())
        start = (rec[:, 0].astype(np.float64) - t0) * tick_us
        end = (rec[:, 1].astype(np.float64) - t0) * tick_us
        xcc = ((rec[:, 2] >> np.uint64(32)) & np.uint64(15)).astype(np.int64)
        hw = (rec[:, 2] & np.uint64(0xffffffff)).astype(np.int64)
        cu = xcc * 1000 + ((hw >> 8) & 0xff)
        keys = (rec[:, 3] & np.uint64(0xffffffff)).astype(np.float64)
        rate = keys * 512 / np.maximum(end - start, 1e-3) * 1e-3          # GB/s: K + V rows of one KV head
        # Perfect balance at the measured per-workgroup rates: every
        # workgroup busy until the same instant.
        balanced = float(keys.sum() * 512 / (rate.sum() * 1e3)) + float(np.median(start))
        # Is a workgroup's rate a property of its work (the same blockIdx
        # each call) or of the CU it lands on?  Correlation with the previous
        # sample of the same plan, matched by workgroup id and by CU.
        by_wid = dict(zip(wid.tolist(), rate.tolist()))
        by_cu = {}
        for c, x in zip(cu.tolist(), rate.tolist()):
            by_cu.setdefault(c, []).append(x)
        by_cu = {c: float(np.mean(v)) for c, v in by_cu.items()}

        def corr(a, b):
            common = sorted(set(a) & set(b))
            return float(np.corrcoef([a[k] for k in common], [b[k] for k in common])[0, 1]) if len(common) > 2 else 0.0
        prev = last.get(name)
        last[name] = (by_wid, by_cu)
        rows[name].append(dict(
            span_us=float(end.max()), workgroups=int(len(rec)), cus=int(len(np.unique(cu))),
            start_max_us=float(start.max()), end_p10_us=float(np.percentile(end, 10)),
            end_p50_us=float(np.median(end)), end_p90_us=float(np.percentile(end, 90)),
            end_mean_us=float(end.mean()), balanced_us=balanced,
            rate_p10_gbs=float(np.percentile(rate, 10)), rate_p50_gbs=float(np.median(rate)),
            rate_p90_gbs=float(np.percentile(rate, 90)),
            keys_min=int(keys.min()), keys_max=int(keys.max()),
            rate_corr_by_workgroup=corr(prev[0], by_wid) if prev else float('nan'),
            rate_corr_by_cu=corr(prev[1], by_cu) if prev else float('nan'),
            cus_with_one_of_each=int(sum(1 for c in np.unique(cu)
                                         if ((cu == c) & (wid < n_cu)).sum() == 1 and ((cu == c) & (wid >= n_cu)).sum() == 1)),
            first_slot_end_mean_us=float(end[wid < n_cu].mean()) if (wid < n_cu).any() else 0.0,
            second_slot_end_mean_us=float(end[wid >= n_cu].mean()) if (wid >= n_cu).any() else 0.0,
            **{f'xcd{x}_end_mean_us': float(end[xcc == x].mean()) for x in range(8) if (xcc == x).any()}))
        r = rows[name][-1]
        log(f'[verify-timeline] {name}: span {r["span_us"]:.1f} us, ends p10/p50/p90 {r["end_p10_us"]:.1f}/'
            f'{r["end_p50_us"]:.1f}/{r["end_p90_us"]:.1f} us, first/second slot mean end '
            f'{r["first_slot_end_mean_us"]:.1f}/{r["second_slot_end_mean_us"]:.1f} us, balanced {balanced:.1f} us, '
            f'rate p10/p50/p90 {r["rate_p10_gbs"]:.1f}/{r["rate_p50_gbs"]:.1f}/{r["rate_p90_gbs"]:.1f} GB/s')
    pool.set_xcd_speed(speed)
    pool.set_slot_balance(True)
    summary = {n: {k: round(float(np.nanmedian([r[k] for r in v])), 3) for k in v[0]} for n, v in rows.items()}
    print(json.dumps({'timeline': 'verification attention', 'workload': '64 requests, contexts log-uniform '
                      '[256, 8192], 7 new rows each, last layer of 28', 'xcd_speed': speed, 'samples': samples,
                      'median': summary, 'per_sample': rows}), flush=True)


def stream_probe(gib=16, reps=10):
    """The streaming-read ceiling: dspark_stream_read over a `gib` GiB
    buffer (far beyond the last-level cache), each workgroup streaming its
    own contiguous slice, for the default and the non-temporal cache policy
    and 512 / 1024 / 2048 workgroups of 256 threads.  Median of `reps`
    event-timed launches after one warm-up, on the launch stream."""
    import torch

    from qwen3_dspark_amd import _native
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    nbytes = gib << 30
    src = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    out = torch.empty(4096, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    rows = []
    for nt in (0, 1):
        for wgs in (512, 1024, 2048):
            def launch():
                _native.call('dspark_stream_read', src.data_ptr(), nbytes, nt, wgs, out.data_ptr(),
                             stream.cuda_stream)
            launch()
            times = []
            for _ in range(reps):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(stream)
                launch()
                b.record(stream)
                b.synchronize()
                times.append(a.elapsed_time(b))
            ms = sorted(times)[len(times) // 2]
            rows.append({'nontemporal': bool(nt), 'workgroups': wgs, 'median_ms': round(ms, 4),
                         'gbs': round(nbytes / ms / 1e6, 1), 'frac_of_8tbs': round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4)})
            log(f'[stream] nt={nt} workgroups={wgs}: {rows[-1]["gbs"]} GB/s')
    print(json.dumps({'stream_probe': rows, 'bytes': nbytes, 'threads_per_workgroup': 256}), flush=True)


def streaming_reference(dev, src, dst, reps=10):
    """What the runtime's own 1 GiB device copy streams on this box (read +
    write bytes over its time; median of `reps` event-timed launches after
    one warm-up), as a reference for the attention kernels' GB/s."""
    import torch

    def median_ms(fn):
        fn()
        times = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            b.synchronize()
            times.append(a.elapsed_time(b))
        return sorted(times)[len(times) // 2]
    copy_ms = median_ms(lambda: dst.copy_(src))
    return {'copy_1gib_gbs': round(2 * (1 << 30) / copy_ms / 1e6, 1)}


def kernel_source_hash():
    """sha256 of the attention kernels' product code: stamps the traffic and
    trace figures measured with them.  Comments, blank lines and the
    timeline build's `#ifdef DSPARK_TIMELINE` parts (kept up to their
    `#else`) are left out, so that only a change to what the product library
    compiles moves the stamp."""
    import hashlib
    import re
    h = hashlib.sha256()
    for name in ('attn.hip', 'common.h'):
        with open(os.path.join(ROOT, 'qwen3_dspark_amd', 'csrc', name)) as f:
            text = f.read()
        text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
        skip = False
        for line in text.splitlines():
            code = line.split('//', 1)[0].strip()
            if code.startswith('#ifdef DSPARK_TIMELINE'):
                skip = True
                continue
            if skip and code.startswith('#else'):
                skip = False
                continue
            if skip and code.startswith('#endif'):
                skip = False
                continue
            if code and not skip:
                h.update(code.encode() + b'\n')
    return h.hexdigest()


def traffic_summary(args, fetch_dir, write_dir):
    """profiles/{verify,draft}_attn_traffic.json from the counter CSVs of
    `rocprofv3 --pmc FETCH_SIZE` and `--pmc WRITE_SIZE` runs of
    --traffic-probe.  Dispatches in order: 3 x (verification chunk kernel,
    merge), 3 x (draft chunk kernel, merge), then the 2**30-byte copy, whose
    counts calibrate KiB to bytes.  Per call = chunk + merge, mean of 3."""
    import csv
    import glob

    def read(directory, counter):
        path = glob.glob(os.path.join(directory, '**', '*counter_collection.csv'), recursive=True)[0]
        rows = [r for r in csv.DictReader(open(path)) if r['Counter_Name'] == counter]
        rows.sort(key=lambda r: int(r['Dispatch_Id']))
        phase, out = None, {'verify_chunk': [], 'verify_merge': [], 'draft_chunk': [], 'draft_merge': [], 'copy': []}
        for r in rows:
            name, value = r['Kernel_Name'], float(r['Counter_Value'])
            if 'varlen_attn_kernel' in name:
                phase = 'verify'
                out['verify_chunk'].append(value)
            elif 'draft_attn' in name:          # draft_attn_kernel or draft_attn_persistent_kernel
                phase = 'draft'
                out['draft_chunk'].append(value)
            elif 'merge_kernel' in name and phase:
                out[phase + '_merge'].append(value)
            elif 'copyBuffer' in name and phase == 'draft' and int(r['Grid_Size']) >= 65536:   # the 1 GiB copy
                out['copy'].append(value)
        if not all(len(out[k]) == 3 for k in ('verify_chunk', 'verify_merge', 'draft_chunk', 'draft_merge')):
            raise SystemExit(f'unexpected dispatches in {path}: { {k: len(v) for k, v in out.items()} }')
        return {k: (v[0] if k == 'copy' else sum(v) / len(v)) for k, v in out.items()}

    fetch, write = read(fetch_dir, 'FETCH_SIZE'), read(write_dir, 'WRITE_SIZE')
    copy_bytes = 1 << 30
    f_factor, w_factor = fetch['copy'] * 1024 / copy_bytes, write['copy'] * 1024 / copy_bytes
    contexts, anchors, accepted = workload(args.warmup + args.steps)
    grown = grown_contexts(contexts, accepted)
    source = kernel_source_hash()
    for kind, algorithmic in (('verify', verify_bytes(grown)), ('draft', draft_bytes(anchors))):
        read_b = (fetch[kind + '_chunk'] + fetch[kind + '_merge']) * 1024 / f_factor
        write_b = (write[kind + '_chunk'] + write[kind + '_merge']) * 1024 / w_factor
        total = read_b + write_b
        doc = dict(hbm_bytes_per_launch=round(total), read_bytes=round(read_b), write_bytes=round(write_b),
                   algorithmic_bytes_per_launch=int(algorithmic), ratio=round(total / algorithmic, 4),
                   fetch_factor=round(f_factor, 4), write_factor=round(w_factor, 4),
                   fetch_kib={'chunk': fetch[kind + '_chunk'], 'merge': fetch[kind + '_merge'],
                              'calibration_copy': fetch['copy']},
                   write_kib={'chunk': write[kind + '_chunk'], 'merge': write[kind + '_merge'],
                              'calibration_copy': write['copy']},
                   context_rows=sum(grown) if kind == 'verify' else sum(contexts),
                   workload_round=('contexts after the warm-up and timed rounds, those of the instrumented rounds'
                                   if kind == 'verify' else 'the draft contexts of every round'),
                   kernel_source_sha256=source)
        with open(os.path.join(ROOT, 'profiles', f'{kind}_attn_traffic.json'), 'w') as f:
            json.dump(doc, f, indent=1)
        print(json.dumps({kind: {k: doc[k] for k in ('hbm_bytes_per_launch', 'read_bytes', 'write_bytes',
                                                     'algorithmic_bytes_per_launch', 'ratio', 'fetch_kib',
                                                     'write_kib')}}))


def traced_launches(trace_dir):
    """The results database under `trace_dir` and, in launch order, the
    durations (us) of the verification and draft chunk kernels and of the
    merge launch that follows each kind."""
    import sqlite3
    db = [os.path.join(d, f) for d, _, fs in os.walk(trace_dir) for f in fs if f.endswith('_results.db')]
    if len(db) != 1:
        raise SystemExit(f'expected one results database under {trace_dir}, found {db}')
    con = sqlite3.connect(db[0])
    got = {'verify_chunk': [], 'verify_merge': [], 'draft_chunk': [], 'draft_merge': []}
    phase = None
    for name, t0, t1 in con.execute('select name, start, end from kernels order by start'):
        if 'varlen_attn_kernel' in name:
            phase = 'verify'
            got['verify_chunk'].append((t1 - t0) * 1e-3)
        elif 'draft_attn' in name:
            phase = 'draft'
            got['draft_chunk'].append((t1 - t0) * 1e-3)
        elif 'merge_kernel' in name and phase:
            got[phase + '_merge'].append((t1 - t0) * 1e-3)
    return db[0], got


def layer_summary(pairs):
    """Per model layer, from kernel traces of the plain bench command (each
    a trace directory and the bench line its process printed): the mean
    duration of the verification chunk kernel over the instrumented rounds,
    and the means of each run of four consecutive layers (one layer's K, and
    its V, is 1 GiB of the store)."""
    import numpy as np
    out = []
    for pair in pairs:
        trace_dir, log_path = pair.split(':', 1)
        db, got = traced_launches(trace_dir)
        with open(log_path) as f:
            line = json.loads([x for x in f.read().splitlines() if x.startswith('{"metric"')][-1])
        plain, instrumented = line['steps'] + line['warmup'], line['steps']
        v = got['verify_chunk'][VERIFY_LAYERS * plain:VERIFY_LAYERS * (plain + instrumented)]
        if len(v) < VERIFY_LAYERS * instrumented:
            raise SystemExit(f'{db}: fewer verification launches than the rounds hold')
        per_round = np.array(v).reshape(instrumented, VERIFY_LAYERS)
        per_layer = per_round.mean(axis=0)
        out.append({'bench_value_tokens_per_s': line['value'], 'mean_us': round(float(per_layer.mean()), 2),
                    'per_layer_us': [round(float(x), 2) for x in per_layer],
                    'per_4_layers_us': [round(float(x), 2) for x in per_layer.reshape(-1, 4).mean(axis=1)],
                    'sd_over_rounds_us': round(float(per_round.std(axis=0).mean()), 2)})
    print(json.dumps({'what': 'verification chunk kernel per layer, instrumented rounds', 'processes': out,
                      'kernel_source_sha256': kernel_source_hash()}))


def trace_summary(pairs):
    """profiles/attn_64req_kernel_trace.json from kernel traces of the plain
    bench command, one process each: per process, the mean duration of the
    verification chunk kernel and its merge over the launches of the
    instrumented rounds (the steps x 28 after the warmup + steps plain
    rounds), the same for the draft chunk kernel and its merge (x 5): the
    very calls behind the per-call event figures and algorithmic bytes that
    the process's bench line reports, which are set beside them; stamped
    with the kernel sources' sha256."""
    import numpy as np
    procs = []
    for pair in pairs:
        trace_dir, log_path = pair.split(':', 1)
        db, got = traced_launches(trace_dir)
        with open(log_path) as f:
            line = json.loads([x for x in f.read().splitlines() if x.startswith('{"metric"')][-1])
        plain, instrumented = line['steps'] + line['warmup'], line['steps']
        per_round = {'verify': VERIFY_LAYERS, 'draft': DRAFT_LAYERS}
        row = {'bench_value_tokens_per_s': line['value'], 'ms_per_step': line['ms_per_step']}
        for kind, k in per_round.items():
            lo, hi = k * plain, k * (plain + instrumented)
            chunk, merge = got[kind + '_chunk'][lo:hi], got[kind + '_merge'][lo:hi]
            if len(chunk) < hi - lo or len(merge) < hi - lo:
                raise SystemExit(f'{db}: fewer {kind} launches than the rounds hold')
            b = line['breakdown']
            event_ms = b[kind + '_layer_ms']
            algorithmic = (line['roofline']['algorithmic_bytes_per_launch'] if kind == 'verify'
                           else b['draft_algorithmic_bytes_per_launch'])
            kernel_us = float(np.mean(chunk)) + float(np.mean(merge))
            row[kind] = dict(chunk_us=round(float(np.mean(chunk)), 2), merge_us=round(float(np.mean(merge)), 2),
                             chunk_plus_merge_us=round(kernel_us, 2), event_us_per_call=round(event_ms * 1e3, 2),
                             algorithmic_bytes_per_launch=int(algorithmic),
                             frac_from_kernels=round(algorithmic / (kernel_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                             frac_from_events=round(algorithmic / (event_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4))
        procs.append(row)
    doc = {'what': 'kernel traces of `python bench.py --no-cpu-baseline`, one process each', 'processes': procs,
           'kernel_source_sha256': kernel_source_hash()}
    for kind in ('verify', 'draft'):
        fr = [p[kind]['frac_from_kernels'] for p in procs]
        doc[kind + '_frac_from_kernels_range'] = [min(fr), max(fr)]
    with open(os.path.join(ROOT, 'profiles', 'attn_64req_kernel_trace.json'), 'w') as f:
        json.dump(doc, f, indent=1)
    print(json.dumps(doc))


def trace_merge(paths):
    """One profiles/attn_64req_kernel_trace.json from --trace-summary outputs
    of separate sets of processes (each set run back to back, the sets at
    different times): the processes of output i are tagged set i + 1, the
    ranges cover all of them; every output must carry the sha256 of the
    current kernel sources."""
    procs, want = [], kernel_source_hash()
    for n, path in enumerate(paths, 1):
        with open(path) as f:
            doc = json.load(f)
        if doc['kernel_source_sha256'] != want:
            raise SystemExit(f'{path} was measured on other kernel sources')
        procs += [dict(p, set=n) for p in doc['processes']]
    out = {'what': 'kernel traces of `python bench.py --no-cpu-baseline`, one process each, in '
                   f'{len(paths)} sets', 'processes': procs, 'kernel_source_sha256': want}
    for kind in ('verify', 'draft'):
        fr = [p[kind]['frac_from_kernels'] for p in procs]
        out[kind + '_frac_from_kernels_range'] = [min(fr), max(fr)]
    with open(os.path.join(ROOT, 'profiles', 'attn_64req_kernel_trace.json'), 'w') as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out))


def cpu_threads():
    """(threads, reason): the host threads the CPU baseline uses - the
    process's OpenMP share when OMP_NUM_THREADS is set (a shared host sets
    it to its CPU share per GPU, e.g. 16), else every core os.cpu_count()
    reports."""
    n = os.cpu_count() or 1
    env = os.environ.get('OMP_NUM_THREADS', '')
    if env.isdigit() and int(env) >= 1:
        return min(int(env), n), f'OMP_NUM_THREADS={env} (the host CPU share of this process; os.cpu_count()={n})'
    return n, f'os.cpu_count()={n}'


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), for the CPU baseline."""
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return 'unknown'


def cpu_configs(threads):
    """The C oracle's attention time at the four smaller workloads, on the
    host, at `threads` threads and at 2 threads (the reference CI's count):
      1. draft, 2 requests, contexts 128 / 96, one 7-row block each;
      2. verification, 1 layer, 4 requests, contexts U[64, 512], 7 new rows;
      3. draft attention of 5 layers, 16 requests, contexts U[128, 1024],
         4 blocks each at anchors U[0, c];
      4. verification of 28 layers, 32 requests, contexts U[256, 2048].
    Inputs are seeded N(0,1) draws rounded to bf16 (the oracle computes in
    FP32).  Every layer of a config is executed (one call per layer, on the
    config's inputs), nothing is scaled: round time = median over `reps`
    rounds."""
    import numpy as np
    import torch

    from oracle import cref

    scale = 128 ** -0.5
    rng = np.random.default_rng(SEED + 21)
    gen = torch.Generator().manual_seed(SEED + 21)

    def bits(*shape):
        return torch.randn(*shape, generator=gen).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)

    def median_s(fn, reps):
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return float(np.median(times))

    def report(call, rows, layers, reps):
        row = {'query_rows': rows, 'layers': layers}
        for th in (threads, 2):
            def one_round():
                for _ in range(layers):
                    call(th)
            t = median_s(one_round, reps)
            row[f'{th}_threads'] = {'round_ms': round(1e3 * t, 2), 'call_ms': round(1e3 * t / layers, 3),
                                    'tokens_per_s': round(rows / t, 1), 'rounds': reps, 'layers_executed': layers}
        return row

    def draft_case(contexts, anchors, layers, reps):
        rows = BLOCK * sum(len(a) for a in anchors)
        ck, cv = bits(sum(contexts), 8, 128), bits(sum(contexts), 8, 128)
        q, bk, bv = bits(rows, 16, 128), bits(rows, 8, 128), bits(rows, 8, 128)
        offs = np.concatenate([[0], np.cumsum(contexts)[:-1]]).tolist()
        cu_b = np.cumsum([0] + [len(a) for a in anchors])
        flat = [x for a in anchors for x in a]
        return report(lambda th: cref.draft_attention(q, ck, cv, offs, contexts, bk, bv, cu_b, flat, scale=scale,
                                                      threads=th), rows, layers, reps)

    def verify_case(contexts, layers, reps):
        n = len(contexts)
        k_res, v_res = bits(n, max(contexts), 8, 128), bits(n, max(contexts), 8, 128)
        ks, vs, q = bits(n * Q_LEN, 8, 128), bits(n * Q_LEN, 8, 128), bits(n * Q_LEN, 16, 128)
        cu_q = [Q_LEN * i for i in range(n + 1)]
        return report(lambda th: cref.verify_attention(q, k_res, v_res, ks, vs, list(range(n)), contexts, cu_q,
                                                       scale=scale, threads=th), n * Q_LEN, layers, reps)

    c3 = [int(x) for x in rng.integers(128, 1025, size=16)]
    configs = {
        '1_draft_2_requests': draft_case([128, 96], [[128], [96]], 1, 5),
        '2_verify_4_requests_1_layer': verify_case([int(x) for x in rng.integers(64, 513, size=4)], 1, 5),
        '3_draft_5_layers_16_requests_4_blocks': draft_case(
            c3, [[int(a) for a in rng.integers(0, c + 1, size=4)] for c in c3], 5, 5),
        '4_verify_28_layers_32_requests': verify_case([int(x) for x in rng.integers(256, 2049, size=32)], 28, 5),
    }
    return {'cpu': cpu_model(), 'threads': [threads, 2], 'threads_reason': cpu_threads()[1],
            'kind': 'port (oracle/attn_ref.c, FP32, OpenMP)', 'configs': configs}


def gpu_configs(dev, blocks=12, per_block=10):
    """The four smaller workloads on the GPU, each call of the attention
    path timed as in the round: blocks of `per_block` back-to-back calls
    queued behind GPU work (so host launch latency never shows), one event
    pair per block; per-call latency median / p10 / p90 over `blocks` blocks
    (after two warm-up blocks), algorithmic bytes per call, GB/s, fraction
    of 8 TB/s.
      1. draft, 2 requests, contexts 128 / 96, one 7-row block each at its
         context length (fp32 Q and K, bf16 V: the kernel's fp32 form);
      2. verification, 1 layer, 4 requests, contexts U[64, 512], 7 new
         rows staged beforehand (a timed call is the attention launch over
         resident + staged rows: the round's fused launch without its copy
         of the new rows into scratch, since a layer stages once per
         transaction);
      3. draft, 5 layers, 16 requests, contexts U[128, 1024], 4 blocks each
         (one at c, three at U[0, c]);
    The draft workloads run with the default, batch-sized chunk and, for
    comparison, with the fixed 4096-row chunk of the stress workload.
      4. verification, 28 layers, 32 requests, contexts U[256, 2048], timed
         like 2 (a call is one layer; a round is 28)."""
    import numpy as np
    import torch

    from qwen3_dspark_amd.draft import DraftBatch, HipDraftAttention
    from qwen3_dspark_amd.kernels import SCALE
    from qwen3_dspark_amd.persistent_kv import Bucket, PersistentTargetKV
    from qwen3_dspark_amd.schedule import DRAFT_CHUNK
    rng = np.random.default_rng(SEED + 41)
    gen = torch.Generator(device=dev).manual_seed(SEED + 41)

    def rnd(*shape, dtype=torch.bfloat16):
        return torch.randn(*shape, generator=gen, device=dev).to(dtype)

    def timed(call, layers, nbytes, rows):
        for _ in range(2):
            for i in range(per_block):
                call(i % layers)
        times = []
        for _ in range(blocks):
            queue_ahead(dev, copies=2)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for i in range(per_block):
                call(i % layers)
            b.record()
            b.synchronize()
            times.append(a.elapsed_time(b) / per_block)
        ms = float(np.median(times))
        return {'call_us': {'median': round(ms * 1e3, 2), 'p10': round(float(np.percentile(times, 10)) * 1e3, 2),
                            'p90': round(float(np.percentile(times, 90)) * 1e3, 2)},
                'layers': layers, 'round_us': round(ms * 1e3 * layers, 1), 'query_rows': rows,
                'attn_tokens_per_s': round(rows / (ms * 1e-3), 1), 'algorithmic_bytes_per_call': int(nbytes),
                'gbs': round(nbytes / ms / 1e6, 1), 'frac_of_8tbs': round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
                'blocks': blocks, 'calls_per_block': per_block}

    def draft_config(contexts, anchors, layers, kdtype):
        n = sum(len(a) for a in anchors)
        ctx_k, ctx_v = rnd(layers, sum(contexts), 8, 128, dtype=kdtype), rnd(layers, sum(contexts), 8, 128)
        q, bk, bv = rnd(layers, 7 * n, 16, 128, dtype=kdtype), rnd(layers, 7 * n, 8, 128, dtype=kdtype), \
            rnd(layers, 7 * n, 8, 128)
        offs = [int(x) for x in np.concatenate([[0], np.cumsum(contexts)[:-1]])]
        batch = DraftBatch(dev, offs, contexts, anchors)
        kernel = HipDraftAttention(dev)          # the default: draft chunk sized to the batch
        kernel.plan(batch, ctx_k[0])
        res = timed(lambda l: kernel(q[l], bk[l], bv[l], ctx_k[l], ctx_v[l], batch, scale=SCALE), layers,
                    draft_bytes(anchors), 7 * n)
        res['draft_chunk'] = kernel.chunk_for(batch)
        # the same calls with the stress workload's fixed 4096-row chunk, for comparison
        fixed = HipDraftAttention(dev, chunk=DRAFT_CHUNK)
        fixed.plan(batch, ctx_k[0])
        res['fixed_4096_call_us'] = timed(lambda l: fixed(q[l], bk[l], bv[l], ctx_k[l], ctx_v[l], batch, scale=SCALE),
                                          layers, draft_bytes(anchors), 7 * n)['call_us']
        return res

    def verify_config(contexts, layers):
        n, cap = len(contexts), max(contexts) + 2 * Q_LEN
        pool = PersistentTargetKV(layers=layers, slots=n, context_capacity=cap, max_query_tokens=n * Q_LEN,
                                  heads=8, dim=128, device=dev)
        hs = [pool.add_request(f'c{i}') for i in range(n)]
        for layer in range(layers):
            pool.keys[layer].normal_(generator=gen)
            pool.values[layer].normal_(generator=gen)
        for h, c in zip(hs, contexts):
            pool.load_prefix(h, pool.keys[:, h.index, :c], pool.values[:, h.index, :c])
        bucket = Bucket((Q_LEN,) * n, (cap - Q_LEN,) * n, 'config')
        pool.register_bucket(bucket)
        q, kn, vn = rnd(layers, n * Q_LEN, 16, 128), rnd(layers, n * Q_LEN, 8, 128), rnd(layers, n * Q_LEN, 8, 128)
        out = torch.empty_like(q)
        tx = pool.begin(hs, bucket)
        for layer in range(layers):           # staged once; the timed calls attend over resident + staged rows
            pool.stage_layer(tx, layer, kn[layer], vn[layer])
        nbytes = sum(c + Q_LEN for c in contexts) * 2 * ROW_BYTES + 2 * n * Q_LEN * Q_ROW_BYTES
        res = timed(lambda l: pool.attend(tx, l, q[l], out=out[l]), layers, nbytes, n * Q_LEN)
        pool.abort(tx)
        del pool
        return res

    c3 = [int(x) for x in rng.integers(128, 1025, size=16)]
    a3 = [[c] + sorted(int(x) for x in rng.integers(0, c + 1, size=3)) for c in c3]
    out = {
        '1_draft_2_requests_fp32qk': draft_config([128, 96], [[128], [96]], 1, torch.float32),
        '2_verify_4_requests_1_layer': verify_config([int(x) for x in rng.integers(64, 513, size=4)], 1),
        '3_draft_5_layers_16_requests_4_blocks': draft_config(c3, a3, 5, torch.bfloat16),
        '4_verify_28_layers_32_requests': verify_config([int(x) for x in rng.integers(256, 2049, size=32)], 28),
    }
    for name, r in out.items():
        log(f'[gpu-configs] {name}: {r["call_us"]["median"]} us per call, {r["gbs"]} GB/s')
    return out


def draft_pairs(anchors):
    """Visible (query row, key) pairs of draft attention: each block's 7
    rows see the context up to its anchor and the block's 7 rows."""
    return sum(BLOCK * (a + BLOCK) for row in anchors for a in row)


def mfma_probe(args):
    """Kernels for a `rocprofv3 --pmc MfmaUtil MfmaFlopsBF16` pass (MFMA busy
    cycles over active SIMD cycles, and bf16 MFMA flops, per dispatch):
    three launches each of
      1. draft attention in the long-context 8-block case: 64 requests with
         8192-row contexts, 8 blocks each, anchors evenly spread up to 8192;
      2. draft attention of the bench workload (1..8 blocks per request);
      3. the 9,840-row draft context projection of 5 layers: the fused
         kernel, then the hipBLASLt GEMM + epilogue path.
    Pool and input contents are zero: MFMA work does not depend on them."""
    import numpy as np
    import torch

    from qwen3_dspark_amd.draft import DraftBatch, HipDraftAttention
    from qwen3_dspark_amd.draft_projection import DraftContextProjector
    from qwen3_dspark_amd.kernels import SCALE
    from qwen3_dspark_amd._device import upload

    dev = torch.device('cuda:0')
    contexts, anchors, _ = workload(args.warmup + args.steps)
    long_ctx = [CAPACITY] * B
    long_anchors = [[CAPACITY * (j + 1) // 8 for j in range(8)] for _ in range(B)]
    from qwen3_dspark_amd._device import kv_pair
    ctx_k, ctx_v = kv_pair((B, 8, CAPACITY, 128), torch.bfloat16, torch.bfloat16, dev)
    draft = HipDraftAttention(dev)
    cases = {}
    for name, ctx, anc in (('draft_8_blocks_8192', long_ctx, long_anchors), ('draft_workload', contexts, anchors)):
        rows = BLOCK * sum(len(a) for a in anc)
        qd = torch.zeros(rows, 16, 128, dtype=torch.bfloat16, device=dev)
        kd = torch.zeros(rows, 8, 128, dtype=torch.bfloat16, device=dev)
        batch = DraftBatch(dev, [i * CAPACITY for i in range(B)], ctx, anc)
        for _ in range(3):
            draft(qd, kd, kd, ctx_k, ctx_v, batch, scale=SCALE)
        torch.cuda.synchronize()
        cases[name] = {'flops_per_launch': 8192 * draft_pairs(anc), 'algorithmic_bytes_per_launch': draft_bytes(anc)}
    del ctx_k, ctx_v
    h, f, n_req = 1024, 5 * 1024, 16
    z = torch.zeros(1024, h, dtype=torch.bfloat16, device=dev)
    proj = DraftContextProjector(torch.zeros(h, f, dtype=torch.bfloat16, device=dev),
                                 torch.ones(h, dtype=torch.bfloat16, device=dev),
                                 [(z, torch.ones(128, dtype=torch.bfloat16, device=dev), z)] * 5)
    counts = [int(c) for c in np.random.default_rng(SEED + 11).integers(128, 1025, size=n_req)]
    keys = torch.zeros(5, n_req, 8, max(counts) + 1, 128, dtype=torch.bfloat16, device=dev)
    values = torch.zeros_like(keys)
    rec, first = [], 0
    for i, n in enumerate(counts):
        rec += (i, 0, first, n)
        first += n
    records = upload(dev, rec)
    fc_out = torch.zeros(first, h, dtype=torch.bfloat16, device=dev)
    for path in ('fused', 'gemm'):
        for _ in range(3):
            proj.project_into(fc_out, records, n_req, keys, values, path=path)
        torch.cuda.synchronize()
    cases['context_projection'] = {'tokens': first, 'flops_per_launch': 2 * first * h * 5 * 2 * 1024}
    print(json.dumps({'mfma_probe': 'done', 'cases': cases}), flush=True)


def cpu_leg(args, pool, bucket, handles, contexts, anchors, qv, qd, bkd, bvd, dctx_k, dctx_v, draft, draft_offsets):
    """Time the C oracle (FP32, OpenMP over the host cores) on one more round
    of the same workload - by default all 28 verification and 5 draft layers,
    nothing extrapolated - and check every GPU output of that round
    against it."""
    import numpy as np
    import torch

    from oracle import cref
    from qwen3_dspark_amd.draft import DraftBatch
    from qwen3_dspark_amd.kernels import SCALE

    threads, reason = cpu_threads()
    dev = pool.device
    n_verify = max(1, min(VERIFY_LAYERS, args.cpu_verify_layers))
    n_draft = max(1, min(DRAFT_LAYERS, args.cpu_draft_layers))

    def bits(t):
        # make the layout contiguous on the device, then one D2H copy
        return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)

    stats = {'verify_max_abs': 0.0, 'verify_mean_abs': 0.0, 'draft_max_abs': 0.0, 'draft_mean_abs': 0.0}

    def gate(out, ref, kind):
        d = np.abs(out.astype(np.float64) - ref)
        finite = bool(np.isfinite(d).all())     # a NaN/Inf output fails the gate
        stats[kind + '_max_abs'] = max(stats[kind + '_max_abs'], float(d.max()) if finite else float('inf'))
        stats[kind + '_mean_abs'] = max(stats[kind + '_mean_abs'], float(d.mean()) if finite else float('inf'))

    # Verification: a transaction on the current lengths, fresh staged rows.
    ctx = [pool.length(h) for h in handles]
    tx = pool.begin(handles, bucket)
    gen = torch.Generator(device=dev).manual_seed(SEED + 1)
    cu_q = [Q_LEN * i for i in range(B + 1)]
    slots = [h.index for h in handles]
    cmax = max(ctx)
    t_verify = 0.0
    two = {'verify': 0.0, 'draft': 0.0}      # the same layers at 2 threads
    for layer in range(n_verify):
        kn = torch.randn(B * Q_LEN, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
        vn = torch.randn(B * Q_LEN, 8, 128, generator=gen, device=dev).to(torch.bfloat16)
        pool.stage_layer(tx, layer, kn, vn)
        out = pool.attend(tx, layer, qv[layer]).float().cpu().numpy()
        # token-major host copy of the active rows: [64, max c, 8, 128]
        kres, vres = bits(pool.keys[layer, :, :cmax]), bits(pool.values[layer, :, :cmax])
        ks, vs, q = bits(pool.scratch_keys[layer]), bits(pool.scratch_values[layer]), bits(qv[layer])
        t0 = time.perf_counter()
        ref = cref.verify_attention(q, kres, vres, ks, vs, slots, ctx, cu_q, scale=SCALE, threads=threads)
        t_verify += time.perf_counter() - t0
        gate(out, ref, 'verify')
        t0 = time.perf_counter()
        cref.verify_attention(q, kres, vres, ks, vs, slots, ctx, cu_q, scale=SCALE, threads=2)
        two['verify'] += time.perf_counter() - t0
        del kres, vres
    pool.abort(tx)

    # Draft: the round's blocks over each layer's slotted context pool.
    batch = DraftBatch(dev, draft_offsets, contexts, anchors)
    offs_host = np.concatenate([[0], np.cumsum(contexts)[:-1]]).tolist()
    cu_b = np.cumsum([0] + [len(a) for a in anchors])
    flat = [x for a in anchors for x in a]
    t_draft = 0.0
    for layer in range(n_draft):
        dout = draft(qd[layer], bkd[layer], bvd[layer], dctx_k[layer], dctx_v[layer], batch,
                     scale=SCALE).float().cpu().numpy()
        # token-major host copies of each request's context rows
        ck = bits(torch.cat([dctx_k[layer, o // CAPACITY, :, :c].transpose(0, 1)
                             for o, c in zip(draft_offsets, contexts)]))
        cv = bits(torch.cat([dctx_v[layer, o // CAPACITY, :, :c].transpose(0, 1)
                             for o, c in zip(draft_offsets, contexts)]))
        t0 = time.perf_counter()
        dref = cref.draft_attention(bits(qd[layer]), ck, cv, offs_host, contexts, bits(bkd[layer]),
                                    bits(bvd[layer]), cu_b, flat, scale=SCALE, threads=threads)
        t_draft += time.perf_counter() - t0
        gate(dout, dref, 'draft')
        t0 = time.perf_counter()
        cref.draft_attention(bits(qd[layer]), ck, cv, offs_host, contexts, bits(bkd[layer]), bits(bvd[layer]),
                             cu_b, flat, scale=SCALE, threads=2)
        two['draft'] += time.perf_counter() - t0
    stats['within_tolerance'] = bool(stats['verify_max_abs'] <= 2e-2 and stats['verify_mean_abs'] <= 2e-3
                                     and stats['draft_max_abs'] <= 2e-2 and stats['draft_mean_abs'] <= 2e-3)
    stats['checked_layers'] = {'verify': n_verify, 'draft': n_draft}
    full = (n_verify, n_draft) == (VERIFY_LAYERS, DRAFT_LAYERS)
    round_s = VERIFY_LAYERS * t_verify / n_verify + DRAFT_LAYERS * t_draft / n_draft
    round_2 = VERIFY_LAYERS * two['verify'] / n_verify + DRAFT_LAYERS * two['draft'] / n_draft
    scaled = '' if full else ', scaled to 28 + 5 layers (a reduced --cpu-*-layers sample)'
    cpu = {
        'value': round(B * Q_LEN / round_s, 3), 'unit': 'tokens/s', 'cores': threads, 'kind': 'port',
        'threads_reason': reason, 'cpu': cpu_model(), 'layers_executed': {'verify': n_verify, 'draft': n_draft},
        'sample': f'C oracle (oracle/attn_ref.c, FP32, OpenMP, {threads} threads) over one round of the same '
                  f'64-request workload: {n_verify} verification layers ({t_verify:.2f} s) and {n_draft} draft '
                  f'layers ({t_draft:.2f} s){scaled}; round time {round_s:.2f} s; host CPU {cpu_model()}',
        'two_threads': {'value': round(B * Q_LEN / round_2, 3), 'unit': 'tokens/s', 'cores': 2,
                        'sample': f'the same C oracle at 2 threads (the reference CI thread count) on the same '
                                  f'{n_verify} verification layers ({two["verify"]:.2f} s) and {n_draft} draft '
                                  f'layers ({two["draft"]:.2f} s){scaled}: {round_2:.2f} s per round'},
    }
    return cpu, stats


if __name__ == '__main__':
    main()
