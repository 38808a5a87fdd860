"""bench.py's kernel-trace summaries on a synthetic trace database: the
per-call kernel figures must come from the launches of the instrumented
rounds (after the warm-up and timed rounds), the calls the bench line's
event figures describe."""
import json
import os
import sqlite3
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402

WARMUP, STEPS = 2, 3


def _trace(tmp_path):
    """A results database of 2 plain + 3 plain + 3 instrumented rounds and
    a bench log: plain-round verification launches take 200 us, the
    instrumented ones 100 + layer us; drafts 300 us plain, 120 us
    instrumented; every merge 5 us."""
    d = tmp_path / 'trace'
    d.mkdir()
    con = sqlite3.connect(str(d / 'run_results.db'))
    con.execute('create table kernels (name text, start int, end int)')
    rows, t = [], 0
    for r in range(WARMUP + 2 * STEPS):
        instrumented = r >= WARMUP + STEPS
        for _ in range(bench.DRAFT_LAYERS):
            rows.append(('draft_attn_persistent_kernel<false, false>', t, t + (120000 if instrumented else 300000)))
            t += 400000
            rows.append(('merge_kernel', t, t + 5000))
            t += 10000
        for layer in range(bench.VERIFY_LAYERS):
            rows.append(('varlen_attn_kernel<true>', t, t + (100000 + 1000 * layer if instrumented else 200000)))
            t += 300000
            rows.append(('merge_kernel', t, t + 5000))
            t += 10000
    rows.append(('varlen_attn_kernel<true>', t, t + 999000))   # a later leg of the command
    con.executemany('insert into kernels values (?, ?, ?)', rows)
    con.commit()
    con.close()
    line = {'metric': 'm', 'value': 1000.0, 'steps': STEPS, 'warmup': WARMUP, 'ms_per_step': 4.0,
            'roofline': {'algorithmic_bytes_per_launch': 672141312},
            'breakdown': {'verify_layer_ms': 0.12, 'draft_layer_ms': 0.13,
                          'draft_algorithmic_bytes_per_launch': 668893184}}
    log = tmp_path / 'bench.log'
    log.write_text('[bench] progress\n' + json.dumps(line) + '\n')
    return d, log


def test_traced_launches_splits_kinds_and_merges(tmp_path):
    d, _ = _trace(tmp_path)
    _, got = bench.traced_launches(str(d))
    rounds = WARMUP + 2 * STEPS
    assert len(got['verify_chunk']) == rounds * bench.VERIFY_LAYERS + 1
    assert len(got['verify_merge']) == rounds * bench.VERIFY_LAYERS
    assert len(got['draft_chunk']) == len(got['draft_merge']) == rounds * bench.DRAFT_LAYERS


def test_layer_summary_reads_the_instrumented_rounds(tmp_path):
    d, log = _trace(tmp_path)
    out = subprocess.run([sys.executable, os.path.join(ROOT, 'bench.py'), '--layer-summary', f'{d}:{log}'],
                         capture_output=True, text=True, check=True, cwd=ROOT)
    proc = json.loads(out.stdout)['processes'][0]
    assert proc['per_layer_us'] == [100.0 + layer for layer in range(bench.VERIFY_LAYERS)]
    assert proc['per_4_layers_us'][0] == 101.5
    assert proc['sd_over_rounds_us'] == 0.0


def test_trace_summary_reads_the_instrumented_rounds(tmp_path, monkeypatch):
    d, log = _trace(tmp_path)
    written = {}

    class Sink:
        def __init__(self, path):
            self.path = path

        def __enter__(self):
            return self

        def __exit__(self, *a):
            return False

        def write(self, s):
            written[self.path] = written.get(self.path, '') + s

    real_open = open

    def fake_open(path, mode='r', *a, **k):
        if 'w' in mode and str(path).endswith('attn_64req_kernel_trace.json'):
            return Sink(path)
        return real_open(path, mode, *a, **k)

    monkeypatch.setattr('builtins.open', fake_open)
    bench.trace_summary([f'{d}:{log}'])
    doc = json.loads(next(iter(written.values())))
    p = doc['processes'][0]
    assert p['verify']['chunk_us'] == 113.5          # mean of 100 + layer over the instrumented rounds
    assert p['verify']['merge_us'] == 5.0
    assert p['draft']['chunk_us'] == 120.0
