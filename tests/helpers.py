"""Shared test helpers: seeded bf16 inputs and the attention tolerance gate."""
import numpy as np
import torch

SEED = 20261009
SCALE = 128 ** -0.5
# Target tolerance (bf16 vs FP32/FP64 oracle) plus the reference gate
# (scripts/probe_qwen_varlen.py:84-96): |d| <= .02 + .02|ref|, RMS <= .005.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3
ATOL, RTOL, MAX_RMS = 0.02, 0.02, 0.005


def randn_bf16(gen, *shape):
    """CPU FP32 N(0,1) draws rounded to bf16 (as scripts/probe_varlen.py:108-110)."""
    return torch.randn(*shape, generator=gen, dtype=torch.float32).to(torch.bfloat16)


def bits(t):
    """bf16 tensor -> numpy uint16 bit patterns (CPU)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f64(t):
    return t.detach().cpu().double().numpy()


def attention_gate(actual, expected, segments=None):
    """Assert the tolerance gate pooled and per segment; returns stats."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    assert np.isfinite(a).all(), 'non-finite output'
    stats = []
    for lo, hi in ([(0, a.shape[0])] + list(segments or [])):
        d = np.abs(a[lo:hi] - e[lo:hi])
        if d.size == 0:
            continue
        s = dict(max_abs=float(d.max()), mean_abs=float(d.mean()), rms=float(np.sqrt((d ** 2).mean())),
                 mismatched=int((d > ATOL + RTOL * np.abs(e[lo:hi])).sum()))
        assert s['max_abs'] <= MAX_ABS, s
        assert s['mean_abs'] <= MEAN_ABS, s
        assert s['rms'] <= MAX_RMS, s
        assert s['mismatched'] == 0, s
        stats.append(s)
    return stats


def segments(cu):
    cu = list(cu)
    return [(cu[i], cu[i + 1]) for i in range(len(cu) - 1)]
