"""Relative XCD read speeds (qwen3_dspark_amd/xcd.py) on the CPU: stamps that
do not cover every XCD, zero-byte slices and non-finite values give no plan
skew (None: equal runs) instead of a silently clipped one."""
import math

import numpy as np
import pytest

from qwen3_dspark_amd.xcd import clipped, normalised, xcd_rates


def stamps(rates, per_xcd=4, nbytes=1 << 20):
    """Slice bytes, tick counts and XCC ids for workgroups dealt round-robin."""
    wgs = 8 * per_xcd
    xcc = np.arange(wgs) % 8
    ticks = np.array([nbytes / rates[x] for x in xcc])
    return np.full(wgs, float(nbytes)), ticks, xcc


def test_rates_relative_to_their_mean():
    got = xcd_rates(*stamps([2, 1, 1, 1, 1, 1, 1, 2]))
    assert np.allclose(got, np.array([2, 1, 1, 1, 1, 1, 1, 2]) / 1.25)
    assert math.isclose(sum(got), 8)


def test_zero_byte_slices_do_not_pull_a_mean_down():
    b, t, x = stamps([1] * 8)
    b[0] = 0.0          # an empty slice on XCD 0 (its tick count is whatever)
    t[0] = 1.0
    assert np.allclose(xcd_rates(b, t, x), 1.0)


def test_uncovered_xcd_or_nonfinite_gives_none():
    b, t, x = stamps([1] * 8)
    assert xcd_rates(b, t, x & 3) is None            # a partitioned mode: XCDs 4..7 never seen
    b2 = b.copy()
    b2[x == 5] = 0.0                                  # XCD 5 only got empty slices
    assert xcd_rates(b2, t, x) is None
    t2 = t.copy()
    t2[x == 2] = np.inf
    assert xcd_rates(b, t2, x) is None                # a zero rate


def test_clip_and_normalise_refuse_nan():
    assert clipped(None, 0.25) is None and normalised(None) is None
    assert clipped([1.5, 0.5] + [1.0] * 6, 0.25)[:2] == [1.25, 0.75]
    with pytest.raises(ValueError, match='finite'):
        clipped([float('nan')] + [1.0] * 7, 0.25)
    with pytest.raises(ValueError, match='positive finite'):
        normalised([float('nan')] + [1.0] * 7)
