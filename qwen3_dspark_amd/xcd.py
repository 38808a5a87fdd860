"""XCD-aware planning on MI355X: how fast each of the 8 XCDs reads a region.

Workgroups of a launch are dealt round-robin over the 8 XCDs (workgroup b
runs on XCD b mod 8), each with its own L2 and its own path to HBM.  The XCDs
do not read a given allocation equally fast, and which ones are slower
depends on where the allocation landed, so the verification plans size each
XCD's runs to speeds measured over the store they stream
(PersistentTargetKV.calibrate_xcd).  No reference counterpart.
"""
import numpy as np
import torch

from . import _native
from .schedule import XCDS


def measure_read_speed(tensors, *, workgroups=1024, passes=2):
    """Relative read bandwidth of the 8 XCDs over the given device tensors
    (each contiguous, same device): dspark_xcd_read_stamps over every tensor
    `passes` times, one host synchronisation at the end.  Returns each XCD's
    mean per-workgroup rate over the mean of the 8 (xcd_rates), or None if
    the stamps do not cover every XCD."""
    tensors = [t for t in tensors if t.numel()]
    if not tensors or any(not t.is_contiguous() or t.device != tensors[0].device for t in tensors):
        raise ValueError('Contiguous device tensors on one device required')
    device = tensors[0].device
    sizes = [t.numel() * t.element_size() // 16 * 16 for t in tensors]
    if min(sizes) < 16:
        raise ValueError('Every region must hold at least 16 bytes')
    # at least 64 KiB per workgroup slice of the smallest region
    wgs = max(XCDS, min(int(workgroups), min(sizes) // (64 << 10)) // XCDS * XCDS)
    launches = len(tensors) * int(passes)
    stamps = torch.zeros((launches, wgs, 3), dtype=torch.int64, device=device)
    stream = _native.stream_handle(device)
    i = 0
    for _ in range(int(passes)):
        for t, n in zip(tensors, sizes):
            _native.call('dspark_xcd_read_stamps', t.data_ptr(), n, wgs, stamps[i].data_ptr(), stream)
            i += 1
    st = stamps.cpu().numpy()

    def slices(n):          # bytes of each workgroup's slice of an n-byte region
        per = -(-(n // 16) // wgs) * 16
        return [min(per, max(n - per * w, 0)) for w in range(wgs)]
    slice_bytes = np.array([slices(n) for _ in range(int(passes)) for n in sizes], dtype=np.float64)
    return xcd_rates(slice_bytes, st[..., 1] - st[..., 0], st[..., 2])


def xcd_rates(slice_bytes, ticks, xcc):
    """Each XCD's mean read rate over its workgroups' nonempty slices,
    relative to the mean of the 8; None when some XCD has no nonempty slice
    or a rate is not finite and positive (a partitioned mode, or a region
    too small to spread over every XCD), so that plans then use equal runs."""
    slice_bytes = np.asarray(slice_bytes, dtype=np.float64)
    ticks = np.asarray(ticks, dtype=np.float64)
    xcd = np.asarray(xcc, dtype=np.int64) & (XCDS - 1)
    used = slice_bytes > 0
    rate = slice_bytes / np.maximum(ticks, 1)
    means = []
    for x in range(XCDS):
        mine = rate[used & (xcd == x)]
        if mine.size == 0:
            return None
        means.append(mine.mean())
    means = np.array(means)
    if not (np.isfinite(means).all() and (means > 0).all()):
        return None
    return [float(x) for x in means / means.mean()]


def normalised(speed, what='xcd_speed'):
    """8 positive finite relative speeds scaled to mean 1, or None."""
    if speed is None:
        return None
    speed = tuple(float(x) for x in speed)
    if len(speed) != XCDS or not all(np.isfinite(x) and x > 0 for x in speed):
        raise ValueError(f'{what} must give {XCDS} positive finite relative speeds')
    mean = sum(speed) / XCDS
    return tuple(x / mean for x in speed)


def clipped(speed, clip):
    """Speeds limited to 1 +- clip (a measurement's noise never skews a plan
    further); None stays None.  A speed that is not finite is refused."""
    if speed is None:
        return None
    speed = [float(x) for x in speed]
    if not all(np.isfinite(x) for x in speed):
        raise ValueError('Relative XCD speeds must be finite')
    return [min(1.0 + clip, max(1.0 - clip, x)) for x in speed]
