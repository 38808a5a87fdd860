"""Device selection and per-device reusable buffers for the HIP path."""
import collections
import threading

import numpy as np
import torch

ARCH = 'gfx950'


def require_gfx950(device):
    """Canonical torch.device of an explicitly selected gfx950 GPU, else raise.

    There is no CPU or non-gfx950 path: callers fail loudly instead.
    """
    device = torch.device(device)
    if device.type != 'cuda' or torch.version.hip is None or not torch.cuda.is_available():
        raise RuntimeError('The MI355X HIP path requires an explicitly selected ROCm gfx950 GPU; no CPU fallback')
    if device.index is None:
        device = torch.device('cuda', torch.cuda.current_device())
    arch = getattr(torch.cuda.get_device_properties(device), 'gcnArchName', '') or ''
    if arch.split(':')[0] != ARCH:
        raise RuntimeError(f'The MI355X HIP path requires a {ARCH} GPU, found {arch!r}')
    return device


# Bytes between the end of K and the start of V in a kv_pair allocation.
KV_PAIR_SKEW = 32 << 20


def kv_pair(shape, key_dtype, value_dtype, device, skew=KV_PAIR_SKEW):
    """Zeroed K and V tensors of `shape` in one allocation, V starting
    `skew` bytes after the end of K.  The attention kernels read a K row and
    the V row at the same position together, and how fast such pairs stream
    depends on the distance between the two tensors: with V a whole number
    of GiB after K, as two separate allocations of GiB-sized stores usually
    land, a draft call over a [64, 8, 8192, 128] pool measured ≈121.8 us;
    with V 8-64 MiB further it measured ≈118.4 us (one allocation, V moved,
    three processes)."""
    shape = tuple(int(x) for x in shape)
    count = int(np.prod(shape))
    kb = count * torch.empty((), dtype=key_dtype).element_size()
    vb = count * torch.empty((), dtype=value_dtype).element_size()
    skew = int(skew)
    if skew < 0 or skew % 256:
        raise ValueError('kv_pair skew must be a nonnegative multiple of 256 bytes')
    flat = torch.zeros(kb + skew + vb, dtype=torch.uint8, device=device)
    return (flat[:kb].view(key_dtype).view(shape), flat[kb + skew:kb + skew + vb].view(value_dtype).view(shape))


_CU_COUNTS = {}


def cu_count(device):
    """Compute units of a GPU (cached per device index)."""
    device = torch.device(device)
    idx = device.index if device.index is not None else torch.cuda.current_device()
    n = _CU_COUNTS.get(idx)
    if n is None:
        n = _CU_COUNTS[idx] = int(torch.cuda.get_device_properties(idx).multi_processor_count)
    return n


class Workspace:
    """Grow-only device scratch (uint8) reused across calls on one device."""

    def __init__(self, device):
        self.device = device
        self._buf = None

    def get(self, nbytes):
        nbytes = max(int(nbytes), 16)
        if self._buf is None or self._buf.numel() < nbytes:
            self._buf = torch.zeros(nbytes, dtype=torch.uint8, device=self.device)
        return self._buf

    @property
    def nbytes(self):
        return 0 if self._buf is None else self._buf.numel()


class HostStaging:
    """Pinned host ring for the small host-to-device metadata uploads of the
    hot path (work lists, offsets, transaction requests, accepted counts).

    The pinned buffer is allocated once.  Each upload writes the next
    256-byte-aligned region and enqueues an asynchronous copy on the current
    stream.  Regions are retired in groups: the copies issued since the last
    event form an open span, and one event is recorded after the span's
    last copy once the span reaches MARK_BYTES, the stream changes, or a new
    upload would reuse a byte of it.  A region is rewritten only after the
    event of its span has completed.  An event per upload would put a
    marker between every metadata copy and the next kernel (≈5-6 us each on
    the launch stream); a round's handful of uploads now share one.  Steady
    state performs no pinned allocation (which can stall the host for
    milliseconds) and never synchronises the device.  One instance per
    device, guarded by a lock.
    """

    MARK_BYTES = 64 << 10

    def __init__(self, device, nbytes=1 << 20):
        self.device = device
        self._buf = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
        self._head = 0
        self._inflight = collections.deque()    # (start, end, event) per closed span, oldest first
        self._open = None                       # [start, end, stream] of the copies since the last event
        self._events = []
        self._lock = threading.Lock()

    def _close(self):
        # One event after the open span's last copy, on the span's stream.
        if self._open is None:
            return
        start, end, stream = self._open
        ev = self._events.pop() if self._events else torch.cuda.Event()
        ev.record(stream)
        self._inflight.append((start, end, ev))
        self._open = None

    def _retire(self, start, end):
        # Spans on one stream complete in order: drop finished ones first,
        # then wait only for a still-pending span that the new region reuses.
        q = self._inflight
        while q and q[0][2].query():
            self._events.append(q.popleft()[2])
        pending = collections.deque()
        for s, e, ev in q:
            if s < end and start < e:
                ev.synchronize()
                self._events.append(ev)
            else:
                pending.append((s, e, ev))
        self._inflight = pending

    def upload(self, values, dtype=torch.int32, out=None):
        """Copy `values` (ints or a numpy array) into a device tensor of
        `dtype` (a new one unless `out`, a contiguous device tensor of the
        same size and dtype, is given); returns it.  Asynchronous."""
        arr = np.ascontiguousarray(np.asarray(values, dtype=torch.empty(0, dtype=dtype).numpy().dtype).reshape(-1))
        n = arr.nbytes
        if out is None:
            out = torch.empty(arr.size, dtype=dtype, device=self.device)
        elif out.dtype != dtype or out.numel() != arr.size or not out.is_contiguous() or out.device != self.device:
            raise ValueError('Upload target must be a contiguous device tensor of matching size and dtype')
        if n == 0:
            return out
        with self._lock:
            stream = torch.cuda.current_stream(self.device)
            span = (n + 255) & ~255
            if span > self._buf.numel():
                self._close()
                for _, _, ev in self._inflight:
                    ev.synchronize()
                self._inflight.clear()
                self._buf = torch.empty(max(span, 2 * self._buf.numel()), dtype=torch.uint8, pin_memory=True)
                self._head = 0
            if self._head + span > self._buf.numel():
                self._head = 0
            start, end = self._head, self._head + span
            if self._open is not None and (self._open[2].cuda_stream != stream.cuda_stream
                                           or (self._open[0] < end and start < self._open[1])):
                self._close()
            self._retire(start, end)
            self._head = end
            host = self._buf[start:start + n].view(dtype)
            host.copy_(torch.from_numpy(arr))
            out.copy_(host, non_blocking=True)
            if self._open is None:
                self._open = [start, end, stream]
            else:
                self._open[0], self._open[1] = min(self._open[0], start), max(self._open[1], end)
            if self._open[1] - self._open[0] >= self.MARK_BYTES:
                self._close()
        return out


_STAGING = {}
_STAGING_LOCK = threading.Lock()


def upload(device, values, dtype=torch.int32, out=None):
    """Asynchronous host-to-device upload through the device's HostStaging."""
    with _STAGING_LOCK:
        staging = _STAGING.get(device)
        if staging is None:
            staging = _STAGING[device] = HostStaging(device)
    return staging.upload(values, dtype, out)
