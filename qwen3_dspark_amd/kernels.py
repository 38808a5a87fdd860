"""HIP attention kernels behind the reference's kernel-callable contract.

    kernel(query, key, value, layout, *, scale) -> Tensor

Drop-ins for
  * dspark_qwen/rocm_varlen.py:42-117   PinnedRocmVarlenKernel (causal, exact K)
  * dspark_qwen/packed_draft.py:19-32   PinnedRocmDraftKernel (noncausal, exact K)
  * dspark_qwen/persistent_qwen_target.py:223-234 _native_attention (causal,
    capacity-tail K with fixed bucket maxima)
with the same argument meaning, the same ValueError-before-device-work
contract and no fallback: a failing launch raises.
"""
import math

import torch

from . import _native, backends
from ._device import Workspace, cu_count, require_gfx950
from .schedule import DEFAULT_CHUNK, SPLITS, run_count, segment_plan, upload_work

Q_HEADS, KV_HEADS, HEAD_DIM = 16, 8, 128
SCALE = 128 ** -0.5


def _check_scale(scale, what):
    if not isinstance(scale, (float, int)) or not math.isfinite(scale) or scale != SCALE:
        raise ValueError(f'{what} requires the 1/sqrt(128) scale')


class HipVarlenKernel:
    """Bottom-right causal packed attention over an exact-K PackedLayout."""
    backend_name = backends.TARGET_BACKEND
    native_varlen_calls_per_layer = 1
    causal = True

    def __init__(self, device, *, chunk=DEFAULT_CHUNK, split='balanced'):
        self.device = require_gfx950(device)
        _native.load()
        if split not in SPLITS:
            raise ValueError(f'split must be one of {SPLITS}')
        self.chunk = int(chunk)
        self.split = split
        self._workspace = Workspace(self.device)
        self._validated_layout = None
        self._layout_versions = None
        self._work_for = None
        self._work = None

    # Same contract and error classes as rocm_varlen.py:65-106.
    def _validate_inputs(self, query, key, value, layout, scale):
        tensors = (query, key, value)
        if any(not isinstance(t, torch.Tensor) or not t.is_cuda or t.device != self.device
               or t.dtype != torch.bfloat16 or t.requires_grad or t.ndim != 3 or not t.is_contiguous()
               for t in tensors):
            raise ValueError('HIP varlen requires no-autograd contiguous BF16 THD tensors on its selected GPU')
        if (tuple(query.shape[1:]) != (Q_HEADS, HEAD_DIM) or tuple(key.shape[1:]) != (KV_HEADS, HEAD_DIM)
                or value.shape != key.shape or query.shape[0] == 0 or key.shape[0] == 0):
            raise ValueError('HIP varlen supports nonempty Hq16/Hkv8/D128 Qwen tensors only')
        _check_scale(scale, 'HIP varlen')
        for name in ('query_lengths', 'key_lengths', 'cu_query', 'cu_key', 'request_markers'):
            if not hasattr(layout, name):
                raise ValueError('HIP varlen requires a PackedLayout')
        if query.shape[0] != sum(layout.query_lengths) or key.shape[0] != sum(layout.key_lengths):
            raise ValueError('Tensor token dimensions differ from packed layout')
        self._validate_layout(layout, markers=True)

    def _validate_layout(self, layout, *, markers):
        cu = (layout.cu_query, layout.cu_key)
        if any(not isinstance(t, torch.Tensor) or t.device != self.device or t.dtype != torch.int32
               or t.ndim != 1 or not t.is_contiguous() for t in cu):
            raise ValueError('HIP varlen requires contiguous int32 cumulative lengths on its selected GPU')
        try:
            versions = tuple(t._version for t in cu)
        except RuntimeError:
            versions = None  # inference tensors: revalidate every call
        if versions is not None and layout is self._validated_layout and versions == self._layout_versions:
            return
        qs, ks = layout.query_lengths, layout.key_lengths
        if (not qs or len(qs) != len(ks)
                or (markers and (len(layout.request_markers) != len(qs) or len(set(layout.request_markers)) != len(qs)))
                or any(type(q) is not int or type(k) is not int or not 0 < q <= k for q, k in zip(qs, ks))):
            raise ValueError('Invalid packed lengths/markers for bottom-right causal suffixes')

        def cumulative(lengths):
            out = [0]
            for n in lengths:
                out.append(out[-1] + n)
            if out[-1] >= 2 ** 31:
                raise ValueError('Packed cumulative length exceeds int32')
            return out
        if layout.cu_query.tolist() != cumulative(qs) or layout.cu_key.tolist() != cumulative(ks):
            raise ValueError('Cumulative lengths differ from packed metadata')
        self._validated_layout, self._layout_versions = layout, versions

    def _work_list(self, layout, tiles):
        # One balanced segment list per layout shape (its lengths are
        # immutable host tuples), uploaded once and reused by every layer.
        key = (layout.query_lengths, layout.key_lengths, tiles)
        if self._work_for != key:
            starts, acc = [], 0
            for k in layout.key_lengths:
                starts.append(acc)
                acc += k
            n_cu = cu_count(self.device)
            runs = run_count(acc, n_cu, tiles)
            records, n_segments, runs = segment_plan(self.split, layout.query_lengths, layout.key_lengths, starts,
                                                     runs, self.chunk, n_cu=n_cu)
            self._work = (upload_work(records, self.device), n_segments, runs)
            self._work_for = key
        return self._work

    def _launch(self, query, key, value, layout, max_q, key_rows):
        out = torch.empty_like(query)
        n_req = len(layout.query_lengths)
        tiles = (max_q + 7) // 8
        work, n_work, runs = self._work_list(layout, tiles) or (None, 0, 0)
        lib = _native.load()
        need = (lib.dspark_attn_workspace_bytes(n_work, 0, tiles, self.chunk) if work is not None
                else lib.dspark_attn_workspace_bytes(n_req, key_rows, tiles, self.chunk))
        ws = self._workspace.get(need)
        _native.call('dspark_varlen_attn_fwd', _native.ptr(query), _native.ptr(key), _native.ptr(value),
                     _native.ptr(layout.cu_query), _native.ptr(layout.cu_key), n_req, query.shape[0], key_rows,
                     max_q, int(self.causal), float(SCALE), self.chunk, _native.ptr(work), n_work, runs,
                     _native.ptr(out), _native.ptr(ws), ws.numel(), _native.stream_handle(self.device))
        return out

    def __call__(self, query, key, value, layout, *, scale):
        self._validate_inputs(query, key, value, layout, scale)
        output = self._launch(query, key, value, layout, max(layout.query_lengths), key.shape[0])
        if output.shape != query.shape or output.dtype != query.dtype or output.device != query.device:
            raise RuntimeError('HIP varlen returned incompatible output')
        return output


class HipDraftVarlenKernel(HipVarlenKernel):
    """Noncausal packed attention: every query sees all keys of its request
    (the single-block packed draft path, packed_draft.py:19-47)."""
    backend_name = backends.DRAFT_BACKEND
    causal = False


class HipCapacityKernel(HipVarlenKernel):
    """Causal attention over capacity-length K/V (persistent_qwen_target.py:223-234).

    len(key) is the bucket key capacity; rows past cu_key[-1] are never read,
    so zero, finite or NaN tails give bit-identical outputs.  The launch grid
    depends only on the bucket (capacity and maximum query length), never on
    the current lengths.
    """
    backend_name = backends.CAPACITY_BACKEND

    def _work_list(self, layout, tiles):
        # Request-order dispatch of fixed chunks over a grid sized from the
        # capacity: the same launch for every transaction of a bucket.
        return None

    def __call__(self, query, key, value, layout, *, scale):
        if (not all(isinstance(t, torch.Tensor) for t in (query, key, value))
                or query.dtype != torch.bfloat16 or key.dtype != query.dtype or value.dtype != query.dtype
                or query.ndim != 3 or key.ndim != 3
                or tuple(query.shape[1:]) != (Q_HEADS, HEAD_DIM) or tuple(key.shape[1:]) != (KV_HEADS, HEAD_DIM)
                or key.shape != value.shape or len(key) != layout.physical_key_capacity
                or len(query) != sum(layout.query_lengths)):
            raise ValueError('HIP capacity attention shape/dtype/scale differs')
        _check_scale(scale, 'HIP capacity attention')
        if any(not t.is_contiguous() or t.device != self.device or t.requires_grad for t in (query, key, value)):
            raise ValueError('HIP capacity attention requires contiguous no-autograd tensors on its GPU')
        if sum(layout.key_lengths) > layout.physical_key_capacity:
            raise ValueError('Key lengths exceed the physical key capacity')
        max_q = int(layout.maximum_query_length) or max(layout.query_lengths)
        if max_q < max(layout.query_lengths):
            raise ValueError('Bucket maximum query length below an actual query length')
        self._validate_layout(layout, markers=False)
        return self._launch(query, key, value, layout, max_q, layout.physical_key_capacity)
