"""Device half of the persistent target KV store: HBM allocations and every
HIP launch of a transaction.  PersistentTargetKV (persistent_kv.py) owns the
host state machine and calls into an object of this shape; HipKVDevice is the
only implementation in the package (there is no CPU path).

Layout in HBM: resident K and V are stored head-major,
[layers, slots, heads, context_capacity, dim], so the attention of one
(request, KV head) streams one contiguous run of 256-byte rows; `keys` /
`values` are [layers, slots, context_capacity, heads, dim] views of that
storage (the shape persistent_target_kv.py:174-202 allocates).  Scratch K
and V are token-major [layers, max_query_tokens, heads, dim], the shape the
model produces.

Per bucket, a Workspace holds the seven transaction arrays of
persistent_target_kv.py:127-153 (built on the device by one
dspark_txn_metadata launch), the per-request (slot, context, query) triples
the kernels read, a fixed-capacity split-K work list and the split-K
partials.  Every launch argument of a bucket's attention depends only on the
bucket, so a captured launch replays for every later transaction of it.
"""
import torch

from . import _native
from ._device import KV_PAIR_SKEW, cu_count, kv_pair, require_gfx950, upload
from .kernels import HEAD_DIM, KV_HEADS, SCALE
from .schedule import REQ_INTS, WORK_INTS, run_count, segment_plan, varlen_list_bound

MAX_BUCKET_REQUESTS = 4096      # requests per transaction (one metadata workgroup scans them in LDS)


def _list_runs(shape, device):
    """Most balanced-list runs any transaction of a bucket uses (its key
    capacity bounds the keys of every transaction)."""
    return run_count(shape.key_capacity, cu_count(device), (shape.maximum_query_length + 7) // 8)


def _list_segments(shape, device, chunk, split):
    return varlen_list_bound(shape.request_count, _list_runs(shape, device), shape.key_capacity,
                             None if split == 'balanced' else chunk)


def _list_ints(shape, device, chunk, split):
    """int32 length of the largest work list of a bucket."""
    return (WORK_INTS * _list_segments(shape, device, chunk, split) + _list_runs(shape, device) + 1
            + REQ_INTS * shape.request_count)


def _partials_bytes(shape, device, chunk, split):
    """Split-K partials for the largest work list of a bucket (one slot per
    segment at most)."""
    tiles = (shape.maximum_query_length + 7) // 8
    return max(16, int(_native.load().dspark_attn_workspace_bytes(_list_segments(shape, device, chunk, split), 0,
                                                                  tiles, chunk)))


class Workspace:
    """Fixed device buffers of one bucket (or one shared family arena)."""

    def __init__(self, tensors):
        for name, t in tensors.items():
            setattr(self, name, t)
        self._names = tuple(tensors)

    def tensors(self):
        return {name: getattr(self, name) for name in self._names}

    def pointers(self):
        return {name: t.data_ptr() for name, t in self.tensors().items()}

    def nbytes(self):
        return sum(t.numel() * t.element_size() for t in self.tensors().values())

    def signature(self):
        """Identity, addresses and geometry of every buffer (an external
        writer's captured launches are valid only while this is unchanged)."""
        return (id(self), tuple((name, t.data_ptr(), tuple(t.shape), tuple(t.stride()), t.storage_offset(), t.dtype,
                                 t.device) for name, t in self.tensors().items()))

    def view(self, shape):
        """The leading parts of a shared arena's buffers that a smaller shape
        uses (same addresses)."""
        r, q, n = shape.request_count, shape.query_tokens, shape.key_capacity
        cut = dict(cu_query=r + 1, cu_key=r + 1, positions=q, req=3 * r, work=None, attn=None)
        return Workspace({name: (t if cut.get(name, n) is None else t[:cut.get(name, n)])
                          for name, t in self.tensors().items()})


class HipKVDevice:
    """Resident and scratch KV in HBM plus the store's launches on gfx950."""

    def __init__(self, *, layers, slots, context_capacity, max_query_tokens, heads, dim, dtype, device, chunk,
                 split, kv_skew=KV_PAIR_SKEW):
        # the copy kernels move 16-byte pieces of a head row
        if (dim * torch.empty((), dtype=dtype).element_size()) % 16:
            raise ValueError('A KV head row (dim * element size) must be a multiple of 16 bytes')
        self.device = require_gfx950(device)
        _native.load()
        self.layers, self.slots, self.capacity = layers, slots, context_capacity
        self.max_rows, self.heads, self.dim, self.dtype = max_query_tokens, heads, dim, dtype
        self.chunk, self.split = chunk, split
        self.xcd_speed = None          # relative speed of each XCD for balanced plans (None: equal runs)
        self.slot_balance = True       # balanced plans give second-resident workgroups SECOND_SLOT_SHARE
        self.elem = torch.empty((), dtype=dtype).element_size()
        # K and V in one allocation, V kv_skew bytes after K (kv_pair)
        self._keys, self._values = kv_pair((layers, slots, heads, context_capacity, dim), dtype, dtype, self.device,
                                           kv_skew)
        self.keys = self._keys.permute(0, 1, 3, 2, 4)
        self.values = self._values.permute(0, 1, 3, 2, 4)
        self.scratch_keys = torch.zeros((layers, max_query_tokens, heads, dim), dtype=dtype, device=self.device)
        self.scratch_values = torch.zeros_like(self.scratch_keys)
        lk, ls = self._keys[0].numel() * self.elem, self.scratch_keys[0].numel() * self.elem
        # Per-layer device addresses (the allocations never move).
        self.layer_pointers = tuple((self._keys.data_ptr() + l * lk, self._values.data_ptr() + l * lk,
                                     self.scratch_keys.data_ptr() + l * ls, self.scratch_values.data_ptr() + l * ls)
                                    for l in range(layers))

    # -- geometry -----------------------------------------------------------
    def strides(self):
        """Resident byte strides: (layer, slot, head, token) and row-piece bytes."""
        e, H, C, D = self.elem, self.heads, self.capacity, self.dim
        return (self.slots * H * C * D * e, H * C * D * e, C * D * e, D * e, D * e)

    def launch_shape(self, shape):
        """(record capacity, runs) of a bucket's fixed-capacity work list."""
        return _list_segments(shape, self.device, self.chunk, self.split), _list_runs(shape, self.device)

    # -- workspaces -----------------------------------------------------------
    def workspace(self, shape):
        """Allocate the buffers of a bucket, or of a family arena whose shape
        is the elementwise maximum of its families."""
        n, r, q = shape.key_capacity, shape.request_count, shape.query_tokens
        d = self.device
        return Workspace(dict(
            committed_indices=torch.zeros(n, dtype=torch.long, device=d),
            scratch_indices=torch.zeros(n, dtype=torch.long, device=d),
            from_scratch=torch.zeros((n, 1, 1), dtype=torch.bool, device=d),
            valid=torch.zeros((n, 1, 1), dtype=torch.bool, device=d),
            cu_query=torch.zeros(r + 1, dtype=torch.int32, device=d),
            cu_key=torch.zeros(r + 1, dtype=torch.int32, device=d),
            positions=torch.zeros(q, dtype=torch.long, device=d),
            req=torch.zeros(3 * r, dtype=torch.int32, device=d),
            work=torch.zeros(_list_ints(shape, d, self.chunk, self.split), dtype=torch.int32, device=d),
            keys=torch.empty((n, self.heads, self.dim), dtype=self.dtype, device=d),
            values=torch.empty((n, self.heads, self.dim), dtype=self.dtype, device=d),
            attn=torch.zeros(_partials_bytes(shape, d, self.chunk, self.split), dtype=torch.uint8, device=d)))

    def workspace_bytes(self, shape):
        """Exact allocation of workspace(shape), before allocating it."""
        n, r, q = shape.key_capacity, shape.request_count, shape.query_tokens
        kv = 2 * n * self.heads * self.dim * self.elem
        return (kv + 18 * n + 8 * (r + 1) + 8 * q + 12 * r + 4 * _list_ints(shape, self.device, self.chunk, self.split)
                + _partials_bytes(shape, self.device, self.chunk, self.split))

    # -- XCD calibration -------------------------------------------------------
    def measure_xcd_speed(self, workgroups=1024, passes=2):
        """Relative read bandwidth of the 8 XCDs over this store's resident
        K and V (every layer's K and V region; xcd.measure_read_speed)."""
        from .xcd import measure_read_speed
        return measure_read_speed([t for layer in range(self.layers) for t in (self._keys[layer], self._values[layer])],
                                  workgroups=workgroups, passes=passes)

    # -- resident rows --------------------------------------------------------
    def write_prefix(self, slot, keys, values):
        n = keys.shape[1]
        self.keys[:, slot, :n].copy_(keys)
        self.values[:, slot, :n].copy_(values)

    def copy_out(self, slot, n):
        return (self.keys[:, slot, :n].detach().clone(memory_format=torch.contiguous_format),
                self.values[:, slot, :n].detach().clone(memory_format=torch.contiguous_format))

    # -- one transaction --------------------------------------------------------
    def build_metadata(self, ws, shape, slots, contexts, query_lengths):
        """Upload the request triples and the bucket's work list, then build
        the seven metadata arrays in one launch.  Raises before anything is
        published if the list does not fit or a launch fails."""
        key_lengths = [c + q for c, q in zip(contexts, query_lengths)]
        n_cu = cu_count(self.device)
        runs = run_count(sum(key_lengths), n_cu, (shape.maximum_query_length + 7) // 8)
        records, _, _ = segment_plan(self.split, query_lengths, key_lengths, slots, runs, self.chunk,
                                     self.launch_shape(shape), xcd_speed=self.xcd_speed,
                                     n_cu=n_cu if self.slot_balance else None)
        if len(records) > ws.work.numel():
            raise ValueError('Work list exceeds the bucket workspace')
        r = len(slots)
        upload(self.device, list(slots) + list(contexts) + list(query_lengths), out=ws.req[:3 * r])
        upload(self.device, records, out=ws.work[:len(records)])
        _native.call('dspark_txn_metadata', _native.ptr(ws.req), r, self.capacity, shape.key_capacity,
                     shape.query_tokens, _native.ptr(ws.committed_indices), _native.ptr(ws.scratch_indices),
                     _native.ptr(ws.from_scratch), _native.ptr(ws.valid), _native.ptr(ws.positions),
                     _native.ptr(ws.cu_query), _native.ptr(ws.cu_key), _native.stream_handle(self.device))

    def stage(self, layer, keys, values, rows):
        keys, values = keys.contiguous(), values.contiguous()
        _, _, sk, sv = self.layer_pointers[layer]
        _native.call('dspark_kv_stage', keys.data_ptr(), values.data_ptr(), sk, sv, rows,
                     self.heads * self.dim * self.elem, _native.stream_handle(self.device))

    def gather(self, ws, shape, layer):
        _, slot_b, head_b, tok_b, piece_b = self.strides()
        _native.call('dspark_kv_gather', _native.ptr(self._keys[layer]), _native.ptr(self._values[layer]),
                     _native.ptr(self.scratch_keys[layer]), _native.ptr(self.scratch_values[layer]),
                     _native.ptr(ws.committed_indices), _native.ptr(ws.scratch_indices),
                     _native.ptr(ws.from_scratch), _native.ptr(ws.valid), shape.key_capacity,
                     self.slots, slot_b, head_b, tok_b, self.capacity, self.heads, piece_b,
                     self.max_rows, _native.ptr(ws.keys), _native.ptr(ws.values),
                     _native.stream_handle(self.device))
        return ws.keys, ws.values

    def attend(self, ws, shape, layer, query, out, keys=None, values=None):
        """One layer's fused verification attention (staged in the same
        launch when keys/values, device addresses of the new rows, are
        given).  Arguments depend only on the bucket, the layer and the
        given buffers; the transaction is read from the workspace at run
        time."""
        C = self.capacity
        k, v, sk, sv = self.layer_pointers[layer]
        tail = (ws.cu_query.data_ptr(), ws.cu_key.data_ptr(), ws.req.data_ptr(),
                shape.request_count, KV_HEADS * C * HEAD_DIM, HEAD_DIM, C * HEAD_DIM,
                shape.key_capacity, shape.maximum_query_length, SCALE, self.chunk,
                ws.work.data_ptr(), *self.launch_shape(shape), out, ws.attn.data_ptr(), ws.attn.numel(),
                _native.stream_handle(self.device))
        if keys is not None:
            _native.call('dspark_verify_attn_staged_fwd', query, k, v, keys, values, sk, sv, *tail)
        else:
            _native.call('dspark_verify_attn_fwd', query, k, v, sk, sv, *tail)

    def commit(self, ws, counts, max_query):
        """Copy each request's accepted prefix of scratch into its resident
        rows, every layer, in one launch (nothing to do when none is kept)."""
        if not any(counts):
            return
        acc = upload(self.device, counts)
        layer_b, slot_b, head_b, tok_b, piece_b = self.strides()
        _native.call('dspark_kv_commit', _native.ptr(self._keys), _native.ptr(self._values),
                     _native.ptr(self.scratch_keys), _native.ptr(self.scratch_values),
                     _native.ptr(ws.req), _native.ptr(ws.cu_query), _native.ptr(acc),
                     len(counts), max_query, self.layers, layer_b, slot_b, head_b, tok_b,
                     self.capacity, self.heads, piece_b, self.max_rows, _native.stream_handle(self.device))
