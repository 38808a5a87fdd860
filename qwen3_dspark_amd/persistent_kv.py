"""Persistent target KV store with transaction semantics on MI355X.

Drop-in for dspark_qwen/persistent_target_kv.py (PersistentTargetKV and its
Slot / Bucket / QueryFamily / Transaction / ExternalWriter types): the same
constructor, methods, validation order, error classes and fail-closed
poisoning.  The device work is HIP:

  begin             -> dspark_txn_metadata  (one launch; the reference builds
                       O(key capacity) Python lists and copies seven arrays)
  stage_layer       -> dspark_kv_stage
  prepare_attention -> dspark_kv_gather     (one pass instead of two
                       index_selects + where + masked_fill per tensor)
  commit            -> dspark_kv_commit     (all layers and requests, one launch)
  attend            -> dspark_verify_attn_fwd: causal attention reading the
                       resident rows and staged scratch rows in place; the
                       capacity-length K/V is never materialised.

Layout in HBM: resident K and V are stored head-major,
[layers, slots, heads, context_capacity, dim], so the attention of one
(request, KV head) streams one contiguous run of 256-byte rows; `keys` /
`values` are [layers, slots, context_capacity, heads, dim] views of that
storage (the reference's shape).  Scratch K and V are token-major
[layers, max_query_tokens, heads, dim], the shape the model produces.
"""
from dataclasses import dataclass
from typing import Mapping

import torch

from . import _native
from ._device import cu_count, require_gfx950, upload
from .kernels import HEAD_DIM, KV_HEADS, Q_HEADS, SCALE, _check_scale
from .schedule import DEFAULT_CHUNK, REQ_INTS, SPLITS, WORK_INTS, run_count, segment_plan, varlen_list_bound


@dataclass(frozen=True)
class Slot:
    request: str
    index: int
    incarnation: int


@dataclass(frozen=True)
class Bucket:
    """Exact ordered query shape plus per-entry context ceilings
    (persistent_target_kv.py:21-62)."""
    query_lengths: tuple
    context_ceilings: tuple
    source: str

    def __post_init__(self):
        if (not self.query_lengths or len(self.query_lengths) != len(self.context_ceilings)
                or any(type(n) is not int or n < 1 for n in self.query_lengths)
                or any(type(n) is not int or n < 0 for n in self.context_ceilings)
                or not isinstance(self.source, str) or not self.source.strip()):
            raise ValueError('Bucket requires exact positive Q lengths, nonnegative C ceilings and provenance')
        if not isinstance(self.query_lengths, tuple) or not isinstance(self.context_ceilings, tuple):
            raise ValueError('Immutable tuple shapes required')

    @property
    def query_tokens(self):
        return sum(self.query_lengths)

    @property
    def key_capacity(self):
        return sum(self.query_lengths) + sum(self.context_ceilings)

    @property
    def request_count(self):
        return len(self.query_lengths)

    @property
    def maximum_query_length(self):
        return max(self.query_lengths)

    @property
    def maximum_key_length(self):
        return max(c + q for c, q in zip(self.context_ceilings, self.query_lengths))

    def accepts(self, queries, contexts):
        return (all(type(q) is int and q >= 1 for q in queries)
                and tuple(queries) == self.query_lengths and len(contexts) == self.request_count
                and all(type(c) is int and 0 <= c <= cap for c, cap in zip(contexts, self.context_ceilings)))


@dataclass(frozen=True)
class QueryFamily:
    """Fixed request count and launch bounds; actual ordered Q per transaction
    (persistent_target_kv.py:65-95)."""
    request_count: int
    query_tokens: int
    maximum_query_length: int
    key_capacity: int
    maximum_key_length: int
    source: str

    def __post_init__(self):
        values = (self.request_count, self.query_tokens, self.maximum_query_length,
                  self.key_capacity, self.maximum_key_length)
        if (any(type(n) is not int or n < 1 for n in values)
                or not self.request_count <= self.query_tokens <= self.request_count * self.maximum_query_length
                or self.key_capacity < self.query_tokens
                or self.maximum_key_length < self.maximum_query_length
                or not isinstance(self.source, str) or not self.source.strip()):
            raise ValueError('Positive feasible finite family bounds and provenance required')

    def accepts(self, queries, contexts):
        return (len(queries) == len(contexts) == self.request_count
                and all(type(q) is int and 1 <= q <= self.maximum_query_length for q in queries)
                and sum(queries) == self.query_tokens
                and all(type(c) is int and c >= 0 for c in contexts)
                and all(c + q <= self.maximum_key_length for c, q in zip(contexts, queries))
                and sum(contexts) + self.query_tokens <= self.key_capacity)


@dataclass(frozen=True)
class Transaction:
    sequence: int
    slots: tuple
    context_lengths: tuple
    bucket: object
    query_lengths: tuple


@dataclass(frozen=True)
class ExternalWriter:
    bucket: object
    layers: tuple
    scratch_pointers: tuple
    workspace_signature: tuple


@dataclass(frozen=True)
class ExternalWrite:
    writer: ExternalWriter
    transaction: Transaction
    generation: int


class _Workspace:
    """Per-bucket device metadata, materialised K/V and split-K partials.

    Arrays and meaning follow persistent_target_kv.py:127-153.  The reference's
    old/new intermediates do not exist: dspark_kv_gather writes keys/values
    directly.  `req` holds the per-request (slot, context, query) triples the
    kernels consume and `attn` the split-K partials of attend().
    """
    _COUNTS = {'cu_query': 'r1', 'cu_key': 'r1', 'positions': 'q', 'req': 'r3', 'work': 'full', 'attn': 'full'}

    def __init__(self, bucket, heads, dim, dtype, device, chunk, split, arena=None):
        self.bucket = bucket
        n, r, q = bucket.key_capacity, bucket.request_count, bucket.query_tokens
        if arena is not None:
            for name, value in vars(arena).items():
                if isinstance(value, torch.Tensor):
                    kind = self._COUNTS.get(name)
                    if kind == 'full':
                        setattr(self, name, value)
                    elif kind == 'r1':
                        setattr(self, name, value[:r + 1])
                    elif kind == 'q':
                        setattr(self, name, value[:q])
                    elif kind == 'r3':
                        setattr(self, name, value[:3 * r])
                    else:
                        setattr(self, name, value[:n])
            return
        self.committed_indices = torch.zeros(n, dtype=torch.long, device=device)
        self.scratch_indices = torch.zeros_like(self.committed_indices)
        self.from_scratch = torch.zeros((n, 1, 1), dtype=torch.bool, device=device)
        self.valid = torch.zeros((n, 1, 1), dtype=torch.bool, device=device)
        self.cu_query = torch.zeros(r + 1, dtype=torch.int32, device=device)
        self.cu_key = torch.zeros_like(self.cu_query)
        self.positions = torch.zeros(q, dtype=torch.long, device=device)
        self.req = torch.zeros(3 * r, dtype=torch.int32, device=device)
        self.work = torch.zeros(_work_ints(bucket, device, chunk, split), dtype=torch.int32, device=device)
        self.keys = torch.empty((n, heads, dim), dtype=dtype, device=device)
        self.values = torch.empty_like(self.keys)
        self.attn = torch.zeros(_attn_workspace_bytes(bucket, chunk, device, split), dtype=torch.uint8, device=device)

    def pointers(self):
        return {k: v.data_ptr() for k, v in vars(self).items() if isinstance(v, torch.Tensor) and v.is_cuda}

    def signature(self):
        return (id(self), tuple((k, v.data_ptr(), tuple(v.shape), tuple(v.stride()), v.storage_offset(), v.dtype, v.device)
                                for k, v in vars(self).items() if isinstance(v, torch.Tensor) and v.is_cuda))


def _max_runs(bucket, device):
    """Most balanced-list runs any transaction of the bucket uses (its key
    capacity bounds the keys of every transaction)."""
    return run_count(bucket.key_capacity, cu_count(device), (bucket.maximum_query_length + 7) // 8)


def _max_segments(bucket, device, chunk, split):
    g, r = _max_runs(bucket, device), bucket.request_count
    return varlen_list_bound(r, g, bucket.key_capacity, None if split == 'balanced' else chunk)


def _work_ints(bucket, device, chunk, split):
    """int32 length of the largest work list of the bucket."""
    g, r = _max_runs(bucket, device), bucket.request_count
    return WORK_INTS * _max_segments(bucket, device, chunk, split) + g + 1 + REQ_INTS * r


def _attn_workspace_bytes(bucket, chunk, device, split):
    """Split-K partials for the largest work list of the bucket (one slot
    per segment at most)."""
    tiles = (bucket.maximum_query_length + 7) // 8
    segments = _max_segments(bucket, device, chunk, split)
    return max(16, int(_native.load().dspark_attn_workspace_bytes(segments, 0, tiles, chunk)))


class PersistentTargetKV:
    """Single-owner transaction store with stable resident and bucket addresses.

    KV layout: [layers, resident slots, context capacity, KV heads, head dim].
    Scratch: [layers, maximum query tokens, KV heads, head dim].  Semantics
    of persistent_target_kv.py:163-530: handles bind slot and incarnation,
    one outstanding transaction, commit copies only the accepted prefix,
    a failed copy poisons the store.
    """

    def __init__(self, *, layers, slots, context_capacity, max_query_tokens,
                 heads, dim, dtype=torch.bfloat16, device='cuda', chunk=DEFAULT_CHUNK, split='balanced'):
        dims = (layers, slots, context_capacity, max_query_tokens, heads, dim)
        if any(type(n) is not int or n < 1 for n in dims):
            raise ValueError('All capacities and dimensions must be positive integers')
        if not dtype.is_floating_point:
            raise ValueError('Floating point KV dtype required')
        elem = torch.empty((), dtype=dtype).element_size()
        if (dim * elem) % 16:
            raise ValueError('A KV head row (dim * element size) must be a multiple of 16 bytes')
        self.device = require_gfx950(device)
        _native.load()
        self.layers, self.slot_capacity, self.context_capacity = layers, slots, context_capacity
        self.max_query_tokens, self.heads, self.dim = max_query_tokens, heads, dim
        self.dtype = dtype
        if split not in SPLITS:
            raise ValueError(f'split must be one of {SPLITS}')
        self.chunk = int(chunk)
        self.split = split
        self._elem = elem
        # Head-major storage; the public tensors are reference-shaped views.
        self._keys = torch.zeros((layers, slots, heads, context_capacity, dim), dtype=dtype, device=self.device)
        self._values = torch.zeros_like(self._keys)
        self.keys = self._keys.permute(0, 1, 3, 2, 4)
        self.values = self._values.permute(0, 1, 3, 2, 4)
        self.scratch_keys = torch.zeros((layers, max_query_tokens, heads, dim), dtype=dtype, device=self.device)
        self.scratch_values = torch.zeros_like(self.scratch_keys)
        self._owners = [None] * slots
        self._handles = [None] * slots
        self._incarnations = [0] * slots
        self._lengths = [0] * slots
        self._workspaces = {}
        self._family_arena = None
        self._families = ()
        self._sequence = 0
        self._pending = None
        self._staged = set()
        self._writers = {}
        self._external = None
        self._submission_generation = 0
        # Committed-state generation: bumped by every mutation of slots or
        # lengths; a transaction is valid only while it is unchanged, which
        # replaces a per-call scan over the transaction's handles.
        self._mutations = 0
        self._tx_mutations = None
        self._tx_shape = None
        # Per-layer device addresses (the allocations never move).
        lk, ls = self._keys[0].numel() * elem, self.scratch_keys[0].numel() * elem
        self._layer_ptrs = tuple((self._keys.data_ptr() + l * lk, self._values.data_ptr() + l * lk,
                                  self.scratch_keys.data_ptr() + l * ls, self.scratch_values.data_ptr() + l * ls)
                                 for l in range(layers))
        self.failed = False

    def _geometry(self):
        """Resident byte strides: (layer, slot, head, token) and piece bytes."""
        e, H, C, D = self._elem, self.heads, self.context_capacity, self.dim
        return (self.slot_capacity * H * C * D * e, H * C * D * e, C * D * e, D * e, D * e)

    # -- state guards ------------------------------------------------------
    def _healthy(self):
        if self.failed:
            raise RuntimeError('Store invalidated by copy failure; construct a new store')

    def _idle(self):
        self._healthy()
        if self._pending is not None:
            raise RuntimeError('Outstanding verification transaction')

    def _slot(self, handle):
        self._healthy()
        if (not isinstance(handle, Slot) or not 0 <= handle.index < self.slot_capacity
                or self._handles[handle.index] is not handle
                or self._owners[handle.index] != handle.request
                or self._incarnations[handle.index] != handle.incarnation):
            raise ValueError('Stale or foreign request incarnation')
        return handle.index

    # -- request lifecycle ---------------------------------------------------
    def add_request(self, request):
        self._idle()
        if not isinstance(request, str) or not request or request in self._owners:
            raise ValueError('New nonempty request identity required')
        if None not in self._owners:
            raise ValueError('Resident slot capacity exhausted')
        i = self._owners.index(None)
        self._incarnations[i] += 1
        self._owners[i], self._lengths[i] = request, 0
        handle = Slot(request, i, self._incarnations[i])
        self._handles[i] = handle
        self._mutations += 1
        return handle

    def remove_request(self, handle):
        self._idle()
        i = self._slot(handle)
        self._owners[i], self._lengths[i], self._handles[i] = None, 0, None
        self._mutations += 1

    def length(self, handle):
        return self._lengths[self._slot(handle)]

    def _kv(self, keys, values, shape):
        for x in (keys, values):
            if (not isinstance(x, torch.Tensor) or tuple(x.shape) != shape
                    or x.device != self.device or x.dtype != self.dtype or x.requires_grad):
                raise ValueError('KV shape, device, dtype and no-autograd contract required')

    @torch.no_grad()
    def load_prefix(self, handle, keys, values):
        """Bootstrap exact real-model KV into an empty resident slot."""
        self._idle()
        i = self._slot(handle)
        if self._lengths[i] or not isinstance(keys, torch.Tensor) or keys.ndim != 4:
            raise ValueError('Prefix bootstrap requires empty slot and [L,C,H,D] KV')
        n = keys.shape[1]
        if not 0 <= n <= self.context_capacity:
            raise ValueError('Prefix exceeds resident context capacity')
        self._kv(keys, values, (self.layers, n, self.heads, self.dim))
        try:
            self.keys[:, i, :n].copy_(keys)
            self.values[:, i, :n].copy_(values)
            self._lengths[i] = n
            self._mutations += 1
        except Exception:
            self.failed = True
            raise

    # -- buckets and families -------------------------------------------------
    def register_bucket(self, bucket):
        self._idle()
        if isinstance(bucket, QueryFamily):
            if bucket not in self._workspaces:
                raise ValueError('Family must belong to the explicitly registered shared arena')
            return
        if (not isinstance(bucket, Bucket) or len(bucket.query_lengths) > self.slot_capacity
                or bucket.query_tokens > self.max_query_tokens
                or any(c + q > self.context_capacity for c, q in zip(bucket.context_ceilings, bucket.query_lengths))):
            raise ValueError('Bucket exceeds resident/query capacity')
        if bucket.request_count > 4096:
            raise ValueError('At most 4096 requests per bucket')
        if bucket not in self._workspaces:
            self._workspaces[bucket] = _Workspace(bucket, self.heads, self.dim, self.dtype, self.device, self.chunk,
                                                  self.split)

    def workspace_bytes(self, bucket):
        """Exact device allocation of a bucket workspace before registering it."""
        n, r, q = bucket.key_capacity, bucket.request_count, bucket.query_tokens
        kv = 2 * n * self.heads * self.dim * self.keys.element_size()
        return (kv + 18 * n + 8 * (r + 1) + 8 * q + 12 * r + 4 * _work_ints(bucket, self.device, self.chunk, self.split)
                + _attn_workspace_bytes(bucket, self.chunk, self.device, self.split))

    def family_arena_shape(self, families):
        """Validate the complete finite declaration before allocating any storage."""
        from types import SimpleNamespace
        if (not isinstance(families, tuple) or not families
                or any(not isinstance(f, QueryFamily) for f in families)
                or len(set(families)) != len(families)
                or any(f.request_count > self.slot_capacity or f.query_tokens > self.max_query_tokens
                       or f.maximum_key_length > self.context_capacity for f in families)):
            raise ValueError('Distinct finite families within resident/query capacity required')
        return SimpleNamespace(request_count=max(f.request_count for f in families),
                               query_tokens=max(f.query_tokens for f in families),
                               key_capacity=max(f.key_capacity for f in families),
                               maximum_query_length=max(f.maximum_query_length for f in families))

    def register_families(self, families):
        """One immutable declaration and one shared workspace; no resize or lazy family."""
        self._idle()
        if self._family_arena is not None:
            raise ValueError('Shared family arena already registered; no dynamic extension')
        shape = self.family_arena_shape(families)
        if shape.request_count > 4096:
            raise ValueError('At most 4096 requests per bucket')
        arena = _Workspace(shape, self.heads, self.dim, self.dtype, self.device, self.chunk, self.split)
        views = {f: _Workspace(f, self.heads, self.dim, self.dtype, self.device, self.chunk, self.split, arena)
                 for f in families}
        self._family_arena = arena
        self._families = families
        self._workspaces.update(views)

    # -- registered external scratch writers (persistent_target_kv.py:309-362) --
    def register_external_writer(self, bucket, layers, completion_check):
        self._idle()
        if bucket not in self._workspaces or tuple(layers) != tuple(range(self.layers)) or not callable(completion_check):
            raise ValueError('Registered bucket, complete ordered layer signature and completion checker required')
        writer = ExternalWriter(bucket, tuple(layers),
                                (self.scratch_keys.data_ptr(), self.scratch_values.data_ptr()),
                                self._workspaces[bucket].signature())
        self._writers[id(writer)] = (writer, completion_check)
        return writer

    def prepare_external_write(self, tx, writer):
        self._transaction(tx)
        registered = self._writers.get(id(writer))
        if (registered is None or registered[0] is not writer or writer.bucket != tx.bucket
                or self._staged or self._external is not None):
            raise ValueError('Fresh transaction and exact registered external writer required')
        self._submission_generation += 1
        receipt = ExternalWrite(writer, tx, self._submission_generation)
        self._external = dict(receipt=receipt, state='prepared', event=None)
        return receipt

    def _external_write(self, receipt):
        if self._external is None or self._external['receipt'] is not receipt:
            raise ValueError('Stale, copied or foreign external write receipt')
        self._transaction(receipt.transaction)
        if receipt.writer.scratch_pointers != (self.scratch_keys.data_ptr(), self.scratch_values.data_ptr()):
            self.failed = True
            raise RuntimeError('Registered scratch allocation changed')
        if receipt.writer.workspace_signature != self._workspaces[receipt.transaction.bucket].signature():
            self.failed = True
            raise RuntimeError('Registered workspace view/layout changed')
        return self._external

    def submit_external_write(self, receipt, event):
        state = self._external_write(receipt)
        if state['state'] != 'prepared':
            raise ValueError('External write must be submitted exactly once')
        state.update(state='submitted', event=event)

    def complete_external_write(self, receipt):
        state = self._external_write(receipt)
        if state['state'] != 'submitted':
            raise ValueError('Submitted, unpublished external write required')
        checker = self._writers[id(receipt.writer)][1]
        if not self._check_external_completion(checker, state['event'], receipt):
            raise RuntimeError('External write completion has not been observed')
        self._staged = set(receipt.writer.layers)
        state['state'] = 'completed'

    def _check_external_completion(self, checker, event, receipt):
        try:
            return bool(checker(event, receipt))
        except BaseException:
            self.failed = True
            raise

    def invalidate(self):
        """Fail closed after uncertain external/device writes; never reuse buffers."""
        self.failed = True

    # -- transactions ---------------------------------------------------------
    @torch.no_grad()
    def begin(self, handles, bucket, *, query_lengths=None):
        """Validate on the host, then build all seven metadata arrays with one
        small pinned upload and one dspark_txn_metadata launch.  No
        transaction is published unless both succeed."""
        self._idle()
        handles = tuple(handles)
        if bucket not in self._workspaces or len(handles) != bucket.request_count:
            raise ValueError('Registered exact-query bucket required')
        if query_lengths is None:
            if isinstance(bucket, QueryFamily):
                raise ValueError('Family requires actual ordered query lengths')
            query_lengths = bucket.query_lengths
        query_lengths = tuple(query_lengths)
        indices = [self._slot(h) for h in handles]
        if len(set(indices)) != len(indices):
            raise ValueError('Active request slots must be unique')
        contexts = tuple(self._lengths[i] for i in indices)
        if not bucket.accepts(query_lengths, contexts):
            raise ValueError('Actual context exceeds declared bucket applicability')
        if sum(contexts) + sum(query_lengths) >= 2 ** 31:
            raise ValueError('Varlen cumulative lengths exceed int32')
        ws = self._workspaces[bucket]
        r = len(handles)
        key_lengths = [c + q for c, q in zip(contexts, query_lengths)]
        runs = run_count(sum(key_lengths), cu_count(self.device), (bucket.maximum_query_length + 7) // 8)
        # fixed-capacity list: the same launch for every transaction of the bucket
        capacity = (_max_segments(bucket, self.device, self.chunk, self.split), _max_runs(bucket, self.device))
        records, n_items, runs = segment_plan(self.split, query_lengths, key_lengths, indices, runs, self.chunk,
                                              capacity)
        if len(records) > ws.work.numel():
            raise ValueError('Work list exceeds the bucket workspace')
        upload(self.device, list(indices) + list(contexts) + list(query_lengths), out=ws.req[:3 * r])
        upload(self.device, records, out=ws.work[:len(records)])
        _native.call('dspark_txn_metadata', _native.ptr(ws.req), r, self.context_capacity,
                     bucket.key_capacity, bucket.query_tokens,
                     _native.ptr(ws.committed_indices), _native.ptr(ws.scratch_indices),
                     _native.ptr(ws.from_scratch), _native.ptr(ws.valid), _native.ptr(ws.positions),
                     _native.ptr(ws.cu_query), _native.ptr(ws.cu_key), _native.stream_handle(self.device))
        self._sequence += 1
        tx = Transaction(self._sequence, handles, contexts, bucket, query_lengths)
        self._pending, self._staged = tx, set()
        self._tx_mutations = self._mutations
        # (query tokens, launch maximum query length, bucket key capacity)
        self._tx_shape = (sum(query_lengths), bucket.maximum_query_length, bucket.key_capacity)
        return tx

    def _transaction(self, tx):
        self._healthy()
        if tx is not self._pending:
            raise ValueError('Stale, copied or foreign transaction')
        if self._mutations != self._tx_mutations:
            raise RuntimeError('Committed state changed during verification')
        return self._workspaces[tx.bucket]

    @torch.no_grad()
    def stage_layer(self, tx, layer, keys, values):
        """Copy the model's new KV rows of one layer into scratch only."""
        self._transaction(tx)
        if self._external is not None:
            raise ValueError('Cannot mix eager and registered external scratch writes')
        if type(layer) is not int or not 0 <= layer < self.layers or layer in self._staged:
            raise ValueError('Each model layer must stage exactly once')
        q = self._tx_shape[0]
        self._kv(keys, values, (q, self.heads, self.dim))
        keys, values = keys.contiguous(), values.contiguous()
        _, _, sk, sv = self._layer_ptrs[layer]
        _native.call('dspark_kv_stage', keys.data_ptr(), values.data_ptr(), sk, sv,
                     q, self.heads * self.dim * self._elem, _native.stream_handle(self.device))
        self._staged.add(layer)

    @torch.no_grad()
    def stage_projected(self, tx, layer, hidden, prologue):
        """Run the layer's attention prologue (QKVPrologue: q/k/v projection,
        q/k RMSNorm, RoPE at each row's absolute position) on the packed
        hidden states [sum Q, H] and write K/V straight into this layer's
        scratch - stage_layer without the separate copy.  Returns the
        queries [sum Q, 16, 128] for attend()."""
        ws = self._transaction(tx)
        if self._external is not None:
            raise ValueError('Cannot mix eager and registered external scratch writes')
        if type(layer) is not int or not 0 <= layer < self.layers or layer in self._staged:
            raise ValueError('Each model layer must stage exactly once')
        if (self.heads, self.dim, self.dtype) != (KV_HEADS, HEAD_DIM, torch.bfloat16):
            raise ValueError('The fused prologue requires bf16 Hkv8/D128 storage')
        q = self._tx_shape[0]
        if not isinstance(hidden, torch.Tensor) or hidden.ndim != 2 or hidden.shape[0] != q:
            raise ValueError('Hidden states must be [sum Q, hidden] for the transaction')
        queries, _, _ = prologue(hidden, ws.positions, k_out=self.scratch_keys[layer], v_out=self.scratch_values[layer])
        self._staged.add(layer)
        return queries

    @torch.no_grad()
    def prepare_attention(self, tx, layer):
        """Materialise the capacity-length K/V (parity mode); attend() is the
        fused path that never builds it."""
        ws = self._transaction(tx)
        if layer not in self._staged:
            raise ValueError('Layer scratch missing')
        n = tx.bucket.key_capacity
        _, slot_b, head_b, tok_b, piece_b = self._geometry()
        _native.call('dspark_kv_gather', _native.ptr(self._keys[layer]), _native.ptr(self._values[layer]),
                     _native.ptr(self.scratch_keys[layer]), _native.ptr(self.scratch_values[layer]),
                     _native.ptr(ws.committed_indices), _native.ptr(ws.scratch_indices),
                     _native.ptr(ws.from_scratch), _native.ptr(ws.valid), n,
                     self.slot_capacity, slot_b, head_b, tok_b, self.context_capacity, self.heads, piece_b,
                     self.max_query_tokens, _native.ptr(ws.keys), _native.ptr(ws.values),
                     _native.stream_handle(self.device))
        return ws.keys, ws.values, ws.cu_query, ws.cu_key, ws.positions

    @torch.no_grad()
    def attend(self, tx, layer, query, *, scale=SCALE, keys=None, values=None, out=None):
        """Bottom-right causal attention of one layer: request r's queries see
        its committed rows (resident) then its new rows, read in place.
        query [sum Q, 16, 128] bf16 -> output of the same shape.

        With keys/values (the layer's new [sum Q, 8, 128] rows) the layer is
        staged in the same launch: the kernel reads the new rows from them
        and copies them into scratch, exactly what stage_layer followed by
        attend does, minus one launch and one pass over the new rows.
        Otherwise the layer must have been staged with stage_layer.  out: an
        optional output buffer (written and returned)."""
        self._transaction(tx)
        fused = keys is not None or values is not None
        if fused:
            if self._external is not None:
                raise ValueError('Cannot mix eager and registered external scratch writes')
            if type(layer) is not int or not 0 <= layer < self.layers or layer in self._staged:
                raise ValueError('Each model layer must stage exactly once')
            self._kv(keys, values, (self._tx_shape[0], self.heads, self.dim))
            keys, values = keys.contiguous(), values.contiguous()
        elif layer not in self._staged:
            raise ValueError('Layer scratch missing')
        if (self.heads, self.dim, self.dtype) != (KV_HEADS, HEAD_DIM, torch.bfloat16):
            raise ValueError('Fused attention requires bf16 Hkv8/D128 storage')
        q = self._tx_shape[0]
        if (not isinstance(query, torch.Tensor) or query.dtype != torch.bfloat16 or query.device != self.device
                or query.shape != (q, Q_HEADS, HEAD_DIM) or not query.is_contiguous() or query.requires_grad):
            raise ValueError('Expected contiguous no-autograd bf16 [Q,16,128] queries on the store device')
        _check_scale(scale, 'Fused verification attention')
        if out is None:
            out = torch.empty_like(query)
        elif (not isinstance(out, torch.Tensor) or out.dtype != torch.bfloat16 or out.device != self.device
              or out.shape != query.shape or not out.is_contiguous()):
            raise ValueError('out must be a contiguous bf16 tensor shaped like the queries')
        self._attention_launch(tx.bucket, layer, query.data_ptr(), out.data_ptr(),
                               keys.data_ptr() if fused else None, values.data_ptr() if fused else None)
        if fused:
            self._staged.add(layer)
        return out

    def _launch_shape(self, bucket):
        """(record capacity, runs) of the bucket's fixed-capacity work list."""
        return _max_segments(bucket, self.device, self.chunk, self.split), _max_runs(bucket, self.device)

    def _attention_launch(self, bucket, layer, query, out, keys=None, values=None):
        """One layer's fused verification attention (staged when keys/values
        are given) for the bucket's workspace.  Every argument depends only on
        the bucket, the layer and the given buffers; the transaction's data is
        read from the workspace at run time, so a captured launch replays for
        every later transaction of the bucket."""
        ws = self._workspaces[bucket]
        C = self.context_capacity
        k, v, sk, sv = self._layer_ptrs[layer]
        tail = (ws.cu_query.data_ptr(), ws.cu_key.data_ptr(), ws.req.data_ptr(),
                bucket.request_count, KV_HEADS * C * HEAD_DIM, HEAD_DIM, C * HEAD_DIM,
                bucket.key_capacity, bucket.maximum_query_length, SCALE, self.chunk,
                ws.work.data_ptr(), *self._launch_shape(bucket), out, ws.attn.data_ptr(), ws.attn.numel(),
                _native.stream_handle(self.device))
        if keys is not None:
            _native.call('dspark_verify_attn_staged_fwd', query, k, v, keys, values, sk, sv, *tail)
        else:
            _native.call('dspark_verify_attn_fwd', query, k, v, sk, sv, *tail)

    @torch.no_grad()
    def commit(self, tx, committed_query_lengths: Mapping):
        """Commit caller-decided verified prefix lengths (anchor included).

        The whole decision is validated before any resident write; all
        layers and requests are then copied by one kernel.  A launch failure
        poisons the store.
        """
        ws = self._transaction(tx)
        if set(committed_query_lengths) != set(tx.slots) or len(self._staged) != self.layers:
            raise ValueError('Complete layer scratch and one prefix count per active handle required')
        counts = []
        for h, c, q in zip(tx.slots, tx.context_lengths, tx.query_lengths):
            n = committed_query_lengths[h]
            if type(n) is not int or not 0 <= n <= q or c + n > self.context_capacity:
                raise ValueError('Commit must be a valid verified prefix')
            counts.append(n)
        r = len(tx.slots)
        try:
            if any(counts):
                acc = upload(self.device, counts)
                layer_b, slot_b, head_b, tok_b, piece_b = self._geometry()
                _native.call('dspark_kv_commit', _native.ptr(self._keys), _native.ptr(self._values),
                             _native.ptr(self.scratch_keys), _native.ptr(self.scratch_values),
                             _native.ptr(ws.req), _native.ptr(ws.cu_query), _native.ptr(acc),
                             r, max(tx.query_lengths), self.layers, layer_b, slot_b, head_b, tok_b,
                             self.context_capacity, self.heads, piece_b, self.max_query_tokens,
                             _native.stream_handle(self.device))
            for h, n in zip(tx.slots, counts):
                self._lengths[h.index] += n
            self._mutations += 1
        except Exception:
            self.failed = True
            raise
        self._pending, self._staged, self._external = None, set(), None
        total = sum(counts)
        return dict(committed_tokens=total,
                    copied_kv_bytes=2 * self.layers * self.heads * self.dim * self.keys.element_size() * total)

    def abort(self, tx):
        self._transaction(tx)
        if self._external is not None and self._external['state'] == 'submitted':
            receipt = self._external['receipt']
            if not self._check_external_completion(self._writers[id(receipt.writer)][1], self._external['event'], receipt):
                raise RuntimeError('Cannot abort buffers with an unfinished external write')
        self._pending, self._staged, self._external = None, set(), None

    def request_kv(self, handle):
        i = self._slot(handle)
        n = self._lengths[i]
        return (self.keys[:, i, :n].detach().clone(memory_format=torch.contiguous_format),
                self.values[:, i, :n].detach().clone(memory_format=torch.contiguous_format))

    def pointers(self, bucket):
        """Audit stable allocation identities."""
        return dict(committed_keys=self.keys.data_ptr(), committed_values=self.values.data_ptr(),
                    scratch_keys=self.scratch_keys.data_ptr(), scratch_values=self.scratch_values.data_ptr(),
                    **self._workspaces[bucket].pointers())

    def work(self, tx):
        """Work counters with the keys and formulas of persistent_target_kv.py:511-530,
        plus the rows the fused attention actually streams."""
        self._transaction(tx)
        q = sum(tx.query_lengths)
        actual_k = sum(tx.context_lengths) + q
        resident = sum(self._lengths)
        ws = self._workspaces[tx.bucket]
        return dict(active_requests=len(tx.slots), resident_requests=sum(x is not None for x in self._owners),
                    logical_query_tokens=q, physical_query_tokens=q, logical_active_key_tokens=actual_k,
                    physical_key_capacity=tx.bucket.key_capacity, padded_key_capacity=tx.bucket.key_capacity - actual_k,
                    inactive_resident_key_tokens=resident - sum(tx.context_lengths),
                    gather_rows_per_kv_per_layer=2 * tx.bucket.key_capacity,
                    staging_output_rows_per_layer=tx.bucket.key_capacity,
                    allowed_causal_pairs=sum(c * n + n * (n + 1) // 2 for c, n in zip(tx.context_lengths, tx.query_lengths)),
                    query_lengths=list(tx.query_lengths), queried_context_lengths=list(tx.context_lengths),
                    maximum_query_length=tx.bucket.maximum_query_length, maximum_key_length=tx.bucket.maximum_key_length,
                    resident_allocated_kv_bytes=2 * self.keys.numel() * self.keys.element_size(),
                    scratch_allocated_kv_bytes=2 * self.scratch_keys.numel() * self.keys.element_size(),
                    bucket_workspace_bytes=sum(t.numel() * t.element_size() for t in vars(ws).values()
                                               if isinstance(t, torch.Tensor) and t.is_cuda),
                    workspace_is_shared=isinstance(tx.bucket, QueryFamily),
                    shared_arena_allocated_bytes=(self.workspace_bytes(self._family_arena.bucket)
                                                  if isinstance(tx.bucket, QueryFamily) else 0),
                    fused_attention_key_rows_per_layer=actual_k,
                    bucket_source=tx.bucket.source, capture_or_replay_verified=False)
