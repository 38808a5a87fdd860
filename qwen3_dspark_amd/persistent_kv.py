"""Persistent target KV store with transaction semantics on MI355X.

Drop-in for dspark_qwen/persistent_target_kv.py (PersistentTargetKV and its
Slot / Bucket / QueryFamily / Transaction / ExternalWriter types): the same
constructor, methods, validation order, error classes and messages, and
fail-closed poisoning.

Host design: the store is a small state machine.  Phase names where a round
stands (idle, open with eager staging, an external writer prepared /
submitted / published, poisoned) and a transition table lists which event
each phase admits; a refused event raises that event's error.  A slot ledger
tracks tenancy, incarnations and committed lengths.  Every device buffer and
launch lives in an injected device half (kv_device.HipKVDevice):

  begin             -> dspark_txn_metadata  (one launch; the reference builds
                       O(key capacity) Python lists and copies seven arrays)
  stage_layer       -> dspark_kv_stage
  prepare_attention -> dspark_kv_gather     (one pass instead of two
                       index_selects + where + masked_fill per tensor)
  commit            -> dspark_kv_commit     (all layers and requests, one launch)
  attend            -> dspark_verify_attn_fwd: causal attention reading the
                       resident rows and staged scratch rows in place; the
                       capacity-length K/V is never materialised.
"""
import enum
import heapq
from dataclasses import dataclass
from types import SimpleNamespace
from typing import Mapping

import torch

from .kernels import HEAD_DIM, KV_HEADS, Q_HEADS, SCALE, _check_scale
from .kv_device import MAX_BUCKET_REQUESTS, HipKVDevice
from .schedule import DEFAULT_CHUNK, SPLITS
from .xcd import clipped, normalised


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



class Phase(enum.Enum):
    """Where the store stands in a verification round."""
    IDLE = 'idle'                # no transaction: requests, prefixes and buckets may change
    OPEN = 'open'                # transaction begun; layers staged eagerly one by one
    PREPARED = 'prepared'        # a registered external writer holds the scratch, not yet submitted
    SUBMITTED = 'submitted'      # the external write is in flight on the device
    PUBLISHED = 'published'      # its completion was observed: every layer is staged
    POISONED = 'poisoned'        # a device write may have been lost: every call fails, for good


# (phase, event) -> next phase.  An event absent from a phase's row is refused
# with that event's error below; POISONED has no row.
_TRANSITIONS = {
    Phase.IDLE: {'admin': Phase.IDLE, 'begin': Phase.OPEN},
    Phase.OPEN: {'stage': Phase.OPEN, 'prepare_external': Phase.PREPARED, 'commit': Phase.IDLE,
                 'abort': Phase.IDLE},
    Phase.PREPARED: {'submit_external': Phase.SUBMITTED, 'abort': Phase.IDLE},
    Phase.SUBMITTED: {'complete_external': Phase.PUBLISHED, 'abort': Phase.IDLE},
    Phase.PUBLISHED: {'commit': Phase.IDLE, 'abort': Phase.IDLE},
}

# The error class and message of each refused event: the messages and classes
# callers of persistent_target_kv.py observe.
_REFUSALS = {
    'admin': (RuntimeError, 'Outstanding verification transaction'),
    'begin': (RuntimeError, 'Outstanding verification transaction'),
    'stage': (ValueError, 'Cannot mix eager and registered external scratch writes'),
    'prepare_external': (ValueError, 'Fresh transaction and exact registered external writer required'),
    'submit_external': (ValueError, 'External write must be submitted exactly once'),
    'complete_external': (ValueError, 'Submitted, unpublished external write required'),
    'commit': (ValueError, 'Complete layer scratch and one prefix count per active handle required'),
    'abort': (ValueError, 'Stale, copied or foreign transaction'),
}

_POISONED = 'Store invalidated by copy failure; construct a new store'


@dataclass
class _Tenant:
    handle: Slot
    length: int = 0


class _SlotLedger:
    """Which request owns each resident slot, under which incarnation, and
    how many committed rows it holds.

    Vacant slots sit in a min-heap, so admission reuses the lowest free slot.
    A slot's incarnation counter survives its tenants, so a handle of an
    earlier tenant never matches again.  `generation` changes with every
    change of tenancy or length: a transaction records it at begin and is
    valid only while it is unchanged.
    """

    def __init__(self, slots):
        self.tenants = [None] * slots
        self.incarnations = [0] * slots
        self.vacant = list(range(slots))
        self.by_request = {}
        self.generation = 0

    def admit(self, request):
        if not isinstance(request, str) or not request or request in self.by_request:
            raise ValueError('New nonempty request identity required')
        if not self.vacant:
            raise ValueError('Resident slot capacity exhausted')
        i = heapq.heappop(self.vacant)
        self.incarnations[i] += 1
        handle = Slot(request, i, self.incarnations[i])
        self.tenants[i] = _Tenant(handle)
        self.by_request[request] = i
        self.generation += 1
        return handle

    def release(self, i):
        # The slot's old rows stay allocated; no later handle can address them.
        del self.by_request[self.tenants[i].handle.request]
        self.tenants[i] = None
        heapq.heappush(self.vacant, i)
        self.generation += 1

    def locate(self, handle):
        """Slot index of a live handle (the very object admit returned)."""
        i = handle.index if isinstance(handle, Slot) else None
        if type(i) is int and 0 <= i < len(self.tenants) and self.tenants[i] is not None \
                and self.tenants[i].handle is handle:
            return i
        raise ValueError('Stale or foreign request incarnation')

    def length(self, i):
        return self.tenants[i].length

    def set_lengths(self, updates):
        for i, n in updates:
            self.tenants[i].length = n
        self.generation += 1

    def occupied(self):
        return len(self.by_request)

    def resident_rows(self):
        return sum(t.length for t in self.tenants if t is not None)


@dataclass
class _Registration:
    writer: ExternalWriter
    completion_check: object


class PersistentTargetKV:
    """Single-owner transaction store with stable resident and bucket addresses
    (the contract of persistent_target_kv.py:163-530).

    KV: [layers, resident slots, context capacity, KV heads, head dim];
    scratch: [layers, maximum query tokens, KV heads, head dim].  A handle
    binds a slot and its incarnation; one transaction is open at a time and
    nothing about requests or buckets changes meanwhile; commit copies only
    the accepted prefix of each request's staged rows; a failed device write
    poisons the store.

    The host state is a Phase with a transition table, a slot ledger and the
    open transaction; every device buffer and launch belongs to `kv_device`
    (a HipKVDevice unless one is injected), whose shape is documented in
    kv_device.py.
    """

    def __init__(self, *, layers, slots, context_capacity, max_query_tokens,
                 heads, dim, dtype=torch.bfloat16, device='cuda', chunk=DEFAULT_CHUNK, split='balanced',
                 kv_device=None):
        dims = (layers, slots, context_capacity, max_query_tokens, heads, dim)
        if any(type(n) is not int or n < 1 for n in dims):
            raise ValueError('All capacities and dimensions must be positive integers')
        if not dtype.is_floating_point:
            raise ValueError('Floating point KV dtype required')
        if split not in SPLITS:
            raise ValueError(f'split must be one of {SPLITS}')
        if kv_device is None:
            kv_device = HipKVDevice(layers=layers, slots=slots, context_capacity=context_capacity,
                                    max_query_tokens=max_query_tokens, heads=heads, dim=dim, dtype=dtype,
                                    device=device, chunk=int(chunk), split=split)
        self.kv_device = kv_device
        self.device = kv_device.device
        self.layers, self.slot_capacity, self.context_capacity = layers, slots, context_capacity
        self.max_query_tokens, self.heads, self.dim, self.dtype = max_query_tokens, heads, dim, dtype
        self.chunk, self.split = int(chunk), split
        self.keys, self.values = kv_device.keys, kv_device.values
        self.scratch_keys, self.scratch_values = kv_device.scratch_keys, kv_device.scratch_values
        self._phase = Phase.IDLE
        self._ledger = _SlotLedger(slots)
        self._workspaces = {}            # bucket or family -> Workspace
        self._arena = None               # (shape, Workspace) of the one family declaration
        self._families = ()
        self._registrations = {}         # id(writer) -> _Registration
        self._transactions = 0
        self._receipts = 0
        # the open transaction: Transaction, its ledger generation, staged layers, rows
        self._tx = None
        self._tx_generation = None
        self._staged = set()
        self._tx_rows = 0
        self._rope = {}                  # theta -> rotary table of the open transaction's rows
        self._receipt = None             # (ExternalWrite, completion event) while one is live

    # -- phase ------------------------------------------------------------
    @property
    def phase(self):
        return self._phase

    @property
    def failed(self):
        return self._phase is Phase.POISONED

    @property
    def open_transaction(self):
        """The transaction in flight (kept after poisoning), else None."""
        return self._tx

    def staged_layers(self):
        return len(self._staged)

    def _permit(self, event):
        """The phase `event` leads to, or raise the event's refusal."""
        if self._phase is Phase.POISONED:
            raise RuntimeError(_POISONED)
        nxt = _TRANSITIONS[self._phase].get(event)
        if nxt is None:
            cls, message = _REFUSALS[event]
            raise cls(message)
        return nxt

    def _poison(self):
        self._phase = Phase.POISONED

    def invalidate(self):
        """Fail closed after uncertain external or device writes; buffers are never reused."""
        self._poison()

    def _close(self):
        self._phase = Phase.IDLE
        self._tx, self._tx_generation, self._staged, self._receipt = None, None, set(), None

    def _index(self, handle):
        if self.failed:
            raise RuntimeError(_POISONED)
        return self._ledger.locate(handle)

    def _of(self, tx):
        """Workspace of the open transaction `tx`, after checking that it is
        the open one and that the committed state it was built on holds."""
        if self.failed:
            raise RuntimeError(_POISONED)
        if tx is not self._tx:
            raise ValueError('Stale, copied or foreign transaction')
        if self._ledger.generation != self._tx_generation:
            raise RuntimeError('Committed state changed during verification')
        return self._workspaces[tx.bucket]

    def _check_kv(self, keys, values, shape):
        for x in (keys, values):
            if (not isinstance(x, torch.Tensor) or tuple(x.shape) != shape
                    or x.device != self.device or x.dtype != self.dtype or x.requires_grad):
                raise ValueError('KV shape, device, dtype and no-autograd contract required')

    def _check_fused_storage(self, what):
        if (self.heads, self.dim, self.dtype) != (KV_HEADS, HEAD_DIM, torch.bfloat16):
            raise ValueError(f'{what} requires bf16 Hkv8/D128 storage')

    def _stage_target(self, layer):
        """Phase after staging `layer` eagerly: refuses external-writer
        rounds and a layer outside the model or already staged."""
        nxt = self._permit('stage')
        if type(layer) is not int or not 0 <= layer < self.layers or layer in self._staged:
            raise ValueError('Each model layer must stage exactly once')
        return nxt

    # -- requests --------------------------------------------------------------
    def add_request(self, request):
        self._permit('admin')
        return self._ledger.admit(request)

    def remove_request(self, handle):
        self._permit('admin')
        self._ledger.release(self._index(handle))

    def length(self, handle):
        return self._ledger.length(self._index(handle))

    @torch.no_grad()
    def load_prefix(self, handle, keys, values):
        """Bootstrap exact model KV [layers, n, heads, dim] into an empty slot."""
        self._permit('admin')
        i = self._index(handle)
        if self._ledger.length(i) or not isinstance(keys, torch.Tensor) or keys.ndim != 4:
            raise ValueError('Prefix bootstrap requires empty slot and [L,C,H,D] KV')
        n = keys.shape[1]
        if not 0 <= n <= self.context_capacity:
            raise ValueError('Prefix exceeds resident context capacity')
        self._check_kv(keys, values, (self.layers, n, self.heads, self.dim))
        try:
            self.kv_device.write_prefix(i, keys, values)
        except Exception:
            self._poison()
            raise
        self._ledger.set_lengths(((i, n),))

    def request_kv(self, handle):
        i = self._index(handle)
        return self.kv_device.copy_out(i, self._ledger.length(i))

    # -- buckets and families ------------------------------------------------------
    def is_registered(self, bucket):
        return bucket in self._workspaces

    def registered(self):
        """Every registered bucket and family."""
        return tuple(self._workspaces)

    def workspace(self, bucket):
        """Device buffers of a registered bucket or family."""
        return self._workspaces[bucket]

    # -- XCD-balanced plans (no reference counterpart) -------------------------
    @property
    def xcd_speed(self):
        """Relative speeds of the 8 XCDs that size the runs of later balanced
        plans (run w executes on XCD w mod 8), or None for equal runs."""
        return self.kv_device.xcd_speed

    def set_xcd_speed(self, speed):
        """Use the given 8 relative XCD speeds (positive, finite; None: equal
        runs) for the plans of later transactions."""
        self._permit('admin')
        self.kv_device.xcd_speed = normalised(speed)

    @property
    def slot_balance(self):
        """Whether later balanced plans give the runs whose workgroups are the
        second resident on their CUs a smaller share of the cost
        (schedule.SECOND_SLOT_SHARE; on by default)."""
        return self.kv_device.slot_balance

    def set_slot_balance(self, enabled):
        """Switch the second-slot share of later balanced plans on or off."""
        self._permit('admin')
        if not isinstance(enabled, bool):
            raise ValueError('slot balance must be True or False')
        self.kv_device.slot_balance = enabled

    def calibrate_xcd(self, *, workgroups=1024, passes=2, clip=0.25):
        """Measure the read bandwidth each XCD gets from this store's resident
        K/V and size the runs of later balanced plans to it, so that the
        XCDs finish together: the 8 XCDs of an MI355X do not read a given
        allocation equally fast, and which are slower depends on where it
        landed.  Relative speeds are clipped to 1 +- clip.  Opt-in: cut
        points then depend on the measurement, so outputs can differ in the
        last bits between processes (as between batches).  Returns the
        speeds in use: None (equal runs) when the measurement does not
        cover all 8 XCDs."""
        self._permit('admin')
        self.set_xcd_speed(clipped(self.kv_device.measure_xcd_speed(workgroups=workgroups, passes=passes), clip))
        return self.xcd_speed

    def register_bucket(self, bucket):
        self._permit('admin')
        if isinstance(bucket, QueryFamily):
            if bucket not in self._workspaces:
                raise ValueError('Family must belong to the explicitly registered shared arena')
            return
        if (not isinstance(bucket, Bucket) or bucket.request_count > self.slot_capacity
                or bucket.query_tokens > self.max_query_tokens
                or bucket.maximum_key_length > self.context_capacity):
            raise ValueError('Bucket exceeds resident/query capacity')
        if bucket.request_count > MAX_BUCKET_REQUESTS:
            raise ValueError(f'At most {MAX_BUCKET_REQUESTS} requests per bucket')
        if bucket not in self._workspaces:
            self._workspaces[bucket] = self.kv_device.workspace(bucket)

    def workspace_bytes(self, bucket):
        """Exact device allocation of a bucket workspace before registering it."""
        return self.kv_device.workspace_bytes(bucket)

    def family_arena_shape(self, families):
        """Validate a complete family declaration before allocating anything;
        returns the shape of the one arena all of them share."""
        valid = (isinstance(families, tuple) and families
                 and all(isinstance(f, QueryFamily) for f in families)
                 and len(set(families)) == len(families))
        if not valid or any(f.request_count > self.slot_capacity or f.query_tokens > self.max_query_tokens
                            or f.maximum_key_length > self.context_capacity for f in families):
            raise ValueError('Distinct finite families within resident/query capacity required')
        fields = ('request_count', 'query_tokens', 'key_capacity', 'maximum_query_length')
        return SimpleNamespace(**{name: max(getattr(f, name) for f in families) for name in fields})

    def register_families(self, families):
        """One immutable family declaration sharing one workspace; no resize."""
        self._permit('admin')
        if self._arena is not None:
            raise ValueError('Shared family arena already registered; no dynamic extension')
        shape = self.family_arena_shape(families)
        if shape.request_count > MAX_BUCKET_REQUESTS:
            raise ValueError(f'At most {MAX_BUCKET_REQUESTS} requests per bucket')
        arena = self.kv_device.workspace(shape)
        self._arena = (shape, arena)
        self._families = families
        self._workspaces.update((f, arena.view(f)) for f in families)

    # -- registered external scratch writers (persistent_target_kv.py:309-362) --
    def _scratch_pointers(self):
        return self.scratch_keys.data_ptr(), self.scratch_values.data_ptr()

    def register_external_writer(self, bucket, layers, completion_check):
        self._permit('admin')
        if bucket not in self._workspaces or tuple(layers) != tuple(range(self.layers)) or not callable(completion_check):
            raise ValueError('Registered bucket, complete ordered layer signature and completion checker required')
        writer = ExternalWriter(bucket, tuple(layers), self._scratch_pointers(),
                                self._workspaces[bucket].signature())
        self._registrations[id(writer)] = _Registration(writer, completion_check)
        return writer

    def prepare_external_write(self, tx, writer):
        self._of(tx)
        entry = self._registrations.get(id(writer))
        if entry is None or entry.writer is not writer or writer.bucket != tx.bucket or self._staged:
            raise ValueError(_REFUSALS['prepare_external'][1])
        self._phase = self._permit('prepare_external')
        self._receipts += 1
        receipt = ExternalWrite(writer, tx, self._receipts)
        self._receipt = (receipt, None)
        return receipt

    def _live_receipt(self, receipt):
        """Check that `receipt` is the live one, its transaction is open and
        the buffers its writer captured are still the store's."""
        if self._receipt is None or self._receipt[0] is not receipt:
            raise ValueError('Stale, copied or foreign external write receipt')
        self._of(receipt.transaction)
        if receipt.writer.scratch_pointers != self._scratch_pointers():
            self._poison()
            raise RuntimeError('Registered scratch allocation changed')
        if receipt.writer.workspace_signature != self._workspaces[receipt.transaction.bucket].signature():
            self._poison()
            raise RuntimeError('Registered workspace view/layout changed')

    def submit_external_write(self, receipt, event):
        self._live_receipt(receipt)
        self._phase = self._permit('submit_external')
        self._receipt = (receipt, event)

    def _observed(self):
        """Ask the live receipt's writer whether its write finished; a
        checker that raises poisons the store."""
        receipt, event = self._receipt
        try:
            return bool(self._registrations[id(receipt.writer)].completion_check(event, receipt))
        except BaseException:
            self._poison()
            raise

    def complete_external_write(self, receipt):
        self._live_receipt(receipt)
        nxt = self._permit('complete_external')
        if not self._observed():
            raise RuntimeError('External write completion has not been observed')
        self._staged = set(receipt.writer.layers)
        self._phase = nxt

    # -- transactions ------------------------------------------------------------
    @torch.no_grad()
    def begin(self, handles, bucket, *, query_lengths=None):
        """Validate on the host, then build the seven metadata arrays on the
        device (one small upload, one dspark_txn_metadata launch).  Nothing
        is published unless both succeed; a failed begin may be retried and
        never revives an earlier transaction."""
        nxt = self._permit('begin')
        handles = tuple(handles)
        if bucket not in self._workspaces or len(handles) != bucket.request_count:
            raise ValueError('Registered exact-query bucket required')
        if query_lengths is None:
            if isinstance(bucket, QueryFamily):
                raise ValueError('Family requires actual ordered query lengths')
            query_lengths = bucket.query_lengths
        query_lengths = tuple(query_lengths)
        slots = [self._index(h) for h in handles]
        if len(set(slots)) != len(slots):
            raise ValueError('Active request slots must be unique')
        contexts = tuple(self._ledger.length(i) for i in slots)
        if not bucket.accepts(query_lengths, contexts):
            raise ValueError('Actual context exceeds declared bucket applicability')
        if sum(contexts) + sum(query_lengths) >= 2 ** 31:
            raise ValueError('Varlen cumulative lengths exceed int32')
        self.kv_device.build_metadata(self._workspaces[bucket], bucket, slots, contexts, query_lengths)
        self._transactions += 1
        tx = Transaction(self._transactions, handles, contexts, bucket, query_lengths)
        self._phase, self._tx, self._tx_generation = nxt, tx, self._ledger.generation
        self._staged, self._tx_rows, self._receipt = set(), sum(query_lengths), None
        self._rope = {}                  # theta -> rotary table of this transaction's rows
        return tx

    @torch.no_grad()
    def stage_layer(self, tx, layer, keys, values):
        """Copy the model's new K/V rows of one layer into scratch only."""
        self._of(tx)
        self._stage_target(layer)
        self._check_kv(keys, values, (self._tx_rows, self.heads, self.dim))
        self.kv_device.stage(layer, keys, values, self._tx_rows)
        self._staged.add(layer)

    @torch.no_grad()
    def stage_projected(self, tx, layer, hidden, prologue):
        """Run the layer's attention prologue (QKVPrologue: q/k/v projection,
        q/k RMSNorm, RoPE at each row's absolute position) on the packed
        hidden states [sum Q, H] and write K/V straight into this layer's
        scratch - stage_layer without the separate copy.  Returns the
        queries [sum Q, 16, 128] for attend()."""
        ws = self._of(tx)
        self._stage_target(layer)
        self._check_fused_storage('The fused prologue')
        if not isinstance(hidden, torch.Tensor) or hidden.ndim != 2 or hidden.shape[0] != self._tx_rows:
            raise ValueError('Hidden states must be [sum Q, hidden] for the transaction')
        rope = self._rope.get(prologue.theta)
        if rope is None:                 # once per transaction: every layer's rows sit at the same positions
            rope = self._rope[prologue.theta] = prologue.rope_table(ws.positions)
        queries, _, _ = prologue(hidden, ws.positions, k_out=self.scratch_keys[layer], v_out=self.scratch_values[layer],
                                 rope=rope)
        self._staged.add(layer)
        return queries

    @torch.no_grad()
    def prepare_attention(self, tx, layer):
        """Materialise the capacity-length K/V of one layer (parity mode);
        attend() is the fused path that never builds it."""
        ws = self._of(tx)
        if layer not in self._staged:
            raise ValueError('Layer scratch missing')
        keys, values = self.kv_device.gather(ws, tx.bucket, layer)
        return keys, values, ws.cu_query, ws.cu_key, ws.positions

    @torch.no_grad()
    def attend(self, tx, layer, query, *, scale=SCALE, keys=None, values=None, out=None):
        """Bottom-right causal attention of one layer: request r's queries see
        its committed rows (resident) then its new rows, read in place.
        query [sum Q, 16, 128] bf16 -> output of the same shape.

        With keys/values (the layer's new [sum Q, 8, 128] rows) the layer is
        staged in the same launch: the kernel reads the new rows from them
        and copies them into scratch, exactly what stage_layer followed by
        attend does, minus one launch and one pass over the new rows.
        Otherwise the layer must have been staged.  out: an optional output
        buffer (written and returned)."""
        ws = self._of(tx)
        fused = keys is not None or values is not None
        if fused:
            self._stage_target(layer)
            self._check_kv(keys, values, (self._tx_rows, self.heads, self.dim))
            keys, values = keys.contiguous(), values.contiguous()
        elif layer not in self._staged:
            raise ValueError('Layer scratch missing')
        self._check_fused_storage('Fused attention')
        if (not isinstance(query, torch.Tensor) or query.dtype != torch.bfloat16 or query.device != self.device
                or query.shape != (self._tx_rows, Q_HEADS, HEAD_DIM) or not query.is_contiguous()
                or query.requires_grad):
            raise ValueError('Expected contiguous no-autograd bf16 [Q,16,128] queries on the store device')
        _check_scale(scale, 'Fused verification attention')
        if out is None:
            out = torch.empty_like(query)
        elif (not isinstance(out, torch.Tensor) or out.dtype != torch.bfloat16 or out.device != self.device
              or out.shape != query.shape or not out.is_contiguous()):
            raise ValueError('out must be a contiguous bf16 tensor shaped like the queries')
        self.kv_device.attend(ws, tx.bucket, layer, query.data_ptr(), out.data_ptr(),
                              keys.data_ptr() if fused else None, values.data_ptr() if fused else None)
        if fused:
            self._staged.add(layer)
        return out

    def launch_attention(self, bucket, layer, query, out, keys=None, values=None):
        """The fused attention launch of a registered bucket with raw device
        addresses and no transaction check: what a captured round records
        once and replays under an external-write receipt."""
        self.kv_device.attend(self._workspaces[bucket], bucket, layer, query, out, keys, values)

    @torch.no_grad()
    def commit(self, tx, committed_query_lengths: Mapping):
        """Commit caller-decided verified prefix lengths (anchor included).

        The whole decision is validated before any resident write; one
        launch then copies every layer of every request's accepted prefix.
        A failed launch poisons the store.
        """
        ws = self._of(tx)
        if (set(committed_query_lengths) != set(tx.slots) or len(self._staged) != self.layers
                or 'commit' not in _TRANSITIONS[self._phase]):
            raise ValueError(_REFUSALS['commit'][1])
        counts = [committed_query_lengths[h] for h in tx.slots]
        for n, c, q in zip(counts, tx.context_lengths, tx.query_lengths):
            if type(n) is not int or not 0 <= n <= q or c + n > self.context_capacity:
                raise ValueError('Commit must be a valid verified prefix')
        try:
            self.kv_device.commit(ws, counts, max(tx.query_lengths))
        except Exception:
            self._poison()
            raise
        self._ledger.set_lengths((h.index, c + n) for h, c, n in zip(tx.slots, tx.context_lengths, counts))
        self._close()
        total = sum(counts)
        return dict(committed_tokens=total,
                    copied_kv_bytes=2 * self.layers * self.heads * self.dim * self.keys.element_size() * total)

    def abort(self, tx):
        """Drop the open transaction's scratch (an external write in flight
        must have been observed finished first)."""
        self._of(tx)
        self._permit('abort')
        if self._phase is Phase.SUBMITTED and not self._observed():
            raise RuntimeError('Cannot abort buffers with an unfinished external write')
        self._close()

    def pointers(self, bucket):
        """Audit stable allocation identities."""
        return dict(committed_keys=self.keys.data_ptr(), committed_values=self.values.data_ptr(),
                    scratch_keys=self.scratch_keys.data_ptr(), scratch_values=self.scratch_values.data_ptr(),
                    **self._workspaces[bucket].pointers())

    def work(self, tx):
        """Work counters of the open transaction: the keys and formulas of
        persistent_target_kv.py:511-530, plus the rows the fused attention
        actually streams."""
        ws = self._of(tx)
        bucket, contexts, queries = tx.bucket, tx.context_lengths, tx.query_lengths
        rows, context_rows = sum(queries), sum(contexts)
        keys = context_rows + rows
        elem = self.keys.element_size()
        shared = isinstance(bucket, QueryFamily)
        counters = dict(
            active_requests=len(tx.slots), resident_requests=self._ledger.occupied(),
            logical_query_tokens=rows, physical_query_tokens=rows, logical_active_key_tokens=keys,
            physical_key_capacity=bucket.key_capacity, padded_key_capacity=bucket.key_capacity - keys,
            inactive_resident_key_tokens=self._ledger.resident_rows() - context_rows,
            gather_rows_per_kv_per_layer=2 * bucket.key_capacity,
            staging_output_rows_per_layer=bucket.key_capacity,
            allowed_causal_pairs=sum(c * n + n * (n + 1) // 2 for c, n in zip(contexts, queries)),
            query_lengths=list(queries), queried_context_lengths=list(contexts),
            maximum_query_length=bucket.maximum_query_length, maximum_key_length=bucket.maximum_key_length,
            resident_allocated_kv_bytes=2 * self.keys.numel() * elem,
            scratch_allocated_kv_bytes=2 * self.scratch_keys.numel() * elem,
            bucket_workspace_bytes=ws.nbytes(),
            workspace_is_shared=shared,
            shared_arena_allocated_bytes=self.workspace_bytes(self._arena[0]) if shared else 0)
        counters.update(fused_attention_key_rows_per_layer=keys, bucket_source=bucket.source,
                        capture_or_replay_verified=False)
        return counters
