"""Hugging Face transformers adapters for the DSpark attention hot path.

* varlen_attention_forward - the attention-registry callback of
  dspark_qwen/varlen_target.py:115-129: [1,Hq,Q,D] queries, a PackedLayout
  over the model's [1,Hkv,N,D] cache, HIP gather + HIP varlen kernel,
  [1,Q,Hq,D] out.
* FusedVerificationCache + fused_verification_attention - the verification
  hooks of dspark_qwen/persistent_qwen_target.py:45-95.  The reference's
  update stages the layer and materialises the capacity-length K/V with
  prepare_attention for the kernel; here update only checks the new rows and
  the callback passes them to PersistentTargetKV.attend, whose one launch
  stages them and attends over resident + new rows in place.
* FusedVerifier - binds a PersistentTargetKV transaction to one model forward
  (the callback finds it through the `fused_verification` forward kwarg, as
  the reference passes `persistent_target`).
* PersistentQwenTarget - the full-model transaction adapter of
  dspark_qwen/persistent_qwen_target.py:100-472 (verify / commit / abort /
  prefill / predict / request_kv, captured layer features) on that path.
* VarlenPackedTarget + PackedVarlenCache - the append-order adapter of
  dspark_qwen/varlen_target.py:132-167 over PackedTarget
  (packed_target.py:30-200): one packed forward per append over an
  AppendOrderKV, a PackedLayout per forward, the varlen callback per layer,
  and the reference's work counters.

The callbacks keep the reference's contract: no attention mask or dropout,
the module must belong to the bound model, ValueError otherwise.
"""
import contextlib
import weakref
from collections.abc import Mapping
from dataclasses import dataclass

import torch
from transformers import Cache
from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

from . import backends
from ._device import upload
from .kernels import HEAD_DIM, KV_HEADS, Q_HEADS, HipCapacityKernel
from .layout import PackedLayout
from .packed_kv import AppendOrderKV
from .persistent_kv import Bucket, PersistentTargetKV, QueryFamily
from .schedule import DEFAULT_CHUNK

VARLEN_BACKEND = 'dspark_mi355x_varlen'
FUSED_BACKEND = 'dspark_mi355x_fused_verify'


def varlen_attention_forward(module, query, key, value, attention_mask, scaling=None, dropout=0.0,
                             packed_layout=None, packed_varlen_kernel=None, **kwargs):
    """Registry callback with the contract of varlen_target.py:115-129."""
    if attention_mask is not None or dropout:
        raise ValueError('Varlen callback requires metadata-only causal attention without dropout')
    if not isinstance(packed_layout, PackedLayout) or packed_varlen_kernel is None:
        raise ValueError('Missing explicit packed layout/kernel')
    if query.ndim != 4 or query.shape[0] != 1 or query.shape[2] != packed_layout.query_tokens:
        raise ValueError('Expected [1,Hq,Q,D] query with layout Q')
    q = query.squeeze(0).transpose(0, 1).contiguous()
    k, v = packed_layout.gather_kv(key, value)
    out = packed_varlen_kernel(q, k, v, packed_layout, scale=scaling)
    if not isinstance(out, torch.Tensor) or out.shape != q.shape or out.dtype != q.dtype or out.device != q.device:
        raise RuntimeError('Varlen kernel returned an incompatible output')
    return out[None], None


class FusedVerificationCache(Cache):
    """Cache.update for one verification transaction: check the layer's new
    K/V rows against the transaction and return them unchanged.  The
    callback hands them to the fused attention, which copies them into the
    store's scratch in the same launch that attends (and reads the committed
    rows from the resident store in place)."""

    def __init__(self, verifier):
        super().__init__(layers=[])
        self.verifier = verifier

    @property
    def is_compileable(self):
        return False

    def update(self, key_states, value_states, layer_idx, *args, **kwargs):
        v = self.verifier
        tx = v.transaction
        if tx is None:
            raise RuntimeError('Cache update outside owned transaction')
        q = sum(tx.query_lengths)
        expected = (1, v.store.heads, q, v.store.dim)
        if tuple(key_states.shape) != expected or value_states.shape != key_states.shape:
            raise ValueError('HF layer KV differs from exact packed query shape')
        return key_states, value_states

    def get_seq_length(self, layer_idx=0):
        return sum(self.verifier.store.length(h) for h in self.verifier.handles)

    def get_mask_sizes(self, *args, **kwargs):
        raise RuntimeError('Fused verification requires explicit request-local attention metadata')

    def get_max_cache_shape(self, layer_idx=0):
        return self.verifier.store.slot_capacity * self.verifier.store.context_capacity


def fused_verification_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0,
                                 fused_verification=None, **kwargs):
    """Registry callback of persistent_qwen_target.py:45-60 on the fused path."""
    v = fused_verification
    if not isinstance(v, FusedVerifier) or v.transaction is None:
        raise ValueError('Owned persistent verification transaction required')
    if attention_mask is not None or dropout or v.attention_module(module.layer_idx) is not module:
        raise ValueError('Unexpected mask/dropout/foreign model attention')
    q = query[0].transpose(0, 1).contiguous()
    out = v.store.attend(v.transaction, module.layer_idx, q, scale=scaling,
                         keys=key[0].transpose(0, 1).contiguous(), values=value[0].transpose(0, 1).contiguous())
    if not isinstance(out, torch.Tensor) or out.shape != q.shape or out.dtype != q.dtype or out.device != q.device:
        raise ValueError('Persistent attention returned incompatible output')
    return out[None], None


class FusedVerifier:
    """One HF Qwen3 model over a PersistentTargetKV: registers the fused
    callback, owns the verification cache and binds a transaction to each
    forward.

        verifier = FusedVerifier(model, store)
        with verifier.transaction_for(handles, bucket) as tx:
            logits = verifier.forward(input_ids, position_ids)
        store.commit(tx, accepted)          # or store.abort(tx)
    """

    def __init__(self, model, store):
        if not isinstance(store, PersistentTargetKV):
            raise ValueError('PersistentTargetKV store required')
        cfg = model.config
        if (cfg.num_hidden_layers != store.layers or cfg.num_key_value_heads != store.heads
                or cfg.head_dim != store.dim):
            raise ValueError('Model attention geometry differs from the store')
        self.model = model.eval().requires_grad_(False)
        self.store = store
        self.cache = FusedVerificationCache(self)
        self.transaction = None
        self.handles = ()
        ALL_ATTENTION_FUNCTIONS.register(FUSED_BACKEND, fused_verification_attention)
        cfg._attn_implementation = FUSED_BACKEND

    def attention_module(self, layer_idx):
        return self.model.model.layers[layer_idx].self_attn

    @contextlib.contextmanager
    def transaction_for(self, handles, bucket, *, query_lengths=None):
        if self.transaction is not None:
            raise RuntimeError('Finish existing verification transaction first')
        tx = self.store.begin(handles, bucket, query_lengths=query_lengths)
        self.transaction, self.handles = tx, tuple(handles)
        try:
            yield tx
        finally:
            self.transaction = None

    @torch.no_grad()
    def forward(self, input_ids, position_ids):
        """Packed verification forward: input_ids/position_ids [1, sum Q]
        (request-local absolute positions); returns the model output."""
        if self.transaction is None:
            raise RuntimeError('Forward outside owned transaction')
        return self.model(input_ids=input_ids, position_ids=position_ids, attention_mask=None,
                          past_key_values=self.cache, use_cache=True, fused_verification=self)


# ---------------------------------------------------------------------------
# Full-model transaction adapter (dspark_qwen/persistent_qwen_target.py:100-472)
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class CachedFeatures:
    """One request's slice of a verification forward (cached_target.py:15-22)."""
    start: int
    last: torch.Tensor
    context: torch.Tensor

    @property
    def end(self):
        return self.start + self.last.shape[1]


@dataclass(frozen=True)
class PackedFeatures:
    """Hidden states of one packed verification forward (packed_target.py:18-28):
    last [1, sum Q, hidden], context = captured layer outputs concatenated on
    the feature axis (or None), spans request -> (offset, count, start)."""
    last: torch.Tensor
    context: object
    spans: dict
    work: dict

    def for_request(self, request_id):
        offset, count, start = self.spans[request_id]
        return CachedFeatures(start, self.last[:, offset:offset + count],
                              None if self.context is None else self.context[:, offset:offset + count])


GRAPH_BACKEND = 'mi355x_hip_full_model_graph'


@dataclass(frozen=True)
class GraphTicket:
    """A prepared graph verification: the open transaction, the store's
    external-write receipt, the captured program and the request spans."""
    transaction: object
    receipt: object
    execution: object
    spans: dict


@dataclass(frozen=True)
class GraphCompletion:
    """A submitted replay and the event recorded after it on the owner stream."""
    ticket: GraphTicket
    event: object


class FullModelGraph:
    """One captured verification forward of a registered bucket: the
    embedding, every decoder layer (with its fused stage + attention
    launches) and the final norm, replayed under the store's external-write
    receipts (FullTargetExecution + TorchGraphBackend,
    persistent_qwen_graph.py:97-275).  Token ids go into a fixed buffer; the
    positions come from the bucket's fixed workspace; the last hidden states
    and captured layer features live in the graph's memory and are
    overwritten by the next replay (hence the target's feature lease)."""
    kind = GRAPH_BACKEND

    def __init__(self, target, bucket, reserve_bytes):
        self.target, self.bucket, self.reserve_bytes = target, bucket, reserve_bytes
        self.ids = torch.zeros((1, bucket.query_tokens), dtype=torch.long, device=target.device)
        self.writer = target.store.register_external_writer(bucket, range(target.store.layers), self.complete)
        self.graph = None
        self.last = self.context = None
        self.invalid = False
        self._submitted = {}      # id(receipt) -> (receipt, event)
        self._addresses = None

    @staticmethod
    def output_buffer_bytes(target, bucket):
        """Fixed buffers a capture keeps besides the graph's own pool: ids,
        last hidden states and captured features."""
        hidden = target.model.config.hidden_size
        return bucket.query_tokens * (8 + 2 * hidden * (1 + len(target.layer_ids)))

    def pointers(self):
        return dict(ids=self.ids.data_ptr(), last=None if self.last is None else self.last.data_ptr(),
                    context=None if self.context is None else self.context.data_ptr(),
                    **self.target.store.pointers(self.bucket))

    def validate(self):
        if self.invalid or self.target.store.failed:
            raise RuntimeError('Captured program invalidated')
        if self._addresses is not None and self.pointers() != self._addresses:
            raise RuntimeError('Captured buffer addresses changed')

    def load(self, chunks):
        self.ids.copy_(torch.cat(tuple(chunks.values()), dim=1))

    def _forward(self):
        t = self.target
        out = t.model.model(input_ids=self.ids, position_ids=t.store.workspace(self.bucket).positions[None],
                            attention_mask=None, past_key_values=t.verifier.cache, use_cache=True, return_dict=True,
                            fused_verification=t.verifier)
        if t.store.staged_layers() != t.store.layers or set(t._captured) != set(t.layer_ids):
            raise RuntimeError('Full layer cache update or selected feature capture missing')
        context = torch.cat([t._captured[i] for i in t.layer_ids], dim=-1) if t.layer_ids else None
        t._captured = {}
        return out.last_hidden_state, context

    @torch.no_grad()
    def capture(self, handles, query_lengths):
        """One eager forward (lazy library state settles), then the capture,
        each in a transaction of its own that is aborted: nothing runs
        during capture and nothing is committed."""
        t = self.target
        if self.graph is not None:
            raise ValueError('Bucket already captured')
        for capture in (False, True):
            with t.verifier.transaction_for(handles, self.bucket, query_lengths=query_lengths) as tx:
                try:
                    if not capture:
                        self._forward()
                    else:
                        device = t.device
                        stream = torch.cuda.Stream(device=device)
                        stream.wait_stream(torch.cuda.current_stream(device))
                        graph = torch.cuda.CUDAGraph()
                        with torch.cuda.graph(graph, stream=stream):
                            self.last, self.context = self._forward()
                        torch.cuda.current_stream(device).wait_stream(stream)
                        stream.synchronize()
                        self.graph = graph
                finally:
                    t._captured = {}
                    t.store.abort(tx)
        self._addresses = self.pointers()

    def submit(self, receipt):
        """Replay on the current stream; returns the event recorded after it."""
        self.validate()
        self.graph.replay()
        event = torch.cuda.Event()
        event.record(torch.cuda.current_stream(self.target.device))
        self._submitted = {id(receipt): (receipt, event)}
        return event

    def complete(self, event, receipt):
        """The store's completion check: this program's event for this
        receipt, observed complete."""
        entry = self._submitted.get(id(receipt))
        return entry is not None and entry[0] is receipt and entry[1] is event and event.query()


class PersistentQwenTarget:
    """HF Qwen3 target over a PersistentTargetKV with the fused MI355X
    attention: the API of persistent_qwen_target.py:100-472.

    verify() runs one packed forward whose layers stage their new K/V rows
    into scratch and attend over resident + scratch rows in place; nothing is
    committed until commit() keeps the caller's accepted prefixes (the rest
    is rolled back by omission).  prefill() = verify + commit of every row.
    Decoder outputs of `layer_ids` are captured as draft context features.
    A registered graph bucket (register_graph_bucket + capture_graph) is
    verified by replaying the captured full-model forward under the store's
    external-write receipts; verify_eager() remains the explicit eager path.
    Every call comes from the stream current at construction (the owner
    stream); features are leases that predict() checks by identity.
    """
    BACKEND_NAME = FUSED_BACKEND

    def __init__(self, model, layer_ids=(), *, slots, context_capacity, max_query_tokens, chunk=DEFAULT_CHUNK,
                 graph_backend=None, max_buckets=32, workspace_byte_budget=256 * 1024 ** 2, max_graph_buckets=0,
                 graph_byte_budget=0):
        cfg = model.config
        if (cfg.model_type != 'qwen3' or getattr(cfg, 'use_sliding_window', False)
                or any(kind != 'full_attention' for kind in cfg.layer_types)
                or (cfg.rope_parameters or {}).get('rope_type', 'default') != 'default'):
            raise ValueError('Owned dense Qwen3 with default RoPE required')
        if (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim) != (16, 8, 128):
            raise ValueError('The MI355X attention path requires 16 query heads, 8 KV heads, head dim 128')
        self.layer_ids = tuple(layer_ids)
        if (tuple(sorted(set(self.layer_ids))) != self.layer_ids
                or any(type(i) is not int or not 0 <= i < cfg.num_hidden_layers for i in self.layer_ids)):
            raise ValueError('Unique increasing valid decoder layer IDs required')
        device = model.get_input_embeddings().weight.device
        dtype = model.get_input_embeddings().weight.dtype
        if dtype != torch.bfloat16:
            raise ValueError('The MI355X attention path requires a bf16 model')
        if any(type(x) is not int or x < 1 for x in (max_buckets, workspace_byte_budget)):
            raise ValueError('Positive finite bucket/workspace budget required')
        if graph_backend is not None:
            if graph_backend != GRAPH_BACKEND:
                raise ValueError('Explicit device-compatible graph backend required')
            if any(type(x) is not int or x < 1 for x in (max_graph_buckets, graph_byte_budget)):
                raise ValueError('Positive finite graph count and byte budget required')
        self._old_backend = cfg._attn_implementation
        self.store = PersistentTargetKV(layers=cfg.num_hidden_layers, slots=slots, context_capacity=context_capacity,
                                        max_query_tokens=max_query_tokens, heads=cfg.num_key_value_heads,
                                        dim=cfg.head_dim, dtype=dtype, device=device, chunk=chunk)
        self.verifier = FusedVerifier(model, self.store)
        self.model = self.verifier.model
        # The kernel identity the reference's session guard reads
        # (packed_sampling.py:110-115): the capacity-tail drop-in of
        # _native_attention.  verify() itself runs the fused store attention.
        self._varlen_kernel = HipCapacityKernel(device)
        self._graph_backend = graph_backend
        self._max_buckets, self._workspace_budget = max_buckets, workspace_byte_budget
        self._max_graph_buckets, self._graph_budget = max_graph_buckets, graph_byte_budget
        self._workspace_bytes = self._graph_reserved_bytes = 0
        self._handles = {}
        self._pending = None
        self._captured = {}
        self._graphs = {}
        self._graph_ticket = self._graph_completion = self._feature_lease = None
        self._features = weakref.WeakValueDictionary()
        self._closed = False
        self._owner_stream = torch.cuda.current_stream(device).cuda_stream
        self._hooks = [self.model.model.layers[i].register_forward_hook(self._hook(i)) for i in self.layer_ids]

    @property
    def device(self):
        return self.store.device

    @property
    def lengths(self):
        return {r: self.store.length(h) for r, h in self._handles.items()}

    def _hook(self, index):
        def capture(_module, _inputs, output):
            if self.verifier.transaction is None:
                raise RuntimeError('Foreign model forward while the adapter owns the model')
            self._captured[index] = output[0] if isinstance(output, tuple) else output
        return capture

    # -- ownership -------------------------------------------------------------
    def _check_stream(self):
        if torch.cuda.current_stream(self.device).cuda_stream != self._owner_stream:
            raise RuntimeError('Target, head, draft feature consumers and release must use the owner stream')

    def _idle(self):
        self._check_stream()
        if self._closed:
            raise RuntimeError('Target adapter closed')
        if self._pending is not None or self.verifier.transaction is not None:
            raise RuntimeError('Finish existing verification transaction first')
        if self._graph_ticket is not None or self._feature_lease is not None:
            raise RuntimeError('Finish graph submission and release feature lease first')
        if self.store.failed:
            raise RuntimeError('Store invalidated by copy failure; construct a new store')
        if self.store.open_transaction is not None:
            raise RuntimeError('Outstanding verification transaction')

    def invalidate(self):
        """Fail closed after an uncertain asynchronous or device failure."""
        self.store.invalidate()
        for graph in self._graphs.values():
            graph.invalid = True
        self._pending = self._graph_ticket = self._graph_completion = None

    def release_features(self, features):
        self._check_stream()
        if self._features.get(id(features)) is not features:
            raise ValueError('Foreign, copied or already released features')
        if self._pending is not None and self._pending[0] is features:
            raise RuntimeError('Commit or abort before releasing feature lease')
        if self._feature_lease is features:
            self._feature_lease = None
        del self._features[id(features)]

    # -- requests and buckets ---------------------------------------------------------
    def add_request(self, request):
        self._idle()
        handle = self.store.add_request(request)
        self._handles[request] = handle
        return handle

    def remove_request(self, request):
        self._idle()
        self.store.remove_request(self._handles[request])
        del self._handles[request]

    def reset(self):
        """Release every request incarnation; bucket addresses stay."""
        self._idle()
        for request in tuple(self._handles):
            self.remove_request(request)

    def close(self):
        self._idle()
        for hook in self._hooks:
            hook.remove()
        self._hooks = []
        self.model.config._attn_implementation = self._old_backend
        self._closed = True

    def _fits(self, size, count):
        if len(self._registered()) + count > self._max_buckets or self._workspace_bytes + size > self._workspace_budget:
            raise ValueError('Finite bucket/workspace budget exceeded')
        if self._graph_backend is not None and self._workspace_bytes + size + self._graph_reserved_bytes > self._graph_budget:
            raise ValueError('Combined graph/workspace byte budget exceeded')

    def _registered(self):
        return self.store.registered()

    def register_bucket(self, bucket):
        self._idle()
        if isinstance(bucket, QueryFamily):
            self.store.register_bucket(bucket)
            return
        if not isinstance(bucket, Bucket):
            raise ValueError('Explicit Bucket or QueryFamily required')
        if not self.store.is_registered(bucket):
            size = self.store.workspace_bytes(bucket)
            self._fits(size, 1)
            self.store.register_bucket(bucket)
            self._workspace_bytes += size

    def register_families(self, families):
        """One finite family declaration sharing one workspace."""
        self._idle()
        size = self.store.workspace_bytes(self.store.family_arena_shape(families))
        self._fits(size, len(families))
        self.store.register_families(families)
        self._workspace_bytes += size

    def _validate_chunks(self, chunks, bucket):
        if not isinstance(chunks, Mapping) or not chunks or not isinstance(bucket, (Bucket, QueryFamily)):
            raise ValueError('Nonempty ordered token mapping and explicit bucket required')
        queries = tuple(x.shape[1] if isinstance(x, torch.Tensor) and x.ndim == 2 else -1 for x in chunks.values())
        lengths = self.lengths
        if not bucket.accepts(queries, tuple(lengths.get(r, -1) for r in chunks)):
            raise ValueError('Ordered query lengths and contexts must match the chosen bucket or family')
        for request, ids in chunks.items():
            if request not in self._handles:
                raise ValueError('Request not resident')
            if ids.shape[0] != 1 or ids.dtype != torch.long or ids.device != self.device:
                raise ValueError('Each token chunk must be [1,Q] long on target device')
            if bool(((ids < 0) | (ids >= self.model.config.vocab_size)).any()):
                raise ValueError('Token outside vocabulary')

    @staticmethod
    def _spans(chunks, tx):
        spans, offset = {}, 0
        for request, c, q in zip(chunks, tx.context_lengths, tx.query_lengths):
            spans[request] = (offset, q, c)
            offset += q
        return spans

    def _publish(self, features, tx, *, lease):
        self._pending = (features, tx)
        self._features[id(features)] = features
        if lease:
            self._feature_lease = features
        return features

    # -- graph buckets (persistent_qwen_target.py:243-336) ------------------------------
    def register_graph_bucket(self, bucket, *, reserve_bytes):
        """Explicit registration; reserve_bytes covers the capture's own pool."""
        self._idle()
        if self._graph_backend is None or type(reserve_bytes) is not int or reserve_bytes < 1:
            raise ValueError('Graph backend and positive allocation reservation required')
        if bucket in self._graphs or len(self._graphs) >= self._max_graph_buckets:
            raise ValueError('Duplicate graph bucket or finite graph count exceeded')
        workspace = 0 if self.store.is_registered(bucket) else self.store.workspace_bytes(bucket)
        extra = FullModelGraph.output_buffer_bytes(self, bucket) + reserve_bytes
        if self._workspace_bytes + workspace + self._graph_reserved_bytes + extra > self._graph_budget:
            raise ValueError('Combined graph/workspace byte budget exceeded')
        self.register_bucket(bucket)
        self._graphs[bucket] = FullModelGraph(self, bucket, reserve_bytes)
        self._graph_reserved_bytes += extra

    @torch.no_grad()
    def capture_graph(self, chunks, *, bucket):
        """Set-up only: capture the bucket's full-model forward (token ids and
        query lengths of `chunks` shape the capture; nothing is committed)."""
        self._idle()
        self._validate_chunks(chunks, bucket)
        if bucket not in self._graphs:
            raise ValueError('Explicit registered graph bucket required')
        ex = self._graphs[bucket]
        try:
            ex.load(chunks)
            ex.capture(tuple(self._handles[r] for r in chunks), tuple(ids.shape[1] for ids in chunks.values()))
        except BaseException:
            self.invalidate()
            raise

    @torch.no_grad()
    def prepare_graph_verify(self, chunks, *, bucket):
        self._idle()
        self._validate_chunks(chunks, bucket)
        ex = self._graphs.get(bucket)
        if ex is None or ex.graph is None:
            raise ValueError('Explicitly captured bucket required; no capture-on-miss')
        ex.validate()
        tx = self.store.begin(tuple(self._handles[r] for r in chunks), bucket,
                              query_lengths=tuple(ids.shape[1] for ids in chunks.values()))
        try:
            ex.load(chunks)
            receipt = self.store.prepare_external_write(tx, ex.writer)
            self._graph_ticket = GraphTicket(tx, receipt, ex, self._spans(chunks, tx))
            return self._graph_ticket
        except BaseException:
            self.store.abort(tx)
            raise

    @torch.no_grad()
    def submit_graph(self, ticket):
        self._check_stream()
        if ticket is not self._graph_ticket or self._graph_completion is not None:
            raise ValueError('Exact unsubmitted graph ticket required')
        try:
            event = ticket.execution.submit(ticket.receipt)
            self.store.submit_external_write(ticket.receipt, event)
            self._graph_completion = GraphCompletion(ticket, event)
            return self._graph_completion
        except BaseException:
            self.invalidate()
            raise

    @torch.no_grad()
    def finish_graph(self, completion, *, wait=True):
        self._check_stream()
        if completion is None or completion is not self._graph_completion:
            raise ValueError('Exact submitted graph completion required')
        ticket = completion.ticket
        ex = ticket.execution
        try:
            if wait:
                completion.event.synchronize()
            ready = ex.complete(completion.event, ticket.receipt)
        except BaseException:
            self.invalidate()
            raise
        if not ready:
            raise RuntimeError('Graph completion has not been observed')
        try:
            self.store.complete_external_write(ticket.receipt)
            ex.validate()
            work = self.store.work(ticket.transaction)
            work.update(model_forward_calls=1, layers=self.store.layers, selected_layer_ids=list(self.layer_ids),
                        attention_backend=self.BACKEND_NAME, execution_kind=ex.kind,
                        committed_write_policy='scratch_only_until_explicit_commit',
                        graph_scope='HF embedding, every decoder layer with the fused stage + attention, final '
                                    'norm; head and sampling outside',
                        graph_reserved_bytes=self._graph_reserved_bytes, workspace_bytes=self._workspace_bytes)
            features = PackedFeatures(ex.last, ex.context, ticket.spans, work)
            self._graph_ticket = self._graph_completion = None
            return self._publish(features, ticket.transaction, lease=True)
        except BaseException:
            self.invalidate()
            raise

    def cancel_graph(self, ticket):
        self._check_stream()
        if ticket is not self._graph_ticket:
            raise ValueError('Exact graph ticket required')
        try:
            self.store.abort(ticket.transaction)      # refuses an unfinished external write
        except BaseException:
            if self.store.failed:
                self.invalidate()
            raise
        self._graph_ticket = self._graph_completion = None

    # -- verification ------------------------------------------------------------
    @torch.no_grad()
    def verify(self, chunks, *, bucket):
        """One packed forward over {request: ids [1, q]} in bucket order:
        the captured program for a registered graph bucket, else eager."""
        if bucket in self._graphs:
            return self.finish_graph(self.submit_graph(self.prepare_graph_verify(chunks, bucket=bucket)))
        return self.verify_eager(chunks, bucket=bucket)

    @torch.no_grad()
    def verify_eager(self, chunks, *, bucket):
        """The explicit eager forward, also on registered graph buckets."""
        self._idle()
        self._validate_chunks(chunks, bucket)
        handles = tuple(self._handles[r] for r in chunks)
        query_lengths = tuple(ids.shape[1] for ids in chunks.values())
        self._captured = {}
        with self.verifier.transaction_for(handles, bucket, query_lengths=query_lengths) as tx:
            try:
                out = self.model.model(input_ids=torch.cat(tuple(chunks.values()), dim=1),
                                       position_ids=self.store.workspace(tx.bucket).positions[None],
                                       attention_mask=None, past_key_values=self.verifier.cache, use_cache=True,
                                       return_dict=True, fused_verification=self.verifier)
                if self.store.staged_layers() != self.store.layers or set(self._captured) != set(self.layer_ids):
                    raise RuntimeError('Full layer cache update or selected feature capture missing')
            except BaseException:
                if self.store.open_transaction is tx and not self.store.failed:
                    self.store.abort(tx)
                raise
            finally:
                captured, self._captured = self._captured, {}
        context = torch.cat([captured[i] for i in self.layer_ids], dim=-1) if self.layer_ids else None
        work = self.store.work(tx)
        work.update(model_forward_calls=1, layers=self.store.layers, selected_layer_ids=list(self.layer_ids),
                    attention_backend=self.BACKEND_NAME, workspace_bytes=self._workspace_bytes,
                    committed_write_policy='scratch_only_until_explicit_commit')
        if isinstance(bucket, QueryFamily):
            work['execution_kind'] = 'explicit_eager'
        features = PackedFeatures(out.last_hidden_state.detach(), None if context is None else context.detach(),
                                  self._spans(chunks, tx), work)
        return self._publish(features, tx, lease=False)

    @torch.no_grad()
    def commit(self, features, committed_query_lengths):
        self._check_stream()
        if self._pending is None or self._pending[0] is not features:
            raise ValueError('Only the outstanding verification features can commit')
        if not isinstance(committed_query_lengths, Mapping) or set(committed_query_lengths) != set(features.spans):
            raise ValueError('One committed query prefix per verified request required')
        _, tx = self._pending
        result = self.store.commit(tx, {self._handles[r]: n for r, n in committed_query_lengths.items()})
        self._pending = None
        return result

    def abort(self, features):
        self._check_stream()
        if self._pending is None or self._pending[0] is not features:
            raise ValueError('Only outstanding verification features can abort')
        self.store.abort(self._pending[1])
        self._pending = None

    @torch.no_grad()
    def prefill(self, chunks, *, bucket):
        self._idle()
        if any(self.lengths.get(r) != 0 for r in chunks):
            raise ValueError('Prefill is only for newly admitted empty requests')
        features = (self.verify_eager(chunks, bucket=bucket) if bucket in self._graphs
                    else self.verify(chunks, bucket=bucket))
        self.commit(features, {r: ids.shape[1] for r, ids in chunks.items()})
        return features

    @torch.no_grad()
    def predict(self, features, last_only=False):
        """The model's LM head over the verified rows (after its final norm)."""
        self._check_stream()
        if self._features.get(id(features)) is not features:
            raise ValueError('Foreign or released features')
        logits = self.model.get_output_embeddings()(features.last)
        return {r: (logits[:, offset + count - 1] if last_only else logits[:, offset:offset + count])
                for r, (offset, count, _) in features.spans.items()}

    def request_kv(self, request):
        """Per layer (keys, values) [1, Hkv, C, D] copies of a request's committed rows."""
        keys, values = self.store.request_kv(self._handles[request])
        return tuple((k.transpose(0, 1)[None], v.transpose(0, 1)[None]) for k, v in zip(keys, values))


# ---------------------------------------------------------------------------
# Append-order adapter (dspark_qwen/varlen_target.py:132-167 over
# dspark_qwen/packed_target.py:30-200)
# ---------------------------------------------------------------------------

def _check_dense_qwen3(model):
    """The model checks of packed_target.py:31-40 plus the geometry and dtype
    the HIP kernels take."""
    cfg = model.config
    if (cfg.model_type != 'qwen3' or getattr(cfg, 'use_sliding_window', False)
            or any(kind != 'full_attention' for kind in cfg.layer_types)):
        raise ValueError('Only dense full-attention Qwen3 is supported')
    if (cfg.rope_parameters or {}).get('rope_type', 'default') != 'default':
        raise ValueError('Only default RoPE: dynamic scaling can couple request lengths')
    if (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim) != (Q_HEADS, KV_HEADS, HEAD_DIM):
        raise ValueError('The MI355X attention path requires 16 query heads, 8 KV heads, head dim 128')
    if model.get_input_embeddings().weight.dtype != torch.bfloat16:
        raise ValueError('The MI355X attention path requires a bf16 model')


class PackedVarlenCache(Cache):
    """HF cache over an AppendOrderKV: update() grows the layer by the
    forward's new rows (one launch) and returns the layer's whole
    [1, Hkv, N, D] K/V, from which the varlen callback gathers each
    request's rows through the forward's PackedLayout."""

    def __init__(self, target):
        super().__init__(layers=[])
        self.target = target

    @property
    def is_compileable(self):
        return False

    def update(self, key_states, value_states, layer_idx, *args, **kwargs):
        return self.target.kv.append_layer(layer_idx, key_states.contiguous(), value_states.contiguous())

    def get_seq_length(self, layer_idx=0):
        return self.target.kv.rows

    def get_mask_sizes(self, *args, **kwargs):
        raise RuntimeError('Packed varlen attention requires explicit request-local layout metadata')

    def get_max_cache_shape(self, layer_idx=0):
        return -1


class VarlenPackedTarget:
    """HF Qwen3 target over an append-order packed cache with the MI355X
    varlen kernel: the API of VarlenPackedTarget / PackedTarget
    (add_request / append / crop / remove_request / lengths / request_kv /
    predict / reset).

    append() runs one real model forward for any active subset of the
    requests.  Each layer's cache update appends the new rows in one launch;
    the attention callback gathers every active request's rows (the
    layout's gather indices) and runs the causal varlen kernel, so inactive
    requests' rows are never attended.  The work counters carry the keys of
    packed_target.py:177-188 and varlen_target.py:152-167.  A failed forward
    resets every request (the layers may have grown unevenly), as the
    reference does.
    """

    def __init__(self, model, layer_ids=(), *, native_backend=backends.TARGET_BACKEND):
        _check_dense_qwen3(model)
        cfg = model.config
        self.layer_ids = tuple(layer_ids)
        if (tuple(sorted(set(self.layer_ids))) != self.layer_ids
                or any(type(i) is not int or not 0 <= i < cfg.num_hidden_layers for i in self.layer_ids)):
            raise ValueError('layer_ids must be unique increasing decoder block indices')
        if native_backend != backends.TARGET_BACKEND:
            raise ValueError('Unknown explicit native varlen backend')
        device = model.get_input_embeddings().weight.device
        self._varlen_kernel = backends.target_kernel(native_backend, device)
        self.model = model.eval().requires_grad_(False)
        self.kv = AppendOrderKV(layers=cfg.num_hidden_layers, heads=KV_HEADS, dim=HEAD_DIM, dtype=torch.bfloat16,
                                device=device)
        self.cache = PackedVarlenCache(self)
        ALL_ATTENTION_FUNCTIONS.register(VARLEN_BACKEND, varlen_attention_forward)
        cfg._attn_implementation = VARLEN_BACKEND

    @property
    def device(self):
        return self.kv.device

    @property
    def lengths(self):
        return self.kv.lengths

    def reset(self):
        self.kv.reset()

    def add_request(self, request_id):
        self.kv.add_request(request_id)

    def crop(self, request_id, length):
        self.kv.crop(request_id, length)

    def remove_request(self, request_id):
        self.kv.remove_request(request_id)

    def request_kv(self, request_id):
        return self.kv.request_kv(request_id)

    def _validate_chunks(self, chunks):
        if not isinstance(chunks, Mapping) or not chunks:
            raise ValueError('Need a nonempty request-to-token mapping')
        for request, ids in chunks.items():
            self.kv.marker(request)
            if (not isinstance(ids, torch.Tensor) or ids.ndim != 2 or ids.shape[0] != 1
                    or ids.shape[1] < 1 or ids.dtype != torch.long or ids.device != self.device):
                raise ValueError('Each chunk needs nonempty [1,q] long IDs on the model device')
            if bool(((ids < 0) | (ids >= self.model.config.vocab_size)).any()):
                raise ValueError('Token outside vocabulary')

    def _work(self, chunks, layout, lengths):
        """The counters of packed_target.py:177-188 and varlen_target.py:152-167
        for this forward (mask extents are zero: no mask exists)."""
        cfg = self.model.config
        counts = [ids.shape[1] for ids in chunks.values()]
        starts = [lengths[r] for r in chunks]
        q, k = sum(counts), sum(lengths.values()) + sum(counts)
        causal = sum(n * c + n * (n + 1) // 2 for n, c in zip(counts, starts))
        within = sum(n * (c + n) for n, c in zip(counts, starts))
        per_token_kv_bytes = 2 * KV_HEADS * HEAD_DIM * 2
        return dict(
            queried_requests=len(chunks), resident_requests=len(lengths),
            logical_query_tokens=q, physical_query_tokens=q, physical_kv_tokens=k, physical_kv_tokens_before=k - q,
            query_lengths=counts, queried_context_lengths=starts,
            resident_context_lengths_before=list(lengths.values()),
            dense_attention_pairs_per_head_layer=q * k, allowed_causal_pairs=causal,
            masked_cross_request_pairs=q * k - within, masked_future_pairs=within - causal,
            attention_heads=cfg.num_attention_heads, layers=cfg.num_hidden_layers,
            dense_attention_pairs_all_heads_layers=q * k * cfg.num_attention_heads * cfg.num_hidden_layers,
            model_forward_calls=1,
            attention_backend=getattr(self._varlen_kernel, 'backend_name', None), mask_shape=None, mask_bytes=0,
            active_kv_gather_tokens=layout.gathered_key_tokens,
            inactive_kv_tokens_excluded=layout.physical_key_tokens - layout.gathered_key_tokens,
            kv_gather_payload_bytes_per_layer=layout.gathered_key_tokens * per_token_kv_bytes,
            varlen_pair_domain_per_head_layer=layout.pair_domain,
            varlen_cross_request_pair_domain=0,
            attention_adapter_calls_per_layer=1,
            native_varlen_calls_per_layer=getattr(self._varlen_kernel, 'native_varlen_calls_per_layer', 0),
            scope='Metadata-only varlen layout on the MI355X HIP kernels; dense Q*K counts are counterfactual '
                  'domains, no mask is built')

    @torch.no_grad()
    def append(self, chunks):
        """One packed forward over the ordered {request: ids [1, q]}; returns
        PackedFeatures (last hidden states, captured layer outputs, spans,
        work counters).  Invalid inputs fail before any mutation."""
        self._validate_chunks(chunks)
        lengths = self.kv.lengths
        spans, markers, positions, offset = {}, [], [], 0
        for request, ids in chunks.items():
            count, start = ids.shape[1], lengths[request]
            spans[request] = (offset, count, start)
            markers += [self.kv.marker(request)] * count
            positions += range(start, start + count)
            offset += count
        meta = upload(self.device, markers + positions, torch.long)
        q_requests, q_positions = meta[:offset], meta[offset:]
        layout = PackedLayout.from_metadata(q_requests, q_positions, torch.cat((self.kv.key_requests, q_requests)),
                                            torch.cat((self.kv.key_positions, q_positions)))
        work = self._work(chunks, layout, lengths)
        captured, hooks = {}, []

        def hook_for(index):
            def hook(_module, _inputs, output):
                captured[index] = output[0] if isinstance(output, tuple) else output
            return hook
        try:
            for index in self.layer_ids:
                hooks.append(self.model.model.layers[index].register_forward_hook(hook_for(index)))
            output = self.model.model(input_ids=torch.cat(tuple(chunks.values()), dim=1),
                                      position_ids=q_positions[None], attention_mask={'full_attention': None},
                                      past_key_values=self.cache, use_cache=True, return_dict=True,
                                      packed_layout=layout, packed_varlen_kernel=self._varlen_kernel)
            self.kv.commit_rows({r: ids.shape[1] for r, ids in chunks.items()})
        except Exception:
            self.kv.reset()
            raise
        finally:
            for hook in hooks:
                hook.remove()
        context = torch.cat([captured[i] for i in self.layer_ids], dim=-1) if self.layer_ids else None
        return PackedFeatures(output.last_hidden_state.detach(), None if context is None else context.detach(),
                              spans, work)

    @torch.no_grad()
    def predict(self, features, last_only=False):
        """The model's LM head over the physical query rows, split by request
        span (packed_target.py:216-224)."""
        logits = self.model.get_output_embeddings()(features.last)
        return {r: (logits[:, offset + count - 1] if last_only else logits[:, offset:offset + count])
                for r, (offset, count, _) in features.spans.items()}
