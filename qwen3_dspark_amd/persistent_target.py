"""The full-model verification target on MI355X: an HF Qwen3 model over a
PersistentTargetKV with the fused stage + gather + attention launch in every
layer.  Drop-in for PersistentQwenTarget (dspark_qwen/persistent_qwen_target.py:100-472):
the same constructor arguments, methods, error classes and messages.

Host design.  One verification round is in flight at a time, and where it
stands is a Stage.  A transition table lists the events each stage admits;
an event a stage does not admit is refused with the error the reference's
callers observe for it.  The round's objects (transaction, published
features, graph ticket, completion, leased graph features) live in one
_Round record that the stage machine replaces as the round moves on, so no
combination of half-cleared fields can arise.  Published features sit in a
registry of live leases that predict() and release_features() check by
identity.  A captured bucket is a FullModelGraph: the whole HF forward
(embedding, every decoder layer with its fused launch, final norm) replayed
through a graph backend object (graph.TorchGraphBackend) under the store's
external-write receipts.

    READY --verify_eager--> FORWARD --published--> VERIFIED --commit/abort--> READY
    READY --prepare_graph--> TICKETED --submit--> IN_FLIGHT --finish--> LEASED_VERIFIED
    LEASED_VERIFIED --commit/abort--> LEASED --release lease--> READY
    TICKETED / IN_FLIGHT --cancel--> READY          any --close--> CLOSED (from READY)
"""
import enum
import weakref
from collections.abc import Mapping
from dataclasses import dataclass

import torch

from . import backends
from .graph import TorchGraphBackend
from .hf_hooks import FusedVerifier, PackedFeatures
from .kernels import HEAD_DIM, KV_HEADS, Q_HEADS, HipCapacityKernel
from .persistent_kv import Bucket, PersistentTargetKV, QueryFamily
from .schedule import DEFAULT_CHUNK

GRAPH_KIND = TorchGraphBackend.kind


class Stage(enum.Enum):
    READY = 'ready'                        # no round in flight
    FORWARD = 'forward'                    # an eager forward is running
    VERIFIED = 'verified'                  # eager features published; commit or abort settles the round
    TICKETED = 'ticketed'                  # a graph replay is prepared (transaction open, receipt held)
    IN_FLIGHT = 'in_flight'                # the replay was submitted
    LEASED_VERIFIED = 'leased_verified'    # graph features published, aliasing the capture's buffers
    LEASED = 'leased'                      # round settled; the graph features are still leased
    CLOSED = 'closed'


# stage -> {event: next stage}
_TABLE = {
    Stage.READY: {'admin': Stage.READY, 'eager': Stage.FORWARD, 'prepare': Stage.TICKETED},
    Stage.FORWARD: {'published': Stage.VERIFIED, 'failed': Stage.READY},
    Stage.VERIFIED: {'commit': Stage.READY, 'abort': Stage.READY},
    Stage.TICKETED: {'submit': Stage.IN_FLIGHT, 'cancel': Stage.READY},
    Stage.IN_FLIGHT: {'finish': Stage.LEASED_VERIFIED, 'cancel': Stage.READY},
    Stage.LEASED_VERIFIED: {'commit': Stage.LEASED, 'abort': Stage.LEASED},
    Stage.LEASED: {'release_lease': Stage.READY},
    Stage.CLOSED: {},
}

_BUSY_ROUND = 'Finish existing verification transaction first'
_BUSY_GRAPH = 'Finish graph submission and release feature lease first'
# Why a stage refuses the events that need an idle target ('admin', 'eager',
# 'prepare'), in the reference's order of checks: closed, then an open
# transaction, then a graph ticket or lease.
_NOT_READY = {
    Stage.CLOSED: 'Target adapter closed',
    Stage.FORWARD: _BUSY_ROUND, Stage.VERIFIED: _BUSY_ROUND, Stage.LEASED_VERIFIED: _BUSY_ROUND,
    Stage.TICKETED: _BUSY_GRAPH, Stage.IN_FLIGHT: _BUSY_GRAPH, Stage.LEASED: _BUSY_GRAPH,
}
# The error of each round event refused in the current stage.
_REFUSED = {
    'commit': (ValueError, 'Only the outstanding verification features can commit'),
    'abort': (ValueError, 'Only outstanding verification features can abort'),
    'submit': (ValueError, 'Exact unsubmitted graph ticket required'),
    'finish': (ValueError, 'Exact submitted graph completion required'),
    'cancel': (ValueError, 'Exact graph ticket required'),
}


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


@dataclass(frozen=True)
class _Round:
    """The objects of the round in flight (all None when READY)."""
    transaction: object = None
    features: object = None       # published, awaiting commit or abort
    ticket: object = None
    completion: object = None
    lease: object = None          # graph features that alias the capture's output buffers


class _Leases:
    """Published features, live until released; identity is what counts
    (a copy of a features object is foreign)."""

    def __init__(self):
        self._live = weakref.WeakValueDictionary()

    def add(self, features):
        self._live[id(features)] = features

    def live(self, features):
        return self._live.get(id(features)) is features

    def drop(self, features):
        del self._live[id(features)]


@dataclass
class _Budget:
    """Bucket count, workspace bytes and the graph byte budget that workspaces
    and graph reservations share."""
    max_buckets: int
    workspace_limit: int
    graph_limit: int
    graphs_allowed: bool
    workspace: int = 0
    graph_reserved: int = 0
    buckets: int = 0

    def admit_workspace(self, size, count):
        if self.buckets + count > self.max_buckets or self.workspace + size > self.workspace_limit:
            raise ValueError('Finite bucket/workspace budget exceeded')
        if self.graphs_allowed and self.workspace + size + self.graph_reserved > self.graph_limit:
            raise ValueError('Combined graph/workspace byte budget exceeded')

    def admit_graph(self, workspace, extra):
        if self.workspace + workspace + self.graph_reserved + extra > self.graph_limit:
            raise ValueError('Combined graph/workspace byte budget exceeded')


class FullModelGraph:
    """One captured verification forward of a registered bucket: the
    embedding, every decoder layer with its fused stage + attention launch,
    and the final norm (FullTargetExecution, persistent_qwen_graph.py:218-275).
    Token ids go into a fixed buffer; positions come from the bucket's fixed
    workspace; last hidden states and captured features live in the graph's
    memory and are overwritten by the next replay, hence the feature lease."""

    def __init__(self, target, bucket, backend, reserve_bytes):
        self.target, self.bucket, self.backend, self.reserve_bytes = target, bucket, backend, reserve_bytes
        self.ids = torch.zeros((1, bucket.query_tokens), dtype=torch.long, device=target.device)
        self.writer = target.store.register_external_writer(bucket, range(target.store.layers), self.complete)
        self.graph = None
        self.memory = None
        self.last = self.context = None
        self.invalid = False
        self._submitted = None         # (receipt, event) of the last submission
        self._addresses = None

    @staticmethod
    def output_buffer_bytes(target, bucket):
        """Fixed buffers a capture keeps besides the graph's private pool: ids,
        last hidden states and captured features."""
        hidden = target.model.config.hidden_size
        return bucket.query_tokens * (8 + 2 * hidden * (1 + len(target.layer_ids)))

    @property
    def retained_bytes(self):
        return 0 if self.memory is None else self.memory['private_pool_reserved_bytes']

    def pointers(self):
        return dict(ids=self.ids.data_ptr(), last=None if self.last is None else self.last.data_ptr(),
                    context=None if self.context is None else self.context.data_ptr(),
                    **self.target.store.pointers(self.bucket))

    def validate(self):
        if self.invalid or self.target.store.failed:
            raise RuntimeError('Captured program invalidated')
        if self._addresses is not None and self.pointers() != self._addresses:
            raise RuntimeError('Graph executor, model signature or captured buffer addresses changed')

    def load(self, chunks):
        self.ids.copy_(torch.cat(tuple(chunks.values()), dim=1))

    def _forward(self):
        t = self.target
        hidden, context = t._run_forward(self.ids, t.store.workspace(self.bucket).positions[None])
        return hidden, context

    @torch.no_grad()
    def capture(self, handles, query_lengths):
        """One eager forward first (lazy library state settles), then the
        capture, each inside a transaction of its own that is aborted: nothing
        executes during capture and nothing is committed."""
        t = self.target
        if self.graph is not None:
            raise ValueError('Bucket already captured')
        with t.verifier.transaction_for(handles, self.bucket, query_lengths=query_lengths) as tx:
            try:
                self._forward()
            finally:
                t.store.abort(tx)
        with t.verifier.transaction_for(handles, self.bucket, query_lengths=query_lengths) as tx:
            try:
                outputs = {}

                def body():
                    outputs['last'], outputs['context'] = self._forward()
                self.graph, self.memory = self.backend.capture(body, t.device, self.reserve_bytes)
                self.last, self.context = outputs['last'], outputs['context']
            finally:
                t.store.abort(tx)
        self._addresses = self.pointers()

    def submit(self, receipt):
        """Replay on the current stream; returns the event recorded after it."""
        self.validate()
        event = self.backend.replay(self.graph, self.target.device)
        self._submitted = (receipt, event)
        return event

    def complete(self, event, receipt):
        """The store's completion check: this program's last submission, for
        this receipt, observed complete."""
        return (self._submitted is not None and self._submitted[0] is receipt and self._submitted[1] is event
                and self.backend.complete(event))


class PersistentQwenTarget:
    """HF Qwen3 target over a PersistentTargetKV with the fused MI355X
    attention (the API of persistent_qwen_target.py:100-472).

    PersistentQwenTarget(model, layer_ids, *, slots, context_capacity,
    max_query_tokens, test_kernel=None, native_backend=None,
    graph_backend=None, max_buckets=32, workspace_byte_budget=256 MiB,
    max_graph_buckets=0, graph_byte_budget=0).  native_backend names this
    build's persistent-target attention (backends.CAPACITY_BACKEND); there is
    no CPU test_kernel.  graph_backend is a graph.TorchGraphBackend object or
    None.

    verify() runs one packed forward whose layers stage their new K/V rows
    into scratch and attend over resident + scratch rows in place; nothing is
    committed until commit() keeps the caller's accepted prefixes (the rest
    is rolled back by omission).  prefill() = verify + commit of every row.
    Decoder outputs of `layer_ids` are captured as draft context features.
    A registered graph bucket (register_graph_bucket + capture_graph) is
    verified by replaying its captured forward; verify_eager() is the
    explicit eager path.  Every call comes from the stream current at
    construction (the owner stream).
    """

    def __init__(self, model, layer_ids=(), *, slots, context_capacity, max_query_tokens, test_kernel=None,
                 native_backend=None, graph_backend=None, max_buckets=32, workspace_byte_budget=256 * 1024 ** 2,
                 max_graph_buckets=0, graph_byte_budget=0, chunk=DEFAULT_CHUNK):
        cfg = model.config
        if (cfg.model_type != 'qwen3' or getattr(cfg, 'use_sliding_window', False)
                or any(kind != 'full_attention' for kind in cfg.layer_types)
                or cfg._attn_implementation != 'sdpa'
                or (cfg.rope_parameters or {}).get('rope_type', 'default') != 'default'):
            raise ValueError('Owned dense Qwen3 with original SDPA/default RoPE required')
        self.layer_ids = tuple(layer_ids)
        if (tuple(sorted(set(self.layer_ids))) != self.layer_ids
                or any(type(i) is not int or not 0 <= i < cfg.num_hidden_layers for i in self.layer_ids)):
            raise ValueError('Unique increasing valid decoder layer IDs required')
        embed = model.get_input_embeddings().weight
        if native_backend is None:
            # The reference's CPU test-kernel form needs a CPU model; every
            # target here runs on the GPU.
            raise ValueError('Require explicit CPU test attention or pinned native backend')
        if (native_backend != backends.CAPACITY_BACKEND or test_kernel is not None or embed.device.type != 'cuda'
                or embed.dtype != torch.bfloat16
                or (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim) != (Q_HEADS, KV_HEADS, HEAD_DIM)):
            raise ValueError('Explicit pinned BF16 native Qwen architecture/runtime required')
        if any(type(x) is not int or x < 1 for x in (max_buckets, workspace_byte_budget)):
            raise ValueError('Positive finite bucket/workspace budget required')
        if graph_backend is not None:
            if type(graph_backend) is not TorchGraphBackend:
                raise ValueError('Explicit device-compatible graph backend required')
            if any(type(x) is not int or x < 1 for x in (max_graph_buckets, graph_byte_budget)):
                raise ValueError('Positive finite graph count and byte budget required')
        old_backend = cfg._attn_implementation
        store = PersistentTargetKV(layers=cfg.num_hidden_layers, slots=slots, context_capacity=context_capacity,
                                   max_query_tokens=max_query_tokens, heads=cfg.num_key_value_heads,
                                   dim=cfg.head_dim, dtype=embed.dtype, device=embed.device, chunk=chunk)
        # The kernel object the reference's session guards read
        # (packed_sampling.py:110-115): the capacity-tail drop-in of
        # _native_attention.  Verification itself runs the fused store launch.
        self._varlen_kernel = HipCapacityKernel(embed.device)
        self.kernel = self._varlen_kernel
        verifier = FusedVerifier(model, store)
        self._setup(store, verifier, native_backend, graph_backend,
                    _Budget(max_buckets, workspace_byte_budget, graph_byte_budget, graph_backend is not None),
                    max_graph_buckets, old_backend)
        self._owner_stream = self._stream_id()
        self._hooks = [self.model.model.layers[i].register_forward_hook(self._hook(i)) for i in self.layer_ids]

    def _setup(self, store, verifier, attention_backend, graph_backend, budget, max_graphs, old_backend):
        """Host state of a READY target over `store` (FusedVerifier `verifier`
        binds the model to it); layer_ids are set by the caller."""
        self.store = store
        self.verifier = verifier
        self.model = verifier.model
        self.attention_backend = attention_backend
        self._graph_backend = graph_backend
        self._budget = budget
        self._max_graphs = max_graphs
        self._old_backend = old_backend
        self._graphs = {}
        self._handles = {}
        self._stage = Stage.READY
        self._round = _Round()
        self._leases = _Leases()
        self._captured = None      # layer outputs of the forward being run
        self._hooks = []

    # -- the stage machine -------------------------------------------------------
    @property
    def stage(self):
        return self._stage

    @property
    def pool(self):
        """The transaction store (the reference's attribute name)."""
        return self.store

    @property
    def device(self):
        return self.store.device

    @property
    def lengths(self):
        return {r: self.store.length(h) for r, h in self._handles.items()}

    def _stream_id(self):
        return torch.cuda.current_stream(self.device).cuda_stream

    def _owner(self):
        if self._stream_id() != self._owner_stream:
            raise RuntimeError('Target, head, draft feature consumers and release must use the owner stream')

    def _admit(self, event):
        """The next stage for `event`, or the refusal the reference raises."""
        nxt = _TABLE[self._stage].get(event)
        if nxt is not None:
            return nxt
        if event in _REFUSED:
            cls, msg = _REFUSED[event]
            raise cls(msg)
        raise RuntimeError(_NOT_READY[self._stage])

    def _ready(self, event='admin'):
        """Owner stream, a READY target and an idle store; returns the next stage."""
        self._owner()
        nxt = self._admit(event)
        if self.store.failed:
            raise RuntimeError('Store invalidated by copy failure; construct a new store')
        if self.store.open_transaction is not None:
            raise RuntimeError('Outstanding verification transaction')
        return nxt

    def _move(self, stage, round_=None):
        self._stage = stage
        if round_ is not None:
            self._round = round_

    def _hook(self, index):
        def capture(_module, _inputs, output):
            if self._captured is None:
                raise RuntimeError('Foreign model forward while persistent adapter owns model')
            self._captured[index] = output[0] if isinstance(output, tuple) else output
        return capture

    def _run_forward(self, input_ids, position_ids):
        """One packed forward through the fused verification cache; returns
        (last hidden states, captured features or None)."""
        self._captured = {}
        try:
            out = self.model.model(input_ids=input_ids, position_ids=position_ids, attention_mask=None,
                                   past_key_values=self.verifier.cache, use_cache=True, return_dict=True,
                                   fused_verification=self.verifier)
            if self.store.staged_layers() != self.store.layers or set(self._captured) != set(self.layer_ids):
                raise RuntimeError('Full layer cache update or selected feature capture missing')
            context = torch.cat([self._captured[i] for i in self.layer_ids], dim=-1) if self.layer_ids else None
            return out.last_hidden_state, context
        finally:
            self._captured = None

    # -- requests, buckets, lifetime ------------------------------------------------
    def add_request(self, request):
        self._ready()
        handle = self.store.add_request(request)
        self._handles[request] = handle
        return handle

    def remove_request(self, request):
        self._ready()
        self.store.remove_request(self._handles[request])
        del self._handles[request]

    def reset(self):
        """Release every request incarnation; bucket addresses stay."""
        self._ready()
        for request in tuple(self._handles):
            self.remove_request(request)

    def close(self):
        self._ready()
        for hook in self._hooks:
            hook.remove()
        self._hooks = []
        self.model.config._attn_implementation = self._old_backend
        self._move(Stage.CLOSED)

    def invalidate(self):
        """Fail closed after an uncertain asynchronous or device failure: the
        store is poisoned, every captured program is void and the round is
        dropped.  A leased graph output stays leased until released."""
        self.store.invalidate()
        for graph in self._graphs.values():
            graph.invalid = True
        lease = self._round.lease
        if self._stage is not Stage.CLOSED:
            self._move(Stage.LEASED if lease is not None else Stage.READY, _Round(lease=lease))

    def register_bucket(self, bucket):
        self._ready()
        if isinstance(bucket, QueryFamily):
            self.store.register_bucket(bucket)
            return
        if not isinstance(bucket, Bucket):
            raise ValueError('Explicit Bucket or QueryFamily required')
        if self.store.is_registered(bucket):
            return
        size = self.store.workspace_bytes(bucket)
        self._budget.admit_workspace(size, 1)
        self.store.register_bucket(bucket)
        self._budget.workspace += size
        self._budget.buckets += 1

    def register_families(self, families):
        """One finite family declaration sharing one workspace."""
        self._ready()
        size = self.store.workspace_bytes(self.store.family_arena_shape(families))
        self._budget.admit_workspace(size, len(families))
        self.store.register_families(families)
        self._budget.workspace += size
        self._budget.buckets += len(families)

    def register_graph_bucket(self, bucket, *, reserve_bytes):
        """Explicit registration; reserve_bytes bounds the capture's private pool."""
        self._ready()
        if self._graph_backend is None or type(reserve_bytes) is not int or reserve_bytes < 1:
            raise ValueError('Graph backend and positive allocation reservation required')
        if bucket in self._graphs or len(self._graphs) >= self._max_graphs:
            raise ValueError('Duplicate graph bucket or finite graph count exceeded')
        workspace = 0 if self.store.is_registered(bucket) else self.store.workspace_bytes(bucket)
        extra = FullModelGraph.output_buffer_bytes(self, bucket) + reserve_bytes
        self._budget.admit_graph(workspace, extra)
        self.register_bucket(bucket)
        self._graphs[bucket] = FullModelGraph(self, bucket, self._graph_backend, reserve_bytes)
        self._budget.graph_reserved += extra

    # -- request chunks ------------------------------------------------------------
    def _check_chunks(self, chunks, bucket):
        """The reference's chunk contract, in its order: a nonempty mapping
        and an explicit bucket, the bucket's shape, residency, [1, Q] long ids
        on the device, ids inside the vocabulary."""
        if not isinstance(chunks, Mapping) or not chunks or not isinstance(bucket, (Bucket, QueryFamily)):
            raise ValueError('Nonempty ordered token mapping and explicit bucket required')
        shape = [ids.shape[1] if isinstance(ids, torch.Tensor) and ids.ndim == 2 else -1 for ids in chunks.values()]
        lengths = self.lengths
        if not bucket.accepts(tuple(shape), tuple(lengths.get(r, -1) for r in chunks)):
            raise ValueError('Ordered query lengths and contexts must match the chosen bucket or family')
        if any(r not in self._handles for r in chunks):
            raise ValueError('Request not resident')
        if any(ids.shape[0] != 1 or ids.dtype != torch.long or ids.device != self.device for ids in chunks.values()):
            raise ValueError('Each token chunk must be [1,Q] long on target device')
        flat = torch.cat(tuple(chunks.values()), dim=1)
        if bool(((flat < 0) | (flat >= self.model.config.vocab_size)).any()):
            raise ValueError('Token outside vocabulary')
        return flat

    def _open(self, chunks, bucket):
        handles = tuple(self._handles[r] for r in chunks)
        return self.store.begin(handles, bucket, query_lengths=tuple(ids.shape[1] for ids in chunks.values()))

    @staticmethod
    def _spans(chunks, tx):
        """request -> (row offset in the packed forward, query rows, context)."""
        offsets = [0]
        for q in tx.query_lengths:
            offsets.append(offsets[-1] + q)
        return {r: (o, q, c) for r, o, q, c in zip(chunks, offsets, tx.query_lengths, tx.context_lengths)}

    def _work(self, tx, **extra):
        work = self.store.work(tx)
        work.update(model_forward_calls=1, layers=self.store.layers, selected_layer_ids=list(self.layer_ids),
                    attention_backend=self.attention_backend, workspace_bytes=self._budget.workspace,
                    committed_write_policy='scratch_only_until_explicit_commit', **extra)
        return work

    # -- graph buckets -----------------------------------------------------------------
    @torch.no_grad()
    def capture_graph(self, chunks, *, bucket):
        """Set-up only: capture the bucket's full-model forward (the ids and
        query lengths of `chunks` shape it; nothing is committed)."""
        self._ready()
        self._check_chunks(chunks, bucket)
        program = self._graphs.get(bucket)
        if program is None:
            raise ValueError('Explicit registered graph bucket required')
        try:
            program.load(chunks)
            program.capture(tuple(self._handles[r] for r in chunks), tuple(ids.shape[1] for ids in chunks.values()))
        except BaseException:
            self.invalidate()
            raise

    @torch.no_grad()
    def prepare_graph_verify(self, chunks, *, bucket):
        nxt = self._ready('prepare')
        self._check_chunks(chunks, bucket)
        program = self._graphs.get(bucket)
        if program is None or program.graph is None:
            raise ValueError('Explicitly captured bucket required; no capture-on-miss')
        program.validate()
        tx = self._open(chunks, bucket)
        try:
            program.load(chunks)
            receipt = self.store.prepare_external_write(tx, program.writer)
        except BaseException:
            self.store.abort(tx)
            raise
        ticket = GraphTicket(tx, receipt, program, self._spans(chunks, tx))
        self._move(nxt, _Round(transaction=tx, ticket=ticket))
        return ticket

    @torch.no_grad()
    def submit_graph(self, ticket):
        self._owner()
        if ticket is None or ticket is not self._round.ticket:
            raise ValueError(_REFUSED['submit'][1])
        nxt = self._admit('submit')
        try:
            event = ticket.execution.submit(ticket.receipt)
            self.store.submit_external_write(ticket.receipt, event)
        except BaseException:
            self.invalidate()
            raise
        completion = GraphCompletion(ticket, event)
        self._move(nxt, _Round(transaction=ticket.transaction, ticket=ticket, completion=completion))
        return completion

    @torch.no_grad()
    def finish_graph(self, completion, *, wait=True):
        self._owner()
        if completion is None or completion is not self._round.completion:
            raise ValueError(_REFUSED['finish'][1])
        nxt = self._admit('finish')
        ticket = completion.ticket
        program = ticket.execution
        try:
            if wait:
                program.backend.wait(completion.event)
            ready = program.complete(completion.event, ticket.receipt)
        except BaseException:
            self.invalidate()
            raise
        if not ready:
            raise RuntimeError('Graph completion has not been observed')
        try:
            self.store.complete_external_write(ticket.receipt)
            program.validate()
            work = self._work(ticket.transaction, execution_kind=program.backend.kind,
                              graph_scope='HF embedding, every decoder layer with the fused stage + attention, '
                                          'final norm; head and sampling outside',
                              graph_retained_bytes=program.retained_bytes, graph_memory_accounting=program.memory,
                              graph_reserved_bytes=self._budget.graph_reserved)
        except BaseException:
            self.invalidate()
            raise
        features = PackedFeatures(program.last, program.context, ticket.spans, work)
        self._leases.add(features)
        self._move(nxt, _Round(transaction=ticket.transaction, features=features, lease=features))
        return features

    def cancel_graph(self, ticket):
        self._owner()
        if ticket is None or ticket is not self._round.ticket:
            raise ValueError(_REFUSED['cancel'][1])
        nxt = self._admit('cancel')
        try:
            self.store.abort(ticket.transaction)        # refuses an unfinished external write
        except BaseException:
            if self.store.failed:
                self.invalidate()
            raise
        self._move(nxt, _Round())

    # -- verification ---------------------------------------------------------------
    @torch.no_grad()
    def verify(self, chunks, *, bucket):
        """One packed forward over {request: ids [1, q]} in bucket order:
        the captured program of a registered graph bucket, else eager."""
        if bucket in self._graphs:
            return self.finish_graph(self.submit_graph(self.prepare_graph_verify(chunks, bucket=bucket)))
        return self.verify_eager(chunks, bucket=bucket)

    @torch.no_grad()
    def verify_eager(self, chunks, *, bucket):
        """The explicit eager forward, also on registered graph buckets."""
        nxt = self._ready('eager')
        ids = self._check_chunks(chunks, bucket)
        self._move(nxt)
        try:
            with self.verifier.transaction_for(tuple(self._handles[r] for r in chunks), bucket,
                                               query_lengths=tuple(x.shape[1] for x in chunks.values())) as tx:
                try:
                    last, context = self._run_forward(ids, self.store.workspace(bucket).positions[None])
                except BaseException:
                    if self.store.open_transaction is tx and not self.store.failed:
                        self.store.abort(tx)
                    raise
        except BaseException:
            self._move(self._admit('failed'), _Round())
            raise
        work = self._work(tx)
        if isinstance(bucket, QueryFamily):
            work['execution_kind'] = 'explicit_eager'
        features = PackedFeatures(last.detach(), None if context is None else context.detach(),
                                  self._spans(chunks, tx), work)
        self._leases.add(features)
        self._move(self._admit('published'), _Round(transaction=tx, features=features))
        return features

    def _settling(self, features, event):
        self._owner()
        if self._round.features is None or features is not self._round.features:
            raise ValueError(_REFUSED[event][1])
        return self._admit(event)

    @torch.no_grad()
    def commit(self, features, committed_query_lengths):
        nxt = self._settling(features, 'commit')
        if not isinstance(committed_query_lengths, Mapping) or set(committed_query_lengths) != set(features.spans):
            raise ValueError('One committed query prefix per verified request required')
        counts = {self._handles[r]: n for r, n in committed_query_lengths.items()}
        result = self.store.commit(self._round.transaction, counts)
        self._move(nxt, _Round(lease=self._round.lease))
        return result

    def abort(self, features):
        nxt = self._settling(features, 'abort')
        self.store.abort(self._round.transaction)
        self._move(nxt, _Round(lease=self._round.lease))

    def release_features(self, features):
        self._owner()
        if not self._leases.live(features):
            raise ValueError('Foreign, copied or already released features')
        if features is self._round.features:
            raise RuntimeError('Commit or abort before releasing feature lease')
        if features is self._round.lease:
            self._move(self._admit('release_lease'), _Round())
        self._leases.drop(features)

    @torch.no_grad()
    def prefill(self, chunks, *, bucket):
        self._ready()
        if any(self.lengths.get(r) != 0 for r in chunks):
            raise ValueError('Prefill is only for newly admitted empty requests')
        run = self.verify_eager if bucket in self._graphs else self.verify
        features = run(chunks, bucket=bucket)
        self.commit(features, {r: ids.shape[1] for r, ids in chunks.items()})
        return features

    @torch.no_grad()
    def predict(self, features, last_only=False):
        """The model's LM head over the verified rows (after its final norm)."""
        self._owner()
        if not self._leases.live(features):
            raise ValueError('Foreign or released features')
        logits = self.model.get_output_embeddings()(features.last)
        if last_only:
            return {r: logits[:, o + n - 1] for r, (o, n, _) in features.spans.items()}
        return {r: logits[:, o:o + n] for r, (o, n, _) in features.spans.items()}

    def request_kv(self, request):
        """Per layer (keys, values) [1, Hkv, C, D] copies of a request's committed rows."""
        keys, values = self.store.request_kv(self._handles[request])
        return tuple((k.transpose(0, 1)[None], v.transpose(0, 1)[None]) for k, v in zip(keys, values))
