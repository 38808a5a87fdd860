"""Captured verification rounds on MI355X: one HIP graph per bucket holding
every layer's fused verification attention (the layer's new K/V staged into
scratch by the same launch), replayed once per transaction.  The transaction
metadata (PersistentTargetKV.begin), sampling and commit stay outside the
graph; the graph reads the metadata from the bucket's fixed workspace.

This is the attention part of dspark_qwen/persistent_qwen_graph.py:97-275:
  * TorchGraphBackend.capture / submit / wait / complete -> capture(),
    submit(), wait(), complete() (one caller stream, event-backed completion,
    no eager fallback);
  * FullTargetExecution's fixed input/output buffers and its external-writer
    receipts -> the query / keys / values / output buffers below and
    PersistentTargetKV.prepare/submit/complete_external_write;
  * _CapturedCache.update's stage + gather per layer -> the fused launch,
    which never materialises the capacity-length K/V.
Every launch argument depends only on the bucket (fixed-capacity work list,
bucket launch maxima, fixed buffers), so one capture serves every later
transaction of the bucket; the graph holds no memset nodes.
"""
import weakref
from dataclasses import dataclass

import torch

from .kernels import HEAD_DIM, KV_HEADS, Q_HEADS


def _private_pool_bytes(pool_id, device):
    """Reserved bytes of a graph's private memory pool: the sum of the
    segments torch's allocator snapshot lists for that pool on `device`
    (inactive retained blocks included)."""
    total = 0
    for seg in torch.cuda.memory.memory_snapshot(mempool_id=pool_id):
        if seg.get('device', device.index) != device.index:
            continue
        if 'segment_pool_id' in seg and tuple(seg['segment_pool_id']) != tuple(pool_id):
            continue
        total += int(seg['total_size'])
    return total


@dataclass(frozen=True)
class ReplayEvent:
    """The completion handle of one replay: the event recorded after it on
    the caller's stream and the program it belongs to."""
    event: object
    graph: object


class TorchGraphBackend:
    """Graph backend object of the persistent target's captured buckets (the
    role of TorchGraphBackend, persistent_qwen_graph.py:97-138): captures a
    body into a HIP graph (torch's CUDAGraph on ROCm) on a side stream,
    replays it on the caller's stream and reports completion only for the
    events it recorded itself.

    Each capture gets a private memory pool.  Its reserved bytes are counted
    from the allocator's snapshot and must stay within the caller's
    reservation; one backend never shares a pool between captures."""
    kind = 'mi355x_hip_full_model_graph'

    def __init__(self):
        self._pools = set()
        self._issued = weakref.WeakValueDictionary()

    def capture(self, body, device, reserve_bytes):
        """Capture `body` (no execution); returns (graph, memory accounting)."""
        if device.type != 'cuda':
            raise ValueError('Actual CUDA/ROCm device required for graph capture')
        before = torch.cuda.memory_reserved(device)
        stream = torch.cuda.Stream(device=device)
        stream.wait_stream(torch.cuda.current_stream(device))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            body()
        torch.cuda.current_stream(device).wait_stream(stream)
        stream.synchronize()
        pool = graph.pool()
        if pool in self._pools:
            raise RuntimeError('Graph pool sharing is not registered or budgeted')
        self._pools.add(pool)
        reserved = _private_pool_bytes(pool, device)
        after = torch.cuda.memory_reserved(device)
        memory = dict(kind='graph_private_pool_reserved_segments', pool_id=list(pool),
                      private_pool_reserved_bytes=reserved, global_reserved_before=before,
                      global_reserved_after=after, global_reserved_delta=after - before,
                      reservation_bytes=reserve_bytes, includes_inactive_blocks=True)
        if reserved > reserve_bytes:
            raise RuntimeError('Graph private-pool reserved bytes exceed registered reservation: '
                               f'measured={reserved}, reservation={reserve_bytes}')
        return graph, memory

    def replay(self, graph, device):
        """Replay on the current stream; returns a ReplayEvent."""
        graph.replay()
        event = torch.cuda.Event()
        event.record(torch.cuda.current_stream(device))
        handle = ReplayEvent(event, graph)
        self._issued[id(handle)] = handle
        return handle

    def _own(self, handle):
        if not isinstance(handle, ReplayEvent) or self._issued.get(id(handle)) is not handle:
            raise ValueError('Foreign completion event')

    def wait(self, handle):
        self._own(handle)
        handle.event.synchronize()

    def complete(self, handle):
        """True iff `handle` is a replay this backend issued and it finished."""
        try:
            self._own(handle)
        except ValueError:
            return False
        return bool(handle.event.query())


@dataclass(frozen=True)
class GraphCompletion:
    """A submitted replay: the store's external-write receipt and the event
    recorded after the replay on the caller's stream."""
    receipt: object
    event: object


class VerificationGraph:
    """Fixed buffers and one captured program for a registered bucket of a
    PersistentTargetKV.  Per transaction: write the layer inputs into
    query / keys / values (every layer), submit(tx), then wait(completion)
    (or poll complete()); outputs are in `output` and the store may commit.
    """
    kind = 'mi355x_hip_verification_graph'

    def __init__(self, pool, bucket):
        if not pool.is_registered(bucket):
            raise ValueError('Registered bucket required')
        if (pool.heads, pool.dim, pool.dtype) != (KV_HEADS, HEAD_DIM, torch.bfloat16):
            raise ValueError('Captured verification requires bf16 Hkv8/D128 storage')
        self.pool, self.bucket, self.device = pool, bucket, pool.device
        q, L = bucket.query_tokens, pool.layers
        self.query = torch.zeros((L, q, Q_HEADS, HEAD_DIM), dtype=torch.bfloat16, device=self.device)
        self.keys = torch.zeros((L, q, KV_HEADS, HEAD_DIM), dtype=torch.bfloat16, device=self.device)
        self.values = torch.zeros_like(self.keys)
        self.output = torch.zeros_like(self.query)
        self._events = weakref.WeakValueDictionary()
        self.writer = pool.register_external_writer(bucket, range(L), self.complete)
        self.graph = None
        self._addresses = self.pointers()

    def pointers(self):
        own = dict(graph_query=self.query.data_ptr(), graph_keys=self.keys.data_ptr(),
                   graph_values=self.values.data_ptr(), graph_output=self.output.data_ptr())
        return dict(own, **self.pool.pointers(self.bucket))

    def _validate(self):
        if self.pool.failed:
            raise RuntimeError('The store is poisoned')
        if self.pointers() != self._addresses:
            raise RuntimeError('Captured buffer addresses changed')

    def _body(self):
        for layer in range(self.pool.layers):
            self.pool.launch_attention(self.bucket, layer, self.query[layer].data_ptr(),
                                       self.output[layer].data_ptr(), self.keys[layer].data_ptr(),
                                       self.values[layer].data_ptr())

    @torch.no_grad()
    def capture(self):
        """Capture every layer's launch on a side stream (no transaction is
        needed: nothing executes during capture)."""
        self._validate()
        if self.graph is not None:
            raise ValueError('Bucket already captured')
        stream = torch.cuda.Stream(device=self.device)
        stream.wait_stream(torch.cuda.current_stream(self.device))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            self._body()
        torch.cuda.current_stream(self.device).wait_stream(stream)
        stream.synchronize()
        self.graph = graph
        self._validate()
        return self

    def submit(self, tx):
        """Replay for the open transaction tx (which must be on this bucket,
        with no layer staged yet) on the current stream."""
        self._validate()
        if self.graph is None:
            raise RuntimeError('Explicit bucket capture required before submission')
        receipt = self.pool.prepare_external_write(tx, self.writer)
        self.graph.replay()
        event = torch.cuda.Event()
        event.record(torch.cuda.current_stream(self.device))
        self.pool.submit_external_write(receipt, event)
        completion = GraphCompletion(receipt, event)
        self._events[id(completion)] = completion
        return completion

    def complete(self, event, receipt):
        """Completion check the store calls back (an event this graph
        recorded for this receipt, observed complete)."""
        return any(c.event is event and c.receipt is receipt for c in self._events.values()) and event.query()

    def wait(self, completion):
        """Block until the replay finished, then publish its scratch writes
        to the store (the transaction may then commit)."""
        if self._events.get(id(completion)) is not completion:
            raise ValueError('Foreign completion')
        completion.event.synchronize()
        self.pool.complete_external_write(completion.receipt)
        return self.output
