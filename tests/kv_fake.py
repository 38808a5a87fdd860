"""A CPU stand-in for the store's device half, for host-state-machine tests
only.  It implements the HipKVDevice interface with plain torch on the CPU
and builds the transaction arrays and commits with the oracle
(oracle/semantics.py), so the store's validation order, error classes and
fail-closed behaviour run in CPU CI.  The product has no CPU path; this
object exists only under tests/.
"""
import numpy as np
import torch

from oracle import semantics
from qwen3_dspark_amd.kv_device import Workspace


class CpuKVDevice:
    def __init__(self, *, layers, slots, context_capacity, max_query_tokens, heads, dim, dtype=torch.float32):
        self.device = torch.device('cpu')
        self.layers, self.slots, self.capacity = layers, slots, context_capacity
        self.max_rows, self.heads, self.dim, self.dtype = max_query_tokens, heads, dim, dtype
        self.keys = torch.zeros((layers, slots, context_capacity, heads, dim), dtype=dtype)
        self.values = torch.zeros_like(self.keys)
        self.scratch_keys = torch.zeros((layers, max_query_tokens, heads, dim), dtype=dtype)
        self.scratch_values = torch.zeros_like(self.scratch_keys)
        self.calls = []            # device-call names, in order
        self.fail = None           # name of a device call to fail once (injected fault)
        self.xcd_speed = None      # relative XCD speeds for balanced plans (the device half holds them)
        self.slot_balance = True   # second-slot share of balanced plans (the device half holds it)

    def measure_xcd_speed(self, workgroups=1024, passes=2):
        self._enter('measure_xcd_speed')
        return [1.3, 0.7, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0]

    def _enter(self, name):
        self.calls.append(name)
        if self.fail == name:
            self.fail = None
            raise RuntimeError(f'injected {name} failure')

    def workspace(self, shape):
        n, r, q = shape.key_capacity, shape.request_count, shape.query_tokens
        return Workspace(dict(
            committed_indices=torch.zeros(n, dtype=torch.long), scratch_indices=torch.zeros(n, dtype=torch.long),
            from_scratch=torch.zeros((n, 1, 1), dtype=torch.bool), valid=torch.zeros((n, 1, 1), dtype=torch.bool),
            cu_query=torch.zeros(r + 1, dtype=torch.int32), cu_key=torch.zeros(r + 1, dtype=torch.int32),
            positions=torch.zeros(q, dtype=torch.long), req=torch.zeros(3 * r, dtype=torch.int32),
            work=torch.zeros(1, dtype=torch.int32),
            keys=torch.empty((n, self.heads, self.dim), dtype=self.dtype),
            values=torch.empty((n, self.heads, self.dim), dtype=self.dtype),
            attn=torch.zeros(16, dtype=torch.uint8)))

    def workspace_bytes(self, shape):
        n, r, q = shape.key_capacity, shape.request_count, shape.query_tokens
        elem = torch.empty((), dtype=self.dtype).element_size()
        return 2 * n * self.heads * self.dim * elem + 18 * n + 8 * (r + 1) + 8 * q + 12 * r + 4 + 16

    def write_prefix(self, slot, keys, values):
        self._enter('write_prefix')
        n = keys.shape[1]
        self.keys[:, slot, :n].copy_(keys)
        self.values[:, slot, :n].copy_(values)

    def copy_out(self, slot, n):
        return self.keys[:, slot, :n].clone(), self.values[:, slot, :n].clone()

    def build_metadata(self, ws, shape, slots, contexts, query_lengths):
        self._enter('build_metadata')
        meta = semantics.txn_metadata(slots, contexts, query_lengths, self.capacity, shape.key_capacity)
        for name, value in meta.items():
            dst = getattr(ws, name)
            dst.copy_(torch.from_numpy(np.ascontiguousarray(value)).reshape(dst.shape).to(dst.dtype))
        ws.req.copy_(torch.tensor(list(slots) + list(contexts) + list(query_lengths), dtype=torch.int32))

    def stage(self, layer, keys, values, rows):
        self._enter('stage')
        self.scratch_keys[layer, :rows].copy_(keys)
        self.scratch_values[layer, :rows].copy_(values)

    def gather(self, ws, shape, layer):
        self._enter('gather')
        meta = {name: getattr(ws, name).numpy().reshape(-1) for name in
                ('committed_indices', 'scratch_indices', 'from_scratch', 'valid')}
        for res, scr, out in ((self.keys, self.scratch_keys, ws.keys), (self.values, self.scratch_values, ws.values)):
            out.copy_(torch.from_numpy(semantics.materialize(res[layer].numpy(), scr[layer].numpy(), meta)))
        return ws.keys, ws.values

    def attend(self, *args):
        raise RuntimeError('attention needs the GPU')

    def commit(self, ws, counts, max_query):
        self._enter('commit')
        if not any(counts):
            return
        r = len(counts)
        req = ws.req[:3 * r].tolist()
        slots, contexts, queries = req[:r], req[r:2 * r], req[2 * r:]
        for res, scr in ((self.keys, self.scratch_keys), (self.values, self.scratch_values)):
            out, _ = semantics.commit(res.numpy(), scr.numpy(), slots, contexts, queries, list(counts), self.capacity)
            res.copy_(torch.from_numpy(out))


def store(*, layers=2, slots=3, context_capacity=24, max_query_tokens=8, heads=2, dim=4, dtype=torch.float32):
    """A PersistentTargetKV over the CPU stand-in (the reference tests' pool)."""
    from qwen3_dspark_amd.persistent_kv import PersistentTargetKV
    dims = dict(layers=layers, slots=slots, context_capacity=context_capacity, max_query_tokens=max_query_tokens,
                heads=heads, dim=dim)
    return PersistentTargetKV(**dims, dtype=dtype, kv_device=CpuKVDevice(**dims, dtype=dtype))
