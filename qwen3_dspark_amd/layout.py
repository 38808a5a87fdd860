"""Packed varlen layouts (drop-in for dspark_qwen/varlen_target.py:17-82 and
dspark_qwen/persistent_qwen_target.py:19-27).

A layout describes B requests packed back to back: request r owns query rows
cu_query[r]..cu_query[r+1] and key rows cu_key[r]..cu_key[r+1], its queries
being the terminal suffix of its keys (bottom-right alignment).
"""
from dataclasses import dataclass

import torch

from . import _native
from ._device import require_gfx950

INT32_LIMIT = 2 ** 31
MAX_LAYOUT_REQUESTS = 8192    # requests per layout built on the device
_LAYOUT_ERRORS = {
    1: 'Each request query must form one contiguous chunk',
    2: 'Active keys must be a complete request-local prefix',
    3: 'Queries must be the terminal suffix of their own key prefix',
}


@dataclass(frozen=True)
class PackedLayout:
    """Same fields and meaning as the reference PackedLayout (varlen_target.py:17-25)."""
    request_markers: tuple
    query_lengths: tuple
    key_lengths: tuple
    cu_query: torch.Tensor
    cu_key: torch.Tensor
    gather_indices: torch.Tensor
    physical_key_tokens: int

    @classmethod
    def from_metadata(cls, query_requests, query_positions, key_requests, key_positions):
        """Build a layout from flat request markers and request-local positions.

        Contract of varlen_target.py:28-60: queries of a request form one
        contiguous chunk; its keys (in physical order) are exactly positions
        0..k-1; its query positions are the terminal suffix k-q..k-1.
        gather_indices lists every request's keys in physical order, requests
        in query order.  Argument checks raise ValueError first, as in the
        reference; the layout itself is derived and validated on the GPU by
        dspark_layout_build, followed by one small device-to-host read of its
        summary (the reference synchronises as well).  Metadata must live on
        the gfx950 device: there is no CPU path.
        """
        arrays = (query_requests, query_positions, key_requests, key_positions)
        if any(not isinstance(x, torch.Tensor) or x.ndim != 1 or x.dtype != torch.long for x in arrays):
            raise ValueError('Expected flat long request/position metadata')
        if any(x.device != query_requests.device for x in arrays):
            raise ValueError('All layout metadata must share a device')
        if (query_requests.numel() == 0 or query_requests.shape != query_positions.shape
                or key_requests.shape != key_positions.shape):
            raise ValueError('Nonempty queries and matching marker/position lengths required')
        dev = require_gfx950(query_requests.device)
        nq, nk = query_requests.numel(), key_requests.numel()
        if nq >= INT32_LIMIT or nk >= INT32_LIMIT:
            raise ValueError('Varlen cumulative lengths exceed int32')
        lib = _native.load()
        m = min(nq, MAX_LAYOUT_REQUESTS)
        ws = torch.empty(lib.dspark_layout_workspace_bytes(nq, nk, m), dtype=torch.uint8, device=dev)
        cu = torch.empty(2, m + 1, dtype=torch.int32, device=dev)
        gather = torch.empty(max(nk, 1), dtype=torch.long, device=dev)
        summary = torch.empty(4 + 3 * m, dtype=torch.long, device=dev)
        arrays = tuple(x.contiguous() for x in arrays)
        _native.call('dspark_layout_build', arrays[0].data_ptr(), arrays[1].data_ptr(), nq,
                     arrays[2].data_ptr(), arrays[3].data_ptr(), nk, m, cu[0].data_ptr(), cu[1].data_ptr(),
                     gather.data_ptr(), summary.data_ptr(), ws.data_ptr(), ws.numel(),
                     _native.stream_handle(dev))
        host = summary.tolist()
        error, b, total_k = host[0], host[2], host[3]
        if error == 4:
            raise ValueError(f'At most {MAX_LAYOUT_REQUESTS} requests per packed layout')
        if error:
            raise ValueError(_LAYOUT_ERRORS[error])
        return cls(tuple(host[4:4 + b]), tuple(host[4 + m:4 + m + b]), tuple(host[4 + 2 * m:4 + 2 * m + b]),
                   cu[0, :b + 1], cu[1, :b + 1], gather[:total_k], nk)

    @property
    def query_tokens(self):
        return sum(self.query_lengths)

    @property
    def gathered_key_tokens(self):
        return sum(self.key_lengths)

    @property
    def pair_domain(self):
        return sum(q * k for q, k in zip(self.query_lengths, self.key_lengths))

    def gather_kv(self, key, value):
        """[1,Hkv,physical_K,D] cache tensors -> packed [sum K, Hkv, D]
        (varlen_target.py:74-82), one dspark_pool_gather launch for K and V."""
        if (key.ndim != 4 or key.shape[0] != 1 or value.shape != key.shape
                or key.shape[2] != self.physical_key_tokens or key.device != self.gather_indices.device
                or value.device != key.device or value.dtype != key.dtype):
            raise ValueError('Expected matching [1,Hkv,physical_K,D] cache tensors')
        dev = require_gfx950(key.device)
        _, heads, rows, dim = key.shape
        elem = key.element_size()
        if key.stride() != value.stride() or key.stride(3) != 1 or (dim * elem) % 16:
            raise ValueError('gather_kv needs matching strides, contiguous rows and 16-byte head rows')
        strides = (key.stride(1) * elem, key.stride(2) * elem)
        if any(x % 16 for x in strides) or key.data_ptr() % 16 or value.data_ptr() % 16:
            raise ValueError('gather_kv needs 16-byte aligned pool rows')
        n = self.gather_indices.numel()
        out_k = torch.empty((n, heads, dim), dtype=key.dtype, device=dev)
        out_v = torch.empty_like(out_k)
        _native.call('dspark_pool_gather', key.data_ptr(), value.data_ptr(), rows, strides[0], strides[1], heads,
                     dim * elem, self.gather_indices.data_ptr(), n, out_k.data_ptr(), out_v.data_ptr(),
                     _native.stream_handle(dev))
        return out_k, out_v


@dataclass(frozen=True)
class PersistentAttentionLayout:
    """Capacity-tail layout (persistent_qwen_target.py:19-27): K/V hold
    physical_key_capacity rows of which only cu_key[-1] are read; the maxima
    are fixed per bucket so repeated launches keep one grid."""
    query_lengths: tuple
    key_lengths: tuple
    cu_query: torch.Tensor
    cu_key: torch.Tensor
    physical_key_capacity: int
    maximum_key_length: int = 0
    maximum_query_length: int = 0
