"""Packed varlen layouts (drop-in for dspark_qwen/varlen_target.py:17-82 and
dspark_qwen/persistent_qwen_target.py:19-27).

A layout describes B requests packed back to back: request r owns query rows
cu_query[r]..cu_query[r+1] and key rows cu_key[r]..cu_key[r+1], its queries
being the terminal suffix of its keys (bottom-right alignment).
"""
from dataclasses import dataclass

import torch

INT32_LIMIT = 2 ** 31


def _cumulative(lengths, device):
    ends = [0]
    for n in lengths:
        ends.append(ends[-1] + n)
    if ends[-1] >= INT32_LIMIT:
        raise ValueError('Varlen cumulative lengths exceed int32')
    return torch.tensor(ends, device=device, dtype=torch.int32)


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
        in query order.  Validation runs on the tensors' device with a single
        device-to-host transfer of the small per-request summary.
        """
        arrays = (query_requests, query_positions, key_requests, key_positions)
        if any(not isinstance(x, torch.Tensor) or x.ndim != 1 or x.dtype != torch.long for x in arrays):
            raise ValueError('Expected flat long request/position metadata')
        if any(x.device != query_requests.device for x in arrays):
            raise ValueError('All layout metadata must share a device')
        if (query_requests.numel() == 0 or query_requests.shape != query_positions.shape
                or key_requests.shape != key_positions.shape):
            raise ValueError('Nonempty queries and matching marker/position lengths required')
        dev = query_requests.device
        nq = query_requests.numel()
        nk = key_requests.numel()
        # Runs of equal consecutive query markers are the requests.
        starts = torch.ones(nq, dtype=torch.bool, device=dev)
        starts[1:] = query_requests[1:] != query_requests[:-1]
        seg_of_query = torch.cumsum(starts.to(torch.int64), 0) - 1
        markers = query_requests[starts]
        b = markers.numel()
        q_counts = torch.bincount(seg_of_query, minlength=b)
        sorted_markers, order = torch.sort(markers)
        repeated = (sorted_markers[1:] == sorted_markers[:-1]).any().reshape(1).to(torch.long)
        # Map every physical key to the request owning its marker (b = none).
        slot = torch.searchsorted(sorted_markers, key_requests).clamp(max=b - 1)
        hit = sorted_markers[slot] == key_requests
        seg_of_key = torch.where(hit, order[slot], torch.full_like(slot, b))
        k_counts = torch.bincount(seg_of_key, minlength=b + 1)[:b]
        # Keys grouped by request in query order, physical order kept inside.
        phys = torch.argsort(seg_of_key * (nk + 1) + torch.arange(nk, device=dev))
        grouped_seg = seg_of_key[phys]
        k_starts = torch.cat((torch.cumsum(k_counts, 0) - k_counts, k_counts.new_zeros(1)))
        rank = torch.arange(nk, device=dev) - k_starts[grouped_seg]
        wrong_pos = ((key_positions[phys] != rank) & (grouped_seg < b)).to(torch.long)
        bad_prefix = torch.zeros(b + 1, dtype=torch.long, device=dev).index_add_(0, grouped_seg, wrong_pos)[:b]
        bad_prefix = bad_prefix + (k_counts < q_counts).to(torch.long)
        # Query positions must be k-q .. k-1 of their own request.
        q_rank = torch.arange(nq, device=dev) - (torch.cumsum(q_counts, 0) - q_counts)[seg_of_query]
        expected_q = (k_counts - q_counts)[seg_of_query] + q_rank
        bad_suffix = torch.zeros(b, dtype=torch.long, device=dev).index_add_(
            0, seg_of_query, (query_positions != expected_q).to(torch.long))
        summary = torch.cat((repeated, markers, q_counts, k_counts, bad_prefix, bad_suffix)).tolist()
        if summary[0]:
            raise ValueError('Each request query must form one contiguous chunk')
        host_markers = tuple(summary[1:1 + b])
        q_lengths = tuple(summary[1 + b:1 + 2 * b])
        k_lengths = tuple(summary[1 + 2 * b:1 + 3 * b])
        for pre, suf in zip(summary[1 + 3 * b:1 + 4 * b], summary[1 + 4 * b:1 + 5 * b]):
            if pre:
                raise ValueError('Active keys must be a complete request-local prefix')
            if suf:
                raise ValueError('Queries must be the terminal suffix of their own key prefix')
        gather = phys[:sum(k_lengths)]
        return cls(host_markers, q_lengths, k_lengths,
                   _cumulative(q_lengths, dev), _cumulative(k_lengths, dev), gather, nk)

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
        """[1,Hkv,physical_K,D] cache tensors -> packed [sum K, Hkv, D] (varlen_target.py:74-82)."""
        if (key.ndim != 4 or key.shape[0] != 1 or value.shape != key.shape
                or key.shape[2] != self.physical_key_tokens or key.device != self.gather_indices.device
                or value.device != key.device or value.dtype != key.dtype):
            raise ValueError('Expected matching [1,Hkv,physical_K,D] cache tensors')
        return tuple(x.index_select(2, self.gather_indices).squeeze(0).transpose(0, 1).contiguous()
                     for x in (key, value))


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
