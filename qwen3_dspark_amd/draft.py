"""Fused multi-block DSpark draft attention on MI355X.

Semantics (dspark_qwen/model.py:12-19 block_mask, 41-61 DraftAttention):
request r has a committed context of c_r projected K/V rows and n_r draft
blocks of 7 rows (anchor token + 6 MASK).  Block b of request r attends to
context positions j < anchor_b (anchor_b <= c_r) and to all 7 rows of its own
block; it never sees another block or another request.  With one block per
request at anchor = c_r this is exactly the packed noncausal draft call of
dspark_qwen/packed_draft.py:205-236, without the whole-pool cat, the gather
and the copies: context rows are read in place, once per request for all of
its blocks.

The context may live in
  * a row store [rows, 8, 128] (e.g. a slotted pool layer viewed as
    [slots * capacity, 8, 128]); request r uses rows off_r .. off_r + c_r, or
  * the reference's append-order pool layer [1, 8, N, 128] together with the
    per-request physical indices (PackedLayout.gather_indices order).
"""
import torch

from . import _native
from ._device import Workspace, require_gfx950
from .kernels import DEFAULT_CHUNK, HEAD_DIM, KV_HEADS, Q_HEADS, SCALE, _check_scale

BLOCK_SIZE = 7
MAX_BLOCKS = 8


class DraftBatch:
    """Host-validated per-round draft metadata, uploaded once and reused by
    every draft layer.

    context_offsets[r]: first context row (row store) or first entry of
        context_indices (indexed pool) of request r.
    context_lengths[r]: committed context rows c_r.
    anchors[r]: sequence of block anchors, each in [0, c_r], 1..8 blocks.
    context_indices: optional int64 device tensor of physical pool rows.
    """

    def __init__(self, device, context_offsets, context_lengths, anchors, *, context_indices=None):
        self.device = require_gfx950(device)
        offs = [int(x) for x in context_offsets]
        lens = [int(x) for x in context_lengths]
        blocks = [tuple(int(a) for a in row) for row in anchors]
        if not offs or not (len(offs) == len(lens) == len(blocks)):
            raise ValueError('One offset, context length and anchor list per request required')
        if any(c < 0 for c in lens) or any(o < 0 for o in offs):
            raise ValueError('Context offsets and lengths must be nonnegative')
        if any(not 1 <= len(b) <= MAX_BLOCKS for b in blocks):
            raise ValueError(f'Each request needs 1..{MAX_BLOCKS} draft blocks')
        if any(not 0 <= a <= c for b, c in zip(blocks, lens) for a in b):
            raise ValueError('Every anchor must lie in [0, context length]')
        self.context_offsets = tuple(offs)
        self.context_lengths = tuple(lens)
        self.anchors = tuple(blocks)
        self.request_count = len(offs)
        self.block_count = sum(len(b) for b in blocks)
        self.max_blocks = max(len(b) for b in blocks)
        self.context_rows = sum(lens)
        self.query_rows = BLOCK_SIZE * self.block_count
        cu_b = [0]
        for b in blocks:
            cu_b.append(cu_b[-1] + len(b))
        flat_anchors = [a for b in blocks for a in b]
        self.cu_blocks_host = tuple(cu_b)
        if context_indices is not None:
            if (not isinstance(context_indices, torch.Tensor) or context_indices.dtype != torch.long
                    or context_indices.ndim != 1 or context_indices.device != self.device
                    or not context_indices.is_contiguous()):
                raise ValueError('context_indices must be a contiguous int64 vector on the draft device')
            if any(o + c > context_indices.numel() for o, c in zip(offs, lens)):
                raise ValueError('Context index ranges exceed context_indices')
        self.context_indices = context_indices
        self._index_max = None
        pinned64 = torch.tensor(offs, dtype=torch.int64).pin_memory()
        pinned32 = torch.tensor(lens + cu_b + flat_anchors, dtype=torch.int32).pin_memory()
        self.ctx_off = pinned64.to(self.device, non_blocking=True)
        meta = pinned32.to(self.device, non_blocking=True)
        b = self.request_count
        self.ctx_len = meta[:b]
        self.cu_blocks = meta[b:2 * b + 1]
        self.anchor_rows = meta[2 * b + 1:]

    def index_max(self):
        """Largest physical context row addressed (one device sync, cached)."""
        if self.context_indices is None:
            return max((o + c for o, c in zip(self.context_offsets, self.context_lengths)), default=0) - 1
        if self._index_max is None:
            used = [self.context_indices[o:o + c] for o, c in zip(self.context_offsets, self.context_lengths) if c]
            if used:
                cat = torch.cat(used)
                lo, hi = int(cat.min()), int(cat.max())
                if lo < 0:
                    raise ValueError('Negative context index')
                self._index_max = hi
            else:
                self._index_max = -1
        return self._index_max


class HipDraftAttention:
    """Multi-block draft attention kernel object (one launch per layer, plus a
    split-K merge for contexts longer than one chunk)."""
    backend_name = 'mi355x_hip_draft_blocks_v1'
    native_varlen_calls_per_layer = 1

    def __init__(self, device, *, chunk=DEFAULT_CHUNK):
        self.device = require_gfx950(device)
        _native.load()
        if chunk % 64:
            raise ValueError('Draft chunk must be a multiple of 64')
        self.chunk = int(chunk)
        self._workspace = Workspace(self.device)

    def __call__(self, query, block_keys, block_values, context_keys, context_values, batch, *, scale):
        if not isinstance(batch, DraftBatch) or batch.device != self.device:
            raise ValueError('DraftBatch on the kernel device required')
        _check_scale(scale, 'HIP draft attention')
        nq = batch.query_rows
        for t, shape in ((query, (nq, Q_HEADS, HEAD_DIM)), (block_keys, (nq, KV_HEADS, HEAD_DIM)),
                         (block_values, (nq, KV_HEADS, HEAD_DIM))):
            if (not isinstance(t, torch.Tensor) or t.dtype != torch.bfloat16 or t.device != self.device
                    or tuple(t.shape) != shape or not t.is_contiguous() or t.requires_grad):
                raise ValueError('Draft Q/block K/V must be contiguous no-autograd bf16 [7*blocks,H,128] on the GPU')
        if (not isinstance(context_keys, torch.Tensor) or not isinstance(context_values, torch.Tensor)
                or context_keys.shape != context_values.shape or context_keys.dtype != torch.bfloat16
                or context_values.dtype != torch.bfloat16 or context_keys.device != self.device
                or context_values.device != self.device
                or not context_keys.is_contiguous() or not context_values.is_contiguous()):
            raise ValueError('Context K/V must be matching contiguous bf16 tensors on the GPU')
        if context_keys.ndim == 3 and tuple(context_keys.shape[1:]) == (KV_HEADS, HEAD_DIM):
            rows, tok_stride, head_stride = context_keys.shape[0], KV_HEADS * HEAD_DIM, HEAD_DIM
        elif context_keys.ndim == 4 and context_keys.shape[0] == 1 and context_keys.shape[1] == KV_HEADS \
                and context_keys.shape[3] == HEAD_DIM:
            rows, tok_stride, head_stride = context_keys.shape[2], HEAD_DIM, context_keys.shape[2] * HEAD_DIM
            if batch.context_indices is None:
                raise ValueError('A [1,8,N,128] pool needs per-request context indices')
        else:
            raise ValueError('Context K/V must be [rows,8,128] or [1,8,N,128]')
        if batch.index_max() >= rows:
            raise ValueError('Context rows addressed beyond the context tensor')
        out = torch.empty_like(query)
        bound = max(batch.context_rows, 1)
        need = _native.load().dspark_attn_workspace_bytes(batch.request_count, bound, batch.max_blocks, self.chunk)
        ws = self._workspace.get(need)
        _native.call('dspark_draft_attn_fwd', _native.ptr(query), _native.ptr(context_keys), _native.ptr(context_values),
                     _native.ptr(batch.context_indices), _native.ptr(batch.ctx_off), _native.ptr(batch.ctx_len),
                     tok_stride, head_stride, _native.ptr(block_keys), _native.ptr(block_values),
                     _native.ptr(batch.cu_blocks), _native.ptr(batch.anchor_rows), batch.request_count, bound,
                     batch.max_blocks, float(SCALE), self.chunk, _native.ptr(out), _native.ptr(ws), ws.numel(),
                     _native.stream_handle(self.device))
        return out
