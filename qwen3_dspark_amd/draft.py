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

The context K/V of one draft layer may live in
  * a row store [rows, 8, 128]: request r uses rows off_r .. off_r + c_r;
  * a head-major slotted pool [slots, 8, capacity, 128] (one contiguous run
    per (slot, KV head), the layout the draft kernel streams fastest): off_r =
    slot * capacity + first position;
  * the reference's append-order pool layer [1, 8, N, 128] with per-request
    physical indices (PackedLayout.gather_indices order): off_r indexes the
    index vector.
"""
import numpy as np
import torch

from . import _native, backends
from ._device import Workspace, cu_count, kv_pair, require_gfx950, upload
from .kernels import HEAD_DIM, KV_HEADS, Q_HEADS, SCALE, _check_scale
from .schedule import draft_chunk_for, draft_run_count, draft_work, upload_work

BLOCK_SIZE = 7
MAX_BLOCKS = 8
APPEND_LAYERS = 16            # layers per dspark_pool_append launch (its pointer arrays)
_QK_DTYPES = (torch.bfloat16, torch.float32)


def draft_work_counters(context_lengths, anchors, *, layers=1, physical_context_rows=None, block_size=BLOCK_SIZE,
                        key_element_bytes=2, value_element_bytes=2):
    """Work counters of a packed draft backbone's attention, with the keys
    of packed_draft.py:245-249, for the fused multi-block path.

    Rows and pair domain follow the reference's layout (a request's keys are
    its context up to its largest anchor plus its blocks' rows; each block
    pairs its rows with anchor + block_size keys).  The reference's
    concatenation, gather and cast copies do not exist on this path (the
    kernel reads the pool in place and rounds K to bf16 in registers), so
    their counters are 0; kv_bytes_read_per_layer is what the kernel reads.
    """
    blocks = sum(len(b) for b in anchors)
    streamed = sum(max(b) for b in anchors)
    gathered = streamed + block_size * blocks
    row_bytes = KV_HEADS * HEAD_DIM * (key_element_bytes + value_element_bytes)
    return dict(
        requests=len(anchors), query_rows=block_size * blocks, gathered_key_rows=gathered,
        physical_context_rows=sum(context_lengths) if physical_context_rows is None else physical_context_rows,
        attention_pair_domain=sum(block_size * (a + block_size) for b in anchors for a in b),
        attention_calls=layers,
        context_block_concatenation_kv_elements=0, context_block_concatenation_kv_bytes=0,
        gathered_kv_elements=0, gathered_kv_bytes=0, attention_cast_elements=0, attention_cast_output_bytes=0,
        draft_blocks=blocks, context_rows_read_per_layer=streamed, kv_bytes_read_per_layer=gathered * row_bytes,
        scope='Work counts only; context rows read in place once per request for all of its blocks')


class DraftBatch:
    """Host-validated per-round draft metadata, uploaded once and reused by
    every draft layer.

    context_offsets[r]: see the module docstring for each pool form.
    context_lengths[r]: committed context rows c_r.
    anchors[r]: sequence of block anchors, each in [0, c_r], one or more.
    context_indices: optional int64 device tensor of physical pool rows.

    The kernel attends at most MAX_BLOCKS blocks of a request per pass over
    its context: a request with more blocks is planned as consecutive views
    of at most MAX_BLOCKS blocks over the same context (each view streams
    the context once).  Output rows stay block-major in the given order.
    The per-request attributes below (context_offsets, context_lengths,
    anchors, request_count, ...) describe these views, which is what the
    kernel and the work counters see; `views[i]` names view i's request and
    first block, and `requests` is the number of requests given.
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
        if any(not b for b in blocks):
            raise ValueError('Each request needs at least one draft block')
        if any(not 0 <= a <= c for b, c in zip(blocks, lens) for a in b):
            raise ValueError('Every anchor must lie in [0, context length]')
        self.requests = len(blocks)
        views = [(r, j) for r, b in enumerate(blocks) for j in range(0, len(b), MAX_BLOCKS)]
        self.views = tuple(views)
        offs = [offs[r] for r, _ in views]
        lens = [lens[r] for r, _ in views]
        blocks = [blocks[r][j:j + MAX_BLOCKS] for r, j in views]
        if context_indices is not None:
            if (not isinstance(context_indices, torch.Tensor) or context_indices.dtype != torch.long
                    or context_indices.ndim != 1 or context_indices.device != self.device
                    or not context_indices.is_contiguous()):
                raise ValueError('context_indices must be a contiguous int64 vector on the draft device')
            if any(o + c > context_indices.numel() for o, c in zip(offs, lens)):
                raise ValueError('Context index ranges exceed context_indices')
        self.context_offsets = tuple(offs)
        self.context_lengths = tuple(lens)
        self.anchors = tuple(blocks)
        self.context_indices = context_indices
        self.request_count = len(offs)
        self.block_count = sum(len(b) for b in blocks)
        self.max_blocks = max(len(b) for b in blocks)
        self.context_rows = sum(lens)
        self.query_rows = BLOCK_SIZE * self.block_count
        cu_b = [0]
        for b in blocks:
            cu_b.append(cu_b[-1] + len(b))
        self.cu_blocks_host = tuple(cu_b)
        # Device metadata (lengths, block offsets, anchors) is uploaded on
        # first use, together with a plan's offsets and work list when
        # prepare() comes first (one copy instead of three).
        self._meta_host = lens + cu_b + [a for b in blocks for a in b]
        self._meta = None
        self._offsets = {}
        self._work = {}
        self._chunk = None            # the batch-sized draft chunk, once computed
        self._index_max = None
        self.physical_context_rows = self.context_rows

    def _device_meta(self):
        if self._meta is None:
            self._meta = upload(self.device, self._meta_host)
        return self._meta

    @property
    def ctx_len(self):
        """[n] int32 device: committed context rows per (view of a) request."""
        return self._device_meta()[:self.request_count]

    @property
    def cu_blocks(self):
        """[n+1] int32 device: block offsets."""
        n = self.request_count
        return self._device_meta()[n:2 * n + 1]

    @property
    def anchor_rows(self):
        """[blocks] int32 device: context rows visible to each block."""
        return self._device_meta()[2 * self.request_count + 1:]

    @classmethod
    def from_packed_layout(cls, layout, *, block_size=BLOCK_SIZE):
        """The batch of the reference's one-block backbone call
        (packed_draft.py:205-226), from the PackedLayout it builds over the
        metadata of cat(pool, block): request r's keys are its c_r context
        rows (pool rows in position order) followed by its own block_size
        rows, and its queries are those block rows.  The batch reads the
        context through layout.gather_indices from the [1, 8, N, 128] pool
        in place (one block per request at anchor c_r); the block's own rows
        come as separate block K/V."""
        qs, ks = tuple(layout.query_lengths), tuple(layout.key_lengths)
        if not qs or len(qs) != len(ks) or any(q != block_size for q in qs) or any(k < block_size for k in ks):
            raise ValueError('Each request must query exactly its own draft block')
        first = [0]
        for k in ks[:-1]:
            first.append(first[-1] + k)
        contexts = [k - block_size for k in ks]
        indices = layout.gather_indices
        return cls(indices.device, first, contexts, [[c] for c in contexts], context_indices=indices)

    def counters(self, layers=1, *, key_element_bytes=2, value_element_bytes=2):
        """draft_work_counters of this batch over `layers` attention calls."""
        return draft_work_counters(self.context_lengths, self.anchors, layers=layers,
                                   physical_context_rows=self.physical_context_rows,
                                   key_element_bytes=key_element_bytes, value_element_bytes=value_element_bytes)

    def kernel_offsets(self, capacity):
        """Per-request first kernel row: offsets as given, or - for a
        head-major slotted pool of `capacity` positions - slot*8*capacity +
        position, the row index in units of 128 elements."""
        offs = list(self.context_offsets)
        if capacity:
            offs = [o + (KV_HEADS - 1) * capacity * (o // capacity) for o in offs]
        return offs

    def device_offsets(self, capacity):
        """kernel_offsets(capacity) as an int64 device vector."""
        if capacity not in self._offsets:
            self._offsets[capacity] = upload(self.device, self.kernel_offsets(capacity), torch.int64)
        return self._offsets[capacity]

    def prepare(self, chunk, runs=None, capacity=None):
        """(device_offsets(capacity), work(chunk, runs, capacity)), with the
        batch metadata, the offsets and the work list that are not on the
        device yet uploaded in one copy: int32 [metadata | int64 offsets |
        work list], each part 16-byte aligned."""
        key = (chunk, runs, capacity)
        missing = (self._meta is None) + (capacity not in self._offsets) + (key not in self._work)
        if missing >= 2:
            meta = self._meta_host if self._meta is None else []
            offs = (np.asarray(self.kernel_offsets(capacity), dtype=np.int64).view(np.int32).tolist()
                    if capacity not in self._offsets else [])
            plan = self._work_host(chunk, runs, capacity) if key not in self._work else None
            parts, at = [], []
            for part in (meta, offs, plan[0] if plan else []):
                at.append(sum(len(p) for p in parts))
                parts.append(list(part) + [0] * (-len(part) % 4))
            dev = upload(self.device, [x for p in parts for x in p])
            if meta:
                self._meta = dev[at[0]:at[0] + len(meta)]
            if offs:
                self._offsets[capacity] = dev[at[1]:at[1] + len(offs)].view(torch.int64)
            if plan:
                records, n_seg, n_runs, anchor_at = plan
                w = dev[at[2]:at[2] + len(records)]
                self._work[key] = (w, n_seg, n_runs, None if anchor_at is None else w[anchor_at:])
        return self.device_offsets(capacity), self.work(chunk, runs, capacity)

    def work(self, chunk, runs=None, capacity=None):
        """(device list, segment count, run count, segment anchors) of the
        draft plan: fixed chunks longest first (runs None), or `runs`
        balanced runs per KV head (0: one per CU).  With a pool capacity (0:
        flat rows) the segment records also carry each request's kernel
        offset.  Segment anchors (fixed-chunk plans, for the persistent
        kernel): 8 int32 per segment record, the anchors of its request's
        blocks, zero-padded, in the same upload at a 16-byte boundary (None
        for balanced runs).  Uploaded once per plan."""
        key = (chunk, runs, capacity)
        if key not in self._work:
            records, n_seg, n_runs, anchor_at = self._work_host(chunk, runs, capacity)
            dev = upload_work(records, self.device)
            self._work[key] = (dev, n_seg, n_runs, None if anchor_at is None else dev[anchor_at:])
        return self._work[key]

    def _work_host(self, chunk, runs, capacity):
        """The host side of work(): (records, segment count, run count,
        index of the segment anchor table or None)."""
        flat = [a for b in self.anchors for a in b]
        offs = None if capacity is None else self.kernel_offsets(capacity)
        if runs is None:
            plan = draft_work(self.context_lengths, self.cu_blocks_host, flat, chunk=chunk, offsets=offs)
        else:
            runs = runs or draft_run_count(sum(max(b) for b in self.anchors), cu_count(self.device))
            plan = draft_work(self.context_lengths, self.cu_blocks_host, flat, runs, offsets=offs)
        records, n_seg, n_runs = plan
        records = list(records)
        anchor_at = None
        if runs is None:
            records += [0] * (-len(records) % 4)           # the anchor table starts 16-byte aligned
            anchor_at = len(records)
            for i in range(n_seg):
                b0, nb = records[8 * i + 4], records[8 * i + 5]
                records += flat[b0:b0 + nb] + [0] * (8 - nb)
        return records, n_seg, n_runs, anchor_at

    def index_max(self):
        """Largest physical index addressed through context_indices (one
        device sync, cached)."""
        if self._index_max is None:
            used = [self.context_indices[o:o + c] for o, c in zip(self.context_offsets, self.context_lengths) if c]
            if used:
                cat = torch.cat(used)
                if int(cat.min()) < 0:
                    raise ValueError('Negative context index')
                self._index_max = int(cat.max())
                if self._index_max >= 2 ** 31:
                    raise ValueError('Context indices must lie below 2^31 (the kernel reads their low words)')
            else:
                self._index_max = -1
        return self._index_max


class HipDraftAttention:
    """Multi-block draft attention kernel object (one chunk launch per layer
    plus a split-K merge launch)."""
    backend_name = backends.DRAFT_BLOCKS_BACKEND
    native_varlen_calls_per_layer = 1

    def __init__(self, device, *, chunk=None, runs=None, persistent=1):
        """chunk: rows per (chunk, KV head) item of the fixed-chunk plan, a
        multiple of 64; None (the default) sizes it to each batch
        (schedule.draft_chunk_for: about one item per CU, at most 4096 rows).
        persistent: 1 (the default) or 8 for one persistent workgroup per CU
        taking (chunk, KV head) items, longest chunks first, from one device
        queue or from one queue per KV head (head g on XCD g); None for one
        workgroup per (run, KV head) dispatched by the hardware (the only
        form for balanced runs).  Outputs are bitwise the same in every
        mode.  One object's launches must not overlap (they share its ticket
        counters): use it from one stream."""
        self.device = require_gfx950(device)
        _native.load()
        if chunk is not None and (type(chunk) is not int or chunk <= 0 or chunk % 64):
            raise ValueError('Draft chunk must be None or a positive multiple of 64')
        if runs is not None and (type(runs) is not int or runs < 0):
            raise ValueError('runs must be None (fixed chunks) or a nonnegative integer (balanced runs)')
        if persistent not in (None, 1, 8):
            raise ValueError('persistent must be None, 1 or 8 (queues)')
        if runs is not None and persistent is not None:
            raise ValueError('balanced runs (runs=...) need persistent=None')
        self.chunk = chunk          # None: sized to each batch
        self.runs = runs            # None: fixed chunks; else balanced runs per KV head (0: one per CU)
        self.persistent = persistent
        # Ticket counters of the persistent mode: zero now, zero again after every launch.
        self._queue = torch.zeros(16, dtype=torch.int32, device=self.device) if persistent else None
        self._workgroups = -(-cu_count(self.device) // 8) * 8 if persistent else 0
        self._workspace = Workspace(self.device)
        self._geometry_for = None
        self._geometry = None
        self._packed = None         # (layout, DraftBatch) of over_append_order_pool

    def _context_geometry(self, keys, batch):
        """(offset capacity for DraftBatch.kernel_offsets, token stride, head
        stride) for the pool form."""
        if keys.ndim == 3 and tuple(keys.shape[1:]) == (KV_HEADS, HEAD_DIM):
            if batch.context_indices is not None:
                if batch.index_max() >= keys.shape[0]:
                    raise ValueError('Context rows addressed beyond the context tensor')
            elif any(o + c > keys.shape[0] for o, c in zip(batch.context_offsets, batch.context_lengths)):
                raise ValueError('Context rows addressed beyond the context tensor')
            return 0, KV_HEADS * HEAD_DIM, HEAD_DIM
        if keys.ndim == 4 and keys.shape[1] == KV_HEADS and keys.shape[3] == HEAD_DIM:
            slots, cap = keys.shape[0], keys.shape[2]
            if batch.context_indices is not None:
                if slots != 1 or batch.index_max() >= cap:
                    raise ValueError('An indexed pool must be [1,8,N,128] with indices < N')
                return 0, HEAD_DIM, cap * HEAD_DIM
            for o, c in zip(batch.context_offsets, batch.context_lengths):
                if o // cap >= slots or (o % cap) + c > cap:
                    raise ValueError('Context rows addressed beyond their pool slot')
            return cap, HEAD_DIM, cap * HEAD_DIM
        raise ValueError('Context K/V must be [rows,8,128], [slots,8,capacity,128] or [1,8,N,128]')

    def plan(self, batch, context_keys):
        """Check the batch against the context pool form and upload its plan
        (kernel offsets, work list, segment anchors) and size the split-K
        workspace: what a call does before its launch.  Cached per batch and
        pool shape, so a caller may prepare a round's batch ahead of its
        draft layers (as begin() prepares a verification transaction)."""
        key = (batch, context_keys.shape)
        if self._geometry_for is None or self._geometry_for[0] is not batch or self._geometry_for[1] != key[1]:
            self._geometry = self._context_geometry(context_keys, batch)
            self._geometry_for = key
        capacity, tok_stride, head_stride = self._geometry
        chunk = self.chunk_for(batch)
        offsets, (work, n_work, n_runs, seg_anchors) = batch.prepare(chunk, self.runs, capacity)
        need = _native.load().dspark_attn_workspace_bytes(n_work, 0, batch.max_blocks, chunk)
        ws = self._workspace.get(need)
        return capacity, tok_stride, head_stride, offsets, work, n_work, n_runs, seg_anchors, ws, chunk

    def chunk_for(self, batch):
        """The fixed chunk the plan of `batch` uses: the constructor's, or
        sized to the batch's visible context rows."""
        if self.chunk is not None:
            return self.chunk
        if batch._chunk is None:
            batch._chunk = draft_chunk_for(sum(max(b) for b in batch.anchors), cu_count(self.device))
        return batch._chunk

    def __call__(self, query, block_keys, block_values, context_keys, context_values, batch, *, scale):
        """Q [7*blocks, 16, 128], block K/V [7*blocks, 8, 128], context K/V in
        one of the pool forms of the module docstring.  V is bf16.  Q and K
        (context and block K alike) may be bf16 or fp32: fp32 values are
        rounded to bf16 as the kernel loads them, the cast the reference
        applies at its kernel boundary under autocast (packed_draft.py:222-235),
        so an fp32-K pool (the reference's AMP form: FP32 K, BF16 V) needs no
        cast copy.  Returns bf16 [7*blocks, 16, 128]."""
        if not isinstance(batch, DraftBatch) or batch.device != self.device:
            raise ValueError('DraftBatch on the kernel device required')
        _check_scale(scale, 'HIP draft attention')
        nq = batch.query_rows
        for t, shape, dtypes in ((query, (nq, Q_HEADS, HEAD_DIM), _QK_DTYPES),
                                 (block_keys, (nq, KV_HEADS, HEAD_DIM), _QK_DTYPES),
                                 (block_values, (nq, KV_HEADS, HEAD_DIM), (torch.bfloat16,))):
            if (not isinstance(t, torch.Tensor) or t.dtype not in dtypes or t.device != self.device
                    or tuple(t.shape) != shape or not t.is_contiguous() or t.requires_grad):
                raise ValueError('Draft Q/block K (bf16 or fp32) and block V (bf16) must be contiguous '
                                 'no-autograd [7*blocks,H,128] tensors on the GPU')
        if (not isinstance(context_keys, torch.Tensor) or not isinstance(context_values, torch.Tensor)
                or context_keys.shape != context_values.shape or context_keys.dtype not in _QK_DTYPES
                or context_values.dtype != torch.bfloat16 or context_keys.device != self.device
                or context_values.device != self.device
                or not context_keys.is_contiguous() or not context_values.is_contiguous()):
            raise ValueError('Context K (bf16 or fp32) and V (bf16) must be matching contiguous tensors on the GPU')
        if block_keys.dtype != context_keys.dtype:
            raise ValueError('Backbone/cache precision mismatch')
        capacity, tok_stride, head_stride, offsets, work, n_work, n_runs, seg_anchors, ws, chunk = self.plan(
            batch, context_keys)
        out = torch.empty(query.shape, dtype=torch.bfloat16, device=self.device)
        bound = max(batch.context_rows, 1)
        _native.call('dspark_draft_attn_fwd', _native.ptr(query), int(query.dtype == torch.float32),
                     _native.ptr(context_keys), _native.ptr(context_values), int(context_keys.dtype == torch.float32),
                     _native.ptr(batch.context_indices), _native.ptr(offsets), _native.ptr(batch.ctx_len),
                     tok_stride, head_stride, _native.ptr(block_keys), _native.ptr(block_values),
                     _native.ptr(batch.cu_blocks), _native.ptr(batch.anchor_rows), batch.request_count, bound,
                     batch.max_blocks, float(SCALE), chunk, _native.ptr(work), n_work, n_runs,
                     self._workgroups, self.persistent or 0, _native.ptr(self._queue),
                     _native.ptr(seg_anchors) if self.persistent else None,
                     _native.ptr(out), _native.ptr(ws), ws.numel(), _native.stream_handle(self.device))
        return out


    def over_append_order_pool(self, query, block_keys, block_values, pool_keys, pool_values, layout, *, scale):
        """The attention of the reference's backbone layer over its own
        append-order pool (packed_draft.py:219-236 in one call): query
        [7B, 16, 128]; block K/V as project_kv returns them, [1, 8, 7B, 128]
        (or [7B, 8, 128]); pool K/V the layer's [1, 8, N, 128] tensors (None
        before the first append); layout the PackedLayout of that backbone
        call.  The context is read through the layout's gather indices in
        place: no cat, no gather copy and no cast copy of the pool.  V must
        be bf16; fp32 Q/K (the AMP pool) are rounded as they are loaded."""
        if self._packed is None or self._packed[0] is not layout:
            self._packed = (layout, DraftBatch.from_packed_layout(layout))
        batch = self._packed[1]

        def rows(t):
            if isinstance(t, torch.Tensor) and t.ndim == 4 and t.shape[0] == 1:
                t = t[0].transpose(0, 1)
            return t.contiguous() if isinstance(t, torch.Tensor) else t
        block_keys, block_values = rows(block_keys), rows(block_values)
        if pool_keys is None and pool_values is None:
            if batch.context_rows:
                raise ValueError('Context rows addressed beyond the context tensor')
            kdt = block_keys.dtype if isinstance(block_keys, torch.Tensor) else torch.bfloat16
            pool_keys = torch.zeros((1, KV_HEADS, 1, HEAD_DIM), dtype=kdt, device=self.device)
            pool_values = torch.zeros((1, KV_HEADS, 1, HEAD_DIM), dtype=torch.bfloat16, device=self.device)
        return self(query, block_keys, block_values, pool_keys, pool_values, batch, scale=scale)


class DraftKVPool:
    """Projected draft context per request: the cache state of PackedDraft
    (dspark_qwen/packed_draft.py:63-185) without the model.

    Storage: K and V are [layers, slots, 8, capacity, 128] head-major, one
    contiguous run per (layer, slot, KV head), each request owning one slot.
    Consequences against the reference's append-order pool [1, 8, N, 128]:
      * append_projected writes the new rows in place (one launch for all
        layers and requests); the reference concatenates the whole pool;
      * crop / remove_request only change lengths; the reference compacts
        every layer with a keep mask;
      * draft attention streams each request's context as one linear run.
    Rows arrive either already projected (append_projected) or as target
    features that a DraftContextProjector turns into every layer's K/V in
    place (append_committed, the reference's method: fc, context_norm, RoPE,
    k_proj, k_norm, v_proj of packed_draft.py:147-158).
    Appends are transactional: rows land beyond the committed lengths and
    become visible only when every check, including finiteness, passed.

    K and V may differ in precision: key_dtype / value_dtype (default dtype).
    The reference's pool under bf16 autocast holds FP32 K (its k_norm runs in
    FP32) and BF16 V (packed_draft.py:222-235); attention reads such a pool in
    place and rounds K to bf16 in registers.

    With growable=True the slot count and per-slot capacity are starting
    sizes: a request admitted with every slot taken doubles the slots, an
    append beyond a slot's capacity at least doubles the capacity (rounded up
    to GROW_ALIGN rows).  A resize allocates the new pool and copies every
    committed row once, so n appends cost O(log n) copies of the pool where
    the reference's append-order pool concatenates all of it on every append
    (packed_draft.py:157-158).  Without growable the sizes are fixed and an
    overflow raises.
    """

    GROW_ALIGN = 256

    def __init__(self, *, layers, slots, capacity, heads=KV_HEADS, dim=HEAD_DIM, dtype=torch.bfloat16,
                 key_dtype=None, value_dtype=None, device='cuda', chunk=None, projector=None,
                 growable=False):
        if any(type(n) is not int or n < 1 for n in (layers, slots, capacity, heads, dim)):
            raise ValueError('All pool sizes must be positive integers')
        key_dtype = dtype if key_dtype is None else key_dtype
        value_dtype = dtype if value_dtype is None else value_dtype
        if any(d not in (torch.bfloat16, torch.float32) for d in (dtype, key_dtype, value_dtype)):
            raise ValueError('Draft pool dtype must be bfloat16 or float32')
        self.device = require_gfx950(device)
        _native.load()
        self.layers, self.slot_capacity, self.capacity, self.heads, self.dim = layers, slots, capacity, heads, dim
        self.key_dtype, self.value_dtype = key_dtype, value_dtype
        self.dtype = key_dtype if key_dtype == value_dtype else None
        self._elems = (torch.empty((), dtype=key_dtype).element_size(),
                       torch.empty((), dtype=value_dtype).element_size())
        if any((dim * e) % 16 for e in self._elems):
            raise ValueError('A KV head row must be a multiple of 16 bytes')
        self.keys, self.values = kv_pair((layers, slots, heads, capacity, dim), key_dtype, value_dtype, self.device)
        self.growable = bool(growable)
        self.resizes = 0
        self._lengths = {}
        self._slots = {}
        self._free = list(range(slots))
        self._attention = HipDraftAttention(self.device, chunk=chunk) if (heads, dim) == (KV_HEADS, HEAD_DIM) else None
        self._flag = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.last_append_work = None
        if projector is not None and (projector.layers != layers or projector.device != self.device
                                      or (heads, dim, self.dtype) != (KV_HEADS, HEAD_DIM, torch.bfloat16)):
            raise ValueError('The projector needs a bf16 8x128 pool with its layer count on its device')
        self.projector = projector

    @property
    def lengths(self):
        return dict(self._lengths)

    @property
    def kernel(self):
        """The pool's HipDraftAttention (None unless the geometry is 8 x 128)."""
        return self._attention

    def length(self, request):
        """Committed context rows of a request (KeyError if unknown)."""
        self._request(request)
        return self._lengths[request]

    def slot(self, request):
        self._request(request)
        return self._slots[request]

    def add_request(self, request):
        if not isinstance(request, str) or not request or request in self._lengths:
            raise ValueError('Require a fresh nonempty request name')
        if not self._free:
            if not self.growable:
                raise ValueError('Draft pool slot capacity exhausted')
            self._resize(2 * self.slot_capacity, self.capacity)
        self._slots[request] = self._free.pop(0)
        self._lengths[request] = 0

    def _resize(self, slots, capacity):
        """Reallocate the pool as [layers, slots, heads, capacity, dim] and
        copy every slot's committed rows to the same slot and positions."""
        old_k, old_v, old_s, old_c = self.keys, self.values, self.slot_capacity, self.capacity
        shape = (self.layers, slots, self.heads, capacity, self.dim)
        keys, values = kv_pair(shape, self.key_dtype, self.value_dtype, self.device)
        used = max(self._lengths.values(), default=0)
        if used:
            keys[:, :old_s, :, :used].copy_(old_k[:, :, :, :used])
            values[:, :old_s, :, :used].copy_(old_v[:, :, :, :used])
        self.keys, self.values = keys, values
        self._free += list(range(old_s, slots))
        self.slot_capacity, self.capacity = slots, capacity
        self.resizes += 1

    def _reserve(self, needed):
        """Make room for `needed` committed rows in a slot: grow the capacity
        of a growable pool, else raise."""
        if needed <= self.capacity:
            return
        if not self.growable:
            raise ValueError('Committed draft context exceeds the pool capacity')
        align = self.GROW_ALIGN
        self._resize(self.slot_capacity, max(2 * self.capacity, -(-needed // align) * align))

    def _request(self, request):
        if request not in self._lengths:
            raise KeyError(request)

    def validate_cache(self):
        """Host state invariants (packed_draft.py:102-122 checks the same
        prefix property on its append-order metadata)."""
        if len(set(self._slots.values())) != len(self._slots) or set(self._slots) != set(self._lengths):
            raise RuntimeError('Draft cache metadata length mismatch')
        if any(not 0 <= n <= self.capacity for n in self._lengths.values()):
            raise RuntimeError('Draft cache must be the complete request-local committed prefix')

    def _source(self, t, rows, dtype):
        """(head stride, row stride) in bytes of a [1, H, rows, D] or
        [rows, H, D] tensor of new K or V rows of the pool's `dtype`."""
        if not isinstance(t, torch.Tensor) or t.device != self.device:
            raise ValueError('Projected K/V must be tensors on the pool device')
        if t.dtype != dtype:
            raise ValueError('Draft cache precision cannot change across appends')
        e = t.element_size()
        if t.ndim == 4 and tuple(t.shape) == (1, self.heads, rows, self.dim) and t.stride(3) == 1:
            strides = (t.stride(1) * e, t.stride(2) * e)
        elif t.ndim == 3 and tuple(t.shape) == (rows, self.heads, self.dim) and t.stride(2) == 1:
            strides = (t.stride(1) * e, t.stride(0) * e)
        else:
            raise ValueError('Projected K/V must be [1, heads, rows, dim] or [rows, heads, dim]')
        if any(x % 16 for x in strides) or t.data_ptr() % 16:
            raise ValueError('Projected K/V rows must be 16-byte aligned')
        return strides

    @torch.no_grad()
    def append_projected(self, chunks, projected, *, check_finite=True):
        """Append committed context rows.  chunks: ordered {request: rows};
        projected: per layer (keys, values) holding the rows of all chunks in
        that order (what one projection over the concatenated features
        yields, packed_draft.py:147-158).  With check_finite (the reference
        always checks), one device read decides whether the append is
        published; a nonfinite element raises and leaves the pool as it was."""
        if not chunks:
            raise ValueError('Require at least one committed feature chunk')
        self.validate_cache()
        order = list(chunks.items())
        for request, n in order:
            self._request(request)
            if type(n) is not int or n < 1:
                raise ValueError('Each committed chunk needs a positive row count')
            if self._lengths[request] + n > self.capacity and not self.growable:
                raise ValueError('Committed draft context exceeds the pool capacity')
        rows = sum(n for _, n in order)
        if len(projected) != self.layers:
            raise ValueError('Draft cache layer count mismatch')
        strides = [None, None]
        for k, v in projected:
            for i, (t, dt) in enumerate(((k, self.key_dtype), (v, self.value_dtype))):
                st = self._source(t, rows, dt)
                if strides[i] is not None and st != strides[i]:
                    raise ValueError('Projected K/V must share one layout across layers')
                strides[i] = st
        self._reserve(max(self._lengths[r] + n for r, n in order))
        req, offset = [[], [], [], []], 0
        for request, n in order:
            req[0].append(self._slots[request])
            req[1].append(self._lengths[request])
            req[2].append(offset)
            req[3].append(n)
            offset += n
        dev_req = upload(self.device, [x for row in req for x in row])
        if check_finite:
            self._flag.zero_()
        H, C, D = self.heads, self.capacity, self.dim
        ks, vs = [k for k, _ in projected], [v for _, v in projected]
        # One launch for K and V together when they share a row size, else one each.
        if self._elems[0] == self._elems[1] and strides[0] == strides[1]:
            parts = [(self.keys, self.values, ks, vs, self._elems[0], strides[0])]
        else:
            parts = [(self.keys, None, ks, None, self._elems[0], strides[0]),
                     (None, self.values, None, vs, self._elems[1], strides[1])]
        launches = 0
        for kp, vp, ksrc, vsrc, e, st in parts:
            # one launch takes the source pointers of up to APPEND_LAYERS layers
            for l0 in range(0, self.layers, APPEND_LAYERS):
                l1 = min(self.layers, l0 + APPEND_LAYERS)
                _native.call('dspark_pool_append', None if kp is None else _native.ptr(kp[l0]),
                             None if vp is None else _native.ptr(vp[l0]),
                             self.slot_capacity * H * C * D * e, H * C * D * e, C * D * e, D * e, C, H, D * e, e,
                             l1 - l0, None if ksrc is None else _native.pointer_array(ksrc[l0:l1]),
                             None if vsrc is None else _native.pointer_array(vsrc[l0:l1]), st[0], st[1], rows,
                             dev_req.data_ptr(), len(order), self._flag.data_ptr() if check_finite else None,
                             _native.stream_handle(self.device))
                launches += 1
        if check_finite and int(self._flag.item()):
            raise RuntimeError('Nonfinite projected draft context')
        for request, n in order:
            self._lengths[request] += n
        self.last_append_work = dict(requests=len(order), new_context_tokens=rows, append_launches=launches,
                                     appended_kv_bytes=self.layers * rows * H * D * sum(self._elems),
                                     cache_concatenation_kv_bytes=0)
        return self.last_append_work

    @torch.no_grad()
    def append_committed(self, chunks):
        """Project and append committed target features (packed_draft.py:130-168).
        chunks: ordered {request: features [1, tokens, 5*hidden]}.  One fc
        over all chunks and one fused projection launch for every layer
        write the rows beyond the committed lengths; one device read then
        decides: non-finite features raise ValueError, a non-finite
        projection RuntimeError, and either leaves the pool as it was."""
        proj = self.projector
        if proj is None:
            raise ValueError('append_committed needs a DraftContextProjector')
        if not chunks:
            raise ValueError('Require at least one committed feature chunk')
        self.validate_cache()
        order = list(chunks.items())
        feats = []
        for request, value in order:
            self._request(request)
            if (not isinstance(value, torch.Tensor) or value.ndim != 3 or value.shape[0] != 1 or value.shape[1] < 1
                    or value.shape[2] != proj.features or value.device != self.device
                    or not value.is_floating_point()):
                raise ValueError('Expected finite nonempty [1, tokens, target_features] on draft device')
            if self._lengths[request] + value.shape[1] > self.capacity and not self.growable:
                raise ValueError('Committed draft context exceeds the pool capacity')
            feats.append(value[0])
        self._reserve(max(self._lengths[r] + f.shape[0] for (r, _), f in zip(order, feats)))
        x = (torch.cat(feats) if len(feats) > 1 else feats[0]).to(torch.bfloat16).contiguous()
        rec, first = [], 0
        for (request, _), f in zip(order, feats):
            rec += (self._slots[request], self._lengths[request], first, f.shape[0])
            first += f.shape[0]
        records = upload(self.device, rec)
        self._flag.zero_()
        proj.project_into(proj.fc_forward(x), records, len(order), self.keys, self.values, flag=self._flag)
        bad_in, bad_out = torch.stack((torch.isfinite(x).all().logical_not().to(torch.int32), self._flag[0])).tolist()
        if bad_in:
            raise ValueError('Expected finite nonempty [1, tokens, target_features] on draft device')
        if bad_out:
            raise RuntimeError('Nonfinite projected draft context')
        for request, f in zip(order, feats):
            self._lengths[request[0]] += f.shape[0]
        e, H, D = self._elems[0], self.heads, self.dim
        self.last_append_work = dict(requests=len(order), new_context_tokens=first, context_projection_calls=1,
                                     kv_projection_calls=self.layers, projection_launches=2,
                                     appended_kv_bytes=2 * self.layers * first * H * D * e,
                                     cache_concatenation_kv_elements=0, cache_concatenation_kv_bytes=0)
        return self.last_append_work

    def crop(self, request, length):
        self._request(request)
        if type(length) is not int or not 0 <= length <= self._lengths[request]:
            raise ValueError('Invalid committed draft crop length')
        self._lengths[request] = length

    def remove_request(self, request):
        self.crop(request, 0)
        self._free.append(self._slots.pop(request))
        del self._lengths[request]
        self.validate_cache()

    def request_kv(self, request):
        """Per layer (keys, values) [1, heads, length, dim] copies of the
        request's committed context (packed_draft.py:124-127)."""
        i, n = self.slot(request), self._lengths[request]
        return tuple((self.keys[l, i, :, :n][None].clone(), self.values[l, i, :, :n][None].clone())
                     for l in range(self.layers))

    def batch(self, anchors):
        """DraftBatch over this pool for an ordered {request: anchors}
        mapping (one or more anchors in [0, length] each)."""
        if not anchors:
            raise ValueError('Require active anchor requests')
        names = list(anchors)
        for r in names:
            self._request(r)
        batch = DraftBatch(self.device, [self._slots[r] * self.capacity for r in names],
                           [self._lengths[r] for r in names], [list(anchors[r]) for r in names])
        batch.physical_context_rows = sum(self._lengths.values())
        return batch

    def counters(self, batch):
        """draft_work_counters of a batch over every pool layer, with this
        pool's element sizes."""
        return batch.counters(self.layers, key_element_bytes=self.keys.element_size(),
                              value_element_bytes=self.values.element_size())

    def attention(self, layer, query, block_keys, block_values, batch, *, scale=SCALE):
        """Multi-block draft attention of one layer over the pool."""
        if self._attention is None:
            raise ValueError('Draft attention requires the 8-head, 128-dim geometry')
        if type(layer) is not int or not 0 <= layer < self.layers:
            raise ValueError('Invalid draft layer')
        return self._attention(query, block_keys, block_values, self.keys[layer], self.values[layer], batch,
                               scale=scale)
