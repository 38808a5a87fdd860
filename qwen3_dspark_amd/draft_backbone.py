"""PackedDraft on MI355X: the packed DSpark draft of
dspark_qwen/packed_draft.py:63-249 (cache state, context projection and the
backbone's layer stack) over the slotted draft pool and the fused kernels.

What runs where, per draft round:
  * append_committed: fc on hipBLASLt plus one fused launch that projects
    every layer's context K/V into the pool in place (draft_projection);
  * backbone: the block rows' own path through each draft layer - input
    norm, q/k/v projections, q/k norm and RoPE, o_proj and the MLP - runs on
    the draft module's own torch modules (hipBLASLt GEMMs), exactly the
    modules and order of packed_draft.py:205-245; the attention of every
    layer is one dspark_draft_attn_fwd launch that reads the request's
    context from the pool in place (no whole-pool cat, no gather, no cast
    copy), for all of a request's blocks at once.

The draft module is DSparkDraft-shaped (dspark_qwen/model.py:76-98):
embedding, fc, context_norm, rotary, norm, layers[i] with input_norm,
post_norm, mlp and attention (q_proj, k_proj, v_proj, o_proj, q_norm,
k_norm, heads, kv_heads, dim, project_kv), spec.block_size and
spec.mask_token_id.
"""
from dataclasses import dataclass

import torch

from . import backends
from ._device import require_gfx950
from .draft import BLOCK_SIZE, DraftKVPool
from .draft_projection import DraftContextProjector
from .kernels import HEAD_DIM, KV_HEADS, Q_HEADS


def _rotate(x, cos, sin):
    """Rotate-half RoPE of dspark_qwen/model.py:22-24 (x [1, H, T, D], cos/sin [1, T, D])."""
    left, right = x.chunk(2, dim=-1)
    return x * cos[:, None] + torch.cat((-right, left), -1) * sin[:, None]


@dataclass(frozen=True)
class PackedDraftFeatures:
    """Final draft hidden rows of one backbone call (packed_draft.py:50-60):
    hidden [7 * blocks, hidden] in request order, each request's blocks in
    the order given; blocks[i] blocks for requests[i]."""
    hidden: torch.Tensor
    requests: tuple
    block_size: int
    context_lengths: tuple
    work: dict
    blocks: tuple = ()

    def for_request(self, request):
        index = self.requests.index(request)
        counts = self.blocks or (1,) * len(self.requests)
        first = sum(counts[:index]) * self.block_size
        return self.hidden[first:first + counts[index] * self.block_size]


class PackedDraft:
    """Drop-in for dspark_qwen/packed_draft.py:PackedDraft.

    Constructed like the reference, PackedDraft(draft, native_backend=...,
    test_kernel=None), with the same methods, argument meaning and errors:
    add_request / append_committed / crop / remove_request / request_kv /
    lengths / validate_cache / backbone.  Differences:
      * storage is a slotted pool that grows on demand (DraftKVPool with
        growable=True: slots double when every slot is taken, a slot's
        capacity at least doubles when an append overflows it); passing
        `slots` and `capacity` fixes the sizes instead, and an overflow
        then raises;
      * native_backend must name this build's multi-block draft kernel
        (backends.DRAFT_BLOCKS_BACKEND); a CPU test_kernel is refused with
        the reference's message, since every draft here is on the GPU;
      * backbone_blocks adds one or more blocks per request at any anchors
        (DSparkDraft.backbone's multi-anchor form, model.py:101-119);
        backbone is its one-block form at anchor = committed length.
    Draft weights in float32 (the reference's autocast form) are snapshotted
    to bf16 for the context projection, whose GEMMs the reference's autocast
    runs in bf16 as well.  The attention takes bf16 Q/K/V, or FP32 Q/K under
    bf16 autocast (rounded as the kernel loads them); a float32 draft run
    without autocast is refused with the ValueError of the reference's native
    kernel (rocm_varlen.py:65-70), which takes BF16 tensors only.
    """

    # Starting sizes of the growable pool.
    INITIAL_SLOTS = 8
    INITIAL_CAPACITY = 1024

    def __init__(self, draft, *, native_backend=None, test_kernel=None, slots=None, capacity=None,
                 chunk=None):
        if draft.training:
            raise ValueError('Packed draft is inference-only; call eval first')
        if test_kernel is not None:
            # The reference admits an injected kernel only on a CPU draft with
            # no native backend (packed_draft.py:75-78); drafts here are GPU.
            raise ValueError('CPU-only test injection cannot select a native backend')
        if native_backend != backends.DRAFT_BLOCKS_BACKEND:
            raise ValueError('Select explicit noncausal draft backend; no default/fallback')
        if (slots is None) != (capacity is None):
            raise ValueError('Give both slots and capacity for a fixed pool, or neither for a growable one')
        self.draft = draft
        self.device = require_gfx950(draft.embedding.weight.device)
        attn = [layer.attention for layer in draft.layers]
        if any((a.heads, a.kv_heads, a.dim) != (Q_HEADS, KV_HEADS, HEAD_DIM) for a in attn):
            raise ValueError('HIP packed draft supports Hq16/Hkv8/D128 draft layers only')
        self.block_size = int(draft.spec.block_size)
        if self.block_size != BLOCK_SIZE:
            raise ValueError(f'HIP packed draft supports {BLOCK_SIZE}-row blocks only')
        self.mask_token_id = int(draft.spec.mask_token_id)
        self.projector = self._projector(draft)
        growable = slots is None
        self.pool = DraftKVPool(layers=len(draft.layers), slots=self.INITIAL_SLOTS if growable else slots,
                                capacity=self.INITIAL_CAPACITY if growable else capacity, device=self.device,
                                chunk=chunk, projector=self.projector, growable=growable)
        self.kernel = self.pool.kernel
        self.last_projection_work = None

    def _projector(self, draft):
        """Context projection weights, bf16 (copies of float32 weights)."""
        bf = lambda t: t.detach().to(torch.bfloat16)
        rotary = getattr(draft, 'rotary', None)
        cfg = getattr(rotary, 'config', None)
        params = getattr(cfg, 'rope_parameters', None) or {}
        theta = params.get('rope_theta', getattr(cfg, 'rope_theta', 1e6))
        layers = [(bf(l.attention.k_proj.weight), bf(l.attention.k_norm.weight), bf(l.attention.v_proj.weight))
                  for l in draft.layers]
        eps = getattr(draft.context_norm, 'variance_epsilon', 1e-6)
        return DraftContextProjector(bf(draft.fc.weight), bf(draft.context_norm.weight), layers, eps=eps,
                                     theta=theta)

    # -- cache state (packed_draft.py:88-185) --------------------------------
    @property
    def lengths(self):
        return self.pool.lengths

    def add_request(self, request):
        self.pool.add_request(request)

    def validate_cache(self):
        self.pool.validate_cache()

    def request_kv(self, request):
        return self.pool.request_kv(request)

    def append_committed(self, chunks):
        self.last_projection_work = self.pool.append_committed(chunks)
        return self.last_projection_work

    def crop(self, request, length):
        self.pool.crop(request, length)

    def remove_request(self, request):
        self.pool.remove_request(request)

    # -- backbone (packed_draft.py:187-249) ------------------------------------
    @torch.no_grad()
    def backbone(self, anchors):
        """One block per active request: {request: anchor token [1, 1] long}.
        The block is the anchor and block_size - 1 MASK tokens at positions
        length .. length + block_size - 1, attending its request's whole
        committed context and its own rows."""
        if not anchors:
            raise ValueError('Require active anchor requests')
        if self.draft.training:
            raise ValueError('Packed draft is inference-only')
        self.validate_cache()
        blocks = {request: (anchor, (self.pool.length(request),)) for request, anchor in anchors.items()}
        return self._run(blocks, one_block=True)

    @torch.no_grad()
    def backbone_blocks(self, blocks):
        """One or more blocks per request: {request: (anchor tokens [1, n] long,
        n anchor positions in [0, length])}.  Block b holds its anchor token
        and MASK tokens at positions anchor_b .. anchor_b + block_size - 1 and
        sees context positions j < anchor_b plus its own rows
        (model.py:12-19, 101-119)."""
        if not blocks:
            raise ValueError('Require active anchor requests')
        return self._run(blocks, one_block=False)

    def _run(self, blocks, *, one_block):
        draft = self.draft
        if draft.training:
            raise ValueError('Packed draft is inference-only')
        self.validate_cache()
        size, vocab = self.block_size, draft.embedding.num_embeddings
        requests = tuple(blocks)
        tokens, positions, anchors = [], [], {}
        lengths = self.pool.lengths
        for request in requests:
            length = self.pool.length(request)
            anchor, where = blocks[request]
            where = tuple(int(a) for a in where)
            n = len(where)
            if (not isinstance(anchor, torch.Tensor) or anchor.shape != (1, n) or anchor.dtype != torch.long
                    or anchor.device != self.device or n < 1
                    or not bool(((anchor >= 0) & (anchor < vocab)).all())):
                raise ValueError('Require one valid [1,1] long anchor per active request' if one_block else
                                 'Require [1, n] long anchor tokens for n >= 1 blocks per request')
            if any(not 0 <= a <= length for a in where):
                raise ValueError('Every anchor must lie in [0, committed length]')
            block = anchor.new_full((n, size), self.mask_token_id)
            block[:, 0] = anchor[0]
            tokens.append(block.reshape(1, -1))
            positions.append((torch.tensor(where, device=self.device)[:, None]
                              + torch.arange(size, device=self.device)).reshape(-1))
            anchors[request] = where
        batch = self.pool.batch(anchors)
        query_positions = torch.cat(positions)
        z = draft.embedding(torch.cat(tokens, dim=1))
        cos, sin = draft.rotary(z, query_positions[None])
        nq = z.shape[1]
        autocast = torch.is_autocast_enabled(self.device.type)
        bad = torch.zeros((), dtype=torch.bool, device=self.device)
        for index, layer in enumerate(draft.layers):
            attention = layer.attention
            normalized = layer.input_norm(z)
            q = attention.q_norm(attention.q_proj(normalized).view(1, -1, attention.heads, attention.dim)).transpose(1, 2)
            q = _rotate(q, cos, sin).squeeze(0).transpose(0, 1)
            kb, vb = attention.project_kv(normalized, cos, sin)
            kb = kb.squeeze(0).transpose(0, 1)
            vb = vb.squeeze(0).transpose(0, 1)
            if not autocast and any(t.dtype != torch.bfloat16 for t in (q, kb, vb)):
                raise ValueError('Pinned varlen requires no-autograd contiguous BF16 THD tensors on its selected GPU')
            # Under autocast the kernel rounds fp32 Q/K to bf16 as it loads
            # them: the cast the reference applies at its kernel boundary
            # (packed_draft.py:229-235).  V arrives in bf16 there.
            q = (q if q.dtype == torch.float32 else q.to(torch.bfloat16)).contiguous()
            kb = kb.to(self.pool.key_dtype).contiguous()
            vb = vb.to(torch.bfloat16).contiguous()
            output = self.pool.attention(index, q, kb, vb, batch, scale=attention.dim ** -.5)
            if output.shape != (nq, attention.heads, attention.dim) or output.device != self.device:
                raise RuntimeError('Invalid packed draft attention output')
            # The reference's per-layer finiteness check (packed_draft.py:237-239),
            # kept on the device and read once after the last layer.
            bad = bad | ~torch.isfinite(output).all()
            z = z + attention.o_proj(output.reshape(1, nq, -1))
            z = z + layer.mlp(layer.post_norm(z))
        hidden = draft.norm(z).squeeze(0)
        bad_attention, bad_hidden = torch.stack((bad, ~torch.isfinite(hidden).all())).tolist()
        if bad_attention:
            raise RuntimeError('Invalid packed draft attention output')
        if bad_hidden:
            raise RuntimeError('Nonfinite packed draft hidden')
        work = self.pool.counters(batch)
        work.update(mlp_calls=len(draft.layers))
        return PackedDraftFeatures(hidden, requests, size, tuple(lengths[r] for r in requests), work,
                                   tuple(len(anchors[r]) for r in requests))
