"""Verify-layer prologue on MI355X: the Qwen3 attention steps that produce
the attention kernel's inputs (transformers' Qwen3Attention as driven by
dspark_qwen/persistent_qwen_target.py:45-95, RoPE as dspark_qwen/model.py:22-24):

    q = RoPE(RMSNorm_q(x Wq^T)),  k = RoPE(RMSNorm_k(x Wk^T)),  v = x Wv^T

in one HIP launch per layer (dspark_qkv_prologue).  K/V can be written
straight into a PersistentTargetKV transaction's scratch
(PersistentTargetKV.stage_projected), which replaces stage_layer's copy.
The rows' rotary cos/sin can be computed once (QKVPrologue.rope_table) and
shared by every layer, as the model computes its position embeddings once
per forward; the prologue then gives the same bits without its per-layer
sincos.
"""
import torch

from . import _native
from ._device import require_gfx950
from .kernels import HEAD_DIM, KV_HEADS, Q_HEADS


def rope_inv_freq(theta=1e6, dim=HEAD_DIM):
    """The model's float32 inverse frequencies, 1 / theta**(2j/dim), computed
    with torch's float32 pow exactly as transformers' default RoPE does."""
    return 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float) / dim))


class QKVPrologue:
    """One layer's projection weights in nn.Linear layout: q_proj [16*128, H],
    k_proj / v_proj [8*128, H], q_norm / k_norm [128]; bf16 on a gfx950 GPU."""

    def __init__(self, q_proj, k_proj, v_proj, q_norm, k_norm, *, eps=1e-6, theta=1e6):
        self.device = require_gfx950(q_proj.device)
        _native.load()
        hidden = q_proj.shape[-1] if q_proj.ndim == 2 else 0
        shapes = ((q_proj, (Q_HEADS * HEAD_DIM, hidden)), (k_proj, (KV_HEADS * HEAD_DIM, hidden)),
                  (v_proj, (KV_HEADS * HEAD_DIM, hidden)), (q_norm, (HEAD_DIM,)), (k_norm, (HEAD_DIM,)))
        for t, shape in shapes:
            if (not isinstance(t, torch.Tensor) or t.dtype != torch.bfloat16 or t.device != self.device
                    or tuple(t.shape) != shape):
                raise ValueError('Prologue weights must be bf16 q/k/v projections [Hq*128|Hkv*128, H] and '
                                 '[128] norms on one gfx950 device')
        if hidden < 128 or hidden % 128:
            raise ValueError('Hidden size must be a positive multiple of 128')
        if not (eps > 0 and theta > 0):
            raise ValueError('eps and theta must be positive')
        self.hidden = hidden
        self.eps = float(eps)
        self.theta = float(theta)
        self.weights = tuple(t.detach().contiguous() for t in (q_proj, k_proj, v_proj, q_norm, k_norm))
        self.inv_freq = rope_inv_freq(theta).to(self.device)

    @classmethod
    def from_attention(cls, attn, *, theta=None):
        """From a transformers Qwen3Attention module (its weights are used in
        place when already bf16 and contiguous)."""
        cfg = attn.config
        theta = theta if theta is not None else (cfg.rope_parameters or {}).get('rope_theta', 1e6)
        return cls(attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight, attn.q_norm.weight,
                   attn.k_norm.weight, eps=cfg.rms_norm_eps, theta=theta)

    def _positions(self, positions, t):
        if (not isinstance(positions, torch.Tensor) or positions.dtype != torch.long or positions.shape != (t,)
                or positions.device != self.device or not positions.is_contiguous()):
            raise ValueError('Positions must be a contiguous int64 [T] device tensor')

    def rope_table(self, positions):
        """The rows' rotary table [T, 128] float32: cos(positions[t] *
        inv_freq[d]) for d < 64, then the sines (one dspark_rope_table
        launch).  Valid for every prologue of the same theta on these
        positions."""
        t = positions.shape[0] if isinstance(positions, torch.Tensor) and positions.ndim == 1 else 0
        if t < 1:
            raise ValueError('Positions must be a contiguous int64 [T] device tensor')
        self._positions(positions, t)
        table = torch.empty((t, HEAD_DIM), dtype=torch.float32, device=self.device)
        _native.call('dspark_rope_table', self.inv_freq.data_ptr(), positions.data_ptr(), t, table.data_ptr(),
                     _native.stream_handle(self.device))
        return table

    def __call__(self, hidden, positions, *, k_out=None, v_out=None, rope=None):
        """hidden [T, H] bf16, positions [T] int64 (device) -> (q [T,16,128],
        k, v [T,8,128]).  k_out/v_out: optional destinations whose token rows
        are 8*128 elements apart (e.g. a scratch layer); they are returned.
        rope: optional rope_table(positions) of a prologue with this theta."""
        t = hidden.shape[0] if isinstance(hidden, torch.Tensor) and hidden.ndim == 2 else 0
        if (t < 1 or hidden.shape[1] != self.hidden or hidden.dtype != torch.bfloat16
                or hidden.device != self.device or not hidden.is_contiguous()):
            raise ValueError('Hidden states must be contiguous bf16 [T, hidden] on the prologue device')
        self._positions(positions, t)
        if rope is not None and (not isinstance(rope, torch.Tensor) or rope.dtype != torch.float32
                                 or tuple(rope.shape) != (t, HEAD_DIM) or rope.device != self.device
                                 or not rope.is_contiguous()):
            raise ValueError('Rotary table must be a contiguous float32 [T, 128] device tensor (rope_table)')
        q = torch.empty((t, Q_HEADS, HEAD_DIM), dtype=torch.bfloat16, device=self.device)
        outs = []
        for o in (k_out, v_out):
            if o is None:
                o = torch.empty((t, KV_HEADS, HEAD_DIM), dtype=torch.bfloat16, device=self.device)
            elif (o.dtype != torch.bfloat16 or o.device != self.device or o.shape[0] < t
                  or tuple(o.shape[1:]) != (KV_HEADS, HEAD_DIM) or o.stride(0) != KV_HEADS * HEAD_DIM
                  or o.stride(2) != 1 or o.stride(1) != HEAD_DIM):
                raise ValueError('K/V destinations must be bf16 [>=T, 8, 128] token-major on the device')
            outs.append(o)
        wq, wk, wv, qn, kn = self.weights
        _native.call('dspark_qkv_prologue', hidden.data_ptr(), wq.data_ptr(), wk.data_ptr(), wv.data_ptr(),
                     qn.data_ptr(), kn.data_ptr(), self.inv_freq.data_ptr(), positions.data_ptr(),
                     rope.data_ptr() if rope is not None else None, t, self.hidden, self.eps, q.data_ptr(),
                     outs[0].data_ptr(), outs[1].data_ptr(), KV_HEADS * HEAD_DIM, _native.stream_handle(self.device))
        return q, outs[0], outs[1]
