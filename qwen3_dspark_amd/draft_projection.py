"""Draft context projection on MI355X: DSparkDraft.project_context_kv
(dspark_qwen/model.py:141-146) for the rows PackedDraft.append_committed
adds (dspark_qwen/packed_draft.py:130-168), written straight into the slotted
draft pool.

    ctx = context_norm(fc(features))                     [T, hidden]
    k_l = rotate(k_norm_l(k_proj_l(ctx)), cos, sin),  v_l = v_proj_l(ctx)

Two launches for all draft layers and requests:
  * fc, a plain [T, 5*hidden] x [5*hidden, hidden] GEMM, on hipBLASLt
    (torch's bf16 linear, the same rounding point as the draft's autocast);
  * dspark_draft_kv_project: the context norm (its weight folded into the
    projection weights once, its per-token factor applied to the FP32
    result), every layer's k_proj / k_norm / RoPE and v_proj, and the store
    into each request's pool slot at its absolute positions, with a device
    finiteness flag.
From GEMM_MIN_TOKENS appended tokens on, the k/v projection itself is a
plain GEMM that hipBLASLt runs faster than the fused tiles: it then runs as
one library GEMM per GEMM_CHUNK tokens (all layers' folded weights as one
matrix, bf16 operands, FP32 output) followed by dspark_draft_kv_epilogue
(norm factor, k_norm, RoPE, pool store, flag).  Both paths keep the
projection in FP32 through the norms and RoPE and round every output to
bf16 once, so the path a given append length takes changes only the
accumulation order.
"""
import torch

from . import _native
from .kernels import HEAD_DIM, KV_HEADS
from .prologue import rope_inv_freq


GEMM_MIN_TOKENS = 2048   # appends at least this long take the GEMM + epilogue path
GEMM_CHUNK = 16384       # tokens per library GEMM (bounds its FP32 output: 640 MiB at 5 layers)
PATHS = ('fused', 'gemm')


class DraftContextProjector:
    """Weights of the draft's context path, bf16 on one gfx950 device:
    fc [hidden, F] (nn.Linear layout), context_norm [hidden] and per draft
    layer (k_proj [8*128, hidden], k_norm [128], v_proj [8*128, hidden]).
    The weights are snapshotted: the context norm weight is folded into
    copies of k_proj / v_proj (k_proj diag(w_c), formed in FP32, rounded to
    bf16 once)."""

    def __init__(self, fc, context_norm, layers, *, eps=1e-6, theta=1e6):
        from ._device import require_gfx950
        self.device = require_gfx950(fc.device if isinstance(fc, torch.Tensor) else 'cuda')
        _native.load()
        if not isinstance(fc, torch.Tensor) or fc.ndim != 2:
            raise ValueError('fc must be a [hidden, features] weight')
        hidden, features = fc.shape
        layers = list(layers)
        checks = [(fc, (hidden, features)), (context_norm, (hidden,))]
        for kp, kn, vp in layers:
            checks += [(kp, (KV_HEADS * HEAD_DIM, hidden)), (kn, (HEAD_DIM,)), (vp, (KV_HEADS * HEAD_DIM, hidden))]
        for t, shape in checks:
            if (not isinstance(t, torch.Tensor) or t.dtype != torch.bfloat16 or t.device != self.device
                    or tuple(t.shape) != shape):
                raise ValueError('Draft projection weights must be bf16 fc [hidden, F], context_norm [hidden], '
                                 'k_proj/v_proj [8*128, hidden] and k_norm [128] on one gfx950 device')
        if not 1 <= len(layers) <= 64:
            raise ValueError('Between 1 and 64 draft layers')
        if hidden < 128 or hidden % 128:
            raise ValueError('Hidden size must be a positive multiple of 128')
        if not (eps > 0 and theta > 0):
            raise ValueError('eps and theta must be positive')
        self.hidden, self.features, self.layers = hidden, features, len(layers)
        self.eps = float(eps)
        self.fc = fc.detach().contiguous()
        wc = context_norm.detach().float()
        folded = [torch.stack((kp.detach().float() * wc, vp.detach().float() * wc)) for kp, _, vp in layers]
        self.w = torch.stack(folded).to(torch.bfloat16).contiguous()          # [layers, 2, 1024, hidden]
        # The GEMM path's right operand, stored transposed once: [hidden, layers*2*1024].
        self.w_t = self.w.view(-1, self.w.shape[-1]).t().contiguous()
        self.k_norm = torch.stack([kn.detach() for _, kn, _ in layers]).contiguous()   # [layers, 128]
        self.inv_freq = rope_inv_freq(theta).to(self.device)

    @classmethod
    def from_draft(cls, draft, *, theta=None):
        """From a DSparkDraft-shaped module (fc, context_norm, layers[i].attention
        with k_proj / k_norm / v_proj, rotary); bf16 weights are used as the
        snapshot source."""
        if theta is None:
            cfg = getattr(getattr(draft, 'rotary', None), 'config', None)
            params = getattr(cfg, 'rope_parameters', None) or {}
            theta = params.get('rope_theta', getattr(cfg, 'rope_theta', 1e6))
        layers = [(l.attention.k_proj.weight, l.attention.k_norm.weight, l.attention.v_proj.weight)
                  for l in draft.layers]
        eps = getattr(draft.context_norm, 'variance_epsilon', 1e-6)
        return cls(draft.fc.weight, draft.context_norm.weight, layers, eps=eps, theta=theta)

    def fc_forward(self, features):
        """fc over the concatenated features [T, F] -> [T, hidden] bf16."""
        return torch.nn.functional.linear(features, self.fc)

    def project_into(self, fc_out, records, n_req, keys, values, *, flag=None, path=None):
        """The projection of fc_out [T, hidden] into pool tensors keys /
        values [layers, slots, 8, capacity, 128] (bf16); records: int32 device
        tensor of n_req (slot, first position, first token, count) rows.
        path: 'fused', 'gemm' or None (by length: GEMM_MIN_TOKENS)."""
        if path is not None and path not in PATHS:
            raise ValueError(f'path must be one of {PATHS} or None')
        t = fc_out.shape[0]
        s = keys.stride()
        stream = _native.stream_handle(self.device)
        flag_ptr = None if flag is None else flag.data_ptr()
        if (path or ('gemm' if t >= GEMM_MIN_TOKENS else 'fused')) == 'fused':
            _native.call('dspark_draft_kv_project', fc_out.data_ptr(), t, self.hidden, self.w.data_ptr(),
                         self.k_norm.data_ptr(), self.layers, self.inv_freq.data_ptr(), records.data_ptr(), n_req,
                         self.eps, self.eps, keys.data_ptr(), values.data_ptr(), s[0], s[1], s[2], flag_ptr, stream)
            return
        for c0 in range(0, t, GEMM_CHUNK):
            x = fc_out[c0:c0 + GEMM_CHUNK]
            y = torch.mm(x, self.w_t, out_dtype=torch.float32)   # hipBLASLt, [rows, layers*2*1024] FP32
            _native.call('dspark_draft_kv_epilogue', y.data_ptr(), 1, y.stride(0), x.data_ptr(), x.shape[0], c0,
                         self.hidden, self.k_norm.data_ptr(), self.layers, self.inv_freq.data_ptr(),
                         records.data_ptr(), n_req, self.eps, self.eps, keys.data_ptr(), values.data_ptr(), s[0],
                         s[1], s[2], flag_ptr, stream)
