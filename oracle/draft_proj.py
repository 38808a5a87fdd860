"""Draft context K/V projection, restated for the CPU oracle (test
infrastructure only).

DSparkDraft.project_context_kv (dspark_qwen/model.py:141-146) as driven by
PackedDraft.append_committed (dspark_qwen/packed_draft.py:147-158):
    ctx = context_norm(fc(features))                  RMSNorm over the hidden size
    per draft layer (DraftAttention.project_kv, model.py:41-45):
        k = rotate(k_norm(k_proj(ctx) per 128-dim head), cos, sin)
        v = v_proj(ctx)
rotate (model.py:22-24) is the rotate-half RoPE at each row's absolute
position (the context rows of a request are positions start .. start+n-1).
All arithmetic in float64 on inputs already rounded to their storage type;
`fc_out` optionally replaces fc(features) by a given (e.g. bf16-rounded)
fc output, the point where the draft's autocast rounds.
"""
import numpy as np

from .qkv import inv_freq, rms_norm, rope


def project_context_kv(features, fc, context_norm, layers, positions, *, eps=1e-6, theta=1e6, head_dim=128,
                       fc_out=None):
    """features [T, F]; fc [H, F]; context_norm [H]; layers: [(k_proj [Hkv*D, H],
    k_norm [D], v_proj [Hkv*D, H])]; positions [T] -> [(k [T, Hkv, D], v [T, Hkv, D])]
    in float64."""
    x = np.asarray(fc_out, np.float64) if fc_out is not None else (
        np.asarray(features, np.float64) @ np.asarray(fc, np.float64).T)
    ctx = rms_norm(x, context_norm, eps)
    t = ctx.shape[0]
    freqs = inv_freq(head_dim, theta)
    out = []
    for k_proj, k_norm, v_proj in layers:
        k = (ctx @ np.asarray(k_proj, np.float64).T).reshape(t, -1, head_dim)
        v = (ctx @ np.asarray(v_proj, np.float64).T).reshape(t, -1, head_dim)
        out.append((rope(rms_norm(k, k_norm, eps), positions, freqs), v))
    return out
