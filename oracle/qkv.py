"""Verify-layer prologue of the target attention, restated for the CPU oracle
(test infrastructure only).

Qwen3 attention before the kernel call (transformers' Qwen3Attention as used
by dspark_qwen/persistent_qwen_target.py:45-95 and the RoPE of
dspark_qwen/model.py:22-24):
    q = RMSNorm_q(x Wq^T per 128-dim head), k = RMSNorm_k(x Wk^T), v = x Wv^T
    q, k = rope(q, pos), rope(k, pos)       (rotate-half form, theta = 1e6)
RMSNorm: y = w * x / sqrt(mean(x^2) + eps) over the head dim.
RoPE: for d < 64, with a = pos * inv_freq[d], inv_freq[d] = theta^(-2d/128):
    y[d]    = x[d] cos a - x[d+64] sin a
    y[d+64] = x[d+64] cos a + x[d] sin a
All arithmetic in float64 on inputs already rounded to their storage type.
"""
import numpy as np


def inv_freq(dim=128, theta=1e6):
    """float32 table exactly as the model computes it, 1 / theta**(2j/dim)
    with torch's float32 pow (numpy's float32 pow differs by an ulp in some
    entries, which moves angles near position 8k by ~3e-4 rad)."""
    import torch
    return (1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float) / dim))).numpy()


def rms_norm(x, w, eps):
    x = np.asarray(x, np.float64)
    return np.asarray(w, np.float64) * x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)


def rope(x, positions, freqs):
    """x [T, H, D]; positions [T]; angles formed in float32 as the model does."""
    x = np.asarray(x, np.float64)
    half = x.shape[-1] // 2
    ang = (np.asarray(positions, np.float32)[:, None] * freqs[None, :]).astype(np.float64)   # [T, D/2]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    lo, hi = x[..., :half], x[..., half:]
    return np.concatenate((lo * c - hi * s, hi * c + lo * s), axis=-1)


def qkv_prologue(x, wq, wk, wv, q_norm, k_norm, positions, *, eps=1e-6, theta=1e6, head_dim=128):
    """x [T, hidden]; w* [out, hidden] (nn.Linear layout) -> q [T, Hq, D], k, v [T, Hkv, D] (float64)."""
    x = np.asarray(x, np.float64)
    t = x.shape[0]
    freqs = inv_freq(head_dim, theta)
    q = (x @ np.asarray(wq, np.float64).T).reshape(t, -1, head_dim)
    k = (x @ np.asarray(wk, np.float64).T).reshape(t, -1, head_dim)
    v = (x @ np.asarray(wv, np.float64).T).reshape(t, -1, head_dim)
    q = rope(rms_norm(q, q_norm, eps), positions, freqs)
    k = rope(rms_norm(k, k_norm, eps), positions, freqs)
    return q, k, v
