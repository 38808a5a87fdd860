"""The DSpark draft backbone over cached context, restated for the CPU oracle
(test infrastructure only).

DSparkDraft.backbone (dspark_qwen/model.py:101-119) for ONE request, with
its context K/V already projected (as PackedDraft.backbone reads them from
its cache, dspark_qwen/packed_draft.py:205-245):
  * block b is the anchor token and block_size - 1 MASK tokens at positions
    anchor_b .. anchor_b + block_size - 1; it sees context positions
    j < anchor_b and its own rows (block_mask, model.py:12-19);
  * each draft layer (DraftBlock, model.py:63-73; DraftAttention,
    model.py:47-61):
        x  = RMSNorm_in(z)
        q  = rope(RMSNorm_q(x Wq^T per head)),  k = rope(RMSNorm_k(x Wk^T)),  v = x Wv^T
        z += attention(q, [ctx_k; k], [ctx_v; v]) Wo^T
        z += mlp(RMSNorm_post(z)),   mlp(y) = (silu(y Wg^T) * (y Wu^T)) Wd^T  (Qwen3MLP)
  * hidden = RMSNorm_final(z).
All arithmetic in float64 on inputs already rounded to their storage type.
"""
import numpy as np

from .attention import draft_attention
from .qkv import inv_freq, rms_norm, rope


def mlp(y, gate, up, down):
    """Qwen3MLP with SiLU: down(silu(gate(y)) * up(y)) (nn.Linear layouts)."""
    y = np.asarray(y, np.float64)
    g = y @ np.asarray(gate, np.float64).T
    u = y @ np.asarray(up, np.float64).T
    return ((g / (1.0 + np.exp(-g))) * u) @ np.asarray(down, np.float64).T


def draft_layer(z, layer, context_k, context_v, anchors, *, eps=1e-6, theta=1e6, head_dim=128, block_size=7):
    """One DraftBlock over the block rows z [n*7, hidden].  layer: dict with
    input_norm, q_proj, k_proj, v_proj, o_proj, q_norm, k_norm, post_norm,
    gate, up, down; context_k/v [c, Hkv, D] (projected, RoPE'd K)."""
    z = np.asarray(z, np.float64)
    t = z.shape[0]
    positions = (np.asarray(anchors)[:, None] + np.arange(block_size)).reshape(-1)
    freqs = inv_freq(head_dim, theta)
    x = rms_norm(z, layer['input_norm'], eps)
    q = (x @ np.asarray(layer['q_proj'], np.float64).T).reshape(t, -1, head_dim)
    k = (x @ np.asarray(layer['k_proj'], np.float64).T).reshape(t, -1, head_dim)
    v = (x @ np.asarray(layer['v_proj'], np.float64).T).reshape(t, -1, head_dim)
    q = rope(rms_norm(q, layer['q_norm'], eps), positions, freqs)
    k = rope(rms_norm(k, layer['k_norm'], eps), positions, freqs)
    o = draft_attention(q, np.asarray(context_k, np.float64), np.asarray(context_v, np.float64), k, v,
                        list(anchors), scale=head_dim ** -0.5, block_size=block_size)
    z = z + o.reshape(t, -1) @ np.asarray(layer['o_proj'], np.float64).T
    return z + mlp(rms_norm(z, layer['post_norm'], eps), layer['gate'], layer['up'], layer['down'])


def draft_backbone(z, layers, context_kv, anchors, final_norm, *, eps=1e-6, theta=1e6, head_dim=128,
                   block_size=7):
    """Draft hidden rows [n*7, hidden] of one request: z the block tokens'
    embeddings, context_kv [(k [c, Hkv, D], v)] per layer."""
    for layer, (ck, cv) in zip(layers, context_kv):
        z = draft_layer(z, layer, ck, cv, anchors, eps=eps, theta=theta, head_dim=head_dim, block_size=block_size)
    return rms_norm(z, final_norm, eps)
