"""Float64 numpy attention for the CPU oracle (test infrastructure only).

GQA: query head h uses KV head h // (Hq // Hkv) (dspark_qwen/model.py:58-59;
SDPA enable_gqa).  Inputs are float arrays already rounded to the storage
precision by the caller; all arithmetic here is float64.
"""
import numpy as np


def _attend(q, k, v, visible, scale):
    """q [nq,Hq,D], k/v [nk,Hkv,D], visible [nq,nk] bool -> [nq,Hq,D]."""
    hq, hkv = q.shape[1], k.shape[1]
    g = hq // hkv
    q = q.astype(np.float64)
    k = np.repeat(k.astype(np.float64), g, axis=1)
    v = np.repeat(v.astype(np.float64), g, axis=1)
    s = np.einsum('qhd,khd->hqk', q, k) * scale
    s = np.where(visible[None], s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    p = np.exp(s - m)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.einsum('hqk,khd->qhd', p, v)


def varlen_attention(q, k, v, cu_query, cu_key, *, causal, scale):
    """Per-request packed attention.

    causal=True : bottom-right, query i of (q,k) sees keys j <= k-q+i
                  (dspark_qwen/varlen_target.py:98-112,
                   dspark_qwen/persistent_qwen_target.py:30-42)
    causal=False: all keys of the request (dspark_qwen/packed_draft.py:35-47)
    Rows past cu_key[-1] (capacity tail) are never read.
    """
    out = np.zeros(q.shape, np.float64)
    for r in range(len(cu_query) - 1):
        qs, qe, ks, ke = cu_query[r], cu_query[r + 1], cu_key[r], cu_key[r + 1]
        nq, nk = qe - qs, ke - ks
        if causal:
            visible = np.arange(nk)[None, :] <= np.arange(nk - nq, nk)[:, None]
        else:
            visible = np.ones((nq, nk), bool)
        out[qs:qe] = _attend(q[qs:qe], k[ks:ke], v[ks:ke], visible, scale)
    return out


def verify_attention(q, resident_k, resident_v, scratch_k, scratch_v, slots, contexts, queries, *, scale):
    """Verification attention of one layer: request r's keys are its
    committed rows resident[slot_r, :c_r] followed by its staged rows
    scratch[qo_r : qo_r+q_r] (dspark_qwen/persistent_target_kv.py:392-460),
    bottom-right causal."""
    out = np.zeros(q.shape, np.float64)
    qo = 0
    for s, c, n in zip(slots, contexts, queries):
        k = np.concatenate((resident_k[s, :c], scratch_k[qo:qo + n]))
        v = np.concatenate((resident_v[s, :c], scratch_v[qo:qo + n]))
        visible = np.arange(c + n)[None, :] <= np.arange(c, c + n)[:, None]
        out[qo:qo + n] = _attend(q[qo:qo + n], k, v, visible, scale)
        qo += n
    return out


def draft_attention(q, context_k, context_v, block_k, block_v, anchors, *, scale, block_size=7):
    """Multi-block draft attention for ONE request (dspark_qwen/model.py:12-19,
    47-61): q [n*7,Hq,D], context_k/v [c,Hkv,D], block_k/v [n*7,Hkv,D];
    block b sees context j < anchors[b] and its own 7 rows."""
    n = len(anchors)
    c = context_k.shape[0]
    k = np.concatenate((context_k, block_k))
    v = np.concatenate((context_v, block_v))
    visible = np.zeros((n * block_size, c + n * block_size), bool)
    for b, a in enumerate(anchors):
        rows = slice(b * block_size, (b + 1) * block_size)
        visible[rows, :a] = True
        visible[rows, c + b * block_size:c + (b + 1) * block_size] = True
    return _attend(q, k, v, visible, scale)
