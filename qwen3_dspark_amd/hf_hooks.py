"""Hugging Face transformers adapters for the DSpark attention hot path.

* varlen_attention_forward - the attention-registry callback of
  dspark_qwen/varlen_target.py:115-129: [1,Hq,Q,D] queries, a PackedLayout
  over the model's [1,Hkv,N,D] cache, HIP gather + HIP varlen kernel,
  [1,Q,Hq,D] out.
* FusedVerificationCache + fused_verification_attention - the verification
  hooks of dspark_qwen/persistent_qwen_target.py:45-95 (Cache.update stages
  the layer, the callback attends).  The reference's update materialises the
  capacity-length K/V with prepare_attention and hands it to the kernel; here
  update only stages the new rows and the callback calls
  PersistentTargetKV.attend, which reads resident + scratch rows in place.
* FusedVerifier - binds a PersistentTargetKV transaction to one model forward
  (the callback finds it through the `fused_verification` forward kwarg, as
  the reference passes `persistent_target`).

The callbacks keep the reference's contract: no attention mask or dropout,
the module must belong to the bound model, ValueError otherwise.
"""
import contextlib

import torch
from transformers import Cache
from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

from .layout import PackedLayout
from .persistent_kv import PersistentTargetKV

VARLEN_BACKEND = 'dspark_mi355x_varlen'
FUSED_BACKEND = 'dspark_mi355x_fused_verify'


def varlen_attention_forward(module, query, key, value, attention_mask, scaling=None, dropout=0.0,
                             packed_layout=None, packed_varlen_kernel=None, **kwargs):
    """Registry callback with the contract of varlen_target.py:115-129."""
    if attention_mask is not None or dropout:
        raise ValueError('Varlen callback requires metadata-only causal attention without dropout')
    if not isinstance(packed_layout, PackedLayout) or packed_varlen_kernel is None:
        raise ValueError('Missing explicit packed layout/kernel')
    if query.ndim != 4 or query.shape[0] != 1 or query.shape[2] != packed_layout.query_tokens:
        raise ValueError('Expected [1,Hq,Q,D] query with layout Q')
    q = query.squeeze(0).transpose(0, 1).contiguous()
    k, v = packed_layout.gather_kv(key, value)
    out = packed_varlen_kernel(q, k, v, packed_layout, scale=scaling)
    if not isinstance(out, torch.Tensor) or out.shape != q.shape or out.dtype != q.dtype or out.device != q.device:
        raise RuntimeError('Varlen kernel returned an incompatible output')
    return out[None], None


class FusedVerificationCache(Cache):
    """Cache.update for one verification transaction: stage the layer's new
    K/V rows into the store's scratch and return them unchanged (the fused
    attention reads the committed rows from the resident store itself)."""

    def __init__(self, verifier):
        super().__init__(layers=[])
        self.verifier = verifier

    @property
    def is_compileable(self):
        return False

    def update(self, key_states, value_states, layer_idx, *args, **kwargs):
        v = self.verifier
        tx = v.transaction
        if tx is None:
            raise RuntimeError('Cache update outside owned transaction')
        q = sum(tx.query_lengths)
        expected = (1, v.store.heads, q, v.store.dim)
        if tuple(key_states.shape) != expected or value_states.shape != key_states.shape:
            raise ValueError('HF layer KV differs from exact packed query shape')
        v.store.stage_layer(tx, layer_idx, key_states[0].transpose(0, 1).contiguous(),
                            value_states[0].transpose(0, 1).contiguous())
        return key_states, value_states

    def get_seq_length(self, layer_idx=0):
        return sum(self.verifier.store.length(h) for h in self.verifier.handles)

    def get_mask_sizes(self, *args, **kwargs):
        raise RuntimeError('Fused verification requires explicit request-local attention metadata')

    def get_max_cache_shape(self, layer_idx=0):
        return self.verifier.store.slot_capacity * self.verifier.store.context_capacity


def fused_verification_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0,
                                 fused_verification=None, **kwargs):
    """Registry callback of persistent_qwen_target.py:45-60 on the fused path."""
    v = fused_verification
    if not isinstance(v, FusedVerifier) or v.transaction is None:
        raise ValueError('Owned persistent verification transaction required')
    if attention_mask is not None or dropout or v.attention_module(module.layer_idx) is not module:
        raise ValueError('Unexpected mask/dropout/foreign model attention')
    q = query[0].transpose(0, 1).contiguous()
    out = v.store.attend(v.transaction, module.layer_idx, q, scale=scaling)
    if not isinstance(out, torch.Tensor) or out.shape != q.shape or out.dtype != q.dtype or out.device != q.device:
        raise ValueError('Persistent attention returned incompatible output')
    return out[None], None


class FusedVerifier:
    """One HF Qwen3 model over a PersistentTargetKV: registers the fused
    callback, owns the verification cache and binds a transaction to each
    forward.

        verifier = FusedVerifier(model, store)
        with verifier.transaction_for(handles, bucket) as tx:
            logits = verifier.forward(input_ids, position_ids)
        store.commit(tx, accepted)          # or store.abort(tx)
    """

    def __init__(self, model, store):
        if not isinstance(store, PersistentTargetKV):
            raise ValueError('PersistentTargetKV store required')
        cfg = model.config
        if (cfg.num_hidden_layers != store.layers or cfg.num_key_value_heads != store.heads
                or cfg.head_dim != store.dim):
            raise ValueError('Model attention geometry differs from the store')
        self.model = model.eval().requires_grad_(False)
        self.store = store
        self.cache = FusedVerificationCache(self)
        self.transaction = None
        self.handles = ()
        ALL_ATTENTION_FUNCTIONS.register(FUSED_BACKEND, fused_verification_attention)
        cfg._attn_implementation = FUSED_BACKEND

    def attention_module(self, layer_idx):
        return self.model.model.layers[layer_idx].self_attn

    @contextlib.contextmanager
    def transaction_for(self, handles, bucket, *, query_lengths=None):
        if self.transaction is not None:
            raise RuntimeError('Finish existing verification transaction first')
        tx = self.store.begin(handles, bucket, query_lengths=query_lengths)
        self.transaction, self.handles = tx, tuple(handles)
        try:
            yield tx
        finally:
            self.transaction = None

    @torch.no_grad()
    def forward(self, input_ids, position_ids):
        """Packed verification forward: input_ids/position_ids [1, sum Q]
        (request-local absolute positions); returns the model output."""
        if self.transaction is None:
            raise RuntimeError('Forward outside owned transaction')
        return self.model(input_ids=input_ids, position_ids=position_ids, attention_mask=None,
                          past_key_values=self.cache, use_cache=True, fused_verification=self)
