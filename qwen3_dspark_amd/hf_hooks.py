"""Hugging Face transformers adapters for the DSpark attention hot path.

* varlen_attention_forward - the attention-registry callback of
  dspark_qwen/varlen_target.py:115-129: [1,Hq,Q,D] queries, a PackedLayout
  over the model's [1,Hkv,N,D] cache, HIP gather + HIP varlen kernel,
  [1,Q,Hq,D] out.
* FusedVerificationCache + fused_verification_attention - the verification
  hooks of dspark_qwen/persistent_qwen_target.py:45-95.  The reference's
  update stages the layer and materialises the capacity-length K/V with
  prepare_attention for the kernel; here update only checks the new rows and
  the callback passes them to PersistentTargetKV.attend, whose one launch
  stages them and attends over resident + new rows in place.
* FusedVerifier - binds a PersistentTargetKV transaction to one model forward
  (the callback finds it through the `fused_verification` forward kwarg, as
  the reference passes `persistent_target`).
* PackedFeatures / CachedFeatures - the hidden states of one packed forward
  (packed_target.py:18-28, cached_target.py:15-22).  The full-model
  transaction adapter over FusedVerifier is
  persistent_target.PersistentQwenTarget (also importable from here).
* VarlenPackedTarget + PackedVarlenCache - the append-order adapter of
  dspark_qwen/varlen_target.py:132-167 over PackedTarget
  (packed_target.py:30-200): one packed forward per append over an
  AppendOrderKV, a PackedLayout per forward, the varlen callback per layer,
  and the reference's work counters.

The callbacks keep the reference's contract: no attention mask or dropout,
the module must belong to the bound model, ValueError otherwise.
"""
import contextlib
from collections.abc import Mapping
from dataclasses import dataclass

import torch
from transformers import Cache
from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

from . import backends
from ._device import upload
from .kernels import HEAD_DIM, KV_HEADS, Q_HEADS
from .layout import PackedLayout
from .packed_kv import AppendOrderKV
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
    """Cache.update for one verification transaction: check the layer's new
    K/V rows against the transaction and return them unchanged.  The
    callback hands them to the fused attention, which copies them into the
    store's scratch in the same launch that attends (and reads the committed
    rows from the resident store in place)."""

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
    out = v.store.attend(v.transaction, module.layer_idx, q, scale=scaling,
                         keys=key[0].transpose(0, 1).contiguous(), values=value[0].transpose(0, 1).contiguous())
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


# ---------------------------------------------------------------------------
# Packed forward outputs (packed_target.py:18-28)
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class CachedFeatures:
    """One request's slice of a verification forward (cached_target.py:15-22)."""
    start: int
    last: torch.Tensor
    context: torch.Tensor

    @property
    def end(self):
        return self.start + self.last.shape[1]


@dataclass(frozen=True)
class PackedFeatures:
    """Hidden states of one packed verification forward (packed_target.py:18-28):
    last [1, sum Q, hidden], context = captured layer outputs concatenated on
    the feature axis (or None), spans request -> (offset, count, start)."""
    last: torch.Tensor
    context: object
    spans: dict
    work: dict

    def for_request(self, request_id):
        offset, count, start = self.spans[request_id]
        return CachedFeatures(start, self.last[:, offset:offset + count],
                              None if self.context is None else self.context[:, offset:offset + count])


# ---------------------------------------------------------------------------
# Append-order adapter (dspark_qwen/varlen_target.py:132-167 over
# dspark_qwen/packed_target.py:30-200)
# ---------------------------------------------------------------------------

def _check_dense_qwen3(model):
    """The model checks of packed_target.py:31-40 plus the geometry and dtype
    the HIP kernels take."""
    cfg = model.config
    if (cfg.model_type != 'qwen3' or getattr(cfg, 'use_sliding_window', False)
            or any(kind != 'full_attention' for kind in cfg.layer_types)):
        raise ValueError('Only dense full-attention Qwen3 is supported')
    if (cfg.rope_parameters or {}).get('rope_type', 'default') != 'default':
        raise ValueError('Only default RoPE: dynamic scaling can couple request lengths')
    if (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim) != (Q_HEADS, KV_HEADS, HEAD_DIM):
        raise ValueError('The MI355X attention path requires 16 query heads, 8 KV heads, head dim 128')
    if model.get_input_embeddings().weight.dtype != torch.bfloat16:
        raise ValueError('The MI355X attention path requires a bf16 model')


class PackedVarlenCache(Cache):
    """HF cache over an AppendOrderKV: update() grows the layer by the
    forward's new rows (one launch) and returns the layer's whole
    [1, Hkv, N, D] K/V, from which the varlen callback gathers each
    request's rows through the forward's PackedLayout."""

    def __init__(self, target):
        super().__init__(layers=[])
        self.target = target

    @property
    def is_compileable(self):
        return False

    def update(self, key_states, value_states, layer_idx, *args, **kwargs):
        return self.target.kv.append_layer(layer_idx, key_states.contiguous(), value_states.contiguous())

    def get_seq_length(self, layer_idx=0):
        return self.target.kv.rows

    def get_mask_sizes(self, *args, **kwargs):
        raise RuntimeError('Packed varlen attention requires explicit request-local layout metadata')

    def get_max_cache_shape(self, layer_idx=0):
        return -1


class VarlenPackedTarget:
    """HF Qwen3 target over an append-order packed cache with the MI355X
    varlen kernel: the API of VarlenPackedTarget / PackedTarget
    (add_request / append / crop / remove_request / lengths / request_kv /
    predict / reset).

    append() runs one real model forward for any active subset of the
    requests.  Each layer's cache update appends the new rows in one launch;
    the attention callback gathers every active request's rows (the
    layout's gather indices) and runs the causal varlen kernel, so inactive
    requests' rows are never attended.  The work counters carry the keys of
    packed_target.py:177-188 and varlen_target.py:152-167.  A failed forward
    resets every request (the layers may have grown unevenly), as the
    reference does.
    """

    def __init__(self, model, layer_ids=(), *, native_backend=backends.TARGET_BACKEND):
        _check_dense_qwen3(model)
        cfg = model.config
        self.layer_ids = tuple(layer_ids)
        if (tuple(sorted(set(self.layer_ids))) != self.layer_ids
                or any(type(i) is not int or not 0 <= i < cfg.num_hidden_layers for i in self.layer_ids)):
            raise ValueError('layer_ids must be unique increasing decoder block indices')
        if native_backend != backends.TARGET_BACKEND:
            raise ValueError('Unknown explicit native varlen backend')
        device = model.get_input_embeddings().weight.device
        self._varlen_kernel = backends.target_kernel(native_backend, device)
        self.model = model.eval().requires_grad_(False)
        self.kv = AppendOrderKV(layers=cfg.num_hidden_layers, heads=KV_HEADS, dim=HEAD_DIM, dtype=torch.bfloat16,
                                device=device)
        self.cache = PackedVarlenCache(self)
        self._closed = False
        self._old_backend = cfg._attn_implementation
        ALL_ATTENTION_FUNCTIONS.register(VARLEN_BACKEND, varlen_attention_forward)
        cfg._attn_implementation = VARLEN_BACKEND

    def close(self):
        """Give the model its previous attention implementation back; the
        target is unusable afterwards."""
        if self.model.config._attn_implementation == VARLEN_BACKEND:
            self.model.config._attn_implementation = self._old_backend
        self.kv.reset()
        self._closed = True

    @property
    def device(self):
        return self.kv.device

    @property
    def lengths(self):
        return self.kv.lengths

    def reset(self):
        self.kv.reset()

    def add_request(self, request_id):
        self.kv.add_request(request_id)

    def crop(self, request_id, length):
        self.kv.crop(request_id, length)

    def remove_request(self, request_id):
        self.kv.remove_request(request_id)

    def request_kv(self, request_id):
        return self.kv.request_kv(request_id)

    def _validate_chunks(self, chunks):
        if not isinstance(chunks, Mapping) or not chunks:
            raise ValueError('Need a nonempty request-to-token mapping')
        for request, ids in chunks.items():
            self.kv.marker(request)
            if (not isinstance(ids, torch.Tensor) or ids.ndim != 2 or ids.shape[0] != 1
                    or ids.shape[1] < 1 or ids.dtype != torch.long or ids.device != self.device):
                raise ValueError('Each chunk needs nonempty [1,q] long IDs on the model device')
            if bool(((ids < 0) | (ids >= self.model.config.vocab_size)).any()):
                raise ValueError('Token outside vocabulary')

    def _work(self, chunks, layout, lengths):
        """The counters of packed_target.py:177-188 and varlen_target.py:152-167
        for this forward (mask extents are zero: no mask exists)."""
        cfg = self.model.config
        counts = [ids.shape[1] for ids in chunks.values()]
        starts = [lengths[r] for r in chunks]
        q, k = sum(counts), sum(lengths.values()) + sum(counts)
        causal = sum(n * c + n * (n + 1) // 2 for n, c in zip(counts, starts))
        within = sum(n * (c + n) for n, c in zip(counts, starts))
        per_token_kv_bytes = 2 * KV_HEADS * HEAD_DIM * 2
        return dict(
            queried_requests=len(chunks), resident_requests=len(lengths),
            logical_query_tokens=q, physical_query_tokens=q, physical_kv_tokens=k, physical_kv_tokens_before=k - q,
            query_lengths=counts, queried_context_lengths=starts,
            resident_context_lengths_before=list(lengths.values()),
            dense_attention_pairs_per_head_layer=q * k, allowed_causal_pairs=causal,
            masked_cross_request_pairs=q * k - within, masked_future_pairs=within - causal,
            attention_heads=cfg.num_attention_heads, layers=cfg.num_hidden_layers,
            dense_attention_pairs_all_heads_layers=q * k * cfg.num_attention_heads * cfg.num_hidden_layers,
            model_forward_calls=1,
            attention_backend=getattr(self._varlen_kernel, 'backend_name', None), mask_shape=None, mask_bytes=0,
            active_kv_gather_tokens=layout.gathered_key_tokens,
            inactive_kv_tokens_excluded=layout.physical_key_tokens - layout.gathered_key_tokens,
            kv_gather_payload_bytes_per_layer=layout.gathered_key_tokens * per_token_kv_bytes,
            varlen_pair_domain_per_head_layer=layout.pair_domain,
            varlen_cross_request_pair_domain=0,
            attention_adapter_calls_per_layer=1,
            native_varlen_calls_per_layer=getattr(self._varlen_kernel, 'native_varlen_calls_per_layer', 0),
            scope='Metadata-only varlen layout on the MI355X HIP kernels; dense Q*K counts are counterfactual '
                  'domains, no mask is built')

    @torch.no_grad()
    def append(self, chunks):
        """One packed forward over the ordered {request: ids [1, q]}; returns
        PackedFeatures (last hidden states, captured layer outputs, spans,
        work counters).  Invalid inputs fail before any mutation."""
        if self._closed:
            raise RuntimeError('Target adapter closed')
        self._validate_chunks(chunks)
        lengths = self.kv.lengths
        spans, markers, positions, offset = {}, [], [], 0
        for request, ids in chunks.items():
            count, start = ids.shape[1], lengths[request]
            spans[request] = (offset, count, start)
            markers += [self.kv.marker(request)] * count
            positions += range(start, start + count)
            offset += count
        meta = upload(self.device, markers + positions, torch.long)
        q_requests, q_positions = meta[:offset], meta[offset:]
        layout = PackedLayout.from_metadata(q_requests, q_positions, torch.cat((self.kv.key_requests, q_requests)),
                                            torch.cat((self.kv.key_positions, q_positions)))
        work = self._work(chunks, layout, lengths)
        captured, hooks = {}, []

        def hook_for(index):
            def hook(_module, _inputs, output):
                captured[index] = output[0] if isinstance(output, tuple) else output
            return hook
        try:
            for index in self.layer_ids:
                hooks.append(self.model.model.layers[index].register_forward_hook(hook_for(index)))
            output = self.model.model(input_ids=torch.cat(tuple(chunks.values()), dim=1),
                                      position_ids=q_positions[None], attention_mask={'full_attention': None},
                                      past_key_values=self.cache, use_cache=True, return_dict=True,
                                      packed_layout=layout, packed_varlen_kernel=self._varlen_kernel)
            self.kv.commit_rows({r: ids.shape[1] for r, ids in chunks.items()})
        except Exception:
            self.kv.reset()
            raise
        finally:
            for hook in hooks:
                hook.remove()
        context = torch.cat([captured[i] for i in self.layer_ids], dim=-1) if self.layer_ids else None
        return PackedFeatures(output.last_hidden_state.detach(), None if context is None else context.detach(),
                              spans, work)

    @torch.no_grad()
    def predict(self, features, last_only=False):
        """The model's LM head over the physical query rows, split by request
        span (packed_target.py:216-224)."""
        logits = self.model.get_output_embeddings()(features.last)
        return {r: (logits[:, offset + count - 1] if last_only else logits[:, offset:offset + count])
                for r, (offset, count, _) in features.spans.items()}


def __getattr__(name):
    # The full-model adapter lives in persistent_target (which imports this
    # module); resolve its names here lazily.
    if name in ('PersistentQwenTarget', 'FullModelGraph', 'GraphTicket', 'GraphCompletion'):
        from . import persistent_target
        return getattr(persistent_target, name)
    if name == 'GRAPH_BACKEND':
        from .graph import TorchGraphBackend
        return TorchGraphBackend.kind
    raise AttributeError(name)
