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
* PersistentQwenTarget - the full-model transaction adapter of
  dspark_qwen/persistent_qwen_target.py:100-472 (verify / commit / abort /
  prefill / predict / request_kv, captured layer features) on that path.
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
from .kernels import HEAD_DIM, KV_HEADS, Q_HEADS, HipCapacityKernel
from .layout import PackedLayout
from .packed_kv import AppendOrderKV
from .persistent_kv import Bucket, PersistentTargetKV, QueryFamily
from .schedule import DEFAULT_CHUNK

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


# ---------------------------------------------------------------------------
# Full-model transaction adapter (dspark_qwen/persistent_qwen_target.py:100-472)
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


class PersistentQwenTarget:
    """HF Qwen3 target over a PersistentTargetKV with the fused MI355X
    attention (the API of persistent_qwen_target.py:100-472, eager path).

    verify() runs one packed forward whose layers stage their new K/V rows
    into scratch and attend over resident + scratch rows in place; nothing is
    committed until commit() keeps the caller's accepted prefixes (the rest
    is rolled back by omission).  prefill() = verify + commit of every row.
    Decoder outputs of `layer_ids` are captured as draft context features.
    """
    BACKEND_NAME = FUSED_BACKEND

    def __init__(self, model, layer_ids=(), *, slots, context_capacity, max_query_tokens, chunk=DEFAULT_CHUNK):
        cfg = model.config
        if (cfg.model_type != 'qwen3' or getattr(cfg, 'use_sliding_window', False)
                or any(kind != 'full_attention' for kind in cfg.layer_types)
                or (cfg.rope_parameters or {}).get('rope_type', 'default') != 'default'):
            raise ValueError('Owned dense Qwen3 with default RoPE required')
        if (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim) != (16, 8, 128):
            raise ValueError('The MI355X attention path requires 16 query heads, 8 KV heads, head dim 128')
        self.layer_ids = tuple(layer_ids)
        if (tuple(sorted(set(self.layer_ids))) != self.layer_ids
                or any(type(i) is not int or not 0 <= i < cfg.num_hidden_layers for i in self.layer_ids)):
            raise ValueError('Unique increasing valid decoder layer IDs required')
        device = model.get_input_embeddings().weight.device
        dtype = model.get_input_embeddings().weight.dtype
        if dtype != torch.bfloat16:
            raise ValueError('The MI355X attention path requires a bf16 model')
        self.store = PersistentTargetKV(layers=cfg.num_hidden_layers, slots=slots, context_capacity=context_capacity,
                                        max_query_tokens=max_query_tokens, heads=cfg.num_key_value_heads,
                                        dim=cfg.head_dim, dtype=dtype, device=device, chunk=chunk)
        self.verifier = FusedVerifier(model, self.store)
        self.model = self.verifier.model
        # The kernel identity the reference's session guard reads
        # (packed_sampling.py:110-115): the capacity-tail drop-in of
        # _native_attention.  verify() itself runs the fused store attention.
        self._varlen_kernel = HipCapacityKernel(device)
        self._handles = {}
        self._pending = None
        self._captured = {}
        self._hooks = [self.model.model.layers[i].register_forward_hook(self._hook(i)) for i in self.layer_ids]

    @property
    def device(self):
        return self.store.device

    @property
    def lengths(self):
        return {r: self.store.length(h) for r, h in self._handles.items()}

    def _hook(self, index):
        def capture(_module, _inputs, output):
            if self.verifier.transaction is None:
                raise RuntimeError('Foreign model forward while the adapter owns the model')
            self._captured[index] = output[0] if isinstance(output, tuple) else output
        return capture

    def add_request(self, request):
        self._idle()
        self._handles[request] = self.store.add_request(request)

    def remove_request(self, request):
        self._idle()
        self.store.remove_request(self._handles.pop(request))

    def register_bucket(self, bucket):
        self._idle()
        self.store.register_bucket(bucket)

    def _idle(self):
        if self._pending is not None:
            raise RuntimeError('Finish existing verification transaction first')

    def _validate_chunks(self, chunks, bucket):
        if not isinstance(chunks, Mapping) or not chunks:
            raise ValueError('Need a nonempty request-to-token mapping')
        if not isinstance(bucket, (Bucket, QueryFamily)):
            raise ValueError('Explicit Bucket or QueryFamily required')
        for request, ids in chunks.items():
            if request not in self._handles:
                raise ValueError('Unknown request ID')
            if (not isinstance(ids, torch.Tensor) or ids.ndim != 2 or ids.shape[0] != 1 or ids.shape[1] < 1
                    or ids.dtype != torch.long or ids.device != self.device):
                raise ValueError('Each chunk needs nonempty [1,q] long IDs on the model device')

    @torch.no_grad()
    def verify(self, chunks, *, bucket):
        """One packed forward over {request: ids [1, q]} in bucket order;
        returns PackedFeatures and leaves the transaction open."""
        self._idle()
        self._validate_chunks(chunks, bucket)
        handles = tuple(self._handles[r] for r in chunks)
        query_lengths = tuple(ids.shape[1] for ids in chunks.values())
        self._captured = {}
        with self.verifier.transaction_for(handles, bucket, query_lengths=query_lengths) as tx:
            ws = self.store.workspace(tx.bucket)
            try:
                out = self.model.model(input_ids=torch.cat(tuple(chunks.values()), dim=1),
                                       position_ids=ws.positions[None], attention_mask=None,
                                       past_key_values=self.verifier.cache, use_cache=True, return_dict=True,
                                       fused_verification=self.verifier)
                if self.store.staged_layers() != self.store.layers or set(self._captured) != set(self.layer_ids):
                    raise RuntimeError('Full layer cache update or selected feature capture missing')
            except BaseException:
                if self.store.open_transaction is tx and not self.store.failed:
                    self.store.abort(tx)
                raise
            finally:
                captured, self._captured = self._captured, {}
        spans, offset = {}, 0
        for request, c, q in zip(chunks, tx.context_lengths, tx.query_lengths):
            spans[request] = (offset, q, c)
            offset += q
        context = torch.cat([captured[i] for i in self.layer_ids], dim=-1) if self.layer_ids else None
        work = self.store.work(tx)
        work.update(model_forward_calls=1, layers=self.store.layers, selected_layer_ids=list(self.layer_ids),
                    attention_backend=self.BACKEND_NAME,
                    committed_write_policy='scratch_only_until_explicit_commit')
        features = PackedFeatures(out.last_hidden_state.detach(), None if context is None else context.detach(),
                                  spans, work)
        self._pending = (features, tx)
        return features

    @torch.no_grad()
    def commit(self, features, committed_query_lengths):
        if self._pending is None or self._pending[0] is not features:
            raise ValueError('Only the outstanding verification features can commit')
        if not isinstance(committed_query_lengths, Mapping) or set(committed_query_lengths) != set(features.spans):
            raise ValueError('One committed query prefix per verified request required')
        _, tx = self._pending
        result = self.store.commit(tx, {self._handles[r]: n for r, n in committed_query_lengths.items()})
        self._pending = None
        return result

    def abort(self, features):
        if self._pending is None or self._pending[0] is not features:
            raise ValueError('Only outstanding verification features can abort')
        self.store.abort(self._pending[1])
        self._pending = None

    @torch.no_grad()
    def prefill(self, chunks, *, bucket):
        self._idle()
        if any(self.lengths.get(r) != 0 for r in chunks):
            raise ValueError('Prefill is only for newly admitted empty requests')
        features = self.verify(chunks, bucket=bucket)
        self.commit(features, {r: ids.shape[1] for r, ids in chunks.items()})
        return features

    @torch.no_grad()
    def predict(self, features, last_only=False):
        """The model's LM head over the verified rows (after its final norm)."""
        logits = self.model.get_output_embeddings()(features.last)
        return {r: (logits[:, offset + count - 1] if last_only else logits[:, offset:offset + count])
                for r, (offset, count, _) in features.spans.items()}

    def request_kv(self, request):
        """Per layer (keys, values) [1, Hkv, C, D] copies of a request's committed rows."""
        keys, values = self.store.request_kv(self._handles[request])
        return tuple((k.transpose(0, 1)[None], v.transpose(0, 1)[None]) for k, v in zip(keys, values))


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
        ALL_ATTENTION_FUNCTIONS.register(VARLEN_BACKEND, varlen_attention_forward)
        cfg._attn_implementation = VARLEN_BACKEND

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
