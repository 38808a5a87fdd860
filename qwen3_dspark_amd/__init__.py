"""MI355X-native (gfx950) DSpark attention hot path at Qwen3-0.6B shapes.

Drop-in replacements for the reference's attention boundary:
  kernels.HipVarlenKernel / HipDraftVarlenKernel / HipCapacityKernel
      kernel(query, key, value, layout, *, scale) callables
  persistent_kv.PersistentTargetKV
      begin / stage_layer / prepare_attention / commit / abort transactions,
      plus attend(): verification attention fused with the KV gather
  draft.HipDraftAttention + draft.DraftBatch
      multi-block draft attention streaming the context once per request
  layout.PackedLayout / PersistentAttentionLayout
All device work is hand-written HIP behind the C ABI in include/dspark_amd.h.
"""
from .layout import PackedLayout, PersistentAttentionLayout  # noqa: F401

__all__ = ['PackedLayout', 'PersistentAttentionLayout']
