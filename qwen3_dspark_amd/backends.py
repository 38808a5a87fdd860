"""Backend identities of the MI355X kernels, for the reference's selection points.

The reference picks its native attention by name and checks the identity of
what it picked:
  * VarlenPackedTarget.__init__ builds PinnedRocmVarlenKernel for
    native_backend == rocm_varlen.BACKEND (dspark_qwen/varlen_target.py:136-150),
    and PersistentQwenTarget.__init__ does the same for its capacity-tail
    call (dspark_qwen/persistent_qwen_target.py:126-134);
  * PackedDraft.__init__ accepts only packed_draft.DRAFT_BACKEND
    (dspark_qwen/packed_draft.py:76-82);
  * the sessions compare target._varlen_kernel.backend_name and
    packed_draft.kernel.backend_name with those two names
    (dspark_qwen/packed_sampling.py:110-115,
    dspark_qwen/packed_target_sampling.py:26-29).
A HIP kernel object carries its own backend_name.  The functions below are
the widened selection and guards a reference maintainer puts at those sites:
each accepts the reference's own pinned name as before, plus this build's
names for the same role, and raises the reference's ValueError (same
message) for anything else, before any device work.
"""

# The reference's pinned backend names (dspark_qwen/rocm_varlen.py:11,
# dspark_qwen/packed_draft.py:16).
REFERENCE_TARGET_BACKEND = 'rocm_aten_no_window_pinned_v1'
REFERENCE_DRAFT_BACKEND = 'rocm_aten_no_window_noncausal_pinned_v1'

# This build's kernels by role (each class carries the same backend_name).
TARGET_BACKEND = 'mi355x_hip_varlen_causal_v1'         # kernels.HipVarlenKernel
CAPACITY_BACKEND = 'mi355x_hip_capacity_causal_v1'     # kernels.HipCapacityKernel
DRAFT_BACKEND = 'mi355x_hip_varlen_noncausal_v1'       # kernels.HipDraftVarlenKernel
DRAFT_BLOCKS_BACKEND = 'mi355x_hip_draft_blocks_v1'    # draft.HipDraftAttention

TARGET_BACKENDS = frozenset({REFERENCE_TARGET_BACKEND, TARGET_BACKEND, CAPACITY_BACKEND})
DRAFT_BACKENDS = frozenset({REFERENCE_DRAFT_BACKEND, DRAFT_BACKEND, DRAFT_BLOCKS_BACKEND})


def target_kernel(native_backend, device):
    """The causal varlen kernel for an explicit HIP backend name
    (varlen_target.py:136-150: TARGET_BACKEND; persistent_qwen_target.py:126-134:
    CAPACITY_BACKEND, whose layouts are capacity-length)."""
    if native_backend == TARGET_BACKEND:
        from .kernels import HipVarlenKernel
        return HipVarlenKernel(device)
    if native_backend == CAPACITY_BACKEND:
        from .kernels import HipCapacityKernel
        return HipCapacityKernel(device)
    raise ValueError('Unknown explicit native varlen backend')


def draft_kernel(native_backend, device):
    """The draft kernel for an explicit HIP backend name (packed_draft.py:76-82):
    the packed noncausal varlen callable, or the multi-block fused kernel."""
    if native_backend == DRAFT_BACKEND:
        from .kernels import HipDraftVarlenKernel
        return HipDraftVarlenKernel(device)
    if native_backend == DRAFT_BLOCKS_BACKEND:
        from .draft import HipDraftAttention
        return HipDraftAttention(device)
    raise ValueError('Select explicit noncausal draft backend; no default/fallback')


def _name(obj):
    return getattr(obj, 'backend_name', None)


def check_session_backends(target, packed_draft):
    """packed_sampling.py:110-115, widened: the GPU session's target kernel
    and draft kernel must each be a pinned reference backend or this build's
    kernel for that role."""
    if (_name(getattr(target, '_varlen_kernel', None)) not in TARGET_BACKENDS
            or _name(getattr(packed_draft, 'kernel', None)) not in DRAFT_BACKENDS):
        raise ValueError('GPU session requires explicit pinned target and noncausal draft backends')


def check_target_backend(target):
    """packed_target_sampling.py:26-29, widened the same way."""
    if _name(getattr(target, '_varlen_kernel', None)) not in TARGET_BACKENDS:
        raise ValueError('GPU target-only session requires explicit pinned target backend')
