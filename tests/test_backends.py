"""The reference-side selection binding (CPU): the widened session guards of
dspark_qwen/packed_sampling.py:110-115 and packed_target_sampling.py:26-29,
and the explicit selection of dspark_qwen/varlen_target.py:136-150,
persistent_qwen_target.py:126-134 and packed_draft.py:76-82, as
qwen3_dspark_amd.backends states them.  Kernel objects are stood in for by
their classes (backend_name is a class attribute), so nothing touches a GPU."""
from types import SimpleNamespace

import pytest

from qwen3_dspark_amd import backends
from qwen3_dspark_amd.draft import HipDraftAttention
from qwen3_dspark_amd.kernels import HipCapacityKernel, HipDraftVarlenKernel, HipVarlenKernel


def stand_in(name):
    return SimpleNamespace(backend_name=name)


def test_kernel_classes_carry_the_role_names():
    assert HipVarlenKernel.backend_name == backends.TARGET_BACKEND
    assert HipCapacityKernel.backend_name == backends.CAPACITY_BACKEND
    assert HipDraftVarlenKernel.backend_name == backends.DRAFT_BACKEND
    assert HipDraftAttention.backend_name == backends.DRAFT_BLOCKS_BACKEND
    for cls in (HipVarlenKernel, HipCapacityKernel, HipDraftVarlenKernel, HipDraftAttention):
        assert cls.native_varlen_calls_per_layer == 1
    assert backends.TARGET_BACKENDS.isdisjoint(backends.DRAFT_BACKENDS)


@pytest.mark.parametrize('target', [HipVarlenKernel, HipCapacityKernel, stand_in(backends.REFERENCE_TARGET_BACKEND)])
@pytest.mark.parametrize('draft', [HipDraftVarlenKernel, HipDraftAttention, stand_in(backends.REFERENCE_DRAFT_BACKEND)])
def test_session_guard_accepts_every_target_draft_pair(target, draft):
    backends.check_session_backends(SimpleNamespace(_varlen_kernel=target), SimpleNamespace(kernel=draft))
    backends.check_target_backend(SimpleNamespace(_varlen_kernel=target))


@pytest.mark.parametrize('target,draft', [
    (HipDraftVarlenKernel, HipDraftAttention),          # a noncausal kernel in the target role
    (HipVarlenKernel, HipVarlenKernel),                 # a causal kernel in the draft role
    (stand_in('public'), HipDraftAttention),            # the public (upper-left) varlen
    (None, HipDraftAttention),                          # no _varlen_kernel attribute
    (HipVarlenKernel, None),                            # no draft kernel
])
def test_session_guard_rejects_wrong_roles_and_unknown_names(target, draft):
    t = SimpleNamespace() if target is None else SimpleNamespace(_varlen_kernel=target)
    d = SimpleNamespace() if draft is None else SimpleNamespace(kernel=draft)
    with pytest.raises(ValueError, match='explicit pinned target and noncausal draft backends'):
        backends.check_session_backends(t, d)


def test_target_only_guard_rejects_draft_kernels():
    with pytest.raises(ValueError, match='explicit pinned target backend'):
        backends.check_target_backend(SimpleNamespace(_varlen_kernel=HipDraftVarlenKernel))


def test_selection_refuses_unknown_names_before_device_work():
    for name in ('public', backends.REFERENCE_TARGET_BACKEND, backends.DRAFT_BACKEND, None):
        with pytest.raises(ValueError, match='Unknown explicit native varlen backend'):
            backends.target_kernel(name, 'cuda:0')
    for name in (None, backends.REFERENCE_DRAFT_BACKEND, backends.TARGET_BACKEND):
        with pytest.raises(ValueError, match='explicit noncausal draft backend'):
            backends.draft_kernel(name, 'cuda:0')


def test_selection_of_a_known_name_fails_loudly_without_a_gpu():
    # The selected class is constructed; without an MI355X it raises rather
    # than falling back to anything.
    import torch
    if torch.cuda.is_available():
        pytest.skip('a GPU is present; the GPU tests construct the kernels')
    for fn, name in ((backends.target_kernel, backends.TARGET_BACKEND),
                     (backends.target_kernel, backends.CAPACITY_BACKEND),
                     (backends.draft_kernel, backends.DRAFT_BACKEND),
                     (backends.draft_kernel, backends.DRAFT_BLOCKS_BACKEND)):
        with pytest.raises(RuntimeError, match='no CPU fallback'):
            fn(name, 'cuda:0')


def test_integration_document_names_the_edited_sites():
    import os
    text = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), 'INTEGRATION.md')).read()
    for site in ('varlen_target.py:136-150', 'persistent_qwen_target.py:126-134', 'packed_draft.py:76-82',
                 'packed_sampling.py:110-115', 'packed_target_sampling.py:26-29'):
        assert site in text, site
    for fn in ('backends.target_kernel', 'backends.draft_kernel', 'backends.check_session_backends',
               'backends.check_target_backend'):
        assert fn in text, fn
