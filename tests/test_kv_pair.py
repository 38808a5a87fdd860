"""kv_pair: K and V of one store in one allocation, V a fixed distance
after K (CPU tensors: the layout, not the speed)."""
import pytest
import torch

from qwen3_dspark_amd._device import KV_PAIR_SKEW, kv_pair


@pytest.mark.parametrize('kdt,vdt', [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.bfloat16)])
def test_layout(kdt, vdt):
    shape = (2, 3, 8, 16, 128)
    k, v = kv_pair(shape, kdt, vdt, 'cpu', skew=4096)
    assert k.shape == v.shape == shape and k.dtype == kdt and v.dtype == vdt
    assert k.is_contiguous() and v.is_contiguous()
    assert k.untyped_storage().data_ptr() == v.untyped_storage().data_ptr()
    kb = k.numel() * k.element_size()
    assert v.data_ptr() - k.data_ptr() == kb + 4096
    assert not k.any() and not v.any()
    v.fill_(1)
    assert not k.any()                                       # no overlap
    assert KV_PAIR_SKEW == 32 << 20


def test_refuses_bad_skew():
    for bad in (-256, 100):
        with pytest.raises(ValueError, match='multiple of 256'):
            kv_pair((1, 8, 128), torch.bfloat16, torch.bfloat16, 'cpu', skew=bad)
