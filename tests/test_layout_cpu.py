"""Which operand layouts go to the kernels as they are and which are copied first
(host logic only, fake tensors: nothing is allocated or launched).

The kernels address one (batch, head) slice with 32-bit byte offsets. The Wan
callers hand the op BSHD storage viewed as BHSD (train/wan/rcm/utils/jvp_helper.py:52-66),
whose row stride is H*D, so at long sequences one head's slice spans more than 2 GiB
although the head itself holds only L*D elements. Such views are copied to
contiguous BHSD (row stride D) instead of being refused by the C ABI.
"""
import warnings

import pytest
import torch

from dmad_amd.jvp_attention import MAX_SLICE_BYTES, _pair, _prep, slice_fits


def test_slice_limit_of_the_wan_layout():
    # 14B layer, BSHD view: row stride H*D = 5120 bf16 elements
    last = (MAX_SLICE_BYTES // 2 - 128) // 5120 - 256  # largest L that still fits
    assert slice_fits(last, 5120, 128, 2) and not slice_fits(last + 1, 5120, 128, 2)
    assert 209_000 < last + 1 < 210_000
    assert slice_fits(75600, 5120, 128, 2)          # 720p fits as a view
    assert slice_fits(8_000_000, 128, 128, 2)       # a contiguous head fits far longer
    assert not slice_fits(300_000, 5120, 128, 2)
    assert not slice_fits(300_000, 2560, 64, 4)     # fp32 elements count twice


def _fake(L, H=40, D=128, dtype=torch.bfloat16):
    return torch.empty(1, L, H, D, dtype=dtype).transpose(1, 2)  # BSHD storage as BHSD


@pytest.mark.parametrize("L,copied", [(75600, False), (210_000, True)])
def test_long_bshd_views_are_copied_to_bhsd(L, copied):
    from torch._subclasses.fake_tensor import FakeTensorMode

    with warnings.catch_warnings(), FakeTensorMode():
        warnings.simplefilter("ignore")  # data_ptr of a fake tensor (alignment check)
        q, tq = _fake(L), _fake(L)
        q2, tq2 = _pair(q, tq)
        (k2,) = _prep(_fake(L))
        for x in (q2, tq2, k2):
            assert x.shape == (1, 40, L, 128)
            assert x.stride() == ((40 * L * 128, L * 128, 128, 1) if copied else (L * 40 * 128, 128, 5120, 1))
        assert q2.stride() == tq2.stride()
        # a primal that fits with a tangent that does not: both copied, strides equal
        q3, tq3 = _pair(_fake(L, H=20), _fake(L, H=20).contiguous())
        assert q3.stride() == tq3.stride()
