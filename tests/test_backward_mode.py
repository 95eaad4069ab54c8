"""Saved tensors and backward modes of the autograd op (CPU, fake tensors): the
default keeps exactly what the reference keeps for the backward (q, k, v, o and
the LSE, train/wan/rcm/utils/flash_attention_jvp_triton.py:500-502) unless a
tangent requires grad; mode "full" also keeps the tangent side."""
import pytest
import torch

import dmad_amd  # noqa: F401  (registers the ops)
from dmad_amd.jvp_attention import _attention, set_backward_mode


@pytest.fixture(autouse=True)
def _restore_mode():
    yield
    set_backward_mode("auto")


def _saved(tangent_grad):
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        xs = [torch.empty(1, 2, 64, 32, dtype=torch.bfloat16).requires_grad_(i < 3 or tangent_grad) for i in range(6)]
        o, to = _attention.apply(*xs)
        node = o.grad_fn
        return len(node.saved_tensors), node.full


@pytest.mark.parametrize("mode,tangent_grad,n,full", [
    ("auto", False, 5, False), ("auto", True, 10, True),
    ("reference", False, 5, False), ("reference", True, 5, False),
    ("full", False, 10, True), ("full", True, 10, True),
])
def test_saved_tensors_follow_the_mode(mode, tangent_grad, n, full):
    set_backward_mode(mode)
    assert _saved(tangent_grad) == (n, full)


def test_unknown_mode_is_rejected():
    with pytest.raises(ValueError, match="backward mode"):
        set_backward_mode("exact")


def _saved_d(D, tangent_grad):
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        xs = [torch.empty(1, 2, 64, D, dtype=torch.bfloat16).requires_grad_(i < 3 or tangent_grad) for i in range(6)]
        o, to = _attention.apply(*xs)
        node = o.grad_fn
        return len(node.saved_tensors), node.full


def test_wide_heads_fall_back_to_the_reference_backward_in_auto_mode():
    """Head dim 256 has no full-derivative kernels: "auto" keeps the reference's backward
    (dO-only, tangents get None) with one warning instead of failing in backward."""
    import dmad_amd.jvp_attention as ja

    ja._warned_full_fallback = False
    with pytest.warns(UserWarning, match="no gradients"):
        assert _saved_d(256, True) == (5, False)
    assert _saved_d(128, True) == (10, True)


def test_wide_heads_raise_in_forward_in_full_mode():
    set_backward_mode("full")
    with pytest.raises(NotImplementedError, match="head dims up to 128"):
        _saved_d(256, False)
    assert _saved_d(128, False) == (10, True)
