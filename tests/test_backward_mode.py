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


def test_scoped_mode_overrides_the_default_and_nests():
    from dmad_amd import backward_mode, current_backward_mode

    assert current_backward_mode() == "auto"
    with backward_mode("full"):
        assert _saved(False) == (10, True)
        with backward_mode("reference"):
            assert _saved(True) == (5, False)
        assert current_backward_mode() == "full"
    assert current_backward_mode() == "auto"
    assert _saved(False) == (5, False)
    # a scope wins over the process default while it is open
    set_backward_mode("full")
    with backward_mode("auto"):
        assert _saved(False) == (5, False)
    assert _saved(False) == (10, True)
    with pytest.raises(ValueError, match="backward mode"):
        with backward_mode("exact"):
            pass


def test_scoped_mode_is_local_to_its_thread():
    """A scope opened in one thread leaves the forwards of another thread on the
    process default."""
    import threading

    from dmad_amd import backward_mode

    entered, release = threading.Event(), threading.Event()
    seen = {}

    def worker():
        with backward_mode("full"):
            seen["worker"] = _saved(False)
            entered.set()
            release.wait(10)

    t = threading.Thread(target=worker)
    t.start()
    assert entered.wait(10)
    seen["main"] = _saved(False)
    release.set()
    t.join(10)
    assert seen == {"worker": (10, True), "main": (5, False)}


def test_mode_is_recorded_by_the_forward():
    """The node keeps the mode of the scope its forward ran in."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    from dmad_amd import backward_mode

    with FakeTensorMode():
        xs = [torch.empty(1, 2, 64, 32, dtype=torch.bfloat16).requires_grad_(i < 3) for i in range(6)]
        with backward_mode("full"):
            o, _ = _attention.apply(*xs)
        assert o.grad_fn.full is True


def test_mode_read_traces_under_torch_compile():
    """TorchDynamo cannot trace a context variable: under torch.compile the scope is
    read once at trace time, and the process default is a guarded global, so
    set_backward_mode makes the compiled function retrace (fullgraph: no break)."""
    import torch._dynamo

    from dmad_amd import backward_mode
    from dmad_amd.jvp_attention import current_backward_mode

    torch._dynamo.reset()

    def f(x):
        return x + (1.0 if current_backward_mode() == "full" else 2.0)

    cf = torch.compile(f, backend="eager", fullgraph=True)
    x = torch.zeros(2)
    assert cf(x).tolist() == [2.0, 2.0]
    set_backward_mode("full")
    assert cf(x).tolist() == [1.0, 1.0]
    set_backward_mode("auto")
    assert cf(x).tolist() == [2.0, 2.0]
    torch._dynamo.reset()
    with backward_mode("full"):
        assert cf(x).tolist() == [1.0, 1.0]
    torch._dynamo.reset()
