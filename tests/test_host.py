"""CPU checks of the Python boundary (the drop-in packages): names, signatures, backend strings and the reference's
error types/messages for inputs that fail before any kernel runs."""

import inspect

import pytest
import torch

import weighted_abs_sum
import weighted_laplace_sum
from weighted_abs_sum import _ext, ops


def test_public_names():
    assert weighted_abs_sum.__all__ == ["weighted_abs_sum", "weighted_abs_sum_full", "weighted_sgn_sum",
                                        "set_keops_cutoff"]
    assert weighted_laplace_sum.__all__ == ["weighted_laplace_sum"]
    assert list(inspect.signature(weighted_abs_sum.weighted_abs_sum).parameters) == ["q", "k", "v", "backend"]
    assert list(inspect.signature(weighted_abs_sum.weighted_sgn_sum).parameters) == ["q", "k", "v", "g", "backend"]
    assert list(inspect.signature(weighted_laplace_sum.weighted_laplace_sum).parameters) == ["q", "k", "v"]
    for name in ("weighted_abs_sum_forward", "weighted_abs_sum_full_forward", "weighted_abs_sum_backward",
                 "weighted_abs_sum_full_backward", "weighted_sgn_sum_forward"):
        assert callable(getattr(_ext, name))


def test_backend_strings():
    q = torch.zeros(1, 1, 4)
    with pytest.raises(ValueError, match="backend must be one of"):
        weighted_abs_sum.weighted_abs_sum(q, q, torch.zeros(1, 4, 2), backend="triton")
    for b in ("auto", "keops", "cuda", "cuda-fused", "cuda-global"):
        assert ops._resolve(b, q, q, None) in ("keops", "cuda", "cuda-fused", "cuda-global")
    # a non-CUDA tensor resolves to "cuda" so the extension raises its own message (ops.py:65-66)
    assert ops._resolve("auto", q, q, None) == "cuda"


def test_set_keops_cutoff():
    old = ops.KEOPS_CUTOFF
    try:
        assert weighted_abs_sum.set_keops_cutoff(100) == 100
        assert ops.KEOPS_CUTOFF == 100
        assert weighted_abs_sum.set_keops_cutoff("0") == 0
    finally:
        weighted_abs_sum.set_keops_cutoff(old)


def test_cpu_tensors_raise_reference_messages():
    q = torch.zeros(1, 2, 4)
    v = torch.zeros(1, 4, 3)
    with pytest.raises(RuntimeError, match="q, k, and v must be CUDA tensors"):
        weighted_abs_sum.weighted_abs_sum(q, q, v)
    with pytest.raises(RuntimeError, match="q, k, and v must be CUDA tensors"):
        weighted_abs_sum.weighted_abs_sum_full(q, q, v, backend="cuda-global")
    with pytest.raises(RuntimeError, match="q, k, and v must be CUDA tensors"):
        weighted_abs_sum.weighted_sgn_sum(q, q, v, torch.zeros(1, 4, 3))
    with pytest.raises(RuntimeError, match="q, k and v must be CUDA tensors"):
        weighted_laplace_sum.weighted_laplace_sum(q, q, v)


def test_torch_extension_is_the_boundary():
    """The drop-in packages' entry points are the C++ extension's (no Python in the call or its backward): every
    name of the reference's pybind modules and the differentiable op resolve to _qlka_torch.so built in-tree."""
    from qlka import _lib
    import weighted_laplace_sum._ext as lext
    ext = _lib.torch_ext()
    assert ext.__file__ == _lib.EXT_PATH
    for name in _ext._NAMES:
        assert getattr(_ext, name) is getattr(ext, name)
    assert lext.weighted_laplace_sum_forward is ext.weighted_laplace_sum_forward
    assert ops._DIRECT == ext.DIRECT
    # errors from C++ keep the reference's types and texts, also for the shape and argument checks
    q = torch.zeros(1, 2, 4)
    with pytest.raises(RuntimeError, match="q, k, and v must be CUDA tensors"):
        ext.abs_sum_autograd(q, q, torch.zeros(1, 4, 3), -1, True, False)
    with pytest.raises(TypeError):
        ext.weighted_abs_sum_forward(q, q)
