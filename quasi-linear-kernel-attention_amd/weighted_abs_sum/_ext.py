"""Native entry points of weighted_abs_sum, with the names, arguments, checks and error messages of the reference's
pybind module (Weighted_Abs_Sum/csrc/binding.cpp:442-453): the functions of the PyTorch C++ extension _qlka_torch.so
(csrc/torch_ext.cpp) over libqlka.so's C ABI.

Outputs and the workspace are allocated from torch's caching allocator on q's device; every launch goes on the
current stream of that device. Errors raise RuntimeError with the reference's TORCH_CHECK messages.

    weighted_abs_sum_forward(q, k, v, path=-1)               binding.cpp:229-233
    weighted_abs_sum_full_forward(q, k, v, path=-1)          binding.cpp:235-239
    weighted_abs_sum_backward(q, k, v, g_w)                  binding.cpp:370-374
    weighted_abs_sum_full_backward(q, k, v, g_w, g_u)        binding.cpp:376-380
    weighted_sgn_sum_forward(q, k, v, g)                     binding.cpp:383-439

and, with no counterpart in the reference's module: weighted_abs_sum_forward_keep / weighted_abs_sum_backward_sorted
(the forward keeps its sorts for the backward), weighted_abs_sum_direct_forward / _direct_backward /
weighted_sgn_sum_direct (the dense "keops" route) and abs_sum_autograd (the differentiable ops). The module resolves
them from the extension on first use.
"""

from qlka import _lib

_NAMES = ("weighted_abs_sum_forward", "weighted_abs_sum_full_forward", "weighted_abs_sum_backward",
          "weighted_abs_sum_full_backward", "weighted_sgn_sum_forward", "weighted_abs_sum_forward_keep",
          "weighted_abs_sum_backward_sorted", "weighted_abs_sum_direct_forward", "weighted_abs_sum_direct_backward",
          "weighted_sgn_sum_direct", "abs_sum_autograd", "DIRECT")


def __getattr__(name):
    if name in _NAMES:
        val = getattr(_lib.torch_ext(), name)
        globals()[name] = val
        return val
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")


def __dir__():
    return sorted(list(globals()) + list(_NAMES))
