"""Native entry point of weighted_laplace_sum with the name, checks and messages of the reference's pybind module
(Weighted_Laplace_Sum/csrc/binding.cpp:63-105): weighted_laplace_sum_forward(q, k, v) -> (out_w, out_u) of the PyTorch
C++ extension _qlka_torch.so (csrc/torch_ext.cpp) over libqlka.so's C ABI, resolved on first use."""

from qlka import _lib


def __getattr__(name):
    if name == "weighted_laplace_sum_forward":
        val = _lib.torch_ext().weighted_laplace_sum_forward
        globals()[name] = val
        return val
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
