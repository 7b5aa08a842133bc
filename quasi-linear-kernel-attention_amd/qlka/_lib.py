"""Loading of libqlka.so (the C ABI declared in include/qlka.h): a ctypes binding, and the PyTorch C++ extension
_qlka_torch.so built over the same library (the operators' entry points and autograd).

PyTorch is only plumbing here: it owns device memory (outputs and workspace come from its caching allocator) and the
current stream; every computation runs in the HIP kernels of libqlka.so. There is no CPU or PyTorch fallback: if the
library or the extension is missing or cannot be loaded, loading raises.
"""

import ctypes
import importlib.machinery
import importlib.util
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libqlka.so")
EXT_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_qlka_torch.so")

_c_int = ctypes.c_int
_c_size = ctypes.c_size_t
_c_ptr = ctypes.c_void_p

# name -> (restype, argtypes)
_SIGNATURES = {
    "qlka_last_error": (ctypes.c_char_p, []),
    "qlka_version": (_c_int, []),
    "qlka_laplace_fwd_ws_bytes": (_c_size, [_c_int] * 5),
    "qlka_laplace_fwd": (_c_int, [_c_ptr] * 5 + [_c_int] * 5 + [_c_ptr, _c_size, _c_ptr]),
    "qlka_laplace_fwd_noalloc": (_c_int, [_c_ptr] * 5 + [_c_int] * 5 + [_c_ptr]),
    "qlka_abs_fwd_ws_bytes": (_c_size, [_c_int] * 5),
    "qlka_abs_fwd": (_c_int, [_c_ptr] * 5 + [_c_int] * 6 + [_c_ptr, _c_size, _c_ptr]),
    "qlka_abs_bwd_ws_bytes": (_c_size, [_c_int] * 5),
    "qlka_abs_bwd": (_c_int, [_c_ptr] * 8 + [_c_int] * 5 + [_c_ptr, _c_size, _c_ptr]),
    "qlka_abs_bwd_walks": (_c_int, [_c_int] * 3),
    "qlka_abs_keep_state_bytes": (_c_size, [_c_int] * 5),
    "qlka_abs_fwd_keep": (_c_int, [_c_ptr] * 5 + [_c_int] * 6 + [_c_ptr] * 6 + [_c_ptr, _c_size, _c_ptr]),
    "qlka_abs_bwd_sorted": (_c_int, [_c_ptr] * 8 + [_c_int] * 5 + [_c_ptr] * 5 + [_c_ptr, _c_size, _c_ptr]),
    "qlka_abs_dense_keep_bytes": (_c_size, [_c_int] * 5),
    "qlka_abs_fwd_dense_keep": (_c_int, [_c_ptr] * 6 + [_c_int] * 5 + [_c_ptr]),
    "qlka_abs_bwd_dense_kept": (_c_int, [_c_ptr] * 9 + [_c_int] * 5 + [_c_ptr]),
    "qlka_sgn_fwd_ws_bytes": (_c_size, [_c_int] * 5),
    "qlka_sgn_fwd": (_c_int, [_c_ptr] * 5 + [_c_int] * 5 + [_c_ptr, _c_size, _c_ptr]),
    "qlka_direct_fwd": (_c_int, [_c_int] + [_c_ptr] * 5 + [_c_int] * 5 + [_c_ptr]),
    "qlka_direct_bwd": (_c_int, [ctypes.c_float] + [_c_ptr] * 8 + [_c_int] * 5 + [_c_ptr]),
    "qlka_direct_sgn": (_c_int, [ctypes.c_float] + [_c_ptr] * 5 + [_c_int] * 5 + [_c_ptr]),
    "qlka_layer_fwd_ws_bytes": (_c_size, [_c_int] * 6),
    "qlka_layer_fwd": (_c_int, [_c_int] + [_c_ptr] * 5 + [_c_int] * 5 + [_c_ptr, _c_size, _c_ptr]),
    "qlka_layer_fwd_masked": (_c_int, [_c_int] + [_c_ptr] * 5 + [_c_int] * 5 + [_c_ptr, _c_size, _c_ptr]),
    "qlka_seg_sort_ws_bytes": (_c_size, [_c_int] * 2),
    "qlka_seg_sort": (_c_int, [_c_ptr] * 3 + [_c_int] * 2 + [_c_ptr, _c_size, _c_ptr]),
    "qlka_merge_rank_ws_bytes": (_c_size, [_c_int] * 3),
    "qlka_merge_rank": (_c_int, [_c_ptr] * 3 + [_c_int] * 3 + [_c_ptr, _c_size, _c_ptr]),
    "qlka_set_direct_max": (_c_int, [_c_int]),
    "qlka_set_workspace_budget": (_c_size, [_c_size]),
    "qlka_timing_enable": (_c_int, [_c_int]),
    "qlka_timing_reset": (_c_int, []),
    "qlka_timing_read": (_c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_longlong)]),
}

EXPORTED = tuple(_SIGNATURES)

_lib = None


def load():
    """Load libqlka.so once and return the ctypes handle. Raises OSError/RuntimeError if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libqlka.so not found at {LIB_PATH}; build it with "
                "`python quasi-linear-kernel-attention_amd/qlka/build.py` (hipcc, gfx950)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


_ext = None


def torch_ext():
    """Import the in-tree _qlka_torch.so once (after libqlka.so, which it links) and return the module."""
    global _ext
    if _ext is None:
        load()
        if not os.path.exists(EXT_PATH):
            raise RuntimeError(
                f"_qlka_torch.so not found at {EXT_PATH}; build it with "
                "`python quasi-linear-kernel-attention_amd/qlka/build.py`")
        loader = importlib.machinery.ExtensionFileLoader("_qlka_torch", EXT_PATH)
        spec = importlib.util.spec_from_file_location("_qlka_torch", EXT_PATH, loader=loader)
        mod = importlib.util.module_from_spec(spec)
        loader.exec_module(mod)
        _ext = mod
    return _ext


def check(rc):
    """Turn a nonzero libqlka return code into RuntimeError carrying qlka_last_error()."""
    if rc != 0:
        msg = load().qlka_last_error().decode("utf-8", "replace")
        raise RuntimeError(msg or f"libqlka error {rc}")


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def stream_of(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def stage_time(name):
    """(total_ms, count) accumulated by the library's stage timer for one stage name."""
    ms = ctypes.c_double(0.0)
    n = ctypes.c_longlong(0)
    check(load().qlka_timing_read(name.encode(), ctypes.byref(ms), ctypes.byref(n)))
    return ms.value, n.value


def workspace(nbytes, device):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
