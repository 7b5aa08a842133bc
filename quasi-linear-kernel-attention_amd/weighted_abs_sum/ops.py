"""Public ops and backend dispatch of weighted_abs_sum, mirroring Weighted_Abs_Sum/weighted_abs_sum/ops.py:1-139.

Backends "auto", "keops", "cuda", "cuda-fused", "cuda-global" are all accepted (ops.py:12-13). On MI355X every backend
runs the native gfx950 kernels of libqlka.so:

* "cuda" / "cuda-global" -> path -1 / 0, "cuda-fused" -> path 1 (which, as in the reference, raises for
  max(N, M) > 4096).
* "keops" (passed by Experiments/kernel_attention/attention.py:63 for S < 256) has no pykeops behind it on ROCm. It
  runs the native dense evaluation with KeOps' semantics: the forward (qlka_direct_fwd: A = sum_d |q_d - k_d| reduced
  against [v, 1], keops_backend.py:19-35) on contiguous copies as KeOps makes them, its gradients (qlka_direct_bwd)
  and weighted_sgn_sum (qlka_direct_sgn) with sign(0) = 0 (keops_backend.py:40-41).
* "auto" behaves as in the reference: "keops" strictly below KEOPS_CUTOFF, else "cuda".
"""

import torch

from weighted_abs_sum import _ext as _C

_BACKENDS = ("auto", "keops", "cuda", "cuda-fused", "cuda-global")
_DIRECT = 2             # the keops route: dense evaluation (the extension's DIRECT path code)
_PATH = {"cuda": -1, "cuda-fused": 1, "cuda-global": 0, "keops": _DIRECT}

# "auto" uses the keops route strictly below this max(N,M)
KEOPS_CUTOFF = 512


# Keep the forward's sorted k and q for the backward (the reference's backward sorts again): costs 8*P*D*(N+M)
# bytes per differentiable call until its backward runs, saves two segmented sorts per backward.
KEEP_SORTS = True


def set_keep_sorts(flag):
    """Keep (True, default) or drop (False) the forward's sorts for the backward of differentiable calls."""
    global KEEP_SORTS
    KEEP_SORTS = bool(flag)
    return KEEP_SORTS


def set_keops_cutoff(n):
    """Set the max(N,M) below which backend='auto' uses the keops route (0 disables)."""
    global KEOPS_CUTOFF
    KEOPS_CUTOFF = int(n)
    return KEOPS_CUTOFF


def _resolve(backend, q, k, v):
    if backend not in _BACKENDS:
        raise ValueError(f"backend must be one of {_BACKENDS}, got {backend!r}")
    if backend != "auto":
        return backend
    if not (q.is_cuda and q.dtype == torch.float32):
        return "cuda"   # let the extension raise its precise error message
    if max(q.shape[-1], k.shape[-1]) < KEOPS_CUTOFF:
        return "keops"
    return "cuda"


def _keep(q, k, v):
    """Keep the forward's sorts: KEEP_SORTS and a gradient will be wanted from this call."""
    return KEEP_SORTS and torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)


# The two differentiable ops are one C++ autograd Function of the extension (csrc/torch_ext.cpp, AbsSumFn), the
# counterpart of the reference's _WeightedAbsSum / _WeightedAbsSumFull (ops.py:72-104): its forward runs the dense
# route for "keops" (on contiguous copies) or the native ops, keeping the sorted k and q for the backward when asked;
# its backward is the dense gradient with sign(0) = 0 for "keops", else the native backward over the kept sorts
# (or sorting again), the plain one when out_u gets no gradient. Neither direction runs Python.


def weighted_abs_sum(q, k, v, backend="auto"):
    """out[p,m,c] = sum_{n,d} |k[p,d,n] - q[p,d,m]| * v[p,n,c]

    q: (P, D, M), k: (P, D, N), v: (P, N, C) -> (P, M, C). Differentiable.
    """
    b = _resolve(backend, q, k, v)
    return _C.abs_sum_autograd(q, k, v, _PATH[b], False, _keep(q, k, v))[0]


def weighted_abs_sum_full(q, k, v, backend="auto"):
    """Returns (out_w, out_u): the weighted abs sum (P, M, C) and the unweighted abs sum
    out_u[p,m] = sum_{n,d} |k[p,d,n] - q[p,d,m]| (P, M), from one pass. Differentiable in both outputs.
    """
    b = _resolve(backend, q, k, v)
    out_w, out_u = _C.abs_sum_autograd(q, k, v, _PATH[b], True, _keep(q, k, v))
    return out_w, out_u


def weighted_sgn_sum(q, k, v, g, backend="auto"):
    """out[p,d,m] = sum_n sgn(k[p,d,n] - q[p,d,m]) * dot(v[p,n,:], g[p,m,:])

    (P, D, M). Not differentiable (it IS a gradient).
    """
    b = _resolve(backend, q, k, v)
    if b == "keops":        # KeOps semantics: sign(0) = 0 (keops_backend.py:38-48)
        return _C.weighted_sgn_sum_direct(q.contiguous(), k.contiguous(), v.contiguous(), g.contiguous(), tie=0.0)
    if b == "cuda-fused":
        raise ValueError("weighted_sgn_sum has no fused path; use 'cuda' or 'cuda-global'")
    return _C.weighted_sgn_sum_forward(q, k, v, g.contiguous())
