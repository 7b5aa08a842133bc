"""Native entry points of weighted_abs_sum, with the names, arguments, checks and error messages of the reference's
pybind module (Weighted_Abs_Sum/csrc/binding.cpp:442-453), implemented over libqlka.so's C ABI.

Outputs and the workspace are allocated from torch's caching allocator on q's device; every launch goes on the
current stream of that device. Errors raise RuntimeError with the reference's TORCH_CHECK messages.
"""

import ctypes

import torch

from qlka import _lib


def _check_qkv(q, k, v):
    """Validation of check_qkv (Weighted_Abs_Sum/csrc/binding.cpp:69-84), same messages."""
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError("q, k, and v must be CUDA tensors")
    if not (q.device == k.device and q.device == v.device):
        raise RuntimeError("q, k, and v must be on the same CUDA device")
    if not (q.dtype == torch.float32 and k.dtype == torch.float32 and v.dtype == torch.float32):
        raise RuntimeError("q, k, and v must be float32")
    if not (q.dim() == 3 and k.dim() == 3 and v.dim() == 3):
        raise RuntimeError("q, k, and v must be 3D tensors")
    if not (q.size(0) == k.size(0) and q.size(0) == v.size(0)):
        raise RuntimeError("Batch size of q, k, and v must match")
    if q.size(1) != k.size(1):
        raise RuntimeError("q and k must have same feature dimension")
    if k.size(2) != v.size(1):
        raise RuntimeError("k and v must have same length")
    if not (q.is_contiguous() and k.is_contiguous() and v.is_contiguous()):
        raise RuntimeError("q, k, and v must be contiguous")
    P, D, N, C, M = q.size(0), q.size(1), k.size(2), v.size(2), q.size(2)
    if not (M > 0 and N > 0 and D > 0):
        raise RuntimeError("N, M and D must be > 0")
    if not (1 <= C <= 128):
        raise RuntimeError("C (v.size(2)) must be in [1, 128]")
    if not (N <= 131072 and M <= 131072):
        raise RuntimeError("N and M must be <= 131072")
    if P * D * max(N, M) > 2 ** 31 - 1:
        raise RuntimeError("P*D*max(N,M) must fit int32 (cub sort offsets)")
    return P, D, N, M, C


def _check_grad(name, g, q, shape):
    if not (g.is_cuda and g.device == q.device):
        raise RuntimeError(f"{name} must be on q's CUDA device")
    if g.dtype != torch.float32:
        raise RuntimeError(f"{name} must be float32")
    if len(shape) == 3:
        if g.dim() != 3:
            raise RuntimeError(f"{name} must be 3D")
        if tuple(g.shape) != shape:
            raise RuntimeError(f"{name} must have shape (P, M, C)")
    else:
        if g.dim() != 2 or tuple(g.shape) != shape:
            raise RuntimeError(f"{name} must have shape (P, M)")
    if not g.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _forward(q, k, v, path, full):
    P, D, N, M, C = _check_qkv(q, k, v)
    if not (-1 <= int(path) <= 1):
        raise RuntimeError("path must be -1 (auto), 0 (global) or 1 (fused)")
    lib = _lib.load()
    dev = q.device
    with torch.cuda.device(dev):
        out = torch.empty((P, M, C), dtype=q.dtype, device=dev)
        out_u = torch.empty((P, M), dtype=q.dtype, device=dev) if full else None
        ws = _lib.workspace(lib.qlka_abs_fwd_ws_bytes(P, D, N, M, C), dev)
        _lib.check(lib.qlka_abs_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out), _lib.ptr(out_u),
                                    P, D, N, M, C, int(path), _lib.ptr(ws), ws.numel(), _lib.stream_of(dev)))
    return out, out_u


def weighted_abs_sum_forward(q, k, v, path=-1):
    """out[p,m,c] = sum_{n,d} |k[p,d,n] - q[p,d,m]| * v[p,n,c]  (Weighted_Abs_Sum/csrc/binding.cpp:229-233)."""
    return _forward(q, k, v, path, full=False)[0]


def weighted_abs_sum_full_forward(q, k, v, path=-1):
    """(out_w, out_u) with out_u[p,m] = sum_{n,d} |k - q|  (Weighted_Abs_Sum/csrc/binding.cpp:235-239)."""
    return _forward(q, k, v, path, full=True)


def weighted_abs_sum_forward_keep(q, k, v, path, full):
    """The forward of weighted_abs_sum(_full) (qlka_abs_fwd_keep) that also returns the sorted k and q with their
    permutations when the backward at this shape sorts and walks (else None), for
    weighted_abs_sum_backward_sorted. Not in the reference's pybind module: its backward sorts again."""
    P, D, N, M, C = _check_qkv(q, k, v)
    if not (-1 <= int(path) <= 1):
        raise RuntimeError("path must be -1 (auto), 0 (global) or 1 (fused)")
    lib = _lib.load()
    dev = q.device
    with torch.cuda.device(dev):
        out = torch.empty((P, M, C), dtype=q.dtype, device=dev)
        out_u = torch.empty((P, M), dtype=q.dtype, device=dev) if full else None
        srt = None
        if lib.qlka_abs_bwd_walks(P, N, M):
            srt = (torch.empty((P, D, N), dtype=q.dtype, device=dev),
                   torch.empty((P, D, N), dtype=torch.int32, device=dev),
                   torch.empty((P, D, M), dtype=q.dtype, device=dev),
                   torch.empty((P, D, M), dtype=torch.int32, device=dev))
        kept = ctypes.c_int(0)
        ws = _lib.workspace(lib.qlka_abs_fwd_ws_bytes(P, D, N, M, C), dev)
        if srt is None:
            _lib.check(lib.qlka_abs_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out), _lib.ptr(out_u),
                                        P, D, N, M, C, int(path), _lib.ptr(ws), ws.numel(), _lib.stream_of(dev)))
        else:
            _lib.check(lib.qlka_abs_fwd_keep(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out), _lib.ptr(out_u),
                                             P, D, N, M, C, int(path), *(_lib.ptr(t) for t in srt),
                                             ctypes.byref(kept), _lib.ptr(ws), ws.numel(), _lib.stream_of(dev)))
    return out, out_u, (srt if kept.value else None)


def weighted_abs_sum_backward_sorted(q, k, v, g_w, g_u, srt):
    """The backward of weighted_abs_sum(_full) over the sorts a weighted_abs_sum_forward_keep of the same q, k, v
    left (qlka_abs_bwd_sorted). g_u may be None. Not in the reference's pybind module."""
    P, D, N, M, C = _check_qkv(q, k, v)
    _check_grad("g_w", g_w, q, (P, M, C))
    if g_u is not None:
        _check_grad("g_u", g_u, q, (P, M))
    ks, kp, qs, qp = srt
    if not (ks.shape == (P, D, N) and kp.shape == (P, D, N) and qs.shape == (P, D, M) and qp.shape == (P, D, M)):
        raise RuntimeError("sorted arrays do not match q and k")
    lib = _lib.load()
    dev = q.device
    with torch.cuda.device(dev):
        grad_q = torch.empty((P, D, M), dtype=q.dtype, device=dev)
        grad_k = torch.empty((P, D, N), dtype=q.dtype, device=dev)
        grad_v = torch.empty((P, N, C), dtype=q.dtype, device=dev)
        ws = _lib.workspace(lib.qlka_abs_bwd_ws_bytes(P, D, N, M, C), dev)
        _lib.check(lib.qlka_abs_bwd_sorted(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g_w), _lib.ptr(g_u),
                                           _lib.ptr(grad_q), _lib.ptr(grad_k), _lib.ptr(grad_v), P, D, N, M, C,
                                           *(_lib.ptr(t) for t in srt), _lib.ptr(ws), ws.numel(),
                                           _lib.stream_of(dev)))
    return grad_q, grad_k, grad_v


def weighted_abs_sum_direct_forward(q, k, v, full):
    """Dense evaluation (qlka_direct_fwd): the same (out_w, out_u) without a sort, for the "keops" route (the
    reference's KeOps backend, Weighted_Abs_Sum/weighted_abs_sum/keops_backend.py:19-35). Not in the reference's
    pybind module; out_u is None unless full."""
    P, D, N, M, C = _check_qkv(q, k, v)
    lib = _lib.load()
    dev = q.device
    with torch.cuda.device(dev):
        out = torch.empty((P, M, C), dtype=q.dtype, device=dev)
        out_u = torch.empty((P, M), dtype=q.dtype, device=dev) if full else None
        _lib.check(lib.qlka_direct_fwd(0, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out), _lib.ptr(out_u),
                                       P, D, N, M, C, _lib.stream_of(dev)))
    return out, out_u


def weighted_abs_sum_direct_backward(q, k, v, g_w, g_u, tie):
    """Dense backward (qlka_direct_bwd) with sign(0) = tie: tie 0 is the gradient of the KeOps forward
    (keops_backend.py:40-41), tie -1 the walk's convention. g_u may be None. Not in the reference's pybind module."""
    P, D, N, M, C = _check_qkv(q, k, v)
    _check_grad("g_w", g_w, q, (P, M, C))
    if g_u is not None:
        _check_grad("g_u", g_u, q, (P, M))
    lib = _lib.load()
    dev = q.device
    with torch.cuda.device(dev):
        grad_q = torch.empty((P, D, M), dtype=q.dtype, device=dev)
        grad_k = torch.empty((P, D, N), dtype=q.dtype, device=dev)
        grad_v = torch.empty((P, N, C), dtype=q.dtype, device=dev)
        _lib.check(lib.qlka_direct_bwd(float(tie), _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g_w), _lib.ptr(g_u),
                                       _lib.ptr(grad_q), _lib.ptr(grad_k), _lib.ptr(grad_v), P, D, N, M, C,
                                       _lib.stream_of(dev)))
    return grad_q, grad_k, grad_v


def weighted_sgn_sum_direct(q, k, v, g, tie):
    """Dense weighted_sgn_sum (qlka_direct_sgn) with sign(0) = tie (0: keops_backend.py:38-48). Not in the
    reference's pybind module."""
    P, D, N, M, C = _check_qkv(q, k, v)
    _check_grad("g", g, q, (P, M, C))
    lib = _lib.load()
    dev = q.device
    with torch.cuda.device(dev):
        out = torch.empty((P, D, M), dtype=q.dtype, device=dev)
        _lib.check(lib.qlka_direct_sgn(float(tie), _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(out),
                                       P, D, N, M, C, _lib.stream_of(dev)))
    return out


def _backward(q, k, v, g_w, g_u):
    P, D, N, M, C = _check_qkv(q, k, v)
    _check_grad("g_w", g_w, q, (P, M, C))
    if g_u is not None:
        _check_grad("g_u", g_u, q, (P, M))
    lib = _lib.load()
    dev = q.device
    with torch.cuda.device(dev):
        grad_q = torch.empty((P, D, M), dtype=q.dtype, device=dev)
        grad_k = torch.empty((P, D, N), dtype=q.dtype, device=dev)
        grad_v = torch.empty((P, N, C), dtype=q.dtype, device=dev)
        ws = _lib.workspace(lib.qlka_abs_bwd_ws_bytes(P, D, N, M, C), dev)
        _lib.check(lib.qlka_abs_bwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g_w), _lib.ptr(g_u),
                                    _lib.ptr(grad_q), _lib.ptr(grad_k), _lib.ptr(grad_v),
                                    P, D, N, M, C, _lib.ptr(ws), ws.numel(), _lib.stream_of(dev)))
    return grad_q, grad_k, grad_v


def weighted_abs_sum_backward(q, k, v, g_w):
    """(grad_q, grad_k, grad_v) of weighted_abs_sum  (Weighted_Abs_Sum/csrc/binding.cpp:370-374)."""
    return _backward(q, k, v, g_w, None)


def weighted_abs_sum_full_backward(q, k, v, g_w, g_u):
    """(grad_q, grad_k, grad_v) of weighted_abs_sum_full  (Weighted_Abs_Sum/csrc/binding.cpp:376-380)."""
    return _backward(q, k, v, g_w, g_u)


def weighted_sgn_sum_forward(q, k, v, g):
    """out[p,d,m] = sum_n sgn(k[p,d,n] - q[p,d,m]) * dot(v[p,n,:], g[p,m,:]), a tie counted +1
    (Weighted_Abs_Sum/csrc/binding.cpp:383-439)."""
    P, D, N, M, C = _check_qkv(q, k, v)
    _check_grad("g", g, q, (P, M, C))
    lib = _lib.load()
    dev = q.device
    with torch.cuda.device(dev):
        out = torch.empty((P, D, M), dtype=q.dtype, device=dev)
        ws = _lib.workspace(lib.qlka_sgn_fwd_ws_bytes(P, D, N, M, C), dev)
        _lib.check(lib.qlka_sgn_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(out),
                                    P, D, N, M, C, _lib.ptr(ws), ws.numel(), _lib.stream_of(dev)))
    return out
