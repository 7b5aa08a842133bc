"""Native entry point of weighted_laplace_sum with the name, checks and messages of the reference's pybind module
(Weighted_Laplace_Sum/csrc/binding.cpp:63-105), implemented over libqlka.so's C ABI."""

import torch

from qlka import _lib


def weighted_laplace_sum_forward(q, k, v):
    """(out_w, out_u): out_w[p,m,c] = sum_{d,n} exp(-|k[p,d,n] - q[p,d,m]|) v[p,n,c],
    out_u[p,m] = sum_{d,n} exp(-|k[p,d,n] - q[p,d,m]|)."""
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError("q, k and v must be CUDA tensors")
    if not (q.device == k.device and q.device == v.device):
        raise RuntimeError("q, k and v must be on one device")
    if not (q.dtype == torch.float32 and k.dtype == torch.float32 and v.dtype == torch.float32):
        raise RuntimeError("q, k and v must be float32")
    if not (q.dim() == 3 and k.dim() == 3 and v.dim() == 3):
        raise RuntimeError("q, k and v must be 3D")
    if not (q.size(0) == k.size(0) and q.size(0) == v.size(0)):
        raise RuntimeError("batch size must match")
    if q.size(1) != k.size(1):
        raise RuntimeError("q and k must have the same feature dimension")
    if k.size(2) != v.size(1):
        raise RuntimeError("k and v must have the same length")
    if not (q.is_contiguous() and k.is_contiguous() and v.is_contiguous()):
        raise RuntimeError("q, k and v must be contiguous")
    P, D, N, C, M = q.size(0), q.size(1), k.size(2), v.size(2), q.size(2)
    if not (M > 0 and N > 0 and D > 0):
        raise RuntimeError("N, M and D must be > 0")
    if not (1 <= C <= 128):
        raise RuntimeError("C (v.size(2)) must be in [1, 128]")
    if not (N <= 131072 and M <= 131072):
        raise RuntimeError("N and M must be <= 131072")
    if P * D * max(N, M) > 2 ** 31 - 1:
        raise RuntimeError("P*D*max(N,M) must fit int32 (cub sort offsets)")
    lib = _lib.load()
    dev = q.device
    with torch.cuda.device(dev):
        out = torch.empty((P, M, C), dtype=q.dtype, device=dev)
        out_u = torch.empty((P, M), dtype=q.dtype, device=dev)
        ws = _lib.workspace(lib.qlka_laplace_fwd_ws_bytes(P, D, N, M, C), dev)
        _lib.check(lib.qlka_laplace_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out), _lib.ptr(out_u),
                                        P, D, N, M, C, _lib.ptr(ws), ws.numel(), _lib.stream_of(dev)))
    return out, out_u
