"""Torch wrappers of the C ABI's test entry points: the segmented sort and the merge rank used inside both operators.

They exist so tests can check stage 1 (sort) and stage 2 (merge rank) bit-exactly against numpy
(np.argsort(kind="stable"), np.searchsorted(side="left")).
"""

import torch

from . import _lib


def _check_segments(x, name):
    if not x.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if x.dtype != torch.float32:
        raise RuntimeError(f"{name} must be float32")
    if not x.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if x.dim() < 1 or x.numel() == 0:
        raise RuntimeError(f"{name} must be non-empty")


def seg_sort(keys):
    """Stable ascending sort along the last dim of `keys` (any leading shape). Returns (sorted, perm int64)."""
    _check_segments(keys, "keys")
    L = keys.shape[-1]
    S = keys.numel() // L
    lib = _lib.load()
    out = torch.empty_like(keys)
    perm = torch.empty(keys.shape, dtype=torch.int32, device=keys.device)
    with torch.cuda.device(keys.device):
        ws = _lib.workspace(lib.qlka_seg_sort_ws_bytes(S, L), keys.device)
        _lib.check(lib.qlka_seg_sort(_lib.ptr(keys), _lib.ptr(out), _lib.ptr(perm), S, L,
                                     _lib.ptr(ws), ws.numel(), _lib.stream_of(keys.device)))
    return out, perm.to(torch.int64)


def merge_rank(q, k):
    """rank[..., m] = #{n : k[..., n] < q[..., m]} per segment (leading dims of q and k must match)."""
    _check_segments(q, "q")
    _check_segments(k, "k")
    if q.shape[:-1] != k.shape[:-1]:
        raise RuntimeError("q and k must have the same leading (segment) shape")
    M, N = q.shape[-1], k.shape[-1]
    S = q.numel() // M
    lib = _lib.load()
    rank = torch.empty(q.shape, dtype=torch.int32, device=q.device)
    with torch.cuda.device(q.device):
        ws = _lib.workspace(lib.qlka_merge_rank_ws_bytes(S, N, M), q.device)
        _lib.check(lib.qlka_merge_rank(_lib.ptr(q), _lib.ptr(k), _lib.ptr(rank), S, N, M,
                                       _lib.ptr(ws), ws.numel(), _lib.stream_of(q.device)))
    return rank.to(torch.int64)
