"""fp64 brute-force oracle of the hot path. TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Every function evaluates its definition directly, term by term, in float64 (no sorting, no recurrence), except the
`*_sorted` functions, which are a second, independent formulation (sort + prefix sums, the identity stated at
Weighted_Abs_Sum/csrc/abs_kernels.cu:9-19) used only to pin the brute force in tests/test_oracle.py.

Layouts are the reference's: q (P, D, M), k (P, D, N), v (P, N, C), g (P, M, C), g_u (P, M).
`qidx` (optional, int array (P, Mq)) restricts the evaluation to a subsample of queries of each p.
`keep` (optional, (P, N), nonzero = kept) drops the masked keys from every sum (the in-kernel key mask); it is pinned
by the reference's own composition over zeroed keys: k * keep, v * keep and the n_pad correction of u
(attention.py:122-124, weighted_laplace_sum/__init__.py:12), a different computation of the same value.

Function                       reference                                                     pinned by (tests/test_oracle.py)
abs_sum                        ops.py:107-126, keops_backend.py:19-36                          sorted-prefix closed form, N=1 / D=1 cases,
                                                                                               v==1 -> out_w == out_u, translation, linearity
laplace_sum                    weighted_laplace_sum/__init__.py:4-13, laplace_kernels.cu:5-29   fp64 two-sided recurrence (pure Python),
                                                                                               single key, ties -> 1, underflow, v==1
sgn_sum                        ops.py:129-139, binding.cpp:383-439 (tie +1), keops 40-41 (0)    hand-built ties, == -grad_q, autograd
abs_backward                   binding.cpp:242-380, sgn_kernels.cu:8-15 (tie -1; keops: 0)      torch.autograd.gradcheck of a dense fp64
                                                                                               forward (tie-free), grad_v == abs_sum(k, q, g_w)
stable_sort / merge_rank       sort_utils.cu:85-87, walk_common.cuh:10-20                       pure-Python stable sort / brute-force counts
grad_q_fp32_prefix             sgn_kernels.cu:8-15, binding.cpp:242-262 (the reference's fp32   equals abs_backward's grad_q to fp32 rounding;
                               prefix-sum composition of grad_q, tie -1)                        its error against it is reported, not a bar
"""

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
from threadpoolctl import threadpool_limits


def _map(fn, n):
    """[fn(i) for i in range(n)], run on a thread pool (numpy's array loops release the GIL, so the per-p work of a
    large check runs on all host cores); results in index order."""
    workers = min(n, os.cpu_count() or 1, 16)
    if workers <= 1:
        return [fn(i) for i in range(n)]
    # one BLAS thread per worker: nested BLAS thread pools oversubscribe the cores (and OpenBLAS then spins)
    with threadpool_limits(limits=1), ThreadPoolExecutor(workers) as ex:
        return list(ex.map(fn, range(n)))


def _f64(x):
    return np.asarray(x, dtype=np.float64)


def _pairwise(qp, kp, fn):
    """sum_d fn(q[d, m] - k[d, n]) as an (Mq, N) fp64 matrix; qp (D, Mq), kp (D, N)."""
    out = np.zeros((qp.shape[1], kp.shape[1]), dtype=np.float64)
    for d in range(qp.shape[0]):
        out += fn(qp[d][:, None] - kp[d][None, :])
    return out


def _select(q, qidx):
    q = _f64(q)
    if qidx is None:
        return q, None
    qidx = np.asarray(qidx)
    return np.stack([q[p][:, qidx[p]] for p in range(q.shape[0])]), qidx


def _kept(keep, p, N):
    return np.ones(N, dtype=np.float64) if keep is None else (np.asarray(keep[p]) != 0).astype(np.float64)


def abs_sum(q, k, v, qidx=None, keep=None):
    """(out_w, out_u, norm_w): out_w[p,m,c] = sum_{d,n} |k[p,d,n] - q[p,d,m]| v[p,n,c], out_u[p,m] = sum_{d,n} |k-q|,
    norm_w[p,m,c] = sum_{d,n} |k - q| |v[p,n,c]| (the per-element error normaliser); n over the kept keys."""
    qs, _ = _select(q, qidx)
    k, v = _f64(k), _f64(v)

    def one(p):
        A = _pairwise(qs[p], k[p], np.abs) * _kept(keep, p, k.shape[2])[None, :]
        return A @ v[p], A.sum(axis=1), A @ np.abs(v[p])

    out_w, out_u, norm = zip(*_map(one, qs.shape[0]))
    return np.stack(out_w), np.stack(out_u), np.stack(norm)


def laplace_sum(q, k, v, qidx=None, keep=None):
    """(out_w, out_u, norm_w) with the Laplace kernel exp(-|k - q|) in place of |k - q|; n over the kept keys."""
    qs, _ = _select(q, qidx)
    k, v = _f64(k), _f64(v)

    def one(p):
        A = _pairwise(qs[p], k[p], lambda x: np.exp(-np.abs(x))) * _kept(keep, p, k.shape[2])[None, :]
        return A @ v[p], A.sum(axis=1), A @ np.abs(v[p])

    out_w, out_u, norm = zip(*_map(one, qs.shape[0]))
    return np.stack(out_w), np.stack(out_u), np.stack(norm)


def _sgn(x, tie):
    s = np.sign(x)
    s[x == 0] = tie
    return s


def sgn_sum(q, k, v, g, tie=1.0, qidx=None):
    """(out, norm): out[p,d,m] = sum_n sgn(k[p,d,n] - q[p,d,m]) <v[p,n,:], g[p,m,:]> with sgn(0) = tie
    (+1 for the reference's CUDA walk, 0 for its keops backend); norm[p,d,m] = sum_{n,c} |v[p,n,c] g[p,m,c]|, the sum
    of |term| over the elementary products (a dot product's own cancellation is fp32 rounding of the sum, not of its
    terms)."""
    qs, qidx = _select(q, qidx)
    k, v, g = _f64(k), _f64(v), _f64(g)
    P, D = qs.shape[0], qs.shape[1]
    out = np.zeros((P, D, qs.shape[2]))
    norm = np.zeros_like(out)
    for p in range(P):
        gp = g[p] if qidx is None else g[p][qidx[p]]
        Bm = gp @ v[p].T                                   # (Mq, N) = <g_m, v_n>
        Ba = np.abs(gp) @ np.abs(v[p]).T                   # (Mq, N) = sum_c |g_mc v_nc|
        for d in range(D):
            S = _sgn(k[p, d][None, :] - qs[p, d][:, None], tie)
            out[p, d] = (S * Bm).sum(axis=1)
            norm[p, d] = Ba.sum(axis=1)
    return out, norm


def abs_backward(q, k, v, g_w, g_u=None, tie=-1.0):
    """(grad_q, grad_k, grad_v) of weighted_abs_sum(_full): the derivative of |k - q| w.r.t. q is s(q - k) and w.r.t.
    k is s(k - q), with s(x) = sign(x) and s(0) = tie. tie = -1 is the reference CUDA extension's convention
    (sgn_kernels.cu:8-15, binding.cpp:242-245), tie = 0 the gradient of the KeOps forward (keops_backend.py:40-41).
    Also returns the normalisers (nq, nk, nv): the sums of |term| over the elementary terms, s g_mc v_nc and s g_um for
    grad_q / grad_k, |k - q| g_mc for grad_v."""
    q, k, v, g_w = _f64(q), _f64(k), _f64(v), _f64(g_w)
    g_u = None if g_u is None else _f64(g_u)
    P, D, M = q.shape
    N = k.shape[2]
    gq = np.zeros((P, D, M)); nq = np.zeros_like(gq)
    gk = np.zeros((P, D, N)); nk = np.zeros_like(gk)
    for p in range(P):
        Bm = g_w[p] @ v[p].T                               # (M, N)
        Ba = np.abs(g_w[p]) @ np.abs(v[p]).T               # sum_c |g_mc v_nc|
        if g_u is not None:
            Bm = Bm + g_u[p][:, None]
            Ba = Ba + np.abs(g_u[p])[:, None]
        for d in range(D):
            x = q[p, d][:, None] - k[p, d][None, :]        # (M, N) = q_m - k_n
            sq = np.where(x > 0, 1.0, np.where(x < 0, -1.0, tie))     # s(q - k)
            sk = np.where(x < 0, 1.0, np.where(x > 0, -1.0, tie))     # s(k - q)
            gq[p, d] = (sq * Bm).sum(axis=1)
            gk[p, d] = (sk * Bm).sum(axis=0)
            nq[p, d] = Ba.sum(axis=1)
            nk[p, d] = Ba.sum(axis=0)
    gv, _, nv = abs_sum(k, q, g_w)                         # grad_v = sum_{d,m} |k_n - q_m| g_w[m, :]
    return (gq, gk, gv), (nq, nk, nv)


def grad_q_fp32_prefix(q, k, v, g_w, g_u=None):
    """grad_q as the reference's CUDA walk composes it, in float32 (sgn_kernels.cu:8-15, binding.cpp:242-262): per
    feature, v summed in the keys' sorted order into prefix rows PW_r (float32, one key after the other), and for a
    query of rank r = #{k < q} (a tie counts as a key above: s(0) = -1) grad_q = <g_m, 2 PW_r - W_tot>
    (+ g_u (2 r - N)), the vector expression and the dot product in float32. Its error against the fp64
    abs_backward is the rounding an fp32 implementation of this composition carries; the library's own error is held
    to a small multiple of it."""
    q, k, v, g_w = (np.asarray(a, dtype=np.float32) for a in (q, k, v, g_w))
    g_u = None if g_u is None else np.asarray(g_u, dtype=np.float32)
    P, D, M = q.shape
    N = k.shape[2]
    out = np.zeros((P, D, M), dtype=np.float32)
    for p in range(P):
        for d in range(D):
            order = np.argsort(k[p, d], kind="stable")
            pw = np.zeros((N + 1, v.shape[2]), dtype=np.float32)
            pw[1:] = np.cumsum(v[p][order], axis=0, dtype=np.float32)
            r = np.searchsorted(k[p, d][order], q[p, d], side="left")
            t = np.float32(2.0) * pw[r] - pw[N]
            out[p, d] = np.einsum("mc,mc->m", g_w[p], t, dtype=np.float32)
            if g_u is not None:
                out[p, d] += g_u[p] * (np.float32(2.0) * r.astype(np.float32) - np.float32(N))
    return out


def dot_normaliser(v, g_w, g_u=None):
    """(P, M): sum_n |<g_m, v_n> (+ g_um)|, the per-key magnitude of grad_q's terms (the normaliser of the backward
    before the elementary-product one of abs_backward; tighter when a C-channel dot product cancels)."""
    v, g_w = _f64(v), _f64(g_w)
    B = np.einsum("pmc,pnc->pmn", g_w, v)
    if g_u is not None:
        B = B + _f64(g_u)[:, :, None]
    return np.abs(B).sum(axis=2)


def abs_backward_sub(q, k, v, g_w, g_u, qidx, kidx):
    """abs_backward restricted to subsamples: grad_q / nq for the queries qidx (P, mq), grad_k / nk and grad_v / nv
    for the keys kidx (P, nk); every term still runs over all keys (grad_q) or all queries (grad_k, grad_v)."""
    q, k, v, g_w = _f64(q), _f64(k), _f64(v), _f64(g_w)
    g_u = None if g_u is None else _f64(g_u)
    P, D, M = q.shape
    C = v.shape[2]
    mq, nk_ = qidx.shape[1], kidx.shape[1]
    gq = np.zeros((P, D, mq)); nq = np.zeros_like(gq)
    gk = np.zeros((P, D, nk_)); nk = np.zeros_like(gk)
    gv = np.zeros((P, nk_, C)); nv = np.zeros_like(gv)

    def one(p):                                           # writes only the slices of p
        qi, ki = qidx[p], kidx[p]
        Bq = g_w[p][qi] @ v[p].T                          # (mq, N)
        Bk = g_w[p] @ v[p][ki].T                          # (M, nk)
        Aq = np.abs(g_w[p][qi]) @ np.abs(v[p]).T          # elementary-term normalisers
        Ak = np.abs(g_w[p]) @ np.abs(v[p][ki]).T
        if g_u is not None:
            Bq = Bq + g_u[p][qi][:, None]
            Bk = Bk + g_u[p][:, None]
            Aq = Aq + np.abs(g_u[p][qi])[:, None]
            Ak = Ak + np.abs(g_u[p])[:, None]
        for d in range(D):
            xq = q[p, d][qi][:, None] - k[p, d][None, :]  # (mq, N)
            gq[p, d] = (np.where(xq > 0, 1.0, -1.0) * Bq).sum(axis=1)
            nq[p, d] = Aq.sum(axis=1)
            xk = k[p, d][ki][None, :] - q[p, d][:, None]  # (M, nk) = k_n - q_m
            gk[p, d] = (np.where(xk > 0, 1.0, -1.0) * Bk).sum(axis=0)
            nk[p, d] = Ak.sum(axis=0)
            A = np.abs(xk)                                # |k_n - q_m|
            gv[p] += A.T @ g_w[p]
            nv[p] += A.T @ np.abs(g_w[p])

    _map(one, P)
    return (gq, gk, gv), (nq, nk, nv)


# ------------------------------------------------------------------------------------------- sort / rank contracts
def stable_sort(x):
    """(sorted, perm) along the last axis: np.argsort(kind="stable") on the fp32 values, -0.0 == +0.0, sorted values
    written as +0.0 for -0.0 (the CUB contract at Weighted_Abs_Sum/csrc/sort_utils.cu:85-87)."""
    x = np.asarray(x, dtype=np.float32)
    flat = x.reshape(-1, x.shape[-1])
    perm = np.empty(flat.shape, dtype=np.int64)
    chunk = max(1, (flat.shape[0] + 15) // 16)

    def one(i):                                           # rows [i * chunk, (i + 1) * chunk)
        r = slice(i * chunk, (i + 1) * chunk)
        perm[r] = np.argsort(flat[r], axis=-1, kind="stable")

    _map(one, (flat.shape[0] + chunk - 1) // chunk)
    perm = perm.reshape(x.shape)
    srt = np.take_along_axis(x, perm, axis=-1) + np.float32(0.0)   # -0.0 + 0.0 == +0.0
    return srt, perm


def merge_rank(q, k):
    """rank[..., m] = #{n : k[..., n] < q[..., m]} = np.searchsorted(sorted(k), q, side="left")."""
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    flat_q = q.reshape(-1, q.shape[-1])
    flat_k = k.reshape(-1, k.shape[-1])
    out = _map(lambda i: np.searchsorted(np.sort(flat_k[i]), flat_q[i], side="left"), flat_q.shape[0])
    return np.stack(out).reshape(q.shape)


# ------------------------------------------------------------------------------ independent formulation (pinning)
def abs_sum_sorted(q, k, v):
    """Second formulation of abs_sum through sorting + prefix sums (abs_kernels.cu:9-12):
    sum_n |k_n - q| v_n = 2 (q PV_r - PK_r) + K_tot - q V_tot with r = #{k < q}. fp64, all queries."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    P, D, M = q.shape
    C = v.shape[2]
    out_w = np.zeros((P, M, C))
    out_u = np.zeros((P, M))
    for p in range(P):
        for d in range(D):
            order = np.argsort(k[p, d], kind="stable")
            ks = k[p, d][order]
            vs = v[p][order]
            PV = np.vstack([np.zeros((1, C)), np.cumsum(vs, axis=0)])
            PK = np.vstack([np.zeros((1, C)), np.cumsum(ks[:, None] * vs, axis=0)])
            PKu = np.concatenate([[0.0], np.cumsum(ks)])
            r = np.searchsorted(ks, q[p, d], side="left")
            qq = q[p, d][:, None]
            out_w[p] += 2 * (qq * PV[r] - PK[r]) + PK[-1][None, :] - qq * PV[-1][None, :]
            out_u[p] += 2 * (q[p, d] * r - PKu[r]) + PKu[-1] - q[p, d] * len(ks)
    return out_w, out_u


def laplace_sum_recurrence(q, k, v):
    """Second formulation of laplace_sum: per (p, d) the two-sided decayed recurrences over sorted keys,
    L_j = e^{-(k_j - k_{j-1})} L_{j-1} + v_j and R_j = v_j + e^{-(k_{j+1} - k_j)} R_{j+1}, a query of rank r getting
    e^{-(q - k_{r-1})} L_{r-1} + e^{-(k_r - q)} R_r (laplace_kernels.cu:7-12). Pure-Python loops: tiny sizes only."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    P, D, M = q.shape
    N, C = v.shape[1], v.shape[2]
    out_w = np.zeros((P, M, C))
    out_u = np.zeros((P, M))
    for p in range(P):
        for d in range(D):
            order = np.argsort(k[p, d], kind="stable")
            ks = k[p, d][order]
            vs = np.hstack([v[p][order], np.ones((N, 1))])
            L = np.zeros((N, C + 1))
            R = np.zeros((N, C + 1))
            for j in range(N):
                L[j] = vs[j] + (np.exp(-(ks[j] - ks[j - 1])) * L[j - 1] if j > 0 else 0.0)
            for j in range(N - 1, -1, -1):
                R[j] = vs[j] + (np.exp(-(ks[j + 1] - ks[j])) * R[j + 1] if j < N - 1 else 0.0)
            for m in range(M):
                x = q[p, d, m]
                r = int(np.searchsorted(ks, x, side="left"))
                acc = np.zeros(C + 1)
                if r > 0:
                    acc += np.exp(-(x - ks[r - 1])) * L[r - 1]
                if r < N:
                    acc += np.exp(-(ks[r] - x)) * R[r]
                out_w[p, m] += acc[:C]
                out_u[p, m] += acc[C]
    return out_w, out_u


def rel_err(got, want, norm, floor=1e-30):
    """Per-element |got - want| / norm (norm = sum of |term|), the BASELINE.json error measure."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    norm = np.asarray(norm, dtype=np.float64)
    return np.abs(got - want) / np.maximum(norm, floor)
