"""Pins the CPU oracle (oracle/brute.py) before it is trusted as the parity checker.

The reference ships no tests, fixtures or golden vectors for this path, so every oracle function is pinned by an
independent formulation, closed forms, invariants and brute force on tiny inputs, each chosen so a plausible mistake
(a dropped term, a wrong sign or index, a transposed operand, the wrong tie rule) fails at least one check.
"""

import numpy as np
import pytest
import torch

from oracle import brute, dense, inputs


def _rand(P=2, D=3, N=7, M=5, C=4, seed=0, ties=False):
    rng = np.random.default_rng(seed)
    if ties:
        q = rng.integers(-3, 4, size=(P, D, M)).astype(np.float32) / 2
        k = rng.integers(-3, 4, size=(P, D, N)).astype(np.float32) / 2
    else:
        q = rng.standard_normal((P, D, M)).astype(np.float32)
        k = rng.standard_normal((P, D, N)).astype(np.float32)
    v = rng.standard_normal((P, N, C)).astype(np.float32)
    return q, k, v


# ------------------------------------------------------------------------------------------------------- abs sum
@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("shape", [(2, 3, 7, 5, 4), (1, 1, 1, 1, 1), (3, 2, 9, 13, 3)])
def test_abs_brute_matches_sorted_prefix_form(shape, ties):
    P, D, N, M, C = shape
    q, k, v = _rand(P, D, N, M, C, ties=ties)
    w, u, _ = brute.abs_sum(q, k, v)
    w2, u2 = brute.abs_sum_sorted(q, k, v)
    np.testing.assert_allclose(w, w2, rtol=1e-12, atol=1e-10)
    np.testing.assert_allclose(u, u2, rtol=1e-12, atol=1e-10)


def test_abs_hand_computed():
    # P=1, D=2, keys (0,2) and (1,-1), queries (1, 0): sum_d |k_d - q_d| per key, times v
    q = np.array([[[1.0], [0.0]]], dtype=np.float32)               # (1, 2, 1)
    k = np.array([[[0.0, 2.0], [1.0, -1.0]]], dtype=np.float32)    # (1, 2, 2)
    v = np.array([[[1.0, 10.0], [2.0, 20.0]]], dtype=np.float32)   # (1, 2, 2)
    # key 0: |0-1| + |1-0| = 2 ; key 1: |2-1| + |-1-0| = 2
    w, u, _ = brute.abs_sum(q, k, v)
    np.testing.assert_allclose(w[0, 0], [2 * 1 + 2 * 2, 2 * 10 + 2 * 20])
    np.testing.assert_allclose(u[0, 0], 4.0)


def test_abs_invariants():
    q, k, v = _rand(2, 4, 11, 6, 3, seed=3)
    w, u, _ = brute.abs_sum(q, k, v)
    # v == 1 -> every channel equals out_u
    w1, u1, _ = brute.abs_sum(q, k, np.ones_like(v))
    np.testing.assert_allclose(w1, np.repeat(u1[:, :, None], 3, axis=2), rtol=1e-12)
    # translation invariance
    wt, ut, _ = brute.abs_sum(q + 5.0, k + 5.0, v)
    np.testing.assert_allclose(wt, w, rtol=1e-5, atol=1e-5)
    # linearity in v
    w2, _, _ = brute.abs_sum(q, k, 2 * v.astype(np.float64) + 1)
    np.testing.assert_allclose(w2, 2 * w + w1, rtol=1e-10, atol=1e-9)
    # symmetry: swapping the roles of q and k transposes the distance matrix
    A = np.zeros((2, 6, 11))
    for d in range(4):
        A += np.abs(q[:, d, :, None].astype(np.float64) - k[:, d, None, :])
    np.testing.assert_allclose(u, A.sum(axis=2), rtol=1e-12)


def test_abs_subsample_matches_full():
    q, k, v = _rand(2, 3, 20, 17, 5, seed=4)
    idx = inputs.query_subsample(2, 17, per_p=6, seed=9)
    w, u, n = brute.abs_sum(q, k, v)
    ws, us, ns = brute.abs_sum(q, k, v, qidx=idx)
    for p in range(2):
        np.testing.assert_allclose(ws[p], w[p][idx[p]])
        np.testing.assert_allclose(us[p], u[p][idx[p]])
        np.testing.assert_allclose(ns[p], n[p][idx[p]])


# ---------------------------------------------------------------------------------------------------- laplace sum
@pytest.mark.parametrize("ties", [False, True])
def test_laplace_brute_matches_recurrence(ties):
    q, k, v = _rand(2, 3, 9, 7, 3, seed=5, ties=ties)
    w, u, _ = brute.laplace_sum(q, k, v)
    w2, u2 = brute.laplace_sum_recurrence(q, k, v)
    np.testing.assert_allclose(w, w2, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(u, u2, rtol=1e-12, atol=1e-12)


def test_laplace_special_cases():
    # single key: out_u = sum_d exp(-|k_d - q_d|)
    q = np.array([[[0.5, -1.0], [2.0, 0.0]]], dtype=np.float32)     # (1, 2, 2)
    k = np.array([[[0.0], [1.0]]], dtype=np.float32)                # (1, 2, 1)
    v = np.array([[[3.0]]], dtype=np.float32)
    w, u, _ = brute.laplace_sum(q, k, v)
    want = np.exp(-np.abs(k[0, :, 0][:, None].astype(np.float64) - q[0])).sum(axis=0)
    np.testing.assert_allclose(u[0], want, rtol=1e-12)
    np.testing.assert_allclose(w[0, :, 0], 3.0 * want, rtol=1e-12)
    # exact ties give exp(0) = 1 per feature
    qt = np.zeros((1, 3, 1), np.float32)
    kt = np.zeros((1, 3, 4), np.float32)
    _, ut, _ = brute.laplace_sum(qt, kt, np.ones((1, 4, 1), np.float32))
    np.testing.assert_allclose(ut, [[12.0]])
    # a huge spread underflows to 0, never NaN
    qf = np.full((1, 1, 1), 1e4, np.float32)
    kf = np.zeros((1, 1, 2), np.float32)
    wf, uf, _ = brute.laplace_sum(qf, kf, np.ones((1, 2, 2), np.float32))
    assert np.all(wf == 0) and np.all(uf == 0) and not np.isnan(wf).any()
    # v == 1 -> out_w channels == out_u
    q2, k2, v2 = _rand(2, 3, 6, 5, 2, seed=8)
    w1, u1, _ = brute.laplace_sum(q2, k2, np.ones_like(v2))
    np.testing.assert_allclose(w1, np.repeat(u1[:, :, None], 2, axis=2), rtol=1e-12)


def test_laplace_padded_key_identity():
    # a padded key (k = 0, v = 0) adds exp(-|q_d|) per feature to out_u only (__init__.py:12, attention.py:69-71)
    q, k, v = _rand(1, 3, 5, 4, 2, seed=11)
    kp = np.concatenate([k, np.zeros((1, 3, 2), np.float32)], axis=2)
    vp = np.concatenate([v, np.zeros((1, 2, 2), np.float32)], axis=1)
    w, u, _ = brute.laplace_sum(q, k, v)
    wp, up, _ = brute.laplace_sum(q, kp, vp)
    np.testing.assert_allclose(wp, w, rtol=1e-12)
    np.testing.assert_allclose(up - 2 * np.exp(-np.abs(q[0].astype(np.float64))).sum(axis=0), u, rtol=1e-12)


# ------------------------------------------------------------------------------------------------- sgn / backward
def test_sgn_tie_conventions_by_hand():
    # one feature, keys (0, 1, 1, 2), query 1 -> keys below: 0; equal: two 1s; above: 2
    q = np.array([[[1.0]]], np.float32)
    k = np.array([[[0.0, 1.0, 1.0, 2.0]]], np.float32)
    v = np.array([[[1.0], [10.0], [100.0], [1000.0]]], np.float32)
    g = np.ones((1, 1, 1), np.float32)
    plus, _ = brute.sgn_sum(q, k, v, g, tie=1.0)       # CUDA walk: tie +1
    zero, _ = brute.sgn_sum(q, k, v, g, tie=0.0)       # keops: tie 0
    assert plus[0, 0, 0] == -1 + 10 + 100 + 1000
    assert zero[0, 0, 0] == -1 + 1000
    (gq, gk, _), _ = brute.abs_backward(q, k, v, g)
    assert gq[0, 0, 0] == -plus[0, 0, 0]                # sgn op == -grad_q (binding.cpp:383,438)
    # grad_k[n] = sum_m s(k_n - q_m) <g_m, v_n>, tie -1
    np.testing.assert_array_equal(gk[0, 0], [-1.0, -10.0, -100.0, 1000.0])


def test_sgn_is_negated_grad_q_random():
    q, k, v = _rand(2, 3, 8, 6, 4, seed=12, ties=True)
    g = np.random.default_rng(1).standard_normal((2, 6, 4)).astype(np.float32)
    s, _ = brute.sgn_sum(q, k, v, g, tie=1.0)
    (gq, _, _), _ = brute.abs_backward(q, k, v, g)
    np.testing.assert_allclose(s, -gq, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("full", [False, True])
def test_backward_matches_autograd(full):
    P, D, N, M, C = 2, 3, 6, 5, 2
    q, k, v = _rand(P, D, N, M, C, seed=13)
    rng = np.random.default_rng(2)
    g_w = rng.standard_normal((P, M, C)).astype(np.float32)
    g_u = rng.standard_normal((P, M)).astype(np.float32) if full else None
    tq = torch.tensor(q, dtype=torch.float64, requires_grad=True)
    tk = torch.tensor(k, dtype=torch.float64, requires_grad=True)
    tv = torch.tensor(v, dtype=torch.float64, requires_grad=True)
    d1 = (tq.unsqueeze(3) - tk.unsqueeze(2)).abs().sum(dim=1)      # (P, M, N)
    loss = ((d1 @ tv) * torch.tensor(g_w, dtype=torch.float64)).sum()
    if full:
        loss = loss + (d1.sum(-1) * torch.tensor(g_u, dtype=torch.float64)).sum()
    loss.backward()
    (gq, gk, gv), _ = brute.abs_backward(q, k, v, g_w, g_u)
    np.testing.assert_allclose(gq, tq.grad.numpy(), rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(gk, tk.grad.numpy(), rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(gv, tv.grad.numpy(), rtol=1e-10, atol=1e-10)


def test_dense_forward_gradcheck():
    # the dense fp64 forward the backward oracle is checked against is itself differentiable-correct (tie-free)
    P, D, N, M, C = 1, 2, 4, 3, 2
    q, k, v = _rand(P, D, N, M, C, seed=14)
    args = [torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (q, k, v)]

    def f(tq, tk, tv):
        return dense.dense_abs_sum(tq, tk, tv)
    assert torch.autograd.gradcheck(f, args)


# ------------------------------------------------------------------------------------------------ sort / rank
def test_stable_sort_matches_python_sort():
    x = np.array([[1.0, -0.0, 0.0, -1.0, 1.0, 0.0, -0.0, 2.0, -1.0]], np.float32)
    srt, perm = brute.stable_sort(x)
    py = sorted(range(x.shape[1]), key=lambda i: (float(x[0, i]), i))   # Python's sort is stable; -0.0 == 0.0
    np.testing.assert_array_equal(perm[0], py)
    assert not np.signbit(srt).any() or np.all(srt[np.signbit(srt)] < 0)   # no -0.0 in the output


def test_merge_rank_brute_force():
    rng = np.random.default_rng(3)
    k = rng.integers(-5, 6, size=(3, 40)).astype(np.float32)
    q = rng.integers(-6, 7, size=(3, 25)).astype(np.float32)
    r = brute.merge_rank(q, k)
    want = (k[:, None, :] < q[:, :, None]).sum(axis=2)
    np.testing.assert_array_equal(r, want)


# ------------------------------------------------------------------------------------------ dense (reference) path
def test_dense_ops_match_brute():
    q, k, v = _rand(2, 3, 9, 7, 4, seed=15)
    tq, tk, tv = (torch.tensor(a, dtype=torch.float64) for a in (q, k, v))
    w, u = dense.dense_abs_sum(tq, tk, tv)
    bw, bu, _ = brute.abs_sum(q, k, v)
    np.testing.assert_allclose(w.numpy(), bw, rtol=1e-12)
    np.testing.assert_allclose(u.numpy(), bu, rtol=1e-12)
    w, u = dense.dense_laplace_sum(tq, tk, tv)
    bw, bu, _ = brute.laplace_sum(q, k, v)
    np.testing.assert_allclose(w.numpy(), bw, rtol=1e-12)
    np.testing.assert_allclose(u.numpy(), bu, rtol=1e-12)


@pytest.mark.parametrize("kernel", ["add_laplace", "add_riesz", "add_bump"])
def test_layer_epilogues_match_kernel_matrix(kernel):
    # attention() over the fast ops (here: the dense ops) equals the normalised naive kernel matrix (attention.py:29)
    B, H, S, D = 1, 2, 6, 3
    g = torch.Generator().manual_seed(0)
    q = torch.randn(B, H, S, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, H, S, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, H, S, D, generator=g, dtype=torch.float64)
    tau = dense.TAU[kernel]
    out = dense.attention(q, k, v, kernel, tau, dense.dense_abs_sum, dense.dense_laplace_sum)
    P = B * H
    qq = q.transpose(2, 3).reshape(P, D, S)
    kk = k.transpose(2, 3).reshape(P, D, S)
    vv = v.reshape(P, S, D)
    A = dense.dense_kernel_matrix(kernel, qq, kk, tau)
    ref = (A @ vv) / A.sum(dim=2, keepdim=True).clamp_min(dense.CLAMP)
    np.testing.assert_allclose(out.reshape(P, S, D).numpy(), ref.numpy(), rtol=1e-9, atol=1e-9)


def test_bump_identity():
    x = np.linspace(-3, 3, 61)
    np.testing.assert_allclose(np.maximum(0, 1 - np.abs(x)), np.abs(x + 1) / 2 + np.abs(x - 1) / 2 - np.abs(x),
                               atol=1e-15)


def test_inputs_are_seeded():
    a = inputs.make(2, 3, 5, 4, 2, seed=0, grads=True)
    b = inputs.make(2, 3, 5, 4, 2, seed=0, grads=True)
    for key in a:
        np.testing.assert_array_equal(a[key], b[key])
    m = inputs.make(1, 2, 5000, 10, 2, kind="mixture")
    lv = m["k"][np.abs(m["k"] * 16 - np.round(m["k"] * 16)) == 0]
    assert lv.size > 0.4 * m["k"].size                   # about half the keys sit on the 256 exact levels


def test_backward_subsample_matches_full():
    P, D, N, M, C = 2, 3, 9, 7, 4
    q, k, v = _rand(P, D, N, M, C, seed=16, ties=True)
    rng = np.random.default_rng(5)
    g_w = rng.standard_normal((P, M, C)).astype(np.float32)
    g_u = rng.standard_normal((P, M)).astype(np.float32)
    qidx = np.stack([np.array([0, 3, 6])] * P)
    kidx = np.stack([np.array([1, 2, 8])] * P)
    (fq, fk, fv), (nfq, nfk, nfv) = brute.abs_backward(q, k, v, g_w, g_u)
    (sq, sk, sv), (nsq, nsk, nsv) = brute.abs_backward_sub(q, k, v, g_w, g_u, qidx, kidx)
    np.testing.assert_allclose(sq, fq[:, :, qidx[0]], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(sk, fk[:, :, kidx[0]], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(sv, fv[:, kidx[0]], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(nsq, nfq[:, :, qidx[0]], rtol=1e-12)
    np.testing.assert_allclose(nsv, nfv[:, kidx[0]], rtol=1e-12)


def test_backward_tie_convention():
    # s(0) = tie enters linearly: grad(tie) - grad(-1) = (tie + 1) * (sum of B' over the exact ties), with the tie mass
    # counted here by explicit loops; the KeOps sgn sum is -grad_q at tie 0 (keops_backend.py:38-48)
    rng = np.random.default_rng(21)
    P, D, N, M, C = 2, 3, 9, 7, 4
    q = (rng.integers(-2, 3, size=(P, D, M)) / 2).astype(np.float32)
    k = (rng.integers(-2, 3, size=(P, D, N)) / 2).astype(np.float32)
    v = rng.standard_normal((P, N, C)).astype(np.float32)
    g_w = rng.standard_normal((P, M, C)).astype(np.float32)
    g_u = rng.standard_normal((P, M)).astype(np.float32)
    (q1, k1, v1), _ = brute.abs_backward(q, k, v, g_w, g_u, tie=-1.0)
    tq = np.zeros((P, D, M)); tk = np.zeros((P, D, N))
    for p in range(P):
        for d in range(D):
            for m in range(M):
                for n in range(N):
                    if q[p, d, m] == k[p, d, n]:
                        b = float(np.dot(g_w[p, m].astype(np.float64), v[p, n].astype(np.float64))) + float(g_u[p, m])
                        tq[p, d, m] += b
                        tk[p, d, n] += b
    assert np.abs(tq).sum() > 0, "the inputs must contain ties"
    for tie in (0.0, 0.5, 1.0):
        (qt, kt, vt), _ = brute.abs_backward(q, k, v, g_w, g_u, tie=tie)
        np.testing.assert_allclose(qt - q1, (tie + 1) * tq, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(kt - k1, (tie + 1) * tk, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(vt, v1, rtol=1e-12, atol=1e-12)     # grad_v has no sign
    (q0, _, _), _ = brute.abs_backward(q, k, v, g_w, None, tie=0.0)
    sg, _ = brute.sgn_sum(q, k, v, g_w, tie=0.0)
    np.testing.assert_allclose(sg, -q0, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------------------------------------------- key mask
@pytest.mark.parametrize("op", ["abs", "laplace"])
def test_key_mask_matches_reference_composition(op):
    # The in-kernel mask (masked keys dropped from every sum) against the reference's own route to the same value
    # (attention.py:122-124, weighted_laplace_sum/__init__.py:12): zero k and v at masked keys, sum over all keys, then
    # remove from u what each zeroed key adds, n_pad * sum_d f(q_d - 0). A mask applied to the wrong axis, a dropped
    # n_pad term or a mask that also touched v == 1 sums differently fails here.
    P, D, N, M, C = 3, 4, 23, 11, 5
    q, k, v = _rand(P, D, N, M, C, seed=31)
    keep = np.random.default_rng(32).random((P, N)) < 0.6
    keep[1] = False                       # a p with every key masked
    keep[2] = True                        # a p with none masked
    fn = brute.abs_sum if op == "abs" else brute.laplace_sum
    f = np.abs if op == "abs" else (lambda x: np.exp(-np.abs(x)))
    w, u, _ = fn(q, k, v, keep=keep)
    kz = k * keep[:, None, :]
    vz = v * keep[:, :, None]
    wz, uz, _ = fn(q, kz, vz)
    n_pad = (N - keep.sum(axis=1)).astype(np.float64)
    np.testing.assert_allclose(w, wz, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(u, uz - n_pad[:, None] * f(q.astype(np.float64)).sum(axis=1), rtol=1e-12, atol=1e-9)
    assert np.all(w[1] == 0) and np.all(u[1] == 0)
    w2, u2, _ = fn(q, k, v)
    np.testing.assert_array_equal(w[2], w2[2])
    np.testing.assert_array_equal(u[2], u2[2])


@pytest.mark.parametrize("g_u", [False, True])
def test_grad_q_fp32_prefix_matches_fp64_backward(g_u):
    """The fp32 restatement of the reference's grad_q composition (prefix sums in sorted order, <g, 2 PW - W_tot>)
    equals the fp64 brute force to fp32 rounding, with ties (a tie counts as a key above the query, s(0) = -1: a rank
    taken with side="right" misses here by whole terms)."""
    rng = np.random.default_rng(3)
    P, D, N, M, C = 2, 3, 300, 200, 16
    q = (rng.integers(-20, 21, size=(P, D, M)) / 8).astype(np.float32)     # exact ties between q and k
    k = (rng.integers(-20, 21, size=(P, D, N)) / 8).astype(np.float32)
    v = rng.standard_normal((P, N, C)).astype(np.float32)
    gw = rng.standard_normal((P, M, C)).astype(np.float32)
    gu = rng.standard_normal((P, M)).astype(np.float32) if g_u else None
    got = brute.grad_q_fp32_prefix(q, k, v, gw, gu)
    (want, _, _), _ = brute.abs_backward(q, k, v, gw, gu, tie=-1.0)
    dn = brute.dot_normaliser(v, gw, gu)[:, None, :]
    err = np.abs(got - want) / dn
    assert err.max() < 1e-5
    assert err.max() > 0                                  # an fp32 evaluation, not the fp64 one again


def _merged_walk_backward(q, k, v, g_w, g_u, RK):
    """The abs backward as the GPU's merged walk computes it (csrc/mbw.hip), restated in fp64 for small inputs: per
    (p, d), the sorted queries and keys merged (queries first among equal values), ranges of RK elements, per-range
    summaries, the three scans (abs scan with value-gap links for (PG, B), plain sums for (PW, key count), the tie
    carry E as a linked sum with 0/1 links) and a walk of every range from its entry state."""
    P, D, M = q.shape
    N, C = k.shape[2], v.shape[2]
    q, k, v, g_w = (np.asarray(a, np.float64) for a in (q, k, v, g_w))
    g_u = np.zeros((P, M)) if g_u is None else np.asarray(g_u, np.float64)
    gq, gk, gv = np.zeros((P, D, M)), np.zeros((P, D, N)), np.zeros((P, N, C))
    for p in range(P):
        for d in range(D):
            vals = np.concatenate([q[p, d], k[p, d]])
            isq = np.concatenate([np.ones(M, bool), np.zeros(N, bool)])
            idx = np.concatenate([np.arange(M), np.arange(N)])
            order = np.lexsort((idx, ~isq, vals))               # by value, queries first, then by index (stable)
            vals, isq, idx = vals[order], isq[order], idx[order]
            x = np.where(isq[:, None], g_w[p][np.where(isq, idx, 0)], v[p][np.where(isq, 0, idx)])
            u = np.where(isq, g_u[p][np.where(isq, idx, 0)], 0.0)
            L = N + M
            G = (L + RK - 1) // RK
            rng_ = [(g * RK, min(L, (g + 1) * RK)) for g in range(G)]
            # entry states of every range (row G: the totals)
            PG, B, PW, E = np.zeros((G + 1, C)), np.zeros((G + 1, C)), np.zeros((G + 1, C)), np.zeros((G + 1, C))
            PU, CNT, EU = np.zeros(G + 1), np.zeros(G + 1), np.zeros(G + 1)
            for g, (a, b) in enumerate(rng_):
                vl, vf = vals[b - 1], vals[a]
                gap = vl - vals[a - 1] if g > 0 else 0.0
                qs = isq[a:b]
                SG = x[a:b][qs].sum(0)
                SB = ((vl - vals[a:b][qs])[:, None] * x[a:b][qs]).sum(0)
                inlast = qs & (vals[a:b] == vl)
                link = 1.0 if (g > 0 and vf == vals[a - 1] and vf == vl) else 0.0
                B[g + 1] = SB + B[g] + gap * PG[g]
                PG[g + 1] = PG[g] + SG
                PU[g + 1] = PU[g] + u[a:b][qs].sum()
                PW[g + 1] = PW[g] + x[a:b][~qs].sum(0)
                CNT[g + 1] = CNT[g] + (~qs).sum()
                E[g + 1] = x[a:b][inlast].sum(0) + link * E[g]
                EU[g + 1] = u[a:b][inlast].sum() + link * EU[g]
            Gt, Bt, Wt, Ut, vmax = PG[G], B[G], PW[G], PU[G], vals[L - 1]
            for g, (a, b) in enumerate(rng_):
                vbefore = vals[a - 1] if g > 0 else vals[a]
                tie_into = g > 0 and vals[a] == vbefore
                pg, bb, pw, pu, nk = PG[g].copy(), B[g].copy(), PW[g].copy(), PU[g], CNT[g]
                pgb = pg - (E[g] if tie_into else 0.0)
                pub = pu - (EU[g] if tie_into else 0.0)
                vprev = vbefore
                for t in range(a, b):
                    vt = vals[t]
                    if (t == a and not tie_into) or (t > a and vt != vals[t - 1]):
                        pgb, pub = pg.copy(), pu
                    bb = bb + (vt - vprev) * pg
                    if isq[t]:
                        gq[p, d, idx[t]] = x[t] @ (2 * pw - Wt) + u[t] * (2 * nk - N)
                        pg = pg + x[t]
                        pu = pu + u[t]
                    else:
                        gk[p, d, idx[t]] = x[t] @ (2 * pgb - Gt) + 2 * pub - Ut
                        gv[p, idx[t]] += 2 * bb - Bt - (vt - vmax) * Gt
                        pw = pw + x[t]
                        nk += 1
                    vprev = vt
    return gq, gk, gv


@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("full", [False, True])
def test_merged_walk_decomposition_matches_backward(ties, full):
    # The merged walk's ranges, summaries, three scans and tie carry (csrc/mbw.hip) give the brute-force backward with
    # s(0) = -1 in fp64, also when runs of equal values span many ranges (integer-valued inputs, 4-element ranges).
    rng = np.random.default_rng(7 + 2 * ties + full)
    P, D, N, M, C = 2, 2, 37, 29, 3
    if ties:
        q = rng.integers(-3, 4, (P, D, M)).astype(np.float64)
        k = rng.integers(-3, 4, (P, D, N)).astype(np.float64)
    else:
        q, k = rng.standard_normal((P, D, M)), rng.standard_normal((P, D, N))
    v, g_w = rng.standard_normal((P, N, C)), rng.standard_normal((P, M, C))
    g_u = rng.standard_normal((P, M)) if full else None
    got = _merged_walk_backward(q, k, v, g_w, g_u, RK=4)
    (wq, wk, wv), (nq, nk, nv) = brute.abs_backward(q, k, v, g_w, g_u)
    for name, a, b, n in zip(("grad_q", "grad_k", "grad_v"), got, (wq, wk, wv), (nq, nk, nv)):
        err = brute.rel_err(a, b, n)
        assert float(err.max()) < 1e-12, f"{name}: {float(err.max()):.3e}"
