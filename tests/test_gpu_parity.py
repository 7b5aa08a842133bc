"""GPU parity of the HIP path (through the drop-in packages and the C ABI) against the fp64 oracle.

Bars: sort permutations and merge ranks bit-exact; every float output within REL = 1e-5 of the fp64 oracle per element,
normalised by the sum of |term|.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import brute

pytestmark = pytest.mark.gpu

REL = 1e-5


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _np(t):
    return t.detach().cpu().numpy()


def _data(P, D, N, M, C, seed=0, kind="normal"):
    rng = np.random.default_rng(seed)
    if kind == "normal":
        q = rng.standard_normal((P, D, M)).astype(np.float32)
        k = rng.standard_normal((P, D, N)).astype(np.float32)
    elif kind == "ties":                           # few distinct levels: exact q == k ties and repeated keys
        q = (rng.integers(-4, 5, size=(P, D, M)) / 4).astype(np.float32)
        k = (rng.integers(-4, 5, size=(P, D, N)) / 4).astype(np.float32)
    elif kind == "zeros":                          # +-0.0 mixed with a few other tied levels
        lv = np.array([-0.0, 0.0, 1.0, -1.0, 0.5], dtype=np.float32)
        q = rng.choice(lv, size=(P, D, M))
        k = rng.choice(lv, size=(P, D, N))
    elif kind == "wide":                           # wide spread: exp underflow in the Laplace sums
        q = (rng.standard_normal((P, D, M)) * 40).astype(np.float32)
        k = (rng.standard_normal((P, D, N)) * 40).astype(np.float32)
    else:
        raise ValueError(kind)
    v = rng.standard_normal((P, N, C)).astype(np.float32)
    return q, k, v


def _assert_rel(got, want, norm, what):
    err = brute.rel_err(got, want, norm)
    worst = float(err.max()) if err.size else 0.0
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert worst <= REL, f"{what}: max rel err {worst:.3e} > {REL}"


SHAPES = [
    (1, 1, 1, 1, 1),
    (2, 3, 7, 5, 4),
    (2, 2, 64, 64, 64),
    (2, 2, 65, 63, 33),
    (3, 4, 129, 200, 64),
    (2, 3, 1000, 700, 65),
    (1, 2, 300, 257, 128),
    (1, 3, 100, 90, 1),
    (2, 2, 5000, 4097, 32),
    (1, 2, 300, 20000, 33),   # more queries than one LDS transpose holds: v == 1 terms written in query order
    (1, 1, 40000, 2000, 8),   # more key chunks than the staged query grouping holds: grouped straight to HBM
]


@pytest.fixture(params=["auto", "walk"])
def route(request):
    """auto: the library's size routing (dense kernels for short segments); walk: sort + walk at every size
    (qlka_set_direct_max(0)), so the walks stay covered on the short segments the routing sends elsewhere."""
    from qlka import _lib
    lib = _lib.load()
    if request.param == "auto":
        yield "auto"
        return
    prev = lib.qlka_set_direct_max(0)
    try:
        yield "walk"
    finally:
        lib.qlka_set_direct_max(prev)


def _same_route(route, N, M):
    if route == "walk" and max(N, M) > 1024:
        pytest.skip("above the dense cutoffs both routes walk")


# ------------------------------------------------------------------------------------------------ sort / rank
@pytest.mark.parametrize("L", [1, 2, 63, 64, 65, 100, 257, 1000, 2049, 5000, 8192, 16384, 16385, 40000])
@pytest.mark.parametrize("kind", ["normal", "ties", "zeros"])
def test_seg_sort_bit_exact(dev, L, kind):
    from qlka import ops
    S = 3
    q, _, _ = _data(S, 1, 1, L, 1, seed=L, kind=kind)
    keys = q.reshape(S, L)
    srt, perm = ops.seg_sort(_t(keys, dev))
    want_s, want_p = brute.stable_sort(keys)
    np.testing.assert_array_equal(_np(perm), want_p)
    np.testing.assert_array_equal(_np(srt), want_s)
    assert not np.any((_np(srt) == 0) & np.signbit(_np(srt))), "-0.0 must be written as +0.0"


@pytest.mark.parametrize("N,M", [(1, 1), (1, 5), (7, 1), (64, 64), (65, 200), (1000, 999), (3000, 70), (70000, 300)])
@pytest.mark.parametrize("kind", ["normal", "ties"])
def test_merge_rank_bit_exact(dev, N, M, kind):
    from qlka import ops
    S = 2
    q, k, _ = _data(S, 1, N, M, 1, seed=N + M, kind=kind)
    q, k = q.reshape(S, M), k.reshape(S, N)
    if kind == "ties":   # some queries equal to keys exactly, some outside the key range
        q[:, ::3] = k[:, (np.arange(0, M, 3) % N)]
        if M > 2:
            q[:, 1] = k.min() - 1
            q[:, -1] = k.max() + 1
    r = ops.merge_rank(_t(q, dev), _t(k, dev))
    np.testing.assert_array_equal(_np(r), brute.merge_rank(q, k))


# --------------------------------------------------------------------------------------------------- forward ops
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("kind", ["normal", "ties"])
def test_laplace_forward(dev, shape, kind, route):
    from weighted_laplace_sum import weighted_laplace_sum
    P, D, N, M, C = shape
    _same_route(route, N, M)
    q, k, v = _data(P, D, N, M, C, seed=sum(shape), kind=kind)
    w, u = weighted_laplace_sum(_t(q, dev), _t(k, dev), _t(v, dev))
    ow, ou, nw = brute.laplace_sum(q, k, v)
    _assert_rel(_np(w), ow, nw, "laplace out_w")
    _assert_rel(_np(u), ou, ou, "laplace out_u")


@pytest.mark.parametrize("N,M", [(500, 400), (3000, 2500)])
def test_laplace_wide_spread_underflow(dev, N, M, route):
    """Spread 40: most decay factors underflow to 0 and whole key ranges are cut off from each other; both routes,
    and N = 3000 walks on either (above the dense cutoff)."""
    from weighted_laplace_sum import weighted_laplace_sum
    _same_route(route, N, M)
    q, k, v = _data(2, 3, N, M, 16, seed=5, kind="wide")
    w, u = weighted_laplace_sum(_t(q, dev), _t(k, dev), _t(v, dev))
    ow, ou, nw = brute.laplace_sum(q, k, v)
    _assert_rel(_np(w), ow, nw, "laplace out_w (wide)")
    _assert_rel(_np(u), ou, ou, "laplace out_u (wide)")
    _assert_rel(_np(u), ou, ou, "laplace out_u (wide)")


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("kind", ["normal", "ties"])
def test_abs_forward_full(dev, shape, kind, route):
    from weighted_abs_sum import weighted_abs_sum, weighted_abs_sum_full
    P, D, N, M, C = shape
    _same_route(route, N, M)
    q, k, v = _data(P, D, N, M, C, seed=sum(shape) + 1, kind=kind)
    tq, tk, tv = _t(q, dev), _t(k, dev), _t(v, dev)
    w, u = weighted_abs_sum_full(tq, tk, tv, backend="cuda")
    w0 = weighted_abs_sum(tq, tk, tv, backend="cuda-global")
    ow, ou, nw = brute.abs_sum(q, k, v)
    _assert_rel(_np(w), ow, nw, "abs out_w")
    _assert_rel(_np(u), ou, ou, "abs out_u")
    _assert_rel(_np(w0), ow, nw, "abs (plain) out")


@pytest.mark.parametrize("layout", ["all_equal", "all_above", "all_below", "on_range_ends"])
def test_forward_query_grouping_edges(dev, layout):
    # The forward ops group the queries by key chunk instead of sorting them: one bucket holding every query (its
    # LDS slot counter taken by every lane at once), every query above or below every key (the last and the first
    # range own them all), and queries equal to the last key of a range (their bucket is that range, rank at its end).
    from weighted_abs_sum import weighted_abs_sum_full
    from weighted_laplace_sum import weighted_laplace_sum
    P, D, N, M, C = 2, 2, 1500, 3000, 16
    q, k, v = _data(P, D, N, M, C, seed=11)
    ks = np.sort(k, axis=2)
    if layout == "all_equal":
        q[:] = ks[:, :, N // 2][:, :, None] + np.float32(0.25)
    elif layout == "all_above":
        q = ks[:, :, -1:] + np.abs(q) + np.float32(1.0)
    elif layout == "all_below":
        q = ks[:, :, :1] - np.abs(q) - np.float32(1.0)
    else:
        ends = ks[:, :, 63::64]                                   # the last key of every 64-key range
        q = ends[:, :, np.arange(M) % ends.shape[2]]
    q = np.ascontiguousarray(q, dtype=np.float32)
    tq, tk, tv = _t(q, dev), _t(k, dev), _t(v, dev)
    w, u = weighted_laplace_sum(tq, tk, tv)
    ow, ou, nw = brute.laplace_sum(q, k, v)
    _assert_rel(_np(w), ow, nw, f"laplace out_w ({layout})")
    _assert_rel(_np(u), ou, ou, f"laplace out_u ({layout})")
    w, u = weighted_abs_sum_full(tq, tk, tv, backend="cuda")
    ow, ou, nw = brute.abs_sum(q, k, v)
    _assert_rel(_np(w), ow, nw, f"abs out_w ({layout})")
    _assert_rel(_np(u), ou, ou, f"abs out_u ({layout})")


@pytest.mark.parametrize("layout", ["all_equal", "long_runs", "on_key_ranks"])
def test_backward_tie_runs_across_tiles_and_scan_blocks(dev, layout):
    # The backward's merged walk takes a key's query sums where its run of equal values began, carried across ranges,
    # merge tiles (2048 merged elements) and scan workgroups (256 ranges) by the tie carry. N + M = 18000: 282 ranges,
    # 9 tiles, two scan workgroups per segment. Layouts: every query and key one value (one run over the whole
    # segment); runs of about 3000 equal values mixing queries and keys; queries equal to every 64th sorted key.
    from oracle import inputs
    from weighted_abs_sum import weighted_abs_sum_full
    P, D, N, M, C = 2, 2, 9000, 9000, 16
    print(f"backward tie runs ({layout})", flush=True)
    q, k, v = _data(P, D, N, M, C, seed=41)
    if layout == "all_equal":
        q[:] = np.float32(0.5)
        k[:] = np.float32(0.5)
    elif layout == "long_runs":
        q = np.floor(q * 2).astype(np.float32) / 2      # a handful of levels: runs of ~3000 values
        k = np.floor(k * 2).astype(np.float32) / 2
    else:
        ks = np.sort(k, axis=2)
        q = np.ascontiguousarray(ks[:, :, (np.arange(M) * 64) % N], dtype=np.float32)
    rng = np.random.default_rng(43)
    g_w = rng.standard_normal((P, M, C)).astype(np.float32)
    g_u = rng.standard_normal((P, M)).astype(np.float32)
    tq, tk, tv = (_t(a, dev).requires_grad_(True) for a in (q, k, v))
    w, u = weighted_abs_sum_full(tq, tk, tv, backend="cuda")
    torch.autograd.backward([w, u], [_t(g_w, dev), _t(g_u, dev)])
    bq = inputs.query_subsample(P, M, per_p=6, seed=5)
    bk = inputs.query_subsample(P, N, per_p=6, seed=6)
    (wq, wk, wv), (nq, nk, nv) = brute.abs_backward_sub(q, k, v, g_w, g_u, bq, bk)
    sub = lambda a, idx, axis: np.stack([np.take(a[p], idx[p], axis=axis) for p in range(P)])  # noqa: E731
    _assert_rel(sub(_np(tq.grad), bq, 1), wq, nq, f"grad_q ({layout})")
    _assert_rel(sub(_np(tk.grad), bk, 1), wk, nk, f"grad_k ({layout})")
    _assert_rel(sub(_np(tv.grad), bk, 0), wv, nv, f"grad_v ({layout})")


def test_abs_translation_far_from_zero(dev):
    # keys and queries centred at 1000: the distance-relative walk must not cancel catastrophically
    from weighted_abs_sum import weighted_abs_sum_full
    q, k, v = _data(2, 3, 800, 600, 8, seed=7)
    q = q + np.float32(1000.0)
    k = k + np.float32(1000.0)
    w, u = weighted_abs_sum_full(_t(q, dev), _t(k, dev), _t(v, dev))
    ow, ou, nw = brute.abs_sum(q, k, v)
    _assert_rel(_np(w), ow, nw, "abs out_w (offset 1000)")
    _assert_rel(_np(u), ou, ou, "abs out_u (offset 1000)")


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("kind", ["normal", "ties"])
def test_sgn_sum(dev, shape, kind, route):
    from weighted_abs_sum import weighted_sgn_sum
    P, D, N, M, C = shape
    _same_route(route, N, M)
    q, k, v = _data(P, D, N, M, C, seed=sum(shape) + 2, kind=kind)
    g = np.random.default_rng(3).standard_normal((P, M, C)).astype(np.float32)
    out = weighted_sgn_sum(_t(q, dev), _t(k, dev), _t(v, dev), _t(g, dev), backend="cuda")
    want, norm = brute.sgn_sum(q, k, v, g, tie=1.0)
    _assert_rel(_np(out), want, norm, "sgn")


# ---------------------------------------------------------------------------------------------------- backward
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("full", [False, True])
@pytest.mark.parametrize("kind", ["normal", "ties"])
def test_abs_backward(dev, shape, full, kind, route):
    from weighted_abs_sum import _ext
    P, D, N, M, C = shape
    _same_route(route, N, M)
    q, k, v = _data(P, D, N, M, C, seed=sum(shape) + 3, kind=kind)
    rng = np.random.default_rng(4)
    g_w = rng.standard_normal((P, M, C)).astype(np.float32)
    g_u = rng.standard_normal((P, M)).astype(np.float32) if full else None
    args = [_t(q, dev), _t(k, dev), _t(v, dev), _t(g_w, dev)]
    if full:
        gq, gk, gv = _ext.weighted_abs_sum_full_backward(*args, _t(g_u, dev))
    else:
        gq, gk, gv = _ext.weighted_abs_sum_backward(*args)
    (wq, wk, wv), (nq, nk, nv) = brute.abs_backward(q, k, v, g_w, g_u)
    _assert_rel(_np(gq), wq, nq, "grad_q")
    _assert_rel(_np(gk), wk, nk, "grad_k")
    _assert_rel(_np(gv), wv, nv, "grad_v")


@pytest.mark.parametrize("shape", [(2, 3, 2000, 1500, 64), (1, 2, 600, 900, 128), (2, 2, 3000, 3000, 32)])
@pytest.mark.parametrize("with_u", [False, True])
def test_backward_error_against_reference_fp32_composition(dev, shape, with_u):
    """grad_q under the per-key normaliser sum_n |<g_m, v_n> (+ g_u)| (tighter than the elementary-product one of the
    other tests when a C-channel dot product cancels): the library's error must stay within twice the error of the
    reference's own fp32 composition (prefix sums in sorted order, <g, 2 PW - W_tot>, oracle grad_q_fp32_prefix)
    and below 1e-4. Both walk and dense routes at these sizes are the library's own choice."""
    from weighted_abs_sum import _ext
    P, D, N, M, C = shape
    q, k, v = _data(P, D, N, M, C, seed=sum(shape))
    rng = np.random.default_rng(sum(shape) + 1)
    g_w = rng.standard_normal((P, M, C)).astype(np.float32)
    g_u = rng.standard_normal((P, M)).astype(np.float32) if with_u else None
    tq, tk, tv, tg = (_t(a, dev) for a in (q, k, v, g_w))
    if with_u:
        gq, _, _ = _ext.weighted_abs_sum_full_backward(tq, tk, tv, tg, _t(g_u, dev))
    else:
        gq, _, _ = _ext.weighted_abs_sum_backward(tq, tk, tv, tg)
    (want, _, _), _ = brute.abs_backward(q, k, v, g_w, g_u, tie=-1.0)
    ref32 = brute.grad_q_fp32_prefix(q, k, v, g_w, g_u)
    dn = brute.dot_normaliser(v, g_w, g_u)[:, None, :]
    err_lib = float((np.abs(_np(gq) - want) / dn).max())
    err_ref = float((np.abs(ref32 - want) / dn).max())
    print(f"grad_q error / per-key normaliser {shape} g_u={with_u}: library {err_lib:.3e}, reference fp32 "
          f"composition {err_ref:.3e}")
    assert err_lib <= 1e-4
    assert err_lib <= max(2 * err_ref, 1e-6)


@pytest.mark.parametrize("full", [False, True])
def test_autograd_through_ops(dev, full):
    from weighted_abs_sum import weighted_abs_sum, weighted_abs_sum_full
    P, D, N, M, C = 2, 4, 300, 250, 16
    q, k, v = _data(P, D, N, M, C, seed=21)
    rng = np.random.default_rng(5)
    g_w = rng.standard_normal((P, M, C)).astype(np.float32)
    g_u = rng.standard_normal((P, M)).astype(np.float32)
    tq, tk, tv = (_t(a, dev).requires_grad_(True) for a in (q, k, v))
    if full:
        w, u = weighted_abs_sum_full(tq, tk, tv)
        loss = (w * _t(g_w, dev)).sum() + (u * _t(g_u, dev)).sum()
    else:
        w = weighted_abs_sum(tq, tk, tv)
        loss = (w * _t(g_w, dev)).sum()
    loss.backward()
    (wq, wk, wv), (nq, nk, nv) = brute.abs_backward(q, k, v, g_w, g_u if full else None)
    _assert_rel(_np(tq.grad), wq, nq, "autograd grad_q")
    _assert_rel(_np(tk.grad), wk, nk, "autograd grad_k")
    _assert_rel(_np(tv.grad), wv, nv, "autograd grad_v")


@pytest.mark.parametrize("shape", [(2, 3, 1500, 1300, 16),   # forward and backward walk
                                   (2, 3, 800, 700, 12)])     # dense forward, walking backward: sorts kept anyway
@pytest.mark.parametrize("full", [False, True])
def test_autograd_keeps_sorts_for_backward(dev, shape, full):
    # The "cuda" forward leaves its sorted k and q for the backward (ops.KEEP_SORTS): the gradients must equal those
    # of a backward that sorts again, bit for bit, and the oracle's (a tie counts -1).
    from weighted_abs_sum import ops, weighted_abs_sum, weighted_abs_sum_full
    P, D, N, M, C = shape
    q, k, v = _data(P, D, N, M, C, seed=sum(shape), kind="ties")
    rng = np.random.default_rng(12)
    g_w = rng.standard_normal((P, M, C)).astype(np.float32)
    g_u = rng.standard_normal((P, M)).astype(np.float32)
    grads = {}
    try:
        for keep in (True, False):
            ops.set_keep_sorts(keep)
            tq, tk, tv = (_t(a, dev).requires_grad_(True) for a in (q, k, v))
            if full:
                w, u = weighted_abs_sum_full(tq, tk, tv, backend="cuda")
                loss = (w * _t(g_w, dev)).sum() + (u * _t(g_u, dev)).sum()
            else:
                w = weighted_abs_sum(tq, tk, tv, backend="cuda")
                loss = (w * _t(g_w, dev)).sum()
            loss.backward()
            grads[keep] = [_np(t.grad) for t in (tq, tk, tv)]
    finally:
        ops.set_keep_sorts(True)
    for name, a, b in zip(("grad_q", "grad_k", "grad_v"), grads[True], grads[False]):
        np.testing.assert_array_equal(a, b, err_msg=f"{name}: kept sorts vs sorting again")
    (wq, wk, wv), (nq, nk, nv) = brute.abs_backward(q, k, v, g_w, g_u if full else None)
    _assert_rel(grads[True][0], wq, nq, "kept-sorts grad_q")
    _assert_rel(grads[True][1], wk, nk, "kept-sorts grad_k")
    _assert_rel(grads[True][2], wv, nv, "kept-sorts grad_v")


@pytest.mark.parametrize("shape", [(3, 5, 301, 200, 33),     # dense route, A kept by the forward
                                   (32, 16, 600, 520, 64),  # the dense backward at L = 600 (enough workgroups)
                                   (2, 3, 150, 500, 128)])
@pytest.mark.parametrize("full", [True, False])
def test_autograd_keeps_dense_matrix(dev, shape, full):
    # On the dense route a differentiable "cuda" forward keeps its kernel matrix A for the backward, whose grad_v is
    # then A's contraction with g_w instead of forming A again: the gradients must equal those of the backward that
    # forms it (the extension's plain backward), bit for bit, and the oracle's.
    from qlka import _lib
    from weighted_abs_sum import _ext, weighted_abs_sum, weighted_abs_sum_full
    P, D, N, M, C = shape
    assert _lib.load().qlka_abs_dense_keep_bytes(P, D, N, M, C) > 0
    q, k, v = _data(P, D, N, M, C, seed=sum(shape) + 3, kind="ties")
    rng = np.random.default_rng(13)
    g_w = rng.standard_normal((P, M, C)).astype(np.float32)
    g_u = rng.standard_normal((P, M)).astype(np.float32)
    tq, tk, tv = (_t(a, dev).requires_grad_(True) for a in (q, k, v))
    if full:
        w, u = weighted_abs_sum_full(tq, tk, tv, backend="cuda")
        torch.autograd.backward([w, u], [_t(g_w, dev), _t(g_u, dev)])
        ref = _ext.weighted_abs_sum_full_backward(_t(q, dev), _t(k, dev), _t(v, dev), _t(g_w, dev), _t(g_u, dev))
    else:
        w = weighted_abs_sum(tq, tk, tv, backend="cuda")
        w.backward(_t(g_w, dev))
        ref = _ext.weighted_abs_sum_backward(_t(q, dev), _t(k, dev), _t(v, dev), _t(g_w, dev))
    got = [_np(t.grad) for t in (tq, tk, tv)]
    for name, a, b in zip(("grad_q", "grad_k", "grad_v"), got, ref):
        np.testing.assert_array_equal(a, _np(b), err_msg=f"{name}: kept A vs forming A again")
    (wq, wk, wv), (nq, nk, nv) = brute.abs_backward(q, k, v, g_w, g_u if full else None)
    _assert_rel(got[0], wq, nq, "kept-A grad_q")
    _assert_rel(got[1], wk, nk, "kept-A grad_k")
    _assert_rel(got[2], wv, nv, "kept-A grad_v")


@pytest.mark.parametrize("shape", [(2, 3, 1500, 1300, 18),      # one chunk
                                   (6, 64, 16384, 16384, 30),   # pipelined chunks of 2 p
                                   (2, 8, 40000, 30000, 65)])   # two-launch scans, two channel slots per lane
def test_kept_range_states_match_recomputed(dev, shape):
    # A walking forward that keeps its sorts also leaves its range states and query bounds (a fifth tensor) at the
    # widths whose backward walks twice (C > 64 or C % 4 != 0): the backward over them (its grad_q walk skips its range
    # passes) must equal the backward over the sorts alone, which recomputes them, bit for bit, with and without g_u;
    # the gradients also against the oracle on a subsample.
    from oracle import inputs
    from weighted_abs_sum import _ext
    P, D, N, M, C = shape
    print(f"kept range states {shape}", flush=True)
    q, k, v = _data(P, D, N, M, C, seed=sum(shape) % 997, kind="ties")
    rng = np.random.default_rng(19)
    g_w = _t(rng.standard_normal((P, M, C)).astype(np.float32), dev)
    g_u = _t(rng.standard_normal((P, M)).astype(np.float32), dev)
    tq, tk, tv = _t(q, dev), _t(k, dev), _t(v, dev)
    w, u, srt = _ext.weighted_abs_sum_forward_keep(tq, tk, tv, -1, True)
    assert len(srt) == 5 and srt[4].dtype == torch.uint8
    for gu in (g_u, None):
        with_states = _ext.weighted_abs_sum_backward_sorted(tq, tk, tv, g_w, gu, srt)
        without = _ext.weighted_abs_sum_backward_sorted(tq, tk, tv, g_w, gu, srt[:4])
        for name, a, b in zip(("grad_q", "grad_k", "grad_v"), with_states, without):
            assert torch.equal(a, b), f"{name} (g_u {'given' if gu is not None else 'none'}): kept states differ"
    bq = inputs.query_subsample(P, M, per_p=4, seed=3)
    bk = inputs.query_subsample(P, N, per_p=4, seed=4)
    gq, gk, gv = _ext.weighted_abs_sum_backward_sorted(tq, tk, tv, g_w, g_u, srt)
    (wq, wk, wv), (nq, nk, nv) = brute.abs_backward_sub(q, k, v, _np(g_w), _np(g_u), bq, bk)
    sub = lambda a, idx, axis: np.stack([np.take(a[p], idx[p], axis=axis) for p in range(P)])  # noqa: E731
    _assert_rel(sub(_np(gq), bq, 1), wq, nq, "kept-states grad_q")
    _assert_rel(sub(_np(gk), bk, 1), wk, nk, "kept-states grad_k")
    _assert_rel(sub(_np(gv), bk, 0), wv, nv, "kept-states grad_v")


@pytest.mark.parametrize("shape", [(2, 3, 1500, 1300, 16),      # one chunk
                                   (6, 64, 16384, 16384, 32)])  # pipelined chunks of 2 p
def test_merged_backward_over_kept_sorts(dev, shape):
    # At C <= 64 with C % 4 == 0 the backward walks once over the merged sorted keys and queries and reads no range
    # states: the forward keeps the four sorts only, and the backward over them equals, bit for bit, the backward that
    # sorts again, with and without g_u.
    from weighted_abs_sum import _ext
    P, D, N, M, C = shape
    print(f"merged backward over kept sorts {shape}", flush=True)
    q, k, v = _data(P, D, N, M, C, seed=sum(shape) % 991, kind="ties")
    rng = np.random.default_rng(23)
    g_w = _t(rng.standard_normal((P, M, C)).astype(np.float32), dev)
    g_u = _t(rng.standard_normal((P, M)).astype(np.float32), dev)
    tq, tk, tv = _t(q, dev), _t(k, dev), _t(v, dev)
    _, _, srt = _ext.weighted_abs_sum_forward_keep(tq, tk, tv, -1, True)
    assert len(srt) == 4
    kept = _ext.weighted_abs_sum_backward_sorted(tq, tk, tv, g_w, g_u, srt)
    again = _ext.weighted_abs_sum_full_backward(tq, tk, tv, g_w, g_u)
    for name, a, b in zip(("grad_q", "grad_k", "grad_v"), kept, again):
        assert torch.equal(a, b), f"{name}: over the kept sorts vs sorting again"
    kept = _ext.weighted_abs_sum_backward_sorted(tq, tk, tv, g_w, None, srt)
    again = _ext.weighted_abs_sum_backward(tq, tk, tv, g_w)
    for name, a, b in zip(("grad_q", "grad_k", "grad_v"), kept, again):
        assert torch.equal(a, b), f"{name} (no g_u): over the kept sorts vs sorting again"


def test_backward_with_workspace_above_a_2gib_address_boundary(dev):
    # The backward's kernels build buffer descriptors from 64-bit workspace addresses read through readfirstlane; a
    # low address word with bit 31 set once sign-extended over the high word there. The workspace is placed so that
    # the low 32 bits of every address in its first 2 GiB have bit 31 set, and the call through the C ABI must equal
    # the call on a workspace from the allocator, bit for bit, for a merged-walk width and a two-walk width.
    from qlka import _lib
    lib = _lib.load()
    for C in (64, 30):
        P, D, N, M = 3, 4, 3000, 2600
        print(f"backward, workspace above a 2 GiB boundary, C={C}", flush=True)
        q, k, v = (_t(a, dev) for a in _data(P, D, N, M, C, seed=C + 5, kind="ties"))
        rng = np.random.default_rng(C)
        g_w = _t(rng.standard_normal((P, M, C)).astype(np.float32), dev)
        g_u = _t(rng.standard_normal((P, M)).astype(np.float32), dev)
        need = lib.qlka_abs_bwd_ws_bytes(P, D, N, M, C)
        assert 0 < need < (1 << 30)

        def run(ws_ptr):
            gq, gk = torch.empty((P, D, M), device=dev), torch.empty((P, D, N), device=dev)
            gv = torch.empty((P, N, C), device=dev)
            _lib.check(lib.qlka_abs_bwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g_w), _lib.ptr(g_u),
                                        _lib.ptr(gq), _lib.ptr(gk), _lib.ptr(gv), P, D, N, M, C, ws_ptr, need,
                                        _lib.stream_of(dev)))
            torch.cuda.synchronize()
            return gq, gk, gv

        plain = torch.empty((need,), dtype=torch.uint8, device=dev)
        want = run(_lib.ptr(plain))
        del plain
        big = torch.empty(((4 << 30) + need,), dtype=torch.uint8, device=dev)
        base = big.data_ptr()
        off = (0x80000000 - (base & 0xFFFFFFFF)) % (1 << 32)     # base + off has low word 0x80000000
        assert off + need <= big.numel() and ((base + off) & 0xFFFFFFFF) == 0x80000000
        got = run(ctypes.c_void_p(base + off))
        del big
        for name, a, b in zip(("grad_q", "grad_k", "grad_v"), got, want):
            assert torch.equal(a, b), f"{name} (C={C}): the workspace's address changed the result"


def test_fwd_keep_leaves_unsized_states_untouched(dev):
    # Through the C ABI: where qlka_abs_keep_state_bytes is 0 (the merged backward, C <= 64, C % 4 == 0) the forward
    # keeps the sorts only (*kept = 1) even when handed a states pointer, and writes nothing through it; at a width whose
    # backward walks twice it fills a buffer of the stated size (*kept = 3).
    from qlka import _lib
    lib = _lib.load()
    for C, want in ((64, 1), (62, 3)):
        P, D, N, M = 2, 3, 3000, 2500
        print(f"fwd_keep states C={C}", flush=True)
        q, k, v = (_t(a, dev) for a in _data(P, D, N, M, C, seed=C, kind="ties"))
        out_w = torch.empty((P, M, C), device=dev)
        out_u = torch.empty((P, M), device=dev)
        ks, qs = torch.empty((P, D, N), device=dev), torch.empty((P, D, M), device=dev)
        kp = torch.empty((P, D, N), dtype=torch.int32, device=dev)
        qp = torch.empty((P, D, M), dtype=torch.int32, device=dev)
        nbytes = lib.qlka_abs_keep_state_bytes(P, D, N, M, C)
        assert (nbytes == 0) == (want == 1)
        states = torch.full((max(nbytes, 1 << 20) // 4,), 12345.0, device=dev)   # a sentinel where nothing is sized
        ws = torch.empty((lib.qlka_abs_fwd_ws_bytes(P, D, N, M, C),), dtype=torch.uint8, device=dev)
        kept = ctypes.c_int(-1)
        _lib.check(lib.qlka_abs_fwd_keep(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out_w), _lib.ptr(out_u),
                                         P, D, N, M, C, -1, _lib.ptr(ks), _lib.ptr(kp), _lib.ptr(qs), _lib.ptr(qp),
                                         _lib.ptr(states), ctypes.byref(kept), _lib.ptr(ws), ws.numel(),
                                         _lib.stream_of(dev)))
        torch.cuda.synchronize()
        assert kept.value == want
        if want == 1:
            assert bool((states == 12345.0).all()), "the forward wrote through an unsized states pointer"


def test_full_backward_only_u(dev):
    # out_w unused: g_w is None inside the autograd Function and becomes zeros (ops.py:99-101)
    from weighted_abs_sum import weighted_abs_sum_full
    P, D, N, M, C = 1, 3, 120, 100, 8
    q, k, v = _data(P, D, N, M, C, seed=22)
    g_u = np.random.default_rng(6).standard_normal((P, M)).astype(np.float32)
    tq, tk, tv = (_t(a, dev).requires_grad_(True) for a in (q, k, v))
    _, u = weighted_abs_sum_full(tq, tk, tv)
    (u * _t(g_u, dev)).sum().backward()
    (wq, wk, wv), (nq, nk, nv) = brute.abs_backward(q, k, v, np.zeros((P, M, C), np.float32), g_u)
    _assert_rel(_np(tq.grad), wq, nq, "grad_q (u only)")
    _assert_rel(_np(tk.grad), wk, nk, "grad_k (u only)")
    np.testing.assert_array_equal(_np(tv.grad), np.zeros_like(v))


# ------------------------------------------------------------------------------------------------ boundary on GPU
def test_gpu_validation_errors(dev):
    from weighted_abs_sum import _ext, weighted_abs_sum_full, weighted_sgn_sum
    from weighted_laplace_sum import weighted_laplace_sum
    q = torch.randn(1, 2, 8, device=dev)
    k = torch.randn(1, 2, 8, device=dev)
    with pytest.raises(RuntimeError, match=r"C \(v.size\(2\)\) must be in \[1, 128\]"):
        _ext.weighted_abs_sum_forward(q, k, torch.randn(1, 8, 129, device=dev))
    with pytest.raises(RuntimeError, match=r"C \(v.size\(2\)\) must be in \[1, 128\]"):
        weighted_laplace_sum(q, k, torch.randn(1, 8, 129, device=dev))
    with pytest.raises(RuntimeError, match="N and M must be <= 131072"):
        _ext.weighted_abs_sum_forward(torch.randn(1, 1, 4, device=dev), torch.randn(1, 1, 131073, device=dev),
                                      torch.randn(1, 131073, 1, device=dev))
    with pytest.raises(RuntimeError, match="must be contiguous"):
        qt = q.transpose(1, 2).contiguous().transpose(1, 2)
        _ext.weighted_abs_sum_forward(qt, k, torch.randn(1, 8, 4, device=dev))
    with pytest.raises(RuntimeError, match="must be float32"):
        weighted_laplace_sum(q.double(), k, torch.randn(1, 8, 4, device=dev))
    with pytest.raises(RuntimeError, match="fused path pinned but unavailable"):
        big = torch.randn(1, 1, 5000, device=dev)
        weighted_abs_sum_full(big, big, torch.randn(1, 5000, 2, device=dev), backend="cuda-fused")
    with pytest.raises(ValueError, match="no fused path"):
        weighted_sgn_sum(q, k, torch.randn(1, 8, 4, device=dev), torch.randn(1, 8, 4, device=dev), backend="cuda-fused")
    with pytest.raises(RuntimeError, match=r"g_w must have shape \(P, M, C\)"):
        _ext.weighted_abs_sum_backward(q, k, torch.randn(1, 8, 4, device=dev), torch.randn(1, 8, 5, device=dev))
    # the fused path within its range runs
    w, u = weighted_abs_sum_full(q, k, torch.randn(1, 8, 4, device=dev), backend="cuda-fused")
    assert w.shape == (1, 8, 4) and u.shape == (1, 8)


@pytest.mark.parametrize("backend", ["cuda-fused", "cuda-global"])
@pytest.mark.parametrize("shape", [(2, 3, 600, 500, 64), (1, 2, 4096, 4096, 33)])
def test_pinned_paths_against_oracle(dev, backend, shape):
    """backend="cuda-fused" (path 1, max(N, M) <= 4096) and "cuda-global" (path 0) give the oracle's sums, forward and
    backward, like "auto"."""
    from weighted_abs_sum import weighted_abs_sum, weighted_abs_sum_full
    P, D, N, M, C = shape
    q, k, v = _data(P, D, N, M, C, seed=sum(shape) + 7, kind="ties")
    g_w = np.random.default_rng(8).standard_normal((P, M, C)).astype(np.float32)
    tq, tk, tv = (_t(a, dev).requires_grad_(True) for a in (q, k, v))
    w, u = weighted_abs_sum_full(tq, tk, tv, backend=backend)
    (w * _t(g_w, dev)).sum().backward()
    ow, ou, nw = brute.abs_sum(q, k, v)
    _assert_rel(_np(w), ow, nw, f"{backend} out_w")
    _assert_rel(_np(u), ou, ou, f"{backend} out_u")
    (wq, wk, wv), (nq, nk, nv) = brute.abs_backward(q, k, v, g_w)
    _assert_rel(_np(tq.grad), wq, nq, f"{backend} grad_q")
    _assert_rel(_np(tk.grad), wk, nk, f"{backend} grad_k")
    _assert_rel(_np(tv.grad), wv, nv, f"{backend} grad_v")
    w2 = weighted_abs_sum(tq.detach(), tk.detach(), tv.detach(), backend=backend)
    _assert_rel(_np(w2), ow, nw, f"{backend} plain out_w")


def test_non_default_stream_and_repeat(dev):
    # every launch is on the current stream; repeated calls give identical results up to atomic ordering
    from weighted_laplace_sum import weighted_laplace_sum
    q, k, v = _data(2, 4, 700, 600, 64, seed=30)
    tq, tk, tv = _t(q, dev), _t(k, dev), _t(v, dev)
    s = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(s):
        w1, u1 = weighted_laplace_sum(tq, tk, tv)
    s.synchronize()
    w2, u2 = weighted_laplace_sum(tq, tk, tv)
    ow, ou, nw = brute.laplace_sum(q, k, v)
    _assert_rel(_np(w1), ow, nw, "stream out_w")
    _assert_rel(_np(w2), ow, nw, "default stream out_w")
    _assert_rel(_np(u1), ou, ou, "stream out_u")


@pytest.mark.parametrize("fill", [0x00, 0xFF, 0x7F])
@pytest.mark.parametrize("shape", [(3, 4, 129, 200, 64), (2, 2, 5000, 4097, 32), (2, 3, 1000, 700, 65)])
def test_workspace_contents_do_not_matter(dev, shape, fill):
    # every op through the C ABI with the workspace pre-filled (NaN, zero, large): no stage may read workspace
    # memory before writing it, and no kernel may read memory it also writes
    from qlka import _lib
    lib = _lib.load()
    P, D, N, M, C = shape
    q, k, v = _data(P, D, N, M, C, seed=sum(shape), kind="normal")
    g_w = np.random.default_rng(8).standard_normal((P, M, C)).astype(np.float32)
    tq, tk, tv, tg = _t(q, dev), _t(k, dev), _t(v, dev), _t(g_w, dev)
    st = _lib.stream_of(dev)

    def ws(nb):
        return torch.full((max(nb, 1),), fill, dtype=torch.uint8, device=dev)

    out, out_u = torch.empty((P, M, C), device=dev), torch.empty((P, M), device=dev)
    w = ws(lib.qlka_laplace_fwd_ws_bytes(P, D, N, M, C))
    _lib.check(lib.qlka_laplace_fwd(_lib.ptr(tq), _lib.ptr(tk), _lib.ptr(tv), _lib.ptr(out), _lib.ptr(out_u),
                                    P, D, N, M, C, _lib.ptr(w), w.numel(), st))
    ow, ou, nw = brute.laplace_sum(q, k, v)
    _assert_rel(_np(out), ow, nw, "laplace out_w (poisoned ws)")
    _assert_rel(_np(out_u), ou, ou, "laplace out_u (poisoned ws)")

    w = ws(lib.qlka_abs_fwd_ws_bytes(P, D, N, M, C))
    _lib.check(lib.qlka_abs_fwd(_lib.ptr(tq), _lib.ptr(tk), _lib.ptr(tv), _lib.ptr(out), _lib.ptr(out_u),
                                P, D, N, M, C, -1, _lib.ptr(w), w.numel(), st))
    ow, ou, nw = brute.abs_sum(q, k, v)
    _assert_rel(_np(out), ow, nw, "abs out_w (poisoned ws)")
    _assert_rel(_np(out_u), ou, ou, "abs out_u (poisoned ws)")

    gq, gk, gv = (torch.empty((P, D, M), device=dev), torch.empty((P, D, N), device=dev),
                  torch.empty((P, N, C), device=dev))
    w = ws(lib.qlka_abs_bwd_ws_bytes(P, D, N, M, C))
    _lib.check(lib.qlka_abs_bwd(_lib.ptr(tq), _lib.ptr(tk), _lib.ptr(tv), _lib.ptr(tg), _lib.ptr(None),
                                _lib.ptr(gq), _lib.ptr(gk), _lib.ptr(gv), P, D, N, M, C, _lib.ptr(w), w.numel(), st))
    (wq, wk, wv), (nq, nk, nv) = brute.abs_backward(q, k, v, g_w)
    _assert_rel(_np(gq), wq, nq, "grad_q (poisoned ws)")
    _assert_rel(_np(gk), wk, nk, "grad_k (poisoned ws)")
    _assert_rel(_np(gv), wv, nv, "grad_v (poisoned ws)")


# ------------------------------------------------------------------------------------------ dense (direct) route
DIRECT_SHAPES = [  # P, D, N, M, C: tiles of 64 queries / keys and 32 features, partial tiles on every axis
    (1, 1, 1, 1, 1),
    (3, 5, 65, 63, 33),
    (2, 33, 130, 200, 64),
    (2, 70, 64, 64, 65),
    (1, 2, 257, 300, 128),
    (4, 32, 65, 65, 32),      # the ViT segment shape of BASELINE configs[1]
    (2, 4, 1500, 900, 16),    # long segments: the dense route is valid at any size
    # Segments of at most 128 (padded) keys and queries have one-workgroup-per-p kernels (whole segment in LDS)
    # besides the tiled ones; the shapes above cover both, these add several 64-feature chunks with ragged sizes,
    # the largest segment the small kernels take, and C = 128 (small forward, tiled sign sums).
    (2, 70, 61, 50, 19),
    (1, 8, 108, 112, 8),
    (2, 3, 40, 30, 128),
    (2, 8, 200, 150, 20),     # tiled sign sums with 64-output tiles (D <= 32), C <= 64
]
DIRECT_SIGN_SHAPES = [s for s in DIRECT_SHAPES if s[2] * s[3] < 1_000_000]


@pytest.mark.parametrize("shape", DIRECT_SHAPES)
@pytest.mark.parametrize("kind", ["normal", "ties"])
def test_direct_forward(dev, shape, kind):
    from qlka import _lib
    P, D, N, M, C = shape
    q, k, v = _data(P, D, N, M, C, seed=sum(shape) + 9, kind=kind)
    tq, tk, tv = _t(q, dev), _t(k, dev), _t(v, dev)
    lib = _lib.load()
    for op, oracle in ((0, brute.abs_sum), (1, brute.laplace_sum)):
        ow, ou, nw = oracle(q, k, v)
        for with_u in (True, False):
            w = torch.empty(P, M, C, device=dev)
            u = torch.empty(P, M, device=dev) if with_u else None
            _lib.check(lib.qlka_direct_fwd(op, _lib.ptr(tq), _lib.ptr(tk), _lib.ptr(tv), _lib.ptr(w), _lib.ptr(u),
                                           P, D, N, M, C, _lib.stream_of(dev)))
            _assert_rel(_np(w), ow, nw, f"direct kind {op} out_w")
            if with_u:
                _assert_rel(_np(u), ou, ou, f"direct kind {op} out_u")


@pytest.mark.parametrize("full", [False, True])
def test_keops_route_forward_and_autograd(dev, full):
    # "keops": dense forward on contiguous copies, gradients from the walk backward
    from weighted_abs_sum import weighted_abs_sum, weighted_abs_sum_full
    P, D, N, M, C = 3, 6, 120, 100, 12
    q, k, v = _data(P, D, N, M, C, seed=31)
    rng = np.random.default_rng(6)
    g_w = rng.standard_normal((P, M, C)).astype(np.float32)
    g_u = rng.standard_normal((P, M)).astype(np.float32)
    # non-contiguous views, as a KeOps caller may pass them
    tq = _t(np.ascontiguousarray(q.transpose(0, 2, 1)), dev).transpose(1, 2).requires_grad_(True)
    tk, tv = (_t(a, dev).requires_grad_(True) for a in (k, v))
    if full:
        w, u = weighted_abs_sum_full(tq, tk, tv, backend="keops")
        loss = (w * _t(g_w, dev)).sum() + (u * _t(g_u, dev)).sum()
    else:
        w = weighted_abs_sum(tq, tk, tv, backend="keops")
        loss = (w * _t(g_w, dev)).sum()
    ow, ou, nw = brute.abs_sum(q, k, v)
    _assert_rel(_np(w), ow, nw, "keops route out_w")
    if full:
        _assert_rel(_np(u), ou, ou, "keops route out_u")
    loss.backward()
    (wq, wk, wv), (nq, nk, nv) = brute.abs_backward(q, k, v, g_w, g_u if full else None)
    _assert_rel(_np(tq.grad), wq, nq, "keops route grad_q")
    _assert_rel(_np(tk.grad), wk, nk, "keops route grad_k")
    _assert_rel(_np(tv.grad), wv, nv, "keops route grad_v")


@pytest.mark.parametrize("shape", DIRECT_SIGN_SHAPES)
@pytest.mark.parametrize("tie", [0.0, -1.0, 1.0])      # s(0) = +-1 have their own compare-select sign step
@pytest.mark.parametrize("kind", ["normal", "ties"])
def test_direct_backward(dev, shape, tie, kind):
    from weighted_abs_sum import _ext
    P, D, N, M, C = shape
    q, k, v = _data(P, D, N, M, C, seed=sum(shape) + 11, kind=kind)
    rng = np.random.default_rng(8)
    g_w = rng.standard_normal((P, M, C)).astype(np.float32)
    g_u = rng.standard_normal((P, M)).astype(np.float32)
    for full in (False, True):
        gq, gk, gv = _ext.weighted_abs_sum_direct_backward(_t(q, dev), _t(k, dev), _t(v, dev), _t(g_w, dev),
                                                           _t(g_u, dev) if full else None, tie)
        (wq, wk, wv), (nq, nk, nv) = brute.abs_backward(q, k, v, g_w, g_u if full else None, tie=tie)
        _assert_rel(_np(gq), wq, nq, f"direct grad_q tie={tie} full={full}")
        _assert_rel(_np(gk), wk, nk, f"direct grad_k tie={tie} full={full}")
        _assert_rel(_np(gv), wv, nv, f"direct grad_v full={full}")


@pytest.mark.parametrize("shape", DIRECT_SIGN_SHAPES)
@pytest.mark.parametrize("tie", [0.0, 1.0, -1.0, 0.5])
@pytest.mark.parametrize("kind", ["normal", "ties"])
def test_direct_sgn(dev, shape, tie, kind):
    from weighted_abs_sum import _ext
    P, D, N, M, C = shape
    q, k, v = _data(P, D, N, M, C, seed=sum(shape) + 12, kind=kind)
    g = np.random.default_rng(9).standard_normal((P, M, C)).astype(np.float32)
    out = _ext.weighted_sgn_sum_direct(_t(q, dev), _t(k, dev), _t(v, dev), _t(g, dev), tie)
    want, norm = brute.sgn_sum(q, k, v, g, tie=tie)
    _assert_rel(_np(out), want, norm, f"direct sgn tie={tie}")


def test_keops_route_tie_semantics(dev):
    # exact q == k ties: the "keops" backend follows KeOps' sign(0) = 0 in its gradients and in weighted_sgn_sum
    from weighted_abs_sum import weighted_abs_sum_full, weighted_sgn_sum
    P, D, N, M, C = 2, 3, 90, 70, 8
    q, k, v = _data(P, D, N, M, C, seed=41, kind="ties")
    rng = np.random.default_rng(10)
    g_w = rng.standard_normal((P, M, C)).astype(np.float32)
    g_u = rng.standard_normal((P, M)).astype(np.float32)
    tq, tk, tv = (_t(a, dev).requires_grad_(True) for a in (q, k, v))
    w, u = weighted_abs_sum_full(tq, tk, tv, backend="keops")
    ((w * _t(g_w, dev)).sum() + (u * _t(g_u, dev)).sum()).backward()
    (wq, wk, wv), (nq, nk, nv) = brute.abs_backward(q, k, v, g_w, g_u, tie=0.0)
    _assert_rel(_np(tq.grad), wq, nq, "keops grad_q (tie 0)")
    _assert_rel(_np(tk.grad), wk, nk, "keops grad_k (tie 0)")
    _assert_rel(_np(tv.grad), wv, nv, "keops grad_v")
    out = weighted_sgn_sum(_t(q, dev), _t(k, dev), _t(v, dev), _t(g_w, dev), backend="keops")
    want, norm = brute.sgn_sum(q, k, v, g_w, tie=0.0)
    _assert_rel(_np(out), want, norm, "keops sgn (tie 0)")


def test_stage_timer_busy_is_the_union(dev):
    # the dense backward runs grad_k on the side stream beside grad_q and grad_v: the stage timer's "busy" time (the
    # union of the launches' intervals) is positive, at most the sum of the launches' durations, and at least the
    # longest launch
    from qlka import _lib
    from weighted_abs_sum import _ext
    lib = _lib.load()
    P, D, N, M, C = 32, 64, 600, 600, 64
    q, k, v = _data(P, D, N, M, C, seed=5)
    rng = np.random.default_rng(12)
    g_w = _t(rng.standard_normal((P, M, C)).astype(np.float32), dev)
    g_u = _t(rng.standard_normal((P, M)).astype(np.float32), dev)
    tq, tk, tv = _t(q, dev), _t(k, dev), _t(v, dev)
    _ext.weighted_abs_sum_direct_backward(tq, tk, tv, g_w, g_u, -1.0)
    torch.cuda.synchronize()
    lib.qlka_timing_reset()
    lib.qlka_timing_enable(1)
    try:
        _ext.weighted_abs_sum_direct_backward(tq, tk, tv, g_w, g_u, -1.0)
        torch.cuda.synchronize()
    finally:
        lib.qlka_timing_enable(0)
    sign_ms, sign_n = _lib.stage_time("direct_sign")
    fwd_ms, fwd_n = _lib.stage_time("direct_fwd")
    busy, _ = _lib.stage_time("busy")
    lib.qlka_timing_reset()
    assert (sign_n, fwd_n) == (2, 1)
    assert 0.0 < busy <= sign_ms + fwd_ms + 1e-3
    assert busy >= max(fwd_ms, sign_ms / 2) - 1e-3


@pytest.mark.parametrize("shape", [(1, 2, 131072, 70000, 128), (2, 1, 50000, 131072, 65)])
def test_long_segments_wide_channels(dev, shape):
    # segments past one LDS sort run on both sides (merge passes, two-launch range scans, sorted queries instead of
    # grouped ones, v == 1 terms written in query order) with two channel slots per lane or an odd width and M != N:
    # both forwards on 8 queries per p, the _full backward on 8 queries and 8 keys per p, against the fp64 oracle
    from oracle import inputs
    from weighted_abs_sum import _ext
    from weighted_laplace_sum import weighted_laplace_sum
    P, D, N, M, C = shape
    print(f"long segments {shape}", flush=True)
    q, k, v = _data(P, D, N, M, C, seed=sum(shape) % 1000 + 21)
    rng = np.random.default_rng(23)
    g_w = rng.standard_normal((P, M, C)).astype(np.float32)
    g_u = rng.standard_normal((P, M)).astype(np.float32)
    tq, tk, tv = _t(q, dev), _t(k, dev), _t(v, dev)
    qidx = inputs.query_subsample(P, M, per_p=8, seed=5)

    def sub(a, idx, axis):                                   # (P, ..., X) -> the subsample along axis 1 + axis
        return np.stack([np.take(a[p], idx[p], axis=axis) for p in range(P)])

    w, u = weighted_laplace_sum(tq, tk, tv)
    ow, ou, nw = brute.laplace_sum(q, k, v, qidx=qidx)
    _assert_rel(sub(_np(w), qidx, 0), ow, nw, "long laplace out_w")
    _assert_rel(sub(_np(u), qidx, 0), ou, ou, "long laplace out_u")
    w, u = _ext.weighted_abs_sum_full_forward(tq, tk, tv)
    ow, ou, nw = brute.abs_sum(q, k, v, qidx=qidx)
    _assert_rel(sub(_np(w), qidx, 0), ow, nw, "long abs out_w")
    _assert_rel(sub(_np(u), qidx, 0), ou, ou, "long abs out_u")
    del w, u
    bq = inputs.query_subsample(P, M, per_p=8, seed=6)
    bk = inputs.query_subsample(P, N, per_p=8, seed=7)
    gq, gk, gv = _ext.weighted_abs_sum_full_backward(tq, tk, tv, _t(g_w, dev), _t(g_u, dev))
    (wq, wk, wv), (nq, nk, nv) = brute.abs_backward_sub(q, k, v, g_w, g_u, bq, bk)
    _assert_rel(sub(_np(gq), bq, 1), wq, nq, "long grad_q")
    _assert_rel(sub(_np(gk), bk, 1), wk, nk, "long grad_k")
    _assert_rel(sub(_np(gv), bk, 0), wv, nv, "long grad_v")


def test_largest_inputs(dev):
    # P * D * max(N, M) at the limit the boundary accepts (INT32_MAX): 255 p of 64 features over 131072 keys and
    # queries, 8.6 GB per input. The calls run 85 pipelined chunks of 3 p, the last of them 8.5 GB into each input and
    # output. Both forwards on 4 queries of the first, middle and last p, the _full backward on 4 queries and 4 keys
    # of the first and last p, against the fp64 oracle (every key, feature and channel).
    from weighted_abs_sum import _ext
    from weighted_laplace_sum import weighted_laplace_sum
    P, D, N, M, C = 255, 64, 131072, 131072, 64
    assert P * D * max(N, M) <= 2**31 - 1 < (P + 1) * D * max(N, M)
    print(f"largest inputs P={P} D={D} N={N} M={M} C={C}", flush=True)
    g = torch.Generator(device=dev).manual_seed(31)
    tq = torch.randn((P, D, M), generator=g, device=dev)
    tk = torch.randn((P, D, N), generator=g, device=dev)
    tv = torch.randn((P, N, C), generator=g, device=dev)
    ps = [0, P // 2, P - 1]
    ms = [0, 1, M // 2 + 3, M - 1]
    q, k, v = _np(tq[ps]), _np(tk[ps]), _np(tv[ps])
    qidx = np.array([ms] * len(ps))

    w, u = weighted_laplace_sum(tq, tk, tv)
    ow, ou, nw = brute.laplace_sum(q, k, v, qidx=qidx)
    _assert_rel(_np(w[ps][:, ms]), ow, nw, "largest laplace out_w")
    _assert_rel(_np(u[ps][:, ms]), ou, ou, "largest laplace out_u")
    del w, u
    w, u = _ext.weighted_abs_sum_full_forward(tq, tk, tv)
    ow, ou, nw = brute.abs_sum(q, k, v, qidx=qidx)
    _assert_rel(_np(w[ps][:, ms]), ow, nw, "largest abs out_w")
    _assert_rel(_np(u[ps][:, ms]), ou, ou, "largest abs out_u")
    del w, u

    g_w = torch.randn((P, M, C), generator=g, device=dev)
    g_u = torch.randn((P, M), generator=g, device=dev)
    gq, gk, gv = _ext.weighted_abs_sum_full_backward(tq, tk, tv, g_w, g_u)
    pb = [0, P - 1]
    bq = np.array([[2, 77, M // 3, M - 2]] * len(pb))
    bk = np.array([[0, 5000, N // 2, N - 1]] * len(pb))
    (wq, wk, wv), (nq, nk, nv) = brute.abs_backward_sub(_np(tq[pb]), _np(tk[pb]), _np(tv[pb]), _np(g_w[pb]),
                                                        _np(g_u[pb]), bq, bk)
    _assert_rel(_np(gq[pb][:, :, bq[0]]), wq, nq, "largest grad_q")
    _assert_rel(_np(gk[pb][:, :, bk[0]]), wk, nk, "largest grad_k")
    _assert_rel(_np(gv[pb][:, bk[0]]), wv, nv, "largest grad_v")


def test_largest_inputs_dense(dev):
    # The same limit on the dense route: 65535 p of 64 features over 512 keys and queries (8.6 GB per input) go to
    # the dense kernels in one launch each (about a million workgroups), whose per-p offsets pass 8 GB. Both forwards
    # and the _full backward on 4 queries / keys of the first, middle and last p against the fp64 oracle.
    from weighted_abs_sum import _ext
    from weighted_laplace_sum import weighted_laplace_sum
    P, D, N, M, C = 65535, 64, 512, 512, 64
    assert P * D * max(N, M) <= 2**31 - 1 < (P + 1) * D * max(N, M)
    print(f"largest dense inputs P={P} D={D} N={N} M={M} C={C}", flush=True)
    g = torch.Generator(device=dev).manual_seed(37)
    tq = torch.randn((P, D, M), generator=g, device=dev)
    tk = torch.randn((P, D, N), generator=g, device=dev)
    tv = torch.randn((P, N, C), generator=g, device=dev)
    ps = [0, P // 2, P - 1]
    ms = [0, 7, M // 2, M - 1]
    q, k, v = _np(tq[ps]), _np(tk[ps]), _np(tv[ps])
    qidx = np.array([ms] * len(ps))

    w, u = weighted_laplace_sum(tq, tk, tv)
    ow, ou, nw = brute.laplace_sum(q, k, v, qidx=qidx)
    _assert_rel(_np(w[ps][:, ms]), ow, nw, "largest dense laplace out_w")
    _assert_rel(_np(u[ps][:, ms]), ou, ou, "largest dense laplace out_u")
    del w, u
    w, u = _ext.weighted_abs_sum_full_forward(tq, tk, tv)
    ow, ou, nw = brute.abs_sum(q, k, v, qidx=qidx)
    _assert_rel(_np(w[ps][:, ms]), ow, nw, "largest dense abs out_w")
    _assert_rel(_np(u[ps][:, ms]), ou, ou, "largest dense abs out_u")
    del w, u

    g_w = torch.randn((P, M, C), generator=g, device=dev)
    g_u = torch.randn((P, M), generator=g, device=dev)
    gq, gk, gv = _ext.weighted_abs_sum_full_backward(tq, tk, tv, g_w, g_u)
    bq = np.array([[1, 100, 300, M - 1]] * len(ps))
    bk = np.array([[0, 64, 257, N - 2]] * len(ps))
    (wq, wk, wv), (nq, nk, nv) = brute.abs_backward_sub(q, k, v, _np(g_w[ps]), _np(g_u[ps]), bq, bk)
    _assert_rel(_np(gq[ps][:, :, bq[0]]), wq, nq, "largest dense grad_q")
    _assert_rel(_np(gk[ps][:, :, bk[0]]), wk, nk, "largest dense grad_k")
    _assert_rel(_np(gv[ps][:, bk[0]]), wv, nv, "largest dense grad_v")
