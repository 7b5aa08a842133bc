"""Golden fixtures (tests/golden/golden.npz, written by tests/golden/make_golden.py from the fp64 oracle): the oracle
must keep reproducing them (CPU), and the GPU kernels must match them (GPU, 1e-5 of the sum of |term|, bit-exact
sort permutations and ranks)."""

import os

import numpy as np
import pytest

from oracle import brute

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
CASES = ("small", "ties_pm0", "odd_c_m_ne_n", "single")


def _case(name):
    z = np.load(GOLDEN)
    return {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(name + "/")}


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_golden(name):
    c = _case(name)
    q, k, v, g_w, g_u = c["q"], c["k"], c["v"], c["g_w"], c["g_u"]
    w, u, _ = brute.abs_sum(q, k, v)
    np.testing.assert_array_equal(w, c["abs_w"])
    np.testing.assert_array_equal(u, c["abs_u"])
    w, u, _ = brute.laplace_sum(q, k, v)
    np.testing.assert_array_equal(w, c["lap_w"])
    s, _ = brute.sgn_sum(q, k, v, g_w, tie=1.0)
    np.testing.assert_array_equal(s, c["sgn"])
    (gq, gk, gv), _ = brute.abs_backward(q, k, v, g_w, g_u)
    np.testing.assert_array_equal(gq, c["gq"])
    np.testing.assert_array_equal(gk, c["gk"])
    np.testing.assert_array_equal(gv, c["gv"])
    srt, perm = brute.stable_sort(k)
    np.testing.assert_array_equal(perm, c["k_perm"])
    np.testing.assert_array_equal(brute.merge_rank(q, k), c["rank"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_gpu_matches_golden(dev, name):
    import torch

    from qlka import ops
    from weighted_abs_sum import _ext, weighted_sgn_sum
    from weighted_laplace_sum import weighted_laplace_sum

    c = _case(name)
    t = {key: torch.from_numpy(np.ascontiguousarray(val)).to(dev) for key, val in c.items()
         if key in ("q", "k", "v", "g_w", "g_u")}

    def rel(got, want, norm, what):
        err = float(brute.rel_err(got.detach().cpu().numpy(), want, norm).max())
        assert err <= 1e-5, f"{name} {what}: {err:.3e}"

    w, u = _ext.weighted_abs_sum_full_forward(t["q"], t["k"], t["v"])
    rel(w, c["abs_w"], c["abs_norm"], "abs out_w")
    rel(u, c["abs_u"], c["abs_u"], "abs out_u")
    w, u = weighted_laplace_sum(t["q"], t["k"], t["v"])
    rel(w, c["lap_w"], c["lap_norm"], "laplace out_w")
    rel(u, c["lap_u"], c["lap_u"], "laplace out_u")
    s = weighted_sgn_sum(t["q"], t["k"], t["v"], t["g_w"], backend="cuda")
    rel(s, c["sgn"], c["sgn_norm"], "sgn")
    gq, gk, gv = _ext.weighted_abs_sum_full_backward(t["q"], t["k"], t["v"], t["g_w"], t["g_u"])
    rel(gq, c["gq"], c["nq"], "grad_q")
    rel(gk, c["gk"], c["nk"], "grad_k")
    rel(gv, c["gv"], c["nv"], "grad_v")
    P, D, N = c["k"].shape
    srt, perm = ops.seg_sort(t["k"])
    np.testing.assert_array_equal(perm.cpu().numpy(), c["k_perm"])
    np.testing.assert_array_equal(srt.cpu().numpy(), c["k_sorted"])
    r = ops.merge_rank(t["q"], t["k"])
    np.testing.assert_array_equal(r.cpu().numpy(), c["rank"])
