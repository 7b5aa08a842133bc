"""Writes tests/golden/golden.npz: small input/output vectors of every boundary function, produced by the fp64
oracle (oracle/brute.py). The reference ships no test vectors for this path, so these fixtures pin regressions of
both the oracle and the GPU kernels; the oracle itself is pinned by tests/test_oracle.py.

    python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import brute  # noqa: E402

CASES = {
    # name: (P, D, N, M, C, kind)
    "small": (2, 3, 7, 5, 4, "normal"),
    "ties_pm0": (2, 2, 9, 11, 3, "ties"),
    "odd_c_m_ne_n": (1, 3, 40, 23, 5, "normal"),
    "single": (1, 1, 1, 1, 1, "normal"),
}


def make_case(P, D, N, M, C, kind, seed):
    rng = np.random.default_rng(seed)
    if kind == "ties":
        lv = np.array([-1.0, -0.5, -0.0, 0.0, 0.5, 1.0], dtype=np.float32)
        q = rng.choice(lv, size=(P, D, M)).astype(np.float32)
        k = rng.choice(lv, size=(P, D, N)).astype(np.float32)
    else:
        q = rng.standard_normal((P, D, M)).astype(np.float32)
        k = rng.standard_normal((P, D, N)).astype(np.float32)
    v = rng.standard_normal((P, N, C)).astype(np.float32)
    g_w = rng.standard_normal((P, M, C)).astype(np.float32)
    g_u = rng.standard_normal((P, M)).astype(np.float32)
    out = {"q": q, "k": k, "v": v, "g_w": g_w, "g_u": g_u}
    out["abs_w"], out["abs_u"], out["abs_norm"] = brute.abs_sum(q, k, v)
    out["lap_w"], out["lap_u"], out["lap_norm"] = brute.laplace_sum(q, k, v)
    out["sgn"], out["sgn_norm"] = brute.sgn_sum(q, k, v, g_w, tie=1.0)
    (out["gq"], out["gk"], out["gv"]), (out["nq"], out["nk"], out["nv"]) = brute.abs_backward(q, k, v, g_w, g_u)
    out["k_sorted"], out["k_perm"] = brute.stable_sort(k)
    out["rank"] = brute.merge_rank(q, k)
    return out


def main():
    arrays = {}
    for i, (name, (P, D, N, M, C, kind)) in enumerate(CASES.items()):
        for key, val in make_case(P, D, N, M, C, kind, seed=100 + i).items():
            arrays[f"{name}/{key}"] = val
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **arrays)
    print(f"wrote {len(arrays)} arrays")


if __name__ == "__main__":
    main()
