"""Seeded synthetic inputs for the five BASELINE.json configurations. TEST / BENCH INFRASTRUCTURE ONLY.

Every config draws from numpy default_rng(PCG64(seed)) in the order q, k, v[, g_w, g_u], fp32, in the reference's
layouts q (P, D, M), k (P, D, N), v (P, N, C), g_w (P, M, C), g_u (P, M).
"""

import numpy as np

# name: (P, D, N, M, C, kind)
CONFIGS = {
    0: dict(name="abs fwd+bwd, associative-recall scale", P=32, D=64, N=600, M=600, C=64, kind="normal", scale=1.0),
    1: dict(name="ViT-scale many small segments", P=512, D=32, N=65, M=65, C=32, kind="normal", scale=1.0),
    2: dict(name="laplace fwd, text inference", P=12, D=64, N=8192, M=8192, C=64, kind="normal", scale=2.0),
    3: dict(name="headline B=1 H=12 N=16384 D=Dv=64", P=12, D=64, N=16384, M=16384, C=64, kind="normal", scale=1.0),
    4: dict(name="stress N=131072, heavy ties", P=12, D=64, N=131072, M=131072, C=64, kind="mixture", scale=1.0),
}


def _mixture(rng, shape):
    """Per element, Bernoulli(0.5) picks 8 * N(0,1) or one of 256 exact levels (randint(0, 256) - 128) / 16."""
    pick = rng.random(shape) < 0.5
    wide = rng.standard_normal(shape, dtype=np.float32) * np.float32(8.0)
    lvl = ((rng.integers(0, 256, size=shape) - 128) / 16).astype(np.float32)
    return np.where(pick, wide, lvl).astype(np.float32)


def make(P, D, N, M, C, kind="normal", scale=1.0, seed=0, grads=False):
    """dict with q, k, v (and g_w, g_u if grads) as fp32 numpy arrays."""
    rng = np.random.default_rng(np.random.PCG64(seed))
    out = {}
    if kind == "normal":
        out["q"] = rng.standard_normal((P, D, M), dtype=np.float32) * np.float32(scale)
        out["k"] = rng.standard_normal((P, D, N), dtype=np.float32) * np.float32(scale)
        out["v"] = rng.standard_normal((P, N, C), dtype=np.float32)
    elif kind == "mixture":
        out["q"] = _mixture(rng, (P, D, M))
        out["k"] = _mixture(rng, (P, D, N))
        out["v"] = rng.standard_t(3, size=(P, N, C)).astype(np.float32)
    else:
        raise ValueError(kind)
    if grads:
        out["g_w"] = rng.standard_normal((P, M, C), dtype=np.float32)
        out["g_u"] = rng.standard_normal((P, M), dtype=np.float32)
    return out


def config(i, seed=0, grads=False, **override):
    c = dict(CONFIGS[i])
    c.update(override)
    return make(c["P"], c["D"], c["N"], c["M"], c["C"], c["kind"], c["scale"], seed=seed, grads=grads)


def query_subsample(P, M, per_p=32, seed=1):
    """Seeded (P, per_p) query indices for oracle checks at large M (sorted, without replacement)."""
    rng = np.random.default_rng(np.random.PCG64(seed))
    per_p = min(per_p, M)
    return np.stack([np.sort(rng.choice(M, size=per_p, replace=False)) for _ in range(P)])
