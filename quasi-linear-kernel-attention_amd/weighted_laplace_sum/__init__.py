"""MI355X drop-in for the reference's weighted_laplace_sum package
(Weighted_Laplace_Sum/weighted_laplace_sum/__init__.py:1-16): same name, arguments, outputs and errors."""

from . import _ext


def weighted_laplace_sum(q, k, v):
    """The Laplace-kernel sums of every query against every key, in O((N + M) log N) per feature on gfx950.

    Inputs are float32, contiguous and on one device: queries q of shape (P, D, M), keys k (P, D, N) and value rows
    v (P, N, C), with C at most 128 and N, M at most 131072. Returns the pair

        out_w (P, M, C):  sum over features d and keys n of exp(-|k[p, d, n] - q[p, d, m]|) * v[p, n, :]
        out_u (P, M):     the same sum with every value row replaced by 1.

    There is no backward. For a batch padded with keys at k = 0, v = 0, each padded key adds exp(-|q_d|) per feature
    to out_u, which the caller removes (n_pad * sum_d exp(-|q_d|)).
    """
    return _ext.weighted_laplace_sum_forward(q, k, v)


__all__ = ["weighted_laplace_sum"]
