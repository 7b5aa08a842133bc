"""torch restatement of the reference's own PyTorch path for this hot path. TEST / BASELINE INFRASTRUCTURE ONLY.

* dense_abs_sum / dense_laplace_sum: the dense formulas of Experiments/kernel_attention/kernels.py:73,81
  (|q - k| and exp(-|q - k|) summed over D into a (P, Mq, N) matrix, then @ v and .sum(-1)), evaluated in query
  chunks so one chunk's (P, D, chunk, N) intermediate stays below CHUNK = 2**28 entries (attention.py:21,41-50).
  bench.py times these on the host CPU as the reported CPU baseline ("kind": "port").
* add_laplace_layer / add_riesz_layer / add_bump_layer: the epilogues of Experiments/kernel_attention/attention.py:
  67-92 around the two ops, parameterised by the op implementations so the same epilogue runs over the GPU ops (the
  reference's own call pattern) or the dense CPU ops.
* attention: the layout/tau/keep handling of attention.py:95-126 for the three additive kernels.
"""

import torch

CHUNK = 2 ** 28     # attention.py:21
CLAMP = 1e-6        # attention.py:20
EPS = 1e-3          # kernels.py:9
TAU = {"add_laplace": 0.5, "add_riesz": 1.0, "add_bump": 1.5}   # kernels.py:18-20


def _chunks(P, D, M, N):
    c = max(1, CHUNK // max(1, P * D * N))
    return range(0, M, c), c


def dense_abs_sum(q, k, v):
    """(out_w, out_u) = (d1 @ v, d1.sum(-1)) with d1 = (q.unsqueeze(3) - k.unsqueeze(2)).abs().sum(1) (kernels.py:73)."""
    P, D, M = q.shape
    N = k.shape[2]
    starts, c = _chunks(P, D, M, N)
    ws, us = [], []
    for i in starts:
        d1 = (q[:, :, i:i + c].unsqueeze(3) - k.unsqueeze(2)).abs().sum(dim=1)   # (P, c, N)
        ws.append(d1 @ v)
        us.append(d1.sum(dim=-1))
    return torch.cat(ws, dim=1), torch.cat(us, dim=1)


def dense_laplace_sum(q, k, v):
    """(A @ v, A.sum(-1)) with A = exp(-|q - k|).sum(1) (kernels.py:81)."""
    P, D, M = q.shape
    N = k.shape[2]
    starts, c = _chunks(P, D, M, N)
    ws, us = [], []
    for i in starts:
        A = (-(q[:, :, i:i + c].unsqueeze(3) - k.unsqueeze(2)).abs()).exp().sum(dim=1)
        ws.append(A @ v)
        us.append(A.sum(dim=-1))
    return torch.cat(ws, dim=1), torch.cat(us, dim=1)


def add_laplace_layer(q, k, v, n_pad, laplace_fn):
    """attention.py:67-72."""
    out_w, out_u = laplace_fn(q.contiguous(), k.contiguous(), v.contiguous())
    den = out_u - n_pad * (-q.abs()).exp().sum(dim=1)
    return out_w / den.clamp_min(CLAMP)[:, :, None]


def add_riesz_layer(q, k, v, n_pad, abs_full_fn):
    """attention.py:75-81."""
    out_w, out_u = abs_full_fn(q.contiguous(), k.contiguous(), v.contiguous())
    aq, ak, S = q.abs().sum(dim=1), k.abs().sum(dim=1), q.shape[2]
    num = (aq + EPS)[:, :, None] * v.sum(dim=1)[:, None, :] + (ak[:, :, None] * v).sum(dim=1)[:, None, :] - out_w
    den = (aq + EPS) * S + ak.sum(dim=1, keepdim=True) - out_u - EPS * n_pad
    return num / den.clamp_min(CLAMP)[:, :, None]


def add_bump_layer(q, k, v, n_pad, abs_full_fn):
    """attention.py:84-92: max(0, 1 - |x|) = |x + 1| / 2 + |x - 1| / 2 - |x| with three abs sums."""
    w0, u0 = abs_full_fn(q.contiguous(), k.contiguous(), v.contiguous())
    wp, up = abs_full_fn((q + 1).contiguous(), k.contiguous(), v.contiguous())
    wm, um = abs_full_fn((q - 1).contiguous(), k.contiguous(), v.contiguous())
    num = (wp + wm) / 2 - w0
    den = (up + um) / 2 - u0 - n_pad * (1 - q.abs()).clamp_min(0).sum(dim=1)
    return num / den.clamp_min(CLAMP)[:, :, None]


def attention(q, k, v, kernel, tau, abs_full_fn, laplace_fn, keep=None):
    """The additive-kernel branch of attention() (attention.py:95-126): q, k, v (B, H, S, D) fp32 -> (B, H, S, D)."""
    B, H, S, D = q.shape
    P = B * H
    q = q.transpose(2, 3).reshape(P, D, S)
    k = k.transpose(2, 3).reshape(P, D, S)
    v = v.reshape(P, S, D)
    keep = None if keep is None else keep.repeat_interleave(H, dim=0)
    q, k, n_pad = q / tau, k / tau, 0
    if keep is not None:
        k, v = k * keep[:, None, :], v * keep[:, :, None]
        n_pad = S - keep.sum(dim=1, keepdim=True)
    if kernel == "add_laplace":
        out = add_laplace_layer(q, k, v, n_pad, laplace_fn)
    elif kernel == "add_riesz":
        out = add_riesz_layer(q, k, v, n_pad, abs_full_fn)
    elif kernel == "add_bump":
        out = add_bump_layer(q, k, v, n_pad, abs_full_fn)
    else:
        raise ValueError(kernel)
    return out.view(B, H, S, D)


def dense_kernel_matrix(kernel, q, k, tau=1.0, mask=None):
    """The naive kernel matrices of kernels.py:68-89 (P, Sq, Sk), for small-size layer checks."""
    q, k = q / tau, k / tau
    x = q.unsqueeze(3) - k.unsqueeze(2)
    if kernel == "add_riesz":
        A = q.abs().sum(dim=1)[:, :, None] + k.abs().sum(dim=1)[:, None, :] - x.abs().sum(dim=1) + EPS
    elif kernel == "add_laplace":
        A = (-x.abs()).exp().sum(dim=1)
    elif kernel == "add_bump":
        A = (1.0 - x.abs()).clamp(min=0.0).sum(dim=1)
    else:
        raise ValueError(kernel)
    return A if mask is None else A * mask[:, None, :]
