"""Fused additive-kernel attention layers (add_laplace, add_riesz, add_bump) over libqlka's qlka_layer_fwd.

Mirrors Experiments/kernel_attention/attention.py:
  * add_laplace / add_riesz / add_bump(q, k, v, n_pad) are attention.py:67-92 (`_add_laplace`, `_add_riesz`,
    `_add_bump`): q (P, D, S) and k (P, D, N) already divided by tau, k and v already multiplied by the key mask,
    n_pad the number of masked keys per p (0 or a (P,) / (P, 1) tensor); returns (P, S, C).
  * attention(q, k, v, kernel, tau, keep=None) is the additive-kernel branch of attention() (attention.py:95-126):
    (B, H, S, D) in and out, tau scaling, key mask.
  * layer_forward(kernel, q, k, v, keep=...) applies a key mask inside the sums (qlka_layer_fwd_masked): k and v are
    passed as they are, masked keys weigh 0, and no n_pad correction is needed. attention() takes this route for a
    mask when no gradient is needed.

Forward through one library call per layer: the op(s) and the normalising epilogue run on the GPU in one stream of
kernels, and add_bump's three abs sums (q, q + 1, q - 1) share one sort of k and q and one set of key-range
summaries. The fused call has no gradient. When a gradient is needed, add_riesz and add_bump evaluate the reference's
own formulas over the differentiable weighted_abs_sum_full (the same arithmetic as attention.py:75-92); add_laplace
raises like weighted_laplace_sum, which has no backward (attention.py:110-114 routes that case elsewhere).
"""

import torch

from . import _lib

CLAMP = 1e-6    # attention.py:20
EPS = 1e-3      # kernels.py:9
KEOPS_BELOW = 256   # attention.py:22: the reference's abs sums take backend "keops" below this many queries
KINDS = {"add_laplace": 0, "add_riesz": 1, "add_bump": 2}


def _check(q, k, v):
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not t.is_cuda:
            raise RuntimeError(f"{name} must be a CUDA tensor")
        if t.dtype != torch.float32:
            raise RuntimeError(f"{name} must be float32")
        if t.dim() != 3:
            raise RuntimeError(f"{name} must be 3D")
    if q.shape[0] != k.shape[0] or q.shape[1] != k.shape[1] or v.shape[0] != q.shape[0] or v.shape[1] != k.shape[2]:
        raise RuntimeError("expected q (P, D, M), k (P, D, N), v (P, N, C)")
    if not (q.device == k.device == v.device):
        raise RuntimeError("q, k and v must be on the same device")


def _n_pad(n_pad, P, device):
    if n_pad is None or (isinstance(n_pad, (int, float)) and n_pad == 0):
        return None
    t = torch.as_tensor(n_pad, dtype=torch.float32, device=device)
    if t.numel() == 1:
        t = t.reshape(1).expand(P)
    return t.reshape(P).contiguous()


def _keep(keep, P, N, device):
    """(P, N) key mask (bool or 0/1) as contiguous bytes, nonzero = kept."""
    if keep.shape != (P, N):
        raise RuntimeError(f"keep must be (P, N) = ({P}, {N}), got {tuple(keep.shape)}")
    if keep.device != device:
        raise RuntimeError("keep must be on the device of q, k and v")
    return (keep != 0).to(torch.uint8).contiguous()


def layer_forward(kernel, q, k, v, n_pad=0, keep=None):
    """One fused forward of `kernel` in ("add_laplace", "add_riesz", "add_bump"); returns (P, M, C). No autograd.

    keep=None: the reference's composition, k and v already multiplied by the key mask and n_pad the count of masked
    keys per p. keep (P, N): the mask applied inside the sums (k and v unmasked, n_pad unused)."""
    if kernel not in KINDS:
        raise ValueError(f"unknown additive kernel {kernel!r}")
    _check(q, k, v)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    P, D, M = q.shape
    N, C = k.shape[2], v.shape[2]
    out = torch.empty(P, M, C, dtype=torch.float32, device=q.device)
    lib = _lib.load()
    kind = KINDS[kernel]
    with torch.cuda.device(q.device):
        nbytes = lib.qlka_layer_fwd_ws_bytes(kind, P, D, N, M, C)
        ws = _lib.workspace(nbytes, q.device)
        if keep is None:
            npad = _n_pad(n_pad, P, q.device)
            rc = lib.qlka_layer_fwd(kind, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(npad), _lib.ptr(out),
                                    P, D, N, M, C, _lib.ptr(ws), nbytes, _lib.stream_of(q.device))
        else:
            kb = _keep(keep, P, N, q.device)
            rc = lib.qlka_layer_fwd_masked(kind, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(kb), _lib.ptr(out),
                                           P, D, N, M, C, _lib.ptr(ws), nbytes, _lib.stream_of(q.device))
        _lib.check(rc)
    return out


def _needs_grad(*ts):
    return torch.is_grad_enabled() and any(t.requires_grad for t in ts)


def add_laplace(q, k, v, n_pad=0):
    """attention.py:67-72: weighted_laplace_sum normalised by its row sum (padded keys removed). Forward only."""
    if _needs_grad(q, k, v):
        raise RuntimeError("add_laplace: weighted_laplace_sum has no backward (forward-only operator)")
    return layer_forward("add_laplace", q, k, v, n_pad)


def unfused(kernel, q, k, v, n_pad=0):
    """The layer as separate op calls plus a torch epilogue: the arithmetic of attention.py:67-92, differentiable for
    add_riesz / add_bump through weighted_abs_sum_full's autograd. The abs sums run on the backend the reference's
    _abs_sum picks (attention.py:60-63): "keops" below KEOPS_BELOW queries (a gradient tie then counts 0), else
    "cuda". q (P, D, M), k (P, D, N), v (P, N, C); n_pad a number or (P, 1)."""
    from weighted_abs_sum import weighted_abs_sum_full
    from weighted_laplace_sum import weighted_laplace_sum

    backend = "keops" if q.shape[2] < KEOPS_BELOW else "cuda"
    keys, vals = k.contiguous(), v.contiguous()

    def sums(queries):                                   # (w (P, M, C), u (P, M)) of the abs kernel at these queries
        return weighted_abs_sum_full(queries.contiguous(), keys, vals, backend=backend)

    def normalise(num, den):                             # rows divided by their clamped weight
        return num / den.clamp_min(CLAMP).unsqueeze(2)

    if kernel == "add_laplace":
        w, u = weighted_laplace_sum(q.contiguous(), keys, vals)
        per_pad = torch.exp(-q.abs()).sum(dim=1)         # a key at 0: sum_d e^{-|q_d|} in u, nothing in w
        return normalise(w, u - n_pad * per_pad)
    if kernel == "add_riesz":
        # A[m, n] = |q_m|_1 + |k_n|_1 - |q_m - k_n|_1 + EPS summed against [v, 1]
        w, u = sums(q)
        qn = q.abs().sum(dim=1) + EPS                    # (P, M)
        kn = k.abs().sum(dim=1)                          # (P, N)
        v_tot = v.sum(dim=1).unsqueeze(1)                # (P, 1, C)
        kv_tot = torch.bmm(kn.unsqueeze(1), vals)        # (P, 1, C): sum_n |k_n|_1 v_n
        num = qn.unsqueeze(2) * v_tot + kv_tot - w
        den = qn * q.shape[2] + kn.sum(dim=1, keepdim=True) - u - EPS * n_pad
        return normalise(num, den)
    if kernel == "add_bump":
        # max(0, 1 - |x|) = (|x + 1| + |x - 1|) / 2 - |x|, x = q_d - k_d
        (w0, u0), (w1, u1), (w2, u2) = sums(q), sums(q + 1), sums(q - 1)
        per_pad = (1 - q.abs()).clamp_min(0).sum(dim=1)  # a key at 0: sum_d max(0, 1 - |q_d|) in u
        return normalise((w1 + w2) / 2 - w0, (u1 + u2) / 2 - u0 - n_pad * per_pad)
    raise ValueError(f"unknown additive kernel {kernel!r}")


def add_riesz(q, k, v, n_pad=0):
    """attention.py:75-81: A = |q|_1 + |k|_1 - |q - k|_1 + eps through one weighted_abs_sum_full."""
    if _needs_grad(q, k, v):
        return unfused("add_riesz", q, k, v, n_pad)
    return layer_forward("add_riesz", q, k, v, n_pad)


def add_bump(q, k, v, n_pad=0):
    """attention.py:84-92: max(0, 1 - |x|) = |x + 1| / 2 + |x - 1| / 2 - |x| through three abs sums."""
    if _needs_grad(q, k, v):
        return unfused("add_bump", q, k, v, n_pad)
    return layer_forward("add_bump", q, k, v, n_pad)


LAYERS = {"add_laplace": add_laplace, "add_riesz": add_riesz, "add_bump": add_bump}


def attention(q, k, v, kernel, tau, keep=None):
    """The additive-kernel branch of attention() (attention.py:95-126): q, k, v (B, H, S, D) fp32 -> (B, H, S, D).

    keep (B, S) marks the real keys (bool or 0/1). Without a gradient the mask is applied inside the fused layer's
    sums; with one, masked keys become k = 0, v = 0 and leave the row sums through n_pad, as in the reference.
    """
    if kernel not in LAYERS:
        raise ValueError(f"attention: kernel {kernel!r} is not one of {sorted(LAYERS)}")
    assert q.dtype == k.dtype == v.dtype == torch.float32, "kernel attention runs in fp32 only"
    B, H, S, D = q.shape

    def features_first(x):                               # (B, H, S, D) -> (B*H, D, S), scaled by 1 / tau
        return x.permute(0, 1, 3, 2).reshape(B * H, D, S) / tau

    qf, kf, vf = features_first(q), features_first(k), v.reshape(B * H, S, D)
    head_keep = None if keep is None else keep.unsqueeze(1).expand(B, H, S).reshape(B * H, S)
    if head_keep is not None and not _needs_grad(qf, kf, vf):
        return layer_forward(kernel, qf, kf, vf, keep=head_keep).view(B, H, S, D)
    n_pad = 0
    if head_keep is not None:
        w8 = head_keep.to(kf.dtype)
        kf, vf = kf * w8.unsqueeze(1), vf * w8.unsqueeze(2)
        n_pad = S - w8.sum(dim=1, keepdim=True)
    return LAYERS[kernel](qf, kf, vf, n_pad).view(B, H, S, D)

