"""GPU checks of the workspace budget (qlka_set_workspace_budget): with a budget below one p's workspace every operator
runs its pipeline one p at a time, and its outputs must equal the unchunked call's bit for bit (each p's arithmetic
does not depend on the chunking) and the fp64 oracle within the usual 1e-5 of the sum of |term|."""

import numpy as np
import pytest
import torch

from oracle import brute

pytestmark = pytest.mark.gpu

REL = 1e-5


@pytest.fixture
def budget():
    """Call set(bytes) to change the workspace budget; the previous budget is restored afterwards."""
    from qlka import _lib
    lib = _lib.load()
    prev = lib.qlka_set_workspace_budget(8 << 30)
    lib.qlka_set_workspace_budget(prev)
    yield lambda b: lib.qlka_set_workspace_budget(int(b))
    lib.qlka_set_workspace_budget(prev)


def _inputs(P, D, N, M, C, seed, dev):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((P, D, M)).astype(np.float32)
    k = rng.standard_normal((P, D, N)).astype(np.float32)
    k[:, :, ::7] = q[:, :, :1]                      # exact ties between keys and one query per segment
    v = rng.standard_normal((P, N, C)).astype(np.float32)
    g = rng.standard_normal((P, M, C)).astype(np.float32)
    gu = rng.standard_normal((P, M)).astype(np.float32)
    return [torch.from_numpy(a).to(dev) for a in (q, k, v, g, gu)]


def _all_ops(q, k, v, g, gu):
    """Every operator that walks, on q, k, v: the forward ops, the backward (re-sorting and with kept sorts), the sgn
    sum and the three fused layers with and without a key mask."""
    from qlka import layers
    from weighted_abs_sum import _ext, weighted_abs_sum_full, weighted_sgn_sum
    from weighted_laplace_sum import weighted_laplace_sum
    out = {}
    out["laplace"] = weighted_laplace_sum(q, k, v)
    out["abs"] = _ext.weighted_abs_sum_full_forward(q, k, v)
    out["abs_plain"] = (_ext.weighted_abs_sum_forward(q, k, v),)
    out["bwd"] = _ext.weighted_abs_sum_full_backward(q, k, v, g, gu)
    tq, tk, tv = (t.detach().requires_grad_(True) for t in (q, k, v))
    w, u = weighted_abs_sum_full(tq, tk, tv, backend="cuda")          # kept sorts, then the sorted backward
    torch.autograd.backward([w, u], [g, gu])
    out["autograd"] = (w.detach(), u.detach(), tq.grad, tk.grad, tv.grad)
    out["sgn"] = (weighted_sgn_sum(q, k, v, g),)
    keep = torch.ones(q.shape[0], k.shape[2], dtype=torch.bool, device=q.device)
    keep[:, ::5] = False
    with torch.no_grad():
        for kern in layers.KINDS:
            out[kern] = (layers.layer_forward(kern, q, k, v),)
            out[kern + "_masked"] = (layers.layer_forward(kern, q, k, v, keep=keep),)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("shape", [(5, 4, 1500, 1300, 64), (3, 3, 20000, 700, 33)])
def test_one_p_chunks_equal_unchunked(dev, budget, shape):
    from qlka import _lib
    lib = _lib.load()
    P, D, N, M, C = shape
    q, k, v, g, gu = _inputs(P, D, N, M, C, seed=sum(shape), dev=dev)
    budget(8 << 30)
    whole = _all_ops(q, k, v, g, gu)
    one_p = lib.qlka_laplace_fwd_ws_bytes(1, D, N, M, C)
    assert lib.qlka_laplace_fwd_ws_bytes(P, D, N, M, C) > one_p
    budget(1)                                       # below one p: one p per pass
    assert lib.qlka_laplace_fwd_ws_bytes(P, D, N, M, C) == one_p
    chunked = _all_ops(q, k, v, g, gu)
    for name, outs in whole.items():
        for i, (a, b) in enumerate(zip(outs, chunked[name])):
            assert torch.equal(a, b), f"{name}[{i}]: chunked result differs from the unchunked one"
    # and the chunked forward sums against the oracle
    qn, kn, vn = (t.cpu().numpy() for t in (q, k, v))
    ow, ou, nw = brute.laplace_sum(qn, kn, vn)
    assert float(brute.rel_err(chunked["laplace"][0].cpu().numpy(), ow, nw).max()) <= REL
    ow, ou, nw = brute.abs_sum(qn, kn, vn)
    assert float(brute.rel_err(chunked["abs"][0].cpu().numpy(), ow, nw).max()) <= REL
    assert float(brute.rel_err(chunked["abs"][1].cpu().numpy(), ou, ou).max()) <= REL


def test_workspace_between_chunk_sizes(dev, budget):
    """A workspace that holds two p but not three runs in chunks of two (P = 5: 2 + 2 + 1), and a workspace below one
    p's is refused with the usual message."""
    from qlka import _lib
    from weighted_laplace_sum import weighted_laplace_sum
    lib = _lib.load()
    P, D, N, M, C = 5, 3, 2000, 1800, 16
    q, k, v, _, _ = _inputs(P, D, N, M, C, seed=3, dev=dev)
    want_w, want_u = weighted_laplace_sum(q, k, v)
    two = lib.qlka_laplace_fwd_ws_bytes(2, D, N, M, C)
    assert two < lib.qlka_laplace_fwd_ws_bytes(3, D, N, M, C)
    w = torch.empty(P, M, C, device=dev)
    u = torch.empty(P, M, device=dev)
    ws = torch.empty(two, dtype=torch.uint8, device=dev)
    _lib.check(lib.qlka_laplace_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(w), _lib.ptr(u), P, D, N, M, C,
                                    _lib.ptr(ws), two, _lib.stream_of(dev)))
    torch.cuda.synchronize()
    assert torch.equal(w, want_w) and torch.equal(u, want_u)
    one = lib.qlka_laplace_fwd_ws_bytes(1, D, N, M, C)
    rc = lib.qlka_laplace_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(w), _lib.ptr(u), P, D, N, M, C,
                              _lib.ptr(ws), one - 1, _lib.stream_of(dev))
    assert rc != 0 and "workspace too small" in lib.qlka_last_error().decode()
