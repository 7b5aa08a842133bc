"""The allocation-free entry point qlka_laplace_fwd_noalloc, called through the C ABI, against qlka_laplace_fwd (the
entry point it is a variant of): the same kernels over a static workspace, so its outputs must equal qlka_laplace_fwd's
bit for bit, on consecutive calls of decreasing size (the static array keeps the previous call's contents), one of
them at the headline shape, where the static workspace holds one p and the call runs one p at a time."""

import numpy as np
import pytest
import torch

from oracle import brute

pytestmark = pytest.mark.gpu


def _noalloc():
    from qlka import _lib
    return _lib.load().qlka_laplace_fwd_noalloc


def _call(fn, q, k, v):
    """(out_w, out_u) of the entry point. The device's free memory (hipMemGetInfo, which sees every allocation on the
    device, the library's own included, unlike torch's allocator statistics) is the same before and after each of two
    calls; a first call may create the calling thread's side stream and events and resolve the static array's address,
    so it runs before the measured ones."""
    from qlka import _lib
    P, D, M = q.shape
    N, C = v.shape[1], v.shape[2]
    w = torch.full((P, M, C), float("nan"), device=q.device)
    u = torch.full((P, M), float("nan"), device=q.device)

    def call():
        _lib.check(fn(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(w), _lib.ptr(u), P, D, N, M, C,
                      _lib.stream_of(q.device)))

    call()
    for _ in range(2):
        w.fill_(float("nan"))
        u.fill_(float("nan"))
        torch.cuda.synchronize()
        free_before = torch.cuda.mem_get_info(q.device)[0]
        call()
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info(q.device)[0] == free_before, "the entry point allocated device memory"
    return w, u


def _inputs(P, D, N, M, C, seed, dev):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(P, D, M, generator=g)
    k = torch.randn(P, D, N, generator=g)
    v = torch.randn(P, N, C, generator=g)
    return q.to(dev), k.to(dev), v.to(dev)


def test_noalloc_equals_laplace_fwd(dev):
    from weighted_laplace_sum import weighted_laplace_sum
    fn = _noalloc()
    for shape, seed in (((12, 64, 16384, 16384, 64), 1), ((3, 5, 3000, 2500, 33), 2), ((2, 2, 700, 650, 8), 3)):
        P, D, N, M, C = shape
        q, k, v = _inputs(P, D, N, M, C, seed, dev)
        want_w, want_u = weighted_laplace_sum(q, k, v)
        w, u = _call(fn, q, k, v)
        assert torch.equal(w, want_w), f"{shape}: out_w differs from qlka_laplace_fwd"
        assert torch.equal(u, want_u), f"{shape}: out_u differs from qlka_laplace_fwd"
        if N <= 3000:    # and the oracle, where it is cheap
            qn, kn, vn = (t.cpu().numpy() for t in (q, k, v))
            ow, ou, nw = brute.laplace_sum(qn, kn, vn)
            assert float(brute.rel_err(w.cpu().numpy(), ow, nw).max()) <= 1e-5
            assert float(brute.rel_err(u.cpu().numpy(), ou, ou).max()) <= 1e-5
        del q, k, v, w, u, want_w, want_u


def test_noalloc_refuses_shapes_beyond_its_scratch(dev):
    """One p at N = M = 131072, D = C = 64 needs more than the static scratch: refused on the host with a message."""
    from qlka import _lib
    fn = _noalloc()
    lib = _lib.load()
    x = torch.zeros(16, device=dev)
    rc = fn(_lib.ptr(x), _lib.ptr(x), _lib.ptr(x), _lib.ptr(x), _lib.ptr(x), 1, 64, 131072, 131072, 64,
            _lib.stream_of(dev))
    assert rc != 0
    assert "static scratch" in lib.qlka_last_error().decode()
