"""The ops under HIP graph capture (torch.cuda.graph).

Each case is captured once and replayed three times, with eager work and synchronisations between the replays; every
replay must equal the eager result bit for bit (the library is deterministic, launches no memset and allocates
nothing itself). The forward ops and the fused layers fork a side stream for the q sort and the query bounds and join
it with events; under capture that fork / join becomes graph dependencies, which these cases exercise.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(dev, P, D, N, M, C, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(P, D, M, generator=g)
    k = torch.randn(P, D, N, generator=g)
    v = torch.randn(P, N, C, generator=g)
    g_w = torch.randn(P, M, C, generator=g)
    g_u = torch.randn(P, M, generator=g)
    return [t.to(dev) for t in (q, k, v, g_w, g_u)]


def _cases():
    from weighted_abs_sum import _ext, weighted_abs_sum_full
    from weighted_laplace_sum import weighted_laplace_sum
    from qlka import layers

    return {
        # N = M = 1500: above every dense cutoff, so sort + walk with the side-stream fork
        "laplace_walk": ((2, 3, 1500, 1500, 16), lambda q, k, v, gw, gu: weighted_laplace_sum(q, k, v)),
        "abs_full_walk": ((2, 3, 1500, 1500, 16),
                          lambda q, k, v, gw, gu: weighted_abs_sum_full(q, k, v, backend="cuda")),
        "abs_full_backward_walk": ((2, 3, 1500, 1400, 16),
                                   lambda q, k, v, gw, gu: _ext.weighted_abs_sum_full_backward(q, k, v, gw, gu)),
        "add_bump_layer": ((2, 3, 1500, 1500, 16), lambda q, k, v, gw, gu: layers.layer_forward("add_bump", q, k, v)),
        # masked keys: the Laplace layer replaces them by FLT_MAX in its workspace before the sort
        "add_laplace_masked_layer": ((2, 3, 1500, 1500, 16),
                                     lambda q, k, v, gw, gu: layers.layer_forward("add_laplace", q, k, v,
                                                                                  keep=v[:, :, 0] > -0.5)),
        # the allocation-free entry point (a static workspace, two chunks of p pipelined over the side stream)
        "laplace_noalloc": ((3, 4, 3000, 2500, 33), _laplace_noalloc),
        # short segments: the dense kernels
        "abs_full_dense": ((64, 8, 65, 65, 32),
                           lambda q, k, v, gw, gu: weighted_abs_sum_full(q, k, v, backend="cuda")),
        "abs_backward_dense": ((16, 8, 300, 250, 20),
                               lambda q, k, v, gw, gu: _ext.weighted_abs_sum_full_backward(q, k, v, gw, gu)),
    }


def _laplace_noalloc(q, k, v, gw, gu):
    """qlka_laplace_fwd_noalloc through the C ABI on the current (capturing) stream: the library's static workspace,
    no allocation by the library inside the capture."""
    from qlka import _lib
    P, D, M = q.shape
    N, C = v.shape[1], v.shape[2]
    w = torch.empty(P, M, C, device=q.device)
    u = torch.empty(P, M, device=q.device)
    _lib.check(_lib.load().qlka_laplace_fwd_noalloc(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(w), _lib.ptr(u),
                                                    P, D, N, M, C, _lib.stream_of(q.device)))
    return w, u


def _flat(out):
    return [t for t in (out if isinstance(out, (tuple, list)) else (out,)) if t is not None]


@pytest.mark.parametrize("case", ["laplace_walk", "abs_full_walk", "abs_full_backward_walk", "add_bump_layer",
                                  "add_laplace_masked_layer", "laplace_noalloc", "abs_full_dense",
                                  "abs_backward_dense"])
def test_graph_replays_equal_eager(dev, case):
    shape, fn = _cases()[case]
    args = _inputs(dev, *shape, seed=sum(shape))
    with torch.no_grad():
        eager = [t.clone() for t in _flat(fn(*args))]
        side = torch.cuda.Stream(device=dev)              # warm up off the capture stream (torch's pattern)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(2):
                fn(*args)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            captured = _flat(fn(*args))
        for r in range(3):
            for t in captured:
                t.fill_(float("nan"))                     # a replay must rewrite every output
            graph.replay()
            torch.cuda.synchronize(dev)
            for i, (got, want) in enumerate(zip(captured, eager)):
                assert torch.equal(got, want), f"{case}: replay {r}, output {i} differs from the eager result"
            busy = torch.randn(1 << 20, device=dev)       # eager work between replays
            assert torch.isfinite(busy.sum())
            torch.cuda.synchronize(dev)


def test_first_call_of_a_thread_captured(dev):
    # A thread whose very first library call is captured has no side stream yet; creating one inside the capture would
    # invalidate it, so that call runs in order on the captured stream. Checked on a fresh thread, against eager.
    import threading
    shape, fn = _cases()["abs_full_walk"]
    args = _inputs(dev, *shape, seed=7)
    with torch.no_grad():
        eager = [t.clone() for t in _flat(fn(*args))]
    result = {}

    def body():
        try:
            torch.cuda.set_device(dev)
            with torch.no_grad():
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    captured = _flat(fn(*args))
                for _ in range(2):
                    for t in captured:
                        t.fill_(float("nan"))
                    graph.replay()
                    torch.cuda.synchronize(dev)
                    result.setdefault("equal", []).append(all(torch.equal(a, b) for a, b in zip(captured, eager)))
        except Exception as e:                            # reported on the test's thread
            result["error"] = repr(e)

    th = threading.Thread(target=body)
    th.start()
    th.join()
    assert "error" not in result, result.get("error")
    assert result["equal"] == [True, True]
