"""Concurrent calls from several host threads, each on its own stream.

The library keeps per-thread state only: the last error message and, per device, the side stream with its events to
which the chunk pipeline, the q sort and the dense backward fork. Two threads that issue pipelined calls on their own
torch streams at the same time must get, call after call, the results one thread gets alone, bit for bit (the library
is deterministic). Each thread has its own inputs, so a call that read or wrote another call's workspace, or waited
on another thread's events, would show as a difference.
"""

import threading

import pytest
import torch

pytestmark = pytest.mark.gpu

ITERS = 4
THREADS = 2
# P * D * M >= 2^22, so every op runs the two-copy chunk pipeline: at N = 16384 with the query grouping, at N = 22000
# with the q sort and the merge passes; N = 600 takes the dense kernels (the backward forks grad_k)
SHAPES = {
    "grouped": (4, 64, 16384, 16384, 64),
    "sorted_q": (3, 64, 22000, 22000, 32),
    "dense": (32, 64, 600, 600, 64),
}


def _inputs(dev, P, D, N, M, C, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(P, D, M, generator=g)
    k = torch.randn(P, D, N, generator=g)
    v = torch.randn(P, N, C, generator=g)
    g_w = torch.randn(P, M, C, generator=g)
    g_u = torch.randn(P, M, generator=g)
    return [t.to(dev) for t in (q, k, v, g_w, g_u)]


def _ops(q, k, v, g_w, g_u):
    from weighted_abs_sum import _ext, weighted_abs_sum_full
    from weighted_laplace_sum import weighted_laplace_sum
    w, u = weighted_laplace_sum(q, k, v)
    aw, au = weighted_abs_sum_full(q, k, v, backend="cuda")
    gq, gk, gv = _ext.weighted_abs_sum_full_backward(q, k, v, g_w, g_u)
    return [w, u, aw, au, gq, gk, gv]


@pytest.mark.parametrize("shape", list(SHAPES))
def test_threads_on_own_streams_match_one_thread(dev, shape):
    P, D, N, M, C = SHAPES[shape]
    print(f"threads x{THREADS}: {shape} P={P} D={D} N={N} M={M} C={C}", flush=True)
    inputs = [_inputs(dev, P, D, N, M, C, seed=100 + i) for i in range(THREADS)]
    with torch.no_grad():
        want = [[t.clone() for t in _ops(*inputs[i])] for i in range(THREADS)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device=dev) for _ in range(THREADS)]
    start = threading.Barrier(THREADS)
    errors = []

    def body(i):
        try:
            with torch.no_grad(), torch.cuda.stream(streams[i]):
                start.wait()
                got = [_ops(*inputs[i]) for _ in range(ITERS)]       # issued back to back, compared at the end
                for it, outs in enumerate(got):
                    for j, (a, b) in enumerate(zip(outs, want[i])):
                        if not torch.equal(a, b):
                            errors.append(f"thread {i} call {it} output {j}: max diff "
                                          f"{(a - b).abs().max().item():.3e}")
                streams[i].synchronize()
        except Exception as e:  # noqa: BLE001
            errors.append(f"thread {i}: {e!r}")

    ths = [threading.Thread(target=body, args=(i,)) for i in range(THREADS)]
    for t in ths:
        t.start()
    for t in ths:
        t.join(timeout=90)
    assert not any(t.is_alive() for t in ths), "a thread did not finish"
    torch.cuda.synchronize()
    assert not errors, "; ".join(errors[:5])
