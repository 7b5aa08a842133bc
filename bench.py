"""Benchmark of the MI355X hot path: weighted_laplace_sum + weighted_abs_sum_full forward at the headline shape.

One step = one weighted_laplace_sum forward and one weighted_abs_sum_full forward (the two ops the add_laplace and
add_riesz / add_bump layers call) over one batch of BASELINE.json configs[3]: B=1, H=12 (P=12), N=M=16384,
D=Dv=64, fp32, q, k, v ~ N(0,1) drawn from numpy PCG64(seed 0) in the order q, k, v, resident in HBM before timing.

Prints ONE JSON line (rank 0, N=1), only after both ops' outputs on the bench inputs match the fp64 oracle on a
query subsample (`parity`). `value` = query-feature sums per second over the whole step (2 * P*M*D units per step),
timed with events around the steps only. `roofline.frac` = B_scan of the step's two op calls / step time / 8 TB/s
(the op-level figure the north-star target is set on, also per op in `op_frac`); `roofline.kernel` is the kernel
with the most GPU time on its own algorithmic bytes per launch, its launch time taken in a second, instrumented pass
(libqlka's hipEvent stage timer on the kernel's own stream). `cpu_baseline` times the reference's dense PyTorch path
(restated in oracle/dense.py) on the host CPU on a bounded query sample of the same workload.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu-baseline] [--no-layers] [--no-configs]
    python bench.py --profile-config I [--steps K]     (one other configuration alone, e.g. under rocprofv3)
"""

import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "quasi-linear-kernel-attention_amd")
sys.path.insert(0, PKG)
sys.path.insert(0, REPO)

import numpy as np  # noqa: E402
import torch  # noqa: E402

METRIC = "query-feature sums/sec (B·H·N·D) at N=16384 D=64 fp32; achieved HBM GB/s %peak"
HBM_PEAK_GBS = 8000.0
P, D, N, M, C = 12, 64, 16384, 16384, 64

# Algorithmic bytes per (p, d, m) query-feature unit of one op call at N = M ("B_scan"):
# read the key and query segments once (4 N + 4 M per (p, d)), stream v once in sorted order (4 N C), emit one fp32
# contribution per (query, channel) (4 M C) plus out_u (4 M); divided by the M units of a (p, d) segment.
def bscan_bytes_per_unit(n, m, c, with_u=True):
    return 4.0 * (n + m + n * c + m * c + (m if with_u else 0)) / m


def make_inputs(dev, seed=0):
    rng = np.random.default_rng(np.random.PCG64(seed))
    q = rng.standard_normal((P, D, M), dtype=np.float32)
    k = rng.standard_normal((P, D, N), dtype=np.float32)
    v = rng.standard_normal((P, N, C), dtype=np.float32)
    return [torch.from_numpy(a).to(dev) for a in (q, k, v)]


# The other BASELINE.json configurations, timed as extra fields of the JSON line (their workloads as BASELINE.json
# states them; `value` stays the headline). Inputs are drawn on the GPU with a seeded torch generator in the same
# distributions as the parity tests: N(0,1) * scale, or for configs[4] a per-element 50/50 mixture of 8 * N(0,1) and
# 256 exact levels (heavy ties) with v ~ Student-t(3).
CONFIGS = {
    0: dict(P=32, D=64, N=600, C=64, kind="normal", scale=1.0, work="weighted_abs_sum_full fwd+bwd (autograd)"),
    1: dict(P=512, D=32, N=65, C=32, kind="normal", scale=1.0, work="weighted_laplace_sum + weighted_abs_sum_full fwd"),
    2: dict(P=12, D=64, N=8192, C=64, kind="normal", scale=2.0, work="weighted_laplace_sum fwd"),
    4: dict(P=12, D=64, N=131072, C=64, kind="mixture", scale=1.0,
            work="weighted_abs_sum_full fwd+bwd + weighted_laplace_sum fwd"),
}


def config_inputs(c, dev, seed=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    P, D, N, C = c["P"], c["D"], c["N"], c["C"]

    def side(shape):
        if c["kind"] == "normal":
            return torch.randn(shape, generator=g, device=dev) * c["scale"]
        pick = torch.rand(shape, generator=g, device=dev) < 0.5
        wide = torch.randn(shape, generator=g, device=dev) * 8.0
        lvl = (torch.randint(0, 256, shape, generator=g, device=dev) - 128).float() / 16
        return torch.where(pick, wide, lvl)

    q, k = side((P, D, N)), side((P, D, N))
    if c["kind"] == "normal":
        v = torch.randn((P, N, C), generator=g, device=dev)
    else:   # Student-t(3) = N(0,1) / sqrt(chi2(3) / 3)
        z = torch.randn((P, N, C), generator=g, device=dev)
        chi2 = torch.randn((3, P, N, C), generator=g, device=dev).square().sum(0)
        v = z / torch.sqrt(chi2 / 3)
    g_w = torch.randn((P, N, C), generator=g, device=dev)
    g_u = torch.randn((P, N), generator=g, device=dev)
    return q, k, v, g_w, g_u


FP32_PEAK_TFLOPS = 157.3     # MI355X dense fp32 (matrix and vector with packed math)


def dense_flops(i, c):
    """Algorithmic flops of configuration i's workload on the dense route (configs[0], [1]): forming
    A[m, n] = sum_d f(q_d - k_d) costs a subtract and an add per (m, n, d) (|x| is a free operand modifier) plus the
    exponential for the Laplace kernel, the contraction A^T [v, 1] 2 (C + 1) per (m, n); each sign sum of the backward
    forms G = X Y^T (2 C per (i, j)) and adds a selected +-G per (d, i, j) (2); grad_v contracts the A the forward kept
    with g_w (2 C per (m, n): a differentiable dense call keeps A, qlka_abs_fwd_dense_keep)."""
    P, D, N, C = c["P"], c["D"], c["N"], c["C"]
    M = N
    fwd_abs = 2.0 * P * M * N * D + 2.0 * P * M * N * (C + 1)
    if i == 0:
        sign = 2.0 * P * M * N * C + 2.0 * P * D * M * N
        grad_v = 2.0 * P * M * N * C
        return fwd_abs + 2 * sign + grad_v
    if i == 1:
        fwd_lap = 3.0 * P * M * N * D + 2.0 * P * M * N * (C + 1)
        return fwd_lap + fwd_abs
    return None


def config_timings(dev, reps=None, only=None):
    """ms per call of each configuration's workload: the mean over `reps` calls (default 20; 3 for configs[4]), each
    bracketed by events after a synchronisation, following warmup calls (5; 1 for configs[4]), as the reference's
    speed bench times a step (Experiments/speed_and_memory/bench.py:106-118). For the dense-route configurations [0]
    and [1] also the library kernels' own time per call (libqlka's stage timer, a separate pass: `kernel_ms` is the
    time in which at least one library kernel ran, the union over both streams; `kernel_sum_ms` the sum of the
    launches' durations), the share of the call that is not kernel time (`host_frac`) and the flop rate against the
    fp32 peak (`flop_frac`, over the whole call; `flop_frac_kernels` over `kernel_ms`). only: one config index."""
    from qlka import _lib
    from weighted_abs_sum import weighted_abs_sum_full
    from weighted_laplace_sum import weighted_laplace_sum
    lib = _lib.load()
    out = {}
    for i, c in CONFIGS.items():
        if only is not None and i != only:
            continue
        q, k, v, g_w, g_u = config_inputs(c, dev)

        def fwd_bwd():
            tq, tk, tv = (t.detach().requires_grad_(True) for t in (q, k, v))
            w, u = weighted_abs_sum_full(tq, tk, tv)
            torch.autograd.backward([w, u], [g_w, g_u])

        if i == 0:
            fn = fwd_bwd
        elif i == 1:
            def fn():
                weighted_laplace_sum(q, k, v)
                weighted_abs_sum_full(q, k, v)
        elif i == 2:
            def fn():
                weighted_laplace_sum(q, k, v)
        else:
            def fn():
                fwd_bwd()
                weighted_laplace_sum(q, k, v)
        n_rep = reps or (3 if i == 4 else 20)
        for _ in range(1 if i == 4 else 5):
            fn()
        ts = []
        for _ in range(n_rep):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1))
        ms = statistics.fmean(ts)
        # device memory of one call above its inputs (torch's allocator: outputs, workspace, kept sorts and range
        # states, gradients), as the reference's speed bench records torch.cuda.max_memory_allocated
        # (Experiments/speed_and_memory/bench.py:101-104)
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        base = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        fn()
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated() - base
        entry = {"ms": round(ms, 4), "ms_median": round(statistics.median(ts), 4), "calls": n_rep,
                 "work": c["work"], "shape": f"P={c['P']} D={c['D']} N=M={c['N']} C={c['C']}",
                 "peak_mem_bytes": int(peak)}
        flops = dense_flops(i, c)
        if flops is not None:
            lib.qlka_timing_reset()
            lib.qlka_timing_enable(1)
            for _ in range(n_rep):
                fn()
            torch.cuda.synchronize()
            lib.qlka_timing_enable(0)
            ksum = sum(_lib.stage_time(name)[0] for name in STAGES + DENSE_STAGES) / n_rep
            kms = _lib.stage_time("busy")[0] / n_rep
            entry.update({"kernel_ms": round(kms, 4), "kernel_sum_ms": round(ksum, 4),
                          "host_frac": round(max(ms - kms, 0.0) / ms, 4),
                          "gflop": round(flops / 1e9, 3), "flop_peak_tflops": FP32_PEAK_TFLOPS,
                          "flop_frac": round(flops / (ms / 1e3) / 1e12 / FP32_PEAK_TFLOPS, 4),
                          "flop_frac_kernels": round(flops / (kms / 1e3) / 1e12 / FP32_PEAK_TFLOPS, 4)})
        out[f"configs[{i}]"] = entry
        del q, k, v, g_w, g_u
        torch.cuda.empty_cache()
    return out


def sort_compare(dev, reps=10):
    """ms per call of libqlka's segmented stable sort (qlka_seg_sort: LDS radix runs + merge passes) and of
    torch.sort(dim=1, stable=True) (rocPRIM's segmented radix sort) on (a) 192 segments of 131072 keys, a configs[4]
    chunk of 3 p, half of the keys on 256 exact levels, (b) 1536 segments of 16384 N(0,1) keys and (c) 256 segments of
    16384, the key sort of one headline chunk of 4 p; both sorts must give the same permutation."""
    from qlka import _lib
    lib = _lib.load()
    out = {}
    g = torch.Generator(device=dev).manual_seed(0)
    for name, S, L, ties in (("192x131072", 192, 131072, True), ("1536x16384", 1536, 16384, False),
                             ("256x16384", 256, 16384, False)):
        x = torch.randn(S, L, device=dev, generator=g)
        if ties:
            x[:, ::2] = torch.round(x[:, ::2] * 16) / 16
        keys = torch.empty_like(x)
        perm = torch.empty(S, L, dtype=torch.int32, device=dev)
        ws = _lib.workspace(lib.qlka_seg_sort_ws_bytes(S, L), dev)

        def ours():
            _lib.check(lib.qlka_seg_sort(_lib.ptr(x), _lib.ptr(keys), _lib.ptr(perm), S, L, _lib.ptr(ws), ws.numel(),
                                         _lib.stream_of(dev)))

        def theirs():
            return torch.sort(x, dim=1, stable=True)

        def tm(fn):
            for _ in range(2):
                fn()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            return round(e0.elapsed_time(e1) / reps, 4)

        t_ours, t_theirs = tm(ours), tm(theirs)
        ref = theirs()
        same = bool(torch.equal(ref.indices.int(), perm)) and bool(torch.equal(ref.values, keys))
        if not same:
            raise SystemExit(f"bench: qlka_seg_sort and torch.sort disagree on {name}")
        out[name] = {"qlka_seg_sort_ms": t_ours, "torch_sort_ms": t_theirs, "same_permutation": same}
    return {"sort_compare": out}


def cpu_baseline(seed=0, mq=256, reps=3):
    """The reference's dense PyTorch path (kernels.py:73,81 restated in oracle/dense.py), torch-CPU fp32 eager, on a
    seeded sample of mq queries per p against all N keys of the headline workload. Cost is linear in the number of
    queries, so query-feature sums/s = 2 * P * mq * D / t (both ops)."""
    from oracle import dense
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    rng = np.random.default_rng(np.random.PCG64(seed))
    q = torch.from_numpy(rng.standard_normal((P, D, M), dtype=np.float32)[:, :, :mq].copy())
    k = torch.from_numpy(rng.standard_normal((P, D, N), dtype=np.float32))
    v = torch.from_numpy(rng.standard_normal((P, N, C), dtype=np.float32))

    def step():
        dense.dense_laplace_sum(q, k, v)
        dense.dense_abs_sum(q, k, v)

    step()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        step()
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    return {"value": 2 * P * mq * D / t, "unit": "query-feature sums/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"dense torch-CPU fp32 laplace + abs sums (oracle/dense.py), P={P} D={D} N={N} C={C}, "
                      f"{mq} queries per p (of {M}), 1 warmup + median of {reps}; "
                      f"cpu={_cpu_model()}"}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


STAGES = ("lds_radix_sort", "lds_count_sort", "merge_runs", "group_queries", "query_bounds", "fill_zero", "lap_range_sums",
          "lap_range_scan", "lap_range_walk", "abs_range_sums", "abs_range_scan", "abs_range_walk", "u_to_query",
          "u_sum", "slab_reduce")
DENSE_STAGES = ("direct_fwd", "direct_sign")


def kernel_algorithmic_bytes(name):
    """Algorithmic bytes of one launch of a headline-op kernel (one op call's worth of its work):
    walks read the sorted keys and their perm, the grouped queries and their indices, gather v once per key and
    feature, and write one contribution row per (p, d, query) plus one v == 1 term; the reduce reads the D rows of
    each query and writes one output row + out_u; the sort reads keys and writes sorted keys + perm; the range
    sums gather v once per key and feature; the query grouping reads q and writes values + indices."""
    S = P * D
    walk = 4.0 * S * (2 * N + 2 * M + N * C + M * C + M)
    table = {
        "lap_range_walk": walk, "abs_range_walk": walk,
        "slab_reduce": 4.0 * P * M * (D * C + D + C + 1),
        "lds_radix_sort": 12.0 * S * N, "lds_count_sort": 12.0 * S * N,
        "lap_range_sums": 4.0 * S * (2 * N + N * C), "abs_range_sums": 4.0 * S * (2 * N + N * C),
        "group_queries": 12.0 * S * M,
    }
    return table.get(name)


def _op_traffic():
    """Measured HBM bytes of one step (both ops): the sum over each op's kernels of FETCH_SIZE + WRITE_SIZE per launch
    (rocprofv3 --pmc, copy-calibrated), committed in profiles/traffic.json; None when not measured."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(path) as f:
            ops = json.load(f).get("ops", {})
        return sum(ops[o]["bytes_per_call"] for o in ("weighted_laplace_sum", "weighted_abs_sum_full"))
    except (OSError, ValueError, KeyError):
        return None


def oracle_check(q, k, v, laplace, abs_full, per_p=32, seed=1):
    """Both ops on the bench inputs against the fp64 oracle (oracle/brute.py) on a seeded subsample of per_p queries
    of every p (all keys, features and channels), at the north-star bar of 1e-5 of the sum of |term| per element.
    Raises if either op misses it, so that no number is printed for wrong outputs."""
    from oracle import brute, inputs
    qn, kn, vn = (t.cpu().numpy() for t in (q, k, v))
    idx = inputs.query_subsample(P, M, per_p=per_p, seed=seed)

    def sub(a):
        a = a.cpu().numpy()
        return np.stack([a[p][idx[p]] for p in range(P)])

    worst = {}
    for name, fn, ref in (("weighted_laplace_sum", laplace, brute.laplace_sum),
                          ("weighted_abs_sum_full", abs_full, brute.abs_sum)):
        w, u = fn(q, k, v)
        ow, ou, nw = ref(qn, kn, vn, qidx=idx)
        err = max(float(brute.rel_err(sub(w), ow, nw).max()), float(brute.rel_err(sub(u), ou, ou).max()))
        worst[name] = err
        if not err <= 1e-5:
            raise SystemExit(f"bench: {name} misses the oracle (max rel err {err:.3e} > 1e-5); no number reported")
    return {"max_rel_err": worst, "bar": 1e-5, "queries_per_p": per_p,
            "oracle": "fp64 brute force (oracle/brute.py), all keys, features and channels"}


def _traffic(kernel):
    """HBM bytes per launch of `kernel` measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, copy-calibrated),
    committed in profiles/traffic.json; None when not measured."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(kernel, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-layers", action="store_true",
                    help="skip the attention-layer timings (layer_ms), e.g. to profile the two ops alone")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the timings of the other BASELINE configurations (config_ms)")
    ap.add_argument("--profile-config", type=int, default=None, choices=sorted(CONFIGS),
                    help="only time this configuration's workload (--steps calls) and print its config_ms entry, "
                         "e.g. under rocprofv3")
    ap.add_argument("--ws-budget-gib", type=float, default=None,
                    help="libqlka workspace budget (qlka_set_workspace_budget) for every timed call, in GiB; "
                         "default: the library's")
    ap.add_argument("--sort-compare", action="store_true",
                    help="only time libqlka's segmented sort against torch.sort(stable=True) (rocPRIM's segmented "
                         "radix sort) on a configs[4]-sized chunk and on headline-length segments, check that the two "
                         "permutations agree, and print one JSON line")
    ap.add_argument("--op", choices=("laplace", "abs", "abs_fwd_bwd", "add_laplace", "add_riesz", "add_bump"),
                    default=None,
                    help="only run --warmup + --steps calls of this one headline op or fused attention layer (on the "
                         "headline q, k, v; abs_fwd_bwd: weighted_abs_sum_full forward and backward through autograd "
                         "against fixed random output gradients) and print the call count (for per-call rocprofv3 "
                         "runs: traffic per call = the sum over its dispatches / calls)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy 3 times (reference kernel of known traffic for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.calibrate_copy:
        dev = torch.device("cuda", 0)
        x = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_per_launch": x.numel() * 4, "launches": 3}), flush=True)
        return
    if args.sort_compare:
        print(json.dumps(sort_compare(torch.device("cuda", 0), reps=args.steps)), flush=True)
        return
    if args.ws_budget_gib is not None:
        from qlka import _lib as _l
        _l.load().qlka_set_workspace_budget(int(args.ws_budget_gib * (1 << 30)))
    if args.profile_config is not None:
        dev = torch.device("cuda", 0)
        print(json.dumps(config_timings(dev, reps=args.steps, only=args.profile_config)), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU (got --gpus {args.gpus}); this build has no multi-GPU path "
              "(the ops would shard over P = B*H, or over the features d with one reduce-scatter of the partial "
              "outputs).",
              file=sys.stderr)
        sys.exit(2)

    from qlka import _lib
    from weighted_abs_sum import weighted_abs_sum_full
    from weighted_laplace_sum import weighted_laplace_sum

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    q, k, v = make_inputs(dev)
    lib = _lib.load()

    def step():
        weighted_laplace_sum(q, k, v)
        weighted_abs_sum_full(q, k, v, backend="cuda")

    if args.op is not None:
        if args.op == "laplace":
            fn = lambda: weighted_laplace_sum(q, k, v)  # noqa: E731
        elif args.op == "abs":
            fn = lambda: weighted_abs_sum_full(q, k, v, backend="cuda")  # noqa: E731
        elif args.op == "abs_fwd_bwd":
            gen = torch.Generator(device=dev).manual_seed(1)
            g_w = torch.randn(q.shape[0], q.shape[2], v.shape[2], generator=gen, device=dev)
            g_u = torch.randn(q.shape[0], q.shape[2], generator=gen, device=dev)

            def fn():
                tq, tk, tv = (t.detach().requires_grad_(True) for t in (q, k, v))
                w, u = weighted_abs_sum_full(tq, tk, tv, backend="cuda")
                torch.autograd.backward([w, u], [g_w, g_u])
        else:
            from qlka import layers
            fn = lambda: layers.layer_forward(args.op, q, k, v)  # noqa: E731
        for _ in range(args.warmup + args.steps):
            fn()
        torch.cuda.synchronize()
        print(json.dumps({"op": args.op, "calls": args.warmup + args.steps}), flush=True)
        return

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # The timed region: library stage timer off, events around the steps only.
    lib.qlka_timing_enable(0)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        step()
    stop.record()
    torch.cuda.synchronize()
    ms_total = start.elapsed_time(stop)
    ms_per_step = ms_total / args.steps
    units = P * M * D
    value = 2 * units / (ms_per_step / 1e3)

    # Per-kernel times from a separate pass of the same steps, with libqlka's hipEvent stage timer on (each launch
    # bracketed on its own stream).
    lib.qlka_timing_reset()
    lib.qlka_timing_enable(1)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    stages = {}
    for name in STAGES:
        ms, cnt = _lib.stage_time(name)
        if cnt:
            stages[name] = {"ms_total": ms, "launches": cnt, "ms_per_launch": ms / cnt}
    lib.qlka_timing_enable(0)

    # per-op time, each op timed alone over the same number of calls (north-star target: B_scan / op time), and the
    # op's peak device memory (torch.cuda.max_memory_allocated over one call, inputs excluded)
    def op_time(fn):
        for _ in range(2):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(args.steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps

    def op_peak(fn):
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        base = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        fn()
        torch.cuda.synchronize()
        return torch.cuda.max_memory_allocated() - base

    ops = {
        "weighted_laplace_sum": lambda: weighted_laplace_sum(q, k, v),
        "weighted_abs_sum_full": lambda: weighted_abs_sum_full(q, k, v, backend="cuda"),
    }
    op_ms = {name: op_time(fn) for name, fn in ops.items()}
    op_peak_bytes = {name: op_peak(fn) for name, fn in ops.items()}
    bscan = bscan_bytes_per_unit(N, M, C) * units
    op_frac = {kk: round(bscan / (vv / 1e3) / 1e9 / HBM_PEAK_GBS, 4) for kk, vv in op_ms.items()}

    # Roofline of the step: B_scan of both op calls / step time. The op is the unit the north-star target is set on;
    # its measured HBM traffic (sum over its kernels of FETCH_SIZE + WRITE_SIZE, copy-calibrated) is `traffic`.
    # `kernel` is the kernel with the most GPU time in the step, on its own algorithmic bytes per launch.
    achieved = 2 * bscan / (ms_per_step / 1e3) / 1e9
    dom = max(stages, key=lambda s_: stages[s_]["ms_total"])
    # the ops run their kernels once per chunk of p: a launch does (op-call bytes) / (launches per op call)
    calls = args.steps * (1 if dom.startswith(("lap_", "abs_")) else 2)
    per_call = kernel_algorithmic_bytes(dom)
    kbytes = per_call * calls / stages[dom]["launches"] if per_call else None
    kach = kbytes / (stages[dom]["ms_per_launch"] / 1e3) / 1e9 if kbytes else None
    roof = {"bound": "hbm", "scope": "op: B_scan of weighted_laplace_sum + weighted_abs_sum_full per step",
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": _op_traffic(),
            "algorithmic_bytes_per_step": 2 * bscan, "op_frac": op_frac,
            "kernel": {"name": dom, "ms_per_launch": round(stages[dom]["ms_per_launch"], 4),
                       "launches_per_op_call": stages[dom]["launches"] / calls,
                       "algorithmic_bytes_per_launch": kbytes,
                       "achieved": round(kach, 1) if kach else None,
                       "frac": round(kach / HBM_PEAK_GBS, 4) if kach else None,
                       "traffic": _traffic(dom)}}

    # The numbers above are reported only if the ops' outputs on these inputs match the fp64 oracle.
    parity = oracle_check(q, k, v, weighted_laplace_sum, weighted_abs_sum_full)

    # The three attention layers of configs[3] on the same q, k, v (already tau-scaled inputs do not change the
    # work): fused (one library call: ops + epilogue, add_bump's three abs sums sharing one sort) vs the reference's
    # composition (separate op calls + torch epilogue, attention.py:67-92).
    from qlka import layers
    layer_ms = {}
    kinds = () if args.no_layers else layers.KINDS
    # Padded batch: the last 10% of the keys of every p masked (attention.py:122-124). In-kernel mask (one masked
    # layer call on the raw k, v) vs the reference's route (k * keep, v * keep, the ops, the n_pad epilogue).
    keep = torch.ones(P, N, dtype=torch.bool, device=dev)
    keep[:, N - N // 10:] = False
    kf = keep.float()
    n_pad = N - kf.sum(dim=1, keepdim=True)

    def reference_masked(kern):
        return layers.unfused(kern, q, k * kf[:, None, :], v * kf[:, :, None], n_pad)

    with torch.no_grad():
        for kern in kinds:
            layer_ms[kern] = {
                "fused": round(op_time(lambda: layers.layer_forward(kern, q, k, v)), 4),
                "unfused": round(op_time(lambda: layers.unfused(kern, q, k, v)), 4),
                "masked_in_kernel": round(op_time(lambda: layers.layer_forward(kern, q, k, v, keep=keep)), 4),
                "masked_reference_route": round(op_time(lambda: reference_masked(kern)), 4),
            }

    out = {
        "metric": METRIC,
        "value": value,
        "unit": "query-feature sums/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: q, k, v ~ N(0,1) fp32 from numpy PCG64(0), resident in HBM",
        "config": {"workload": "BASELINE configs[3] raw ops: weighted_laplace_sum + weighted_abs_sum_full forward, "
                               "B=1 H=12 N=M=16384 D=Dv=64 fp32",
                   "P": P, "D": D, "N": N, "M": M, "C": C, "units_per_step": 2 * units},
        "roofline": roof,
        "op_ms": {kk: round(vv, 4) for kk, vv in op_ms.items()},
        "op_bscan_roofline_frac": op_frac,
        "op_peak_mem_bytes": op_peak_bytes,
        "parity": parity,
        "layer_ms": layer_ms,
        "stages": {kk: round(vv["ms_per_launch"], 4) for kk, vv in stages.items()},
        "device": torch.cuda.get_device_name(dev),
    }
    if not args.no_configs:
        del q, k, v
        torch.cuda.empty_cache()
        out["config_ms"] = config_timings(dev)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
