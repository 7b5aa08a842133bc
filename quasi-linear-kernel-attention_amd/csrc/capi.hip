// The C ABI of libqlka (include/qlka.h): validation, workspace layout and the launch sequence of each operator.
// The reference's host bindings (Weighted_Abs_Sum/csrc/binding.cpp, Weighted_Laplace_Sum/csrc/binding.cpp) do the
// same jobs with ATen tensors; here the caller owns every buffer and the library only carves the workspace.
#include "qlka.h"
#include "qlka_internal.h"

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>
#include <vector>

using namespace qlka;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_status(int e, const char* where) {
    if (e == 0) return QLKA_OK;
    return fail(QLKA_EHIP, "%s: %s", where, hipGetErrorString((hipError_t)e));
}

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Where the dense evaluation (direct.hip) beats sort + scans + walk + reduce, whose cost at short segments is launch
// and per-segment overhead. With B = the base cutoff (qlka_set_direct_max, default 512; 0: always sort + walk) and
// L = max(N, M), measured on MI355X (P = 12, 32, 48, 512; D, C = 32, 64):
//   abs forward      L <= 2B   (dense 0.28 vs walk 0.51 ms at L = 1024, P = 48)
//   Laplace forward  L <= B    (its exp per term: about even at L = 700 for P = 12)
//   backward, sgn    L <= B, or L <= 5B/4 when P * ceil(L / 32) >= 512 workgroups fill the GPU (at L = 600: dense
//                    0.30 vs 0.44 ms at P = 32, but 0.22 vs 0.20 at P = 12)
// Segments of at most FEW_KEYS keys go dense whatever the other side's length, the cutoff (B = 0 included) and the
// pinned path: the abs walk's row emission adds the segment totals as -Btot - (q - k_max) Wtot, whose fp32 rounding
// is about eps * sum_n (k_max - k_n) |w_n|; with a handful of keys that can exceed 1e-5 of the sum of |term| (2 keys,
// one heavy near q and one light far away: 1.8e-5 measured), while the dense kernels sum the terms themselves. (The
// backward's second walk takes the queries as its keys, so there the fewer of N and M counts.) The Laplace walk has
// no totals and keeps its rule. The routing does not depend on the path: path 1 only adds the reference's error for
// max(N, M) > 4096.
constexpr int FEW_KEYS = 16;
std::atomic<int> g_direct_max{512};
inline int64_t direct_base() { return g_direct_max.load(std::memory_order_relaxed); }
inline bool few_keys(int keys) { return keys <= FEW_KEYS; }
inline bool dense_abs_fwd(int N, int M) { return std::max(N, M) <= 2 * direct_base() || few_keys(N); }
inline bool dense_laplace_fwd(int N, int M) { return std::max(N, M) <= direct_base(); }
inline bool dense_sign(int P, int N, int M) {
    const int64_t L = std::max(N, M), B = direct_base();
    return L <= B || (4 * L <= 5 * B && (int64_t)P * ((L + 31) / 32) >= 512) || few_keys(std::min(N, M));
}

// Same limits and wording as check_qkv (Weighted_Abs_Sum/csrc/binding.cpp:79-83).
int check_dims(int P, int D, int N, int M, int C) {
    if (P <= 0) return fail(QLKA_EINVAL, "P must be > 0");
    if (M <= 0 || N <= 0 || D <= 0) return fail(QLKA_EINVAL, "N, M and D must be > 0");
    if (C < 1 || C > 128) return fail(QLKA_EINVAL, "C (v.size(2)) must be in [1, 128]");
    if (N > 131072 || M > 131072) return fail(QLKA_EINVAL, "N and M must be <= 131072");
    if ((int64_t)P * D * std::max(N, M) > (int64_t)INT32_MAX)
        return fail(QLKA_EINVAL, "P*D*max(N,M) must fit int32 (element offsets)");
    return QLKA_OK;
}

// Workspace of one call: sorted k and q of every segment, the sort scratch, the range arrays of the walks and, for
// the row-emitting walks, the per-feature contribution slab (+ the sorted-order v == 1 contributions and the LDS
// scatter partials when out_u is wanted).
struct SortedWs {
    float* ks; uint32_t* kp; float* qs; uint32_t* qp;
    void* sort_scratch; RangeArrays ra;
    float* slab; float* uslab; float* uq;
};

struct WsSpec {
    int P, D, N, M, C;
    int range_stream_max;   // longest stream a walk runs over (N, or max(N, M) for the backward)
    int slab_rows;          // queries per feature of the row slab (0: no row emission)
    bool want_u;            // v == 1 contributions (out_u)
};

// Sort scratch of a call: one array at a time, or k and q as one sort when N == M (seg_sort2).
size_t sort_scratch_need(const WsSpec& w) {
    const int S = w.P * w.D;
    const size_t one = std::max(seg_sort_scratch_bytes(S, w.N), seg_sort_scratch_bytes(S, w.M));
    return w.N == w.M ? std::max(one, seg_sort_scratch_bytes(2 * S, w.N)) : one;
}

// The sorts run in a chunk's prep and are done before its walks write the slab, and the pipeline's prep of a chunk
// waits for the reduce that last read its workspace copy's slab, so the sort scratch lives inside the slab when the
// slab holds it (at N = M = 131072 that saves 268 MB a copy).
bool scratch_in_slab(const WsSpec& w) {
    const size_t slab = w.slab_rows ? (size_t)w.P * w.D * slab_rows(w.slab_rows) * slab_stride(w.C) * 4 : 0;
    return sort_scratch_need(w) <= slab;
}

size_t ws_part(const WsSpec& w, int i) {
    const size_t S = (size_t)w.P * w.D;
    switch (i) {
        case 0: case 1: return align256(S * w.N * 4);
        case 2: case 3: return align256(S * w.M * 4);
        case 4: return scratch_in_slab(w) ? 0 : align256(sort_scratch_need(w));
        case 5: return align256(range_arrays_bytes((int)S, w.range_stream_max, w.C));
        case 6: return w.slab_rows ? align256(S * slab_rows(w.slab_rows) * (size_t)slab_stride(w.C) * 4) : 0;
        case 7: return (w.slab_rows && w.want_u) ? align256(S * w.slab_rows * 4) : 0;
        case 8: return (w.slab_rows && w.want_u) ? align256(S * w.M * 4) : 0;   // v == 1 terms in query order
    }
    return 0;
}

constexpr int WS_PARTS = 9;

size_t ws_bytes(const WsSpec& w) {
    size_t b = 0;
    for (int i = 0; i < WS_PARTS; ++i) b += ws_part(w, i);
    return b;
}

SortedWs carve(void* ws, const WsSpec& w) {
    char* b = (char*)ws;
    char* part[WS_PARTS];
    for (int i = 0; i < WS_PARTS; ++i) { part[i] = b; b += ws_part(w, i); }
    SortedWs r;
    r.ks = (float*)part[0]; r.kp = (uint32_t*)part[1]; r.qs = (float*)part[2]; r.qp = (uint32_t*)part[3];
    r.sort_scratch = scratch_in_slab(w) ? part[6] : part[4];
    r.ra = carve_range_arrays(part[5], w.P * w.D, w.range_stream_max, w.C);
    r.slab = (float*)part[6]; r.uslab = (float*)part[7];
    r.uq = ws_part(w, 8) ? (float*)part[8] : nullptr;
    return r;
}

int check_ws(void* ws, size_t have, size_t need) {
    if (need > have || (need > 0 && ws == nullptr))
        return fail(QLKA_EWORKSPACE, "workspace too small: %zu bytes given, %zu needed", have, need);
    return QLKA_OK;
}

// ---- p-chunking. Every stage of every operator works on each p = (batch, head) on its own, so a call can run its
// whole pipeline (sorts, range passes, walks, reduce, epilogue) on a chunk of pc consecutive p at a time, with a
// workspace sized for pc. An operator takes the largest chunk that the workspace it is given holds; the *_ws_bytes()
// queries size the workspace for the largest chunk within the process-wide budget (qlka_set_workspace_budget).
// Default 5 GiB: at configs[4] (P = 12, N = M = 131072) a call took 86.4 ms at 5 GiB and 86.6 ms at 16 GiB (one call's
// peak 9.2 vs 19.5 GB); the headline's pipelined chunks (2.43 GB) fit either.
std::atomic<size_t> g_ws_budget{size_t(5) << 30};

// largest pc in [1, P] with bytes(pc) <= cap, or 1 when even one p does not fit (bytes() grows with pc)
template <class Bytes>
int fit_chunk(int P, size_t cap, Bytes bytes) {
    if (bytes(P) <= cap) return P;
    int lo = 1, hi = P - 1;
    while (lo < hi) {
        const int mid = lo + (hi - lo + 1) / 2;
        if (bytes(mid) <= cap) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// bytes(pc) of the chunk a workspace query reports: the largest within the budget
template <class Bytes>
size_t budget_bytes(int P, Bytes bytes) {
    return bytes(fit_chunk(P, g_ws_budget.load(std::memory_order_relaxed), bytes));
}

// f(p0, np) for the chunks [p0, p0 + np) of [0, P); stops at the first error
template <class F>
int for_chunks(int P, int pc, F f) {
    for (int p0 = 0; p0 < P; p0 += pc)
        if (int e = f(p0, std::min(pc, P - p0))) return e;
    return QLKA_OK;
}

// k and q sorted; in one launch when N == M (a hipError_t value, 0 on success)
int sort_pair(const float* q, const float* k, SortedWs& w, int S, int N, int M, hipStream_t st) {
    if (N == M) return seg_sort2(k, w.ks, w.kp, q, w.qs, w.qp, S, N, w.sort_scratch, st);
    if (int e = seg_sort(k, w.ks, w.kp, S, N, w.sort_scratch, st)) return e;
    return seg_sort(q, w.qs, w.qp, S, M, w.sort_scratch, st);
}

int sort_both(const float* q, const float* k, SortedWs& w, int S, int N, int M, hipStream_t st) {
    return hip_status(sort_pair(q, k, w, S, N, M, st), "segmented sort of k and q");
}

// The query side of a forward walk that keeps no sorts, after the k sort: q grouped by key chunk, with the range
// bounds, in one pass (the walks take grouped queries as well as sorted ones) where a segment's queries and chunk
// bounds fit one workgroup's LDS; longer segments sort q instead and search the bounds (at N = M = 131072 the
// multi-workgroup grouping's scattered 4-byte stores wrote 6.8x their bytes: 1.19 ms a chunk of 3 p, against 0.77
// for the q sort and the bounds).
static int group_q(const float* q, SortedWs& w, float qshift, int S, int N, int M, int C, hipStream_t st) {
    if (group_fits(N, M, C))
        return hip_status(group_queries(w.ks, q, w.qs, w.qp, w.ra.qb, qshift, S, N, M, C, st), "query grouping");
    if (int e = hip_status(seg_sort(q, w.qs, w.qp, S, M, w.sort_scratch, st), "segmented sort of q")) return e;
    return hip_status(query_bounds(w.ks, w.qs, w.ra.qb, qshift, S, N, M, C, st), "query bounds");
}

// The prep of a forward walk that keeps no sorts: the k sort, then the query side (group_q). (One kernel doing both,
// the grouping in the sort's workgroup against the sorted keys still in LDS, measured slower: 1.760 vs 1.748 ms per
// Laplace call. Beside the previous chunk's reduce it holds its CU slots for the grouping too, while the grouping as
// its own launch mostly waits for the reduce to drain and then runs alone.)
static int sort_k_group_q(const float* k, const float* q, SortedWs& w, float qshift, int S, int N, int M, int C,
                          hipStream_t st) {
    if (N == M && !group_fits(N, M, C)) {   // both sorted: as one sort
        if (int e = hip_status(seg_sort2(k, w.ks, w.kp, q, w.qs, w.qp, S, N, w.sort_scratch, st),
                               "segmented sort of k and q"))
            return e;
        return hip_status(query_bounds(w.ks, w.qs, w.ra.qb, qshift, S, N, M, C, st), "query bounds");
    }
    if (int e = hip_status(seg_sort(k, w.ks, w.kp, S, N, w.sort_scratch, st), "segmented sort of k")) return e;
    return group_q(q, w, qshift, S, N, M, C, st);
}

// ---- overlap of the query side (q sort, range boundaries) with the key side (range summaries, scan)
// The two sides read and write disjoint parts of the workspace and both need only the sorted keys. The key side runs
// on the caller's stream, the query side on a side stream of the calling thread (one per device, created on first
// uncaptured use, default priority, non-blocking, kept until the process ends). Events order the side stream after
// the work already on the caller's stream, and the caller's stream after the side stream's work. A host thread issues
// its calls in order, so reusing its two events is safe; a fork / join through events is also how work on a captured
// stream reaches another stream.
struct SideStream {
    hipStream_t s = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    hipEvent_t walked = nullptr, reduced[2] = {nullptr, nullptr};   // the chunk pipeline's events (run_pipeline)
};

// Side streams outlive the threads that created them: a thread that exits hands its side streams (and their events)
// back to a process-wide pool, and a thread's first call on a device takes one from there before creating a new one.
// So a server whose worker threads come and go holds at most one side stream per device per thread alive at a time.
// The pool is never destroyed, and returning to it makes no HIP call (a thread may exit after the runtime has shut
// down, at process exit).
constexpr int MAX_DEVICES = 64;
struct SidePool {
    std::mutex mu;
    std::vector<SideStream> free[MAX_DEVICES];
};
SidePool& side_pool() {
    static SidePool* p = new SidePool;                    // never destroyed: threads may exit after static teardown
    return *p;
}
struct ThreadSides {
    SideStream sides[MAX_DEVICES];
    ~ThreadSides() {
        SidePool& p = side_pool();
        std::lock_guard<std::mutex> lock(p.mu);
        for (int d = 0; d < MAX_DEVICES; ++d)
            if (sides[d].s != nullptr) p.free[d].push_back(sides[d]);
    }
};

hipError_t side_stream(hipStream_t st, SideStream** out) {
    *out = nullptr;
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (st != nullptr) {
        hipDevice_t dev = cur;
        if ((e = hipStreamGetDevice(st, &dev)) != hipSuccess) return e;
        if (dev != cur) return hipSuccess;              // stream of another device: run in order on it
    }
    thread_local ThreadSides mine;
    if (cur >= MAX_DEVICES) return hipSuccess;
    SideStream& sd = mine.sides[cur];
    if (sd.s == nullptr) {
        SidePool& p = side_pool();
        std::lock_guard<std::mutex> lock(p.mu);
        if (!p.free[cur].empty()) {
            sd = p.free[cur].back();
            p.free[cur].pop_back();
        }
    }
    if (sd.s == nullptr) {
        // Creating a stream inside a stream capture would invalidate it: a thread whose first call is captured runs
        // that call in order on the caller's stream and creates its side stream with a later, uncaptured call.
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if ((e = hipStreamIsCapturing(st, &cs)) != hipSuccess) return e;
        if (cs != hipStreamCaptureStatusNone) return hipSuccess;
        SideStream n;
        hipEvent_t* evs[5] = {&n.join, &n.fork, &n.walked, &n.reduced[0], &n.reduced[1]};
        e = hipStreamCreateWithFlags(&n.s, hipStreamNonBlocking);
        // Only work on this device waits for the fork and pipeline events, so they record without the system-scope
        // fence (its cache write-back cost 5-10 us of GPU time at each of them: a Laplace call at the headline shape
        // 1.735 -> 1.721 ms). The join, after which the caller's stream may hand the outputs to the host, keeps it.
        for (int i = 0; i < 5 && e == hipSuccess; ++i)
            e = hipEventCreateWithFlags(evs[i], hipEventDisableTiming | (i == 0 ? 0u : hipEventDisableSystemFence));
        if (e != hipSuccess) {                            // release what was created; the call reports the error
            for (hipEvent_t* ev : evs)
                if (*ev != nullptr) (void)hipEventDestroy(*ev);
            if (n.s != nullptr) (void)hipStreamDestroy(n.s);
            return e;
        }
        sd = n;
    }
    *out = &sd;
    return hipSuccess;
}

template <class KeySide, class QuerySide>
int fork_join(hipStream_t st, KeySide key_side, QuerySide query_side) {
    SideStream* sd = nullptr;
    if (hipError_t e = side_stream(st, &sd)) return hip_status((int)e, "side stream");
    if (sd == nullptr) {
        if (int e = query_side(st)) return e;
        return key_side(st);
    }
    if (hipError_t e = hipEventRecord(sd->fork, st)) return hip_status((int)e, "fork");
    if (hipError_t e = hipStreamWaitEvent(sd->s, sd->fork, 0)) return hip_status((int)e, "fork");
    const int eq = query_side(sd->s);
    const int ek = key_side(st);
    // join whatever happened, so that nothing later on st can overtake work issued on the side stream
    const hipError_t r = hipEventRecord(sd->join, sd->s);
    const hipError_t w = r == hipSuccess ? hipStreamWaitEvent(st, sd->join, 0) : r;
    if (eq) return eq;
    if (ek) return ek;
    return w == hipSuccess ? QLKA_OK : hip_status((int)w, "join");
}

// Dense abs backward with sign(0) = tie (0: KeOps, -1: the walks' convention), g_u nullable. Its three products are
// independent and none fills the GPU at the sizes the dense route takes (608 workgroups each at P = 32, N = M = 600),
// so grad_k runs on the side stream beside grad_q and then grad_v on the caller's stream: 0.355 -> 0.313 ms for a
// forward + backward at that size. grad_q is launched before the side stream's wait (12-16 us of host time), so the
// GPU does not wait for it.
// A (nullable): the forward's kernel matrix (direct_fwd_keep_a); grad_v is then its contraction with g_w instead of
// the dense sum with the roles of q and k swapped, which forms A again (1.47 G of the 7.4 G VALU lane-operations of a
// forward + backward at P = 32, N = M = 600), with the same bits.
int dense_bwd(float tie, const float* q, const float* k, const float* v, const float* g_w, const float* g_u,
              float* grad_q, float* grad_k, float* grad_v, int P, int D, int N, int M, int C, hipStream_t st,
              const float* A = nullptr) {
    // grad_q[d, m] = sum_n s(q - k) (<g_w[m], v[n]> + g_u[m])
    auto gq = [&](hipStream_t s) { return direct_sign(true, q, k, g_w, v, g_u, grad_q, tie, 1.f, P, D, M, N, C, s); };
    // grad_k[d, n] = sum_m s(k - q) (<v[n], g_w[m]> + g_u[m])
    auto gk = [&](hipStream_t s) { return direct_sign(false, k, q, v, g_w, g_u, grad_k, tie, 1.f, P, D, N, M, C, s); };
    // grad_v[n, :] = sum_m A[m, n] g_w[m, :]: the dense abs sum with the roles of q and k swapped
    auto gv = [&](hipStream_t s) {
        return A ? dense_at_g(A, g_w, grad_v, P, N, M, C, s) : direct_fwd(0, k, q, g_w, grad_v, nullptr, P, D, M, N, C, s);
    };
    SideStream* sd = nullptr;
    if (hipError_t e = side_stream(st, &sd)) return hip_status((int)e, "side stream");
    int e = QLKA_OK;
    if (sd == nullptr) {
        if (!(e = gq(st)) && !(e = gk(st))) e = gv(st);
        return hip_status(e, "dense backward");
    }
    if (hipError_t r = hipEventRecord(sd->fork, st)) return hip_status((int)r, "fork");
    e = gq(st);
    const hipError_t w = hipStreamWaitEvent(sd->s, sd->fork, 0);
    if (w != hipSuccess) return e ? hip_status(e, "dense backward") : hip_status((int)w, "fork");
    const int ek = e ? QLKA_OK : gk(sd->s);
    if (!e) e = gv(st);
    // join whatever happened, so that nothing later on st can overtake work issued on the side stream
    const hipError_t r = hipEventRecord(sd->join, sd->s);
    const hipError_t j = r == hipSuccess ? hipStreamWaitEvent(st, sd->join, 0) : r;
    if (e || ek) return hip_status(e ? e : ek, "dense backward");
    return j == hipSuccess ? QLKA_OK : hip_status((int)j, "join");
}

// ---- pipelined p-chunks
// A chunk's work falls in three parts: prep (the sorts and the query grouping: LDS- and VALU-bound), main (the range
// passes and the walk) and back (the reduce of the chunk's slab: an HBM-bound stream). With two workspace copies the
// chunks are pipelined over the caller's stream and the side stream: prep and main of chunk j run on the caller's
// stream, its back on the side stream once its walk is done, so that the reduce of chunk j runs beside the prep of
// chunk j + 1. The main part of chunk j + 1 waits for that reduce: measured beside it, the range passes' gathers ran
// 3x slower (71 -> 212 us a pass at the headline shape), the sorts and the grouping at about their own speed. The
// prep of chunk j + 2 overwrites copy j % 2 and so waits for the reduce of chunk j. With one copy, or without a side
// stream (a thread's first call inside a stream capture, a stream of another device), the chunks run in order on the
// caller's stream. Every fork is joined back to the caller's stream before returning, errors included.
constexpr int PIPE_CHUNKS = 3;       // chunks of a pipelined call (3 of 2, 3, 4, 6 measured fastest at the headline)

struct Plan { int pc; int nbuf; };

// Chunking of a call over P p whose chunk buffer of pc p needs bytes1(pc) workspace bytes, within `cap` bytes:
// pipelined (PIPE_CHUNKS chunks, two copies) when `pipeline` and P >= 2, with smaller chunks if needed to fit two
// copies; else in order with one copy, the largest chunk that fits (one p at least).
template <class Bytes>
Plan plan_chunks(int P, size_t cap, bool pipeline, Bytes bytes1) {
    if (pipeline && P >= 2) {
        const int nc = std::min(P, PIPE_CHUNKS);
        const int pc = (P + nc - 1) / nc;
        if (2 * bytes1(pc) <= cap) return Plan{pc, 2};
        const int pc2 = fit_chunk(P, cap, [&](int c) { return 2 * bytes1(c); });
        if (2 * bytes1(pc2) <= cap) return Plan{pc2, 2};
    }
    return Plan{fit_chunk(P, cap, bytes1), 1};
}

template <class Bytes>
size_t plan_bytes(const Plan& pl, Bytes bytes1) { return (size_t)pl.nbuf * bytes1(pl.pc); }

// A call is pipelined when each of its chunks still fills the GPU many times over (below about 4M query-features
// the per-chunk launch tails outweigh the overlap).
inline bool pipelined(int P, int D, int M) { return P >= 2 && (int64_t)P * D * M >= (int64_t(1) << 22); }

// prep / main / back: int(p0, np, buf, stream) for the chunk [p0, p0 + np) over workspace copy `buf`. `early`, the
// same, runs after prep and before main's wait for the previous chunk's reduce: the part of main that may share the
// GPU with that reduce (add_bump's range passes beside its three-slab reduce, 0.55 ms: 4.43 -> 4.42 ms; making that
// reduce wait for the next chunk's sort, which it slows from 0.12 to 0.64 ms, cost 0.1 ms instead).
inline int no_early(int, int, void*, hipStream_t) { return QLKA_OK; }

template <class Prep, class Main, class Back, class Early = decltype(&no_early)>
int run_pipeline(int P, const Plan& pl, void* ws, size_t copy, hipStream_t st, Prep prep, Main main, Back back,
                 Early early = &no_early) {
    SideStream* sd = nullptr;
    if (pl.nbuf == 2 && (P + pl.pc - 1) / pl.pc > 1) {
        if (hipError_t e = side_stream(st, &sd)) return hip_status((int)e, "side stream");
    }
    if (sd == nullptr) {
        return for_chunks(P, pl.pc, [&](int p0, int np) {
            if (int e = prep(p0, np, ws, st)) return e;
            if (int e = early(p0, np, ws, st)) return e;
            if (int e = main(p0, np, ws, st)) return e;
            return back(p0, np, ws, st); });
    }
    // The side stream needs no fork: its first work waits for `walked` of chunk 0, recorded on st after everything
    // before it. Copy j % 2 is free for the prep of chunk j >= 2 because main of chunk j - 1 already waited on st for
    // the reduce of chunk j - 2. (A stream wait costs 12-16 us of host time here, a record about 1 us.)
    auto hipc = [](hipError_t e, const char* what) { return e == hipSuccess ? QLKA_OK : hip_status((int)e, what); };
    int err = QLKA_OK;
    bool joined = false;                                  // st already waited for everything on the side stream
    int j = 0;
    for (int p0 = 0; p0 < P && !err; p0 += pl.pc, ++j) {
        const int np = std::min(pl.pc, P - p0);
        void* buf = (char*)ws + (size_t)(j % 2) * copy;
        err = prep(p0, np, buf, st);
        if (!err) err = early(p0, np, buf, st);
        const bool last = p0 + np >= P, next_last = !last && p0 + np + pl.pc >= P;
        if (!err && j >= 1)
            err = hipc(hipStreamWaitEvent(st, last ? sd->join : sd->reduced[(j - 1) % 2], 0), "pipeline");
        if (!err) err = main(p0, np, buf, st);
        if (last) {
            // The last chunk's back has nothing to run beside: on the caller's stream it skips a cross-stream wait
            // (about 9 us of GPU time at the headline shape). The wait before this main was for the side stream's
            // last work through the join event (system-scope fence), so no join is needed after it.
            if (!err) err = back(p0, np, buf, st);
            joined = !err;
            break;
        }
        if (!err) err = hipc(hipEventRecord(sd->walked, st), "pipeline");
        if (!err) err = hipc(hipStreamWaitEvent(sd->s, sd->walked, 0), "pipeline");
        if (!err) err = back(p0, np, buf, sd->s);
        if (!err) err = hipc(hipEventRecord(next_last ? sd->join : sd->reduced[j % 2], sd->s), "pipeline");
    }
    if (joined) return QLKA_OK;
    // join whatever happened, so that nothing later on st can overtake work issued on the side stream
    const hipError_t r = hipEventRecord(sd->join, sd->s);
    const hipError_t w = r == hipSuccess ? hipStreamWaitEvent(st, sd->join, 0) : r;
    if (err) return err;
    return w == hipSuccess ? QLKA_OK : hip_status((int)w, "join");
}

}  // namespace

extern "C" {

const char* qlka_last_error(void) { return g_err.c_str(); }

int qlka_version(void) { return 1; }

int qlka_set_direct_max(int n) {
    g_err.clear();
    if (n < 0) return -fail(QLKA_EINVAL, "the dense cutoff must be >= 0");   // negative: not a cutoff
    return g_direct_max.exchange(n);
}

size_t qlka_set_workspace_budget(size_t bytes) { return g_ws_budget.exchange(bytes); }

// ------------------------------------------------------------------------------------------------ laplace forward
static WsSpec laplace_spec(int P, int D, int N, int M, int C) { return WsSpec{P, D, N, M, C, N, M, true}; }

size_t qlka_laplace_fwd_ws_bytes(int P, int D, int N, int M, int C) {
    if (P <= 0 || D <= 0 || N <= 0 || M <= 0 || C <= 0) return 0;
    if (dense_laplace_fwd(N, M)) return 0;        // the dense route takes no workspace
    auto b1 = [&](int pc) { return ws_bytes(laplace_spec(pc, D, N, M, C)); };
    return plan_bytes(plan_chunks(P, g_ws_budget.load(std::memory_order_relaxed), pipelined(P, D, M), b1), b1);
}

int qlka_laplace_fwd(const float* q, const float* k, const float* v, float* out_w, float* out_u,
                     int P, int D, int N, int M, int C, void* ws, size_t ws_bytes_given, void* stream) {
    g_err.clear();
    if (int e = check_dims(P, D, N, M, C)) return e;
    if (!q || !k || !v || !out_w || !out_u) return fail(QLKA_EINVAL, "q, k, v, out_w and out_u must be non-null");
    hipStream_t st = (hipStream_t)stream;
    if (dense_laplace_fwd(N, M))
        return hip_status(direct_fwd(1, q, k, v, out_w, out_u, P, D, N, M, C, st), "laplace direct sum");
    auto b1 = [&](int pc) { return ws_bytes(laplace_spec(pc, D, N, M, C)); };
    const Plan pl = plan_chunks(P, ws_bytes_given, pipelined(P, D, M), b1);
    if (int e = check_ws(ws, ws_bytes_given, plan_bytes(pl, b1))) return e;
    // per chunk: sort k and group q; range passes and walk; reduce
    auto prep = [&](int p0, int np, void* buf, hipStream_t s) {
        SortedWs w = carve(buf, laplace_spec(np, D, N, M, C));
        const size_t p = (size_t)p0;
        return sort_k_group_q(k + p * D * N, q + p * D * M, w, 0.f, np * D, N, M, C, s);
    };
    // the range passes before the wait for the previous chunk's reduce, beside its tail (1.721 -> 1.707 ms)
    auto early = [&](int p0, int np, void* buf, hipStream_t s) {
        SortedWs w = carve(buf, laplace_spec(np, D, N, M, C));
        const float* vp = v + (size_t)p0 * N * C;
        return hip_status(laplace_prepare(w.ks, w.kp, vp, np, D, N, C, w.ra, s), "laplace ranges");
    };
    auto main = [&](int p0, int np, void* buf, hipStream_t s) {
        SortedWs w = carve(buf, laplace_spec(np, D, N, M, C));
        const float* vp = v + (size_t)p0 * N * C;
        if (int e = laplace_emit(w.ks, w.kp, w.qs, w.qp, vp, w.slab, w.uslab, np, D, N, M, C, w.ra, s))
            return hip_status(e, "laplace walk");
        order_u_terms(w.uslab, w.qp, w.uq, np, D, M, s);
        return hip_status((int)hipGetLastError(), "v == 1 terms to query order");
    };
    auto back = [&](int p0, int np, void* buf, hipStream_t s) {
        SortedWs w = carve(buf, laplace_spec(np, D, N, M, C));
        const size_t p = (size_t)p0;
        const float* uq = u_query_order(M) ? w.uslab : w.uq;
        return hip_status(reduce_slabs(w.slab, uq, nullptr, nullptr, out_w + p * M * C, out_u + p * M, np, D, M, C, s),
                          "laplace reduce");
    };
    return run_pipeline(P, pl, ws, b1(pl.pc), st, prep, main, back, early);
}

// ---------------------------------------------------------------------------------------------------- abs forward
static WsSpec abs_fwd_spec(int P, int D, int N, int M, int C, bool full) { return WsSpec{P, D, N, M, C, N, M, full}; }

// The dense route's only workspace: the sort scratch of sorts kept for a backward that walks (none when the backward
// is dense too, and none for segments of one LDS run).
static size_t abs_dense_ws(int P, int pc, int D, int N, int M, int C) {
    return dense_sign(P, N, M) ? 0 : align256(sort_scratch_need(abs_fwd_spec(pc, D, N, M, C, true)));
}

size_t qlka_abs_fwd_ws_bytes(int P, int D, int N, int M, int C) {
    if (P <= 0 || D <= 0 || N <= 0 || M <= 0 || C <= 0) return 0;
    if (dense_abs_fwd(N, M)) return budget_bytes(P, [&](int pc) { return abs_dense_ws(P, pc, D, N, M, C); });
    auto b1 = [&](int pc) { return ws_bytes(abs_fwd_spec(pc, D, N, M, C, true)); };
    return plan_bytes(plan_chunks(P, g_ws_budget.load(std::memory_order_relaxed), pipelined(P, D, M), b1), b1);
}

}  // extern "C"

namespace {
// Sorted k and q of one call, in caller-owned buffers (k_sorted / q_sorted as sorted keys, k_perm / q_perm as their
// permutations), so that the backward of the same inputs can skip both sorts; optionally (states) also the range
// states and query bounds of the walk over sorted k with v as rows and the sorted q as queries, which the forward
// computes and the backward's grad_q walk would compute again (same range sums, scan and bounds).
struct Presorted { float* ks; uint32_t* kp; float* qs; uint32_t* qp; void* states = nullptr; };

Presorted offset(const Presorted& a, size_t p0, int D, int N, int M) {
    return Presorted{a.ks + p0 * D * N, a.kp + p0 * D * N, a.qs + p0 * D * M, a.qp + p0 * D * M, nullptr};
}

// The kept range states of a call over P p: ta and tb ([P*D][G+1][range_stride(C)] floats, the scan's entry states
// with the segment totals in row G) and qb ([P*D][G] ints), G = range_count(N, C); pointers of chunk [p0, ...).
size_t kept_state_bytes(int P, int D, int N, int C) {
    const size_t G = (size_t)range_count(N, C), rows = (size_t)P * D * (G + 1);
    return 2 * align256(rows * range_stride(C) * sizeof(float)) + align256((size_t)P * D * G * sizeof(int));
}

void kept_states(void* base, int P, int D, int N, int C, size_t p0, RangeArrays& ra) {
    const size_t G = (size_t)range_count(N, C), rows = (size_t)P * D * (G + 1);
    char* b = (char*)base;
    float* ta = (float*)b;
    b += align256(rows * range_stride(C) * sizeof(float));
    float* tb = (float*)b;
    b += align256(rows * range_stride(C) * sizeof(float));
    const size_t r0 = p0 * D * (G + 1) * range_stride(C);
    ra.ta = ta + r0;
    ra.tb = tb + r0;
    ra.qb = (int*)b + p0 * D * G;
}

int abs_fwd_impl(const float* q, const float* k, const float* v, float* out_w, float* out_u, int P, int D, int N, int M,
                 int C, int path, const Presorted* keep, int* kept, void* ws, size_t ws_bytes_given, void* stream) {
    g_err.clear();
    if (kept) *kept = 0;
    if (int e = check_dims(P, D, N, M, C)) return e;
    if (path < -1 || path > 1) return fail(QLKA_EINVAL, "path must be -1 (auto), 0 (global) or 1 (fused)");
    if (!q || !k || !v || !out_w) return fail(QLKA_EINVAL, "q, k, v and out_w must be non-null");
    if (keep && (!keep->ks || !keep->kp || !keep->qs || !keep->qp || !kept))
        return fail(QLKA_EINVAL, "the sorted-array buffers and the kept flag must be non-null");
    // The reference's fused kernel only covers max(N, M) <= 4096 (Weighted_Abs_Sum/csrc/binding.cpp:177-188).
    if (path == 1 && std::max(N, M) > 4096)
        return fail(QLKA_EINVAL, "fused path pinned but unavailable: needs max(N,M) <= 4096 and the "
                                 "bucket's shared memory to fit this device");
    hipStream_t st = (hipStream_t)stream;
    const bool keep_sorts = keep && !dense_sign(P, N, M);   // the backward will walk: hand it the sorts
    // the range states only where qlka_abs_keep_state_bytes sizes a buffer for them (a backward that reads them)
    const bool keep_states = keep_sorts && keep->states && qlka_abs_keep_state_bytes(P, D, N, M, C) != 0;
    if (dense_abs_fwd(N, M)) {
        if (keep_sorts) {
            auto db = [&](int pc) { return abs_dense_ws(P, pc, D, N, M, C); };
            const int pc = fit_chunk(P, ws_bytes_given, db);
            if (int e = check_ws(ws, ws_bytes_given, db(pc))) return e;
            const int e = for_chunks(P, pc, [&](int p0, int np) {
                const Presorted ks = offset(*keep, (size_t)p0, D, N, M);
                SortedWs w{};
                w.ks = ks.ks; w.kp = ks.kp; w.qs = ks.qs; w.qp = ks.qp; w.sort_scratch = ws;
                const size_t p = (size_t)p0;
                return sort_both(q + p * D * M, k + p * D * N, w, np * D, N, M, st); });
            if (e) return e;
            *kept = 1;
        }
        return hip_status(direct_fwd(0, q, k, v, out_w, out_u, P, D, N, M, C, st), "abs direct sum");
    }
    // the workspace is sized for the _full op (an upper bound of the plain one), so one size serves both
    auto b1 = [&](int pc) { return ws_bytes(abs_fwd_spec(pc, D, N, M, C, true)); };
    const Plan pl = plan_chunks(P, ws_bytes_given, pipelined(P, D, M), b1);
    if (int e = check_ws(ws, ws_bytes_given, plan_bytes(pl, b1))) return e;
    const int mode = out_u ? (ABS_ROW | ABS_ONES) : ABS_ROW;
    // the chunk's workspace view, with the sorted arrays in the caller's buffers when the sorts are kept
    auto view = [&](int p0, int np, void* buf, SortedWs& w, AbsWalkArgs& a) {
        w = carve(buf, abs_fwd_spec(np, D, N, M, C, true));
        if (keep_sorts) {
            const Presorted ks = offset(*keep, (size_t)p0, D, N, M);
            w.ks = ks.ks; w.kp = ks.kp; w.qs = ks.qs; w.qp = ks.qp;
            if (keep_states) kept_states(keep->states, P, D, N, C, (size_t)p0, w.ra);   // the scan writes them there
        }
        a = AbsWalkArgs{};
        a.ks = w.ks; a.kp = w.kp; a.Ns = N; a.w = v + (size_t)p0 * N * C; a.u = nullptr;
        a.qs = w.qs; a.qp = w.qp; a.Mq = M; a.g = nullptr; a.uq = nullptr;
        a.slab = w.slab; a.uslab = out_u ? w.uslab : nullptr; a.CR = slab_stride(C);
        a.out_dot = nullptr; a.out_rank = nullptr;
        a.sign = 1.f; a.P = np; a.D = D; a.C = C;
    };
    // per chunk: sort k and group q (or, keeping the sorts, sort q and find the query bounds); range passes and walk;
    // reduce
    auto prep = [&](int p0, int np, void* buf, hipStream_t s) {
        SortedWs w; AbsWalkArgs a;
        view(p0, np, buf, w, a);
        const size_t p = (size_t)p0;
        if (keep_sorts) {
            if (int e = hip_status(sort_pair(q + p * D * M, k + p * D * N, w, np * D, N, M, s), "segmented sorts"))
                return e;
            return hip_status(range_bounds(a, w.ra.qb, s), "query bounds");
        }
        return sort_k_group_q(k + p * D * N, q + p * D * M, w, 0.f, np * D, N, M, C, s);
    };
    // the range passes before the wait for the previous chunk's reduce, beside its tail
    auto early = [&](int p0, int np, void* buf, hipStream_t s) {
        SortedWs w; AbsWalkArgs a;
        view(p0, np, buf, w, a);
        return hip_status(abs_prepare(a, mode, w.ra, s), "abs ranges");
    };
    auto main = [&](int p0, int np, void* buf, hipStream_t s) {
        SortedWs w; AbsWalkArgs a;
        view(p0, np, buf, w, a);
        if (int e = hip_status(abs_emit(a, mode, w.ra, s), "abs walk")) return e;
        if (out_u) order_u_terms(w.uslab, w.qp, w.uq, np, D, M, s);
        return hip_status((int)hipGetLastError(), "v == 1 terms to query order");
    };
    auto back = [&](int p0, int np, void* buf, hipStream_t s) {
        SortedWs w; AbsWalkArgs a;
        view(p0, np, buf, w, a);
        const size_t p = (size_t)p0;
        const float* uq = out_u ? (u_query_order(M) ? w.uslab : w.uq) : nullptr;
        return hip_status(reduce_slabs(w.slab, uq, nullptr, nullptr, out_w + p * M * C,
                                       out_u ? out_u + p * M : nullptr, np, D, M, C, s), "abs reduce");
    };
    if (int e = run_pipeline(P, pl, ws, b1(pl.pc), st, prep, main, back, early)) return e;
    if (keep_sorts) *kept = keep_states ? 3 : 1;
    return QLKA_OK;
}
}  // namespace

extern "C" {

int qlka_abs_fwd(const float* q, const float* k, const float* v, float* out_w, float* out_u,
                 int P, int D, int N, int M, int C, int path, void* ws, size_t ws_bytes_given, void* stream) {
    return abs_fwd_impl(q, k, v, out_w, out_u, P, D, N, M, C, path, nullptr, nullptr, ws, ws_bytes_given, stream);
}

int qlka_abs_fwd_keep(const float* q, const float* k, const float* v, float* out_w, float* out_u,
                      int P, int D, int N, int M, int C, int path, float* k_sorted, uint32_t* k_perm,
                      float* q_sorted, uint32_t* q_perm, void* states, int* kept, void* ws, size_t ws_bytes_given,
                      void* stream) {
    const Presorted keep{k_sorted, k_perm, q_sorted, q_perm, states};
    return abs_fwd_impl(q, k, v, out_w, out_u, P, D, N, M, C, path, &keep, kept, ws, ws_bytes_given, stream);
}

// the widths at which the backward walks once over the merged keys and queries (mbw.hip), which reads no range states
// of the forward's walk
static bool mbw_applies(int C) { return C <= 64 && C % 4 == 0; }

size_t qlka_abs_keep_state_bytes(int P, int D, int N, int M, int C) {
    if (P <= 0 || D <= 0 || N <= 0 || M <= 0 || C <= 0 || C > 128 || N > 131072 || dense_sign(P, N, M)) return 0;
    if (mbw_applies(C)) return 0;
    return kept_state_bytes(P, D, N, C);
}

int qlka_abs_bwd_walks(int P, int N, int M) { return (P > 0 && N > 0 && M > 0 && !dense_sign(P, N, M)) ? 1 : 0; }

// ---- dense forward + backward sharing the kernel matrix A[p,m,n] = sum_d |k[p,d,n] - q[p,d,m]|
// Kept where both directions run dense, the forward runs the tiled kernel, and A (P*M rows of pad4(N) floats) stays
// within DENSE_KEEP_MAX: 46 MB at P = 32, N = M = 600.
constexpr size_t DENSE_KEEP_MAX = size_t(256) << 20;

size_t qlka_abs_dense_keep_bytes(int P, int D, int N, int M, int C) {
    if (P <= 0 || D <= 0 || N <= 0 || M <= 0 || C <= 0 || C > 128 || N > 131072 || M > 131072) return 0;
    if ((int64_t)P * D * std::max(N, M) > (int64_t)INT32_MAX) return 0;
    if (!dense_abs_fwd(N, M) || !dense_sign(P, N, M) || !direct_fwd_tiled(D, N, M, C)) return 0;
    const size_t bytes = (size_t)P * M * (size_t)((N + 3) & ~3) * sizeof(float);
    return bytes <= DENSE_KEEP_MAX ? bytes : 0;
}

int qlka_abs_fwd_dense_keep(const float* q, const float* k, const float* v, float* out_w, float* out_u, float* A,
                            int P, int D, int N, int M, int C, void* stream) {
    g_err.clear();
    if (int e = check_dims(P, D, N, M, C)) return e;
    if (!q || !k || !v || !out_w || !A) return fail(QLKA_EINVAL, "q, k, v, out_w and A must be non-null");
    if (qlka_abs_dense_keep_bytes(P, D, N, M, C) == 0)
        return fail(QLKA_EINVAL, "the dense kernel matrix is not kept at this shape (qlka_abs_dense_keep_bytes is 0)");
    return hip_status(direct_fwd_keep_a(q, k, v, out_w, out_u, A, P, D, N, M, C, (hipStream_t)stream),
                      "abs direct sum keeping A");
}

int qlka_abs_bwd_dense_kept(const float* q, const float* k, const float* v, const float* g_w, const float* g_u,
                            float* grad_q, float* grad_k, float* grad_v, const float* A, int P, int D, int N, int M,
                            int C, void* stream) {
    g_err.clear();
    if (int e = check_dims(P, D, N, M, C)) return e;
    if (!q || !k || !v || !g_w || !grad_q || !grad_k || !grad_v || !A)
        return fail(QLKA_EINVAL, "q, k, v, g_w, the three gradients and A must be non-null");
    if (qlka_abs_dense_keep_bytes(P, D, N, M, C) == 0)
        return fail(QLKA_EINVAL, "the dense kernel matrix is not kept at this shape (qlka_abs_dense_keep_bytes is 0)");
    // the walks' convention, as qlka_abs_bwd: a tie counts -1 in both gradients
    return dense_bwd(-1.f, q, k, v, g_w, g_u, grad_q, grad_k, grad_v, P, D, N, M, C, (hipStream_t)stream, A);
}

// --------------------------------------------------------------------------------------------------- abs backward
static WsSpec abs_bwd_spec(int P, int D, int N, int M, int C) {
    return WsSpec{P, D, N, M, C, std::max(N, M), N, false};   // the grad_v slab has one row per key
}

// The backward as one walk over the merged keys and queries (mbw.hip) where its sums can load rows 16 bytes at a time
// and one channel slot per lane covers a row. Its workspace per chunk: the backward's own sorts (when the forward kept
// none), the merged values and tags, the entry states of its scans and their aggregates, and the slab, which also
// holds the backward's own sorts, the sort scratch and the range summaries (all dead before the walk writes it), so
// that two copies of one configs[4] p (N = M = 131072) fit the default 5 GiB budget and the backward pipelines.

struct MbwWs {
    float* ks; uint32_t* kp; float* qs; uint32_t* qp; void* sort_scratch;
    float* mv; uint32_t* mt;
    float *sa_q, *sb_q, *sa_k, *sa_e;              // summaries (in the slab region)
    float *ta_q, *tb_q, *ta_k, *ta_e;              // entry states
    float* aggs; float* slab; int G;
};

static size_t mbw_rows_bytes(size_t S, int G, int C) { return align256(S * (size_t)(G + 1) * (size_t)(C + 2) * 4); }

static size_t mbw_part(int P, int D, int N, int M, int C, int i) {
    const size_t S = (size_t)P * D;
    const int L = N + M, G = (L + 63) / 64;
    switch (i) {
        case 0: case 1: case 2: case 3: return 0;     // the backward's own sorts live in the slab region
        case 4: case 5: return align256(S * L * 4);
        case 6: return 4 * mbw_rows_bytes(S, G, C);
        case 7: return align256(scan_agg_bytes((int)S, L, C));
        case 8: {
            const size_t slab = align256(S * slab_rows(N) * (size_t)slab_stride(C) * 4);
            const size_t sorted = 2 * align256(S * N * 4) + 2 * align256(S * M * 4);
            return std::max(slab, sorted + std::max(4 * mbw_rows_bytes(S, G, C),
                                                    align256(sort_scratch_need(abs_bwd_spec(P, D, N, M, C)))));
        }
    }
    return 0;
}

static size_t mbw_ws_bytes(int P, int D, int N, int M, int C) {
    size_t b = 0;
    for (int i = 0; i < 9; ++i) b += mbw_part(P, D, N, M, C, i);
    return b;
}

static MbwWs mbw_carve(void* ws, int P, int D, int N, int M, int C) {
    char* part[9];
    char* b = (char*)ws;
    for (int i = 0; i < 9; ++i) { part[i] = b; b += mbw_part(P, D, N, M, C, i); }
    const size_t S = (size_t)P * D;
    MbwWs w;
    w.G = (N + M + 63) / 64;
    const size_t rb = mbw_rows_bytes(S, w.G, C);
    // the slab region: the backward's own sorts (read only by the merge), then the sort scratch, then (over the dead
    // scratch) the range summaries; all of it dead before the walk writes the slab
    const size_t kb = align256(S * (size_t)N * 4), qb = align256(S * (size_t)M * 4);
    char* const sr = part[8];
    w.ks = (float*)sr; w.kp = (uint32_t*)(sr + kb); w.qs = (float*)(sr + 2 * kb); w.qp = (uint32_t*)(sr + 2 * kb + qb);
    char* const after = sr + 2 * kb + 2 * qb;
    w.mv = (float*)part[4]; w.mt = (uint32_t*)part[5];
    w.ta_q = (float*)part[6]; w.tb_q = (float*)(part[6] + rb); w.ta_k = (float*)(part[6] + 2 * rb);
    w.ta_e = (float*)(part[6] + 3 * rb);
    w.aggs = mbw_part(P, D, N, M, C, 7) ? (float*)part[7] : nullptr;
    w.slab = (float*)part[8];
    w.sort_scratch = after;
    w.sa_q = (float*)after; w.sb_q = (float*)(after + rb); w.sa_k = (float*)(after + 2 * rb);
    w.sa_e = (float*)(after + 3 * rb);
    return w;
}

size_t qlka_abs_bwd_ws_bytes(int P, int D, int N, int M, int C) {
    if (P <= 0 || D <= 0 || N <= 0 || M <= 0 || C <= 0) return 0;
    if (dense_sign(P, N, M)) return 0;            // the dense route takes no workspace
    if (mbw_applies(C)) {
        auto bm = [&](int pc) { return mbw_ws_bytes(pc, D, N, M, C); };
        return plan_bytes(plan_chunks(P, g_ws_budget.load(std::memory_order_relaxed), pipelined(P, D, N), bm), bm);
    }
    auto b1 = [&](int pc) { return ws_bytes(abs_bwd_spec(pc, D, N, M, C)); };
    return plan_bytes(plan_chunks(P, g_ws_budget.load(std::memory_order_relaxed), pipelined(P, D, N), b1), b1);
}

}  // extern "C"

namespace {
// The merged backward (mbw.hip), per chunk: the sorts (unless the forward kept them) and the merge of the sorted q and k
// with its range summaries (prep); the scans (early, before the wait for the previous chunk's reduce); the walk (main);
// the grad_v reduce (back). Copy j % 2's slab region, which holds the summaries, is free at prep of chunk j: main of
// chunk j - 1 waited for the reduce of chunk j - 2.
int abs_bwd_mbw(const float* q, const float* k, const float* v, const float* g_w, const float* g_u, float* grad_q,
                float* grad_k, float* grad_v, int P, int D, int N, int M, int C, const Presorted* pre, void* ws,
                size_t ws_bytes_given, hipStream_t st) {
    auto b1 = [&](int pc) { return mbw_ws_bytes(pc, D, N, M, C); };
    const Plan pl = plan_chunks(P, ws_bytes_given, pipelined(P, D, N), b1);
    if (int e = check_ws(ws, ws_bytes_given, plan_bytes(pl, b1))) return e;
    auto view = [&](int p0, int np, void* buf) {
        MbwWs w = mbw_carve(buf, np, D, N, M, C);
        if (pre) {
            const Presorted ps = offset(*pre, (size_t)p0, D, N, M);
            w.ks = ps.ks; w.kp = ps.kp; w.qs = ps.qs; w.qp = ps.qp;
        }
        return w;
    };
    auto prep = [&](int p0, int np, void* buf, hipStream_t s) {
        MbwWs w = view(p0, np, buf);
        const size_t p = (size_t)p0;
        if (!pre) {
            SortedWs sw{};
            sw.ks = w.ks; sw.kp = w.kp; sw.qs = w.qs; sw.qp = w.qp; sw.sort_scratch = w.sort_scratch;
            if (int e = sort_both(q + p * D * M, k + p * D * N, sw, np * D, N, M, s)) return e;
        }
        const int e = merge_sums_launch(w.qs, w.qp, w.ks, w.kp, v + p * N * C, g_w + p * M * C,
                                        g_u ? g_u + p * M : nullptr, w.mv, w.mt, w.sa_q, w.sb_q, w.sa_k, w.sa_e,
                                        np * D, D, N, M, C, w.G, s);
        return hip_status(e, "merge of q and k and its range sums");
    };
    auto early = [&](int p0, int np, void* buf, hipStream_t s) {
        MbwWs w = view(p0, np, buf);
        const int S = np * D;
        if (int e = abs_scan_rows(w.sa_q, w.sb_q, w.ta_q, w.tb_q, w.aggs, S, C, w.G, s))
            return hip_status(e, "merged scan (queries)");
        return hip_status(linked_scan_pair(w.sa_k, w.sa_e, w.ta_k, w.ta_e, w.aggs, S, C, w.G, s),
                          "merged scans (keys, ties)");
    };
    auto main = [&](int p0, int np, void* buf, hipStream_t s) {
        MbwWs w = view(p0, np, buf);
        const size_t p = (size_t)p0;
        return hip_status(mbw_walk_launch(w.mv, w.mt, v + p * N * C, g_w + p * M * C, g_u ? g_u + p * M : nullptr,
                                          w.ta_q, w.tb_q, w.ta_k, w.ta_e, w.slab, grad_q + p * D * M,
                                          grad_k + p * D * N, np * D, D, N, M, C, w.G, s), "merged walk");
    };
    auto back = [&](int p0, int np, void* buf, hipStream_t s) {
        MbwWs w = view(p0, np, buf);
        const int e = reduce_slabs(w.slab, nullptr, nullptr, nullptr, grad_v + (size_t)p0 * N * C, nullptr, np, D, N,
                                   C, s);
        return hip_status(e, "grad_v reduce");
    };
    return run_pipeline(P, pl, ws, b1(pl.pc), st, prep, main, back, early);
}

int abs_bwd_impl(const float* q, const float* k, const float* v, const float* g_w, const float* g_u, float* grad_q,
                 float* grad_k, float* grad_v, int P, int D, int N, int M, int C, const Presorted* pre, void* ws,
                 size_t ws_bytes_given, void* stream) {
    g_err.clear();
    if (int e = check_dims(P, D, N, M, C)) return e;
    if (!q || !k || !v || !g_w || !grad_q || !grad_k || !grad_v)
        return fail(QLKA_EINVAL, "q, k, v, g_w and the three gradients must be non-null");
    hipStream_t st = (hipStream_t)stream;
    if (dense_sign(P, N, M))     // the walks' convention: a tie counts -1 in both gradients
        return dense_bwd(-1.f, q, k, v, g_w, g_u, grad_q, grad_k, grad_v, P, D, N, M, C, st);
    if (mbw_applies(C))
        return abs_bwd_mbw(q, k, v, g_w, g_u, grad_q, grad_k, grad_v, P, D, N, M, C, pre, ws, ws_bytes_given, st);
    auto b1 = [&](int pc) { return ws_bytes(abs_bwd_spec(pc, D, N, M, C)); };
    const Plan pl = plan_chunks(P, ws_bytes_given, pipelined(P, D, N), b1);
    if (int e = check_ws(ws, ws_bytes_given, plan_bytes(pl, b1))) return e;
    // the chunk's workspace view, with the forward's sorts of the chunk when given
    auto view = [&](int p0, int np, void* buf) {
        SortedWs w = carve(buf, abs_bwd_spec(np, D, N, M, C));
        if (pre) {
            const Presorted ps = offset(*pre, (size_t)p0, D, N, M);
            w.ks = ps.ks; w.kp = ps.kp; w.qs = ps.qs; w.qp = ps.qp;
        }
        return w;
    };
    // per chunk: the sorts (unless the forward kept them); the grad_q walk; the grad_k / grad_v walk; the grad_v reduce
    auto prep = [&](int p0, int np, void* buf, hipStream_t s) {
        if (pre) return QLKA_OK;
        SortedWs w = view(p0, np, buf);
        const size_t p = (size_t)p0;
        return sort_both(q + p * D * M, k + p * D * N, w, np * D, N, M, s);
    };
    // The grad_q walk of chunk j runs before the wait for the reduce of chunk j - 1 (`early`), so that reduce has it
    // beside it instead of nothing (configs[4] 83.2 -> 82.2 ms; the headline shape's forward + backward 5.12 -> 5.06
    // ms). Only the grad_k / grad_v walk writes the slab copy, which that wait protects.
    auto early = [&](int p0, int np, void* buf, hipStream_t s) {
        SortedWs w = view(p0, np, buf);
        const size_t p = (size_t)p0;
        // grad_q: stream = sorted k with rows v, queries = q, dotted with g_w (+ g_u * (2 rank - N))
        AbsWalkArgs a{};
        a.ks = w.ks; a.kp = w.kp; a.Ns = N; a.w = v + p * N * C; a.u = nullptr;
        a.qs = w.qs; a.qp = w.qp; a.Mq = M; a.g = g_w + p * M * C; a.uq = g_u ? g_u + p * M : nullptr;
        a.out_dot = grad_q + p * D * M; a.sign = 1.f; a.P = np; a.D = D; a.C = C;
        const int mode_q = g_u ? (ABS_DOT | ABS_DOTX1) : ABS_DOT;
        if (pre && pre->states) {   // the forward's range states and bounds of this walk: only the walk runs
            RangeArrays ra = w.ra;
            kept_states(pre->states, P, D, N, C, p, ra);
            if (int e = abs_emit(a, mode_q, ra, s)) return hip_status(e, "grad_q walk");
        } else if (int e = abs_walk(a, mode_q, w.ra, s)) {
            return hip_status(e, "grad_q walk");
        }
        return QLKA_OK;
    };
    auto main = [&](int p0, int np, void* buf, hipStream_t s) {
        SortedWs w = view(p0, np, buf);
        const size_t p = (size_t)p0;
        // grad_k and grad_v: stream = sorted q with rows g_w (+ scalars g_u), queries = k
        AbsWalkArgs b{};
        b.ks = w.qs; b.kp = w.qp; b.Ns = M; b.w = g_w + p * M * C; b.u = g_u ? g_u + p * M : nullptr;
        b.qs = w.ks; b.qp = w.kp; b.Mq = N; b.g = v + p * N * C; b.uq = nullptr;
        b.slab = w.slab; b.uslab = nullptr; b.CR = slab_stride(C);
        b.out_dot = grad_k + p * D * N; b.sign = 1.f; b.P = np; b.D = D; b.C = C;
        const int e = abs_walk(b, g_u ? (ABS_ROW | ABS_DOT | ABS_DOTX2) : (ABS_ROW | ABS_DOT), w.ra, s);
        return hip_status(e, "grad_k/grad_v walk");
    };
    auto back = [&](int p0, int np, void* buf, hipStream_t s) {
        SortedWs w = view(p0, np, buf);
        const int e = reduce_slabs(w.slab, nullptr, nullptr, nullptr, grad_v + (size_t)p0 * N * C, nullptr, np, D, N,
                                   C, s);
        return hip_status(e, "grad_v reduce");
    };
    return run_pipeline(P, pl, ws, b1(pl.pc), st, prep, main, back, early);
}
}  // namespace

extern "C" {

int qlka_abs_bwd(const float* q, const float* k, const float* v, const float* g_w, const float* g_u,
                 float* grad_q, float* grad_k, float* grad_v,
                 int P, int D, int N, int M, int C, void* ws, size_t ws_bytes_given, void* stream) {
    return abs_bwd_impl(q, k, v, g_w, g_u, grad_q, grad_k, grad_v, P, D, N, M, C, nullptr, ws, ws_bytes_given, stream);
}

int qlka_abs_bwd_sorted(const float* q, const float* k, const float* v, const float* g_w, const float* g_u,
                        float* grad_q, float* grad_k, float* grad_v, int P, int D, int N, int M, int C,
                        const float* k_sorted, const uint32_t* k_perm, const float* q_sorted, const uint32_t* q_perm,
                        const void* states, void* ws, size_t ws_bytes_given, void* stream) {
    if (!k_sorted || !k_perm || !q_sorted || !q_perm) {
        g_err.clear();
        return fail(QLKA_EINVAL, "the sorted k / q arrays and their permutations must be non-null");
    }
    const Presorted pre{const_cast<float*>(k_sorted), const_cast<uint32_t*>(k_perm), const_cast<float*>(q_sorted),
                        const_cast<uint32_t*>(q_perm), const_cast<void*>(states)};
    return abs_bwd_impl(q, k, v, g_w, g_u, grad_q, grad_k, grad_v, P, D, N, M, C, &pre, ws, ws_bytes_given, stream);
}

// -------------------------------------------------------------------------------------------------------- sgn sum
static WsSpec sgn_spec(int P, int D, int N, int M, int C) { return WsSpec{P, D, N, M, C, N, 0, false}; }

size_t qlka_sgn_fwd_ws_bytes(int P, int D, int N, int M, int C) {
    if (P <= 0 || D <= 0 || N <= 0 || M <= 0 || C <= 0) return 0;
    if (dense_sign(P, N, M)) return 0;            // the dense route takes no workspace
    return budget_bytes(P, [&](int pc) { return ws_bytes(sgn_spec(pc, D, N, M, C)); });
}

int qlka_sgn_fwd(const float* q, const float* k, const float* v, const float* g, float* out,
                 int P, int D, int N, int M, int C, void* ws, size_t ws_bytes_given, void* stream) {
    g_err.clear();
    if (int e = check_dims(P, D, N, M, C)) return e;
    if (!q || !k || !v || !g || !out) return fail(QLKA_EINVAL, "q, k, v, g and out must be non-null");
    hipStream_t st = (hipStream_t)stream;
    if (dense_sign(P, N, M))     // sgn(k - q) with a tie counted +1 == -(s(q - k) with a tie counted -1)
        return hip_status(direct_sign(true, q, k, g, v, nullptr, out, -1.f, -1.f, P, D, M, N, C, st), "dense sgn sum");
    auto bytes = [&](int pc) { return ws_bytes(sgn_spec(pc, D, N, M, C)); };
    const int pc = fit_chunk(P, ws_bytes_given, bytes);
    if (int e = check_ws(ws, ws_bytes_given, bytes(pc))) return e;
    return for_chunks(P, pc, [&](int p0, int np) {
        const size_t p = (size_t)p0;
        SortedWs w = carve(ws, sgn_spec(np, D, N, M, C));
        if (int e = sort_both(q + p * D * M, k + p * D * N, w, np * D, N, M, st)) return e;
        AbsWalkArgs a{};
        a.ks = w.ks; a.kp = w.kp; a.Ns = N; a.w = v + p * N * C;
        a.qs = w.qs; a.qp = w.qp; a.Mq = M; a.g = g + p * M * C;
        a.out_dot = out + p * D * M; a.sign = -1.f; a.P = np; a.D = D; a.C = C;
        return hip_status(abs_walk(a, ABS_DOT, w.ra, st), "sgn walk");
    });
}

// -------------------------------------------------------------------------------------------- direct evaluation
int qlka_direct_fwd(int kind, const float* q, const float* k, const float* v, float* out_w, float* out_u,
                    int P, int D, int N, int M, int C, void* stream) {
    g_err.clear();
    if (kind < 0 || kind > 1) return fail(QLKA_EINVAL, "kind must be 0 (abs) or 1 (laplace)");
    if (int e = check_dims(P, D, N, M, C)) return e;
    if (!q || !k || !v || !out_w) return fail(QLKA_EINVAL, "q, k, v and out_w must be non-null");
    return hip_status(direct_fwd(kind, q, k, v, out_w, out_u, P, D, N, M, C, (hipStream_t)stream), "direct sum");
}

int qlka_direct_bwd(float tie, const float* q, const float* k, const float* v, const float* g_w, const float* g_u,
                    float* grad_q, float* grad_k, float* grad_v, int P, int D, int N, int M, int C, void* stream) {
    g_err.clear();
    if (int e = check_dims(P, D, N, M, C)) return e;
    if (!q || !k || !v || !g_w || !grad_q || !grad_k || !grad_v)
        return fail(QLKA_EINVAL, "q, k, v, g_w and the three gradients must be non-null");
    return dense_bwd(tie, q, k, v, g_w, g_u, grad_q, grad_k, grad_v, P, D, N, M, C, (hipStream_t)stream);
}

int qlka_direct_sgn(float tie, const float* q, const float* k, const float* v, const float* g, float* out,
                    int P, int D, int N, int M, int C, void* stream) {
    g_err.clear();
    if (int e = check_dims(P, D, N, M, C)) return e;
    if (!q || !k || !v || !g || !out) return fail(QLKA_EINVAL, "q, k, v, g and out must be non-null");
    // sum_n s(k - q) <v_n, g_m> with s(0) = tie  ==  -(sum_n s'(q - k) <g_m, v_n>) with s'(0) = -tie
    return hip_status(direct_sign(true, q, k, g, v, nullptr, out, -tie, -1.f, P, D, M, N, C, (hipStream_t)stream),
                      "direct sgn sum");
}

// ------------------------------------------------------------------------------------------- fused attention layers
// Workspace: the op's (sorted k/q, ranges, slab) + per-query terms + the add_riesz prefixes + the masked keys of
// add_laplace. add_bump, with the epilogue folded into its reduce: the query bounds of its two shifted query sets and
// a second and third slab (+ v == 1 terms) for them; otherwise an out_w / out_u pair per evaluation (the op's slab
// serves the three evaluations in turn). add_laplace / add_riesz fold their epilogue into the reduce or use one pair.
namespace {
struct LayerWs {
    SortedWs op;
    float* w[3]; float* u[3];
    void* pre; int* qb[2];
    float* qt;
    float* kmask;
    float* slab2[2]; float* uslab2[2]; float* uq2[2];   // add_bump's q + 1 and q - 1 rows (folded epilogue)
};

bool bump_folded(int kind, const WsSpec& s) { return kind == LAYER_ADD_BUMP && reduce_folds_epilogue(s.M, s.C); }

size_t layer_part(int kind, const WsSpec& s, int i) {
    const size_t PMC = (size_t)s.P * s.M * s.C, PM = (size_t)s.P * s.M;
    const int nev = bump_folded(kind, s) ? 0 : (kind == LAYER_ADD_BUMP) ? 3 : 1;
    switch (i) {
        case 0: return ws_bytes(s);
        case 1: return nev * (align256(PMC * 4) + align256(PM * 4)) + align256(PM * 4);   // + per-query terms
        case 2: return kind == LAYER_ADD_RIESZ ? align256(riesz_prefix_bytes(s.P, s.N, s.C)) : 0;
        case 3: return kind == LAYER_ADD_BUMP
                       ? 2 * align256((size_t)s.P * s.D * range_count(s.N, s.C) * sizeof(int)) : 0;
        case 4: return kind == LAYER_ADD_LAPLACE ? align256((size_t)s.P * s.D * s.N * 4) : 0;   // masked keys
        case 5: return bump_folded(kind, s) ? 2 * (ws_part(s, 6) + ws_part(s, 7) + ws_part(s, 8)) : 0;
    }
    return 0;
}

size_t layer_ws_bytes(int kind, const WsSpec& s) {
    size_t b = 0;
    for (int i = 0; i < 6; ++i) b += layer_part(kind, s, i);
    return b;
}

LayerWs carve_layer(int kind, void* ws, const WsSpec& s) {
    LayerWs r{};
    char* part[6];
    char* b = (char*)ws;
    for (int i = 0; i < 6; ++i) { part[i] = b; b += layer_part(kind, s, i); }
    r.op = carve(part[0], s);
    const size_t PMC = (size_t)s.P * s.M * s.C, PM = (size_t)s.P * s.M;
    const int nev = bump_folded(kind, s) ? 0 : (kind == LAYER_ADD_BUMP) ? 3 : 1;
    b = part[1];
    for (int e = 0; e < nev; ++e) {
        r.w[e] = (float*)b; b += align256(PMC * 4);
        r.u[e] = (float*)b; b += align256(PM * 4);
    }
    r.qt = (float*)b;
    r.pre = layer_part(kind, s, 2) ? (void*)part[2] : nullptr;
    if (kind == LAYER_ADD_BUMP) {
        const size_t qbb = align256((size_t)s.P * s.D * range_count(s.N, s.C) * sizeof(int));
        r.qb[0] = (int*)part[3];
        r.qb[1] = (int*)(part[3] + qbb);
    }
    r.kmask = layer_part(kind, s, 4) ? (float*)part[4] : nullptr;
    if (bump_folded(kind, s)) {
        b = part[5];
        for (int e = 0; e < 2; ++e) {
            r.slab2[e] = (float*)b;  b += ws_part(s, 6);
            r.uslab2[e] = (float*)b; b += ws_part(s, 7);
            r.uq2[e] = (float*)b;    b += ws_part(s, 8);
        }
    }
    return r;
}
}  // namespace

// add_bump without a foldable epilogue runs three walks and reduces over one slab per chunk: its chunks run in order
static bool layer_pipelined(int kind, int P, int D, int M, int C) {
    return (kind != LAYER_ADD_BUMP || reduce_folds_epilogue(M, C)) && pipelined(P, D, M);
}

size_t qlka_layer_fwd_ws_bytes(int kind, int P, int D, int N, int M, int C) {
    if (P <= 0 || D <= 0 || N <= 0 || M <= 0 || C <= 0 || kind < 0 || kind > 2) return 0;
    auto b1 = [&](int pc) { return layer_ws_bytes(kind, WsSpec{pc, D, N, M, C, N, M, true}); };
    const size_t cap = g_ws_budget.load(std::memory_order_relaxed);
    return plan_bytes(plan_chunks(P, cap, layer_pipelined(kind, P, D, M, C), b1), b1);
}

// Both layer entry points: keep == null is the reference's composition over pre-masked k, v and n_pad; keep != null
// applies the key mask inside the sums (k and v as given, no n_pad).
// add_laplace / add_riesz: the query terms, then the slab reduce with the epilogue folded in (writes out).
static int layer_reduce_folded(int kind, bool masked, const float* q, const float* n_pad, LayerWs& L, float* out,
                               int P, int D, int M, int C, hipStream_t st) {
    ReduceEpilogue ep{};
    if (int e = layer_epilogue_params(kind, masked, q, n_pad, L.pre, L.qt, out, P, D, M, C, &ep, st))
        return hip_status(e, "layer query terms");
    SortedWs& w = L.op;
    return hip_status(reduce_slabs_layer(kind, masked, ep, w.slab, w.uslab, w.qp, w.uq, P, D, M, C, st),
                      "layer reduce");
}

// add_bump over one chunk of P p (pointers offset to its first p) when its reduce cannot take the epilogue (C / 4 not
// a power of two): one sort of k and q, one set of range summaries and one scan serve the three query shifts (q + s
// has the sorted order of q, and the key side does not depend on the queries); per shift a walk and a reduce over
// the one slab, then the epilogue.
static int bump_chunk_unfolded(const float* q, const float* k, const float* v, const float* n_pad,
                               const uint8_t* keep, float* out, int P, int D, int N, int M, int C, void* ws,
                               hipStream_t st) {
    const WsSpec spec{P, D, N, M, C, N, M, true};
    const int S = P * D;
    LayerWs L = carve_layer(LAYER_ADD_BUMP, ws, spec);
    SortedWs& w = L.op;
    if (int e = hip_status(seg_sort(k, w.ks, w.kp, S, N, w.sort_scratch, st), "segmented sort of k")) return e;
    AbsWalkArgs a{};
    a.ks = w.ks; a.kp = w.kp; a.Ns = N; a.w = v; a.u = nullptr; a.keep = keep;
    a.qs = w.qs; a.qp = w.qp; a.Mq = M; a.g = nullptr; a.uq = nullptr;
    a.slab = w.slab; a.uslab = w.uslab; a.CR = slab_stride(C);
    a.out_dot = nullptr; a.out_rank = nullptr;
    a.sign = 1.f; a.P = P; a.D = D; a.C = C; a.qshift = 0.f;
    const int mode = ABS_ROW | ABS_ONES | (keep ? ABS_KEEP : 0);
    const float shift[3] = {0.f, 1.f, -1.f};
    int* qbs[3] = {w.ra.qb, L.qb[0], L.qb[1]};
    int e = fork_join(st,
        [&](hipStream_t s) { return hip_status(abs_prepare(a, mode, w.ra, s), "abs ranges"); },
        [&](hipStream_t s) {
            if (int r = hip_status(seg_sort(q, w.qs, w.qp, S, M, w.sort_scratch, s), "segmented sort of q")) return r;
            for (int ev = 0; ev < 3; ++ev) {
                AbsWalkArgs b = a;
                b.qshift = shift[ev];
                if (int r = range_bounds(b, qbs[ev], s)) return hip_status(r, "query bounds");
            }
            return QLKA_OK; });
    if (e) return e;
    for (int ev = 0; ev < 3; ++ev) {
        RangeArrays ra = w.ra;
        a.qshift = shift[ev];
        ra.qb = qbs[ev];
        if ((e = abs_emit(a, mode, ra, st))) return hip_status(e, "abs walk");
        if ((e = reduce_slabs(w.slab, w.uslab, w.qp, w.uq, L.w[ev], L.u[ev], P, D, M, C, st)))
            return hip_status(e, "abs reduce");
    }
    e = layer_epilogue(LAYER_ADD_BUMP, keep != nullptr, q, n_pad, L.w[0], L.u[0], L.w[1], L.u[1], L.w[2], L.u[2],
                       L.pre, L.qt, out, P, D, N, M, C, st);
    return hip_status(e, "layer epilogue");
}

static int layer_fwd(int kind, const float* q, const float* k, const float* v, const float* n_pad,
                     const uint8_t* keep, float* out, int P, int D, int N, int M, int C, void* ws,
                     size_t ws_bytes_given, void* stream) {
    if (kind < 0 || kind > 2) return fail(QLKA_EINVAL, "kind must be 0 (add_laplace), 1 (add_riesz) or 2 (add_bump)");
    if (int e = check_dims(P, D, N, M, C)) return e;
    if (!q || !k || !v || !out) return fail(QLKA_EINVAL, "q, k, v and out must be non-null");
    auto b1 = [&](int pc) { return layer_ws_bytes(kind, WsSpec{pc, D, N, M, C, N, M, true}); };
    const Plan pl = plan_chunks(P, ws_bytes_given, layer_pipelined(kind, P, D, M, C), b1);
    if (int e = check_ws(ws, ws_bytes_given, plan_bytes(pl, b1))) return e;
    hipStream_t st = (hipStream_t)stream;
    auto chunk_in = [&](int p0, const float*& qc, const float*& kc, const float*& vc, const float*& npc,
                        const uint8_t*& keepc, float*& outc) {
        const size_t p = (size_t)p0;
        qc = q + p * D * M; kc = k + p * D * N; vc = v + p * N * C;
        npc = n_pad ? n_pad + p : nullptr; keepc = keep ? keep + p * N : nullptr; outc = out + p * M * C;
    };
    const bool bump = kind == LAYER_ADD_BUMP;
    if (kind == LAYER_ADD_RIESZ && keep == nullptr && few_keys(N))   // the abs sums dense (few_keys), then the epilogue
        return for_chunks(P, pl.pc, [&](int p0, int np) {
            const float *qc, *kc, *vc, *npc; const uint8_t* keepc; float* outc;
            chunk_in(p0, qc, kc, vc, npc, keepc, outc);
            LayerWs L = carve_layer(kind, ws, WsSpec{np, D, N, M, C, N, M, true});
            if (int e = riesz_prefix(kc, vc, nullptr, L.pre, np, D, N, C, st)) return hip_status(e, "riesz prefixes");
            if (int e = direct_fwd(0, qc, kc, vc, L.w[0], L.u[0], np, D, N, M, C, st))
                return hip_status(e, "abs direct sum");
            return hip_status(layer_epilogue(kind, false, qc, npc, L.w[0], L.u[0], nullptr, nullptr, nullptr, nullptr,
                                             L.pre, L.qt, outc, np, D, N, M, C, st), "layer epilogue"); });
    if (bump && !reduce_folds_epilogue(M, C))   // three walks and reduces over one slab per chunk: chunks in order
        return for_chunks(P, pl.pc, [&](int p0, int np) {
            const float *qc, *kc, *vc, *npc; const uint8_t* keepc; float* outc;
            chunk_in(p0, qc, kc, vc, npc, keepc, outc);
            return bump_chunk_unfolded(qc, kc, vc, npc, keepc, outc, np, D, N, M, C, ws, st); });
    // Per chunk: (mask keys,) sort k, group q (add_bump: sort q and find the range bounds of q, q + 1, q - 1); range
    // passes (+ riesz prefixes) and the walk (add_bump: one walk over the three query sets into three slabs); the
    // reduce with the epilogue. fp32 addition of a constant is monotone, so q + 1 and q - 1 keep the sorted order of q,
    // and every walk sees exactly the fp32 values q + 1 and q - 1 the reference passes.
    const bool masked = keep != nullptr;
    const float shift[3] = {0.f, 1.f, -1.f};
    auto prep = [&](int p0, int np, void* buf, hipStream_t s) {
        const float *qc, *kc, *vc, *npc; const uint8_t* keepc; float* outc;
        chunk_in(p0, qc, kc, vc, npc, keepc, outc);
        LayerWs L = carve_layer(kind, buf, WsSpec{np, D, N, M, C, N, M, true});
        if (bump) {   // one launch per step, so that the prep's kernels start together beside a reduce
            SortedWs& w = L.op;
            if (int e = hip_status(sort_pair(qc, kc, w, np * D, N, M, s), "segmented sort of k and q")) return e;
            int* const qbs[3] = {w.ra.qb, L.qb[0], L.qb[1]};
            return hip_status(query_bounds_sets(w.ks, w.qs, qbs, shift, 3, np * D, N, M, C, s), "query bounds");
        }
        // masked add_laplace: masked keys become FLT_MAX (terms exactly 0, sorted last) and the unmasked walk runs
        const bool lap_masked = kind == LAYER_ADD_LAPLACE && masked;
        if (lap_masked)
            if (int e = hip_status(mask_keys(kc, keepc, L.kmask, np, D, N, s), "masked keys")) return e;
        if (kind == LAYER_ADD_RIESZ && masked) {
            // the abs walk's distances and totals between kept keys only (fill_masked_keys); the grouping then runs on
            // the filled keys, as the walk ranks queries among them
            if (int e = hip_status(seg_sort(kc, L.op.ks, L.op.kp, np * D, N, L.op.sort_scratch, s), "segmented sort of k"))
                return e;
            if (int e = hip_status(fill_masked_keys(L.op.ks, L.op.kp, keepc, np, D, N, s), "masked keys")) return e;
            return group_q(qc, L.op, 0.f, np * D, N, M, C, s);
        }
        return sort_k_group_q(lap_masked ? L.kmask : kc, qc, L.op, 0.f, np * D, N, M, C, s);
    };
    // the abs walk's arguments of a chunk (add_riesz, add_bump)
    auto abs_args = [&](const SortedWs& w, const float* vc, const uint8_t* keepc, int np) {
        AbsWalkArgs a{};
        a.ks = w.ks; a.kp = w.kp; a.Ns = N; a.w = vc; a.u = nullptr; a.keep = keepc;
        a.qs = w.qs; a.qp = w.qp; a.Mq = M; a.g = nullptr; a.uq = nullptr;
        a.slab = w.slab; a.uslab = w.uslab; a.CR = slab_stride(C);
        a.out_dot = nullptr; a.out_rank = nullptr;
        a.sign = 1.f; a.P = np; a.D = D; a.C = C; a.qshift = 0.f;
        return a;
    };
    const int abs_mode = ABS_ROW | ABS_ONES | (masked ? ABS_KEEP : 0);
    // the range passes (and add_riesz's per-p prefixes) before the wait for the previous chunk's reduce, beside it
    auto early = [&](int p0, int np, void* buf, hipStream_t s) {
        const float *qc, *kc, *vc, *npc; const uint8_t* keepc; float* outc;
        chunk_in(p0, qc, kc, vc, npc, keepc, outc);
        LayerWs L = carve_layer(kind, buf, WsSpec{np, D, N, M, C, N, M, true});
        SortedWs& w = L.op;
        if (kind == LAYER_ADD_LAPLACE)
            return hip_status(laplace_prepare(w.ks, w.kp, vc, np, D, N, C, w.ra, s), "laplace ranges");
        if (int e = hip_status(abs_prepare(abs_args(w, vc, keepc, np), abs_mode, w.ra, s), "abs ranges")) return e;
        if (!bump)
            if (int e = riesz_prefix(kc, vc, keepc, L.pre, np, D, N, C, s)) return hip_status(e, "riesz prefixes");
        return (int)QLKA_OK;
    };
    auto main = [&](int p0, int np, void* buf, hipStream_t s) {
        const float *qc, *kc, *vc, *npc; const uint8_t* keepc; float* outc;
        chunk_in(p0, qc, kc, vc, npc, keepc, outc);
        LayerWs L = carve_layer(kind, buf, WsSpec{np, D, N, M, C, N, M, true});
        SortedWs& w = L.op;
        if (kind == LAYER_ADD_LAPLACE) {
            if (int e = laplace_emit(w.ks, w.kp, w.qs, w.qp, vc, w.slab, w.uslab, np, D, N, M, C, w.ra, s))
                return hip_status(e, "laplace walk");
            order_u_terms(w.uslab, w.qp, w.uq, np, D, M, s);
            return hip_status((int)hipGetLastError(), "v == 1 terms to query order");
        }
        AbsWalkArgs a = abs_args(w, vc, keepc, np);
        const int mode = abs_mode;
        if (bump) {
            a.nsets = 3;
            for (int ev = 1; ev < 3; ++ev) {
                a.set_shift[ev] = shift[ev];
                a.set_qb[ev] = L.qb[ev - 1];
                a.set_slab[ev] = L.slab2[ev - 1];
                a.set_uslab[ev] = L.uslab2[ev - 1];
            }
        }
        if (int e = hip_status(abs_emit(a, mode, w.ra, s), "abs walk")) return e;
        if (bump) {
            const float* us[3] = {w.uslab, L.uslab2[0], L.uslab2[1]};
            float* uqs[3] = {w.uq, L.uq2[0], L.uq2[1]};
            order_u_terms_sets(us, w.qp, uqs, 3, np, D, M, s);
        } else {
            order_u_terms(w.uslab, w.qp, w.uq, np, D, M, s);
        }
        return hip_status((int)hipGetLastError(), "v == 1 terms to query order");
    };
    auto back = [&](int p0, int np, void* buf, hipStream_t s) {
        const float *qc, *kc, *vc, *npc; const uint8_t* keepc; float* outc;
        chunk_in(p0, qc, kc, vc, npc, keepc, outc);
        LayerWs L = carve_layer(kind, buf, WsSpec{np, D, N, M, C, N, M, true});
        SortedWs& w = L.op;
        w.uslab = u_query_order(M) ? w.uslab : w.uq;       // query order (main put the terms there)
        w.qp = nullptr;
        if (bump) {
            ReduceEpilogue ep{};
            if (int e = layer_epilogue_params(kind, masked, qc, npc, L.pre, L.qt, outc, np, D, M, C, &ep, s))
                return hip_status(e, "layer query terms");
            const float* slabs[3] = {w.slab, L.slab2[0], L.slab2[1]};
            const float* uqs[3] = {w.uslab, u_query_order(M) ? L.uslab2[0] : L.uq2[0],
                                   u_query_order(M) ? L.uslab2[1] : L.uq2[1]};
            return hip_status(reduce_slabs_bump(masked, ep, slabs, uqs, np, D, M, C, s), "layer reduce");
        }
        if (reduce_folds_epilogue(M, C))
            return layer_reduce_folded(kind, masked, qc, npc, L, outc, np, D, M, C, s);
        if (int e = reduce_slabs(w.slab, w.uslab, nullptr, nullptr, L.w[0], L.u[0], np, D, M, C, s))
            return hip_status(e, "layer reduce");
        return hip_status(layer_epilogue(kind, masked, qc, npc, L.w[0], L.u[0], nullptr, nullptr, nullptr, nullptr,
                                         L.pre, L.qt, outc, np, D, N, M, C, s), "layer epilogue");
    };
    return run_pipeline(P, pl, ws, b1(pl.pc), st, prep, main, back, early);
}

int qlka_layer_fwd(int kind, const float* q, const float* k, const float* v, const float* n_pad, float* out,
                   int P, int D, int N, int M, int C, void* ws, size_t ws_bytes_given, void* stream) {
    g_err.clear();
    return layer_fwd(kind, q, k, v, n_pad, nullptr, out, P, D, N, M, C, ws, ws_bytes_given, stream);
}

int qlka_layer_fwd_masked(int kind, const float* q, const float* k, const float* v, const uint8_t* keep, float* out,
                          int P, int D, int N, int M, int C, void* ws, size_t ws_bytes_given, void* stream) {
    g_err.clear();
    if (!keep) return fail(QLKA_EINVAL, "keep must be non-null (qlka_layer_fwd is the unmasked entry)");
    return layer_fwd(kind, q, k, v, nullptr, keep, out, P, D, N, M, C, ws, ws_bytes_given, stream);
}

// ------------------------------------------------------------------------------------------------ test entries
size_t qlka_seg_sort_ws_bytes(int num_segs, int seg_len) {
    if (num_segs <= 0 || seg_len <= 0) return 0;
    return seg_sort_scratch_bytes(num_segs, seg_len);
}

int qlka_seg_sort(const float* keys, float* sorted, uint32_t* perm, int num_segs, int seg_len,
                  void* ws, size_t ws_bytes, void* stream) {
    g_err.clear();
    if (num_segs <= 0 || seg_len <= 0) return fail(QLKA_EINVAL, "num_segs and seg_len must be > 0");
    if ((int64_t)num_segs * seg_len > (int64_t)INT32_MAX) return fail(QLKA_EINVAL, "num_segs*seg_len must fit int32");
    if (!keys || !sorted || !perm) return fail(QLKA_EINVAL, "keys, sorted and perm must be non-null");
    if (int e = check_ws(ws, ws_bytes, qlka_seg_sort_ws_bytes(num_segs, seg_len))) return e;
    return hip_status(seg_sort(keys, sorted, perm, num_segs, seg_len, ws, (hipStream_t)stream),
                      "segmented sort");
}

size_t qlka_merge_rank_ws_bytes(int num_segs, int N, int M) {
    if (num_segs <= 0 || N <= 0 || M <= 0) return 0;
    return ws_bytes(WsSpec{num_segs, 1, N, M, 1, N, 0, false});
}

int qlka_merge_rank(const float* q, const float* k, int32_t* rank, int num_segs, int N, int M,
                    void* ws, size_t ws_bytes_given, void* stream) {
    g_err.clear();
    if (int e = check_dims(num_segs, 1, N, M, 1)) return e;
    if (!q || !k || !rank) return fail(QLKA_EINVAL, "q, k and rank must be non-null");
    if (int e = check_ws(ws, ws_bytes_given, qlka_merge_rank_ws_bytes(num_segs, N, M))) return e;
    hipStream_t st = (hipStream_t)stream;
    SortedWs w = carve(ws, WsSpec{num_segs, 1, N, M, 1, N, 0, false});
    if (int e = sort_both(q, k, w, num_segs, N, M, st)) return e;
    AbsWalkArgs a{};
    a.ks = w.ks; a.kp = w.kp; a.Ns = N; a.w = nullptr;
    a.qs = w.qs; a.qp = w.qp; a.Mq = M;
    a.out_rank = rank; a.P = num_segs; a.D = 1; a.C = 1;
    return hip_status(abs_walk(a, ABS_RANK, w.ra, st), "rank walk");
}

}  // extern "C"

namespace qlka {
// For the allocation-free entry point (noalloc.hip), which runs qlka_laplace_fwd over its own static workspace.
int validate_dims(int P, int D, int N, int M, int C) {
    g_err.clear();
    return check_dims(P, D, N, M, C);
}
size_t laplace_fwd_chunk_ws(int pc, int D, int N, int M, int C) { return ws_bytes(laplace_spec(pc, D, N, M, C)); }
int report_error(int code, const char* msg) { return fail(code, "%s", msg); }
}  // namespace qlka
