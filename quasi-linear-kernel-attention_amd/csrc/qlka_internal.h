// Host-side launchers shared between the kernel files and the C ABI (capi.hip). Not part of the public interface.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace qlka {

// Brackets one kernel launch with hipEvents on its stream when qlka_timing_enable(1) is set (timing.hip).
class StageTimer {
public:
    StageTimer(const char* name, hipStream_t st);
    ~StageTimer();
    StageTimer(const StageTimer&) = delete;
    StageTimer& operator=(const StageTimer&) = delete;
private:
    const char* name_;
    hipStream_t st_;
    hipEvent_t a_ = nullptr, b_ = nullptr;
};

// Longest run the LDS radix sort handles in one workgroup (16384 keys * (4 B key + 4 B index) = 128 KB of LDS).
constexpr int LDS_SORT_MAX = 16384;

// Layer epilogue constants (Weighted_Laplace_Sum/attention.py: the denominator clamp and add_riesz's epsilon).
constexpr float LAYER_CLAMP = 1e-6f;
constexpr float LAYER_EPS = 1e-3f;

// ---- sort.hip ----
size_t seg_sort_scratch_bytes(int S, int L);
// Stable ascending sort of S contiguous segments of length L. Returns a hipError_t value (0 on success).
int seg_sort(const float* in, float* out_keys, uint32_t* out_perm, int S, int L, void* scratch,
             hipStream_t st);
// seg_sort of two arrays of S segments of length L as one sort of 2S segments: one LDS-sort launch (so that the two
// sorts start together when they run beside other work) and, for segments longer than one LDS run, each merge pass
// over both arrays in one launch; scratch of seg_sort_scratch_bytes(2 S, L) bytes
int seg_sort2(const float* a, float* a_keys, uint32_t* a_perm, const float* b, float* b_keys, uint32_t* b_perm,
              int S, int L, void* scratch, hipStream_t st);

// ---- walks.hip ----
// Keys per key range (one wave per range) for a channel count C.
__host__ __device__ inline int range_keys(int C) { return C <= 64 ? 64 : 32; }
// Floats per range row in the range arrays (C channels + 2 scalar extras).
__host__ __device__ inline int range_stride(int C) { return C + 2; }

// Per-range arrays of the walks. The sums kernel writes the summaries (sa, sb); the scan reads them and writes the
// entry/exit states (ta, tb) to separate arrays: a kernel never reads memory it also writes (a uniform-address read
// may become a scalar load that the compiler treats as invariant and moves past the kernel's own vector stores).
struct RangeArrays {
    float* sa;   // [S][G+1][stride] range summaries
    float* sb;   // [S][G+1][stride]
    float* ta;   // [S][G+1][stride] range states (written by the scan)
    float* tb;   // [S][G+1][stride]
    int*   qb;   // [S][G]
    float* aggs; // per-workgroup scan aggregates of segments longer than one scan workgroup (else nullptr)
};
size_t range_arrays_bytes(int S, int Nstream, int C);
RangeArrays carve_range_arrays(void* base, int S, int Nstream, int C);

// Fill n floats with zero (a kernel, so it can sit inside a captured graph).
int fill_zero(float* p, size_t n, hipStream_t st);

// Row stride (floats) of the per-feature contribution slab: C rounded up to whole 128-byte lines.
__host__ __device__ inline int slab_stride(int C) { return (C + 31) / 32 * 32; }

// Slab layout. One row of slab_stride(C) floats per (p, d, query m). The D features of a p form groups of
// G = slab_group(D) features (2 when D is even, else 1); inside a group the rows are blocked by 64 queries:
//   [p][d / G][m / 64][d % G][m % 64][row]
// so the D-fold reduce reads G * 64 contiguous rows at a time. Measured at the headline shape against the plain
// [p][d][m] layout (G = 1): the reduce reads faster (0.57 vs 0.64 ms) for slightly slower walk stores (+0.03 ms);
// G = 4, 8, 16 and 32- or 128-query blocks come within 1% of G = 2. A feature has slab_rows(M) rows, and a
// (p, group) region stays far below 2^31 bytes (32-bit buffer offsets).
constexpr int SLAB_QB_LOG = 6;
constexpr int SLAB_QB = 1 << SLAB_QB_LOG;
constexpr int SLAB_GMAX = 2;
__host__ __device__ inline int slab_group(int D) {
    for (int g = D < SLAB_GMAX ? D : SLAB_GMAX; g > 1; --g)
        if (D % g == 0) return g;
    return 1;
}
__host__ __device__ inline int slab_rows(int M) { return (M + SLAB_QB - 1) / SLAB_QB * SLAB_QB; }
// float offset of segment (p, d)'s first row, and the bytes from there to the end of its group's region
__host__ __device__ inline size_t slab_seg_base(int p, int d, int D, int M, int CR) {
    const int G = slab_group(D);
    return ((size_t)p * D + (size_t)(d / G) * G) * slab_rows(M) * CR + (size_t)(d % G) * SLAB_QB * CR;
}
__host__ __device__ inline uint32_t slab_seg_bytes(int d, int D, int M, int CR) {
    const int G = slab_group(D);
    return (uint32_t)(((size_t)G * slab_rows(M) - (size_t)(d % G) * SLAB_QB) * CR * 4);
}
// byte offset of query m's row from its segment's first row (G = slab_group(D))
__host__ __device__ inline int slab_row_off(int m, int G, int CR) {
    return (((m >> SLAB_QB_LOG) * G) * SLAB_QB + (m & (SLAB_QB - 1))) * CR * 4;
}

// The Laplace walk, in two parts. Per feature d of p it writes slab[(p*D + d)*M + m][c] = sum_n exp(-|k_n - q_m|)
// v[p,n,c] (row stride slab_stride(C)) and the v == 1 sums into uslab. laplace_prepare is the key side (range summaries
// and scan into ra.ta / ra.tb) and needs only the sorted keys; laplace_emit is the walk, which also needs the sorted
// queries and their range boundaries (query_bounds into ra.qb). A key of value FLT_MAX adds exactly 0 to the sums
// of every query below FLT_MAX (its decay factor e^{-(FLT_MAX - q)} is 0): that is how masked keys drop out
// (mask_keys).
int laplace_prepare(const float* ks, const uint32_t* kp, const float* v, int P, int D, int N, int C, RangeArrays ra,
                    hipStream_t st);
int laplace_emit(const float* ks, const uint32_t* kp, const float* qs, const uint32_t* qp, const float* v,
                 float* slab, float* uslab, int P, int D, int N, int M, int C, RangeArrays ra, hipStream_t st);

// Order of the per-feature v == 1 terms (uslab) the walks write: sorted-query order (coalesced stores, put in query
// order through LDS before the reduce) when a segment's M terms fit one workgroup's LDS, else query order (one
// 4-byte store per query; a segment's waves run on one XCD, so its lines fill in that L2).
constexpr int U_LDS_CAP = 16384;
__host__ __device__ inline bool u_query_order(int M) { return M > U_LDS_CAP; }

// D-reduction of the slabs: out[p,m,c] = sum_d slab rows of (p, d, m); out_u[p,m] = sum_d of the v == 1 terms of
// (p, d, m). uslab as the walks write it (see u_query_order); for sorted order it is put in query order in uq (P*D*M
// floats of scratch) by the sort's permutation qperm first; qperm == null: uslab is already in query order (from
// order_u_terms). out_u / uslab / qperm / uq may be null (no out_u).
int reduce_slabs(const float* slab, const float* uslab, const uint32_t* qperm, float* uq, float* out, float* out_u,
                 int P, int D, int M, int C, hipStream_t st);
// The v == 1 terms in query order: uslab itself when the walks wrote them so, else uq after the transpose through
// LDS by the permutation qperm (launched on st).
const float* order_u_terms(const float* uslab, const uint32_t* qperm, float* uq, int P, int D, int M, hipStream_t st);
// the same for nsets (<= 3) sets of terms sorted alike, in one launch
void order_u_terms_sets(const float* const* uslab, const uint32_t* qperm, float* const* uq, int nsets, int P, int D,
                        int M, hipStream_t st);

// Emission modes of the abs-family walk (bit set).
enum AbsMode : int {
    ABS_ROW   = 1,    // slab[(p,d), m, :] = sum_n |k_n - q_m| w_n            (row store)
    ABS_ONES  = 2,    // uslab[(p,d), i]   = sum_n |k_n - q_(i)|, sorted order (store)
    ABS_DOT   = 4,    // out_dot[s, m]     = sign * sum_n s(q_m - k_n) <w_n, g_m>, s(0) = -1   (store)
    ABS_DOTX1 = 8,    //   ... + uq[p, m] * (2 rank - Ns)
    ABS_DOTX2 = 16,   //   ... + sum_n s(q_m - k_n) u_n
    ABS_RANK  = 32,   // out_rank[s, m]    = #{n : k_n < q_m}                 (store)
    ABS_KEEP  = 64,   // with ABS_ROW | ABS_ONES: keys masked by a.keep weigh 0 (a.keep non-null exactly with this bit)
};

struct AbsWalkArgs {
    // stream: sorted values + perm of the "keys" the prefix runs over, and their weight rows
    const float* ks; const uint32_t* kp; int Ns;
    const float* w;          // (P, Ns, C) weight rows, gathered by kp
    const float* u;          // (P, Ns) scalar weights (ABS_DOTX2) or null
    const uint8_t* keep;     // (P, Ns) key mask, nonzero = kept, or null (all kept); masked keys weigh 0 in every sum
    // queries
    const float* qs; const uint32_t* qp; int Mq;
    const float* g;          // (P, Mq, C) rows dotted at emission (ABS_DOT) or null
    const float* uq;         // (P, Mq) (ABS_DOTX1) or null
    float* slab;             // (P*D, Mq, CR) per-feature contribution rows (ABS_ROW)
    float* uslab;            // (P*D, Mq) per-feature v == 1 contributions in sorted order (ABS_ONES)
    int CR;                  // slab row stride
    float* out_dot;          // (P, D, Mq)
    int32_t* out_rank;       // (P, D, Mq)
    float sign;
    int P, D, C;
    float qshift;            // added to every query value (0: the queries as given); the sorted order is unchanged
    // More query sets over the same sorted queries (nsets = 3, ROW | ONES walks only): set i > 0 adds set_shift[i]
    // to the queries, has its own range bounds set_qb[i] (query_bounds for that shift) and writes set_slab[i] /
    // set_uslab[i]. Set 0 is qshift / the walk's qb / slab / uslab. nsets = 0 or 1: one set.
    int nsets;
    float set_shift[3];
    const int* set_qb[3];
    float* set_slab[3];
    float* set_uslab[3];
};
// query boundaries + sums + scan + walk
int abs_walk(const AbsWalkArgs& a, int mode, RangeArrays ra, hipStream_t st);
// the parts of abs_walk: the key side (range summaries and scan, from the sorted keys alone); the query boundaries
// (range_bounds, for a.qshift, from the sorted keys and queries); then the walk, which may run several times over one
// prepared ra with different qshift / ra.qb
int abs_prepare(const AbsWalkArgs& a, int mode, RangeArrays ra, hipStream_t st);
int abs_emit(const AbsWalkArgs& a, int mode, RangeArrays ra, hipStream_t st);
// query boundaries of every key range for queries shifted by qshift (what abs_prepare writes to ra.qb for a.qshift)
int range_bounds(const AbsWalkArgs& a, int* qb, hipStream_t st);
// qb[s, g] = #{i : qs[s, i] + qshift <= largest key of range g} over the sorted keys ks (S segments of Ns) and sorted
// queries qs (S segments of Mq), ranges of range_keys(C) keys
int query_bounds(const float* ks, const float* qs, int* qb, float qshift, int S, int Ns, int Mq, int C,
                 hipStream_t st);
// query_bounds for nsets <= 3 shifts in one launch: qb[i] for shift[i]
int query_bounds_sets(const float* ks, const float* qs, int* const qb[], const float shift[], int nsets, int S,
                      int Ns, int Mq, int C, hipStream_t st);
// The queries of every segment (shifted by qshift) grouped by key chunk, a quarter of a key range: qs / qp (S segments
// of Mq) get the values and original indices of chunk 0's queries, then chunk 1's, ... (a query's chunk holds the first
// key >= q + qshift), so each range's queries are contiguous and come chunk by chunk; the order inside a chunk is not
// fixed. qb as query_bounds writes it. The forward walks accept these grouped queries as well as sorted ones. Only for
// segments that group_fits (one workgroup stages them in LDS); longer ones are sorted.
int group_queries(const float* ks, const float* q, float* qs, uint32_t* qp, int* qb, float qshift, int S, int Ns,
                  int Mq, int C, hipStream_t st);
bool group_fits(int Ns, int Mq, int C);
int range_count(int Ns, int C);          // key ranges per segment

// The range scans of the walks over caller-given summary rows (C <= 64; aggs: scan_agg_bytes for G > 256 ranges)
int abs_scan_rows(const float* sa, const float* sb, float* ta, float* tb, float* aggs, int S, int C, int G,
                  hipStream_t st);
// two independent linked sums X <- a_g + link_g X (link in slot C + 1) over range rows, totals in row G
int linked_scan_pair(const float* sa, const float* sb, float* ta, float* tb, float* aggs, int S, int C, int G,
                     hipStream_t st);
size_t scan_agg_bytes(int S, int Ns, int C);

// ---- mbw.hip: the abs backward as one walk over the merged keys and queries (C <= 64, C % 4 == 0)
// merged values mv and tags mt (index, | 0x80000000 for a query; queries first among equal values) of the sorted
// queries (qs, qp) and keys (ks, kp) of S segments (D per p), and the range summaries of the merged sequence (G =
// ranges of 64 elements) for the scans: sa_q, sb_q (abs scan), sa_k, sa_e (linked sums)
int merge_sums_launch(const float* qs, const uint32_t* qp, const float* ks, const uint32_t* kp, const float* v,
                      const float* gw, const float* gu, float* mv, uint32_t* mt, float* sa_q, float* sb_q,
                      float* sa_k, float* sa_e, int S, int D, int N, int M, int C, int G, hipStream_t st);
// the walk: grad_q, grad_k, and the grad_v rows into the slab (one row per (p, d, key))
int mbw_walk_launch(const float* mv, const uint32_t* mt, const float* v, const float* gw, const float* gu,
                    const float* ta_q, const float* tb_q, const float* ta_k, const float* ta_e, float* slab,
                    float* grad_q, float* grad_k, int S, int D, int N, int M, int C, int G, hipStream_t st);

// Dense evaluation for short segments (direct.hip): kind 0 abs, 1 Laplace; out_u may be null
int direct_fwd(int kind, const float* q, const float* k, const float* v, float* out_w, float* out_u,
               int P, int D, int N, int M, int C, hipStream_t st);
// The dense abs forward keeping its kernel matrix A[p][m][n] = sum_d |q[p,d,m] - k[p,d,n]| (P*M rows of pad4(N) floats)
// in a_out, where the tiled kernel runs (direct_fwd_tiled); and out[p,n,:] = sum_m A[p,m,n] g[p,m,:] from such an A (the
// dense grad_v, bit-identical to forming A again)
bool direct_fwd_tiled(int D, int N, int M, int C);
int direct_fwd_keep_a(const float* q, const float* k, const float* v, float* out_w, float* out_u, float* a_out,
                      int P, int D, int N, int M, int C, hipStream_t st);
int dense_at_g(const float* A, const float* g, float* out, int P, int N, int M, int C, hipStream_t st);
// out[d, i] = scale * sum_j s(a[d,i] - b[d,j]) (<x[i], y[j]> + g_u[own ? i : j]), s(0) = tie; a (P, D, I), b (P, D, J),
// x (P, I, C), y (P, J, C), g_u nullable
int direct_sign(bool gu_own, const float* a, const float* b, const float* x, const float* y, const float* gu,
                float* out, float tie, float scale, int P, int D, int I, int J, int C, hipStream_t st);

// Fused attention-layer epilogues (layers.hip)
enum LayerKind { LAYER_ADD_LAPLACE = 0, LAYER_ADD_RIESZ = 1, LAYER_ADD_BUMP = 2 };
size_t riesz_prefix_bytes(int P, int N, int C);
// add_riesz per-p constants over the kept keys (keep (P, N) bytes, nonzero = kept, or null): vsum[p][c] = sum_n v,
// akv[p][c] = sum_n |k_n|_1 v_n, sak[p] = sum_n |k_n|_1, npad[p] = N - #kept (pre must hold riesz_prefix_bytes)
int riesz_prefix(const float* k, const float* v, const uint8_t* keep, void* pre, int P, int D, int N, int C,
                 hipStream_t st);
// out[p][d][n] = keep[p][n] ? k[p][d][n] : FLT_MAX: keys whose every Laplace term is exactly 0 and which sort last
int mask_keys(const float* k, const uint8_t* keep, float* out, int P, int D, int N, hipStream_t st);
// Sorted keys ks (P*D segments of N, permutation kp) of a masked abs walk, in place: every masked key (keep (P, N),
// indexed by the original position) takes the value of the last kept key before it; masked keys before the first kept
// key keep theirs. The abs walk's distances, its segment totals included, then run between kept keys only.
int fill_masked_keys(float* ks, const uint32_t* kp, const uint8_t* keep, int P, int D, int N, hipStream_t st);
// out[p][m][:] from the op outputs: w0/u0 (and, for add_bump, w+/u+ and w-/u- of q + 1 and q - 1). masked: the op
// outputs are sums over the kept keys and n_pad is ignored (add_riesz takes its n_pad from pre); else n_pad (P) is
// the reference's padded-key count (null: none). qt: (P, M) scratch for the per-query d-reductions
int layer_epilogue(int kind, bool masked, const float* q, const float* n_pad, const float* w0, const float* u0,
                   const float* wp, const float* up, const float* wm, const float* um, const void* pre, float* qt,
                   float* out, int P, int D, int N, int M, int C, hipStream_t st);
// The add_laplace / add_riesz epilogue folded into the slab reduce: the reduce writes out = num / max(den, clamp)
// instead of w and u (no 2 x 50 MB round trip, no separate pass). Applies when reduce_folds_epilogue(M, C); q gives
// the query terms (written to qt first), pre the add_riesz constants; masked as for layer_epilogue.
struct ReduceEpilogue {
    const float* qt; const float* n_pad; const float* vsum; const float* akv; const float* sak; float* out;
};
bool reduce_folds_epilogue(int M, int C);
int layer_epilogue_params(int kind, bool masked, const float* q, const float* n_pad, const void* pre, float* qt,
                          float* out, int P, int D, int M, int C, ReduceEpilogue* ep, hipStream_t st);
int reduce_slabs_layer(int kind, bool masked, const ReduceEpilogue& ep, const float* slab, const float* uslab,
                       const uint32_t* qperm, float* uq, int P, int D, int M, int C, hipStream_t st);
// add_bump in one reduce: the slabs and query-order v == 1 terms of the abs sums at q, q + 1, q - 1 (indices 0, 1, 2),
// with the bump epilogue folded in (writes ep.out); requires reduce_folds_epilogue(M, C)
int reduce_slabs_bump(bool masked, const ReduceEpilogue& ep, const float* const slab[3], const float* const uq[3],
                      int P, int D, int M, int C, hipStream_t st);

// ---- capi.hip helpers for noalloc.hip
// check_dims of the C ABI (clears the thread's error first); the workspace of a Laplace forward over pc p at a time;
// set the thread's error message and return code
int validate_dims(int P, int D, int N, int M, int C);
size_t laplace_fwd_chunk_ws(int pc, int D, int N, int M, int C);
int report_error(int code, const char* msg);

}  // namespace qlka
