// Stages 2-4 of the hot path: merge rank, prefix/suffix scans and emission, for both operators.
//
// Per segment s = (p, d) the keys are sorted (sort.hip) and cut into key ranges of RK keys; one wave owns one range
// and the queries whose merge rank r = #{keys < q} falls in it (the last range also owns r = N). Four kernels:
//
//   query_bounds   the query bounds of every range from the sorted queries (pieces of them staged in LDS, one
//                  binary search per range there), or group_queries: the queries grouped by key chunk instead.
//   *_range_sums   one wave per range: the range's summary, computed directly (every term has its own weight,
//                  no recurrence).
//   *_range_scan   one workgroup per segment (or per 256 ranges of a longer one, in two launches): turns the
//                  summaries into each range's entry state (exclusive prefix over the ranges to the left) and, for
//                  the Laplace sum, exit state (exclusive suffix to the right).
//   *_range_walk   one wave per range: gathers the range's RK value rows into registers (lane = channel), runs the
//                  recurrences key by key in 4 chunks, stages each chunk's state rows in wave-private LDS and emits
//                  the owned queries ranked in the chunk from there, 64 / LQ query rows per 16-byte-per-lane store.
//
// Laplace (Weighted_Laplace_Sum/csrc/laplace_kernels.cu:5-29 states the same math): with sorted keys k_0..k_{N-1}
//   L_j = e^{-(k_j - k_{j-1})} L_{j-1} + v_j,   R_j = v_j + e^{-(k_{j+1} - k_j)} R_{j+1},
//   query q of rank r gets  e^{-(q - k_{r-1})} L_{r-1} + e^{-(k_r - q)} R_r.
// Every exponent argument is <= 0 and every decay factor is <= 1, so nothing overflows and nothing cancels. The walk
// keeps R only at its chunk boundaries (computed backwards from the range's exit state) and rebuilds each chunk's R
// rows from there, so v is gathered twice per key and feature (sums + walk) instead of the reference's three times.
//
// Abs family (Weighted_Abs_Sum/csrc/abs_kernels.cu:9-19 and sgn_kernels.cu:8-15 state the same identities): the
// stream state after the keys below q is PW = sum w_n and B = sum (k_prev - k_n) w_n, all distances measured from
// the last absorbed key k_prev, so
//   sum_{k_n < q} (q - k_n) w_n = (q - k_prev) PW + B,
//   sum_n |k_n - q| w_n        = 2 [(q - k_prev) PW + B] - Btot - (q - k_max) Wtot,
//   sum_n s(q - k_n) <w_n, g>  = <g, 2 PW - Wtot>          (s(0) = -1: a tie counts as a key above q).
// Distances from k_prev and k_max (instead of raw k*v sums) keep the walk translation invariant. Only a prefix is
// needed, so the abs walks gather each row once in the walk plus once in the sums.
//
// Row emissions go to a per-feature slab (one row per query and feature, reduce.hip sums the D features of a p in a
// fixed order); scalar emissions (v == 1 sums, dots, ranks) have exactly one writer each and are plain stores.
#include "qlka_common.h"
#include "qlka_internal.h"
#include "group_device.h"

namespace qlka {

constexpr int WPB = 4;             // waves per workgroup for the range kernels


static inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

size_t scan_agg_bytes(int S, int Ns, int C);

size_t range_arrays_bytes(int S, int Ns, int C) {
    const int RK = range_keys(C);
    const size_t G = (size_t)((Ns + RK - 1) / RK);
    const size_t rows = (size_t)S * (G + 1);
    return 4 * align256(rows * range_stride(C) * sizeof(float)) + align256((size_t)S * G * sizeof(int)) +
           align256(scan_agg_bytes(S, Ns, C));
}

RangeArrays carve_range_arrays(void* base, int S, int Ns, int C) {
    const int RK = range_keys(C);
    const size_t G = (size_t)((Ns + RK - 1) / RK);
    const size_t rows = (size_t)S * (G + 1);
    char* b = (char*)base;
    RangeArrays r;
    r.sa = (float*)b; b += align256(rows * range_stride(C) * sizeof(float));
    r.sb = (float*)b; b += align256(rows * range_stride(C) * sizeof(float));
    r.ta = (float*)b; b += align256(rows * range_stride(C) * sizeof(float));
    r.tb = (float*)b; b += align256(rows * range_stride(C) * sizeof(float));
    r.qb = (int*)b; b += align256((size_t)S * G * sizeof(int));
    r.aggs = scan_agg_bytes(S, Ns, C) ? (float*)b : nullptr;
    return r;
}

__global__ __launch_bounds__(256)
void fill_zero_kernel(float4* __restrict__ p4, float* __restrict__ p, const size_t n4, const size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t j = i; j < n4; j += stride) p4[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (size_t j = n4 * 4 + i; j < n; j += stride) p[j] = 0.f;
}

int fill_zero(float* p, size_t n, hipStream_t st) {
    if (n == 0) return 0;
    const bool al = (((uintptr_t)p) & 15) == 0;
    const size_t n4 = al ? n / 4 : 0;
    const size_t work = n4 ? n4 : n;
    const unsigned blocks = (unsigned)std::min<size_t>((work + 255) / 256, 8192);
    StageTimer t("fill_zero", st);
    hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0, st, (float4*)p, p, n4, n);
    return (int)hipGetLastError();
}

// Rank of query value q among the first nk (<= RK) keys of the range held one per lane in kl (ascending):
// #{t < nk : k_t < q}, in [0, nk]. Branch-free binary search over lane shuffles, valid for any per-lane q.
template <int RK>
__device__ __forceinline__ int range_rank(const float kl, const int nk, const float q) {
    int pos = 0;
#pragma unroll
    for (int step = RK / 2; step >= 1; step >>= 1) {
        const float kv = __shfl(kl, pos + step - 1, WAVE);
        if (pos + step <= nk && kv < q) pos += step;
    }
    const float kv = __shfl(kl, min(pos, RK - 1), WAVE);
    if (pos < nk && kv < q) ++pos;
    return pos;
}

// Weight of a key in the sums: 0 for the pad lanes of a partial range and for keys masked out by keep (P, Ns bytes,
// nonzero = kept, indexed by the key's original position n), else 1. A masked key keeps its value and its place in the
// sorted order; weighing 0, it adds nothing to any sum, so no correction for padded keys is needed afterwards.
__device__ __forceinline__ float key_weight(const uint8_t* keep, const int p, const int Ns, const uint32_t n,
                                            const bool real) {
    if (!real) return 0.f;
    return (keep && keep[(size_t)p * Ns + n] == 0) ? 0.f : 1.f;
}

// Zero the gathered rows of masked keys (x[t] holds key t of the range; kw is lane t's key weight). A select, not a
// product, so a masked key's row is dropped whatever it holds.
template <int NV, int RK>
__device__ __forceinline__ void mask_rows(float (&x)[RK][NV], const float kw) {
#pragma unroll
    for (int t = 0; t < RK; ++t) {
        const bool kept = bcast(kw, t) != 0.f;
#pragma unroll
        for (int j = 0; j < NV; ++j) x[t][j] = kept ? x[t][j] : 0.f;
    }
}

// The two weighted row sums of a 64-key range, oa = sum_t a_t x_t and ob = sum_t b_t x_t, x_t the v row of key t
// (row index pl, weights a, b: lane t's values), for C <= 64 with C % 4 == 0; lane c returns channel c. 16 lanes
// cover a row with one 16-byte load each and lane group r takes keys r, r + 4, ..., so the 64 rows take 16 load
// instructions (64 with a lane per channel). Each lane stages its key's row offset and weights in wave-private LDS
// and reads those of the keys it loads 16 bytes at a time (one LDS read per row instead of three lane shuffles: range
// sums 0.069 -> 0.064 ms at the headline shape); the groups' partial sums meet across lanes at the end.
__device__ __forceinline__ void range_row_sums_v4(const rsrc_t vr, const int C, const uint32_t pl, const float a,
                                                  const float b, float& oa, float& ob) {
    const int l = lane_id(), grp = l >> 4, sub = l & 15;
    const int coff = min(4 * sub, C - 4) * 4;
    __shared__ f4_t stage_all[WPB][64];
    f4_t* stage = stage_all[wave_in_block()];
    stage[l] = f4_t{__uint_as_float(pl * (uint32_t)C * 4u), a, b, 0.f};
    __builtin_amdgcn_wave_barrier();
    f4_t sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int t = 4 * i + grp;
        const f4_t w = stage[t];
        const f4_t x = buf_load4(vr, (int)__float_as_uint(w[0]) + coff, 0);
        sa += w[1] * x;
        sb += w[2] * x;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        sa[e] += __shfl_xor(sa[e], 16, WAVE);
        sb[e] += __shfl_xor(sb[e], 16, WAVE);
        sa[e] += __shfl_xor(sa[e], 32, WAVE);
        sb[e] += __shfl_xor(sb[e], 32, WAVE);
    }
    // lane = channel: channel c sits in element c % 4 of lane c / 4
    const int src = min(l, C - 1) >> 2, e = l & 3;
    float ya[4], yb[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) { ya[k] = __shfl(sa[k], src, WAVE); yb[k] = __shfl(sb[k], src, WAVE); }
    oa = e == 0 ? ya[0] : e == 1 ? ya[1] : e == 2 ? ya[2] : ya[3];
    ob = e == 0 ? yb[0] : e == 1 ? yb[1] : e == 2 ? yb[2] : yb[3];
}

// =================================================================================================================
// Laplace
// =================================================================================================================

// Range summary: Lt = sum_t e^{-(k_last - k_t)} v_t (the L state at the range's last key, starting from zero),
// Rt = sum_t e^{-(k_t - k_first)} v_t (the R state at its first key, zero beyond the range). Slot C: the v == 1 sums.
template <int NV, int RK>
__global__ __launch_bounds__(WPB * WAVE)
void lap_range_sums(const float* __restrict__ ks, const uint32_t* __restrict__ kp,
                    const float* __restrict__ v, float* __restrict__ ta, float* __restrict__ tb, const int S,
                    const int D, const int N, const int C, const int G)
{
    const long wv = (long)xcd_slice_block(blockIdx.x, gridDim.x) * WPB + wave_in_block();
    if (wv >= (long)S * G) return;
    const int s = (int)(wv / G), g = (int)(wv - (long)s * G);
    const int p = s / D, l = lane_id();
    const int base = g * RK, nk = min(RK, N - base);
    const float* kseg = ks + (size_t)s * N;

    const int li = base + min(l, nk - 1);
    const float kl = kseg[li];
    const uint32_t pl = kp[(size_t)s * N + li];
    const float kfirst = kseg[base], klast = kseg[base + nk - 1];
    const float kw = (l < nk) ? 1.f : 0.f;                   // pad lanes of a partial range weigh 0
    const float wl = kw * __expf(-(klast - kl));
    const float wr = kw * __expf(-(kl - kfirst));

    const rsrc_t vr = make_rsrc(v + (size_t)p * N * C, (uint32_t)((size_t)N * C * 4));
    float sl[NV], sr[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) { sl[j] = 0.f; sr[j] = 0.f; }
    if (NV == 1 && RK == 64 && C % 4 == 0) {
        range_row_sums_v4(vr, C, pl, wl, wr, sl[0], sr[0]);
    } else {
#pragma unroll
        for (int t = 0; t < RK; ++t) {
            const uint32_t row = bcast(pl, t);
            const float a = bcast(wl, t), b = bcast(wr, t);
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const int c = l + WAVE * j;
                const float xr = buf_load(vr, min(c, C - 1) * 4, (int)(row * C * 4));   // unconditional gather
                const float x = (c < C) ? xr : 0.f;
                sl[j] += a * x;
                sr[j] += b * x;
            }
        }
    }
    const float l1 = wave_sum(wl), r1 = wave_sum(wr);

    const int CS = range_stride(C);
    float* ra = ta + ((size_t)s * (G + 1) + g) * CS;
    float* rb = tb + ((size_t)s * (G + 1) + g) * CS;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = l + WAVE * j;
        if (c < C) { ra[c] = sl[j]; rb[c] = sr[j]; }
    }
    if (l == 0) {
        ra[C] = l1;
        rb[C] = r1;
        // slot C+1: the scan's decays into this range from the one before (L) and after (R)
        ra[C + 1] = (g > 0) ? __expf(-(klast - kseg[base - 1])) : 0.f;
        rb[C + 1] = (g < G - 1) ? __expf(-(kseg[base + RK] - kfirst)) : 0.f;
    }

}

// The range scans run one workgroup of SCAN_W waves per segment. Each wave owns a contiguous piece of the segment's
// ranges: pass 1 runs its piece from a zero state to the piece's aggregate (an affine map of the incoming state), the
// waves exchange aggregates through LDS and compose those of the pieces before (or after) their own, and pass 2 runs
// the piece again from the true incoming state, writing every range's entry (exit) state. Slot C+1 of every summary
// row holds the range's link to its neighbour (a decay factor or a key gap, written by the sums kernel), so the scan
// loop is loads and FMAs only.
constexpr int SCAN_W = 16;
constexpr int SCAN_BLOCK = 256;     // ranges of a scan workgroup
template <int NV>
__device__ __forceinline__ void store_scan_row(float* __restrict__ row, const int C, const float (&r)[NV + 1]) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = lane_id() + WAVE * j;
        if (c < C) row[c] = r[j];
    }
    if (lane_id() == 0) row[C] = r[NV];
}

// A wave's piece of at most SCAN_PIECE range summaries, loaded once with all its loads in flight together and kept in
// registers for both passes of the scan (instead of reloading it per pass and direction in batches): the lane's
// channels of row i in v[i], and the row's two scalars (slot C and the link to the neighbour) in lane i of u / link.
// Rows past the piece repeat its last row and are never used.
template <int NV>
struct ScanPiece {
    float v[SCAN_BLOCK / SCAN_W][NV];
    float u, link;
    __device__ __forceinline__ void load(const float* __restrict__ rows, const int CS, const int C, const int glo,
                                         const int ghi) {
        if (ghi <= glo) return;                           // empty piece (uniform)
        const int l = lane_id();
#pragma unroll
        for (int i = 0; i < SCAN_BLOCK / SCAN_W; ++i) {
            const float* row = rows + (size_t)min(glo + i, ghi - 1) * CS;
#pragma unroll
            for (int j = 0; j < NV; ++j) v[i][j] = row[min(l + WAVE * j, C - 1)];   // lanes >= C are never stored
        }
        const float* row = rows + (size_t)min(glo + l, ghi - 1) * CS;
        u = row[C];
        link = row[C + 1];
    }
    // row i (a constant after unrolling): its NV lane values, slot C, and the link
    __device__ __forceinline__ void get(const int i, float (&r)[NV + 1], float& lk) const {
#pragma unroll
        for (int j = 0; j < NV; ++j) r[j] = v[i][j];
        r[NV] = bcast(u, i);
        lk = bcast(link, i);
    }
};

// Long segments are scanned by several workgroups of SCAN_BLOCK ranges each, in two launches: phase 1 runs every wave's
// piece from a zero state and writes the wave aggregates and, composed in order, the workgroup's aggregate; phase 2
// composes the aggregates of the workgroups before (and, for a suffix, after) its own into its incoming state, then
// the waves of its own before (after) theirs, and reruns each piece from the true state, writing the range states.
// Segments of up to SCAN_BLOCK ranges (N <= 16384 at 64-key ranges) run both phases in one workgroup (phase 0).
__host__ __device__ inline int scan_blocks(int G) { return (G + SCAN_BLOCK - 1) / SCAN_BLOCK; }
// floats of one workgroup's aggregate record: SCAN_W wave aggregates + the workgroup aggregate, each two (state,
// link) pairs of NV + 1 lane vectors and one lane vector
template <int NV> __host__ __device__ constexpr int scan_rec_floats() { return (SCAN_W + 1) * 2 * (NV + 2) * WAVE; }
size_t scan_agg_bytes(int S, int Ns, int C) {
    const int G = (Ns + range_keys(C) - 1) / range_keys(C);
    const int nb = scan_blocks(G);
    if (nb <= 1) return 0;
    return (size_t)S * nb * (C <= WAVE ? scan_rec_floats<1>() : scan_rec_floats<2>()) * sizeof(float);
}

// one aggregate (two lane-vector sets of NV + 1 values plus one lane vector) in a record: slot i of SCAN_W + 1
template <int NV>
__device__ __forceinline__ float* agg_slot(float* rec, int i, int part) {
    return rec + ((size_t)i * 2 + part) * (NV + 2) * WAVE;
}

// Laplace: entry L state of every range (relative to the last key before the range) and exit R state (relative to
// the first key after it). Forward: L <- a_g + e^{-(klast_g - klast_{g-1})} L; backward: R <- b_g +
// e^{-(kfirst_{g+1} - kfirst_g)} R. A piece composes to  out = local + (product of its decays) in.
// FF: both arrays run the forward recurrence (two independent linked sums, X <- a_g + link_g X, link in the rows' last
// slot), and row G of both outputs takes the segment's final state.
template <int NV, int RK, int PHASE, bool FF = false>
__global__ __launch_bounds__(SCAN_W * WAVE)
void lap_range_scan(const float* __restrict__ sa, const float* __restrict__ sb, float* __restrict__ ta,
                    float* __restrict__ tb, float* __restrict__ aggs, const int S, const int C, const int G)
{
    __shared__ float agg[2][SCAN_W][NV + 1][WAVE];
    __shared__ float span[2][SCAN_W];
    const int nb = PHASE == 0 ? 1 : scan_blocks(G);
    const int s = blockIdx.x / nb, blk = blockIdx.x - s * nb;
    const int w = wave_in_block(), l = lane_id();
    const int CS = range_stride(C);
    const float* SA = sa + (size_t)s * (G + 1) * CS;
    const float* SB = sb + (size_t)s * (G + 1) * CS;
    float* A = ta + (size_t)s * (G + 1) * CS;
    float* B = tb + (size_t)s * (G + 1) * CS;
    const int b0 = PHASE == 0 ? 0 : blk * SCAN_BLOCK, b1 = PHASE == 0 ? G : min(G, b0 + SCAN_BLOCK);
    const int per = (b1 - b0 + SCAN_W - 1) / SCAN_W;
    const int glo = min(b1, b0 + w * per), ghi = min(b1, b0 + w * per + per);
    float* seg_aggs = PHASE == 0 ? nullptr : aggs + (size_t)s * nb * scan_rec_floats<NV>();

    ScanPiece<NV> piece_a, piece_b;
    piece_a.load(SA, CS, C, glo, ghi);
    piece_b.load(SB, CS, C, glo, ghi);
    // forward piece walk from state cur; writes entry states when OUT; returns the product of the piece's decays
    auto fwd = [&](float (&cur)[NV + 1], const bool out) {
        float prod = 1.f;
#pragma unroll
        for (int i = 0; i < SCAN_BLOCK / SCAN_W; ++i) {
            const int g = glo + i;
            if (g >= ghi) break;
            float a[NV + 1], dec;
            piece_a.get(i, a, dec);
            if (out) store_scan_row<NV>(A + (size_t)g * CS, C, cur);
#pragma unroll
            for (int j = 0; j <= NV; ++j) cur[j] = a[j] + dec * cur[j];
            prod *= dec;
        }
        return prod;
    };
    // backward (FF: forward) piece walk from state cur; writes exit (entry) states when OUT; returns the product of
    // the piece's decays
    auto bwd = [&](float (&cur)[NV + 1], const bool out) {
        float prod = 1.f;
#pragma unroll
        for (int ii = 0; ii < SCAN_BLOCK / SCAN_W; ++ii) {
            const int i = FF ? ii : SCAN_BLOCK / SCAN_W - 1 - ii;
            const int g = glo + i;
            if (g >= ghi) continue;
            float b_[NV + 1], dec;
            piece_b.get(i, b_, dec);
            if (out) store_scan_row<NV>(B + (size_t)g * CS, C, cur);
#pragma unroll
            for (int j = 0; j <= NV; ++j) cur[j] = b_[j] + dec * cur[j];
            prod *= dec;
        }
        return prod;
    };

    float cf[NV + 1], cb[NV + 1], pf = 1.f, pb = 1.f;
    if constexpr (PHASE <= 1) {
        // pass 1: every piece from a zero state; empty pieces have product 1 and aggregate 0
#pragma unroll
        for (int j = 0; j <= NV; ++j) { cf[j] = 0.f; cb[j] = 0.f; }
        pf = fwd(cf, false);
        pb = bwd(cb, false);
#pragma unroll
        for (int j = 0; j <= NV; ++j) { agg[0][w][j][l] = cf[j]; agg[1][w][j][l] = cb[j]; }
        if (l == 0) { span[0][w] = pf; span[1][w] = pb; }
    }
    if constexpr (PHASE == 1) {
        // the wave aggregates, and wave 0 (forward) / wave 1 (backward) composes the workgroup's
        float* rec = seg_aggs + (size_t)blk * scan_rec_floats<NV>();
        for (int part = 0; part < 2; ++part) {
            float* ws_ = agg_slot<NV>(rec, w, part);
#pragma unroll
            for (int j = 0; j <= NV; ++j) ws_[j * WAVE + l] = part ? cb[j] : cf[j];
            ws_[(NV + 1) * WAVE + l] = part ? pb : pf;
        }
        __syncthreads();
        if (w < 2) {
            const int part = w;
            float c[NV + 1], d = 1.f;
#pragma unroll
            for (int j = 0; j <= NV; ++j) c[j] = 0.f;
            for (int k = 0; k < SCAN_W; ++k) {
                const int ww = (part == 0 || FF) ? k : SCAN_W - 1 - k;   // forward: left to right; backward: right to left
                const float dd = span[part][ww];
#pragma unroll
                for (int j = 0; j <= NV; ++j) c[j] = agg[part][ww][j][l] + dd * c[j];
                d *= dd;
            }
            float* bs = agg_slot<NV>(rec, SCAN_W, part);
#pragma unroll
            for (int j = 0; j <= NV; ++j) bs[j * WAVE + l] = c[j];
            bs[(NV + 1) * WAVE + l] = d;
        }
        return;
    }
    if constexpr (PHASE == 2) {
        // this workgroup's wave aggregates, from phase 1
        const float* rec = seg_aggs + (size_t)blk * scan_rec_floats<NV>();
        for (int part = 0; part < 2; ++part) {
            const float* ws_ = agg_slot<NV>(const_cast<float*>(rec), w, part);
#pragma unroll
            for (int j = 0; j <= NV; ++j) agg[part][w][j][l] = ws_[j * WAVE + l];
            if (l == 0) span[part][w] = ws_[(NV + 1) * WAVE];
        }
    }
    __syncthreads();

    // incoming states: the workgroups before (forward) / after (backward) this one, then its waves before / after
#pragma unroll
    for (int j = 0; j <= NV; ++j) { cf[j] = 0.f; cb[j] = 0.f; }
    if constexpr (PHASE == 2) {
        for (int bb = 0; bb < blk; ++bb) {
            const float* bs = agg_slot<NV>(seg_aggs + (size_t)bb * scan_rec_floats<NV>(), SCAN_W, 0);
            const float d = bs[(NV + 1) * WAVE + l];
#pragma unroll
            for (int j = 0; j <= NV; ++j) cf[j] = bs[j * WAVE + l] + d * cf[j];
        }
        for (int k = 0; k < (FF ? blk : nb - 1 - blk); ++k) {
            const int bb = FF ? k : nb - 1 - k;            // forward: the workgroups before; backward: those after
            const float* bs = agg_slot<NV>(seg_aggs + (size_t)bb * scan_rec_floats<NV>(), SCAN_W, 1);
            const float d = bs[(NV + 1) * WAVE + l];
#pragma unroll
            for (int j = 0; j <= NV; ++j) cb[j] = bs[j * WAVE + l] + d * cb[j];
        }
    }
    for (int ww = 0; ww < w; ++ww) {
        const float d = span[0][ww];
#pragma unroll
        for (int j = 0; j <= NV; ++j) cf[j] = agg[0][ww][j][l] + d * cf[j];
    }
    for (int k = 0; k < (FF ? w : SCAN_W - 1 - w); ++k) {
        const int ww = FF ? k : SCAN_W - 1 - k;
        const float d = span[1][ww];
#pragma unroll
        for (int j = 0; j <= NV; ++j) cb[j] = agg[1][ww][j][l] + d * cb[j];
    }
    fwd(cf, true);
    bwd(cb, true);
    if constexpr (FF) {
        if (ghi == G && glo < G) {                        // the wave whose piece ends the segment writes the totals
            store_scan_row<NV>(A + (size_t)G * CS, C, cf);
            store_scan_row<NV>(B + (size_t)G * CS, C, cb);
        }
    }
}

// Emission through LDS. Each wave owns a private slice of its workgroup's LDS: the state rows of one chunk of
// CH = RK / 4 keys (plus one row for rank RK) and one record per query of the current block of 64 queries. After the
// wave has written a chunk's rows, the queries ranked in the chunk are emitted with LQ lanes per query (LQ * 4 >= CR
// channels, one 16-byte store per lane), i.e. 64 / LQ query rows per store instruction, with no per-query scalar
// broadcasts. LDS operations of one wave complete in program order, so the wave-private slice needs no barrier.
template <int NV, int RK>
struct alignas(16) WalkLds {
    static constexpr int CH = RK / 4;
    static constexpr int RS = WAVE * NV;           // floats per state row (lane = channel, pads included)
    float a[(CH + 1) * RS];
    float b[(CH + 1) * RS];
    f4_t par[WAVE];
};

// Lane layout of the emission: lane = grp * LQ + sub owns channels c4 .. c4 + 3 (c4 = 4 * sub) of query row grp.
struct EmitLanes {
    int sh, qpi, grp, c4;
    bool ok;
    __device__ __forceinline__ explicit EmitLanes(int CR) {
        sh  = (CR <= 32) ? 3 : (CR <= 64) ? 4 : 5;     // LQ = 1 << sh lanes per query row
        qpi = WAVE >> sh;                               // query rows per instruction
        const int l = lane_id();
        grp = l >> sh;
        c4  = (l & ((1 << sh) - 1)) * 4;
        ok  = c4 < CR;
    }
};


// The first two blocks of 64 owned queries of a range (sorted value and query index, lane = query; indices clamped
// into [0, q1 - 1], as the emission loop clamps them), loaded at the start of the range so that their latency
// overlaps the row gathers. settle() makes the wave wait for them there, before its first store: vmcnt counts loads
// and stores in issue order, so a load issued after the emission stores, or first waited for after them, also waits
// until those stores have reached L2. Blocks from the third on (ranges owning more than 128 queries) load in place.
struct QueryBlocks {
    float v0, v1;
    uint32_t m0, m1;
    __device__ __forceinline__ QueryBlocks(const float* qseg, const uint32_t* qpseg, const int q0, const int q1) {
        const int l = lane_id(), hi = max(q1 - 1, 0);
        const int i0 = min(q0 + l, hi), i1 = min(q0 + WAVE + l, hi);
        v0 = qseg[i0]; m0 = qpseg[i0];
        v1 = qseg[i1]; m1 = qpseg[i1];
    }
    __device__ __forceinline__ void settle() { asm volatile("" : "+v"(v0), "+v"(v1), "+v"(m0), "+v"(m1)); }
    // block b of the range (queries from q0 + 64 b); qi = the lane's clamped query index in it
    __device__ __forceinline__ void get(const int b, const float* qseg, const uint32_t* qpseg, const int qi,
                                        float& qv, uint32_t& mq) const {
        if (b == 0) { qv = v0; mq = m0; }
        else if (b == 1) { qv = v1; mq = m1; }
        else { qv = qseg[qi]; mq = qpseg[qi]; }
    }
};

constexpr int RPW = 1;             // consecutive key ranges walked by one wave of a walk kernel
constexpr int STORE_OOB = 0x7fff0000;   // a buffer store offset past every slab descriptor: the store is dropped

template <int NV, int RK>
__global__ __launch_bounds__(WPB * WAVE)
void lap_range_walk(const float* __restrict__ ks, const uint32_t* __restrict__ kp, const float* __restrict__ qs,
                    const uint32_t* __restrict__ qp, const float* __restrict__ v, const float* __restrict__ ta,
                    const float* __restrict__ tb, const int* __restrict__ qb,
                    float* __restrict__ slab, float* __restrict__ uslab,
                    const int S, const int D, const int N, const int M, const int C, const int CR, const int G)
{
    using Lds = WalkLds<NV, RK>;
    constexpr int CH = Lds::CH, RS = Lds::RS;
    __shared__ Lds lds[WPB];
    const int GW = (G + RPW - 1) / RPW;
    const long wv = (long)xcd_slice_block(blockIdx.x, gridDim.x) * WPB + wave_in_block();
    if (wv >= (long)S * GW) return;
    Lds& sm = lds[wave_in_block()];
    const int s = (int)(wv / GW), gw = (int)(wv - (long)s * GW);
    const int p = s / D, l = lane_id();
    const float* kseg = ks + (size_t)s * N;
    const uint32_t* kpseg = kp + (size_t)s * N;
    const float* qseg = qs + (size_t)s * M;
    const uint32_t* qpseg = qp + (size_t)s * M;
    const rsrc_t vr = make_rsrc(v + (size_t)p * N * C, (uint32_t)((size_t)N * C * 4));
    const int SG = slab_group(D);
    const rsrc_t sr_ = make_rsrc(slab + slab_seg_base(p, s - p * D, D, M, CR), slab_seg_bytes(s - p * D, D, M, CR));
    float* useg = uslab + (size_t)s * M;
    const int CS = range_stride(C);
    const EmitLanes el_(CR);

    const int g_end = min(G, gw * RPW + RPW);
    for (int g = gw * RPW; g < g_end; ++g) {
        const int base = g * RK, nk = min(RK, N - base);
        const int li = base + min(l, nk - 1);
        const float kl = kseg[li];
        const bool real = l < nk;
        const bool has_prev = g > 0, has_next = g < G - 1;
        const float kbefore = has_prev ? kseg[base - 1] : 0.f;
        const float kafter  = has_next ? kseg[base + RK] : 0.f;
        const float kw = real ? 1.f : 0.f;

        // value rows of the range, lane = channel (pad keys and pad channels: zero). The row indices are read with
        // scalar loads straight into SGPRs (the buffer offset of each row gather).
        float x[RK][NV];
        if (nk == RK) {
#pragma unroll
            for (int t = 0; t < RK; ++t) {
                const int rowoff = (int)(kpseg[base + t] * C * 4);
#pragma unroll
                for (int j = 0; j < NV; ++j)
                    x[t][j] = buf_load(vr, min(l + WAVE * j, C - 1) * 4, rowoff);   // unconditional gather
            }
        } else {
#pragma unroll
            for (int t = 0; t < RK; ++t) {
                const int rowoff = (int)(kpseg[base + min(t, nk - 1)] * C * 4);
#pragma unroll
                for (int j = 0; j < NV; ++j)
                    x[t][j] = buf_load(vr, min(l + WAVE * j, C - 1) * 4, rowoff);
            }
        }
        // owned queries [q0, q1): their bounds are scalar loads issued after the gathers (an earlier scalar load would
        // hold back the gathers, which wait for the row offsets' scalar loads), then the first two query blocks
        const int q0 = has_prev ? qb[(size_t)s * G + g - 1] : 0;
        const int q1 = has_next ? qb[(size_t)s * G + g] : M;
        QueryBlocks qbk(qseg, qpseg, q0, q1);
        if (nk < RK || C < RS) {                          // partial last range or pad channels (uniform branch)
#pragma unroll
            for (int t = 0; t < RK; ++t)
#pragma unroll
                for (int j = 0; j < NV; ++j)
                    x[t][j] = (t < nk && l + WAVE * j < C) ? x[t][j] : 0.f;
        }

        const float* ra = ta + ((size_t)s * (G + 1) + g) * CS;
        const float* rb = tb + ((size_t)s * (G + 1) + g) * CS;
        float L[NV], Rx[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int c = l + WAVE * j;
            L[j]  = (c < C) ? ra[min(c, C - 1)] : 0.f;
            Rx[j] = (c < C) ? rb[min(c, C - 1)] : 0.f;
        }
        const float L1in = ra[C], R1out = rb[C];

        // lane t: decay into key t from the key before it, and from key t to the key after it. Both go to LDS, from
        // where the key loops read four at a time as a broadcast (no per-key lane-to-scalar moves).
        float kbef = __shfl_up(kl, 1, WAVE);
        if (l == 0) kbef = kbefore;
        const float dprev = (l == 0 && !has_prev) ? 0.f : __expf(-(kl - kbef));
        float kaft = __shfl_down(kl, 1, WAVE);
        if (l == RK - 1) kaft = kafter;
        const float dnext = (l == RK - 1 && !has_next) ? 0.f : __expf(-(kaft - kl));

        // v == 1 channel: L1 after key t and R1 at key t, as lane-t values of two affine scans
        float a1 = (l < RK) ? dprev : 1.f, b1 = kw;
        wave_affine_scan_fwd(a1, b1);
        const float l1 = a1 * L1in + b1;
        float a2 = (l < RK) ? dnext : 1.f, b2 = kw;
        wave_affine_scan_bwd(a2, b2);
        const float r1 = a2 * R1out + b2;

        // R at the chunk boundaries, R_{CH}, R_{2CH}, R_{3CH} (R_{RK} is the exit state Rx): each chunk later rebuilds
        // its own R rows backwards from its right boundary, so R never occupies RK rows of registers.
        float Rc[3][NV];
        {
            float r[NV];
#pragma unroll
            for (int j = 0; j < NV; ++j) r[j] = Rx[j];
#pragma unroll
            for (int t = RK - 1; t >= CH; --t) {
                const float dn = bcast(dnext, t);
#pragma unroll
                for (int j = 0; j < NV; ++j) r[j] = x[t][j] + dn * r[j];
                if (t % CH == 0) {
#pragma unroll
                    for (int j = 0; j < NV; ++j) Rc[t / CH - 1][j] = r[j];
                }
            }
        }

        // Owned queries [q0, q1) of the sorted queries, in blocks of 64. Per block, lane i takes query i: its rank t
        // inside the range, its two decay factors and its v == 1 sum; its record (row offset of rank t in the chunk
        // buffers, slab row offset, eL, eR) goes to LDS. Then the keys are walked in 4 chunks of CH: the chunk's rows
        // L_{t-1} (state before key t) and R_t go to LDS and the queries ranked in the chunk are emitted as
        // eL * L_{t-1} + eR * R_t, several query rows per store instruction.
        qbk.settle();
        for (int qb0 = q0, bi = 0; qb0 < q1; qb0 += WAVE, ++bi) {
            const int nq = min(WAVE, q1 - qb0);
            const bool act = l < nq;
            const int qi = min(qb0 + l, q1 - 1);          // clamped: unconditional loads
            float qv;
            uint32_t mq;
            qbk.get(bi, qseg, qpseg, qi, qv, mq);
            const int t = range_rank<RK>(kl, nk, qv);
            const float kpv = __shfl(kl, max(t - 1, 0), WAVE);
            const float knv = __shfl(kl, min(t, RK - 1), WAVE);
            const float l1p = __shfl(l1, max(t - 1, 0), WAVE);
            const float r1n = __shfl(r1, min(t, RK - 1), WAVE);
            const bool lft = t > 0 || has_prev;
            const float eL = lft ? __expf(-(qv - (t > 0 ? kpv : kbefore))) : 0.f;
            const float eR = (t < nk) ? __expf(-(knv - qv)) : 0.f;
            if (act) useg[u_query_order(M) ? (int)mq : qb0 + l] = eL * (t > 0 ? l1p : L1in) + eR * r1n;
            sm.par[l] = f4_t{__int_as_float(t * RS * 4), __int_as_float(slab_row_off((int)mq, SG, CR)), eL, eR};

            float Lc[NV];
#pragma unroll
            for (int j = 0; j < NV; ++j) Lc[j] = L[j];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int t0 = c * CH;
                const int j0 = (c == 0) ? 0 : __popcll(__ballot(act && t < t0));
                const int j1 = (c == 3) ? nq : __popcll(__ballot(act && t < t0 + CH));
                if (j1 > j0) {
                    // the chunk's decays, once into SGPRs: dnext of key t0+i, and dprev of key t0+i+1 is the same value
                    float dn[CH];
#pragma unroll
                    for (int i = 0; i < CH; ++i) dn[i] = bcast(dnext, t0 + i);
                    float r[NV];
#pragma unroll
                    for (int j = 0; j < NV; ++j) r[j] = (c == 3) ? Rx[j] : Rc[c][j];
#pragma unroll
                    for (int i = CH - 1; i >= 0; --i) {
#pragma unroll
                        for (int j = 0; j < NV; ++j) {
                            r[j] = x[t0 + i][j] + dn[i] * r[j];
                            sm.b[i * RS + l + WAVE * j] = r[j];
                        }
                    }
#pragma unroll
                    for (int i = 0; i < CH; ++i) {
                        const float dp = (i == 0) ? bcast(dprev, t0) : dn[i - 1];
#pragma unroll
                        for (int j = 0; j < NV; ++j) {
                            sm.a[i * RS + l + WAVE * j] = Lc[j];
                            Lc[j] = dp * Lc[j] + x[t0 + i][j];
                        }
                    }
                    if (c == 3) {                         // rank RK: above every key of a full last range
#pragma unroll
                        for (int j = 0; j < NV; ++j) {
                            sm.a[CH * RS + l + WAVE * j] = Lc[j];
                            sm.b[CH * RS + l + WAVE * j] = 0.f;
                        }
                    }
                    // Branch-free batches of EU iterations: every lane reads a record and two rows (indices clamped
                    // into the buffers), and only the stores of queries j0 .. j1-1 (ranks in [t0, t0 + CH]) are kept.
                    constexpr int EU = 4;
                    const int rlo = t0 * RS * 4, rhi = (t0 + CH) * RS * 4;
                    for (int jb = j0; jb < j1; jb += EU * el_.qpi) {
                        f4_t pr[EU];
#pragma unroll
                        for (int u = 0; u < EU; ++u) pr[u] = sm.par[min(jb + u * el_.qpi + el_.grp, WAVE - 1)];
#pragma unroll
                        for (int u = 0; u < EU; ++u) {
                            const int j = jb + u * el_.qpi + el_.grp;
                            const int ro = min(max(__float_as_int(pr[u].x), rlo), rhi) - rlo + el_.c4 * 4;
                            const f4_t av = *reinterpret_cast<const f4_t*>(reinterpret_cast<const char*>(sm.a) + ro);
                            const f4_t bv = *reinterpret_cast<const f4_t*>(reinterpret_cast<const char*>(sm.b) + ro);
                            const f4_t o = pr[u].z * av + pr[u].w * bv;
                            if (j < j1 && el_.ok) buf_store4_stream(o, sr_, __float_as_int(pr[u].y) + el_.c4 * 4, 0);
                        }
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < CH; ++i) {
                        const float dp = bcast(dprev, t0 + i);
#pragma unroll
                        for (int j = 0; j < NV; ++j) Lc[j] = dp * Lc[j] + x[t0 + i][j];
                    }
                }
            }
        }
    }
}

template <int NV, int RK>
static int laplace_prepare_t(const float* ks, const uint32_t* kp, const float* v, int P, int D, int N, int C,
                             RangeArrays ra, hipStream_t st) {
    const int S = P * D;
    const int G = (N + RK - 1) / RK;
    const long waves = (long)S * G;
    const unsigned blocks = (unsigned)((waves + WPB - 1) / WPB);
    {
        StageTimer t("lap_range_sums", st);
        hipLaunchKernelGGL((lap_range_sums<NV, RK>), dim3(blocks), dim3(WPB * WAVE), 0, st,
                           ks, kp, v, ra.sa, ra.sb, S, D, N, C, G);
    }
    {
        StageTimer t("lap_range_scan", st);
        const int nb = scan_blocks(G);
        if (nb <= 1) {
            hipLaunchKernelGGL((lap_range_scan<NV, RK, 0>), dim3(S), dim3(SCAN_W * WAVE), 0, st,
                               ra.sa, ra.sb, ra.ta, ra.tb, nullptr, S, C, G);
        } else {
            if (ra.aggs == nullptr) return (int)hipErrorInvalidValue;
            hipLaunchKernelGGL((lap_range_scan<NV, RK, 1>), dim3(S * nb), dim3(SCAN_W * WAVE), 0, st,
                               ra.sa, ra.sb, ra.ta, ra.tb, ra.aggs, S, C, G);
            hipLaunchKernelGGL((lap_range_scan<NV, RK, 2>), dim3(S * nb), dim3(SCAN_W * WAVE), 0, st,
                               ra.sa, ra.sb, ra.ta, ra.tb, ra.aggs, S, C, G);
        }
    }
    return (int)hipGetLastError();
}

template <int NV, int RK>
static int laplace_emit_t(const float* ks, const uint32_t* kp, const float* qs, const uint32_t* qp, const float* v,
                          float* slab, float* uslab, int P, int D, int N, int M, int C, RangeArrays ra,
                          hipStream_t st) {
    const int S = P * D;
    const int G = (N + RK - 1) / RK;
    {
        const long walk_waves = (long)S * ((G + RPW - 1) / RPW);
        const unsigned walk_blocks = (unsigned)((walk_waves + WPB - 1) / WPB);
        StageTimer t("lap_range_walk", st);
        hipLaunchKernelGGL((lap_range_walk<NV, RK>), dim3(walk_blocks), dim3(WPB * WAVE), 0, st,
                           ks, kp, qs, qp, v, ra.ta, ra.tb, ra.qb, slab, uslab, S, D, N, M, C, slab_stride(C), G);
    }
    return (int)hipGetLastError();
}

int laplace_prepare(const float* ks, const uint32_t* kp, const float* v, int P, int D, int N, int C, RangeArrays ra,
                    hipStream_t st) {
    if (C <= WAVE) return laplace_prepare_t<1, 64>(ks, kp, v, P, D, N, C, ra, st);
    return laplace_prepare_t<2, 32>(ks, kp, v, P, D, N, C, ra, st);
}

int laplace_emit(const float* ks, const uint32_t* kp, const float* qs, const uint32_t* qp, const float* v,
                 float* slab, float* uslab, int P, int D, int N, int M, int C, RangeArrays ra, hipStream_t st) {
    if (C <= WAVE) return laplace_emit_t<1, 64>(ks, kp, qs, qp, v, slab, uslab, P, D, N, M, C, ra, st);
    return laplace_emit_t<2, 32>(ks, kp, qs, qp, v, slab, uslab, P, D, N, M, C, ra, st);
}

// =================================================================================================================
// Abs family
// =================================================================================================================

// Range summary: Wt = sum_t w_t, Bt = sum_t (k_last - k_t) w_t; slot C: Ut = sum_t u_t (ta; without u: the key
// weight sum sum_t kw_t, i.e. the range's count of kept keys) and B1t = sum_t kw_t (k_last - k_t) (tb). kw_t is the key
// weight (0 for masked keys); w_t and u_t are taken times kw_t.
template <int NV, int RK, bool WANT_W, bool WANT_U>
__global__ __launch_bounds__(WPB * WAVE)
void abs_range_sums(const float* __restrict__ ks, const uint32_t* __restrict__ kp,
                    const float* __restrict__ w, const float* __restrict__ u, const uint8_t* __restrict__ keep,
                    float* __restrict__ ta, float* __restrict__ tb, const int S, const int D, const int Ns,
                    const int C, const int G)
{
    const long wv = (long)xcd_slice_block(blockIdx.x, gridDim.x) * WPB + wave_in_block();
    if (wv >= (long)S * G) return;
    const int s = (int)(wv / G), g = (int)(wv - (long)s * G);
    const int p = s / D, l = lane_id();
    const int base = g * RK, nk = min(RK, Ns - base);
    const float* kseg = ks + (size_t)s * Ns;

    const int li = base + min(l, nk - 1);
    const float kl = kseg[li];
    const uint32_t pl = kp[(size_t)s * Ns + li];
    const float klast = kseg[base + nk - 1];
    const float kw = key_weight(keep, p, Ns, pl, l < nk);   // pad and masked keys weigh 0
    const float dl = kw * (klast - kl);

    float sw[NV], sb[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) { sw[j] = 0.f; sb[j] = 0.f; }
    if constexpr (WANT_W) {
        const rsrc_t wr_ = make_rsrc(w + (size_t)p * Ns * C, (uint32_t)((size_t)Ns * C * 4));
        if (NV == 1 && RK == 64 && C % 4 == 0) {
            range_row_sums_v4(wr_, C, pl, kw, dl, sw[0], sb[0]);
        } else {
#pragma unroll
            for (int t = 0; t < RK; ++t) {
                const uint32_t row = bcast(pl, t);
                const float a = bcast(kw, t), b = bcast(dl, t);
#pragma unroll
                for (int j = 0; j < NV; ++j) {
                    const int c = l + WAVE * j;
                    const float xr = buf_load(wr_, min(c, C - 1) * 4, (int)(row * C * 4));   // unconditional gather
                    const float x = (c < C) ? xr : 0.f;
                    sw[j] += a * x;
                    sb[j] += b * x;
                }
            }
        }
    }
    const float b1 = wave_sum(dl);
    float u1;
    if constexpr (WANT_U) {
        const float ur = u[(size_t)p * Ns + pl];
        u1 = wave_sum(kw != 0.f ? ur : 0.f);
    } else {
        u1 = wave_sum(kw);
    }

    const int CS = range_stride(C);
    float* ra = ta + ((size_t)s * (G + 1) + g) * CS;
    float* rb = tb + ((size_t)s * (G + 1) + g) * CS;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = l + WAVE * j;
        if (c < C) { ra[c] = sw[j]; rb[c] = sb[j]; }
    }
    if (l == 0) {
        ra[C] = u1;
        rb[C] = b1;
        ra[C + 1] = (g > 0) ? (klast - kseg[base - 1]) : 0.f;   // slot C+1: the scan's key gap into this range
    }

}

// Query bounds of every key range from the sorted queries: qb[s, g] = #{i : fl(q_i + qshift) <= klast_g}, klast_g the
// largest key of range g, for up to three query shifts in one launch (add_bump's q, q + 1, q - 1). fl(q_i + qshift)
// does not decrease with i, so each bound is one binary search over the queries. A workgroup takes one piece of up to
// QB_LDS consecutive queries of a segment into LDS (coalesced) and, for every (shift, range) pair, searches the bound
// there if the piece holds it: every query before the piece is <= klast_g (the last one is) and not every query of
// the piece is (or the piece is the segment's last). Exactly one piece passes both tests, so every bound is written
// once, and coalesced. G searches per shift and segment instead of one per query: 10.5 us a launch for add_bump's
// three shifts at the headline shape (46 us searching per query); 0.081 ms a configs[4] chunk (0.153).
constexpr int QB_T = 1024;         // threads per workgroup
constexpr int QB_LDS = 16384;      // queries per piece
constexpr int QB_MAXG = 4096;      // ranges per segment: N <= 131072 keys in ranges of >= 32

struct BoundSets { int* qb[3]; float shift[3]; };

template <int RK>
__global__ __launch_bounds__(QB_T)
void query_bounds_lds(const float* __restrict__ ks, const float* __restrict__ qs, const BoundSets sets,
                      const int nsets, const int Ns, const int Mq, const int G, const int pieces)
{
    __shared__ float qv[QB_LDS];
    const int s = blockIdx.x / pieces, pc = blockIdx.x - s * pieces;
    const int p0 = pc * QB_LDS, len = min(QB_LDS, Mq - p0);
    const float* qseg = qs + (size_t)s * Mq;
    for (int i = threadIdx.x; i < len; i += QB_T) qv[i] = qseg[p0 + i];
    const float qprev = p0 > 0 ? qseg[p0 - 1] : 0.f;       // the last query before the piece
    __syncthreads();
    const float* kseg = ks + (size_t)s * Ns;
    const bool last = pc == pieces - 1;
    for (int t = threadIdx.x; t < nsets * G; t += QB_T) {
        const int set = t / G, g = t - set * G;
        const float qshift = set == 0 ? sets.shift[0] : set == 1 ? sets.shift[1] : sets.shift[2];
        int* qb = set == 0 ? sets.qb[0] : set == 1 ? sets.qb[1] : sets.qb[2];
        const float kl = kseg[min(Ns, (g + 1) * RK) - 1];
        if (p0 > 0 && !(qprev + qshift <= kl)) continue;   // a query before the piece is above klast_g
        if (!last && qv[len - 1] + qshift <= kl) continue; // the whole piece is <= klast_g: a later piece holds it
        int lo = 0, hi = len;                             // first i of the piece with fl(q_i + qshift) > klast_g
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (qv[mid] + qshift <= kl) lo = mid + 1;
            else hi = mid;
        }
        qb[(size_t)s * G + g] = p0 + lo;
    }
}

int query_bounds_sets(const float* ks, const float* qs, int* const qb[], const float shift[], int nsets, int S,
                      int Ns, int Mq, int C, hipStream_t st) {
    const int RK = range_keys(C);
    const int G = (Ns + RK - 1) / RK;
    if (G > QB_MAXG || nsets < 1 || nsets > 3) return (int)hipErrorInvalidValue;
    BoundSets sets{};
    for (int i = 0; i < nsets; ++i) { sets.qb[i] = qb[i]; sets.shift[i] = shift[i]; }
    const int pieces = (Mq + QB_LDS - 1) / QB_LDS;
    const dim3 grid((unsigned)((long)S * pieces));
    StageTimer t("query_bounds", st);
    if (RK == 64)
        hipLaunchKernelGGL((query_bounds_lds<64>), grid, dim3(QB_T), 0, st, ks, qs, sets, nsets, Ns, Mq, G, pieces);
    else
        hipLaunchKernelGGL((query_bounds_lds<32>), grid, dim3(QB_T), 0, st, ks, qs, sets, nsets, Ns, Mq, G, pieces);
    return (int)hipGetLastError();
}

int query_bounds(const float* ks, const float* qs, int* qb, float qshift, int S, int Ns, int Mq, int C,
                 hipStream_t st) {
    int* const qbs[1] = {qb};
    const float sh[1] = {qshift};
    return query_bounds_sets(ks, qs, qbs, sh, 1, S, Ns, Mq, C, st);
}

template <int CH>
__global__ __launch_bounds__(GQ_T)
void group_queries_staged(const float* __restrict__ ks, const float* __restrict__ q, float* __restrict__ qs,
                          uint32_t* __restrict__ qp, int* __restrict__ qb, const float qshift, const int Ns,
                          const int Mq, const int G, const int Gc)
{
    __shared__ GroupTables tb;
    __shared__ float sv[GQ_STAGE];
    __shared__ uint32_t si[GQ_STAGE];
    const int s = blockIdx.x;
    const float* kseg = ks + (size_t)s * Ns;
    group_segment<CH>([&](int i) { return kseg[i]; }, q + (size_t)s * Mq, qs + (size_t)s * Mq, qp + (size_t)s * Mq,
                      qb + (size_t)s * G, qshift, Ns, Mq, Gc, tb, sv, si);
}

bool group_fits(int Ns, int Mq, int C) {
    const int CH = range_keys(C) / 4;
    return Mq <= GQ_STAGE && (Ns + CH - 1) / CH <= GQ_STAGE_MAXB;
}

int group_queries(const float* ks, const float* q, float* qs, uint32_t* qp, int* qb, float qshift, int S, int Ns,
                  int Mq, int C, hipStream_t st) {
    const int RK = range_keys(C), CH = RK / 4;
    const int G = (Ns + RK - 1) / RK, Gc = (Ns + CH - 1) / CH;
    if (!group_fits(Ns, Mq, C)) return (int)hipErrorInvalidValue;
    StageTimer t("group_queries", st);
    if (CH == 16) hipLaunchKernelGGL((group_queries_staged<16>), dim3(S), dim3(GQ_T), 0, st,
                                     ks, q, qs, qp, qb, qshift, Ns, Mq, G, Gc);
    else hipLaunchKernelGGL((group_queries_staged<8>), dim3(S), dim3(GQ_T), 0, st,
                            ks, q, qs, qp, qb, qshift, Ns, Mq, G, Gc);
    return (int)hipGetLastError();
}

// Abs: entry prefix state of every range and the segment totals (row G). State (PW, B) with B relative to the last
// key absorbed: at range g, B <- b_g + B + gap_g PW, PW <- PW + a_g for every slot, slot C included (gap_g = klast_g -
// klast_{g-1}). A piece composes to  PW = PW_in + sum a,  B = B_in + B_local + (sum of its gaps) PW_in. Long segments
// take two launches over workgroups of SCAN_BLOCK ranges, as the Laplace scan (the record's part 0 holds PW with the
// gap sum in its link vector, part 1 holds B).
template <int NV, int RK, int PHASE>
__global__ __launch_bounds__(SCAN_W * WAVE)
void abs_range_scan(const float* __restrict__ sa, const float* __restrict__ sb, float* __restrict__ ta,
                    float* __restrict__ tb, float* __restrict__ aggs, const int S, const int Ns, const int C,
                    const int G)
{
    __shared__ float agg[2][SCAN_W][NV + 1][WAVE];
    __shared__ float span[SCAN_W];
    const int nb = PHASE == 0 ? 1 : scan_blocks(G);
    const int s = blockIdx.x / nb, blk = blockIdx.x - s * nb;
    const int w = wave_in_block(), l = lane_id();
    const int CS = range_stride(C);
    const float* SA = sa + (size_t)s * (G + 1) * CS;
    const float* SB = sb + (size_t)s * (G + 1) * CS;
    float* A = ta + (size_t)s * (G + 1) * CS;
    float* B = tb + (size_t)s * (G + 1) * CS;
    const int b0 = PHASE == 0 ? 0 : blk * SCAN_BLOCK, b1 = PHASE == 0 ? G : min(G, b0 + SCAN_BLOCK);
    const int per = (b1 - b0 + SCAN_W - 1) / SCAN_W;
    const int glo = min(b1, b0 + w * per), ghi = min(b1, b0 + w * per + per);
    float* seg_aggs = PHASE == 0 ? nullptr : aggs + (size_t)s * nb * scan_rec_floats<NV>();

    // piece walk from (pw, bb); writes entry states when OUT; returns the sum of the piece's gaps. Slot NV (slot C
    // of the rows) runs the same recurrence: its B state (the v == 1 channel) is weighted by its PW state, the count of
    // kept keys so far (for the u-weighted walks that slot of B is not read).
    ScanPiece<NV> piece_a, piece_b;
    piece_a.load(SA, CS, C, glo, ghi);
    piece_b.load(SB, CS, C, glo, ghi);
    auto walk = [&](float (&pw)[NV + 1], float (&bb)[NV + 1], const bool out) {
        float gsum = 0.f;
#pragma unroll
        for (int i = 0; i < SCAN_BLOCK / SCAN_W; ++i) {
            const int g = glo + i;
            if (g >= ghi) break;
            float a[NV + 1], b_[NV + 1], gap, unused;
            piece_a.get(i, a, gap);
            piece_b.get(i, b_, unused);
            if (out) {
                store_scan_row<NV>(A + (size_t)g * CS, C, pw);
                store_scan_row<NV>(B + (size_t)g * CS, C, bb);
            }
#pragma unroll
            for (int j = 0; j <= NV; ++j) { bb[j] = b_[j] + bb[j] + gap * pw[j]; pw[j] += a[j]; }
            gsum += gap;
        }
        return gsum;
    };

    float pw[NV + 1], bb[NV + 1];
    if constexpr (PHASE <= 1) {
        // pass 1: every piece from a zero state (empty pieces: all zero)
#pragma unroll
        for (int j = 0; j <= NV; ++j) { pw[j] = 0.f; bb[j] = 0.f; }
        const float gs = walk(pw, bb, false);
#pragma unroll
        for (int j = 0; j <= NV; ++j) { agg[0][w][j][l] = pw[j]; agg[1][w][j][l] = bb[j]; }
        if (l == 0) span[w] = gs;
    }
    if constexpr (PHASE == 1) {
        // the wave aggregates, and wave 0 composes the workgroup's from left to right
        float* rec = seg_aggs + (size_t)blk * scan_rec_floats<NV>();
        float* w0 = agg_slot<NV>(rec, w, 0);
        float* w1 = agg_slot<NV>(rec, w, 1);
#pragma unroll
        for (int j = 0; j <= NV; ++j) { w0[j * WAVE + l] = pw[j]; w1[j * WAVE + l] = bb[j]; }
        __syncthreads();
        w0[(NV + 1) * WAVE + l] = span[w];
        if (w == 0) {
            float cp[NV + 1], cb[NV + 1], gsum = 0.f;
#pragma unroll
            for (int j = 0; j <= NV; ++j) { cp[j] = 0.f; cb[j] = 0.f; }
            for (int ww = 0; ww < SCAN_W; ++ww) {
                const float sp = span[ww];
#pragma unroll
                for (int j = 0; j <= NV; ++j) { cb[j] += agg[1][ww][j][l] + sp * cp[j]; cp[j] += agg[0][ww][j][l]; }
                gsum += sp;
            }
            float* b0_ = agg_slot<NV>(rec, SCAN_W, 0);
            float* b1_ = agg_slot<NV>(rec, SCAN_W, 1);
#pragma unroll
            for (int j = 0; j <= NV; ++j) { b0_[j * WAVE + l] = cp[j]; b1_[j * WAVE + l] = cb[j]; }
            b0_[(NV + 1) * WAVE + l] = gsum;
        }
        return;
    }
    if constexpr (PHASE == 2) {
        // this workgroup's wave aggregates, from phase 1
        const float* rec = seg_aggs + (size_t)blk * scan_rec_floats<NV>();
        const float* w0 = agg_slot<NV>(const_cast<float*>(rec), w, 0);
        const float* w1 = agg_slot<NV>(const_cast<float*>(rec), w, 1);
#pragma unroll
        for (int j = 0; j <= NV; ++j) { agg[0][w][j][l] = w0[j * WAVE + l]; agg[1][w][j][l] = w1[j * WAVE + l]; }
        if (l == 0) span[w] = w0[(NV + 1) * WAVE];
    }
    __syncthreads();

    // incoming state: the workgroups before this one, then its waves before this wave
#pragma unroll
    for (int j = 0; j <= NV; ++j) { pw[j] = 0.f; bb[j] = 0.f; }
    if constexpr (PHASE == 2) {
        for (int k = 0; k < blk; ++k) {
            const float* r0 = agg_slot<NV>(seg_aggs + (size_t)k * scan_rec_floats<NV>(), SCAN_W, 0);
            const float* r1 = agg_slot<NV>(seg_aggs + (size_t)k * scan_rec_floats<NV>(), SCAN_W, 1);
            const float sp = r0[(NV + 1) * WAVE + l];
#pragma unroll
            for (int j = 0; j <= NV; ++j) { bb[j] += r1[j * WAVE + l] + sp * pw[j]; pw[j] += r0[j * WAVE + l]; }
        }
    }
    for (int ww = 0; ww < w; ++ww) {
        const float sp = span[ww];
#pragma unroll
        for (int j = 0; j <= NV; ++j) { bb[j] += agg[1][ww][j][l] + sp * pw[j]; pw[j] += agg[0][ww][j][l]; }
    }
    walk(pw, bb, true);
    if (ghi == G && glo < G) {                            // the wave whose piece ends the segment writes the totals
        store_scan_row<NV>(A + (size_t)G * CS, C, pw);
        store_scan_row<NV>(B + (size_t)G * CS, C, bb);
    }
}

// NS = 1: the queries a.qs (+ a.qshift) with bounds qb, rows to a.slab / a.uslab. NS = 3 (ROW | ONES only): also the
// query sets 1 and 2 of a.set_* (add_bump's q + 1 and q - 1: the same sorted order, their own bounds and slabs), each
// walked over the same gathered rows and key-side states as set 0.
template <int NV, int RK, int MODE, int NS>
__global__ __launch_bounds__(WPB * WAVE)
void abs_range_walk(AbsWalkArgs a, const float* __restrict__ ta, const float* __restrict__ tb,
                    const int* __restrict__ qb, const int G)
{
    static_assert(NS == 1 || (NS == 3 && (MODE & ~ABS_KEEP) == (ABS_ROW | ABS_ONES)), "query sets: row walks only");
    constexpr bool ROW = MODE & ABS_ROW, ONES = MODE & ABS_ONES, DOT = MODE & ABS_DOT;
    constexpr bool X1 = MODE & ABS_DOTX1, X2 = MODE & ABS_DOTX2, RANK = MODE & ABS_RANK, KEEP = MODE & ABS_KEEP;
    constexpr bool EMIT = ROW || DOT;                     // rows gathered, states staged in LDS, emission
    constexpr bool EXTRA = X1 || X2;
    using Lds = WalkLds<NV, RK>;
    constexpr int CH = Lds::CH, RS = Lds::RS;
    __shared__ Lds lds[EMIT ? WPB : 1];
    __shared__ float exs[EXTRA ? WPB : 1][WAVE];          // per-query scalar added to the dot (X1 / X2)
    const int S = a.P * a.D, C = a.C, Ns = a.Ns, Mq = a.Mq;
    const long wv = (long)xcd_slice_block(blockIdx.x, gridDim.x) * WPB + wave_in_block();
    if (wv >= (long)S * G) return;
    Lds& sm = lds[EMIT ? wave_in_block() : 0];
    float* ex = exs[EXTRA ? wave_in_block() : 0];
    const int s = (int)(wv / G), g = (int)(wv - (long)s * G);
    const int p = s / a.D, l = lane_id();
    const int base = g * RK, nk = min(RK, Ns - base);
    const float* kseg = a.ks + (size_t)s * Ns;
    const uint32_t* kpseg = a.kp + (size_t)s * Ns;
    const float* qseg = a.qs + (size_t)s * Mq;
    const uint32_t* qpseg = a.qp + (size_t)s * Mq;

    const int li = base + min(l, nk - 1);
    const float kl = kseg[li];
    const bool real = l < nk;
    const bool has_prev = g > 0, has_next = g < G - 1;
    const float kbefore = has_prev ? kseg[base - 1] : 0.f;
    const float kmax = kseg[Ns - 1];
    float kw = real ? 1.f : 0.f;                         // key weight (KEEP: 0 for masked keys)
    if constexpr (KEEP) kw = key_weight(a.keep, p, Ns, kpseg[li], real);

    // weight rows of the range, lane = channel (pad keys and pad channels: zero); row indices by scalar loads
    float x[RK][NV];
    if constexpr (EMIT) {
        const rsrc_t wr_ = make_rsrc(a.w + (size_t)p * Ns * C, (uint32_t)((size_t)Ns * C * 4));
        if (nk == RK) {
#pragma unroll
            for (int t = 0; t < RK; ++t) {
                const int rowoff = (int)(kpseg[base + t] * C * 4);
#pragma unroll
                for (int j = 0; j < NV; ++j)
                    x[t][j] = buf_load(wr_, min(l + WAVE * j, C - 1) * 4, rowoff);   // unconditional gather
            }
        } else {
#pragma unroll
            for (int t = 0; t < RK; ++t) {
                const int rowoff = (int)(kpseg[base + min(t, nk - 1)] * C * 4);
#pragma unroll
                for (int j = 0; j < NV; ++j)
                    x[t][j] = buf_load(wr_, min(l + WAVE * j, C - 1) * 4, rowoff);
            }
        }
        if (nk < RK || C < RS) {                          // partial last range or pad channels (uniform branch)
#pragma unroll
            for (int t = 0; t < RK; ++t)
#pragma unroll
                for (int j = 0; j < NV; ++j)
                    x[t][j] = (t < nk && l + WAVE * j < C) ? x[t][j] : 0.f;
        }
        if constexpr (KEEP) mask_rows<NV, RK>(x, kw);
    }
    // owned queries [q0, q1) and (without a key mask, whose walk has no registers to spare) their first block of 64
    // (value and index, clamped like the loop's loads), loaded right after the gathers so that their latency overlaps
    // the prefix work below
    const int q0 = has_prev ? qb[(size_t)s * G + g - 1] : 0;
    const int q1 = has_next ? qb[(size_t)s * G + g] : Mq;
    constexpr bool PREF = !KEEP;
    float qv0 = 0.f;
    uint32_t mq0 = 0;
    if constexpr (PREF) {
        const int qi0 = min(q0 + l, max(q1 - 1, 0));
        qv0 = qseg[qi0];
        mq0 = qpseg[qi0];
    }
    float ul = 0.f;
    if constexpr (X2) {
        const float ur = a.u[(size_t)p * Ns + kpseg[li]];
        ul = real ? ur : 0.f;
    }

    float kbef = __shfl_up(kl, 1, WAVE);
    if (l == 0) kbef = kbefore;
    const float gap = (real && (l > 0 || has_prev)) ? (kl - kbef) : 0.f;   // distance from the key before

    const int CS = range_stride(C);
    const float* rowA = ta + ((size_t)s * (G + 1) + g) * CS;
    const float* rowB = tb + ((size_t)s * (G + 1) + g) * CS;
    const float* totA = ta + ((size_t)s * (G + 1) + G) * CS;
    const float* totB = tb + ((size_t)s * (G + 1) + G) * CS;
    // The segment-total terms -Btot - (q - k_max) Wtot (rows) and -B1t - (q - k_max) N (v == 1) of the three query
    // sets of add_bump cancel in its numerator and denominator, (T+ + T-) / 2 - T0 = 0 for q +- 1: that walk leaves
    // them out, and with them their rounding, which grows with the span of the keys.
    constexpr bool TOT = NS == 1;
    float PW[NV], Bv[NV], Bt[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = l + WAVE * j;
        const bool ok = c < C;
        const int cc = min(c, C - 1);
        PW[j] = (EMIT && ok) ? rowA[cc] : 0.f;
        Bv[j] = (ROW && ok) ? rowB[cc] : 0.f;
        Bt[j] = (ROW && TOT && ok) ? totB[cc] : 0.f;
    }
    float PU = 0.f, Ut = 0.f, B1 = 0.f, B1t = 0.f;
    if constexpr (X2 || (ONES && KEEP)) { PU = rowA[C]; Ut = totA[C]; }   // u sums (X2) / kept-key counts (KEEP)
    if constexpr (ONES) { B1 = rowB[C]; B1t = TOT ? totB[C] : 0.f; }
    const float Nf = (float)Ns;

    // Emission lanes: channels c4 .. c4+3 of one query row; Wtot of those channels
    const EmitLanes el_(slab_stride(C));
    f4_t wt4 = {0.f, 0.f, 0.f, 0.f};
    if constexpr (EMIT && TOT) {
#pragma unroll
        for (int i = 0; i < 4; ++i) wt4[i] = (el_.c4 + i < C) ? totA[min(el_.c4 + i, C - 1)] : 0.f;
    }
    const bool g_vec4 = DOT && (C % 4 == 0) && ((((uintptr_t)a.g) & 15) == 0);

    // Lane-parallel prefixes over the range's keys for the scalar emissions (exclusive prefix at rank t = inclusive
    // value of lane t-1): b1 state  sum_{i<t} gap_i * (keys before key i), u prefix  sum_{i<t} u_i and, with a key
    // mask, kept keys  sum_{i<t} kw_i  (the key counts then count kept keys only, from the scan's count PU).
    float kci = 0.f, gci = 0.f, uli = 0.f;
    if constexpr (ONES && KEEP) {
        kci = wave_prefix_sum(kw);
        gci = wave_prefix_sum(gap * (PU + (kci - kw)));
    } else if constexpr (ONES) {
        gci = wave_prefix_sum(gap * (float)(base + l));
    }
    if constexpr (X2) uli = wave_prefix_sum(ul);

    const int SG = slab_group(a.D);
    const rsrc_t gr_ = DOT ? make_rsrc(a.g + (size_t)p * Mq * C, (uint32_t)((size_t)Mq * C * 4))
                           : make_rsrc(nullptr, 0);
#pragma unroll 1
    for (int set = 0; set < NS; ++set) {
    int sq0 = q0, sq1 = q1;                               // the set's owned queries
    if (set > 0) {
        const int* sqb = a.set_qb[set];
        sq0 = has_prev ? sqb[(size_t)s * G + g - 1] : 0;
        sq1 = has_next ? sqb[(size_t)s * G + g] : Mq;
    }
    const float qshift = set == 0 ? a.qshift : a.set_shift[set];
    float* const slab_s = set == 0 ? a.slab : a.set_slab[set];
    const rsrc_t sr_ = ROW ? make_rsrc(slab_s + slab_seg_base(p, s - p * a.D, a.D, Mq, a.CR),
                                       slab_seg_bytes(s - p * a.D, a.D, Mq, a.CR))
                           : make_rsrc(nullptr, 0);
    float* useg = ONES ? (set == 0 ? a.uslab : a.set_uslab[set]) + (size_t)s * Mq
                       : nullptr;                         // v == 1 terms, order: u_query_order

    // Owned queries in blocks of 64. Lane i takes query i: its rank t inside the range, its distances and its scalar
    // outputs (v == 1 sum, rank, dot extras) from the lane-parallel prefixes; its record (row offset of rank t in the
    // chunk buffers, query index, 2 (q - k_prev), q - k_max) goes to LDS. Then the keys are walked in 4 chunks of CH:
    // the chunk's states PW and 2B - Btot before each key go to LDS and the queries ranked in the chunk are emitted,
    //   row:  2 (q - k_prev) PW + (2B - Btot) - (q - k_max) Wtot,     dot:  <g_q, 2 PW - Wtot> + extra.
    for (int qb0 = sq0; qb0 < sq1; qb0 += WAVE) {
        const int nq = min(WAVE, sq1 - qb0);
        const bool act = l < nq;
        const int qi = min(qb0 + l, sq1 - 1);             // clamped: unconditional loads
        const bool first = PREF && set == 0 && qb0 == sq0;
        const float qv = (first ? qv0 : qseg[qi]) + qshift;
        const uint32_t mq = first ? mq0 : qpseg[qi];
        const int t = range_rank<RK>(kl, nk, qv);
        const float kpv = __shfl(kl, max(t - 1, 0), WAVE);
        const float lq = qv - (t > 0 ? kpv : kbefore);   // distance to the last key below q (unused when none)
        const float qm = qv - kmax;
        const float cnt = (float)(base + min(t, nk));    // keys below q
        if constexpr (RANK) {
            if (act) a.out_rank[(size_t)s * Mq + mq] = base + t;
        }
        if constexpr (ONES) {
            const float gp = __shfl(gci, max(t - 1, 0), WAVE);
            const float b1 = B1 + (t > 0 ? gp : 0.f);
            float below = cnt, all = TOT ? Nf : 0.f;      // (kept) keys below q, all (kept) keys
            if constexpr (KEEP) {
                const float kp_ = __shfl(kci, max(t - 1, 0), WAVE);
                below = PU + (t > 0 ? kp_ : 0.f);
                all = TOT ? Ut : 0.f;
            }
            if (act) useg[u_query_order(Mq) ? (int)mq : qb0 + l] = 2.f * (lq * below + b1) - B1t - qm * all;
        }
        if constexpr (EXTRA) {
            float e = 0.f;
            if constexpr (X1) e += a.uq[(size_t)p * Mq + mq] * (2.f * cnt - Nf);
            if constexpr (X2) {
                const float up = __shfl(uli, max(t - 1, 0), WAVE);
                e += 2.f * (PU + (t > 0 ? up : 0.f)) - Ut;
            }
            ex[l] = e;
        }
        if constexpr (!EMIT) continue;
        sm.par[l] = f4_t{__int_as_float(t * RS * 4), __int_as_float((int)mq), 2.f * lq, qm};

        float pw[NV], bv[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j) { pw[j] = PW[j]; bv[j] = Bv[j]; }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int t0 = c * CH;
            const int j0 = (c == 0) ? 0 : __popcll(__ballot(act && t < t0));
            const int j1 = (c == 3) ? nq : __popcll(__ballot(act && t < t0 + CH));
            if (j1 > j0) {
#pragma unroll
                for (int i = 0; i < CH; ++i) {
                    const float gt = bcast(gap, t0 + i);
#pragma unroll
                    for (int j = 0; j < NV; ++j) {
                        sm.a[i * RS + l + WAVE * j] = pw[j];
                        if constexpr (ROW) {
                            sm.b[i * RS + l + WAVE * j] = 2.f * bv[j] - Bt[j];
                            bv[j] += gt * pw[j];
                        }
                        pw[j] += x[t0 + i][j];
                    }
                }
                if (c == 3) {                             // rank RK: above every key of a full last range
#pragma unroll
                    for (int j = 0; j < NV; ++j) {
                        sm.a[CH * RS + l + WAVE * j] = pw[j];
                        if constexpr (ROW) sm.b[CH * RS + l + WAVE * j] = 2.f * bv[j] - Bt[j];
                    }
                }
                // Branch-free batches of EU iterations (indices clamped into the buffers); only queries j0 .. j1-1
                // (ranks in [t0, t0 + CH]) store.
                constexpr int EU = 4;
                const int rlo = t0 * RS * 4, rhi = (t0 + CH) * RS * 4;
                for (int jb = j0; jb < j1; jb += EU * el_.qpi) {
                    f4_t pr[EU];
#pragma unroll
                    for (int u = 0; u < EU; ++u) pr[u] = sm.par[min(jb + u * el_.qpi + el_.grp, WAVE - 1)];
                    f4_t gv[EU];
                    if constexpr (DOT) {
#pragma unroll
                        for (int u = 0; u < EU; ++u) {
                            const int goff = __float_as_int(pr[u].y) * C * 4 + el_.c4 * 4;
                            if (g_vec4) {
                                gv[u] = buf_load4(gr_, goff, 0);
                            } else {
#pragma unroll
                                for (int i = 0; i < 4; ++i) gv[u][i] = buf_load(gr_, goff + i * 4, 0);
                            }
#pragma unroll
                            for (int i = 0; i < 4; ++i) gv[u][i] = (el_.c4 + i < C) ? gv[u][i] : 0.f;
                        }
                    }
#pragma unroll
                    for (int u = 0; u < EU; ++u) {
                        const int j = jb + u * el_.qpi + el_.grp;
                        const int ro = min(max(__float_as_int(pr[u].x), rlo), rhi) - rlo + el_.c4 * 4;
                        const f4_t av = *reinterpret_cast<const f4_t*>(reinterpret_cast<const char*>(sm.a) + ro);
                        const int m = __float_as_int(pr[u].y);
                        if constexpr (ROW) {
                            const f4_t bw = *reinterpret_cast<const f4_t*>(reinterpret_cast<const char*>(sm.b) + ro);
                            const f4_t o = pr[u].z * av + bw - pr[u].w * wt4;
                            if constexpr (NS == 3) {
                                // three query sets: a branch-free store (an offset past the descriptor drops it) lets
                                // the batch's LDS reads issue together (add_bump 4.34 -> 4.30 ms); with one set the
                                // dropped lanes' store slots cost more than that (Laplace and abs +0.3%)
                                const int so = (j < j1 && el_.ok) ? slab_row_off(m, SG, a.CR) + el_.c4 * 4 : STORE_OOB;
                                buf_store4_stream(o, sr_, so, 0);
                            } else if (j < j1 && el_.ok) {
                                buf_store4_stream(o, sr_, slab_row_off(m, SG, a.CR) + el_.c4 * 4, 0);
                            }
                        }
                        if constexpr (DOT) {
                            const f4_t w2 = 2.f * av - wt4;
                            float d = gv[u][0] * w2[0] + gv[u][1] * w2[1] + gv[u][2] * w2[2] + gv[u][3] * w2[3];
                            for (int off = 1 << (el_.sh - 1); off >= 1; off >>= 1) d += __shfl_xor(d, off, WAVE);
                            if constexpr (EXTRA) d += ex[min(j, WAVE - 1)];
                            if (j < j1 && el_.c4 == 0) a.out_dot[(size_t)s * Mq + m] = a.sign * d;
                        }
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < CH; ++i) {
                    const float gt = bcast(gap, t0 + i);
#pragma unroll
                    for (int j = 0; j < NV; ++j) {
                        if constexpr (ROW) bv[j] += gt * pw[j];
                        pw[j] += x[t0 + i][j];
                    }
                }
            }
        }
    }
    }   // set
}

template <int NV, int RK, int MODE, int NS = 1>
static void launch_abs_walk(const AbsWalkArgs& a, RangeArrays ra, int G, hipStream_t st) {
    const long waves = (long)a.P * a.D * G;
    const unsigned blocks = (unsigned)((waves + WPB - 1) / WPB);
    StageTimer t("abs_range_walk", st);
    hipLaunchKernelGGL((abs_range_walk<NV, RK, MODE, NS>), dim3(blocks), dim3(WPB * WAVE), 0, st, a, ra.ta, ra.tb,
                       ra.qb, G);
}

template <int NV, int RK>
static int abs_prepare_t(const AbsWalkArgs& a, int mode, RangeArrays ra, hipStream_t st) {
    const int S = a.P * a.D;
    const int G = (a.Ns + RK - 1) / RK;
    const long waves = (long)S * G;
    const unsigned blocks = (unsigned)((waves + WPB - 1) / WPB);
    {
        StageTimer t("abs_range_sums", st);
        if (mode & ABS_DOTX2)
            hipLaunchKernelGGL((abs_range_sums<NV, RK, true, true>), dim3(blocks), dim3(WPB * WAVE), 0, st,
                               a.ks, a.kp, a.w, a.u, a.keep, ra.sa, ra.sb, S, a.D, a.Ns, a.C, G);
        else if (mode == ABS_RANK)
            hipLaunchKernelGGL((abs_range_sums<NV, RK, false, false>), dim3(blocks), dim3(WPB * WAVE), 0, st,
                               a.ks, a.kp, a.w, a.u, a.keep, ra.sa, ra.sb, S, a.D, a.Ns, a.C, G);
        else
            hipLaunchKernelGGL((abs_range_sums<NV, RK, true, false>), dim3(blocks), dim3(WPB * WAVE), 0, st,
                               a.ks, a.kp, a.w, a.u, a.keep, ra.sa, ra.sb, S, a.D, a.Ns, a.C, G);
    }
    {
        StageTimer t("abs_range_scan", st);
        const int nb = scan_blocks(G);
        if (nb <= 1) {
            hipLaunchKernelGGL((abs_range_scan<NV, RK, 0>), dim3(S), dim3(SCAN_W * WAVE), 0, st,
                               ra.sa, ra.sb, ra.ta, ra.tb, nullptr, S, a.Ns, a.C, G);
        } else {
            if (ra.aggs == nullptr) return (int)hipErrorInvalidValue;
            hipLaunchKernelGGL((abs_range_scan<NV, RK, 1>), dim3(S * nb), dim3(SCAN_W * WAVE), 0, st,
                               ra.sa, ra.sb, ra.ta, ra.tb, ra.aggs, S, a.Ns, a.C, G);
            hipLaunchKernelGGL((abs_range_scan<NV, RK, 2>), dim3(S * nb), dim3(SCAN_W * WAVE), 0, st,
                               ra.sa, ra.sb, ra.ta, ra.tb, ra.aggs, S, a.Ns, a.C, G);
        }
    }
    return (int)hipGetLastError();
}

template <int NV, int RK>
static int abs_emit_t(const AbsWalkArgs& a, int mode, RangeArrays ra, hipStream_t st) {
    const int G = (a.Ns + RK - 1) / RK;
    if (((mode & ABS_KEEP) != 0) != (a.keep != nullptr)) return (int)hipErrorInvalidValue;   // sums and walk agree
    if (a.nsets == 3) {
        switch (mode) {
            case ABS_ROW | ABS_ONES:            launch_abs_walk<NV, RK, ABS_ROW | ABS_ONES, 3>(a, ra, G, st); break;
            case ABS_ROW | ABS_ONES | ABS_KEEP: launch_abs_walk<NV, RK, ABS_ROW | ABS_ONES | ABS_KEEP, 3>(a, ra, G, st);
                                                break;
            default: return (int)hipErrorInvalidValue;
        }
        return (int)hipGetLastError();
    }
    if (a.nsets > 1) return (int)hipErrorInvalidValue;
    switch (mode) {
        case ABS_ROW:                         launch_abs_walk<NV, RK, ABS_ROW>(a, ra, G, st); break;
        case ABS_ROW | ABS_ONES:              launch_abs_walk<NV, RK, ABS_ROW | ABS_ONES>(a, ra, G, st); break;
        case ABS_ROW | ABS_ONES | ABS_KEEP:   launch_abs_walk<NV, RK, ABS_ROW | ABS_ONES | ABS_KEEP>(a, ra, G, st);
                                              break;
        case ABS_DOT:                         launch_abs_walk<NV, RK, ABS_DOT>(a, ra, G, st); break;
        case ABS_DOT | ABS_DOTX1:             launch_abs_walk<NV, RK, ABS_DOT | ABS_DOTX1>(a, ra, G, st); break;
        case ABS_ROW | ABS_DOT:               launch_abs_walk<NV, RK, ABS_ROW | ABS_DOT>(a, ra, G, st); break;
        case ABS_ROW | ABS_DOT | ABS_DOTX2:   launch_abs_walk<NV, RK, ABS_ROW | ABS_DOT | ABS_DOTX2>(a, ra, G, st);
                                              break;
        case ABS_RANK:                        launch_abs_walk<NV, RK, ABS_RANK>(a, ra, G, st); break;
        default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

int range_count(int Ns, int C) {
    const int RK = range_keys(C);
    return (Ns + RK - 1) / RK;
}

// The range scans over caller-given summary rows (S segments of G ranges, rows of C + 2 floats, one channel slot per
// lane: C <= 64): the abs scan's entry states (PW with its link-weighted B) and the Laplace scan's (forward L with its
// link factors, backward R), as abs_prepare and laplace_prepare run them after their sums.
int abs_scan_rows(const float* sa, const float* sb, float* ta, float* tb, float* aggs, int S, int C, int G,
                  hipStream_t st) {
    if (C > WAVE) return (int)hipErrorInvalidValue;
    StageTimer t("abs_range_scan", st);
    const int nb = scan_blocks(G);
    if (nb <= 1) {
        hipLaunchKernelGGL((abs_range_scan<1, 64, 0>), dim3(S), dim3(SCAN_W * WAVE), 0, st, sa, sb, ta, tb, nullptr, S,
                           G * 64, C, G);
    } else {
        if (aggs == nullptr) return (int)hipErrorInvalidValue;
        hipLaunchKernelGGL((abs_range_scan<1, 64, 1>), dim3(S * nb), dim3(SCAN_W * WAVE), 0, st, sa, sb, ta, tb, aggs,
                           S, G * 64, C, G);
        hipLaunchKernelGGL((abs_range_scan<1, 64, 2>), dim3(S * nb), dim3(SCAN_W * WAVE), 0, st, sa, sb, ta, tb, aggs,
                           S, G * 64, C, G);
    }
    return (int)hipGetLastError();
}

// two independent linked sums over range rows (X <- a_g + link_g X), each row's link in its slot C + 1: the entry
// states of ranges 0 .. G - 1 and the final state in row G
int linked_scan_pair(const float* sa, const float* sb, float* ta, float* tb, float* aggs, int S, int C, int G,
                     hipStream_t st) {
    if (C > WAVE) return (int)hipErrorInvalidValue;
    StageTimer t("linked_scan_pair", st);
    const int nb = scan_blocks(G);
    if (nb <= 1) {
        hipLaunchKernelGGL((lap_range_scan<1, 64, 0, true>), dim3(S), dim3(SCAN_W * WAVE), 0, st, sa, sb, ta, tb,
                           nullptr, S, C, G);
    } else {
        if (aggs == nullptr) return (int)hipErrorInvalidValue;
        hipLaunchKernelGGL((lap_range_scan<1, 64, 1, true>), dim3(S * nb), dim3(SCAN_W * WAVE), 0, st, sa, sb, ta, tb,
                           aggs, S, C, G);
        hipLaunchKernelGGL((lap_range_scan<1, 64, 2, true>), dim3(S * nb), dim3(SCAN_W * WAVE), 0, st, sa, sb, ta, tb,
                           aggs, S, C, G);
    }
    return (int)hipGetLastError();
}

int abs_prepare(const AbsWalkArgs& a, int mode, RangeArrays ra, hipStream_t st) {
    if (a.C <= WAVE) return abs_prepare_t<1, 64>(a, mode, ra, st);
    return abs_prepare_t<2, 32>(a, mode, ra, st);
}

int abs_emit(const AbsWalkArgs& a, int mode, RangeArrays ra, hipStream_t st) {
    if (a.C <= WAVE) return abs_emit_t<1, 64>(a, mode, ra, st);
    return abs_emit_t<2, 32>(a, mode, ra, st);
}

int abs_walk(const AbsWalkArgs& a, int mode, RangeArrays ra, hipStream_t st) {
    if (int e = range_bounds(a, ra.qb, st)) return e;
    if (int e = abs_prepare(a, mode, ra, st)) return e;
    return abs_emit(a, mode, ra, st);
}

int range_bounds(const AbsWalkArgs& a, int* qb, hipStream_t st) {
    return query_bounds(a.ks, a.qs, qb, a.qshift, a.P * a.D, a.Ns, a.Mq, a.C, st);
}

}  // namespace qlka
