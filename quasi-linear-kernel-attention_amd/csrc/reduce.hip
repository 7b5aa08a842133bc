// D-reduction of the per-feature contributions (the last step of stage 4).
//
// The walks leave one contribution row per (p, d, query) in a slab (row stride slab_stride(C), whole 128-byte lines;
// blocked by 64 queries within pairs of features, see slab_group), written with plain row stores. Summing over the
// D features of a p here reads, per block of 64 queries, G * 64 contiguous rows per feature group, so the D-fold
// accumulation costs one HBM write and one HBM read per contribution instead of one fp32 atomic per channel (the L2
// atomic units of the chip sustain about one 4-byte atomic per channel per clock, which bounds an atomic emission at
// P*D*M*C atomics well above the slab's traffic time).
//
// The v == 1 sums (out_u) are one scalar per (p, d, query). For segments of up to U_LDS_CAP queries the walks write
// them in sorted-query order (coalesced) and u_to_query puts each segment's scalars in query order through LDS
// (coalesced reads of them and of the sort's permutation, coalesced writes); longer segments arrive in query order.
// The reduce then sums them like the slab rows.
#include "qlka_common.h"
#include "qlka_internal.h"

namespace qlka {

constexpr int RT = 256;        // threads per block

// uq[s][qperm[s][i]] = uslab[s][i] for every segment s (M <= U_LDS_CAP): one workgroup per segment, through LDS.
// Up to three sets of terms sorted alike (add_bump's q, q + 1, q - 1) go in one launch: the workgroup of a segment
// reads the permutation once and all sets' terms at once, then moves the sets through LDS one after another.
constexpr int UT_T = 1024;
struct USets { const float* uslab[3]; float* uq[3]; };
__global__ __launch_bounds__(UT_T)
void u_to_query(const USets sets, const int nsets, const uint32_t* __restrict__ qperm, const int M)
{
    constexpr int UT_I = U_LDS_CAP / UT_T;          // items per thread; all of a thread's loads are issued at once
    __shared__ float buf[U_LDS_CAP];
    const size_t base = (size_t)blockIdx.x * M;
    const int tid = threadIdx.x;
    float x[3][UT_I];
    uint32_t dst[UT_I];
#pragma unroll
    for (int j = 0; j < UT_I; ++j) {
        const int i = min(tid + j * UT_T, M - 1);     // clamped: unconditional loads
        dst[j] = qperm[base + i];
#pragma unroll
        for (int set = 0; set < 3; ++set)
            x[set][j] = set < nsets ? sets.uslab[set][base + i] : 0.f;
    }
#pragma unroll
    for (int set = 0; set < 3; ++set) {
        if (set >= nsets) break;
        if (set > 0) __syncthreads();                 // the previous set's reads of buf are done
#pragma unroll
        for (int j = 0; j < UT_I; ++j)
            if (tid + j * UT_T < M) buf[dst[j]] = x[set][j];
        __syncthreads();
        float* __restrict__ uq = sets.uq[set];
#pragma unroll
        for (int j = 0; j < UT_I; ++j) {
            const int i = tid + j * UT_T;
            if (i < M) uq[base + i] = buf[i];
        }
    }
}

__global__ __launch_bounds__(RT)
void u_sum(const float* __restrict__ uq, float* __restrict__ out_u, const int P, const int D, const int M)
{
    const long i = (long)blockIdx.x * RT + threadIdx.x;
    if (i >= (long)P * M) return;
    const int p = (int)(i / M);
    const int m = (int)(i - (long)p * M);
    const float* src = uq + (size_t)p * D * M + m;
    float u = 0.f;
#pragma unroll 8
    for (int d = 0; d < D; ++d) u += src[(size_t)d * M];
    out_u[i] = u;
}

// One thread per (p, m, 4 channels) (V4, C % 4 == 0) or per (p, m, channel); features summed in order d = 0..D-1.
// With WITH_U (V4 and C / 4 a power of two, so the C / 4 lanes of one query row are aligned within a wave) the row's
// lanes also produce out_u: lane j sums features d = j, j + C/4, ... of the v == 1 contributions (query order) and the
// partial sums are combined with lane shuffles (fixed order, deterministic).
// EPI (with WITH_U): the add_laplace (LAYER_ADD_LAPLACE) or add_riesz (LAYER_ADD_RIESZ) epilogue on the row's w and u,
// written to ep.out instead of out / out_u (the same arithmetic as layer_epilogue_kernel); EPI < 0: none.
template <bool V4, bool WITH_U, int EPI = -1, bool MASKED = false>
__global__ __launch_bounds__(RT)
void slab_reduce(const float* __restrict__ slab, float* __restrict__ out, const int P, const int D, const int M,
                 const int C, const int CR, const float* __restrict__ uq, float* __restrict__ out_u,
                 const ReduceEpilogue ep = ReduceEpilogue{})
{
    const int CQ = V4 ? C / 4 : C;
    const long i = (long)blockIdx.x * RT + threadIdx.x;
    if (i >= (long)P * M * CQ) return;                 // WITH_U: P*M*CQ is a multiple of CQ, so whole rows return
    const int c = (int)(i % CQ);
    const long pm = i / CQ;
    const int p = (int)(pm / M);
    const int m = (int)(pm - (long)p * M);
    // rows of query m, d = 0 .. D-1 in order: groups of G features, SLAB_QB * CR floats between features of a group
    const int G = slab_group(D);
    const size_t gstride = (size_t)G * slab_rows(M) * CR;
    const size_t fstride = (size_t)SLAB_QB * CR;
    const float* src = slab + (size_t)p * D * slab_rows(M) * CR + (size_t)slab_row_off(m, G, CR) / 4;
    if constexpr (V4) {
        typedef float f4 __attribute__((ext_vector_type(4)));
        f4 a = {0.f, 0.f, 0.f, 0.f};
        for (int g0 = 0; g0 < D; g0 += G) {
            const f4* s4 = reinterpret_cast<const f4*>(src + (size_t)(g0 / G) * gstride) + c;
#pragma unroll 8
            for (int dd = 0; dd < G; ++dd) a += __builtin_nontemporal_load(s4 + (size_t)dd * (fstride / 4));
        }
        if constexpr (EPI < 0) reinterpret_cast<f4*>(out + pm * C)[c] = a;
        if constexpr (WITH_U) {
            const float* us = uq + (size_t)p * D * M + m;
            float u = 0.f;
            for (int d = c; d < D; d += CQ) u += us[(size_t)d * M];
            for (int off = CQ >> 1; off >= 1; off >>= 1) u += __shfl_xor(u, off, WAVE);
            if constexpr (EPI >= 0) {
                const float np = ep.n_pad ? ep.n_pad[p] : 0.f;
                const float qv = ep.qt[pm];
                f4 o;
                if constexpr (EPI == LAYER_ADD_LAPLACE) {
                    const float den = fmaxf(MASKED ? u : u - np * qv, LAYER_CLAMP);
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[e] = a[e] / den;
                } else {
                    const float aqe = qv + LAYER_EPS;
                    const float den = fmaxf(MASKED ? aqe * ((float)M - np) + ep.sak[p] - u
                                                   : aqe * (float)M + ep.sak[p] - u - LAYER_EPS * np, LAYER_CLAMP);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const size_t pc = (size_t)p * C + 4 * c + e;
                        o[e] = (aqe * ep.vsum[pc] + ep.akv[pc] - a[e]) / den;
                    }
                }
                reinterpret_cast<f4*>(ep.out + pm * C)[c] = o;
                return;
            }
            if (c == 0) out_u[pm] = u;
        }
    } else {
        float a = 0.f;
        for (int g0 = 0; g0 < D; g0 += G) {
            const float* sg = src + (size_t)(g0 / G) * gstride + c;
#pragma unroll 8
            for (int dd = 0; dd < G; ++dd) a += sg[(size_t)dd * fstride];
        }
        out[pm * C + c] = a;
    }
}

int reduce_slabs(const float* slab, const float* uslab, const uint32_t* qperm, float* uq, float* out, float* out_u,
                 int P, int D, int M, int C, hipStream_t st) {
    const int CR = slab_stride(C);
    const bool v4 = (C % 4) == 0;
    const int cq = C / 4;
    const bool fused_u = out_u && v4 && (cq & (cq - 1)) == 0;     // row lanes aligned within a wave
    if (out_u && qperm && !u_query_order(M)) {
        order_u_terms_sets(&uslab, qperm, &uq, 1, P, D, M, st);
    } else if (out_u) {
        uq = const_cast<float*>(uslab);                   // already in query order
    }
    if (out_u && !fused_u) {
        StageTimer t("u_sum", st);
        const long n = (long)P * M;
        hipLaunchKernelGGL(u_sum, dim3((unsigned)((n + RT - 1) / RT)), dim3(RT), 0, st, uq, out_u, P, D, M);
    }
    const long threads = (long)P * M * (v4 ? C / 4 : C);
    const unsigned blocks = (unsigned)((threads + RT - 1) / RT);
    StageTimer t("slab_reduce", st);
    if (fused_u)
        hipLaunchKernelGGL((slab_reduce<true, true>), dim3(blocks), dim3(RT), 0, st, slab, out, P, D, M, C, CR, uq,
                           out_u);
    else if (v4)
        hipLaunchKernelGGL((slab_reduce<true, false>), dim3(blocks), dim3(RT), 0, st, slab, out, P, D, M, C, CR,
                           nullptr, nullptr);
    else
        hipLaunchKernelGGL((slab_reduce<false, false>), dim3(blocks), dim3(RT), 0, st, slab, out, P, D, M, C, CR,
                           nullptr, nullptr);
    return (int)hipGetLastError();
}

}  // namespace qlka

namespace qlka {

// add_bump in one pass: the three slabs of the abs sums at q, q + 1 and q - 1 (one walk over the three query sets) and
// their v == 1 terms (query order), each summed over d = 0..D-1 exactly as slab_reduce<true, true> sums one, then the
// bump epilogue of layer_epilogue_kernel on the three sums: num = (w+ + w-) / 2 - w0, den = (u+ + u-) / 2 - u0
// (- n_pad * sum_d max(0, 1 - |q_d|) unmasked), out = num / max(den, clamp). One thread per (p, m, 4 channels);
// C / 4 a power of two.
template <bool MASKED>
__global__ __launch_bounds__(RT)
void slab_reduce_bump(const float* __restrict__ s0, const float* __restrict__ sp, const float* __restrict__ sm,
                      const float* __restrict__ u0q, const float* __restrict__ upq, const float* __restrict__ umq,
                      const ReduceEpilogue ep, const int P, const int D, const int M, const int C, const int CR)
{
    typedef float f4 __attribute__((ext_vector_type(4)));
    const int CQ = C / 4;
    const long i = (long)blockIdx.x * RT + threadIdx.x;
    if (i >= (long)P * M * CQ) return;                 // P*M*CQ is a multiple of CQ: whole rows return
    const int c = (int)(i % CQ);
    const long pm = i / CQ;
    const int p = (int)(pm / M);
    const int m = (int)(pm - (long)p * M);
    const int G = slab_group(D);
    const size_t gstride = (size_t)G * slab_rows(M) * CR;
    const size_t fstride = (size_t)SLAB_QB * CR;
    const size_t off = (size_t)p * D * slab_rows(M) * CR + (size_t)slab_row_off(m, G, CR) / 4;
    f4 a0 = {0.f, 0.f, 0.f, 0.f}, ap = a0, am = a0;
    // 4 feature groups of loads in flight per thread (12 16-byte loads): 4.38 -> 4.34 ms per add_bump call
#pragma unroll 4
    for (int g0 = 0; g0 < D; g0 += G) {
        const size_t go = off + (size_t)(g0 / G) * gstride;
        const f4* r0 = reinterpret_cast<const f4*>(s0 + go) + c;
        const f4* rp = reinterpret_cast<const f4*>(sp + go) + c;
        const f4* rm = reinterpret_cast<const f4*>(sm + go) + c;
#pragma unroll 4
        for (int dd = 0; dd < G; ++dd) {
            const size_t o = (size_t)dd * (fstride / 4);
            a0 += __builtin_nontemporal_load(r0 + o);
            ap += __builtin_nontemporal_load(rp + o);
            am += __builtin_nontemporal_load(rm + o);
        }
    }
    const size_t ub = (size_t)p * D * M + m;
    float u0 = 0.f, up = 0.f, um = 0.f;
    for (int d = c; d < D; d += CQ) {
        u0 += u0q[ub + (size_t)d * M];
        up += upq[ub + (size_t)d * M];
        um += umq[ub + (size_t)d * M];
    }
    for (int o = CQ >> 1; o >= 1; o >>= 1) {
        u0 += __shfl_xor(u0, o, WAVE);
        up += __shfl_xor(up, o, WAVE);
        um += __shfl_xor(um, o, WAVE);
    }
    const float np = ep.n_pad ? ep.n_pad[p] : 0.f;
    const float den = MASKED ? (up + um) / 2.f - u0 : (up + um) / 2.f - u0 - np * ep.qt[pm];
    f4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = ((ap[e] + am[e]) / 2.f - a0[e]) / fmaxf(den, LAYER_CLAMP);
    reinterpret_cast<f4*>(ep.out + pm * C)[c] = o;
}

int reduce_slabs_bump(bool masked, const ReduceEpilogue& ep, const float* const slab[3], const float* const uq[3],
                      int P, int D, int M, int C, hipStream_t st) {
    if (!reduce_folds_epilogue(M, C)) return (int)hipErrorInvalidValue;
    const int CR = slab_stride(C);
    const long threads = (long)P * M * (C / 4);
    const unsigned blocks = (unsigned)((threads + RT - 1) / RT);
    StageTimer t("slab_reduce", st);
    if (masked)
        hipLaunchKernelGGL(slab_reduce_bump<true>, dim3(blocks), dim3(RT), 0, st, slab[0], slab[1], slab[2], uq[0],
                           uq[1], uq[2], ep, P, D, M, C, CR);
    else
        hipLaunchKernelGGL(slab_reduce_bump<false>, dim3(blocks), dim3(RT), 0, st, slab[0], slab[1], slab[2], uq[0],
                           uq[1], uq[2], ep, P, D, M, C, CR);
    return (int)hipGetLastError();
}

const float* order_u_terms(const float* uslab, const uint32_t* qperm, float* uq, int P, int D, int M, hipStream_t st) {
    const float* u[1] = {uslab};
    float* q[1] = {uq};
    order_u_terms_sets(u, qperm, q, 1, P, D, M, st);
    return u_query_order(M) ? uslab : uq;
}

void order_u_terms_sets(const float* const* uslab, const uint32_t* qperm, float* const* uq, int nsets, int P, int D,
                        int M, hipStream_t st) {
    if (u_query_order(M) || nsets < 1 || nsets > 3) return;
    USets sets{};
    for (int i = 0; i < nsets; ++i) { sets.uslab[i] = uslab[i]; sets.uq[i] = uq[i]; }
    StageTimer t("u_to_query", st);
    hipLaunchKernelGGL(u_to_query, dim3((unsigned)(P * D)), dim3(UT_T), 0, st, sets, nsets, qperm, M);
}

bool reduce_folds_epilogue(int M, int C) {
    const int cq = C / 4;
    return C % 4 == 0 && (cq & (cq - 1)) == 0;
}

int reduce_slabs_layer(int kind, bool masked, const ReduceEpilogue& ep, const float* slab, const float* uslab,
                       const uint32_t* qperm, float* uq, int P, int D, int M, int C, hipStream_t st) {
    if (!reduce_folds_epilogue(M, C) || (kind != LAYER_ADD_LAPLACE && kind != LAYER_ADD_RIESZ))
        return (int)hipErrorInvalidValue;
    const int CR = slab_stride(C);
    if (qperm && !u_query_order(M)) {
        order_u_terms_sets(&uslab, qperm, &uq, 1, P, D, M, st);
    } else {
        uq = const_cast<float*>(uslab);                   // already in query order
    }
    const long threads = (long)P * M * (C / 4);
    const unsigned blocks = (unsigned)((threads + RT - 1) / RT);
    StageTimer t("slab_reduce", st);
#define QLKA_REDUCE_EPI(K, MK) \
    hipLaunchKernelGGL((slab_reduce<true, true, K, MK>), dim3(blocks), dim3(RT), 0, st, slab, nullptr, P, D, M, C, CR, \
                       uq, nullptr, ep)
    if (kind == LAYER_ADD_LAPLACE) {
        if (masked) QLKA_REDUCE_EPI(LAYER_ADD_LAPLACE, true);
        else QLKA_REDUCE_EPI(LAYER_ADD_LAPLACE, false);
    } else {
        if (masked) QLKA_REDUCE_EPI(LAYER_ADD_RIESZ, true);
        else QLKA_REDUCE_EPI(LAYER_ADD_RIESZ, false);
    }
#undef QLKA_REDUCE_EPI
    return (int)hipGetLastError();
}

}  // namespace qlka
