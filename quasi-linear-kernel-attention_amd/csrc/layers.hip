// Fused epilogues of the three additive-kernel attention layers around the operators
// (Experiments/kernel_attention/attention.py:67-92, the branch attention.py:119-125 takes for add_laplace,
// add_riesz and add_bump):
//
//   add_laplace:  out = w / clamp(u - n_pad * sum_d e^{-|q_d|}, CLAMP)                       (attention.py:67-72)
//   add_riesz:    num = (|q|_1 + EPS) * sum_n v_n + sum_n |k_n|_1 v_n - w
//                 den = (|q|_1 + EPS) * S + sum_n |k_n|_1 - u - EPS * n_pad,  out = num / clamp(den, CLAMP)
//                                                                                            (attention.py:75-81)
//   add_bump:     num = (w+ + w-) / 2 - w0,  den = (u+ + u-) / 2 - u0 - n_pad * sum_d max(0, 1 - |q_d|)
//                 out = num / clamp(den, CLAMP), with (w, u) of the abs op at q, q + 1 and q - 1  (attention.py:84-92)
//
// with CLAMP = 1e-6 (attention.py:20), EPS = 1e-3 (kernels.py:9) and S = q.shape[2] (the number of queries, as the
// reference writes it). Every expression keeps the reference's operation order in fp32. The per-query d-reductions
// (sum_d e^{-|q_d|}, |q|_1, sum_d max(0, 1 - |q_d|)) are computed once per query before the per-channel pass.
//
// Masked form (key mask applied inside the sums, attention.py:122-124 without materialising k * keep, v * keep): w
// and u then already run over the kept keys only, which is what the n_pad terms above remove from the reference's
// sums over zeroed keys (a zeroed key adds e^{-|q_d|}, |q_d| or max(0, 1 - |q_d|) per feature to u). So add_laplace
// and add_bump drop their n_pad term, and add_riesz, whose u lost n_pad |q|_1, keeps the reference's algebra as
//   den = (|q|_1 + EPS) * (S - n_pad) + sum_kept |k_n|_1 - u,  n_pad = N - #kept,
// with sum_n v and sum_n |k_n|_1 v_n over the kept keys. S - n_pad is an exact integer in fp32; written as
// (|q|_1 + EPS) S - n_pad (|q|_1 + EPS) it would be the difference of two products that cancel when most keys are
// masked (a short document in a long padded batch: 9240 - 9236 at S = 4200 with 2 kept keys, 1e-4 of den lost).
#include <algorithm>
#include <cfloat>

#include "qlka_common.h"
#include "qlka_internal.h"

namespace qlka {

constexpr int RZ_NB = 64;          // key chunks per p of the add_riesz prefix pass
constexpr int RZ_T = 256;          // threads per block of the layer kernels

static inline size_t al256(size_t x) { return (x + 255) & ~size_t(255); }

// pre layout: vsum (P, C) | akv (P, C) | sak (P) | npad (P) | partials (P, RZ_NB, 2C + 2)
size_t riesz_prefix_bytes(int P, int N, int C) {
    (void)N;
    return 2 * al256((size_t)P * C * 4) + 2 * al256((size_t)P * 4) + al256((size_t)P * RZ_NB * (2 * C + 2) * 4);
}

// One block per (p, key chunk): |k_n|_1 of the chunk's keys into LDS (0 for masked keys), then per channel the
// chunk's sum_n v and sum_n |k_n|_1 v over its kept keys (G = RZ_T / C row groups per channel, combined in LDS), the
// chunk's sum_n |k_n|_1 and its count of kept keys.
__global__ __launch_bounds__(RZ_T)
void riesz_partials(const float* __restrict__ k, const float* __restrict__ v, const uint8_t* __restrict__ keep,
                    float* __restrict__ part, const int D, const int N, const int C)
{
    __shared__ float aks[(131072 + RZ_NB - 1) / RZ_NB];
    __shared__ uint8_t kept[(131072 + RZ_NB - 1) / RZ_NB];
    __shared__ float red[2][RZ_T];
    const int p = blockIdx.x / RZ_NB, b = blockIdx.x - p * RZ_NB, tid = threadIdx.x;
    const int chunk = (N + RZ_NB - 1) / RZ_NB;
    const int n0 = min(N, b * chunk), n1 = min(N, n0 + chunk);
    const float* kp = k + (size_t)p * D * N;
    float sak = 0.f, cnt = 0.f;
    for (int n = n0 + tid; n < n1; n += RZ_T) {
        const bool kn = !keep || keep[(size_t)p * N + n] != 0;
        float a = 0.f;
        if (kn) {
#pragma unroll 16
            for (int d = 0; d < D; ++d) a += fabsf(kp[(size_t)d * N + n]);
        }
        aks[n - n0] = a;
        kept[n - n0] = kn;
        sak += a;
        cnt += kn ? 1.f : 0.f;
    }
    __syncthreads();
    const int G = RZ_T / C;                               // >= 2 for C <= 128
    const int c = tid % C, rg = tid / C;
    float sv = 0.f, skv = 0.f;
    if (rg < G) {
        const float* vp = v + (size_t)p * N * C;
#pragma unroll 8
        for (int n = n0 + rg; n < n1; n += G) {
            if (!kept[n - n0]) continue;
            const float x = vp[(size_t)n * C + c];
            sv += x;
            skv += aks[n - n0] * x;
        }
    }
    red[0][tid] = sv;
    red[1][tid] = skv;
    __syncthreads();
    float* out = part + ((size_t)p * RZ_NB + b) * (2 * C + 2);
    if (tid < C) {
        float a0 = 0.f, a1 = 0.f;
        for (int r = 0; r < G; ++r) { a0 += red[0][r * C + tid]; a1 += red[1][r * C + tid]; }
        out[tid] = a0;
        out[C + tid] = a1;
    }
    __syncthreads();
    red[0][tid] = sak;
    red[1][tid] = cnt;
    __syncthreads();
    for (int off = RZ_T / 2; off >= 1; off >>= 1) {
        if (tid < off) { red[0][tid] += red[0][tid + off]; red[1][tid] += red[1][tid + off]; }
        __syncthreads();
    }
    if (tid == 0) { out[2 * C] = red[0][0]; out[2 * C + 1] = red[1][0]; }
}

// Chunk partials summed in chunk order (deterministic): one thread per (p, j), j < 2C + 2; npad = N - kept keys.
__global__ __launch_bounds__(RZ_T)
void riesz_finish(const float* __restrict__ part, float* __restrict__ vsum, float* __restrict__ akv,
                  float* __restrict__ sak, float* __restrict__ npad, const int P, const int N, const int C)
{
    const int W = 2 * C + 2;
    const int i = blockIdx.x * RZ_T + threadIdx.x;
    if (i >= P * W) return;
    const int p = i / W, j = i - p * W;
    float a = 0.f;
    for (int b = 0; b < RZ_NB; ++b) a += part[((size_t)p * RZ_NB + b) * W + j];
    if (j < C) vsum[(size_t)p * C + j] = a;
    else if (j < 2 * C) akv[(size_t)p * C + (j - C)] = a;
    else if (j == 2 * C) sak[p] = a;
    else npad[p] = (float)N - a;
}

int riesz_prefix(const float* k, const float* v, const uint8_t* keep, void* pre, int P, int D, int N, int C,
                 hipStream_t st) {
    char* b = (char*)pre;
    float* vsum = (float*)b;  b += al256((size_t)P * C * 4);
    float* akv = (float*)b;   b += al256((size_t)P * C * 4);
    float* sak = (float*)b;   b += al256((size_t)P * 4);
    float* npad = (float*)b;  b += al256((size_t)P * 4);
    float* part = (float*)b;
    StageTimer t("riesz_prefix", st);
    hipLaunchKernelGGL(riesz_partials, dim3((unsigned)(P * RZ_NB)), dim3(RZ_T), 0, st, k, v, keep, part, D, N, C);
    const int n = P * (2 * C + 2);
    hipLaunchKernelGGL(riesz_finish, dim3((unsigned)((n + RZ_T - 1) / RZ_T)), dim3(RZ_T), 0, st, part, vsum, akv, sak,
                       npad, P, N, C);
    return (int)hipGetLastError();
}

// Masked keys of the Laplace layer: out[p][d][n] = k[p][d][n] if keep[p][n], else FLT_MAX. Every Laplace term of
// such a key, e^{-(FLT_MAX - x)} for any query or key x below FLT_MAX, is exactly 0, two of them are FLT_MAX apart by 0
// (no inf - inf), and they sort after every kept key, so the unmasked walk over these keys gives the sums over the
// kept keys exactly. Grid: x over chunks of n, y (strided) over the P*D rows; no division per element.
__global__ __launch_bounds__(RZ_T)
void mask_keys_kernel(const float* __restrict__ k, const uint8_t* __restrict__ keep, float* __restrict__ out,
                      const int D, const int N, const int PD)
{
    const int n = blockIdx.x * RZ_T + threadIdx.x;
    if (n >= N) return;
    for (int pd = blockIdx.y; pd < PD; pd += gridDim.y) {
        const size_t i = (size_t)pd * N + n;
        out[i] = keep[(size_t)(pd / D) * N + n] ? k[i] : FLT_MAX;
    }
}

// The same four keys at a time (N % 4 == 0, 16-byte aligned k and out, 4-byte aligned keep).
__global__ __launch_bounds__(RZ_T)
void mask_keys_kernel4(const float4* __restrict__ k, const uchar4* __restrict__ keep, float4* __restrict__ out,
                       const int D, const int N4, const int PD)
{
    const int n = blockIdx.x * RZ_T + threadIdx.x;
    if (n >= N4) return;
    for (int pd = blockIdx.y; pd < PD; pd += gridDim.y) {
        const size_t i = (size_t)pd * N4 + n;
        const uchar4 kp = keep[(size_t)(pd / D) * N4 + n];
        const float4 x = k[i];
        out[i] = make_float4(kp.x ? x.x : FLT_MAX, kp.y ? x.y : FLT_MAX, kp.z ? x.z : FLT_MAX, kp.w ? x.w : FLT_MAX);
    }
}

int mask_keys(const float* k, const uint8_t* keep, float* out, int P, int D, int N, hipStream_t st) {
    const int PD = P * D;
    StageTimer t("mask_keys", st);
    const bool v4 = N % 4 == 0 && ((uintptr_t)k & 15) == 0 && ((uintptr_t)out & 15) == 0 && ((uintptr_t)keep & 3) == 0;
    if (v4)
        hipLaunchKernelGGL(mask_keys_kernel4,
                           dim3((unsigned)((N / 4 + RZ_T - 1) / RZ_T), (unsigned)std::min(PD, 65535)), dim3(RZ_T), 0,
                           st, (const float4*)k, (const uchar4*)keep, (float4*)out, D, N / 4, PD);
    else
        hipLaunchKernelGGL(mask_keys_kernel, dim3((unsigned)((N + RZ_T - 1) / RZ_T), (unsigned)std::min(PD, 65535)),
                           dim3(RZ_T), 0, st, k, keep, out, D, N, PD);
    return (int)hipGetLastError();
}

// The sorted keys of a masked abs walk, in place: a masked key takes the value of the last kept key before it in the
// sorted order; masked keys before the first kept key (and every key of a segment with none kept) keep their own. The
// order stays ascending and every distance the walk measures between consecutive keys, from the last key below a query
// and from the largest key (the segment totals -Btot - (q - k_max) Wtot) runs between kept keys: masked keys, weighing 0
// in every sum, become transparent. Without this, the totals of a segment whose largest key is masked and far above
// the kept ones cancel quantities of size (k_max - k_n) |w_n| far larger than the kept keys' own terms.
// One workgroup of FM_T threads per segment; each thread takes FM_I consecutive keys of a piece, and the last kept
// value carries across threads (a wave scan, then the waves' totals through LDS) and across pieces.
constexpr int FM_T = 1024, FM_I = 16;
__global__ __launch_bounds__(FM_T)
void fill_masked_keys_kernel(float* __restrict__ ks, const uint32_t* __restrict__ kp, const uint8_t* __restrict__ keep,
                             const int D, const int N)
{
    __shared__ float wval[FM_T / WAVE];
    __shared__ int whave[FM_T / WAVE];
    const int s = blockIdx.x, p = s / D, t = threadIdx.x, lane = t & (WAVE - 1), w = t / WAVE;
    float* seg = ks + (size_t)s * N;
    const uint32_t* pseg = kp + (size_t)s * N;
    const uint8_t* kk = keep + (size_t)p * N;
    float carry = 0.f;
    int have_carry = 0;
    for (int base = 0; base < N; base += FM_T * FM_I) {
        const int i0 = base + t * FM_I;
        float x[FM_I];
        bool kept[FM_I];
#pragma unroll
        for (int j = 0; j < FM_I; ++j) {
            const int i = min(i0 + j, N - 1);             // clamped: unconditional loads
            x[j] = seg[i];
            kept[j] = i0 + j < N && kk[pseg[i]] != 0;
        }
        // this thread's last kept value, then the last kept value before this thread (exclusive scan)
        float tv = 0.f;
        int th = 0;
#pragma unroll
        for (int j = 0; j < FM_I; ++j)
            if (kept[j]) { tv = x[j]; th = 1; }
        float iv = tv;
        int ih = th;
#pragma unroll
        for (int off = 1; off < WAVE; off <<= 1) {
            const float uv = __shfl_up(iv, off, WAVE);
            const int uh = __shfl_up(ih, off, WAVE);
            if (lane >= off && !ih) { iv = uv; ih = uh; }
        }
        if (lane == WAVE - 1) { wval[w] = iv; whave[w] = ih; }
        // both shuffles unconditional: a cross-lane read inside a lane-dependent branch reads 0 from inactive lanes
        float ev = __shfl_up(iv, 1, WAVE);
        const int eh_up = __shfl_up(ih, 1, WAVE);
        int eh = lane > 0 ? eh_up : 0;
        __syncthreads();
        float pv = carry;                                 // before this wave: earlier pieces, then earlier waves
        int ph = have_carry;
        for (int ww = 0; ww < w; ++ww)
            if (whave[ww]) { pv = wval[ww]; ph = 1; }
        if (!eh) { ev = pv; eh = ph; }
        // the piece's last kept value carries to the next piece
        for (int ww = 0; ww < FM_T / WAVE; ++ww)
            if (whave[ww]) { carry = wval[ww]; have_carry = 1; }
#pragma unroll
        for (int j = 0; j < FM_I; ++j) {
            if (kept[j]) { ev = x[j]; eh = 1; }
            else if (eh) x[j] = ev;
        }
#pragma unroll
        for (int j = 0; j < FM_I; ++j)
            if (i0 + j < N) seg[i0 + j] = x[j];
        __syncthreads();                                  // the wave totals are read before the next piece's
    }
}

int fill_masked_keys(float* ks, const uint32_t* kp, const uint8_t* keep, int P, int D, int N, hipStream_t st) {
    StageTimer t("fill_masked_keys", st);
    hipLaunchKernelGGL(fill_masked_keys_kernel, dim3((unsigned)(P * D)), dim3(FM_T), 0, st, ks, kp, keep, D, N);
    return (int)hipGetLastError();
}

// Per (p, m): the reduction over d of the layer's query-only term (e^{-|q|}, |q| or max(0, 1 - |q|)); one thread per
// query, d in order, coalesced across m.
template <int KIND>
__global__ __launch_bounds__(RZ_T)
void layer_query_terms(const float* __restrict__ q, float* __restrict__ qt, const int P, const int D, const int M)
{
    const long i = (long)blockIdx.x * RZ_T + threadIdx.x;
    if (i >= (long)P * M) return;
    const int p = (int)(i / M), m = (int)(i - (long)p * M);
    const float* qc = q + (size_t)p * D * M + m;
    float a = 0.f;
#pragma unroll 16
    for (int d = 0; d < D; ++d) {
        const float x = fabsf(qc[(size_t)d * M]);
        if constexpr (KIND == LAYER_ADD_LAPLACE) a += expf(-x);
        else if constexpr (KIND == LAYER_ADD_RIESZ) a += x;
        else a += fmaxf(1.f - x, 0.f);
    }
    qt[i] = a;
}

// Every channel of the output rows: one thread per (p, m, c). MASKED: w and u are sums over the kept keys (n_pad then
// only enters add_riesz's count term).
template <int KIND, bool MASKED>
__global__ __launch_bounds__(RZ_T)
void layer_epilogue_kernel(const float* __restrict__ qt, const float* __restrict__ n_pad,
                           const float* __restrict__ w0, const float* __restrict__ u0,
                           const float* __restrict__ wp, const float* __restrict__ up,
                           const float* __restrict__ wm, const float* __restrict__ um,
                           const float* __restrict__ vsum, const float* __restrict__ akv, const float* __restrict__ sak,
                           float* __restrict__ out, const int P, const int M, const int C)
{
    const long i = (long)blockIdx.x * RZ_T + threadIdx.x;
    if (i >= (long)P * M * C) return;
    const long pm = i / C;
    const int c = (int)(i - pm * C);
    const int p = (int)(pm / M);
    const float np = n_pad ? n_pad[p] : 0.f;
    float num, den;
    if constexpr (KIND == LAYER_ADD_LAPLACE) {
        num = w0[i];
        den = MASKED ? u0[pm] : u0[pm] - np * qt[pm];
    } else if constexpr (KIND == LAYER_ADD_RIESZ) {
        const float aqe = qt[pm] + LAYER_EPS;
        num = aqe * vsum[(size_t)p * C + c] + akv[(size_t)p * C + c] - w0[i];
        den = MASKED ? aqe * ((float)M - np) + sak[p] - u0[pm]
                     : aqe * (float)M + sak[p] - u0[pm] - LAYER_EPS * np;
    } else {
        num = (wp[i] + wm[i]) / 2.f - w0[i];
        den = MASKED ? (up[pm] + um[pm]) / 2.f - u0[pm] : (up[pm] + um[pm]) / 2.f - u0[pm] - np * qt[pm];
    }
    out[i] = num / fmaxf(den, LAYER_CLAMP);
}

int layer_epilogue_params(int kind, bool masked, const float* q, const float* n_pad, const void* pre, float* qt,
                          float* out, int P, int D, int M, int C, ReduceEpilogue* ep, hipStream_t st) {
    ep->vsum = ep->akv = ep->sak = nullptr;
    if (kind == LAYER_ADD_RIESZ) {
        const char* b = (const char*)pre;
        ep->vsum = (const float*)b;  b += al256((size_t)P * C * 4);
        ep->akv = (const float*)b;   b += al256((size_t)P * C * 4);
        ep->sak = (const float*)b;   b += al256((size_t)P * 4);
        if (masked) n_pad = (const float*)b;              // N - kept keys, from riesz_prefix
    }
    if (masked && kind != LAYER_ADD_RIESZ) n_pad = nullptr;
    ep->n_pad = n_pad; ep->qt = qt; ep->out = out;
    const long nq = (long)P * M;
    const unsigned qblocks = (unsigned)((nq + RZ_T - 1) / RZ_T);
    StageTimer t("layer_query_terms", st);
    if (kind == LAYER_ADD_LAPLACE)
        hipLaunchKernelGGL(layer_query_terms<LAYER_ADD_LAPLACE>, dim3(qblocks), dim3(RZ_T), 0, st, q, qt, P, D, M);
    else if (kind == LAYER_ADD_RIESZ)
        hipLaunchKernelGGL(layer_query_terms<LAYER_ADD_RIESZ>, dim3(qblocks), dim3(RZ_T), 0, st, q, qt, P, D, M);
    else if (kind == LAYER_ADD_BUMP)
        hipLaunchKernelGGL(layer_query_terms<LAYER_ADD_BUMP>, dim3(qblocks), dim3(RZ_T), 0, st, q, qt, P, D, M);
    else
        return (int)hipErrorInvalidValue;
    return (int)hipGetLastError();
}

int layer_epilogue(int kind, bool masked, const float* q, const float* n_pad, const float* w0, const float* u0,
                   const float* wp, const float* up, const float* wm, const float* um, const void* pre, float* qt,
                   float* out, int P, int D, int N, int M, int C, hipStream_t st) {
    const float *vsum = nullptr, *akv = nullptr, *sak = nullptr;
    if (kind == LAYER_ADD_RIESZ) {
        const char* b = (const char*)pre;
        vsum = (const float*)b;  b += al256((size_t)P * C * 4);
        akv = (const float*)b;   b += al256((size_t)P * C * 4);
        sak = (const float*)b;   b += al256((size_t)P * 4);
        if (masked) n_pad = (const float*)b;              // N - kept keys, from riesz_prefix
    }
    if (masked && kind != LAYER_ADD_RIESZ) n_pad = nullptr;
    (void)N;
    const long nq = (long)P * M, n = nq * C;
    const unsigned qblocks = (unsigned)((nq + RZ_T - 1) / RZ_T), blocks = (unsigned)((n + RZ_T - 1) / RZ_T);
    StageTimer t("layer_epilogue", st);
#define QLKA_LAYER_LAUNCH(K)                                                                                        \
    hipLaunchKernelGGL(layer_query_terms<K>, dim3(qblocks), dim3(RZ_T), 0, st, q, qt, P, D, M);                    \
    if (masked)                                                                                                     \
        hipLaunchKernelGGL((layer_epilogue_kernel<K, true>), dim3(blocks), dim3(RZ_T), 0, st, qt, n_pad, w0, u0, wp,  \
                           up, wm, um, vsum, akv, sak, out, P, M, C);                                               \
    else                                                                                                            \
        hipLaunchKernelGGL((layer_epilogue_kernel<K, false>), dim3(blocks), dim3(RZ_T), 0, st, qt, n_pad, w0, u0, wp, \
                           up, wm, um, vsum, akv, sak, out, P, M, C)
    switch (kind) {
        case LAYER_ADD_LAPLACE: QLKA_LAYER_LAUNCH(LAYER_ADD_LAPLACE); break;
        case LAYER_ADD_RIESZ:   QLKA_LAYER_LAUNCH(LAYER_ADD_RIESZ); break;
        case LAYER_ADD_BUMP:    QLKA_LAYER_LAUNCH(LAYER_ADD_BUMP); break;
        default: return (int)hipErrorInvalidValue;
    }
#undef QLKA_LAYER_LAUNCH
    return (int)hipGetLastError();
}

}  // namespace qlka
