// Direct (dense) evaluation for short segments, the role the reference gives pykeops below KEOPS_CUTOFF
// (Weighted_Abs_Sum/weighted_abs_sum/keops_backend.py:19-35: A_mn = sum_d |q_dm - k_dn| reduced against [v, 1] in
// one pass) and for the Laplace sum at small N (the dense formula of Experiments/kernel_attention/kernels.py:81):
//
//   A[m, n] = sum_d f(q[d, m] - k[d, n]),  f = |x| (abs) or e^{-|x|} (Laplace)
//   out_w[m, :] = sum_n A[m, n] v[n, :],   out_u[m] = sum_n A[m, n]
//
// One workgroup per (p, tile of 64 queries) walks the keys in tiles of 64. Per key tile, q and k columns and the v
// rows are staged in LDS; each of the 256 threads accumulates a 4 x 4 block of A over d (q and k values read as
// 16-byte broadcasts), the A tile goes to LDS, and each thread then accumulates a 4-query x CT-channel block of
// A v and the row sums. Nothing is sorted, so no workspace: below a few hundred keys this beats the sort + scan
// pipeline, whose cost there is launch and per-segment overhead. All arithmetic is fp32, as in the dense and KeOps
// paths of the reference.
#include "qlka_common.h"
#include "qlka_internal.h"

namespace qlka {

constexpr int DT = 64;             // queries and keys per tile
constexpr int DTHREADS = 256;      // 16 x 16 threads
constexpr int DDK = 32;            // features staged per LDS round

template <int KIND, int CT>        // KIND 0: abs, 1: Laplace; CT channels per thread (4: C <= 64, 8: C <= 128)
__global__ __launch_bounds__(DTHREADS)
void direct_fwd_kernel(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
                       float* __restrict__ out_w, float* __restrict__ out_u,
                       const int D, const int N, const int M, const int C, const int mtiles)
{
    constexpr int CW = 16 * CT;                           // channels covered by the 16 thread columns
    __shared__ f4_t qs[DDK][DT / 4];                      // q[d][m0 .. m0+63]
    __shared__ f4_t ks[DDK][DT / 4];                      // k[d][n0 .. n0+63]
    __shared__ float at[DT][DT + 4];                      // A tile [m][n] (+4: no bank conflicts on columns)
    __shared__ float vs[DT][CW];                          // v rows of the key tile

    const int p = blockIdx.x / mtiles, mt = blockIdx.x - p * mtiles;
    const int m0 = mt * DT, tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
    const float* qp = q + (size_t)p * D * M;
    const float* kp = k + (size_t)p * D * N;
    const float* vp = v + (size_t)p * N * C;

    float acc[4][CT], usum[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        usum[i] = 0.f;
#pragma unroll
        for (int j = 0; j < CT; ++j) acc[i][j] = 0.f;
    }

    for (int n0 = 0; n0 < N; n0 += DT) {
        // ---- A tile: thread (ty, tx) owns queries m0 + 4 ty .. +3 and keys n0 + 4 tx .. +3
        float a[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) a[i][j] = 0.f;
        for (int d0 = 0; d0 < D; d0 += DDK) {
            __syncthreads();                              // previous readers of qs / ks are done
            for (int e = tid; e < DDK * DT; e += DTHREADS) {
                const int dd = e / DT, x = e - dd * DT, d = d0 + dd;
                const int m = m0 + x, n = n0 + x;
                // pads (past D, M or N) are never emitted: queries past M are not stored, keys past N weigh 0 below
                reinterpret_cast<float*>(qs[dd])[x] = (d < D && m < M) ? qp[(size_t)d * M + m] : 0.f;
                reinterpret_cast<float*>(ks[dd])[x] = (d < D && n < N) ? kp[(size_t)d * N + n] : 0.f;
            }
            __syncthreads();
            const int dn = min(DDK, D - d0);
            for (int dd = 0; dd < dn; ++dd) {
                const f4_t qv = qs[dd][ty], kv = ks[dd][tx];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float x = fabsf(qv[i] - kv[j]);
                        if constexpr (KIND == 0) a[i][j] += x;
                        else a[i][j] += __expf(-x);
                    }
            }
        }
        // keys past N contribute nothing
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (n0 + 4 * tx + j >= N) {
#pragma unroll
                for (int i = 0; i < 4; ++i) a[i][j] = 0.f;
            }
        __syncthreads();                                  // previous readers of at / vs are done
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) at[4 * ty + i][4 * tx + j] = a[i][j];
        for (int e = tid; e < DT * CW; e += DTHREADS) {
            const int r = e / CW, c = e - r * CW, n = n0 + r;
            vs[r][c] = (n < N && c < C) ? vp[(size_t)n * C + c] : 0.f;
        }
        __syncthreads();
        // ---- A v and row sums: thread (ty, tx) owns queries 4 ty .. +3 and channels CT tx .. +CT-1
        const int nn = min(DT, N - n0);
        for (int r = 0; r < nn; ++r) {
            float av[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) av[i] = at[4 * ty + i][r];
            float vv[CT];
#pragma unroll
            for (int j = 0; j < CT; ++j) vv[j] = vs[r][CT * tx + j];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                usum[i] += av[i];
#pragma unroll
                for (int j = 0; j < CT; ++j) acc[i][j] += av[i] * vv[j];
            }
        }
    }

#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + 4 * ty + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < CT; ++j) {
            const int c = CT * tx + j;
            if (c < C) out_w[((size_t)p * M + m) * C + c] = acc[i][j];
        }
        if (out_u != nullptr && tx == 0) out_u[(size_t)p * M + m] = usum[i];
    }
}

int direct_fwd(int kind, const float* q, const float* k, const float* v, float* out_w, float* out_u,
               int P, int D, int N, int M, int C, hipStream_t st) {
    const int mtiles = (M + DT - 1) / DT;
    const dim3 grid((unsigned)(P * mtiles)), block(DTHREADS);
    StageTimer t("direct_fwd", st);
#define QLKA_DIRECT(K, CTV) \
    hipLaunchKernelGGL((direct_fwd_kernel<K, CTV>), grid, block, 0, st, q, k, v, out_w, out_u, D, N, M, C, mtiles)
    if (kind == 0) { if (C <= 64) QLKA_DIRECT(0, 4); else QLKA_DIRECT(0, 8); }
    else           { if (C <= 64) QLKA_DIRECT(1, 4); else QLKA_DIRECT(1, 8); }
#undef QLKA_DIRECT
    return (int)hipGetLastError();
}

// Dense sign sums, the gradients of the dense abs sum (and weighted_sgn_sum):
//
//   out[d, i] = scale * sum_j s(a[d, i] - b[d, j]) * (<x[i, :], y[j, :]> + gu),   s(z) = sign(z), s(0) = tie
//
// with gu = g_u[i] (GU_OWN) or g_u[j] (otherwise), or 0 without g_u:
//   grad_q:  a = q, b = k, x = g_w, y = v, gu = g_u[m]  (own)
//   grad_k:  a = k, b = q, x = v, y = g_w, gu = g_u[m]  (other)
//   weighted_sgn_sum (KeOps convention): grad_q with g for g_w, no g_u, tie 0, scale -1 (keops_backend.py:38-48).
// tie = 0 is KeOps' sign(0) (keops_backend.py:40-41); tie = -1 is the reference CUDA walk's convention.
// One workgroup per (p, tile of 64 outputs i) walks the j in tiles of 64: the 64 x 64 tile of <x_i, y_j> + gu is
// formed 4 x 4 per thread from LDS rows into LDS, then lane i of wave w accumulates features d = w, w + 4, ... (16
// per pass over 64 features) against b values read as LDS broadcasts.
template <bool GU_OWN, int CT>
__global__ __launch_bounds__(DTHREADS)
void direct_sign_kernel(const float* __restrict__ a, const float* __restrict__ b, const float* __restrict__ x,
                        const float* __restrict__ y, const float* __restrict__ gu, float* __restrict__ out,
                        const float tie, const float scale, const int D, const int I, const int J, const int C,
                        const int itiles)
{
    constexpr int CW = 16 * CT;
    constexpr int DC = 64;                                // features per pass
    __shared__ float xs[DT][CW];
    __shared__ float ys[DT][CW];
    __shared__ float bt[DT][DT + 1];                      // [i][j], stride 65: conflict-free column reads
    __shared__ float bsm[DC][DT];                         // b[d0 + dd][j0 + j]

    const int p = blockIdx.x / itiles, it = blockIdx.x - p * itiles;
    const int i0 = it * DT, tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
    const int lane = tid % DT, wv = tid / DT;             // sign-sum mapping: output i = i0 + lane, d = d0 + wv + 4 jj
    const float* ap = a + (size_t)p * D * I;
    const float* bp = b + (size_t)p * D * J;
    const float* xp = x + (size_t)p * I * C;
    const float* yp = y + (size_t)p * J * C;
    const float* gp = gu ? gu + (size_t)p * (GU_OWN ? I : J) : nullptr;

    for (int e = tid; e < DT * CW; e += DTHREADS) {
        const int r = e / CW, c = e - r * CW, i = i0 + r;
        xs[r][c] = (i < I && c < C) ? xp[(size_t)i * C + c] : 0.f;
    }
    for (int d0 = 0; d0 < D; d0 += DC) {
        float av[16], acc[16];
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) {
            const int d = d0 + wv + 4 * jj, i = i0 + lane;
            av[jj] = (d < D && i < I) ? ap[(size_t)d * I + i] : 0.f;
            acc[jj] = 0.f;
        }
        for (int j0 = 0; j0 < J; j0 += DT) {
            __syncthreads();                              // previous readers of ys / bsm / bt are done (and xs written)
            for (int e = tid; e < DT * CW; e += DTHREADS) {
                const int r = e / CW, c = e - r * CW, j = j0 + r;
                ys[r][c] = (j < J && c < C) ? yp[(size_t)j * C + c] : 0.f;
            }
            for (int e = tid; e < DC * DT; e += DTHREADS) {
                const int dd = e / DT, jl = e - dd * DT, d = d0 + dd, j = j0 + jl;
                bsm[dd][jl] = (d < D && j < J) ? bp[(size_t)d * J + j] : 0.f;
            }
            __syncthreads();
            float bb[4][4];
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int q = 0; q < 4; ++q) bb[r][q] = 0.f;
            for (int c = 0; c < C; ++c) {
                float xv[4], yv[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) { xv[r] = xs[4 * ty + r][c]; yv[r] = ys[4 * tx + r][c]; }
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int q = 0; q < 4; ++q) bb[r][q] += xv[r] * yv[q];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int i = i0 + 4 * ty + r, j = j0 + 4 * tx + q;
                    float g = 0.f;
                    if (gp) g = GU_OWN ? (i < I ? gp[i] : 0.f) : (j < J ? gp[j] : 0.f);
                    bt[4 * ty + r][4 * tx + q] = bb[r][q] + g;
                }
            __syncthreads();
            const int nj = min(DT, J - j0);
            for (int j = 0; j < nj; ++j) {
                const float bv = bt[lane][j];
#pragma unroll
                for (int jj = 0; jj < 16; ++jj) {
                    const float z = av[jj] - bsm[wv + 4 * jj][j];
                    const float sg = z > 0.f ? 1.f : (z < 0.f ? -1.f : tie);
                    acc[jj] += sg * bv;
                }
            }
        }
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) {
            const int d = d0 + wv + 4 * jj, i = i0 + lane;
            if (d < D && i < I) out[(size_t)p * D * I + (size_t)d * I + i] = scale * acc[jj];
        }
    }
}

int direct_sign(bool gu_own, const float* a, const float* b, const float* x, const float* y, const float* gu,
                float* out, float tie, float scale, int P, int D, int I, int J, int C, hipStream_t st) {
    const int itiles = (I + DT - 1) / DT;
    const dim3 grid((unsigned)(P * itiles)), block(DTHREADS);
    StageTimer t("direct_sign", st);
#define QLKA_SIGN(OWN, CTV) \
    hipLaunchKernelGGL((direct_sign_kernel<OWN, CTV>), grid, block, 0, st, a, b, x, y, gu, out, tie, scale, D, I, J, \
                       C, itiles)
    if (gu_own) { if (C <= 64) QLKA_SIGN(true, 4); else QLKA_SIGN(true, 8); }
    else        { if (C <= 64) QLKA_SIGN(false, 4); else QLKA_SIGN(false, 8); }
#undef QLKA_SIGN
    return (int)hipGetLastError();
}

int direct_bwd(float tie, const float* q, const float* k, const float* v, const float* g_w, const float* g_u,
               float* grad_q, float* grad_k, float* grad_v, int P, int D, int N, int M, int C, hipStream_t st) {
    // grad_q[d, m] = sum_n s(q - k) (<g_w[m], v[n]> + g_u[m])
    if (int e = direct_sign(true, q, k, g_w, v, g_u, grad_q, tie, 1.f, P, D, M, N, C, st)) return e;
    // grad_k[d, n] = sum_m s(k - q) (<v[n], g_w[m]> + g_u[m])
    if (int e = direct_sign(false, k, q, v, g_w, g_u, grad_k, tie, 1.f, P, D, N, M, C, st)) return e;
    // grad_v[n, :] = sum_m A[m, n] g_w[m, :]: the dense abs sum with the roles of q and k swapped
    return direct_fwd(0, k, q, g_w, grad_v, nullptr, P, D, M, N, C, st);
}

}  // namespace qlka
