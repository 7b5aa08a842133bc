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

// ---- shared by the small-segment kernels (one workgroup per p, the whole segment in LDS)
constexpr int DS_MAXT = 1024;      // threads per workgroup at most
constexpr int DS_MAX = 128;        // padded segment lengths at most
constexpr int DS_CMAX = 64;        // padded C at most (sign sums)
constexpr int DS_DC = 64;          // features per chunk
constexpr size_t DS_LDS_MAX = 64 * 1024;

static inline int pad4(int x) { return (x + 3) & ~3; }

// One round of a zero-padded copy of the row-major [R][K] block at src into LDS: the thread's SU elements
// e = e0 + u * nt of the padded [Rp][Kp] index space (row e / Kp, column e % Kp, e < n = Rp * Kp). All loads of a
// round are issued before any LDS store, so a round costs one global-memory latency, not SU of them.
template <int SU>
struct StageRound {
    float v[SU];
    __device__ __forceinline__ void load(const float* __restrict__ src, int R, int K, int Kp, int n, int e0, int nt) {
        int r = e0 / Kp, c = e0 - r * Kp;
        const int dq = nt / Kp, dr = nt - dq * Kp;
#pragma unroll
        for (int u = 0; u < SU; ++u) {
            v[u] = (e0 + u * nt < n && r < R && c < K) ? src[(size_t)r * K + c] : 0.f;
            c += dr; r += dq;
            if (c >= Kp) { c -= Kp; ++r; }
        }
    }
    // TRANSPOSE: dst[c * Rp + r] (feature-major), else dst[e] (the padded [Rp][Kp] layout itself)
    template <bool TRANSPOSE>
    __device__ __forceinline__ void store(float* dst, int Rp, int Kp, int n, int e0, int nt) const {
        int r = e0 / Kp, c = e0 - r * Kp;
        const int dq = nt / Kp, dr = nt - dq * Kp;
#pragma unroll
        for (int u = 0; u < SU; ++u) {
            const int e = e0 + u * nt;
            if (e < n) dst[TRANSPOSE ? c * Rp + r : e] = v[u];
            c += dr; r += dq;
            if (c >= Kp) { c -= Kp; ++r; }
        }
    }
};
constexpr int DS_SU = 8;           // elements per thread per staging round

typedef float f2_t __attribute__((ext_vector_type(2)));

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

// Small segments (padded M, N <= 128, the working set within 64 KB of LDS): one workgroup per p. q and k go to LDS
// in chunks of 64 features ([d][m], [d][n], zero-padded) and each thread accumulates a 4-key x 4-query block of
// A[n][m] over all features; A stays in LDS (zero at padded keys) and the q / k space takes v ([n][c]), whose loads
// were issued before A was formed. Each thread then accumulates a 2-query x 4-channel block of A v (and the row sums)
// over all keys. The grid has one workgroup per p and as many threads as the larger phase has blocks.
static size_t direct_fwd_small_lds(int D, int N, int M, int C) {
    const int Mp = pad4(M), Np = pad4(N), Cp = pad4(C), Dc = std::min(pad4(D), DS_DC);
    return 4 * (std::max((size_t)Dc * (Mp + Np), (size_t)Np * Cp) + (size_t)Np * Mp);
}

template <int KIND>
__global__ __launch_bounds__(DS_MAXT)
void direct_fwd_small_kernel(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
                             float* __restrict__ out_w, float* __restrict__ out_u,
                             const int D, const int N, const int M, const int C)
{
    extern __shared__ float lds[];
    const int Mp = (M + 3) & ~3, Np = (N + 3) & ~3, Cp = (C + 3) & ~3, Dc = min((D + 3) & ~3, DS_DC);
    float* qs = lds;                                      // [Dc][Mp]
    float* ks = lds + (size_t)Dc * Mp;                    // [Dc][Np]
    float* vs = lds;                                      // [Np][Cp], once A is formed
    float* A = lds + max((size_t)Dc * (Mp + Np), (size_t)Np * Cp);           // [Np][Mp]
    const int p = blockIdx.x, tid = threadIdx.x, nt = blockDim.x;
    const float* qp = q + (size_t)p * D * M;
    const float* kp = k + (size_t)p * D * N;
    const float* vp = v + (size_t)p * N * C;
    const int nq = Dc * Mp, nk = Dc * Np, nv = Np * Cp;
    StageRound<DS_SU> sv;
    sv.load(vp, N, C, Cp, nv, tid, nt);                   // first round of v, lands while A is formed
    const int bm4 = Mp / 4;
    const bool has_a = tid < bm4 * (Np / 4);              // at most one A block per thread (nt covers them all)
    const int n0 = (tid / bm4) * 4, m0 = (tid - (tid / bm4) * bm4) * 4;
    float a[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int u = 0; u < 4; ++u) a[r][u] = 0.f;
    for (int d0 = 0; d0 < D; d0 += Dc) {
        const int rows = min(Dc, D - d0);
        if (d0 > 0) __syncthreads();                      // the previous chunk's readers are done
        for (int e0 = tid; e0 < max(nq, nk); e0 += DS_SU * nt) {
            StageRound<DS_SU> sq, sk;
            sq.load(qp + (size_t)d0 * M, rows, M, Mp, nq, e0, nt);
            sk.load(kp + (size_t)d0 * N, rows, N, Np, nk, e0, nt);
            sq.template store<false>(qs, Dc, Mp, nq, e0, nt);
            sk.template store<false>(ks, Dc, Np, nk, e0, nt);
        }
        __syncthreads();
        if (has_a)
            for (int dd = 0; dd < rows; ++dd) {           // features past D are not summed (e^0 would count)
                const f4_t qv = *reinterpret_cast<const f4_t*>(qs + (size_t)dd * Mp + m0);
                const f4_t kv = *reinterpret_cast<const f4_t*>(ks + (size_t)dd * Np + n0);
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const float x = fabsf(qv[u] - kv[r]);
                        if constexpr (KIND == 0) a[r][u] += x;
                        else a[r][u] += __expf(-x);
                    }
            }
    }
    if (has_a)
#pragma unroll
        for (int r = 0; r < 4; ++r) {                     // keys past N weigh 0 (v is 0 there, out_u is not)
            const bool kin = n0 + r < N;
            const f4_t row = {kin ? a[r][0] : 0.f, kin ? a[r][1] : 0.f, kin ? a[r][2] : 0.f, kin ? a[r][3] : 0.f};
            *reinterpret_cast<f4_t*>(A + (size_t)(n0 + r) * Mp + m0) = row;
        }
    __syncthreads();                                      // A complete, q / k space free
    for (int e0 = tid; e0 < nv; e0 += DS_SU * nt) {
        if (e0 > tid) sv.load(vp, N, C, Cp, nv, e0, nt);
        sv.template store<false>(vs, Np, Cp, nv, e0, nt);
    }
    __syncthreads();
    const int bm2 = Mp / 2;
    for (int t = tid; t < bm2 * (Cp / 4); t += nt) {
        const int c0 = (t / bm2) * 4, mm = (t - (t / bm2) * bm2) * 2;
        float acc[2][4], us[2] = {0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[u][c] = 0.f;
        for (int n = 0; n < Np; ++n) {
            const f2_t av = *reinterpret_cast<const f2_t*>(A + (size_t)n * Mp + mm);
            const f4_t vv = *reinterpret_cast<const f4_t*>(vs + (size_t)n * Cp + c0);
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                us[u] += av[u];
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[u][c] += av[u] * vv[c];
            }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int m = mm + u;
            if (m >= M) continue;
            float* o = out_w + ((size_t)p * M + m) * C;
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (c0 + c < C) o[c0 + c] = acc[u][c];
            if (out_u != nullptr && c0 == 0) out_u[(size_t)p * M + m] = us[u];
        }
    }
}

int direct_fwd(int kind, const float* q, const float* k, const float* v, float* out_w, float* out_u,
               int P, int D, int N, int M, int C, hipStream_t st) {
    const size_t lds = direct_fwd_small_lds(D, N, M, C);
    if (pad4(M) <= DS_MAX && pad4(N) <= DS_MAX && lds <= DS_LDS_MAX) {
        const int blocks_a = pad4(M) / 4 * (pad4(N) / 4), blocks_av = pad4(M) / 2 * (pad4(C) / 4);
        const int threads = std::min(DS_MAXT, (std::max(blocks_a, blocks_av) + WAVE - 1) / WAVE * WAVE);
        StageTimer t("direct_fwd", st);
        if (kind == 0)
            hipLaunchKernelGGL((direct_fwd_small_kernel<0>), dim3((unsigned)P), dim3(threads), lds, st, q, k, v, out_w,
                               out_u, D, N, M, C);
        else
            hipLaunchKernelGGL((direct_fwd_small_kernel<1>), dim3((unsigned)P), dim3(threads), lds, st, q, k, v, out_w,
                               out_u, D, N, M, C);
        return (int)hipGetLastError();
    }
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

// Small segments (padded I, J <= 128, C <= 64, the whole working set within 64 KB of LDS): one workgroup per p holds
// everything in LDS, sized to the shape, with as many threads as the sign sums have 4-feature x 2-output blocks
// (rounded up to whole waves, at most 1024). x and y go to LDS feature-major (zero-padded), the whole matrix
// G[j][i] = <x_i, y_j> + gu is formed once (a 4 x 4 outer-product block per thread; zero at padded i, j), then the
// x / y space takes the features in chunks of 64 (a as [d][i], b as [d][j]) and each thread accumulates its block over
// all j, four j at a time: 4 two-float reads of G and 4 four-float reads of b per 32 sign products. Comparing a with b
// gives the sign of a - b exactly; with tie = -1 or +1 (the gradients and weighted_sgn_sum of the CUDA route) a sign
// product is one compare, one select and one add.

static size_t direct_sign_small_lds(int D, int I, int J, int C) {
    const int Ip = pad4(I), Jp = pad4(J), Cp = pad4(C), Dc = std::min(pad4(D), DS_DC);
    const size_t xy = (size_t)(Ip + Jp) * Cp, ab = (size_t)Dc * (Ip + Jp);
    return 4 * (std::max(xy, ab) + (size_t)Ip * Jp + std::max(Ip, Jp));
}

// TIE: -1 or +1 for s(0) = -1 / +1, 0 for any other s(0) (the value in `tie`)
template <int TIE>
__device__ __forceinline__ float signed_term(float a, float b, float g, float tg) {
    if constexpr (TIE < 0) return a > b ? g : -g;
    else if constexpr (TIE > 0) return a < b ? -g : g;
    else return a > b ? g : (a < b ? -g : tg);
}

template <bool GU_OWN, int TIE>
__global__ __launch_bounds__(DS_MAXT)
void direct_sign_small_kernel(const float* __restrict__ a, const float* __restrict__ b, const float* __restrict__ x,
                              const float* __restrict__ y, const float* __restrict__ gu, float* __restrict__ out,
                              const float tie, const float scale, const int D, const int I, const int J, const int C)
{
    extern __shared__ float lds[];
    const int Ip = (I + 3) & ~3, Jp = (J + 3) & ~3, Cp = (C + 3) & ~3, Dc = min((D + 3) & ~3, DS_DC);
    float* xs = lds;                                      // [Cp][Ip], then as [Dc][Ip]
    float* ys = lds + (size_t)Ip * Cp;                    // [Cp][Jp], then bs [Dc][Jp]
    float* G = lds + max((size_t)(Ip + Jp) * Cp, (size_t)Dc * (Ip + Jp));   // [Jp][Ip]
    float* gs = G + (size_t)Ip * Jp;                      // gu of the segment, zero-padded
    const int p = blockIdx.x, tid = threadIdx.x, nt = blockDim.x;
    const float* xp = x + (size_t)p * I * C;
    const float* yp = y + (size_t)p * J * C;
    const float* ap = a + (size_t)p * D * I;
    const float* bp = b + (size_t)p * D * J;
    const int nx = Ip * Cp, ny = Jp * Cp, na = Dc * Ip, nb = Dc * Jp;
    const int ng = GU_OWN ? I : J, ngp = GU_OWN ? Ip : Jp;
    const float* gp = gu ? gu + (size_t)p * ng : nullptr;
    for (int e0 = tid; e0 < max(nx, ny); e0 += DS_SU * nt) {   // one round unless the segment is large
        StageRound<DS_SU> sx, sy;
        sx.load(xp, I, C, Cp, nx, e0, nt);
        sy.load(yp, J, C, Cp, ny, e0, nt);
        if (e0 == tid)
            for (int e = tid; e < ngp; e += nt) gs[e] = (gp && e < ng) ? gp[e] : 0.f;
        sx.template store<true>(xs, Ip, Cp, nx, e0, nt);
        sy.template store<true>(ys, Jp, Cp, ny, e0, nt);
    }
    // the first staging round of a / b is loaded now and lands while G is formed
    StageRound<DS_SU> sa, sb;
    sa.load(ap, min(Dc, D), I, Ip, na, tid, nt);
    sb.load(bp, min(Dc, D), J, Jp, nb, tid, nt);
    __syncthreads();
    const int bi4 = Ip / 4, bj4 = Jp / 4;
    for (int t = tid; t < bi4 * bj4; t += nt) {           // i fastest: conflict-free float4 reads of xs
        const int j0 = (t / bi4) * 4, i0 = (t - (t / bi4) * bi4) * 4;
        float acc[4][4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[r][q] = 0.f;
        for (int c = 0; c < Cp; ++c) {
            const f4_t xv = *reinterpret_cast<const f4_t*>(xs + (size_t)c * Ip + i0);
            const f4_t yv = *reinterpret_cast<const f4_t*>(ys + (size_t)c * Jp + j0);
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int q = 0; q < 4; ++q) acc[r][q] += xv[r] * yv[q];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int j = j0 + q;
            f4_t row;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = i0 + r;
                row[r] = (i < I && j < J) ? acc[r][q] + gs[GU_OWN ? i : j] : 0.f;
            }
            *reinterpret_cast<f4_t*>(G + (size_t)j * Ip + i0) = row;
        }
    }
    float* op = out + (size_t)p * D * I;
    const int bi2 = Ip / 2;
    for (int d0 = 0; d0 < D; d0 += Dc) {
        __syncthreads();                                  // G complete / the previous chunk's readers done
        float* as = lds;                                  // [Dc][Ip]
        float* bs = lds + (size_t)Dc * Ip;                // [Dc][Jp]
        const int rows = min(Dc, D - d0);
        for (int e0 = tid; e0 < max(na, nb); e0 += DS_SU * nt) {
            if (d0 > 0 || e0 > tid) {                     // the first round is already in registers
                sa.load(ap + (size_t)d0 * I, rows, I, Ip, na, e0, nt);
                sb.load(bp + (size_t)d0 * J, rows, J, Jp, nb, e0, nt);
            }
            sa.template store<false>(as, Dc, Ip, na, e0, nt);
            sb.template store<false>(bs, Dc, Jp, nb, e0, nt);
        }
        __syncthreads();
        for (int t = tid; t < (Dc / 4) * bi2; t += nt) {
            const int dd0 = (t / bi2) * 4, i0 = (t - (t / bi2) * bi2) * 2;
            float av[4][2], acc[4][2];
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int q = 0; q < 2; ++q) { av[r][q] = as[(size_t)(dd0 + r) * Ip + i0 + q]; acc[r][q] = 0.f; }
            for (int j = 0; j < Jp; j += 4) {             // padded j: b = 0 and G = 0, no contribution
                f2_t gv[4];
                f4_t bv[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) gv[u] = *reinterpret_cast<const f2_t*>(G + (size_t)(j + u) * Ip + i0);
#pragma unroll
                for (int r = 0; r < 4; ++r) bv[r] = *reinterpret_cast<const f4_t*>(bs + (size_t)(dd0 + r) * Jp + j);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    float tg[2];
#pragma unroll
                    for (int q = 0; q < 2; ++q) tg[q] = TIE == 0 ? tie * gv[u][q] : 0.f;
#pragma unroll
                    for (int r = 0; r < 4; ++r)
#pragma unroll
                        for (int q = 0; q < 2; ++q) acc[r][q] += signed_term<TIE>(av[r][q], bv[r][u], gv[u][q], tg[q]);
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int d = d0 + dd0 + r, i = i0 + q;
                    if (d < D && i < I) op[(size_t)d * I + i] = scale * acc[r][q];
                }
        }
    }
}

template <bool GU_OWN>
static void launch_sign_small(const float* a, const float* b, const float* x, const float* y, const float* gu,
                              float* out, float tie, float scale, int P, int D, int I, int J, int C, size_t lds,
                              hipStream_t st) {
    const int tasks = std::min(pad4(D), DS_DC) / 4 * (pad4(I) / 2);
    const int threads = std::min(DS_MAXT, (tasks + WAVE - 1) / WAVE * WAVE);
    if (tie == -1.f)
        hipLaunchKernelGGL((direct_sign_small_kernel<GU_OWN, -1>), dim3((unsigned)P), dim3(threads), lds, st, a, b,
                           x, y, gu, out, tie, scale, D, I, J, C);
    else if (tie == 1.f)
        hipLaunchKernelGGL((direct_sign_small_kernel<GU_OWN, 1>), dim3((unsigned)P), dim3(threads), lds, st, a, b,
                           x, y, gu, out, tie, scale, D, I, J, C);
    else
        hipLaunchKernelGGL((direct_sign_small_kernel<GU_OWN, 0>), dim3((unsigned)P), dim3(threads), lds, st, a, b,
                           x, y, gu, out, tie, scale, D, I, J, C);
}

static bool sign_small_fits(int D, int I, int J, int C) {
    return pad4(I) <= DS_MAX && pad4(J) <= DS_MAX && pad4(C) <= DS_CMAX && direct_sign_small_lds(D, I, J, C) <= DS_LDS_MAX;
}

bool direct_sign_fast(int D, int N, int M, int C) { return sign_small_fits(D, M, N, C) && sign_small_fits(D, N, M, C); }

int direct_sign(bool gu_own, const float* a, const float* b, const float* x, const float* y, const float* gu,
                float* out, float tie, float scale, int P, int D, int I, int J, int C, hipStream_t st) {
    if (sign_small_fits(D, I, J, C)) {
        const size_t lds = direct_sign_small_lds(D, I, J, C);
        StageTimer t("direct_sign", st);
        if (gu_own) launch_sign_small<true>(a, b, x, y, gu, out, tie, scale, P, D, I, J, C, lds, st);
        else launch_sign_small<false>(a, b, x, y, gu, out, tie, scale, P, D, I, J, C, lds, st);
        return (int)hipGetLastError();
    }
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
