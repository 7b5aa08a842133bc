// Direct (dense) evaluation for short segments, the role the reference gives pykeops below KEOPS_CUTOFF
// (Weighted_Abs_Sum/weighted_abs_sum/keops_backend.py:19-35: A_mn = sum_d |q_dm - k_dn| reduced against [v, 1] in
// one pass) and for the Laplace sum at small N (the dense formula of Experiments/kernel_attention/kernels.py:81):
//
//   A[m, n] = sum_d f(q[d, m] - k[d, n]),  f = |x| (abs) or e^{-|x|} (Laplace)
//   out_w[m, :] = sum_n A[m, n] v[n, :],   out_u[m] = sum_n A[m, n]
//
// and the sign sums of their gradients (further below). Segments of up to 128 keys and queries run one workgroup per
// p with the whole segment in LDS; longer ones run one workgroup per (p, tile of outputs) that walks the other side
// in tiles of 64. Nothing is sorted, so no workspace: below a few hundred keys this beats the sort + scan pipeline,
// whose cost there is launch and per-segment overhead. All arithmetic is fp32, as in the dense and KeOps paths of
// the reference.
#include "qlka_common.h"
#include "qlka_internal.h"

namespace qlka {

// ---- tiled kernels (longer segments)
constexpr int ST_T = 256;          // threads per workgroup
constexpr int ST_JT = 64;          // keys (forward) / j (sign sums) per tile

// ---- shared by the small-segment kernels (one workgroup per p, the whole segment in LDS)
constexpr int DS_MAXT = 1024;      // threads per workgroup at most
constexpr int DS_MAX = 128;        // padded segment lengths at most
constexpr int DS_CMAX = 64;        // padded C at most (sign sums)
constexpr int DS_DC = 64;          // features per chunk
constexpr size_t DS_LDS_MAX = 64 * 1024;

static inline int pad4(int x) { return (x + 3) & ~3; }

// One round of a zero-padded copy of the row-major [R][K] block at src (row stride K) into LDS: the thread's SU
// elements e = e0 + u * nt of the padded [Rp][Kp] index space (row e / Kp, column e % Kp, e < n = Rp * Kp). All loads
// of a round are issued before any LDS store, so a round costs one global-memory latency, not SU of them.
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
constexpr int DS_SU = 8;
// Size of a raw buffer descriptor used for staging, and the offset that reads past its end (the load returns 0).
constexpr uint32_t STAGE_OOB = 0x7ffffff0u;           // elements per thread per staging round

typedef float f2_t __attribute__((ext_vector_type(2)));

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

// Longer segments: one workgroup of 256 threads per (p, tile of IT queries) walks the keys in tiles of 64. Per key
// tile and 64-feature chunk the k values ([d][n]) come from registers loaded during the previous step, and each thread
// adds the chunk to its 4-key x (IT / 16)-query block of A on the VALU; after the last chunk the A tile goes to LDS
// ([n][m], zero at keys past N) and the contraction A^T [v, 1] runs on the matrix cores: the IT x CM output tile is
// 16 x 16 blocks, each wave owns BW of them (one query block, BW channel blocks) and adds the tile's 64 keys to them
// with 16 v_mfma_f32_16x16x4_f32 per block (fp32 products and sums, as the VALU form), the tile's v rows, loaded while
// A was formed, in LDS ([n][c]). The waves whose first channel block is 0 also run one MFMA per step against a
// column of ones: the row sums out_u. IT = 64 for C <= 32 (CM = 32), else 32 (CM = 64 or 128). Staging as in the
// tiled sign sums: raw buffer descriptors that end at the segment's end (rows past it read 0), fixed LDS row strides;
// columns past the tile (keys past N, queries past M, channels past C) may read the next row and never reach an
// output or A (an MFMA output column depends only on its own column of v).
template <int KIND, int IT, int CM, bool SAVE = false>
__global__ __launch_bounds__(ST_T)
void direct_fwd_tiled_kernel(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
                             float* __restrict__ out_w, float* __restrict__ out_u, float* __restrict__ a_out,
                             const int D, const int N, const int M, const int C, const int mtiles)
{
    constexpr int DCK = 64;                               // features per chunk
    constexpr int QM = IT / 16;                           // queries per thread in the A phase (4 keys x QM)
    constexpr int KS = ST_JT + 4, VS = CM + 4;            // LDS row strides
    constexpr int KK = ST_JT / 4, KV = CM / 4, KQ = IT / 4;   // staged elements per thread (4 threads per row)
    constexpr int NBC = CM / 16, BW = (IT / 16) * NBC / 4;   // 16-channel blocks; 16 x 16 output blocks per wave
    static_assert(BW >= 1 && NBC % BW == 0, "a wave's output blocks share one query block");
    __shared__ float qs[DCK * IT];                        // [d][m]
    __shared__ float ks[DCK * KS];                        // [d][n]
    __shared__ float vs[ST_JT * VS];                      // [n][c]
    __shared__ float At[ST_JT * IT];                      // [n][m]

    const int p = blockIdx.x / mtiles, mb = (blockIdx.x - p * mtiles) * IT, tid = threadIdx.x;
    const int Ml = min(IT, M - mb);
    const int sr = tid / 4, sc = tid - sr * 4;            // staging: row, first column
    const int ktiles = (N + ST_JT - 1) / ST_JT, chunks = (D + DCK - 1) / DCK, steps = ktiles * chunks;
    float kv[KK], vv[KV];
    auto load_k = [&](int s) {
        const int n0 = (s / chunks) * ST_JT, d0 = (s % chunks) * DCK;
        const rsrc_t rk = make_rsrc(k + ((size_t)p * D + d0) * N + n0, (uint32_t)(((D - d0) * N - n0) * 4));
#pragma unroll
        for (int e = 0; e < KK; ++e) kv[e] = buf_load(rk, (sr * N + sc + 4 * e) * 4, 0);
    };
    auto load_v = [&](int t) {
        const int n0 = t * ST_JT;
        const rsrc_t rv = make_rsrc(v + ((size_t)p * N + n0) * C, (uint32_t)((N - n0) * C * 4));
#pragma unroll
        for (int e = 0; e < KV; ++e) vv[e] = buf_load(rv, (sr * C + sc + 4 * e) * 4, 0);
    };
    auto stage_q = [&](int d0) {                          // q rows d0 .. d0 + 63 of the query tile
        const rsrc_t rq = make_rsrc(q + ((size_t)p * D + d0) * M + mb, (uint32_t)(((D - d0) * M - mb) * 4));
        float qv[KQ];
#pragma unroll
        for (int e = 0; e < KQ; ++e) qv[e] = buf_load(rq, (sr * M + sc + 4 * e) * 4, 0);
#pragma unroll
        for (int e = 0; e < KQ; ++e) qs[sr * IT + sc + 4 * e] = qv[e];
    };
    load_k(0);
    load_v(0);
    if (chunks == 1) stage_q(0);
    const int an = (tid / (IT / QM)) * 4, am = (tid - (tid / (IT / QM)) * (IT / QM)) * QM;   // A block
    const int wv = wave_in_block(), ln = lane_id();
    const int mi = (wv * BW) / NBC, cb0 = (wv * BW) % NBC;  // this wave's query block and first channel block
    const bool uw = cb0 == 0;                              // it also forms the row sums
    float a[4][QM];
    f4_t acc[BW], accu = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int u = 0; u < QM; ++u) a[r][u] = 0.f;
#pragma unroll
    for (int t = 0; t < BW; ++t) acc[t] = f4_t{0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < steps; ++s) {
        const int t = s / chunks, h = s - t * chunks, n0 = t * ST_JT, d0 = h * DCK;
        __syncthreads();                                  // readers of ks (and of vs / At / qs) are done
#pragma unroll
        for (int e = 0; e < KK; ++e) ks[sr * KS + sc + 4 * e] = kv[e];
        if (h == 0)
#pragma unroll
            for (int e = 0; e < KV; ++e) vs[sr * VS + sc + 4 * e] = vv[e];
        if (s + 1 < steps) {
            load_k(s + 1);
            if ((s + 1) % chunks == 0) load_v(t + 1);
        }
        if (chunks > 1) stage_q(d0);
        __syncthreads();
        const int rows = min(DCK, D - d0);
        for (int dd = 0; dd < rows; ++dd) {               // features past D are not summed (e^0 would count)
            const f4_t kr = *reinterpret_cast<const f4_t*>(ks + dd * KS + an);
            float qr[QM];
            if constexpr (QM == 4) {
                const f4_t x4 = *reinterpret_cast<const f4_t*>(qs + dd * IT + am);
                qr[0] = x4[0]; qr[1] = x4[1]; qr[2] = x4[2]; qr[3] = x4[3];
            } else {
                const f2_t x2 = *reinterpret_cast<const f2_t*>(qs + dd * IT + am);
                qr[0] = x2[0]; qr[1] = x2[1];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int u = 0; u < QM; ++u) {
                    const float x = fabsf(qr[u] - kr[r]);
                    if constexpr (KIND == 0) a[r][u] += x;
                    else a[r][u] += __expf(-x);
                }
        }
        if (h + 1 < chunks) continue;
        // the A tile is complete: keys past N weigh 0 (v reads 0 there, out_u would not)
        const int Nl = min(ST_JT, N - n0);
        if constexpr (SAVE) {                             // kept for the backward: A[p][m][n], rows of pad4(N)
            const int NP = (N + 3) & ~3, n = n0 + an;
#pragma unroll
            for (int u = 0; u < QM; ++u) {
                const int m = mb + am + u;
                if (m >= M || n >= N) continue;
                float* row = a_out + ((size_t)p * M + m) * NP + n;
                if (n + 3 < N) {
                    *reinterpret_cast<f4_t*>(row) = f4_t{a[0][u], a[1][u], a[2][u], a[3][u]};
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (n + r < N) row[r] = a[r][u];
                }
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int u = 0; u < QM; ++u) {
                At[(an + r) * IT + am + u] = an + r < Nl ? a[r][u] : 0.f;
                a[r][u] = 0.f;
            }
        __syncthreads();
        // A^T [v, 1] on the matrix cores: lane ln supplies A^T[m][n] and v[n][c] at m, c = block base + ln % 16,
        // n = 4 kk + ln / 16 (keys past N: A = 0 and v = 0)
        const float* Ap = At + (ln >> 4) * IT + mi * 16 + (ln & 15);
        const float* Vp = vs + (ln >> 4) * VS + cb0 * 16 + (ln & 15);
#pragma unroll 4
        for (int kk = 0; kk < ST_JT / 4; ++kk) {
            const float av = Ap[kk * 4 * IT];
#pragma unroll
            for (int t = 0; t < BW; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, Vp[kk * 4 * VS + t * 16], acc[t], 0, 0, 0);
            if (uw) accu = __builtin_amdgcn_mfma_f32_16x16x4f32(av, 1.f, accu, 0, 0, 0);
        }
    }
    // lane ln holds rows m = 16 mi + 4 (ln / 16) + r, r < 4, of column ln % 16 of each of its blocks
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = mi * 16 + 4 * (ln >> 4) + r;
        if (m >= Ml) continue;
        float* o = out_w + ((size_t)p * M + mb + m) * C;
#pragma unroll
        for (int t = 0; t < BW; ++t) {
            const int c = (cb0 + t) * 16 + (ln & 15);
            if (c < C) o[c] = acc[t][r];
        }
        if (uw && (ln & 15) == 0 && out_u != nullptr) out_u[(size_t)p * M + mb + m] = accu[r];
    }
}

template <int KIND, int IT, int CM>
static void launch_fwd_tiled(const float* q, const float* k, const float* v, float* out_w, float* out_u,
                             float* a_out, int P, int D, int N, int M, int C, hipStream_t st) {
    const int mtiles = (M + IT - 1) / IT;
    if constexpr (KIND == 0) {                            // only the abs sum keeps A
        if (a_out != nullptr) {
            hipLaunchKernelGGL((direct_fwd_tiled_kernel<KIND, IT, CM, true>), dim3((unsigned)(P * mtiles)), dim3(ST_T),
                               0, st, q, k, v, out_w, out_u, a_out, D, N, M, C, mtiles);
            return;
        }
    }
        hipLaunchKernelGGL((direct_fwd_tiled_kernel<KIND, IT, CM>), dim3((unsigned)(P * mtiles)), dim3(ST_T), 0, st,
                           q, k, v, out_w, out_u, nullptr, D, N, M, C, mtiles);
}

template <int KIND>
static void launch_fwd_tiled(const float* q, const float* k, const float* v, float* out_w, float* out_u,
                             float* a_out, int P, int D, int N, int M, int C, hipStream_t st) {
    if (pad4(C) <= 32) launch_fwd_tiled<KIND, 64, 32>(q, k, v, out_w, out_u, a_out, P, D, N, M, C, st);
    else if (pad4(C) <= 64) launch_fwd_tiled<KIND, 32, 64>(q, k, v, out_w, out_u, a_out, P, D, N, M, C, st);
    else launch_fwd_tiled<KIND, 32, 128>(q, k, v, out_w, out_u, a_out, P, D, N, M, C, st);
}

// The dense forward runs the tiled kernel (which can keep A) unless the segments fit the one-workgroup kernel.
bool direct_fwd_tiled(int D, int N, int M, int C) {
    return !(pad4(M) <= DS_MAX && pad4(N) <= DS_MAX && direct_fwd_small_lds(D, N, M, C) <= DS_LDS_MAX);
}

// The abs forward of the tiled kernel that also writes A[p][m][n] = sum_d |q[p,d,m] - k[p,d,n]| (rows of pad4(N)
// floats) to a_out, for dense_at_g; only where direct_fwd_tiled(D, N, M, C).
int direct_fwd_keep_a(const float* q, const float* k, const float* v, float* out_w, float* out_u, float* a_out,
                      int P, int D, int N, int M, int C, hipStream_t st) {
    if (!direct_fwd_tiled(D, N, M, C) || a_out == nullptr) return (int)hipErrorInvalidValue;
    StageTimer t("direct_fwd", st);
    launch_fwd_tiled<0>(q, k, v, out_w, out_u, a_out, P, D, N, M, C, st);
    return (int)hipGetLastError();
}

// out[p, n, :] = sum_m A[p, m, n] g[p, m, :] from a kept A ([p][m][pad4(N)], direct_fwd_keep_a): grad_v of the dense
// abs sum without forming A again. The contraction of direct_fwd_tiled_kernel with A loaded instead of formed: one
// workgroup of 256 threads per (p, tile of IT keys) walks the queries in tiles of ST_JT; A's tile ([m][n]) and g's rows
// ([m][c], zero past M) go to LDS and the MFMA blocks, their order over m and so the sums are the forward kernel's
// (its grad_v form, with the roles of q and k swapped, gives the same bits).
template <int IT, int CM>
__global__ __launch_bounds__(ST_T)
void dense_at_g_kernel(const float* __restrict__ A, const float* __restrict__ g, float* __restrict__ out,
                       const int N, const int M, const int C, const int ntiles)
{
    constexpr int VS = CM + 4;
    constexpr int KV = CM / 4;                            // g values per thread (4 threads per row)
    constexpr int AE = ST_JT * IT / ST_T;                 // A values per thread (4 threads per row)
    constexpr int NBC = CM / 16, BW = (IT / 16) * NBC / 4;
    static_assert(BW >= 1 && NBC % BW == 0 && AE % 4 == 0, "tile shape");
    __shared__ float At[ST_JT * IT];                      // [m][n]
    __shared__ float vs[ST_JT * VS];                      // [m][c]
    const int p = blockIdx.x / ntiles, nb = (blockIdx.x - p * ntiles) * IT, tid = threadIdx.x;
    const int Nl = min(IT, N - nb), NP = (N + 3) & ~3;
    const int sr = tid / 4, sc = tid - sr * 4;
    f4_t av[AE / 4];
    float vv[KV];
    auto load = [&](int m0) {
        const int m = m0 + sr;
#pragma unroll
        for (int e = 0; e < AE / 4; ++e) {
            const int n = nb + sc * AE + 4 * e;
            av[e] = (m < M && n < NP) ? *reinterpret_cast<const f4_t*>(A + ((size_t)p * M + m) * NP + n)
                                      : f4_t{0.f, 0.f, 0.f, 0.f};
        }
        const rsrc_t rv = make_rsrc(g + ((size_t)p * M + m0) * C, (uint32_t)((M - m0) * C * 4));
#pragma unroll
        for (int e = 0; e < KV; ++e) vv[e] = buf_load(rv, (sr * C + sc + 4 * e) * 4, 0);
    };
    const int wv = wave_in_block(), ln = lane_id();
    const int ni = (wv * BW) / NBC, cb0 = (wv * BW) % NBC;  // this wave's key block and first channel block
    f4_t acc[BW];
#pragma unroll
    for (int t = 0; t < BW; ++t) acc[t] = f4_t{0.f, 0.f, 0.f, 0.f};
    const int mt = (M + ST_JT - 1) / ST_JT;
    load(0);
    for (int t = 0; t < mt; ++t) {
        __syncthreads();                                  // readers of the previous tile are done
#pragma unroll
        for (int e = 0; e < AE / 4; ++e) *reinterpret_cast<f4_t*>(At + sr * IT + sc * AE + 4 * e) = av[e];
#pragma unroll
        for (int e = 0; e < KV; ++e) vs[sr * VS + sc + 4 * e] = vv[e];
        if (t + 1 < mt) load((t + 1) * ST_JT);
        __syncthreads();
        const float* Ap = At + (ln >> 4) * IT + ni * 16 + (ln & 15);
        const float* Vp = vs + (ln >> 4) * VS + cb0 * 16 + (ln & 15);
#pragma unroll 4
        for (int kk = 0; kk < ST_JT / 4; ++kk) {
            const float a = Ap[kk * 4 * IT];
#pragma unroll
            for (int b = 0; b < BW; ++b)
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, Vp[kk * 4 * VS + b * 16], acc[b], 0, 0, 0);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int n = ni * 16 + 4 * (ln >> 4) + r;
        if (n >= Nl) continue;
        float* o = out + ((size_t)p * N + nb + n) * C;
#pragma unroll
        for (int b = 0; b < BW; ++b) {
            const int c = (cb0 + b) * 16 + (ln & 15);
            if (c < C) o[c] = acc[b][r];
        }
    }
}

int dense_at_g(const float* A, const float* g, float* out, int P, int N, int M, int C, hipStream_t st) {
    StageTimer t("direct_fwd", st);
    if (pad4(C) <= 32) {
        const int nt = (N + 63) / 64;
        hipLaunchKernelGGL((dense_at_g_kernel<64, 32>), dim3((unsigned)(P * nt)), dim3(ST_T), 0, st, A, g, out, N, M, C,
                           nt);
    } else if (pad4(C) <= 64) {
        const int nt = (N + 31) / 32;
        hipLaunchKernelGGL((dense_at_g_kernel<32, 64>), dim3((unsigned)(P * nt)), dim3(ST_T), 0, st, A, g, out, N, M, C,
                           nt);
    } else {
        const int nt = (N + 31) / 32;
        hipLaunchKernelGGL((dense_at_g_kernel<32, 128>), dim3((unsigned)(P * nt)), dim3(ST_T), 0, st, A, g, out, N, M,
                           C, nt);
    }
    return (int)hipGetLastError();
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
    StageTimer t("direct_fwd", st);
    if (kind == 0) launch_fwd_tiled<0>(q, k, v, out_w, out_u, nullptr, P, D, N, M, C, st);
    else launch_fwd_tiled<1>(q, k, v, out_w, out_u, nullptr, P, D, N, M, C, st);
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
    return pad4(I) <= DS_MAX && pad4(J) <= DS_MAX && pad4(C) <= DS_CMAX &&
           direct_sign_small_lds(D, I, J, C) <= DS_LDS_MAX;
}

// Longer segments: one workgroup of 256 threads per (p, tile of IT outputs) walks the j in tiles of 64. The x rows
// of the tile sit in LDS feature-major for the whole walk; per j tile the y rows ([j][c]), the b values of a chunk of
// DCM features ([d][j]) and g_u come from registers loaded during the previous tile, G[j][i] = <x_i, y_j> (+ g_u, zero
// at padded i, j) is formed on the matrix cores (v_mfma_f32_16x16x4_f32, one 16-j block per wave, fp32 products and
// sums) and stored to LDS, and each thread adds 64 j to its block of 4 features x 2 outputs
// with the same sign step as the small kernel. IT = 32 (DCM = 64) in general, IT = 64 (DCM = 32) for D <= 32, so that
// the 256 blocks of a feature chunk are one per thread; more features take further chunks (G formed again per chunk).
// Staging: each thread owns one row of a tile and loads its columns part, part + TPR, ... through a raw buffer
// descriptor that ends at the segment's end, so rows past the segment read 0 and every load is one base register plus
// an immediate offset; LDS rows have a fixed stride (CM + 4 / 64 + 4 floats: no bank conflicts on the four-float reads)
// so stores need no bounds. Columns of b past J read the next row: harmless, as G is 0 there and the sign step selects
// rather than multiplies.
template <bool GU_OWN, int TIE, int IT, int CM>      // CM: padded C at most (64 or 128)
// grad_k's variant (GU_OWN false) is held to 168 VGPRs, 3 waves per SIMD (left alone it takes 172, 2 waves, 30% slower)
__global__ __launch_bounds__(ST_T) __attribute__((amdgpu_waves_per_eu(GU_OWN ? 1 : 3)))
void direct_sign_tiled_kernel(const float* __restrict__ a, const float* __restrict__ b, const float* __restrict__ x,
                              const float* __restrict__ y, const float* __restrict__ gu, float* __restrict__ out,
                              const float tie, const float scale, const int D, const int I, const int J, const int C,
                              const int itiles)
{
    static_assert(ST_JT / 16 == ST_T / WAVE, "one 16-j block of G per wave");
    constexpr int DCM = 2048 / IT;                        // features per chunk
    constexpr int NI2 = IT / 2;                           // output pairs per tile
    constexpr int YS = CM + 4, BS = ST_JT + 4;            // LDS row strides of y and b
    constexpr int TPX = ST_T / IT, KX = CM / TPX;         // x tile: threads per row, columns per thread
    constexpr int TPY = ST_T / ST_JT, KY = CM / TPY;      // y tile
    constexpr int TPB = ST_T / DCM, KB = ST_JT / TPB;     // b chunk
    __shared__ float xs[CM * IT];                         // [c][i]
    __shared__ float ys[ST_JT * YS];                      // [j][c]
    __shared__ float G[ST_JT * IT];                       // [j][i]
    __shared__ float bs[DCM * BS];                        // [d][j]
    __shared__ float gj[ST_JT], gi[IT];                   // g_u of the j tile / of the outputs

    const int p = blockIdx.x / itiles, ib = (blockIdx.x - p * itiles) * IT, tid = threadIdx.x;
    const int Il = min(IT, I - ib);
    const float* gp = gu ? gu + (size_t)p * (GU_OWN ? I : J) : nullptr;
    {
        const int i = tid / TPX, c0 = tid - i * TPX;
        const rsrc_t rx = make_rsrc(x + ((size_t)p * I + ib) * C, (uint32_t)(Il * C * 4));
        float xv[KX];
#pragma unroll
        for (int k = 0; k < KX; ++k) {
            const int c = c0 + TPX * k;
            xv[k] = buf_load(rx, c < C ? (i * C + c) * 4 : (int)STAGE_OOB, 0);
        }
        if (GU_OWN && tid < IT) gi[tid] = (gp && tid < Il) ? gp[ib + tid] : 0.f;
#pragma unroll
        for (int k = 0; k < KX; ++k) xs[(c0 + TPX * k) * IT + i] = xv[k];
    }
    const int yj = tid / TPY, yc0 = tid - yj * TPY;
    const int bd = tid / TPB, bj0 = tid - bd * TPB;
    const int jtiles = (J + ST_JT - 1) / ST_JT, steps = jtiles * ((D + DCM - 1) / DCM);
    float yv[KY], bv[KB], gn = 0.f;
    auto load_step = [&](int s) {                         // step s: feature chunk s / jtiles, j tile s % jtiles
        const int j0 = (s % jtiles) * ST_JT, d0 = (s / jtiles) * DCM;
        const rsrc_t ry = make_rsrc(y + ((size_t)p * J + j0) * C, (uint32_t)(min(ST_JT, J - j0) * C * 4));
#pragma unroll
        for (int k = 0; k < KY; ++k) {
            const int c = yc0 + TPY * k;
            yv[k] = buf_load(ry, c < C ? (yj * C + c) * 4 : (int)STAGE_OOB, 0);
        }
        const rsrc_t rb = make_rsrc(b + ((size_t)p * D + d0) * J + j0, (uint32_t)(((D - d0) * J - j0) * 4));
#pragma unroll
        for (int k = 0; k < KB; ++k) bv[k] = buf_load(rb, (bd * J + bj0 + TPB * k) * 4, 0);
        if (!GU_OWN) gn = (gp && tid < ST_JT && j0 + tid < J) ? gp[j0 + tid] : 0.f;
    };
    load_step(0);
    const int dd0 = (tid / NI2) * 4, i0 = (tid - (tid / NI2) * NI2) * 2;
    const int Cp = (C + 3) & ~3;
    const float* ap = a + (size_t)p * D * I + ib;
    float* op = out + (size_t)p * D * I + ib;
    float av[4][2], acc[4][2];
    for (int s = 0; s < steps; ++s) {
        const int j0 = (s % jtiles) * ST_JT, d0 = (s / jtiles) * DCM;
        if (j0 == 0)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int d = d0 + dd0 + r, i = i0 + q;
                    av[r][q] = (d < D && i < Il) ? ap[(size_t)d * I + i] : 0.f;
                    acc[r][q] = 0.f;
                }
        __syncthreads();                                  // the previous step's readers are done (and xs is written)
#pragma unroll
        for (int k = 0; k < KY; ++k) ys[yj * YS + yc0 + TPY * k] = yv[k];
#pragma unroll
        for (int k = 0; k < KB; ++k) bs[bd * BS + bj0 + TPB * k] = bv[k];
        if (!GU_OWN && tid < ST_JT) gj[tid] = gn;
        if (s + 1 < steps) load_step(s + 1);
        __syncthreads();
        const int Jl = min(ST_JT, J - j0);
        {
            // G = Y X^T on the matrix cores: wave w owns the 16 j of block w and all IT / 16 blocks of i; lane ln
            // supplies y[j][c] and x[i][c] at j, i = block base + ln % 16, c = 4 kk + ln / 16 (columns C .. Cp-1 of
            // xs and ys are 0)
            const int wv = wave_in_block(), ln = lane_id();
            const float* Yp = ys + (wv * 16 + (ln & 15)) * YS + (ln >> 4);
            const float* Xp = xs + (ln >> 4) * IT + (ln & 15);
            f4_t g[IT / 16];
#pragma unroll
            for (int t = 0; t < IT / 16; ++t) g[t] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
            for (int kk = 0; kk < Cp / 4; ++kk) {
                const float yv_ = Yp[kk * 4];
#pragma unroll
                for (int t = 0; t < IT / 16; ++t)
                    g[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(yv_, Xp[kk * 4 * IT + t * 16], g[t], 0, 0, 0);
            }
            // lane ln holds rows j = 16 wv + 4 (ln / 16) + r of column i = 16 t + ln % 16 of each block
#pragma unroll
            for (int t = 0; t < IT / 16; ++t) {
                const int i = t * 16 + (ln & 15);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int j = wv * 16 + 4 * (ln >> 4) + r;
                    G[j * IT + i] = (i < Il && j < Jl) ? g[t][r] + (GU_OWN ? gi[i] : gj[j]) : 0.f;
                }
            }
        }
        __syncthreads();
#pragma unroll 2
        for (int j = 0; j < ST_JT; j += 4) {              // padded j: G = 0, no contribution
            f2_t gv[4];
            f4_t bq[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) gv[u] = *reinterpret_cast<const f2_t*>(G + (j + u) * IT + i0);
#pragma unroll
            for (int r = 0; r < 4; ++r) bq[r] = *reinterpret_cast<const f4_t*>(bs + (dd0 + r) * BS + j);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                float tg[2];
#pragma unroll
                for (int q = 0; q < 2; ++q) tg[q] = TIE == 0 ? tie * gv[u][q] : 0.f;
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int q = 0; q < 2; ++q) acc[r][q] += signed_term<TIE>(av[r][q], bq[r][u], gv[u][q], tg[q]);
            }
        }
        if (j0 + ST_JT >= J)                              // last j tile of the chunk
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int d = d0 + dd0 + r, i = i0 + q;
                    if (d < D && i < Il) op[(size_t)d * I + i] = scale * acc[r][q];
                }
    }
}

template <bool GU_OWN, int IT, int CM>
static void launch_sign_tiled(const float* a, const float* b, const float* x, const float* y, const float* gu,
                              float* out, float tie, float scale, int P, int D, int I, int J, int C, hipStream_t st) {
    const int itiles = (I + IT - 1) / IT;
    const dim3 grid((unsigned)(P * itiles)), block(ST_T);
    if (tie == -1.f)
        hipLaunchKernelGGL((direct_sign_tiled_kernel<GU_OWN, -1, IT, CM>), grid, block, 0, st, a, b, x, y, gu, out,
                           tie, scale, D, I, J, C, itiles);
    else if (tie == 1.f)
        hipLaunchKernelGGL((direct_sign_tiled_kernel<GU_OWN, 1, IT, CM>), grid, block, 0, st, a, b, x, y, gu, out,
                           tie, scale, D, I, J, C, itiles);
    else
        hipLaunchKernelGGL((direct_sign_tiled_kernel<GU_OWN, 0, IT, CM>), grid, block, 0, st, a, b, x, y, gu, out,
                           tie, scale, D, I, J, C, itiles);
}

template <bool GU_OWN>
static void launch_sign_tiled(const float* a, const float* b, const float* x, const float* y, const float* gu,
                              float* out, float tie, float scale, int P, int D, int I, int J, int C, hipStream_t st) {
    const bool wide = pad4(D) <= 32;                      // 64-output tiles: the 8 feature quads x 32 pairs fill 256
    const bool c64 = pad4(C) <= 64;
    if (wide && c64) launch_sign_tiled<GU_OWN, 64, 64>(a, b, x, y, gu, out, tie, scale, P, D, I, J, C, st);
    else if (wide) launch_sign_tiled<GU_OWN, 64, 128>(a, b, x, y, gu, out, tie, scale, P, D, I, J, C, st);
    else if (c64) launch_sign_tiled<GU_OWN, 32, 64>(a, b, x, y, gu, out, tie, scale, P, D, I, J, C, st);
    else launch_sign_tiled<GU_OWN, 32, 128>(a, b, x, y, gu, out, tie, scale, P, D, I, J, C, st);
}

int direct_sign(bool gu_own, const float* a, const float* b, const float* x, const float* y, const float* gu,
                float* out, float tie, float scale, int P, int D, int I, int J, int C, hipStream_t st) {
    if (sign_small_fits(D, I, J, C)) {
        const size_t lds = direct_sign_small_lds(D, I, J, C);
        StageTimer t("direct_sign", st);
        if (gu_own) launch_sign_small<true>(a, b, x, y, gu, out, tie, scale, P, D, I, J, C, lds, st);
        else launch_sign_small<false>(a, b, x, y, gu, out, tie, scale, P, D, I, J, C, lds, st);
        return (int)hipGetLastError();
    }
    StageTimer t("direct_sign", st);
    if (gu_own) launch_sign_tiled<true>(a, b, x, y, gu, out, tie, scale, P, D, I, J, C, st);
    else launch_sign_tiled<false>(a, b, x, y, gu, out, tie, scale, P, D, I, J, C, st);
    return (int)hipGetLastError();
}

}  // namespace qlka
