// D-reduction of the per-feature contributions (the last step of stage 4).
//
// The walks leave one contribution row per (p, d, query) in a slab: slab[(p*D + d)*M + m][0:C] (row stride
// slab_stride(C), whole 128-byte lines), written with plain row stores. Summing over the D features of a p here is a
// streaming read of the slab, so the D-fold accumulation costs one HBM write and one HBM read per contribution
// instead of one fp32 atomic per channel (the L2 atomic units of the chip sustain about one 4-byte atomic per
// channel per clock, which bounds an atomic emission at P*D*M*C atomics well above the slab's traffic time).
//
// The v == 1 sums (out_u) are one scalar per (p, d, query). The walks write them in sorted-query order (coalesced);
// u_scatter turns them back into query order by adding them, through the sort permutation, into an LDS window of
// UWIN queries (LDS atomics), for a group of UG features at a time; the row reduce then adds the group partials.
#include "qlka_common.h"
#include "qlka_internal.h"

namespace qlka {

constexpr int UG   = 8;        // features per u_scatter workgroup
constexpr int UWIN = 16384;    // queries per LDS window (64 KB)
constexpr int RT   = 256;      // threads per block

static inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

size_t reduce_scratch_bytes(int P, int D, int M) {
    const size_t NG = (size_t)((D + UG - 1) / UG);
    return align256((size_t)P * NG * M * sizeof(float));
}

__global__ __launch_bounds__(RT)
void u_scatter(const float* __restrict__ uslab, const uint32_t* __restrict__ qp, float* __restrict__ upart,
               const int P, const int D, const int M, const int NG, const int NW)
{
    __shared__ float acc[UWIN];
    int b = blockIdx.x;
    const int w = b % NW; b /= NW;
    const int g = b % NG;
    const int p = b / NG;
    const int w0 = w * UWIN;
    const int wl = min(UWIN, M - w0);
    for (int j = threadIdx.x; j < wl; j += RT) acc[j] = 0.f;
    __syncthreads();
    const int d1 = min(D, (g + 1) * UG);
    for (int d = g * UG; d < d1; ++d) {
        const size_t so = ((size_t)p * D + d) * M;
        for (int i = threadIdx.x; i < M; i += RT) {
            const uint32_t m = qp[so + i] - (uint32_t)w0;          // wraps for queries below the window
            if (m < (uint32_t)wl) atomicAdd(&acc[m], uslab[so + i]);
        }
    }
    __syncthreads();
    float* dst = upart + ((size_t)p * NG + g) * M + w0;
    for (int j = threadIdx.x; j < wl; j += RT) dst[j] = acc[j];
}

// One thread per (p, m, 4 channels) (V4, C % 4 == 0) or per (p, m, channel); features summed in order d = 0..D-1.
template <bool V4>
__global__ __launch_bounds__(RT)
void slab_reduce(const float* __restrict__ slab, const float* __restrict__ upart, float* __restrict__ out,
                 float* __restrict__ out_u, const int P, const int D, const int M, const int C, const int CR,
                 const int NG)
{
    const int CQ = V4 ? C / 4 : C;
    const long i = (long)blockIdx.x * RT + threadIdx.x;
    if (i >= (long)P * M * CQ) return;
    const int c = (int)(i % CQ);
    const long pm = i / CQ;
    const int p = (int)(pm / M);
    const int m = (int)(pm - (long)p * M);
    const size_t dstride = (size_t)M * CR;                           // floats between features
    const float* src = slab + ((size_t)p * D * M + m) * CR;
    if constexpr (V4) {
        const float4* s4 = reinterpret_cast<const float4*>(src) + c;
        const size_t d4 = dstride / 4;
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
        for (int d = 0; d < D; ++d) {
            const float4 x = s4[(size_t)d * d4];
            a.x += x.x; a.y += x.y; a.z += x.z; a.w += x.w;
        }
        reinterpret_cast<float4*>(out + pm * C)[c] = a;
    } else {
        float a = 0.f;
#pragma unroll 8
        for (int d = 0; d < D; ++d) a += src[(size_t)d * dstride + c];
        out[pm * C + c] = a;
    }
    if (out_u != nullptr && c == 0) {
        float u = 0.f;
        for (int g = 0; g < NG; ++g) u += upart[((size_t)p * NG + g) * M + m];
        out_u[pm] = u;
    }
}

int reduce_slabs(const float* slab, const float* uslab, const uint32_t* qp, float* out, float* out_u,
                 int P, int D, int M, int C, void* scratch, hipStream_t st) {
    const int NG = (D + UG - 1) / UG;
    const int NW = (M + UWIN - 1) / UWIN;
    float* upart = (float*)scratch;
    if (out_u) {
        StageTimer t("u_scatter", st);
        hipLaunchKernelGGL(u_scatter, dim3((unsigned)(P * NG * NW)), dim3(RT), 0, st, uslab, qp, upart, P, D, M, NG,
                           NW);
    }
    const int CR = slab_stride(C);
    const bool v4 = (C % 4) == 0;
    const long threads = (long)P * M * (v4 ? C / 4 : C);
    const unsigned blocks = (unsigned)((threads + RT - 1) / RT);
    StageTimer t("slab_reduce", st);
    if (v4)
        hipLaunchKernelGGL(slab_reduce<true>, dim3(blocks), dim3(RT), 0, st, slab, upart, out, out_u, P, D, M, C, CR,
                           NG);
    else
        hipLaunchKernelGGL(slab_reduce<false>, dim3(blocks), dim3(RT), 0, st, slab, upart, out, out_u, P, D, M, C, CR,
                           NG);
    return (int)hipGetLastError();
}

}  // namespace qlka
