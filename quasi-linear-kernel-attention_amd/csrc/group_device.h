// Device code of the query grouping, the forward walks' alternative to sorting the queries (group_queries_staged in
// walks.hip), as a workgroup-level function that takes its LDS from the caller.
#pragma once

#include "qlka_common.h"

namespace qlka {

// Queries grouped by key chunk, the forward walks' alternative to sorting them. The sorted keys of a segment fall into
// chunks of CH = RK / 4 (four per key range, the walks' emission chunks); a query's bucket is the chunk holding the
// first key >= q + qshift, b = #{c : klast_c < q + qshift} (Gc = ceil(Ns / CH) when it is above every key). Queries
// come out in bucket order, so each range owns a contiguous run (range g: buckets 4g .. 4g + 3, the last range also
// bucket Gc) and, inside it, its queries come chunk by chunk, which is all a walk needs of their order: it ranks each
// query inside the range itself, and a block of 64 queries then covers consecutive chunks as with sorted queries.
// qb[g] = #queries of ranges <= g, as query_bounds writes it. One workgroup per segment: the Gc chunk boundaries go to
// LDS, every query finds its bucket by binary search there and counts it with an LDS atomic; an exclusive scan of the
// Gc + 1 counts gives the bucket offsets; returning LDS atomics then hand out slots in each bucket, staged in LDS for
// coalesced stores when the segment fits. The order inside a bucket is the order in which the atomics return, which
// is not fixed; no output of any walk depends on it (each query's sums come from its own rank and go to its own index,
// directly or through qp).
constexpr int GQ_T = 1024;         // threads per workgroup
constexpr int GQ_STAGE = 16384;    // longest segment staged in LDS (its values and indices: 128 KB)
constexpr int GQ_STAGE_MAXB = 2048;        // most chunk buckets of a staged segment

// The grouping's LDS tables (chunk and range boundaries, bucket offsets); the staging of the grouped segment (values and
// indices, GQ_STAGE each) is passed separately.
struct GroupTables {
    float bnd[GQ_STAGE_MAXB];
    float rb[GQ_STAGE_MAXB / 4];
    int off[GQ_STAGE_MAXB + 1];
    int wsum[GQ_T / WAVE];
};

// Bucket of x among the nb chunk boundaries in LDS: #{c : bnd[c] < x} (bnd ascending). A branch-free descent over
// the range boundaries rb (the last key of each range, in an array of their own so that the descent's reads spread
// over the LDS banks) finds the range, then the range's first three chunk boundaries are compared at once; the NI
// searches of a thread run interleaved step by step, so that their LDS reads overlap.
template <int NI>
__device__ __forceinline__ void buckets(const float* bnd, const float* rb, const int nb, const float (&x)[NI],
                                        int (&b)[NI]) {
    const int ng = (nb + 3) >> 2;
    int g[NI];
#pragma unroll
    for (int j = 0; j < NI; ++j) g[j] = 0;
    int step = 1;
    while (step * 2 <= ng) step *= 2;
    for (; step >= 1; step >>= 1) {
        float y[NI];
#pragma unroll
        for (int j = 0; j < NI; ++j) y[j] = rb[min(g[j] + step, ng) - 1];
#pragma unroll
        for (int j = 0; j < NI; ++j) g[j] += (g[j] + step <= ng && y[j] < x[j]) ? step : 0;
    }
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        const int c0 = min(4 * g[j], nb - 1);
        const float y0 = bnd[c0], y1 = bnd[min(c0 + 1, nb - 1)], y2 = bnd[min(c0 + 2, nb - 1)];
        b[j] = 4 * g[j];
        if (g[j] < ng) b[j] += (y0 < x[j]) + (c0 + 1 < nb && y1 < x[j]) + (c0 + 2 < nb && y2 < x[j]);
        else b[j] = nb;
    }
}

// Exclusive scan of off[0..n) in place by the whole workgroup (thread t owns a contiguous piece), then the range
// bounds: qb[g] = offset of bucket 4 (g + 1), or of bucket n - 1 = Gc for the last range.
__device__ __forceinline__ void group_scan(int* off, int* wsum, const int n, int* qbs) {
    const int tid = threadIdx.x;
    const int E = (n + GQ_T - 1) / GQ_T;
    const int e0 = min(tid * E, n), e1 = min(e0 + E, n);
    int own = 0;
    for (int c = e0; c < e1; ++c) own += off[c];
    int incl = own;
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        const int y = __shfl_up(incl, d, WAVE);
        if (lane_id() >= d) incl += y;
    }
    if (lane_id() == WAVE - 1) wsum[tid / WAVE] = incl;
    __syncthreads();
    int base = incl - own;
    for (int w = 0; w < tid / WAVE; ++w) base += wsum[w];
    for (int c = e0; c < e1; ++c) {
        const int cnt = off[c];
        off[c] = base;
        if (c > 0 && ((c & 3) == 0 || c == n - 1)) qbs[(c - 1) >> 2] = base;
        base += cnt;
    }
    __syncthreads();
}

// Segments of up to GQ_STAGE queries: a thread's GQ_I queries stay in registers from the load to the placement (one
// load and one search each), and the grouped segment is staged in LDS (sv, si) and stored coalesced. The workgroup's
// GQ_T threads group one segment; key_at(i) is the segment's i-th smallest key.
constexpr int GQ_I = GQ_STAGE / GQ_T;

template <int CH, class KeyAt>
__device__ __forceinline__ void group_segment(KeyAt key_at, const float* __restrict__ qseg, float* __restrict__ qso,
                                              uint32_t* __restrict__ qpo, int* __restrict__ qbs, const float qshift,
                                              const int Ns, const int Mq, const int Gc, GroupTables& tb,
                                              float* __restrict__ sv, uint32_t* __restrict__ si)
{
    const int tid = threadIdx.x;
    float x[GQ_I];
#pragma unroll
    for (int j = 0; j < GQ_I; ++j) x[j] = qseg[min(tid + j * GQ_T, Mq - 1)];   // clamped: all loads in flight
    for (int c = tid; c < Gc; c += GQ_T) {
        const float y = key_at(min(Ns, (c + 1) * CH) - 1);
        tb.bnd[c] = y;
        if ((c & 3) == 3 || c == Gc - 1) tb.rb[c >> 2] = y;
    }
    for (int c = tid; c <= Gc; c += GQ_T) tb.off[c] = 0;
    __syncthreads();
    // the searches in two interleaved batches of GQ_I / 2: fewer registers (the sort + grouping kernel runs beside a
    // reduce whose waves need the SIMDs' spare registers)
    int b[GQ_I];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        float xs[GQ_I / 2];
        int bh[GQ_I / 2];
#pragma unroll
        for (int j = 0; j < GQ_I / 2; ++j) xs[j] = x[h * (GQ_I / 2) + j] + qshift;
        buckets<GQ_I / 2>(tb.bnd, tb.rb, Gc, xs, bh);
#pragma unroll
        for (int j = 0; j < GQ_I / 2; ++j) b[h * (GQ_I / 2) + j] = bh[j];
    }
#pragma unroll
    for (int j = 0; j < GQ_I; ++j)
        if (tid + j * GQ_T < Mq) atomicAdd(&tb.off[b[j]], 1);
    __syncthreads();
    group_scan(tb.off, tb.wsum, Gc + 1, qbs);
#pragma unroll
    for (int j = 0; j < GQ_I; ++j) {
        const int i = tid + j * GQ_T;
        if (i < Mq) {
            const int pos = atomicAdd(&tb.off[b[j]], 1);
            sv[pos] = x[j];
            si[pos] = (uint32_t)i;
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < GQ_I; ++j) {
        const int i = tid + j * GQ_T;
        if (i < Mq) { qso[i] = sv[i]; qpo[i] = si[i]; }
    }
}

}  // namespace qlka
