// Stage 1 of the hot path: per-segment stable ascending sort of fp32 keys with a uint32 permutation payload.
//
// Replaces the reference's CUB segmented radix sort + iota (Weighted_Abs_Sum/csrc/sort_utils.cu:17-117,
// Weighted_Laplace_Sum/csrc/sort_utils.cu:14-126) with gfx950 kernels of our own:
//  * lds_count_sort6 (runs of 8193 .. 16384 keys, and the runs of longer segments): one 512-thread workgroup sorts
//    one run entirely in LDS, 6 LSD passes of 6-bit digits ranked with per-thread digit counters (no ballots), two
//    16-bit counters to a word; see the kernel.
//  * lds_count_sort (runs of 4097 .. 8192 keys): the same ranking with 4-bit digits and 32-bit counters, 8 passes,
//    512 threads of 16 keys (the six-pass kernel's 256-thread form measured slower there: 0.070 vs 0.068 ms for
//    768 runs of 8192).
//  * lds_radix_sort (runs of up to 4096 keys): one workgroup sorts one run entirely in LDS, 4 LSD passes of 8-bit
//    digits. Stable ranking inside a wave uses 8 ballots to find the lanes that share a digit (no match instruction on
//    CDNA), per-wave digit counters in LDS, and a digit-major exclusive scan.
//  * merge_runs: for segments longer than one LDS run, stable merge-path merges of sorted runs (ties keep the left
//    run first), ping-ponging between two scratch buffers; the last pass writes floats + perm.
// Output contract: sorted[i] are the keys in stable ascending order (-0.0 written as +0.0), perm[i] the index within
// the segment of the i-th smallest key (== np.argsort(kind="stable")).
#include "qlka_common.h"
#include "qlka_internal.h"

#include <atomic>
#include <utility>

namespace qlka {

template <int WAVES, int ITEMS>
__global__ __launch_bounds__(WAVES * WAVE)
void lds_radix_sort(const float* __restrict__ in1, const int seg_len, const int run_len, const int runs_per_seg,
                    float* __restrict__ out_keys1, uint32_t* __restrict__ out_perm1,      // direct output (1 run)
                    uint32_t* __restrict__ run_keys, uint32_t* __restrict__ run_idx,       // run output (merging)
                    const int blocks1, const float* __restrict__ in2, float* __restrict__ out_keys2,
                    uint32_t* __restrict__ out_perm2)                                     // second array (1 run)
{
    // blocks [0, blocks1) sort the segments of in1, the blocks after them those of in2 (same segment length), so that
    // two arrays are sorted by one launch
    const bool second = (int)blockIdx.x >= blocks1;
    const int bid = second ? (int)blockIdx.x - blocks1 : (int)blockIdx.x;
    const float* in = second ? in2 : in1;
    float* out_keys = second ? out_keys2 : out_keys1;
    uint32_t* out_perm = second ? out_perm2 : out_perm1;
    constexpr int THREADS = WAVES * WAVE;
    constexpr int CAP     = THREADS * ITEMS;
    __shared__ uint32_t skey[CAP];
    __shared__ uint32_t sidx[CAP];
    __shared__ uint32_t hist[WAVES * 256];
    __shared__ uint32_t dbase[256];

    const int seg   = bid / runs_per_seg;
    const int run   = bid - seg * runs_per_seg;
    const int start = run * run_len;
    const int len   = min(run_len, seg_len - start);
    const size_t seg_off = (size_t)seg * seg_len;
    const float* src = in + seg_off + start;

    const int tid  = threadIdx.x;
    const int wave = tid / WAVE;
    const int lane = tid & (WAVE - 1);
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (WAVE - lane));

    float f[ITEMS];
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) f[r] = src[min(tid + r * THREADS, len - 1)];   // clamped: all ITEMS in flight
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
        const int i = tid + r * THREADS;
        // pads become 0xffffffff and sort after every key; f is used unconditionally so that the compiler keeps
        // the loads above unpredicated (a predicated load would wait for each one in turn)
        skey[i] = float_to_ordered(f[r]) | ((i < len) ? 0u : 0xffffffffu);
        sidx[i] = (uint32_t)i;                            // index inside the run (< 16384)
    }

#pragma unroll 1
    for (int shift = 0; shift < 32; shift += 8) {
        // Each wave clears only its own counter row: the previous pass's scatter of this wave (which reads that row)
        // has already completed in program order, while other waves may still be scattering with their rows.
        for (int i = lane; i < 256; i += WAVE) hist[wave * 256 + i] = 0u;
        __syncthreads();                                  // every scatter done, every row cleared

        // pk = run index << 16 | offset within the wave's digit. The keys are read again after the ranking (skey is
        // not written until the scatter), so the ranking holds only pk and one key at a time in registers.
        uint32_t key[ITEMS], pk[ITEMS];
        const int wbase = wave * WAVE * ITEMS;
#pragma unroll
        for (int r = 0; r < ITEMS; ++r) pk[r] = sidx[wbase + r * WAVE + lane] << 16;   // item (wave, r, lane)
#pragma unroll
        for (int r = 0; r < ITEMS; ++r) {
            const uint32_t dig = (skey[wbase + r * WAVE + lane] >> shift) & 255u;
            uint64_t peers = ~0ull;
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const bool bit    = (dig >> b) & 1u;
                const uint64_t m  = __ballot(bit);
                peers &= bit ? m : ~m;
            }
            const uint32_t below = (uint32_t)__popcll(peers & lt_mask);
            const uint32_t cnt   = (uint32_t)__popcll(peers);
            const uint32_t old   = hist[wave * 256 + dig];   // every peer reads before the leader's write below
            if (below == 0) hist[wave * 256 + dig] = old + cnt;
            pk[r] |= old + below;
        }
        __syncthreads();                                  // all per-wave digit counts final
#pragma unroll
        for (int r = 0; r < ITEMS; ++r) key[r] = skey[wbase + r * WAVE + lane];

        for (int d = tid; d < 256; d += THREADS) {        // exclusive over waves (digit-major order)
            uint32_t run_sum = 0;
            for (int w = 0; w < WAVES; ++w) {
                const uint32_t c = hist[w * 256 + d];
                hist[w * 256 + d] = run_sum;
                run_sum += c;
            }
            dbase[d] = run_sum;
        }
        __syncthreads();
        if (wave == 0) {                                  // exclusive scan of the 256 digit totals
            uint32_t a0 = dbase[lane * 4 + 0], a1 = dbase[lane * 4 + 1];
            uint32_t a2 = dbase[lane * 4 + 2], a3 = dbase[lane * 4 + 3];
            uint32_t s = a0 + a1 + a2 + a3, incl = s;
#pragma unroll
            for (int o = 1; o < WAVE; o <<= 1) {
                uint32_t y = (uint32_t)__shfl_up((int)incl, o, WAVE);
                if (lane >= o) incl += y;
            }
            uint32_t e = incl - s;
            dbase[lane * 4 + 0] = e; e += a0;
            dbase[lane * 4 + 1] = e; e += a1;
            dbase[lane * 4 + 2] = e; e += a2;
            dbase[lane * 4 + 3] = e;
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < ITEMS; ++r) {
            const uint32_t dig  = (key[r] >> shift) & 255u;
            const uint32_t dest = dbase[dig] + hist[wave * 256 + dig] + (pk[r] & 0xffffu);
            skey[dest] = key[r];
            sidx[dest] = pk[r] >> 16;
        }
    }
    __syncthreads();

    if (runs_per_seg == 1) {
        for (int i = tid; i < len; i += THREADS) {
            out_keys[seg_off + i] = ordered_to_float(skey[i]);
            out_perm[seg_off + i] = (uint32_t)start + sidx[i];
        }
    } else {
        for (int i = tid; i < len; i += THREADS) {
            run_keys[seg_off + start + i] = skey[i];
            run_idx[seg_off + start + i]  = (uint32_t)start + sidx[i];
        }
    }
}

// Counter-based stable LDS sort for runs of up to THREADS * 16 keys (the long runs: 8192 and 16384 keys). Thread t
// owns the 16 consecutive positions 16t .. 16t + 15 of the current order ("blocked"). Each of 8 LSD passes over 4-bit
// digits:
//  1. every thread counts its items per digit in its own column of a [16 digits][THREADS] counter table (LDS
//     atomics that return the old count, so an item also learns how many of the thread's earlier items share its
//     digit; a column has one writer, so the counts do not depend on timing);
//  2. one exclusive scan of the table in digit-major order (each thread rakes 16 consecutive counters, a workgroup
//     scan joins the threads) turns every counter into the first output slot of its (digit, thread);
//  3. item rank = its (digit, thread) slot + its count among the thread's earlier items: stable, since positions are
//     ordered thread-major and, within a thread, item by item;
//  4. keys and indices are scattered to their ranks and read back blocked for the next pass.
// No ballots: about 8 VALU instructions per item and pass for the ranking, against about 98 for the 8-ballot digit
// match of lds_radix_sort, which made that kernel VALU-bound. The table lives in the key array while the keys are in
// registers (steps 1-3). LDS arrays are padded by one word per 16, so a blocked access (thread t at 16t + j) and a
// counter rake hit 64 different banks.
constexpr int CS_ITEMS = 16;
constexpr int CS_BITS = 4;
constexpr int CS_DIGITS = 1 << CS_BITS;
__device__ __forceinline__ int cs_pad(int i) { return i + (i >> 4); }

template <int THREADS>
struct CountSortLds {
    uint32_t key[THREADS * (CS_ITEMS + 1)];    // padded keys; the digit counters during ranking
    uint32_t idx[THREADS * (CS_ITEMS + 1)];    // padded positions in the run
    uint32_t wsum[THREADS / WAVE];
};
static_assert(CS_DIGITS <= CS_ITEMS, "the digit counters must fit the key array");

// Exclusive workgroup scan of one value per thread (wave scan, then the waves' totals through LDS).
template <int THREADS>
__device__ __forceinline__ uint32_t cs_block_scan(const uint32_t x, uint32_t* wsum) {
    const int lane = lane_id(), w = threadIdx.x / WAVE;
    uint32_t incl = x;
#pragma unroll
    for (int off = 1; off < WAVE; off <<= 1) {
        const uint32_t y = (uint32_t)__shfl_up((int)incl, off, WAVE);
        if (lane >= off) incl += y;
    }
    if (lane == WAVE - 1) wsum[w] = incl;
    __syncthreads();
    uint32_t base = 0;
#pragma unroll
    for (int i = 0; i < THREADS / WAVE; ++i) base += (i < w) ? wsum[i] : 0u;
    return base + incl - x;
}

// The run's sort in LDS: on return sm.key / sm.idx hold the sorted run at padded positions (ordered keys and positions
// in the run). All THREADS threads of the workgroup take part.
template <int THREADS>
__device__ __forceinline__ void count_sort_run(CountSortLds<THREADS>& sm, const float* __restrict__ src, const int len)
{
    const int t = threadIdx.x;
    // striped loads (coalesced, all in flight) into the padded LDS order; pads sort after every key
    {
        float f[CS_ITEMS];
#pragma unroll
        for (int r = 0; r < CS_ITEMS; ++r) f[r] = src[min(t + r * THREADS, len - 1)];
#pragma unroll
        for (int r = 0; r < CS_ITEMS; ++r) {
            const int i = t + r * THREADS;
            sm.key[cs_pad(i)] = float_to_ordered(f[r]) | ((i < len) ? 0u : 0xffffffffu);
            sm.idx[cs_pad(i)] = (uint32_t)i;
        }
    }

    uint32_t* const cnt = sm.key;
#pragma unroll 1
    for (int shift = 0; shift < 32; shift += CS_BITS) {
        __syncthreads();                                  // the previous scatter (or the load) is complete
        uint32_t key[CS_ITEMS];
#pragma unroll
        for (int j = 0; j < CS_ITEMS; ++j) key[j] = sm.key[cs_pad(CS_ITEMS * t + j)];
        __syncthreads();                                  // every thread holds its keys: the key array is free
        // 1. this thread's column of the counter table, and each item's count among the thread's earlier items
#pragma unroll
        for (int d = 0; d < CS_DIGITS; ++d) cnt[cs_pad(d * THREADS + t)] = 0u;
        uint32_t rank[CS_ITEMS];
#pragma unroll
        for (int j = 0; j < CS_ITEMS; ++j) {
            const int d = (int)((key[j] >> shift) & (CS_DIGITS - 1));
            rank[j] = atomicAdd(&cnt[cs_pad(d * THREADS + t)], 1u);
        }
        __syncthreads();
        // 2. exclusive scan of the table in digit-major order: thread t rakes counters 16t .. 16t + 15
        {
            uint32_t s = 0;
#pragma unroll
            for (int i = 0; i < CS_ITEMS; ++i) s += cnt[cs_pad(CS_ITEMS * t + i)];
            uint32_t base = cs_block_scan<THREADS>(s, sm.wsum);
#pragma unroll
            for (int i = 0; i < CS_ITEMS; ++i) {
                const uint32_t c = cnt[cs_pad(CS_ITEMS * t + i)];
                cnt[cs_pad(CS_ITEMS * t + i)] = base;
                base += c;
            }
        }
        __syncthreads();
        // 3. ranks
#pragma unroll
        for (int j = 0; j < CS_ITEMS; ++j) {
            const int d = (int)((key[j] >> shift) & (CS_DIGITS - 1));
            rank[j] += cnt[cs_pad(d * THREADS + t)];
        }
        uint32_t idx[CS_ITEMS];
#pragma unroll
        for (int j = 0; j < CS_ITEMS; ++j) idx[j] = sm.idx[cs_pad(CS_ITEMS * t + j)];
        __syncthreads();                                  // every rank and index read: both arrays take the scatter
        // 4. scatter
#pragma unroll
        for (int j = 0; j < CS_ITEMS; ++j) {
            sm.key[cs_pad((int)rank[j])] = key[j];
            sm.idx[cs_pad((int)rank[j])] = idx[j];
        }
    }
    __syncthreads();
}

// Only the keys and their counts stay in registers through a pass (the indices are read just before the scatter).
// In its 1024-thread form (16384-key runs, before the six-pass kernel) that held it to 103 VGPRs, so that the 16 waves
// of a workgroup left room in each SIMD's registers for the waves of the previous chunk's slab reduce, which runs
// beside the sort (at 127 VGPRs no reduce wave fitted beside it and each op took 0.02-0.04 ms longer).
template <int THREADS>
__global__ __launch_bounds__(THREADS)
void lds_count_sort(const float* __restrict__ in1, const int seg_len, const int run_len, const int runs_per_seg,
                    float* __restrict__ out_keys1, uint32_t* __restrict__ out_perm1,
                    uint32_t* __restrict__ run_keys, uint32_t* __restrict__ run_idx,
                    const int blocks1, const float* __restrict__ in2, float* __restrict__ out_keys2,
                    uint32_t* __restrict__ out_perm2)
{
    const bool second = (int)blockIdx.x >= blocks1;
    const int bid = second ? (int)blockIdx.x - blocks1 : (int)blockIdx.x;
    const float* in = second ? in2 : in1;
    float* out_keys = second ? out_keys2 : out_keys1;
    uint32_t* out_perm = second ? out_perm2 : out_perm1;
    __shared__ CountSortLds<THREADS> sm;

    const int seg   = bid / runs_per_seg;
    const int run   = bid - seg * runs_per_seg;
    const int start = run * run_len;
    const int len   = min(run_len, seg_len - start);
    const size_t seg_off = (size_t)seg * seg_len;
    count_sort_run<THREADS>(sm, in + seg_off + start, len);

    // the sorted run is in LDS: striped, coalesced stores
    const int t = threadIdx.x;
    if (runs_per_seg == 1) {
        for (int i = t; i < len; i += THREADS) {
            out_keys[seg_off + i] = ordered_to_float(sm.key[cs_pad(i)]);
            out_perm[seg_off + i] = (uint32_t)start + sm.idx[cs_pad(i)];
        }
    } else {
        for (int i = t; i < len; i += THREADS) {
            run_keys[seg_off + start + i] = sm.key[cs_pad(i)];
            run_idx[seg_off + start + i]  = (uint32_t)start + sm.idx[cs_pad(i)];
        }
    }
}

// ---- six-pass counting sort
// The same ranking as count_sort_run with 6-bit digits: 6 LSD passes (bits 0-5, ..., 24-29, 30-31) instead of 8.
// Each thread holds C6_ITEMS = 32 consecutive positions (32t .. 32t + 31), so THREADS = 512 cover 16384 keys and the
// workgroup has 8 waves. The counter table has 64 digits per thread; its counts stay below 2^16 (a thread's own at
// most 32, a first slot at most 16384), so the two digits 2dp and 2dp + 1 of a thread share one 32-bit word, low and
// high half: [32 digit pairs][THREADS] words, as many as the 4-bit table's [16][1024], so a pass moves the same LDS
// words as a 4-bit pass over 16 items and 1024 threads. LDS arrays are padded by one word per 32 (blocked accesses at
// 33t + j and the rake hit 64 different banks; a thread's own counter words spread over about 3 accesses a bank).
// Measured on MI355X against the 8-pass kernel (1024 threads of 16 keys): 256 runs of 16384 keys 0.0535 -> 0.0473 ms,
// 64 segments of 131072 (with the merges) 0.224 -> 0.210 ms, both forward ops 0.6-0.8% faster. The workgroup's 8 waves
// take 189 VGPRs each (LDS holds one workgroup per CU, so 2 waves per SIMD whatever the count); they leave a SIMD
// 128 registers, 5 waves of the reduce that runs beside the sort (the 8-pass kernel's 4 waves at 103 left 4).
constexpr int C6_ITEMS = 32;
constexpr int C6_BITS = 6;
constexpr int C6_PAIRS = 1 << (C6_BITS - 1);        // digit pairs (counter words per thread)
__device__ __forceinline__ int c6_pad(int i) { return i + (i >> 5); }

template <int THREADS>
struct CountSort6Lds {
    uint32_t key[THREADS * (C6_ITEMS + 1)];         // padded keys; the digit counters during ranking
    uint32_t idx[THREADS * (C6_ITEMS + 1)];         // padded positions in the run
    uint32_t wsum[THREADS / WAVE];
};
static_assert(C6_PAIRS <= C6_ITEMS, "the digit counters must fit the key array");

// Exclusive scan, in digit-major order, of the counter table's rake sums: rake thread t = dp * BLKS + blk holds the
// sums a (digit 2dp) and b (digit 2dp + 1) of threads 32 blk .. 32 blk + 31 of digit pair dp. In digit-major order
// the sums of one digit pair are a of blocks 0 .. BLKS - 1, then b of blocks 0 .. BLKS - 1; a digit pair's BLKS rake
// threads are consecutive lanes of one wave, and the waves hold consecutive digit pairs.
template <int THREADS>
__device__ __forceinline__ void c6_scan(const uint32_t a, const uint32_t b, uint32_t* wsum, uint32_t& a_ex,
                                        uint32_t& b_ex) {
    constexpr int BLKS = THREADS / 32;
    static_assert(BLKS <= WAVE && WAVE % BLKS == 0, "a digit pair's rake threads lie in one wave");
    const int lane = lane_id(), w = threadIdx.x / WAVE, gb = lane % BLKS, g0 = lane - gb;
    uint32_t ai = a, bi = b;                         // inclusive scans within the digit pair
#pragma unroll
    for (int off = 1; off < BLKS; off <<= 1) {
        const uint32_t ya = (uint32_t)__shfl_up((int)ai, off, WAVE), yb = (uint32_t)__shfl_up((int)bi, off, WAVE);
        if (gb >= off) { ai += ya; bi += yb; }
    }
    const uint32_t A = (uint32_t)__shfl((int)ai, g0 + BLKS - 1, WAVE);   // the pair's digit 2dp total
    const uint32_t B = (uint32_t)__shfl((int)bi, g0 + BLKS - 1, WAVE);
    uint32_t gi = (gb == BLKS - 1) ? A + B : 0u;    // inclusive scan of the pairs' totals over the wave
#pragma unroll
    for (int off = 1; off < WAVE; off <<= 1) {
        const uint32_t y = (uint32_t)__shfl_up((int)gi, off, WAVE);
        if (lane >= off) gi += y;
    }
    const uint32_t before = (uint32_t)__shfl((int)gi, g0 > 0 ? g0 - 1 : 0, WAVE);
    const uint32_t gex = g0 > 0 ? before : 0u;       // the wave's pairs before this one
    if (lane == WAVE - 1) wsum[w] = gi;
    __syncthreads();
    uint32_t base = 0;
#pragma unroll
    for (int i = 0; i < THREADS / WAVE; ++i) base += (i < w) ? wsum[i] : 0u;
    a_ex = base + gex + ai - a;
    b_ex = base + gex + A + bi - b;
}

// The run's sort in LDS. The two arrays trade roles every pass: after the ranks are known (the counter table, in the
// key array, is then dead), each thread streams its indices from the index array into the key array at their ranks,
// and then its keys, held in registers, into the index array: only the keys and the packed ranks stay live across a
// pass, and no extra barrier is needed between the two scatters' reads and writes. Returns the array that holds the
// sorted keys (the other holds the positions), at padded positions.
template <int THREADS, bool OPAQUE_T = false>
__device__ __forceinline__ bool count_sort6_run(CountSort6Lds<THREADS>& sm, const float* __restrict__ src,
                                                const int len)
{
    constexpr int BLKS = THREADS / 32;
    constexpr int ROW = THREADS + THREADS / 32;       // padded words of one digit pair's counter row
    int t = threadIdx.x;
    // OPAQUE_T, for a kernel that sorts several runs in a loop: an opaque copy of t, or the addresses derived from it
    // are hoisted out of that loop and kept live through every pass (256 VGPRs and spills)
    if constexpr (OPAQUE_T) asm volatile("" : "+v"(t));
    {
        float f[C6_ITEMS];
#pragma unroll
        for (int r = 0; r < C6_ITEMS; ++r) f[r] = src[min(t + r * THREADS, len - 1)];
#pragma unroll
        for (int r = 0; r < C6_ITEMS; ++r) {
            const int i = t + r * THREADS;
            sm.key[c6_pad(i)] = float_to_ordered(f[r]) | ((i < len) ? 0u : 0xffffffffu);
            sm.idx[c6_pad(i)] = (uint32_t)i;
        }
    }
    // Padded addresses written out (the compiler does not see that c6_pad(32 t + j) = 33 t + j, and would keep 32 of
    // each kind live): this thread's blocked positions, its counter column, its rake words.
    const int blk0 = (C6_ITEMS + 1) * t;
    const int col = t + (t >> 5);
    const int rbase = (t / BLKS) * ROW + 33 * (t % BLKS);
    bool swapped = false;                             // keys in sm.idx, positions in sm.key
#pragma unroll 1
    for (int shift = 0; shift < 32; shift += C6_BITS) {
        uint32_t* const keys = swapped ? sm.idx : sm.key;
        uint32_t* const pos = swapped ? sm.key : sm.idx;
        uint32_t* const cnt = keys;                   // the counter table takes the key array while keys are in VGPRs
        __syncthreads();                              // the previous scatter (or the load) is complete
        uint32_t key[C6_ITEMS];
#pragma unroll
        for (int j = 0; j < C6_ITEMS; ++j) key[j] = keys[blk0 + j];
        __syncthreads();                              // every thread holds its keys: the key array is free
        // 1. this thread's counter words, and each item's count among the thread's earlier items (8 bits each, four
        //    to a register)
#pragma unroll
        for (int dp = 0; dp < C6_PAIRS; ++dp) cnt[dp * ROW + col] = 0u;
        uint32_t lc[C6_ITEMS / 4];
#pragma unroll
        for (int j = 0; j < C6_ITEMS; ++j) {
            const uint32_t d = (key[j] >> shift) & ((1u << C6_BITS) - 1);
            const uint32_t h = 16u * (d & 1u);       // the digit's half of the word
            const uint32_t old = atomicAdd(&cnt[(int)(d >> 1) * ROW + col], 1u << h);
            const uint32_t c = (old >> h) & 0xffffu;
            if (j % 4 == 0) lc[j / 4] = c;
            else lc[j / 4] |= c << (8 * (j % 4));
        }
        __syncthreads();
        // 2. exclusive scan of the table in digit-major order: this thread rakes 32 words of one digit pair
        {
            uint32_t rw[32];
            uint32_t sa = 0, sb = 0;
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                rw[i] = cnt[rbase + i];
                sa += rw[i] & 0xffffu;
                sb += rw[i] >> 16;
            }
            uint32_t ea, eb;
            c6_scan<THREADS>(sa, sb, sm.wsum, ea, eb);
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                cnt[rbase + i] = ea | (eb << 16);
                ea += rw[i] & 0xffffu;
                eb += rw[i] >> 16;
            }
        }
        __syncthreads();
        // 3. ranks (two to a register). Digits and counter addresses are computed again from opaque copies of the
        //    shift and the column: kept from step 1 instead, 64 more values would stay live across the scan.
        int sh = shift, cl = col;
        asm volatile("" : "+s"(sh), "+v"(cl));
        const uint16_t* const cnt16 = reinterpret_cast<const uint16_t*>(cnt);
        uint32_t rk[C6_ITEMS / 2];
#pragma unroll
        for (int j = 0; j < C6_ITEMS; ++j) {
            const uint32_t d = (key[j] >> sh) & ((1u << C6_BITS) - 1);
            const uint32_t first = cnt16[2 * ((int)(d >> 1) * ROW + cl) + (int)(d & 1u)];
            const uint32_t r = first + ((lc[j / 4] >> (8 * (j % 4))) & 0xffu);
            if (j % 2 == 0) rk[j / 2] = r;
            else rk[j / 2] |= r << 16;
        }
        __syncthreads();                              // every rank read: the key array takes the positions
        // 4. positions into the key array, then (all positions read) keys into the position array
#pragma unroll
        for (int j = 0; j < C6_ITEMS; ++j) {
            const int r = (int)((rk[j / 2] >> (16 * (j % 2))) & 0xffffu);
            keys[c6_pad(r)] = pos[blk0 + j];
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < C6_ITEMS; ++j) {
            const int r = (int)((rk[j / 2] >> (16 * (j % 2))) & 0xffffu);
            pos[c6_pad(r)] = key[j];
        }
        swapped = !swapped;
    }
    __syncthreads();
    return swapped;
}

// One run per workgroup: runs of segments that fit one LDS run (runs_per_seg == 1).
template <int THREADS>
__global__ __launch_bounds__(THREADS)
void lds_count_sort6(const float* __restrict__ in1, const int seg_len, const int run_len, const int runs_per_seg,
                     float* __restrict__ out_keys1, uint32_t* __restrict__ out_perm1,
                     uint32_t* __restrict__ run_keys, uint32_t* __restrict__ run_idx,
                     const int blocks1, const float* __restrict__ in2, float* __restrict__ out_keys2,
                     uint32_t* __restrict__ out_perm2)
{
    const bool second = (int)blockIdx.x >= blocks1;
    const int bid = second ? (int)blockIdx.x - blocks1 : (int)blockIdx.x;
    const float* in = second ? in2 : in1;
    float* out_keys = second ? out_keys2 : out_keys1;
    uint32_t* out_perm = second ? out_perm2 : out_perm1;
    __shared__ CountSort6Lds<THREADS> sm;

    const int seg   = bid / runs_per_seg;
    const int run   = bid - seg * runs_per_seg;
    const int start = run * run_len;
    const int len   = min(run_len, seg_len - start);
    const size_t seg_off = (size_t)seg * seg_len;
    const bool swapped = count_sort6_run<THREADS>(sm, in + seg_off + start, len);
    const uint32_t* const keys = swapped ? sm.idx : sm.key;
    const uint32_t* const pos = swapped ? sm.key : sm.idx;

    const int t = threadIdx.x;
    if (runs_per_seg == 1) {
        for (int i = t; i < len; i += THREADS) {
            out_keys[seg_off + i] = ordered_to_float(keys[c6_pad(i)]);
            out_perm[seg_off + i] = (uint32_t)start + pos[c6_pad(i)];
        }
    } else {
        for (int i = t; i < len; i += THREADS) {
            run_keys[seg_off + start + i] = keys[c6_pad(i)];
            run_idx[seg_off + start + i]  = (uint32_t)start + pos[c6_pad(i)];
        }
    }
}

// Runs of segments longer than one LDS run (runs_per_seg > 1), into the run buffers for the merges (the second
// array's runs after the first array's segments). A grid of at most one workgroup per CU (LDS holds one) loops over
// the runs, so all of it is resident from its start and runs past the first round do not wait for CU slots behind a
// reduce that started beside them (configs[4], 512 runs of 16384 keys a p: 85.6 -> 84.7 ms a call).
template <int THREADS>
__global__ __launch_bounds__(THREADS)
void lds_count_sort6_runs(const float* __restrict__ in1, const int seg_len, const int run_len,
                          const int runs_per_seg, uint32_t* __restrict__ run_keys, uint32_t* __restrict__ run_idx,
                          const int blocks1, const float* __restrict__ in2)
{
    __shared__ CountSort6Lds<THREADS> sm;
    const int total = in2 ? 2 * blocks1 : blocks1;
    for (int b = blockIdx.x; b < total; b += gridDim.x) {
        const bool second = b >= blocks1;
        const int bid = second ? b - blocks1 : b;
        const float* in = second ? in2 : in1;
        const int seg   = bid / runs_per_seg;
        const int run   = bid - seg * runs_per_seg;
        const int start = run * run_len;
        const int len   = min(run_len, seg_len - start);
        const size_t seg_off = (size_t)seg * seg_len;
        const bool swapped = count_sort6_run<THREADS, true>(sm, in + seg_off + start, len);
        const uint32_t* const keys = swapped ? sm.idx : sm.key;
        const uint32_t* const pos = swapped ? sm.key : sm.idx;
        int t = threadIdx.x;
        asm volatile("" : "+v"(t));                       // (see count_sort6_run's OPAQUE_T)
        const size_t ro = seg_off + start + (second ? (size_t)(blocks1 / runs_per_seg) * seg_len : 0);
        for (int i = t; i < len; i += THREADS) {
            run_keys[ro + i] = keys[c6_pad(i)];
            run_idx[ro + i]  = (uint32_t)start + pos[c6_pad(i)];
        }
        __syncthreads();                                  // every read of this run's LDS is done before the next load
    }
}

// One stable merge pass: runs of `width` become runs of 2*width (A = the left run wins ties). A workgroup owns
// MERGE_TILE consecutive outputs of one pair of runs:
//  1. merge_partition, a launch before, finds where every tile starts on the merge path (the number of A elements
//     before its first output) with one wave per tile and a 64-way search per round (3 rounds for 64K-key runs
//     instead of 16 dependent steps); a tile ends where the next one of its pair starts (each boundary is searched
//     once: searched by both of its tiles, the scattered search reads were 2x the merge's own);
//  2. the tile's A and B slices (MERGE_TILE keys + indices in total) are loaded into LDS, coalesced;
//  3. each thread finds its MERGE_ITEMS outputs' start on the merge path inside LDS and merges them;
//  4. the merged tile goes back through LDS and out coalesced (the final pass writes floats and perm).
constexpr int MERGE_ITEMS   = 8;
constexpr int MERGE_THREADS = 256;
constexpr int MERGE_TILE    = MERGE_ITEMS * MERGE_THREADS;

// Smallest i in [lo, hi] with A[i] > B[o - i - 1] (true at i = hi by convention): the number of A elements among the
// first o outputs of the stable merge. Runs in one wave, 64 candidates per round.
__device__ int merge_path_wave(const uint32_t* __restrict__ A, const uint32_t* __restrict__ B, int o, int lo, int hi) {
    const int lane = lane_id();
    while (lo < hi) {
        const int step = (hi - lo + WAVE - 1) / WAVE;
        const int i = lo + lane * step;
        const bool p = i >= hi || A[i] > B[o - i - 1];
        const uint64_t m = __ballot(p);
        if (m == 0) { lo = lo + (WAVE - 1) * step + 1; continue; }
        const int f = __builtin_ctzll(m);
        if (f == 0) { hi = lo; break; }
        const int nlo = lo + (f - 1) * step + 1;
        hi = min(hi, lo + f * step);
        lo = nlo;
    }
    return lo;
}

// splits[seg * blocks_per_seg + blk]: A elements before tile blk's first output within its pair (one wave per tile)
__global__ __launch_bounds__(MERGE_THREADS)
void merge_partition(const uint32_t* __restrict__ src_k, int* __restrict__ splits, const int seg_len, const int width,
                     const int blocks_per_seg, const int tiles)
{
    const int t = blockIdx.x * (MERGE_THREADS / WAVE) + wave_in_block();
    if (t >= tiles) return;                               // whole wave
    const int seg = t / blocks_per_seg, blk = t - seg * blocks_per_seg;
    const int o0 = blk * MERGE_TILE;
    const size_t so = (size_t)seg * seg_len;
    const int pair0 = (o0 / (2 * width)) * (2 * width);
    const int la    = min(width, seg_len - pair0);
    const int lb    = max(0, min(width, seg_len - pair0 - la));
    const int ob    = o0 - pair0;
    const int i = merge_path_wave(src_k + so + pair0, src_k + so + pair0 + la, ob, max(0, ob - lb), min(ob, la));
    if (lane_id() == 0) splits[t] = i;
}

__global__ __launch_bounds__(MERGE_THREADS)
void merge_runs(const uint32_t* __restrict__ src_k, const uint32_t* __restrict__ src_i,
                uint32_t* __restrict__ dst_k, uint32_t* __restrict__ dst_i,
                float* __restrict__ out_keys, uint32_t* __restrict__ out_perm, const int* __restrict__ splits,
                const int seg_len, const int width, const int final_pass, const int blocks_per_seg,
                const int S1, float* __restrict__ out_keys2, uint32_t* __restrict__ out_perm2)
{
    __shared__ uint32_t sk[MERGE_TILE];
    __shared__ uint32_t si[MERGE_TILE];
    const int seg = blockIdx.x / blocks_per_seg;
    const int blk = blockIdx.x - seg * blocks_per_seg;
    const int o0  = blk * MERGE_TILE;                     // tile start within the segment
    if (o0 >= seg_len) return;                            // whole workgroup
    const int tid = threadIdx.x;
    const size_t so = (size_t)seg * seg_len;
    const int pair0 = (o0 / (2 * width)) * (2 * width);
    const int la    = min(width, seg_len - pair0);
    const int b0    = pair0 + la;
    const int lb    = max(0, min(width, seg_len - b0));
    const uint32_t* A  = src_k + so + pair0;
    const uint32_t* B  = src_k + so + b0;
    const uint32_t* Ai = src_i + so + pair0;
    const uint32_t* Bi = src_i + so + b0;
    const int ob = o0 - pair0, oe = min(ob + MERGE_TILE, la + lb);   // tile outputs [ob, oe) of the pair
    // the next tile of the same pair starts where this one ends; the pair's last tile ends with all of A
    const int* sp = splits + (size_t)seg * blocks_per_seg + blk;
    const int ia = sp[0], iend = oe < la + lb ? sp[1] : la;
    const int na = iend - ia;
    const int jb = ob - ia, nb = (oe - iend) - jb;
    const int n = na + nb;                                // == oe - ob
    // two loops, not one with a select: the select form loads both sources for every element (2x the reads)
    for (int e = tid; e < na; e += MERGE_THREADS) {
        sk[e] = A[ia + e];
        si[e] = Ai[ia + e];
    }
    for (int e = tid; e < nb; e += MERGE_THREADS) {
        sk[na + e] = B[jb + e];
        si[na + e] = Bi[jb + e];
    }
    __syncthreads();
    // this thread's outputs d .. d + MERGE_ITEMS - 1 of the tile: A part sk[0, na), B part sk[na, n)
    const int d = min(tid * MERGE_ITEMS, n);
    int lo = max(0, d - nb), hi = min(d, na);
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sk[mid] <= sk[na + d - mid - 1]) lo = mid + 1; else hi = mid;
    }
    int i = lo, j = d - lo;
    uint32_t rk[MERGE_ITEMS], ri[MERGE_ITEMS];
#pragma unroll
    for (int t = 0; t < MERGE_ITEMS; ++t) {
        const bool takea = i < na && (j >= nb || sk[i] <= sk[na + j]);
        const int at = takea ? i : na + j;
        rk[t] = sk[at];
        ri[t] = si[at];
        i += takea;
        j += !takea;
    }
    __syncthreads();                                      // every read of the inputs in LDS is done
#pragma unroll
    for (int t = 0; t < MERGE_ITEMS; ++t)
        if (d + t < n) { sk[d + t] = rk[t]; si[d + t] = ri[t]; }
    __syncthreads();
    if (final_pass) {
        // segments from S1 on belong to the second array (two arrays merged in one pass)
        const bool second = seg >= S1;
        float* const ok = second ? out_keys2 : out_keys;
        uint32_t* const op = second ? out_perm2 : out_perm;
        const size_t fo = (size_t)(second ? seg - S1 : seg) * seg_len + o0;
        for (int e = tid; e < n; e += MERGE_THREADS) {
            ok[fo + e] = ordered_to_float(sk[e]);
            op[fo + e] = si[e];
        }
    } else {
        for (int e = tid; e < n; e += MERGE_THREADS) {
            dst_k[so + o0 + e] = sk[e];
            dst_i[so + o0 + e] = si[e];
        }
    }
}

// Compute units of the current device (cached per device).
static int device_cus() {
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

template <int WAVES, int ITEMS>
static void launch_lds(const float* in, int S, int L, int run_len, int runs, float* ok, uint32_t* op,
                       uint32_t* rk, uint32_t* ri, hipStream_t st, const float* in2 = nullptr, float* ok2 = nullptr,
                       uint32_t* op2 = nullptr) {
    StageTimer t("lds_radix_sort", st);
    const int blocks1 = S * runs;
    hipLaunchKernelGGL((lds_radix_sort<WAVES, ITEMS>), dim3(in2 ? 2 * blocks1 : blocks1), dim3(WAVES * WAVE), 0, st,
                       in, L, run_len, runs, ok, op, rk, ri, blocks1, in2, ok2, op2);
}

template <int THREADS>
static void launch_cs(const float* in, int S, int L, int run_len, int runs, float* ok, uint32_t* op,
                      uint32_t* rk, uint32_t* ri, hipStream_t st, const float* in2 = nullptr, float* ok2 = nullptr,
                      uint32_t* op2 = nullptr) {
    StageTimer t("lds_count_sort", st);
    const int blocks1 = S * runs;
    hipLaunchKernelGGL((lds_count_sort<THREADS>), dim3(in2 ? 2 * blocks1 : blocks1), dim3(THREADS), 0, st,
                       in, L, run_len, runs, ok, op, rk, ri, blocks1, in2, ok2, op2);
}

template <int THREADS>
static void launch_cs6(const float* in, int S, int L, int run_len, int runs, float* ok, uint32_t* op,
                       uint32_t* rk, uint32_t* ri, hipStream_t st, const float* in2 = nullptr, float* ok2 = nullptr,
                       uint32_t* op2 = nullptr) {
    StageTimer t("lds_count_sort", st);
    const int blocks1 = S * runs, total = in2 ? 2 * blocks1 : blocks1;
    if (runs > 1)
        hipLaunchKernelGGL((lds_count_sort6_runs<THREADS>), dim3(std::min(total, device_cus())), dim3(THREADS), 0, st,
                           in, L, run_len, runs, rk, ri, blocks1, in2);
    else
        hipLaunchKernelGGL((lds_count_sort6<THREADS>), dim3(total), dim3(THREADS), 0, st,
                           in, L, run_len, runs, ok, op, rk, ri, blocks1, in2, ok2, op2);
}

static inline int merge_tiles(int L) { return (L + MERGE_TILE - 1) / MERGE_TILE; }

// Merge passes over the S segments of length L whose LDS-sorted runs are in (k0, i0): runs of LDS_SORT_MAX become one
// sorted run per segment, ping-ponging with (k1, i1); the last pass writes floats and permutations, segments from S1
// on to the second output. (The splits of the tiles follow the four run buffers in the scratch.)
static int merge_passes(uint32_t* k0, uint32_t* i0, uint32_t* k1, uint32_t* i1, int* splits, int S, int L, int S1,
                        float* out_keys, uint32_t* out_perm, float* out_keys2, uint32_t* out_perm2, hipStream_t st) {
    const int bps = merge_tiles(L);
    const int tiles = bps * S;
    const dim3 grid((unsigned)tiles), pgrid((unsigned)((tiles + MERGE_THREADS / WAVE - 1) / (MERGE_THREADS / WAVE)));
    for (int width = LDS_SORT_MAX; width < L; width *= 2) {
        const int fin = (2 * width >= L);
        StageTimer t("merge_runs", st);
        hipLaunchKernelGGL(merge_partition, pgrid, dim3(MERGE_THREADS), 0, st, k0, splits, L, width, bps, tiles);
        hipLaunchKernelGGL(merge_runs, grid, dim3(MERGE_THREADS), 0, st, k0, i0, k1, i1, out_keys, out_perm, splits,
                           L, width, fin, bps, S1, out_keys2, out_perm2);
        if (int err = (int)hipGetLastError()) return err;
        std::swap(k0, k1);
        std::swap(i0, i1);
    }
    return 0;
}

size_t seg_sort_scratch_bytes(int S, int L) {
    if (L <= LDS_SORT_MAX) return 0;
    // two (key, idx) ping-pong buffers and the merge pass's tile splits
    return 4 * (size_t)S * (size_t)L * sizeof(uint32_t) + (size_t)S * merge_tiles(L) * sizeof(int);
}

// One launch of the LDS sort over the S segments of `in` (and, with in2, those of in2) of length L <= LDS_SORT_MAX.
static int lds_sort(const float* in, float* out_keys, uint32_t* out_perm, const float* in2, float* out_keys2,
                    uint32_t* out_perm2, int S, int L, hipStream_t st) {
    // smallest (waves, items) whose capacity covers L; more waves for long runs keep 16 items per thread max
#define QLKA_LDS(W, I) launch_lds<W, I>(in, S, L, L, 1, out_keys, out_perm, nullptr, nullptr, st, in2, out_keys2, \
                                        out_perm2)
    if      (L <= 64)    QLKA_LDS(1, 1);
    else if (L <= 128)   QLKA_LDS(1, 2);
    else if (L <= 256)   QLKA_LDS(1, 4);
    else if (L <= 512)   QLKA_LDS(2, 4);
    else if (L <= 1024)  QLKA_LDS(4, 4);
    else if (L <= 2048)  QLKA_LDS(8, 4);
    else if (L <= 4096)  QLKA_LDS(16, 4);
#undef QLKA_LDS
    else if (L <= 8192)  launch_cs<512>(in, S, L, L, 1, out_keys, out_perm, nullptr, nullptr, st, in2, out_keys2,
                                        out_perm2);
    else                 launch_cs6<512>(in, S, L, L, 1, out_keys, out_perm, nullptr, nullptr, st, in2, out_keys2,
                                         out_perm2);
    return (int)hipGetLastError();
}

int seg_sort2(const float* a, float* a_keys, uint32_t* a_perm, const float* b, float* b_keys, uint32_t* b_perm,
              int S, int L, void* scratch, hipStream_t st) {
    if (S <= 0 || L <= 0) return 0;
    if (L <= LDS_SORT_MAX) return lds_sort(a, a_keys, a_perm, b, b_keys, b_perm, S, L, st);
    // both arrays' runs in one LDS-sort launch, then each merge pass over the 2S segments at once
    const size_t n = 2 * (size_t)S * (size_t)L;
    uint32_t* k0 = (uint32_t*)scratch;
    uint32_t* i0 = k0 + n;
    uint32_t* k1 = i0 + n;
    uint32_t* i1 = k1 + n;
    const int runs = (L + LDS_SORT_MAX - 1) / LDS_SORT_MAX;
    launch_cs6<512>(a, S, L, LDS_SORT_MAX, runs, nullptr, nullptr, k0, i0, st, b, nullptr, nullptr);
    if (int err = (int)hipGetLastError()) return err;
    return merge_passes(k0, i0, k1, i1, (int*)(i1 + n), 2 * S, L, S, a_keys, a_perm, b_keys, b_perm, st);
}

int seg_sort(const float* in, float* out_keys, uint32_t* out_perm, int S, int L, void* scratch,
             hipStream_t st) {
    if (S <= 0 || L <= 0) return 0;
    if (L <= LDS_SORT_MAX) return lds_sort(in, out_keys, out_perm, nullptr, nullptr, nullptr, S, L, st);
    const size_t n = (size_t)S * (size_t)L;
    uint32_t* k0 = (uint32_t*)scratch;
    uint32_t* i0 = k0 + n;
    uint32_t* k1 = i0 + n;
    uint32_t* i1 = k1 + n;
    const int runs = (L + LDS_SORT_MAX - 1) / LDS_SORT_MAX;
    launch_cs6<512>(in, S, L, LDS_SORT_MAX, runs, nullptr, nullptr, k0, i0, st);
    if (int err = (int)hipGetLastError()) return err;
    return merge_passes(k0, i0, k1, i1, (int*)(i1 + n), S, L, S, out_keys, out_perm, nullptr, nullptr, st);
}

}  // namespace qlka
