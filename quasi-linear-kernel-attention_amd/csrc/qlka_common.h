// Shared device helpers for the gfx950 (CDNA4, wave64) kernels of libqlka.
//
// Conventions used by every kernel in this library:
//  * A "segment" is one (p, d) pair: s = p * D + d. q is (P, D, M) and k is (P, D, N), so the M queries / N keys of
//    a segment are one contiguous run (layout of Weighted_Abs_Sum/weighted_abs_sum/ops.py:107-110 and
//    Weighted_Laplace_Sum/weighted_laplace_sum/__init__.py:4-12).
//  * Value rows (v, g) are (P, rows, C) row-major. In every walk a wave owns one key range and lane l owns channels
//    l and l + 64 (NV = 1 or 2 channel slots per lane), so one row gather is one coalesced 4*C-byte load.
//  * Sorted order is the stable ascending order of the fp32 values with -0.0 == +0.0 (the CUB contract at
//    Weighted_Abs_Sum/csrc/sort_utils.cu:85-87); the merge rank of a query is #{keys < query}
//    (np.searchsorted(side="left")), so a query is emitted before keys equal to it.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace qlka {

constexpr int WAVE = 64;

// ---------------------------------------------------------------------------------------------------------------
// fp32 <-> order-preserving uint32 (ascending uint order == ascending float order, -0.0 folded onto +0.0)
// ---------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t float_to_ordered(float f) {
    uint32_t b = __float_as_uint(f);
    if (b == 0x80000000u) b = 0u;                         // -0.0 sorts (and ties) as +0.0
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float ordered_to_float(uint32_t u) {
    uint32_t b = (u & 0x80000000u) ? (u & 0x7fffffffu) : ~u;
    return __uint_as_float(b);
}

// ---------------------------------------------------------------------------------------------------------------
// wave64 primitives
// ---------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (WAVE - 1)); }

// Index of this wave inside its workgroup, as a value the compiler knows is wave-uniform (so everything derived from
// it lives in SGPRs and buffer descriptors need no waterfall loop).
__device__ __forceinline__ int wave_in_block() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x / WAVE)); }

// value of x in lane `src` (src must be wave-uniform); lowers to v_readlane_b32
__device__ __forceinline__ float bcast(float x, int src) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), src));
}
__device__ __forceinline__ int bcast(int x, int src) { return __builtin_amdgcn_readlane(x, src); }
__device__ __forceinline__ uint32_t bcast(uint32_t x, int src) {
    return (uint32_t)__builtin_amdgcn_readlane((int)x, src);
}

// A value known to be wave-uniform, read from the first active lane so the compiler keeps it in SGPRs. The builtin
// returns a signed int: each 32-bit half is converted back to unsigned before it is widened, else a low word with bit
// 31 set would sign-extend over the high word of a 64-bit address.
__device__ __forceinline__ uint32_t uniform_u32(uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); }
__device__ __forceinline__ uint64_t uniform_u64(uint64_t x) {
    return (uint64_t)uniform_u32((uint32_t)x) | ((uint64_t)uniform_u32((uint32_t)(x >> 32)) << 32);
}

// number of lanes below this one whose bit is set in the wave-uniform mask m (v_mbcnt)
__device__ __forceinline__ int lanes_below(uint64_t m) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, WAVE);
    return x;
}

// Inclusive forward scan of the affine recurrence y_t = a_t * y_{t-1} + b_t across lanes (lane order). On return
// (a, b) of lane t compose lanes 0..t: y_t = a * y_{-1} + b.
__device__ __forceinline__ void wave_affine_scan_fwd(float& a, float& b) {
    const int l = lane_id();
#pragma unroll
    for (int off = 1; off < WAVE; off <<= 1) {
        float ap = __shfl_up(a, off, WAVE);
        float bp = __shfl_up(b, off, WAVE);
        if (l >= off) { b = a * bp + b; a = a * ap; }
    }
}

// Inclusive backward scan of y_t = a_t * y_{t+1} + b_t across lanes (reverse lane order). On return (a, b) of lane t
// compose lanes t..63: y_t = a * y_{64} + b.
__device__ __forceinline__ void wave_affine_scan_bwd(float& a, float& b) {
    const int l = lane_id();
#pragma unroll
    for (int off = 1; off < WAVE; off <<= 1) {
        float an = __shfl_down(a, off, WAVE);
        float bn = __shfl_down(b, off, WAVE);
        if (l + off < WAVE) { b = a * bn + b; a = a * an; }
    }
}

// Inclusive prefix sum across lanes.
__device__ __forceinline__ float wave_prefix_sum(float x) {
    const int l = lane_id();
#pragma unroll
    for (int off = 1; off < WAVE; off <<= 1) {
        float y = __shfl_up(x, off, WAVE);
        if (l >= off) x += y;
    }
    return x;
}

// Workgroups are dispatched to the 8 XCDs round-robin (block b runs on XCD b % 8), each XCD with its own L2. This
// maps the hardware block id to a logical work id such that every XCD processes one contiguous slice of the logical
// order, so work items that share data (the segments of one p share its v rows) run on the same XCD and L2.
constexpr int NUM_XCD = 8;
__device__ __forceinline__ int xcd_slice_block(int b, int nb) {
    const int x = b % NUM_XCD, i = b / NUM_XCD;
    const int per = nb / NUM_XCD, rem = nb % NUM_XCD;
    return x * per + min(x, rem) + i;
}

// Raw buffer access with a uniform base (descriptor) + SGPR offset + per-lane VGPR offset: the per-row part of an
// address stays in SGPRs, so a row gather/store costs no per-lane address arithmetic and rewrites no address VGPRs.
// `bytes` bounds the descriptor (out-of-range lanes read 0 / drop their store); every caller's region is < 4 GB.
using rsrc_t = __amdgpu_buffer_rsrc_t;
constexpr int RSRC_WORD3 = 0x00020000;     // raw 32-bit dword access, gfx9-family descriptor format

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, RSRC_WORD3);
}
__device__ __forceinline__ float buf_load(rsrc_t r, int voff, int soff) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ void buf_store(float x, rsrc_t r, int voff, int soff) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), r, voff, soff, 0);
}
// Store that is not re-read by this kernel (streaming output): non-temporal cache policy.
__device__ __forceinline__ void buf_store_stream(float x, rsrc_t r, int voff, int soff) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), r, voff, soff, 2 /* slc */);
}

// 16-byte accesses (buffer_load/store_dwordx4): voff must be 16-byte aligned relative to a 16-byte aligned base.
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f4_t buf_load4(rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(f4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
// Non-temporal: rows that are not re-read by the kernel storing them, so they do not evict its L2-resident gathers.
__device__ __forceinline__ void buf_store4_stream(f4_t x, rsrc_t r, int voff, int soff) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4_t, x), r, voff, soff, 2 /* slc */);
}

}  // namespace qlka
