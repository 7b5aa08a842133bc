// The abs backward as one walk over the merged order of the keys and the queries.
//
// The reference's backward (Weighted_Abs_Sum/csrc/binding.cpp:242-380, abs_kernels.cu / sgn_kernels.cu) and this
// library's two-walk form run two walks: one over the sorted keys with v as rows that emits grad_q at every query,
// and one over the sorted queries with g_w as rows that emits grad_k and grad_v at every key. Each walk gathers its
// stream's rows and, for the dot products, the rows of the other side, so v and g_w are gathered twice per walk pair
// (three times with the range sums). Here each segment's sorted queries and keys are merged into one sequence
// (queries first among equal values), and one walk over it carries both prefix states: every element's own row is
// gathered once and is both its contribution to its side's prefix and the operand of its own dot product.
//
// With s(0) = -1 (a tie counts as the other element above), per segment (p, d):
//   grad_q[m] = <g_m, 2 PW - Wtot> + g_u[m] (2 nk - N)      PW, nk: the v sum and count of the keys below q_m
//   grad_k[n] = <v_n, 2 PG - Gtot> + 2 PU - Utot            PG, PU: the g_w and g_u sums of the queries below k_n
//   grad_v[n] = 2 ((k_n - r) PG' + B) - Btot - (k_n - vmax) Gtot   over the queries up to k_n (ties add 0),
// B = sum over those queries of (r - q) g, relative to the value r of the element before k_n (distances from the
// current element, as the two-walk form's B, keep it translation invariant); Btot relative to the segment's last
// value vmax. In the merged order a query's preceding keys are exactly the keys below it, but a key's preceding
// queries include those equal to it; a key therefore takes PG and PU as they stood where its run of equal values
// began. When that run starts in an earlier range, the range's entry state is reduced by the tie carry E: the g_w (and
// g_u) sum of the queries of the run before the range, E(g) = tail(g) + [range g is one value that continues the run
// into it] E(g - 1), an affine scan with 0/1 links.
//
// Kernels, per chunk: merge_sums (the merged values and tags, tag = index | QTAG for a query, and per 64-element range
// the query side's summary for the abs scan, the key side's and the tie carry's for two linked sums), the scans of
// walks.hip (the abs scan; both linked sums in one launch), mbw_walk, and the slab reduce of grad_v.
#include "qlka_common.h"
#include "qlka_internal.h"

namespace qlka {

constexpr int MB_WPB = 4;                      // waves (ranges) per workgroup of the walk
constexpr int MB_RK = 64;                      // elements per range
constexpr uint32_t QTAG = 0x80000000u;         // tag bit of a query
// a buffer offset past every descriptor of this file (rows of one p, a segment's slab rows: at most 67 MB at the widths
// taken here): loads there read 0, stores are dropped
constexpr int MB_OOB = 0x7fff0000;

// ---------------------------------------------------------------------------------------------------- merge_sums
constexpr int MKQ_T = 256, MKQ_ITEMS = 8, MKQ_TILE = MKQ_T * MKQ_ITEMS;
static_assert(MKQ_TILE % MB_RK == 0, "a merge tile holds whole ranges");

// smallest i in [lo, hi] with A[i] > B[o - i - 1] (true at i = hi): the number of A elements among the first o
// outputs of the merge in which A wins ties; one wave, 64 candidates per round
__device__ int merge_path_f(const float* __restrict__ A, const float* __restrict__ B, const int o, int lo, int hi) {
    const int lane = lane_id();
    while (lo < hi) {
        const int step = (hi - lo + WAVE - 1) / WAVE;
        const int i = lo + lane * step;
        const bool pr = i >= hi || A[i] > B[o - i - 1];
        const uint64_t m = __ballot(pr);
        if (m == 0) { lo = lo + (WAVE - 1) * step + 1; continue; }
        const int f = __builtin_ctzll(m);
        if (f == 0) { hi = lo; break; }
        const int nlo = lo + (f - 1) * step + 1;
        hi = min(hi, lo + f * step);
        lo = nlo;
    }
    return lo;
}

// Four weighted row sums of a 64-element range whose elements take their rows from two buffers (lane = channel on
// return, C <= 64, C % 4 == 0): oa = sum a_t x_t, ob = sum b_t x_t, oc = sum c_t x_t, od = sum d_t x_t, x_t the row
// at address row_t. 16 lanes cover a row with one 16-byte load each, lane group r takes elements r, r + 4, ...; each
// lane stages its element's address and weights in wave-private LDS, so every element's row is loaded once, from
// whichever buffer holds it.
__device__ __forceinline__ void row_sums4(const float* row, const int C, const float a, const float b, const float c,
                                          const float d, f4_t* stage, float& oa, float& ob, float& oc, float& od) {
    const int l = lane_id(), grp = l >> 4, sub = l & 15;
    const int coff = min(4 * sub, C - 4);
    f4_t* const st2 = stage + WAVE;
    const uint64_t ra = (uint64_t)row;
    stage[l] = f4_t{__uint_as_float((uint32_t)ra), __uint_as_float((uint32_t)(ra >> 32)), a, b};
    st2[l] = f4_t{c, d, 0.f, 0.f};
    __builtin_amdgcn_wave_barrier();
    f4_t sa = {0.f, 0.f, 0.f, 0.f}, sb = sa, sc = sa, sd = sa;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int t = 4 * i + grp;
        const f4_t wv = stage[t];
        const f4_t w2 = st2[t];
        const uint64_t rt = (uint64_t)__float_as_uint(wv[0]) | ((uint64_t)__float_as_uint(wv[1]) << 32);
        const f4_t x = *(reinterpret_cast<const __attribute__((address_space(1))) f4_t*>(rt) + (coff >> 2));
        sa += wv[2] * x;
        sb += wv[3] * x;
        sc += w2[0] * x;
        sd += w2[1] * x;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        sa[e] += __shfl_xor(sa[e], 16, WAVE);
        sb[e] += __shfl_xor(sb[e], 16, WAVE);
        sc[e] += __shfl_xor(sc[e], 16, WAVE);
        sd[e] += __shfl_xor(sd[e], 16, WAVE);
        sa[e] += __shfl_xor(sa[e], 32, WAVE);
        sb[e] += __shfl_xor(sb[e], 32, WAVE);
        sc[e] += __shfl_xor(sc[e], 32, WAVE);
        sd[e] += __shfl_xor(sd[e], 32, WAVE);
    }
    const int src = min(l, C - 1) >> 2, e = l & 3;
    float ya[4], yb[4], yc[4], yd[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        ya[k] = __shfl(sa[k], src, WAVE);
        yb[k] = __shfl(sb[k], src, WAVE);
        yc[k] = __shfl(sc[k], src, WAVE);
        yd[k] = __shfl(sd[k], src, WAVE);
    }
    oa = e == 0 ? ya[0] : e == 1 ? ya[1] : e == 2 ? ya[2] : ya[3];
    ob = e == 0 ? yb[0] : e == 1 ? yb[1] : e == 2 ? yb[2] : yb[3];
    oc = e == 0 ? yc[0] : e == 1 ? yc[1] : e == 2 ? yc[2] : yc[3];
    od = e == 0 ? yd[0] : e == 1 ? yd[1] : e == 2 ? yd[2] : yd[3];
    __builtin_amdgcn_wave_barrier();
}

// One workgroup per (segment, tile of MKQ_TILE merged outputs = MKQ_TILE / MB_RK ranges). Waves 0 and 1 find where the
// tile starts and ends on the merge path of the sorted queries (A, length M) and keys (B, length N), the slices go to
// LDS, each thread merges 8 outputs there and the tile leaves through LDS, coalesced. Then each wave takes every
// fourth range of the tile and writes its summary rows (CS = C + 2 floats at (s, g); slot C: a scalar channel, slot
// C + 1: the scan link):
//   sa_q: the queries' g_w sum SG, slot C their g_u sum, link the value gap vlast_g - vlast_{g-1}   (abs scan)
//   sb_q: SB = sum over the queries of (vlast_g - q) g_w, slot C and C + 1 zero                     (abs scan's B)
//   sa_k: the keys' v sum, slot C their count, link 1                                              (linked sum)
//   sa_e: the tie carry's summary: the g_w (slot C: g_u) sum of the queries equal to the range's last value, link 1
//         when the range is one value that continues the run of the element before it, else 0     (linked sum)
// The merged tile makes no second trip through memory before its sums, and every element's row is gathered once.
__global__ __launch_bounds__(MKQ_T)
void merge_sums(const float* __restrict__ qs, const uint32_t* __restrict__ qp, const float* __restrict__ ks,
                const uint32_t* __restrict__ kp, const float* __restrict__ v, const float* __restrict__ gw,
                const float* __restrict__ gu, float* __restrict__ mv, uint32_t* __restrict__ mt,
                float* __restrict__ sa_q, float* __restrict__ sb_q, float* __restrict__ sa_k, float* __restrict__ sa_e,
                const int D, const int N, const int M, const int C, const int G, const int tiles)
{
    __shared__ float sv[MKQ_TILE];
    __shared__ uint32_t stg[MKQ_TILE];
    __shared__ f4_t stage_all[MKQ_T / WAVE][2 * WAVE];
    __shared__ int split[2];
    const int bid = xcd_slice_block(blockIdx.x, gridDim.x);
    const int seg = bid / tiles, blk = bid - seg * tiles;
    const int L = N + M, o0 = blk * MKQ_TILE, o1 = min(o0 + MKQ_TILE, L);
    const float* A = qs + (size_t)seg * M;
    const float* B = ks + (size_t)seg * N;
    const int w = wave_in_block(), tid = threadIdx.x, l = lane_id();
    if (w < 2) {
        const int o = w == 0 ? o0 : o1;
        const int i = merge_path_f(A, B, o, max(0, o - N), min(o, M));
        if (l == 0) split[w] = i;
    }
    __syncthreads();
    const int i0 = split[0], i1 = split[1];
    const int na = i1 - i0, j0 = o0 - i0, n = o1 - o0, nb = n - na;
    const uint32_t* Ap = qp + (size_t)seg * M;
    const uint32_t* Bp = kp + (size_t)seg * N;
    for (int e = tid; e < na; e += MKQ_T) { sv[e] = A[i0 + e]; stg[e] = Ap[i0 + e] | QTAG; }
    for (int e = tid; e < nb; e += MKQ_T) { sv[na + e] = B[j0 + e]; stg[na + e] = Bp[j0 + e]; }
    // the value of the merged element before the tile (o0 > 0): the larger of the last query and the last key before it
    const float vb_tile = (i0 > 0 && j0 > 0) ? fmaxf(A[i0 - 1], B[j0 - 1]) : i0 > 0 ? A[i0 - 1] : j0 > 0 ? B[j0 - 1]
                                                                                                     : 0.f;
    __syncthreads();
    const int d = min(tid * MKQ_ITEMS, n);
    int lo = max(0, d - nb), hi = min(d, na);
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sv[mid] <= sv[na + d - mid - 1]) lo = mid + 1; else hi = mid;
    }
    int i = lo, j = d - lo;
    float rv[MKQ_ITEMS];
    uint32_t rt[MKQ_ITEMS];
#pragma unroll
    for (int t = 0; t < MKQ_ITEMS; ++t) {
        const bool takea = i < na && (j >= nb || sv[i] <= sv[na + j]);
        const int at = takea ? i : na + j;
        rv[t] = sv[at];
        rt[t] = stg[at];
        i += takea;
        j += !takea;
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < MKQ_ITEMS; ++t)
        if (d + t < n) { sv[d + t] = rv[t]; stg[d + t] = rt[t]; }
    __syncthreads();
    const size_t so = (size_t)seg * L + o0;
    for (int e = tid; e < n; e += MKQ_T) { mv[so + e] = sv[e]; mt[so + e] = stg[e]; }

    // the range summaries
    const int p = seg / D, CS = C + 2;
    f4_t* stage = stage_all[w];
    for (int r = w; r * MB_RK < n; r += MKQ_T / WAVE) {
        const int g = blk * (MKQ_TILE / MB_RK) + r;
        const int rb = r * MB_RK, nk = min(MB_RK, n - rb);
        const int li = rb + min(l, nk - 1);
        const float val = sv[li];
        const uint32_t tag = stg[li];
        const bool real = l < nk;
        const bool isq = real && (tag & QTAG), isk = real && !(tag & QTAG);
        const uint32_t idx = tag & ~QTAG;
        const float vfirst = sv[rb], vlast = sv[rb + nk - 1];
        const float vbefore = r > 0 ? sv[rb - 1] : g > 0 ? vb_tile : vfirst;
        const float u = (isq && gu) ? gu[(size_t)p * M + idx] : 0.f;
        const bool inlast = isq && val == vlast;           // a query of the range's last run of equal values
        // the element's own row: g_w for a query, v for a key (lanes past the range repeat its last element, weight 0)
        const float* row = (tag & QTAG) ? gw + ((size_t)p * M + idx) * C : v + ((size_t)p * N + idx) * C;
        float SG, SB, TL, SW;
        row_sums4(row, C, isq ? 1.f : 0.f, isq ? vlast - val : 0.f, inlast ? 1.f : 0.f, isk ? 1.f : 0.f, stage, SG,
                  SB, TL, SW);
        const float su = wave_sum(u), tu = wave_sum(inlast ? u : 0.f);
        const float nkeys = (float)__popcll(__ballot(isk));
        const bool tie_into = g > 0 && vfirst == vbefore;
        const float link_e = (tie_into && vfirst == vlast) ? 1.f : 0.f;
        const float gap = g > 0 ? vlast - vbefore : 0.f;
        const size_t ro = ((size_t)seg * (G + 1) + g) * CS;
        if (l < C) {
            sa_q[ro + l] = SG;
            sb_q[ro + l] = SB;
            sa_k[ro + l] = SW;
            sa_e[ro + l] = TL;
        }
        if (l == 0) {
            sa_q[ro + C] = su;     sa_q[ro + C + 1] = gap;
            sb_q[ro + C] = 0.f;    sb_q[ro + C + 1] = 0.f;
            sa_k[ro + C] = nkeys;  sa_k[ro + C + 1] = 1.f;
            sa_e[ro + C] = tu;     sa_e[ro + C + 1] = link_e;
        }
    }
}

int merge_sums_launch(const float* qs, const uint32_t* qp, const float* ks, const uint32_t* kp, const float* v,
                      const float* gw, const float* gu, float* mv, uint32_t* mt, float* sa_q, float* sb_q,
                      float* sa_k, float* sa_e, int S, int D, int N, int M, int C, int G, hipStream_t st) {
    if (C > WAVE || C % 4 != 0 || G != (N + M + MB_RK - 1) / MB_RK) return (int)hipErrorInvalidValue;
    const int tiles = (N + M + MKQ_TILE - 1) / MKQ_TILE;
    StageTimer t("merge_sums", st);
    hipLaunchKernelGGL(merge_sums, dim3((unsigned)((size_t)S * tiles)), dim3(MKQ_T), 0, st, qs, qp, ks, kp, v, gw, gu,
                       mv, mt, sa_q, sb_q, sa_k, sa_e, D, N, M, C, G, tiles);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------- mbw_walk
// One wave per 64-element range. The elements' rows (g_w for a query, v for a key) are gathered into registers
// (lane = channel), 32 at a time (62 VGPRs, 8 waves per SIMD; all 64 at once took 94-96 and 5), and walked in order: at element t the B state moves its reference to the element's value, a query
// emits its dot with 2 PW - Wtot and adds its row to PG, a key emits its dot with 2 PG' - Gtot (PG' = PG where the key's
// run of equal values began) and its grad_v row (a 4-byte store per lane, non-temporal) and adds its row to PW. The
// dots' lane products go to wave-private LDS, 16 elements at a time, and are summed there (4 lanes per element, 16
// channels each, then two lane shuffles) with the scalar g_u terms, computed per element beforehand.
// The walk has no branches: every element's row address and slab row offset are computed lane-parallel beforehand and
// read lane by lane, the query/key choice is a select, and a query's (or a padding element's) slab store goes to an
// out-of-range offset, which drops it. Padding elements past a short last range have zero rows, the last value, no
// new run and no store, so they leave every state as it was.
__global__ __launch_bounds__(MB_WPB * WAVE)
void mbw_walk(const float* __restrict__ mv, const uint32_t* __restrict__ mt, const float* __restrict__ v,
              const float* __restrict__ gw, const float* __restrict__ gu, const float* __restrict__ ta_q,
              const float* __restrict__ tb_q, const float* __restrict__ ta_k, const float* __restrict__ ta_e,
              float* __restrict__ slab, float* __restrict__ grad_q, float* __restrict__ grad_k, const int S,
              const int D, const int N, const int M, const int C, const int CR, const int G)
{
    __shared__ float dot_all[MB_WPB][16][WAVE];
    const long wv = (long)xcd_slice_block(blockIdx.x, gridDim.x) * MB_WPB + wave_in_block();
    if (wv >= (long)S * G) return;
    float (&dot)[16][WAVE] = dot_all[wave_in_block()];
    const int s = (int)(wv / G), g = (int)(wv - (long)s * G);
    const int p = s / D, d = s - p * D, l = lane_id(), L = N + M;
    const int base = g * MB_RK, nk = min(MB_RK, L - base);
    const float* mseg = mv + (size_t)s * L;
    const uint32_t* tseg = mt + (size_t)s * L;
    const int li = base + min(l, nk - 1);
    const float val = mseg[li];
    const uint32_t tag = tseg[li];
    const bool real = l < nk;
    const bool isq = real && (tag & QTAG), isk = real && !(tag & QTAG);
    const uint32_t idx = tag & ~QTAG;
    const float vbefore = g > 0 ? mseg[base - 1] : mseg[base];
    const bool tie_into = g > 0 && mseg[base] == vbefore;
    const float vmax = mseg[L - 1];
    const float u = (isq && gu) ? gu[(size_t)p * M + idx] : 0.f;
    const uint64_t qmask = __ballot(isq), kmask = __ballot(isk);

    // the element's own row: g_w for a query, v for a key (lanes past the range repeat its last element)
    const float* row_l = (tag & QTAG) ? gw + ((size_t)p * M + idx) * C : v + ((size_t)p * N + idx) * C;
    const uint32_t ra_lo = (uint32_t)(uint64_t)row_l, ra_hi = (uint32_t)((uint64_t)row_l >> 32);
    const int cl = min(l, C - 1);
    // the rows are gathered and walked in two halves of 32 elements, so that a wave holds 32 rows at a time
    constexpr int HALF = MB_RK / 2;
    auto gather = [&](float (&xs)[HALF], const int h) {
#pragma unroll
        for (int i = 0; i < HALF; ++i) {
            const int t = h * HALF + i;
            const uint64_t rt = (uint64_t)bcast(ra_lo, t) | ((uint64_t)bcast(ra_hi, t) << 32);
            xs[i] = reinterpret_cast<const __attribute__((address_space(1))) float*>(rt)[cl];
        }
    };
    float x0[HALF];
    gather(x0, 0);

    // entry states (lane = channel; slot C: the scalar channel) and the segment totals (row G)
    const int CS = C + 2;
    const size_t r0 = ((size_t)s * (G + 1) + g) * CS, rt = ((size_t)s * (G + 1) + G) * CS;
    const bool ch = l < C;
    float PG = ch ? ta_q[r0 + l] : 0.f, B = ch ? tb_q[r0 + l] : 0.f, PW = ch ? ta_k[r0 + l] : 0.f;
    const float E = ch ? ta_e[r0 + l] : 0.f;
    const float PU = ta_q[r0 + C], cnt_in = ta_k[r0 + C], EU = ta_e[r0 + C];
    const float Gt = ch ? ta_q[rt + l] : 0.f, Bt = ch ? tb_q[rt + l] : 0.f, Wt = ch ? ta_k[rt + l] : 0.f;
    const float Ut = ta_q[rt + C];

    // per element (lane t): the start of a run of equal values, the keys below it, the g_u sum of the queries below
    // it, where its run began (-1: before the range), and its scalar term
    float vprev_l = __shfl_up(val, 1, WAVE);
    if (l == 0) vprev_l = vbefore;
    const bool newrun = real && (l == 0 ? !tie_into : val != vprev_l);
    const uint64_t runmask = __ballot(newrun);
    const uint64_t below = (l == 0) ? 0ull : (~0ull >> (WAVE - l));
    const float nkb = cnt_in + (float)__popcll(__ballot(isk) & below);
    const float ui = wave_prefix_sum(isq ? u : 0.f);
    const float pu_ex = PU + ui - (isq ? u : 0.f);
    const uint64_t upto = runmask & (below | (1ull << l));
    const int rs = upto ? 63 - __builtin_clzll(upto) : -1;
    const float pu_run = __shfl(pu_ex, max(rs, 0), WAVE);
    const float pub = rs >= 0 ? pu_run : PU - (tie_into ? EU : 0.f);
    const float sterm = isq ? u * (2.f * nkb - (float)N) : 2.f * pub - Ut;

    const int SGr = slab_group(D);
    // the segment's slab rows (uniform; read through readfirstlane so the descriptor stays in SGPRs)
    const uint64_t sbu = uniform_u64((uint64_t)(slab + slab_seg_base(p, d, D, N, CR)));
    const rsrc_t sr_ = make_rsrc(reinterpret_cast<const void*>(sbu), uniform_u32(slab_seg_bytes(d, D, N, CR)));
    const int soff = isk ? slab_row_off((int)idx, SGr, CR) : 0;     // element t's slab row, read by lane t
    const int vo = ch ? l * 4 : MB_OOB;
    float* gq = grad_q + (size_t)s * M;
    float* gk = grad_k + (size_t)s * N;
    float PGB = PG - (tie_into ? E : 0.f);
    float vprev = vbefore;
    auto walk_half = [&](float (&xs)[HALF], const int h) {
#pragma unroll
        for (int i = 0; i < HALF; ++i) xs[i] = (h * HALF + i < nk && ch) ? xs[i] : 0.f;
#pragma unroll
        for (int i = 0; i < HALF; ++i) {
            const int t = h * HALF + i;
            const float xt = xs[i];
            const float vt = bcast(val, t);
            const bool q = (qmask >> t) & 1;
            PGB = ((runmask >> t) & 1) ? PG : PGB;
            B += (vt - vprev) * PG;
            dot[t & 15][l] = xt * (q ? 2.f * PW - Wt : 2.f * PGB - Gt);
            const float pg1 = PG + xt, pw1 = PW + xt;
            PG = q ? pg1 : PG;
            PW = q ? PW : pw1;
            const float row = 2.f * B - Bt - (vt - vmax) * Gt;
            buf_store_stream(row, sr_, ((kmask >> t) & 1) ? vo : MB_OOB, bcast(soff, t));
            vprev = vt;
            if ((t & 15) == 15) {
                // the 16 elements t - 15 .. t: lane 4 e + k sums channels 16 k .. 16 k + 15 of element e
                const int c0 = t - 15, e = l >> 2, k4 = l & 3;
                const f4_t* rowp = reinterpret_cast<const f4_t*>(&dot[e][16 * k4]);
                const f4_t a0 = rowp[0], a1 = rowp[1], a2 = rowp[2], a3 = rowp[3];
                float sum = (a0[0] + a0[1] + a0[2] + a0[3]) + (a1[0] + a1[1] + a1[2] + a1[3]) +
                            (a2[0] + a2[1] + a2[2] + a2[3]) + (a3[0] + a3[1] + a3[2] + a3[3]);
                sum += __shfl_xor(sum, 1, WAVE);
                sum += __shfl_xor(sum, 2, WAVE);
                const int te = c0 + e;
                const float st_e = __shfl(sterm, te, WAVE);
                const uint32_t tg_e = __shfl(tag, te, WAVE);
                if (k4 == 0 && te < nk) {
                    const uint32_t ie = tg_e & ~QTAG;
                    if (tg_e & QTAG) gq[ie] = sum + st_e;
                    else gk[ie] = sum + st_e;
                }
            }
        }
    };
    walk_half(x0, 0);
    float x1[HALF];
    gather(x1, 1);
    walk_half(x1, 1);
}

int mbw_walk_launch(const float* mv, const uint32_t* mt, const float* v, const float* gw, const float* gu,
                    const float* ta_q, const float* tb_q, const float* ta_k, const float* ta_e, float* slab,
                    float* grad_q, float* grad_k, int S, int D, int N, int M, int C, int G, hipStream_t st) {
    if (C > WAVE) return (int)hipErrorInvalidValue;
    const long waves = (long)S * G;
    StageTimer t("mbw_walk", st);
    hipLaunchKernelGGL(mbw_walk, dim3((unsigned)((waves + MB_WPB - 1) / MB_WPB)), dim3(MB_WPB * WAVE), 0, st, mv, mt,
                       v, gw, gu, ta_q, tb_q, ta_k, ta_e, slab, grad_q, grad_k, S, D, N, M, C, slab_stride(C), G);
    return (int)hipGetLastError();
}

}  // namespace qlka
