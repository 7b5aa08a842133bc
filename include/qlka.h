/*
 * libqlka: MI355X (gfx950) weighted abs / Laplace sums, the hot path of quasi-linear kernel attention.
 *
 * A plain C ABI: device pointers, sizes and a hipStream_t passed as void*. Nothing here allocates device memory:
 * the caller passes outputs and a workspace of at least the size the matching *_ws_bytes() returns. All launches are
 * asynchronous on `stream`. Every function returns 0 on success or a QLKA_E* code; qlka_last_error() then holds a
 * message for the calling thread.
 *
 * Layouts (the reference's own, Weighted_Abs_Sum/weighted_abs_sum/ops.py:107-110): q (P, D, M), k (P, D, N),
 * v (P, N, C), row outputs (P, M, C), out_u (P, M), per-feature outputs (P, D, M) / (P, D, N); fp32, contiguous.
 * Limits (Weighted_Abs_Sum/csrc/binding.cpp:69-84): P, D, N, M >= 1; 1 <= C <= 128; N, M <= 131072;
 * P*D*max(N, M) <= INT32_MAX.
 */
#ifndef QLKA_H
#define QLKA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QLKA_OK         0
#define QLKA_EINVAL     1   /* argument validation failed (message says which) */
#define QLKA_EWORKSPACE 2   /* workspace null or smaller than *_ws_bytes() */
#define QLKA_EHIP       3   /* a HIP launch failed */

/* Message of the last error on this thread ("" if none). */
const char* qlka_last_error(void);
/* ABI version of this library. */
int qlka_version(void);
/*
 * Base cutoff B of the dense evaluation (the qlka_direct_* kernels: same results to fp32 rounding, same tie
 * conventions) in qlka_laplace_fwd, qlka_abs_fwd (path -1), qlka_abs_bwd and qlka_sgn_fwd, with L = max(N, M): the
 * abs forward goes dense for L <= 2B, the Laplace forward for L <= B, the backward and the sgn sum for L <= B or for
 * L <= 5B/4 when P * ceil(L / 32) >= 512. Whatever B (0 included) and the pinned path, the abs forward also goes
 * dense for N <= 16 keys, and the backward and the sgn sum for min(N, M) <= 16 (the walk's segment totals lose
 * accuracy with a handful of keys). Default 512; 0 sorts and walks everything else. Process-wide; returns the previous
 * value (or -QLKA_EINVAL for n < 0). The C-level counterpart of the reference's set_keops_cutoff
 * (Weighted_Abs_Sum/weighted_abs_sum/ops.py:21-25), which picks the KeOps backend in Python.
 */
int qlka_set_direct_max(int n);
/*
 * Workspace budget in bytes (default 5 GiB). Every operator below runs its whole pipeline on chunks of consecutive
 * p = (batch, head) indices (every stage works on each p alone), taking the largest chunk the workspace it is given
 * holds (at least one p), so the caller bounds device memory by the workspace it passes. The *_ws_bytes() queries
 * report the workspace of the largest chunk within this budget (one p when even one p exceeds it); results do not
 * depend on the chunking. They report 0 for a call that takes the dense route at the current cutoff (qlka_laplace_fwd,
 * qlka_abs_fwd, qlka_abs_bwd, qlka_abs_bwd_sorted, qlka_sgn_fwd): such a call takes no workspace, and ws may be null
 * (a dense abs forward that keeps its sorts for a walking backward needs sort scratch only for segments longer than
 * 16384). Process-wide; returns the previous value. The reference has no counterpart: its
 * workspace is O(P*D*(N+M)) (Weighted_Abs_Sum/csrc/binding.cpp:101-111), where this build's per-feature slab of
 * contribution rows is O(P*D*M*C).
 */
size_t qlka_set_workspace_budget(size_t bytes);

/*
 * weighted_laplace_sum forward.
 *   out_w[p,m,c] = sum_{d,n} exp(-|k[p,d,n] - q[p,d,m]|) v[p,n,c],  out_u[p,m] = sum_{d,n} exp(-|k[p,d,n] - q[p,d,m]|)
 * max(N, M) <= B (the dense cutoff, default 512; see qlka_set_direct_max) runs the dense evaluation of
 * qlka_direct_fwd (no workspace: qlka_laplace_fwd_ws_bytes reports 0).
 * Replaces _ext.weighted_laplace_sum_forward (Weighted_Laplace_Sum/csrc/binding.cpp:63-100).
 */
size_t qlka_laplace_fwd_ws_bytes(int P, int D, int N, int M, int C);
int qlka_laplace_fwd(const float* q, const float* k, const float* v, float* out_w, float* out_u,
                     int P, int D, int N, int M, int C, void* ws, size_t ws_bytes, void* stream);
/*
 * qlka_laplace_fwd without a workspace argument and without any device allocation. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Its workspace is a static 512 MiB device array of the library, held on every device the
 * library runs on until the process ends; the call runs qlka_laplace_fwd over it one chunk of p at a time and gives
 * the same results. Shapes whose single-p workspace (qlka_laplace_fwd_ws_bytes(1, D, N, M, C)) exceeds 512 MiB are
 * refused with QLKA_EINVAL (N = M = 16384, D = C = 64 needs 297 MiB). `stream` must belong to the current device.
 * All calls on one device share the array: calls that overlap in time on one device (e.g. on two streams) race and
 * must be serialised by the caller. The array takes device memory from the first call on a device on (hipMemGetInfo
 * on MI355X: free memory unchanged by loading the library, 6 MiB less after a first qlka_laplace_fwd call, whose
 * kernels' code loads on first use, and 512 MiB less after this entry's first call; unchanged by its later calls); a
 * process that never calls it does not hold it. A thread's first uncaptured call on a
 * device may create that thread's side stream and its events (hipStreamCreateWithFlags, hipEventCreateWithFlags:
 * no device memory); under stream capture, or once they exist, the call creates nothing.
 */
int qlka_laplace_fwd_noalloc(const float* q, const float* k, const float* v, float* out_w, float* out_u,
                             int P, int D, int N, int M, int C, void* stream);

/*
 * weighted_abs_sum forward; out_u == NULL gives the plain op, out_u != NULL the _full op.
 *   out_w[p,m,c] = sum_{d,n} |k[p,d,n] - q[p,d,m]| v[p,n,c],  out_u[p,m] = sum_{d,n} |k[p,d,n] - q[p,d,m]|
 * path: -1 auto, 0 global, 1 fused (the fused path exists for max(N, M) <= 4096 only, as in the reference). Under
 * auto, short segments run the dense evaluation of qlka_direct_fwd (see qlka_set_direct_max).
 * Replaces _ext.weighted_abs_sum_forward / weighted_abs_sum_full_forward (Weighted_Abs_Sum/csrc/binding.cpp:229-239).
 */
size_t qlka_abs_fwd_ws_bytes(int P, int D, int N, int M, int C);
int qlka_abs_fwd(const float* q, const float* k, const float* v, float* out_w, float* out_u,
                 int P, int D, int N, int M, int C, int path, void* ws, size_t ws_bytes, void* stream);

/*
 * weighted_abs_sum backward; g_u == NULL gives the plain backward, g_u != NULL the _full backward.
 *   grad_q[p,d,m] = sum_n s(q_m - k_n) (<v_n, g_w[m]> + g_u[m]),
 *   grad_k[p,d,n] = sum_m s(k_n - q_m) (<g_w[m], v_n> + g_u[m]),
 *   grad_v[p,n,c] = sum_{d,m} |k_n - q_m| g_w[p,m,c];  s(x) = +1 for x > 0, -1 otherwise (a tie counts -1).
 * Replaces _ext.weighted_abs_sum_backward / weighted_abs_sum_full_backward (Weighted_Abs_Sum/csrc/binding.cpp:242-380).
 */
size_t qlka_abs_bwd_ws_bytes(int P, int D, int N, int M, int C);
int qlka_abs_bwd(const float* q, const float* k, const float* v, const float* g_w, const float* g_u,
                 float* grad_q, float* grad_k, float* grad_v,
                 int P, int D, int N, int M, int C, void* ws, size_t ws_bytes, void* stream);

/*
 * Forward and backward that share their sorts. The reference's backward sorts k and q again
 * (Weighted_Abs_Sum/csrc/binding.cpp:242-380 after :229-239); here a forward can leave the sorted k and q and their
 * permutations in caller buffers (k_sorted, k_perm: P*D*N each; q_sorted, q_perm: P*D*M each) for the backward of
 * the same inputs. qlka_abs_bwd_walks tells whether qlka_abs_bwd would sort and walk at this shape (1) or run the
 * dense kernels (0), i.e. whether keeping the sorts pays; qlka_abs_fwd_keep computes what qlka_abs_fwd computes and
 * sets *kept = 1 when it filled the four buffers (0: left untouched, the backward would not use them); after
 * *kept != 0, qlka_abs_bwd_sorted with the same q, k, v computes what qlka_abs_bwd computes without sorting. Same
 * workspace sizes as qlka_abs_fwd / qlka_abs_bwd.
 * states (optional, may be NULL; qlka_abs_keep_state_bytes() bytes, 0 when the backward would read none: it takes the
 * dense kernels, or, at C <= 64 with C % 4 == 0, walks once over the merged sorted keys and queries): the forward
 * also leaves there the range states and query bounds of its walk over the sorted keys, which the backward's grad_q
 * walk would compute again (the same range sums, scan and bounds); it sets *kept = 3 when it wrote them (its own walk
 * ran; a forward on the dense kernels keeps only the sorts). Passing them to qlka_abs_bwd_sorted after *kept = 3
 * skips one range-sum pass, one scan and one bound search per chunk of the backward, with bit-identical gradients.
 */
int qlka_abs_bwd_walks(int P, int N, int M);
size_t qlka_abs_keep_state_bytes(int P, int D, int N, int M, int C);
int qlka_abs_fwd_keep(const float* q, const float* k, const float* v, float* out_w, float* out_u,
                      int P, int D, int N, int M, int C, int path, float* k_sorted, uint32_t* k_perm,
                      float* q_sorted, uint32_t* q_perm, void* states, int* kept, void* ws, size_t ws_bytes,
                      void* stream);
int qlka_abs_bwd_sorted(const float* q, const float* k, const float* v, const float* g_w, const float* g_u,
                        float* grad_q, float* grad_k, float* grad_v, int P, int D, int N, int M, int C,
                        const float* k_sorted, const uint32_t* k_perm, const float* q_sorted, const uint32_t* q_perm,
                        const void* states, void* ws, size_t ws_bytes, void* stream);

/*
 * Dense forward and backward that share the kernel matrix A[p,m,n] = sum_d |k[p,d,n] - q[p,d,m]|. No counterpart in
 * the reference, whose dense (KeOps) route forms A again in the backward (Weighted_Abs_Sum/weighted_abs_sum/
 * keops_backend.py:19-48). qlka_abs_dense_keep_bytes is the size of A (P*M rows of (N + 3) & ~3 floats) where the
 * forward and the backward both run the dense kernels and A stays within 256 MB, else 0; then qlka_abs_fwd_dense_keep
 * computes what qlka_abs_fwd computes and also writes A, and qlka_abs_bwd_dense_kept, given that A and the same q, k, v,
 * computes what qlka_abs_bwd computes, with grad_v as the contraction of A with g_w instead of forming A again
 * (bit-identical gradients). Both take no workspace; both return QLKA_EINVAL where the size is 0.
 */
size_t qlka_abs_dense_keep_bytes(int P, int D, int N, int M, int C);
int qlka_abs_fwd_dense_keep(const float* q, const float* k, const float* v, float* out_w, float* out_u, float* A,
                            int P, int D, int N, int M, int C, void* stream);
int qlka_abs_bwd_dense_kept(const float* q, const float* k, const float* v, const float* g_w, const float* g_u,
                            float* grad_q, float* grad_k, float* grad_v, const float* A, int P, int D, int N, int M,
                            int C, void* stream);

/*
 * weighted_sgn_sum: out[p,d,m] = sum_n sgn(k[p,d,n] - q[p,d,m]) <v[p,n,:], g[p,m,:]>, with a tie counted +1
 * (it is the negated grad_q walk). Replaces _ext.weighted_sgn_sum_forward (Weighted_Abs_Sum/csrc/binding.cpp:384-439).
 */
size_t qlka_sgn_fwd_ws_bytes(int P, int D, int N, int M, int C);
int qlka_sgn_fwd(const float* q, const float* k, const float* v, const float* g, float* out,
                 int P, int D, int N, int M, int C, void* ws, size_t ws_bytes, void* stream);

/*
 * Dense evaluation for short segments: A[m,n] = sum_d f(q[p,d,m] - k[p,d,n]) with f = |x| (kind 0, the weighted abs
 * sum) or exp(-|x|) (kind 1, the weighted Laplace sum), out_w[p,m,:] = sum_n A[m,n] v[p,n,:], out_u[p,m] = sum_n
 * A[m,n] (out_u may be NULL). Same values as qlka_abs_fwd / qlka_laplace_fwd; no sort and no workspace, O(N M D)
 * work, so it is the faster route only for short segments (the ops pick it by size). The role of the reference's
 * KeOps backend below KEOPS_CUTOFF (Weighted_Abs_Sum/weighted_abs_sum/keops_backend.py:19-35).
 */
#define QLKA_DIRECT_ABS     0
#define QLKA_DIRECT_LAPLACE 1
int qlka_direct_fwd(int kind, const float* q, const float* k, const float* v, float* out_w, float* out_u,
                    int P, int D, int N, int M, int C, void* stream);

/*
 * Dense evaluation of the abs backward and of weighted_sgn_sum with an explicit value `tie` of sign(0): the
 * formulas of qlka_abs_bwd / qlka_sgn_fwd with s(0) = tie (0: the KeOps convention of keops_backend.py:40-41 and of
 * autograd through the KeOps forward; -1 for the gradients / +1 for the sgn sum: the walk's convention). g_u may be
 * NULL. No workspace; O(N M (D + C)) work, for short segments.
 */
int qlka_direct_bwd(float tie, const float* q, const float* k, const float* v, const float* g_w, const float* g_u,
                    float* grad_q, float* grad_k, float* grad_v, int P, int D, int N, int M, int C, void* stream);
int qlka_direct_sgn(float tie, const float* q, const float* k, const float* v, const float* g, float* out,
                    int P, int D, int N, int M, int C, void* stream);

/*
 * Fused additive-kernel attention layer, forward: the op(s) plus the normalising epilogue in one call.
 *   kind QLKA_ADD_LAPLACE: out = w / clamp(u - n_pad sum_d e^{-|q_d|}, 1e-6), (w, u) = weighted_laplace_sum(q, k, v)
 *   kind QLKA_ADD_RIESZ:   out = ((|q|_1 + 1e-3) sum_n v_n + sum_n |k_n|_1 v_n - w)
 *                               / clamp((|q|_1 + 1e-3) M + sum_n |k_n|_1 - u - 1e-3 n_pad, 1e-6),
 *                          (w, u) = weighted_abs_sum_full(q, k, v)
 *   kind QLKA_ADD_BUMP:    out = ((w+ + w-)/2 - w0) / clamp((u+ + u-)/2 - u0 - n_pad sum_d max(0, 1 - |q_d|), 1e-6),
 *                          (w0, u0), (w+, u+), (w-, u-) = weighted_abs_sum_full at q, q + 1, q - 1; the three share one
 *                          sort of k and q and one set of key-range summaries.
 * q (P, D, M) and k (P, D, N) already divided by tau, k and v already multiplied by the key mask; n_pad (P) is the
 * number of masked keys per p (NULL: none); out (P, M, C). No gradient.
 * Replaces _add_laplace / _add_riesz / _add_bump (Experiments/kernel_attention/attention.py:67-92).
 */
#define QLKA_ADD_LAPLACE 0
#define QLKA_ADD_RIESZ   1
#define QLKA_ADD_BUMP    2
size_t qlka_layer_fwd_ws_bytes(int kind, int P, int D, int N, int M, int C);
int qlka_layer_fwd(int kind, const float* q, const float* k, const float* v, const float* n_pad, float* out,
                   int P, int D, int N, int M, int C, void* ws, size_t ws_bytes, void* stream);

/*
 * The same layers with the key mask applied inside the sums: q (P, D, M) and k (P, D, N) divided by tau, k and v NOT
 * multiplied by the mask, keep (P, N) bytes (nonzero = real key, non-null). Masked keys weigh 0 in every sum, so w and
 * u run over the real keys only and the n_pad corrections become exact (add_laplace: out = w / clamp(u, 1e-6), ...);
 * no k * keep or v * keep is materialised. Same values as qlka_layer_fwd on k * keep, v * keep and n_pad = N - #kept,
 * without the cancellation of the n_pad terms. Workspace: qlka_layer_fwd_ws_bytes.
 * Replaces the keep branch of attention() (Experiments/kernel_attention/attention.py:122-124) around _add_laplace /
 * _add_riesz / _add_bump, and the padded-key rule of Weighted_Laplace_Sum/weighted_laplace_sum/__init__.py:12.
 */
int qlka_layer_fwd_masked(int kind, const float* q, const float* k, const float* v, const uint8_t* keep, float* out,
                          int P, int D, int N, int M, int C, void* ws, size_t ws_bytes, void* stream);

/*
 * Test entry: stable ascending sort of num_segs contiguous segments of seg_len fp32 keys; perm[i] is the in-segment
 * index of the i-th smallest key (np.argsort(kind="stable"); -0.0 ties +0.0 and is written as +0.0).
 * Replaces launch_iota + launch_cub_sort (Weighted_Abs_Sum/csrc/sort_utils.cu:85-117).
 */
size_t qlka_seg_sort_ws_bytes(int num_segs, int seg_len);
int qlka_seg_sort(const float* keys, float* sorted, uint32_t* perm, int num_segs, int seg_len,
                  void* ws, size_t ws_bytes, void* stream);

/*
 * Test entry: merge rank of every query, rank[s,m] = #{n : k[s,n] < q[s,m]} (np.searchsorted(side="left")), computed
 * by the same sort + range split + merge walk the operators use. Replaces the walk start / emit rule of
 * Weighted_Abs_Sum/csrc/walk_common.cuh:10-30 and abs_kernels.cu:324.
 */
size_t qlka_merge_rank_ws_bytes(int num_segs, int N, int M);
int qlka_merge_rank(const float* q, const float* k, int32_t* rank, int num_segs, int N, int M,
                    void* ws, size_t ws_bytes, void* stream);

/*
 * Optional per-stage timing (no reference counterpart; measurement aid for bench.py). When enabled, every kernel
 * launch is bracketed by hipEvents on its own stream; qlka_timing_read() synchronises them and reports the
 * accumulated milliseconds and launch count of one stage ("lap_range_walk", "abs_range_walk", "lds_radix_sort", ...).
 * The stage "busy" is the union of all bracketed intervals since the last reset (time in which at least one library
 * kernel ran; launches on the side stream overlap those on the caller's stream).
 */
int qlka_timing_enable(int on);
int qlka_timing_reset(void);
int qlka_timing_read(const char* stage, double* total_ms, long long* count);

#ifdef __cplusplus
}
#endif

#endif /* QLKA_H */
