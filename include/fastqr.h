/*
 * fastqr.h — C ABI of the MI355X (gfx950) batched fp32 Householder QR.
 *
 * Drop-in native boundary for the reference's submission entrypoint
 * `custom_kernel(data) -> (H, tau)` (official/submission.py:5-6,
 * official/task.py:4-5).  The reference binds its kernels through pybind
 * functions built with torch.utils.cpp_extension.load_inline; this header is
 * the torch-free replacement for those bindings: plain pointers, int64 element
 * strides and a HIP stream.  No function throws; every function returns a
 * status code and records a message for fastqr_last_error().
 *
 * Output convention (LAPACK geqrf, as torch.geqrf): R in the upper triangle of
 * H (diagonal included), Householder vectors v_k below the diagonal with the
 * implicit v_k[k] = 1, and tau[k] such that H_k = I - tau[k] v_k v_k^T and
 * A = H_0 H_1 ... H_{n-1} R.  Reflector sign convention as LAPACK slarfg:
 * beta = -sign(alpha) * ||(alpha, x)||, tau = (beta - alpha) / beta, and
 * tau = 0 (H column left as is) when x == 0.
 */
#ifndef FASTQR_H_
#define FASTQR_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  Positive values are hipError_t codes from a failed launch. */
#define FASTQR_OK 0
#define FASTQR_EINVAL (-1)      /* bad shape, stride, or null pointer        */
#define FASTQR_EWORKSPACE (-2)  /* workspace missing, misaligned or too small */
#define FASTQR_ELAYOUT (-3)     /* H/tau layout not supported by the path     */
#define FASTQR_EOVERLAP (-4)    /* A and H overlap with different layouts     */
#define FASTQR_ETESTHOOK (-99)  /* error forced by fastqr_debug_force_error   */

/*
 * Batched QR of `batch` square n x n fp32 matrices.
 *
 * Replaces the reference's pybind entry points
 *   geqrf32(data, h, tau)                        submissions/candidate.py:111-124
 *   geqrf176(data, h, tau)                       submissions/candidate.py:251-270
 *   geqrf352(data, h, tau)                       submissions/candidate.py:508-527
 *   geqrf{n}_blocked(data, h, tau, n, false)     submissions/candidate.py:1333-1353
 * with one shape-dispatched entry point (full factorisation only: the
 * reference's factor_cols / project_tail arguments selected data-dependent
 * shortcuts, which are not offered).
 *
 * A      device pointer, element (b, i, j) at A[b*a_s0 + i*a_s1 + j*a_s2]
 *        (any strides, read only; as the reference kernels,
 *        submissions/candidate.py:150-158).
 * H      device pointer, element (b, i, j) at H[b*h_s0 + i*h_s1 + j*h_s2].
 *        Columns must be contiguous (h_s1 == 1, h_s2 >= n); the allocator
 *        layout is column-major (h_s0, h_s1, h_s2) = (n*n, 1, n) as
 *        allocate_column_major_H (submissions/candidate.py:3752-3769).
 *        H may be the same buffer as A only with an identical layout.
 * tau    device pointer, element (b, k) at tau[b*tau_s0 + k*tau_s1].
 * workspace / workspace_bytes   device scratch of at least
 *        fastqr_workspace_bytes(batch, n) bytes, 256-byte aligned; may be
 *        NULL when that size is 0.  It holds the per-panel T factors.
 * stream a hipStream_t (0 = the null stream).  All work is enqueued
 *        asynchronously on it; no host synchronisation.
 *
 * Returns FASTQR_OK, a negative FASTQR_E* argument error (nothing launched),
 * or a positive hipError_t if a launch failed.
 */
int fastqr_geqrf_f32(const float* A, int64_t batch, int64_t n,
                     int64_t a_s0, int64_t a_s1, int64_t a_s2,
                     float* H, int64_t h_s0, int64_t h_s1, int64_t h_s2,
                     float* tau, int64_t tau_s0, int64_t tau_s1,
                     void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * Workspace bytes fastqr_geqrf_f32 needs for (batch, n).  Replaces the
 * reference's per-input cached policy/workspace tensors
 * (allocate_h_tau / allocate_blocked_policy_workspace,
 * submissions/candidate.py:3801-3880); only the T-factor scratch remains.
 */
size_t fastqr_workspace_bytes(int64_t batch, int64_t n);

/*
 * fastqr_geqrf_f32 without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops and
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 *
 * Same arguments, results and errors as fastqr_geqrf_f32 minus the workspace:
 * the scratch it needs (fastqr_workspace_bytes(batch, n) bytes, less for
 * n > 2048, where one stream needs one set of partial products instead of
 * two) is a static device array of FASTQR_NOALLOC_SCRATCH_BYTES inside the
 * library, one per GPU, held until the process ends.  Calls needing more
 * return FASTQR_EWORKSPACE without launching anything (split the batch, or
 * use fastqr_geqrf_f32): up to 682 matrices for 176 < n <= 1024, one matrix
 * for 2048 < n <= 2100; none above.  It calls no hipMalloc/hipFree and creates no stream or
 * event: every kernel runs on `stream`, in order (the blocked path's panel
 * look-ahead on a second stream is not used).  All calls on one GPU share the
 * array, so calls that overlap in time on one GPU (different streams or
 * threads) race and must be serialised by the caller.
 */
#define FASTQR_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int fastqr_geqrf_f32_noalloc(const float* A, int64_t batch, int64_t n,
                             int64_t a_s0, int64_t a_s1, int64_t a_s2,
                             float* H, int64_t h_s0, int64_t h_s1, int64_t h_s2,
                             float* tau, int64_t tau_s0, int64_t tau_s1,
                             void* stream);

/*
 * Explicit Q of batched compact-Householder factors: Q = H_0 H_1 ... H_{n-1}
 * with H_k = I - tau[k] v_k v_k^T, v_k below the diagonal of column k of H
 * (implicit unit at row k).  Replaces torch.linalg.householder_product(H, tau),
 * the reference checker's call (official/reference.py:199), for square H and
 * n reflectors.
 *
 * H      device pointer, element (b, i, j) at H[b*h_s0 + i*h_s1 + j*h_s2]
 *        (any strides, read only; only the strictly lower part is read).
 * tau    device pointer, element (b, k) at tau[b*tau_s0 + k*tau_s1].
 * Q      device pointer, element (b, i, j) at Q[b*q_s0 + i*q_s1 + j*q_s2];
 *        columns contiguous (q_s1 == 1, q_s2 >= n).  Q may be H itself with
 *        the identical layout (formed in place, as LAPACK sorgqr); otherwise
 *        the two must not overlap.
 * workspace / workspace_bytes  at least fastqr_orgqr_workspace_bytes(batch, n)
 *        bytes of device scratch, 16-byte aligned (T and T V1^T per 32-column
 *        panel; for n > 2048 also the row-split partial products); may be
 *        NULL when that size is 0 (n <= 32).
 * stream a hipStream_t; asynchronous, no host synchronisation.
 *
 * Returns FASTQR_OK, a negative FASTQR_E* argument error, or a positive
 * hipError_t if a launch failed.
 */
int fastqr_orgqr_f32(const float* H, int64_t batch, int64_t n,
                     int64_t h_s0, int64_t h_s1, int64_t h_s2,
                     const float* tau, int64_t tau_s0, int64_t tau_s1,
                     float* Q, int64_t q_s0, int64_t q_s1, int64_t q_s2,
                     void* workspace, size_t workspace_bytes,
                     void* stream);

/* Workspace bytes fastqr_orgqr_f32 needs for (batch, n).  The reference's
 * householder_product call allocates its own (official/reference.py:199). */
size_t fastqr_orgqr_workspace_bytes(int64_t batch, int64_t n);

/*
 * Q C or Q^T C for batched compact-Householder factors, in place in C
 * (LAPACK sormqr with SIDE = 'L'), without forming Q: Q = H_0 H_1 ... H_{r-1},
 * H_k = I - tau[k] v_k v_k^T.  Replaces torch.ormqr(H, tau, C, left=True,
 * transpose=...), the call the reference makes on geqrf factors
 * (submissions/candidate.py:7231-7237).
 *
 * H      device pointer to (batch, m, r) factors, r <= m: element (b, i, j)
 *        at H[b*h_s0 + i*h_s1 + j*h_s2], columns contiguous (h_s1 == 1,
 *        h_s2 >= m); only the strictly lower part is read.
 * tau    device pointer, element (b, j) at tau[b*tau_s0 + j*tau_s1], j < r.
 * C      device pointer to (batch, m, k): element (b, i, j) at
 *        C[b*c_s0 + i*c_s1 + j*c_s2], columns contiguous (c_s1 == 1,
 *        c_s2 >= m); overwritten by Q C (transpose == 0) or Q^T C (!= 0).
 *        C must not overlap H or tau.
 * workspace / workspace_bytes  at least fastqr_ormqr_workspace_bytes(batch, m,
 *        r, k) bytes of device scratch, 16-byte aligned (T of every 32-column
 *        panel; for m > 2048 also a group T and the row-split partial
 *        products); may be NULL when that size is 0.
 * stream a hipStream_t; asynchronous, no host synchronisation.
 *
 * 1 <= m <= 4096.  Returns FASTQR_OK, a negative FASTQR_E* argument error, or
 * a positive hipError_t if a launch failed.
 */
int fastqr_ormqr_f32(const float* H, int64_t batch, int64_t m, int64_t r,
                     int64_t h_s0, int64_t h_s1, int64_t h_s2,
                     const float* tau, int64_t tau_s0, int64_t tau_s1,
                     float* C, int64_t k, int64_t c_s0, int64_t c_s1, int64_t c_s2,
                     int transpose, void* workspace, size_t workspace_bytes,
                     void* stream);

/* Workspace bytes fastqr_ormqr_f32 needs for (batch, m, r, k). */
size_t fastqr_ormqr_workspace_bytes(int64_t batch, int64_t m, int64_t r, int64_t k);

/* Operand precision of the mixed-precision variant's trailing update. */
#define FASTQR_PREC_FP32 0        /* no rounding (fp32 MFMA)                      */
#define FASTQR_PREC_TF32_INPUT 1  /* operands rounded to 10 mantissa bits          */
#define FASTQR_PREC_FP16_INPUT 2  /* operands in fp16 (fp16 MFMA, fp32 accumulate) */
#define FASTQR_PREC_BF16_INPUT 3  /* operands in bf16 (bf16 MFMA, fp32 accumulate) */
/* Repair steps of the mixed-precision variant (bit flags). */
#define FASTQR_MIXED_R_MAINTENANCE 1  /* r_maintenance_mode="panel-prefix" */
#define FASTQR_MIXED_PANEL_REFRESH 2  /* panel_refresh_mode="prefix"       */

/*
 * Blocked QR with a reduced-precision trailing update and optional fp32
 * repair: an experimental, separately labelled variant, not the fp32 path of
 * fastqr_geqrf_f32.  Replaces the reference's prototype
 * blocked_geqrf_reference(data, panel_width, update_mode="compact-wy",
 * precision_mode, r_maintenance_mode, panel_refresh_mode)
 * (tools/blocked_qr_reference.py:193-262) and its CUDA kernels
 * blocked512_panel_refresh_kernel / blocked512_panel_r_repair_kernel with
 * update_operand_352 (submissions/candidate.py:539-554, 2240-2402).
 *
 * Per panel of `panel_width` columns at column k: with PANEL_REFRESH (k > 0)
 * the panel's rows k.. are recomputed in fp32 from A by the k reflectors
 * before it; the panel is factored in fp32; the trailing columns get
 * X - r(V) r(r(T)^T r(r(V)^T r(X))), r() the rounding of `precision`; with
 * R_MAINTENANCE rows k .. k+w-1 of columns k.. (upper triangle) are
 * recomputed in fp32 from A by the first k+w reflectors.  Without repair a
 * reduced precision fails the reference checker's factor gate; with both
 * repairs the result meets the fp32 gates.
 *
 * Arguments as fastqr_geqrf_f32, plus panel_width (16 or 32), precision
 * (FASTQR_PREC_*) and flags (FASTQR_MIXED_*).  A is read again by the repair
 * steps, so A and H must not overlap.  1 <= n <= 2048, batch <= 65535.
 * workspace: fastqr_geqrf_mixed_workspace_bytes(batch, n, panel_width, flags)
 * bytes, 256-byte aligned.
 */
int fastqr_geqrf_mixed_f32(const float* A, int64_t batch, int64_t n,
                           int64_t a_s0, int64_t a_s1, int64_t a_s2,
                           float* H, int64_t h_s0, int64_t h_s1, int64_t h_s2,
                           float* tau, int64_t tau_s0, int64_t tau_s1,
                           int64_t panel_width, int precision, int flags,
                           void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes fastqr_geqrf_mixed_f32 needs (0 for invalid arguments). */
size_t fastqr_geqrf_mixed_workspace_bytes(int64_t batch, int64_t n, int64_t panel_width, int flags);

/*
 * Name of the kernel path fastqr_geqrf_f32 takes for size n ("wave64",
 * "lds", "blocked"); the reference's shape switch is custom_kernel
 * (submissions/candidate.py:8383-8415).  Never NULL.
 */
const char* fastqr_path_name(int64_t n);

/* Message for the last non-zero status on the calling thread (static storage,
 * "" when none).  Replaces TORCH_CHECK / C10_CUDA_KERNEL_LAUNCH_CHECK text
 * (submissions/candidate.py:112-122, 246). */
const char* fastqr_last_error(void);

/* ABI version of this header; bumped on any signature change. */
int fastqr_version(void);

/*
 * Test hook: when `code` is non-zero the next fastqr_geqrf_f32,
 * fastqr_orgqr_f32 or fastqr_ormqr_f32 call on this thread returns `code` without launching
 * anything (used to test the host's error path without faulting a GPU).  No
 * counterpart in the reference.
 */
void fastqr_debug_force_error(int code);

/*
 * Profiling hooks (no counterpart in the reference; the reference times only
 * whole calls with CUDA events, official/eval.py:200-206).  While enabled,
 * every kernel launch that fastqr_geqrf_f32 makes on the calling thread is
 * bracketed by hipEvents recorded on the launch stream, and its algorithmic
 * work (flops, HBM bytes) is accumulated per kernel kind.  Recording events
 * adds a little host work per launch; leave it disabled for headline timing.
 *
 * fastqr_profile_enable(on)   1 starts a fresh collection, 0 stops recording.
 * fastqr_profile_collect(kind, ...)  waits for the recorded events and returns
 *   launch count, summed kernel milliseconds, and summed algorithmic flops and
 *   bytes for kind `kind` (0 .. FASTQR_PROFILE_KINDS-1); returns 0 or a status.
 * fastqr_profile_kind_name(kind)  "copy", "panel", "update" (the strip-resident
 *   trailing update, one kernel per launch), "wave64", "lds", "update_rowsplit"
 *   (the row-split trailing update of tall matrices: one record per call of
 *   its partial-product / T / W / apply kernel sequence).
 */
#define FASTQR_PROFILE_KINDS 6
int fastqr_profile_enable(int on);
int fastqr_profile_collect(int kind, int64_t* launches, double* milliseconds, double* flops, double* bytes);
const char* fastqr_profile_kind_name(int kind);

#ifdef __cplusplus
}
#endif

#endif /* FASTQR_H_ */
