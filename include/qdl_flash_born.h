/*
 * qdl_flash_born.h -- C ABI of the MI355X (gfx950) flash-Born attention library
 * (libqdl_flash_born.so).
 *
 * Born attention, per (b, h):
 *   a_ij = max(0, scale_h * q_i . k_j) * M_ij,  p_ij = a_ij^2,
 *   Z_i  = sum_j p_ij + eps,                    O_i  = sum_j p_ij v_j / Z_i,
 *   M_ij = [causal => j <= i] & [window > 0 => i - j < window] & [doc_i == doc_j].
 *
 * Conventions shared by every entry point:
 *   - q, k, v, out, dout, dq, dk, dv: contiguous (B, H, T, D) arrays of the
 *     element type `dtype`, base addresses 16-byte aligned.
 *   - z, delta: contiguous (B, H, T) fp32.
 *   - scale: `n_scale` fp32 values in device memory, n_scale == 1 (shared) or
 *     n_scale == H (per head, indexed by h).
 *   - doc_ids: contiguous (B, T) int32 in device memory, or NULL.
 *   - D must be a multiple of 8 in [8, 256].  (The Python host zero-pads other
 *     head dims up to the next multiple of 8; padding is exact.)
 *   - Every call is asynchronous on `stream` (a hipStream_t; NULL is the null
 *     stream), allocates nothing and keeps no state between calls.  The caller
 *     owns all buffers, including the workspace.
 *   - Return value: 0 on success; a negative QDL_BORN_E_* code for invalid
 *     arguments (nothing was launched); a positive hipError_t value when a
 *     launch failed.  qdl_flash_born_strerror() describes any code.
 */
#ifndef QDL_FLASH_BORN_H
#define QDL_FLASH_BORN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (the compute dtype of the reference's autograd Function). */
#define QDL_BORN_DTYPE_F32 0
#define QDL_BORN_DTYPE_F16 1
#define QDL_BORN_DTYPE_BF16 2

/* Error codes (negative: rejected before any launch). */
#define QDL_BORN_OK 0
#define QDL_BORN_E_DTYPE (-1)
#define QDL_BORN_E_SHAPE (-2)
#define QDL_BORN_E_HEADDIM (-3)
#define QDL_BORN_E_ALIGN (-4)
#define QDL_BORN_E_NULL (-5)
#define QDL_BORN_E_SCALE (-6)
#define QDL_BORN_E_WINDOW (-7)
#define QDL_BORN_E_WORKSPACE (-8)
#define QDL_BORN_E_TAU (-9)
#define QDL_BORN_E_TABLE (-10)
#define QDL_BORN_E_ROPEDIM (-11)
#define QDL_BORN_E_SCRATCH (-12)

/* Size of the fixed device array qdl_flash_born_bwd_noalloc takes its
 * workspace from (one per GPU): 16 MiB, enough for B * H * T up to about
 * 1.39 million rows (C5's B16 H16 T2048 needs 6.3 MB). */
#define QDL_BORN_BWD_SCRATCH_BYTES (16 * 1024 * 1024)

typedef struct ihipStream_t *qdl_stream_t; /* == hipStream_t */

/* Library version string, e.g. "qdl_flash_born 0.1.0 gfx950". */
const char *qdl_flash_born_version(void);

/* Human-readable text for a return code of any entry point. */
const char *qdl_flash_born_strerror(int code);

/* 1 if (dtype, head_dim) is served by the kernels without host padding. */
int qdl_flash_born_supported(int dtype, int64_t head_dim);

/*
 * Forward pass.  Writes out (B, H, T, D) and z (B, H, T) = sum_j p_ij + eps.
 *
 * Replaces the launch of `_flash_born_fwd_kernel[grid](...)` in
 * `_FlashBornAttentionFn.forward` (Vengo/QuantumDLBlocks
 * src/qdlblocks/kernels/flash_born.py:475-513); arguments carry the same
 * meaning as that launch's (pointers, B/H/T/D, PER_HEAD_SCALE via n_scale,
 * IS_CAUSAL, WINDOW_SIZE, HAS_DOC_IDS via doc_ids != NULL, EPS).
 */
int qdl_flash_born_fwd(int dtype, int64_t B, int64_t H, int64_t T, int64_t D,
                       const void *q, const void *k, const void *v, void *out,
                       float *z, const float *scale, int64_t n_scale,
                       const int32_t *doc_ids, int is_causal,
                       int64_t window_size, double eps, qdl_stream_t stream);

/* Bytes of device workspace qdl_flash_born_bwd needs for this problem. */
int64_t qdl_flash_born_bwd_workspace_size(int dtype, int64_t B, int64_t H,
                                          int64_t T, int64_t D,
                                          int64_t n_scale);

/*
 * Backward pass.  Given the forward's out and z and the upstream gradient
 * dout, writes dq, dk, dv (B, H, T, D) and dscale (n_scale fp32 values:
 * per-head sums, or the total when n_scale == 1).  The dscale reduction is
 * deterministic (fixed-order, no atomics).
 *
 * Replaces the two launches `_flash_born_bwd_kernel[grid_n](...)` and
 * `_flash_born_bwd_dq_kernel[grid_m](...)` in `_FlashBornAttentionFn.backward`
 * (flash_born.py:554-612) together with the zero-initialised dscale buffer
 * they accumulate into (flash_born.py:536).
 */
int qdl_flash_born_bwd(int dtype, int64_t B, int64_t H, int64_t T, int64_t D,
                       const void *q, const void *k, const void *v,
                       const void *out, const void *dout, const float *z,
                       const float *scale, int64_t n_scale,
                       const int32_t *doc_ids, int is_causal,
                       int64_t window_size, double eps, void *dq, void *dk,
                       void *dv, float *dscale, void *workspace,
                       int64_t workspace_bytes, qdl_stream_t stream);

/*
 * Backward pass that allocates nothing: qdl_flash_born_bwd with the
 * workspace taken from a fixed device array of QDL_BORN_BWD_SCRATCH_BYTES
 * inside the library instead of from the caller.
 *
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  It calls no hipMalloc, hipFree or allocating
 * library routine; the caller still passes every input and output.  Each GPU
 * holds its own array until the process ends; its device address is looked
 * up on the first call on that GPU, so call with the device of `stream`
 * current.  Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (other streams or threads) race.  A problem whose workspace
 * (qdl_flash_born_bwd_workspace_size) exceeds QDL_BORN_BWD_SCRATCH_BYTES is
 * rejected with QDL_BORN_E_SCRATCH before any HIP call; otherwise arguments,
 * results and return codes are those of qdl_flash_born_bwd.
 */
int qdl_flash_born_bwd_noalloc(int dtype, int64_t B, int64_t H, int64_t T,
                               int64_t D, const void *q, const void *k,
                               const void *v, const void *out,
                               const void *dout, const float *z,
                               const float *scale, int64_t n_scale,
                               const int32_t *doc_ids, int is_causal,
                               int64_t window_size, double eps, void *dq,
                               void *dk, void *dv, float *dscale,
                               qdl_stream_t stream);

/*
 * Purified-Born attention (flash_born.py:693-1341): weights
 *   p_ij = relu(scale_h (q_i.k_j - tau_h))^4 + eps_base relu(q_i.k_j)^2
 * under the same masks, Z_i = sum_j p_ij + eps, O_i = sum_j p_ij v_j / Z_i.
 * `tau` holds n_tau fp32 values in device memory (1 or H, like scale).  The
 * output is fp32 whatever the input dtype, as the reference's kernel writes
 * an fp32 output (flash_born.py:1102) that its autograd function then casts.
 */

/* Forward: writes out (B, H, T, D) fp32 and z (B, H, T) fp32.
 * Replaces the launch of `_flash_purified_born_fwd_kernel[grid](...)` in
 * `_FlashPurifiedBornAttentionFn.forward` (flash_born.py:1110-1151). */
int qdl_flash_purified_born_fwd(int dtype, int64_t B, int64_t H, int64_t T,
                                int64_t D, const void *q, const void *k,
                                const void *v, float *out, float *z,
                                const float *scale, int64_t n_scale,
                                const float *tau, int64_t n_tau,
                                double eps_base, const int32_t *doc_ids,
                                int is_causal, int64_t window_size,
                                double eps, qdl_stream_t stream);

/* Bytes of device workspace qdl_flash_purified_born_bwd needs. */
int64_t qdl_flash_purified_born_bwd_workspace_size(int dtype, int64_t B,
                                                   int64_t H, int64_t T,
                                                   int64_t D);

/* Backward: given the forward's fp32 out and z and the upstream gradient dout
 * (input dtype), writes dq, dk, dv (input dtype), dscale (n_scale fp32) and
 * dtau (n_tau fp32), both reduced in a fixed order (deterministic).
 * Replaces the two launches `_flash_purified_born_bwd_kernel[grid_n](...)`
 * and `_flash_purified_born_bwd_dq_kernel[grid_m](...)` in
 * `_FlashPurifiedBornAttentionFn.backward` (flash_born.py:1197-1262) with
 * the zero-initialised dscale / dtau buffers they accumulate into
 * (flash_born.py:1178-1179). */
int qdl_flash_purified_born_bwd(int dtype, int64_t B, int64_t H, int64_t T,
                                int64_t D, const void *q, const void *k,
                                const void *v, const float *out,
                                const void *dout, const float *z,
                                const float *scale, int64_t n_scale,
                                const float *tau, int64_t n_tau,
                                double eps_base, const int32_t *doc_ids,
                                int is_causal, int64_t window_size, void *dq,
                                void *dk, void *dv, float *dscale, float *dtau,
                                void *workspace, int64_t workspace_bytes,
                                qdl_stream_t stream);

/*
 * Q/K prologue of SubspaceProjectorBornAttention.forward (attention.py:573-589,
 * without the optional wave filter and partial key offset), fused into one
 * pass per tensor:
 *   x' = l2_normalize(apply_unitary_rope(x, c, s), eps)       for x in {q, k}
 * with apply_unitary_rope (functional.py:104-121) rotating column pairs
 * (i, i + D/2):  y_i = x_i c_ti - x_{i+D/2} s_ti,  y_{i+D/2} = x_i s_ti + x_{i+D/2} c_ti,
 * and l2_normalize (functional.py:36-80): x' = y / sqrt(sum y^2 + eps), the
 * sum in fp32.  For 16-bit dtypes every product, sum and c, s themselves are
 * rounded to the dtype as the reference's tensor ops round them; the norm is
 * formed in fp32 from the rounded y.
 *
 * Row tensors (q, k, dq, dk) are (B, H, T, D) with element strides
 * strides[0..2] for b, h, t and unit stride along D, so the (B, T, H, D)
 * output of a Q/K projection is passed without a transposing copy.  q_out,
 * k_out, dq_out, dk_out are contiguous (B, H, T, D); q_rinv, k_rinv are
 * contiguous (B, H, T) fp32 holding 1 / sqrt(sum y^2 + eps) per row.
 * cos_table, sin_table: fp32, row t (t = 0 .. T-1) at t * table_ld; column
 * i < n_freq holds the angle table for pair i; pairs i >= n_freq are rotated
 * by angle 0 (cos 1, sin 0), the reference's padding of short tables
 * (attention.py:574-582).  cos_table == NULL skips the rotation.
 * Either tensor may be left out by passing NULL for all of its pointers;
 * q_rinv, k_rinv may be NULL on their own (1/norm is then not written: no
 * backward follows).  D must be even, 2 <= D <= 256.
 */

/* Forward.  Replaces the apply_unitary_rope and l2_normalize calls on Q and K
 * at attention.py:583-589 (and the .contiguous() copies at attention.py:516-517
 * when the projection output is passed strided). */
int qdl_flash_born_qk_prologue_fwd(int dtype, int64_t B, int64_t H, int64_t T,
                                   int64_t D, const void *q,
                                   const int64_t *q_strides, const void *k,
                                   const int64_t *k_strides,
                                   const float *cos_table,
                                   const float *sin_table, int64_t n_freq,
                                   int64_t table_ld, double eps, void *q_out,
                                   void *k_out, float *q_rinv, float *k_rinv,
                                   qdl_stream_t stream);

/* Backward: given the gradients dq_out, dk_out of q_out, k_out, the forward's
 * outputs and q_rinv, k_rinv, writes dq, dk (strided like the forward's
 * inputs):  g = (dx' - (dx'.x') x') rinv  (functional.py:50-57, rounded to
 * the dtype), then the transposed rotation  dx_i = g_i c + g_{i+D/2} s,
 * dx_{i+D/2} = g_{i+D/2} c - g_i s, each product and sum rounded to the dtype
 * as autograd's bf16 / fp16 ops round them.  Replaces the autograd backward of
 * the calls at attention.py:583-589. */
int qdl_flash_born_qk_prologue_bwd(int dtype, int64_t B, int64_t H, int64_t T,
                                   int64_t D, const void *dq_out,
                                   const void *dk_out, const void *q_out,
                                   const void *k_out, const float *q_rinv,
                                   const float *k_rinv,
                                   const float *cos_table,
                                   const float *sin_table, int64_t n_freq,
                                   int64_t table_ld, void *dq,
                                   const int64_t *dq_strides, void *dk,
                                   const int64_t *dk_strides,
                                   qdl_stream_t stream);

/*
 * Forward with the Q/K prologue folded into the attention kernel's loads:
 *   q' = l2_normalize(apply_unitary_rope(q, c, s)), k' likewise (exactly as
 *   qdl_flash_born_qk_prologue_fwd computes them), then Born attention of
 *   (q', k', v) as qdl_flash_born_fwd computes it.
 * q, k: raw rows with (b, h, t) element strides (q_strides, k_strides: host
 * arrays of 3, unit stride along D), e.g. the (B, T, H, D) projection output;
 * v, out: contiguous (B, H, T, D); the tables and norm_eps as for the
 * prologue; scale, doc_ids, is_causal, window_size, eps as for the forward.
 * Also writes q_out, k_out (contiguous (B, H, T, D), the normalised rows) and
 * q_rinv, k_rinv (1/norm per row), which the backward needs.  For bf16 with
 * D == 64 and no window (with document ids: no window or a causal one), the
 * keys are normalised by the prologue kernel (keys only) and the attention
 * kernel normalises each query block in registers as it loads it, so the
 * normalised queries are never read back from memory; other cases run the
 * prologue kernel on both and then the attention kernels.  The results are those of the two separate calls, bit
 * for bit.  q_rinv and k_rinv may be NULL when no backward follows: then
 * neither 1/norm is written, and q_out is scratch (the one-kernel path does
 * not write it).
 * Replaces the apply_unitary_rope + l2_normalize calls on Q and K
 * (attention.py:583-589) together with the flash_born_attention call that
 * consumes them (attention.py:704-713, flash_born.py:475-513).
 */
int qdl_flash_born_fwd_qk_prologue(int dtype, int64_t B, int64_t H, int64_t T,
                                   int64_t D, const void *q,
                                   const int64_t *q_strides, const void *k,
                                   const int64_t *k_strides, const void *v,
                                   const float *cos_table,
                                   const float *sin_table, int64_t n_freq,
                                   int64_t table_ld, double norm_eps,
                                   const float *scale, int64_t n_scale,
                                   const int32_t *doc_ids, int is_causal,
                                   int64_t window_size, double eps, void *out,
                                   float *z, void *q_out, void *k_out,
                                   float *q_rinv, float *k_rinv,
                                   qdl_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QDL_FLASH_BORN_H */
