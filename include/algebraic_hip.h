/*
 * algebraic_hip.h -- C ABI of the MI355X (gfx950) algebraic attention and fused
 * algebraic LM head kernels (libalgebraic_hip.so).
 *
 * Every entry point is a pure function over caller-owned device buffers: plain pointers,
 * sizes, scalars and a HIP stream. No entry point allocates device memory; scratch comes
 * from a caller workspace sized by the *_workspace_size queries. Calls are asynchronous
 * on `stream` and reentrant (no global mutable state besides the thread-local error text),
 * with one exception: alg_attn_bwd_noalloc keeps its scratch in one library-held device
 * array per GPU, so calls of it that overlap on one GPU (two streams, two host threads)
 * race and must be serialised by the caller.
 * ABI: alg_abi_version() returns ALG_ABI_VERSION of the header the library was built from;
 * a caller compares it with its own before binding (signatures change between versions).
 * Return value: ALG_OK or an error code; alg_last_error() describes the last failure on
 * the calling thread.
 *
 * Tensor layouts are row-major: attention (B, H, T, D) or (B, T, H, D) (the `layout`
 * argument); head h (N, d), E (V, d).
 * Reference interfaces replaced (paths relative to the reference repository root):
 *   src/algebraic/kernels/flash.py       flash_attention 763-857, _forward 292-326,
 *                                        _backward 630-687, _flash_bwd 718-726
 *   src/algebraic/kernels/head_resident.py forward 125-142, backward 145-163
 *   src/algebraic/kernels/fused_head.py  _forward 174-191, _backward 194-216,
 *                                        _telemetry 219-229, fused_head 260-275
 *   src/algebraic/model.py 170-174, src/algebraic/algebraic.py 76-83, 124-179
 *                                        (QK norm, Cayley tables and rotation: the
 *                                        attention prologue)
 */
#ifndef ALGEBRAIC_HIP_H
#define ALGEBRAIC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* alg_stream_t; /* a hipStream_t; NULL = the null stream */

enum {
  ALG_OK = 0,
  ALG_ERR_INVALID = 1,      /* bad shape, pointer, size or parameter */
  ALG_ERR_UNSUPPORTED = 2,  /* valid in the reference but not built for gfx950 here */
  ALG_ERR_HIP = 3           /* a HIP launch error */
};

enum { ALG_DTYPE_BF16 = 0, ALG_DTYPE_F32 = 1 };

/* Storage of the (B, ., ., D) tensors of an attention call (q, k, v, o, dO, dq, dk, dv and the
 * prologue's outputs): (B, H, T, D), the reference's layout, or the projection layout
 * (B, T, H, D) that model.py:167-169 transposes away and model.py:182 transposes back; with it
 * o reads as (B, T, H*D) with no copy. Per-row vectors (stat, di, tau) are (B, H, T). */
enum { ALG_LAYOUT_BHTD = 0, ALG_LAYOUT_BTHD = 1 };

/* Attention variants (flash.py:59-73, 732-760, 850-852).
 *   INRANGE  unshifted, unclipped weights, stat = 1/Z ("low" branch of range_guard)
 *   CLIPPED  unshifted with x = min(s, clamp) (range_guard=False, shift=False)
 *   SHIFTED  running-max accumulation (explicit shift=True, or the guard's fallback)
 *   GUARDED  INRANGE or SHIFTED chosen on the device by guard_flag (range_guard=True) */
enum { ALG_ATTN_INRANGE = 0, ALG_ATTN_CLIPPED = 1, ALG_ATTN_SHIFTED = 2, ALG_ATTN_GUARDED = 3 };

/* Version 2: alg_attn_workspace_size and alg_head_* take a leading dtype argument and
 * alg_attn_bwd has no o_precise argument (version 1 had one). */
#define ALG_ABI_VERSION 2

const char* alg_last_error(void);
const char* alg_version(void);
int alg_abi_version(void);

/* Bytes of workspace alg_attn_prepare / alg_attn_bwd need for this dtype and shape: the sink
 * gradient's and the guard's partials, and for ALG_DTYPE_F32 also an f32 dQ accumulator
 * (B*H*T*D floats). 0 for an invalid dtype or shape. */
size_t alg_attn_workspace_size(int dtype, int B, int H, int T, int D);

/* Prologue and range guard, flash.py:823-849.
 * q_s = round(q * 1/(sqrt(D) c)) in the input dtype; sink_scaled[h] = sink_logit[h or 0] / c
 * (sink_logit may be NULL; sink_count is 1 or H); guard_flag = 1 when
 *   max||q_s||^2 max||k||^2 <= (bound/1.01)^2, max|sink/c| <= bound/1.01 and
 *   max|v| <= min(1e8, 1e37/((T+has_sink)(2 bound+1)^n)), bound = min(16, clamp/2),
 * else 0; with range_guard = 0 the flag is set to 1 and k, v are not read. The pass is
 * elementwise over rows, so q_s has q's layout, whichever of the two it is. */
int alg_attn_prepare(alg_stream_t stream, int dtype, int B, int H, int T, int D,
                     const void* q, const void* k, const void* v,
                     const float* sink_logit, int sink_count, float c, int n, int range_guard,
                     void* q_s, float* sink_scaled, int* guard_flag,
                     void* workspace, size_t workspace_bytes);

/* Forward, flash.py:189-326 / head_resident.py:25-89 (kernel contract of _forward):
 * in q_s, k, v (in `layout`) and sink_scaled (H) f32 or NULL; out o (in `layout`) in the input
 * dtype and stat (B,H,T) f32 (1/Z, or rho(-m) Z^(-1/n) when shifted, or Z^(-1/n) when
 * CLIPPED with inv_stat = 0). o_precise (f32, optional) receives the unrounded output of
 * the SHIFTED branch (precise_output, flash.py:322). guard_flag is read for GUARDED. */
int alg_attn_fwd(alg_stream_t stream, int dtype, int layout, int B, int H, int T, int D,
                 const void* q_s, const void* k, const void* v, const float* sink_scaled,
                 int n, int variant, const int* guard_flag, float clamp, int fast_rho, int inv_stat,
                 void* o, float* o_precise, float* stat);

/* Guarded forward from the unscaled queries, flash.py:823-856 with range_guard=True
 * (kind="asinh", n <= 32, where the guard applies, flash.py:834): the same outputs as
 * alg_attn_prepare(range_guard = 1) followed by alg_attn_fwd(ALG_ATTN_GUARDED) with the
 * guard's own clamp (q_s, sink_scaled, guard_flag, o, stat; o_precise as in alg_attn_fwd), in
 * one call. For bf16 inputs, and f32 inputs at D = 64, there is no separate pass over q, k
 * and v: the in-range forward forms q * alpha itself, writes q_s and leaves the guard maxima of
 * its rows, the guard runs after it, and the shifted branch (flag-checked on the device)
 * replaces o and stat when the guard fails. sink_scaled is written, and required, only with a
 * sink (sink_logit not NULL). f32 inputs at D = 128 take the two calls. */
int alg_attn_fwd_guarded(alg_stream_t stream, int dtype, int layout, int B, int H, int T, int D,
                         const void* q, const void* k, const void* v,
                         const float* sink_logit, int sink_count, float c, int n,
                         void* q_s, float* sink_scaled, int* guard_flag,
                         void* o, float* o_precise, float* stat,
                         void* workspace, size_t workspace_bytes);

/* Backward, flash.py:333-361, 515-687, 694-726 / head_resident.py:91-119:
 * in the forward residuals (q_s, k, v, sink_scaled, o, stat) and dO; out
 * dq = round(round(n * dq_s_acc) * dq_scale) (dq_scale = 1 gives the kernel's dq_s;
 * = 1/(sqrt(D) c) chains back to q), dk, dv in the input dtype and `layout` (as are q_s, k, v,
 * o, dO), di (B,H,T) f32 = sum_d dO*o and dsink_scaled (H) f32 = dL/d(sink/c) (may be NULL).
 * The bf16 SHIFTED branch needs no f32 copy of the output: it forms di = sum_j p_ij dP_ij from
 * its own weights (equal to sum_d dO*o in exact arithmetic). */
int alg_attn_bwd(alg_stream_t stream, int dtype, int layout, int B, int H, int T, int D,
                 const void* q_s, const void* k, const void* v, const float* sink_scaled,
                 const void* o, const float* stat, const void* dO,
                 int n, int variant, const int* guard_flag, float clamp, int fast_rho, int inv_stat,
                 float dq_scale,
                 void* dq, void* dk, void* dv, float* di, float* dsink_scaled,
                 void* workspace, size_t workspace_bytes);

/* Allocation-free variant of alg_attn_bwd. It has no counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving or
 * training loops, harnesses that forbid allocation). Same arguments, results and errors as
 * alg_attn_bwd without the workspace: the scratch (the sink-gradient and guard partials, and
 * for ALG_DTYPE_F32 the f32 dQ accumulator) is a device array the library holds per GPU,
 * ALG_ATTN_NOALLOC_SCRATCH_BYTES bytes on each GPU it runs on, until the process ends. A call
 * whose scratch would exceed it (alg_attn_workspace_size above that limit; f32 inputs with
 * more than about two million B*H*T*D elements) fails with ALG_ERR_UNSUPPORTED. The call
 * allocates no device memory (with the measurement hook of alg_timer_enable off, the
 * default); its first call on a device looks up that device's scratch address. Every call on
 * one GPU shares that GPU's scratch: calls that overlap on one GPU (concurrent streams or
 * threads) race and must be ordered by the caller. Nothing in the scratch needs to start at
 * zero: every launch writes what it later reads. */
#define ALG_ATTN_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)
int alg_attn_bwd_noalloc(alg_stream_t stream, int dtype, int layout, int B, int H, int T, int D,
                         const void* q_s, const void* k, const void* v, const float* sink_scaled,
                         const void* o, const float* stat, const void* dO,
                         int n, int variant, const int* guard_flag, float clamp, int fast_rho, int inv_stat,
                         float dq_scale,
                         void* dq, void* dk, void* dv, float* di, float* dsink_scaled);

/* Cayley rotation tables, src/algebraic/algebraic.py:124-149 (cayley_powers): for the
 * frequencies w (half) f32, cos/sin (seq_len, half) f32 hold the rows
 * ((1 + i w)^2 / (1 + w^2))^m, m < seq_len, by binary exponentiation with a renormalisation
 * after every squaring, as the reference builds them. */
int alg_cayley_tables(alg_stream_t stream, const float* w, int half, int seq_len, float* cos, float* sin);

/* Bytes of workspace alg_attn_qk_prologue / alg_attn_qk_prologue_bwd need. */
size_t alg_attn_prologue_workspace_size(int B, int H, int T, int D);

/* Fused attention prologue, replacing model.py:170-174 (qk_norm = rms_norm with a learned
 * gain, algebraic.py:76-83; apply_rotary, algebraic.py:172-179) followed by
 * flash_attention's prologue and guard (flash.py:823-849), in one pass:
 *   k_r = rot(round((k tau_k) k_gain)),  q_s = round(rot(round((q tau_q) q_gain)) alpha),
 *   tau = 1/sqrt(mean(x^2) + eps) per row (written to tau_q / tau_k for the backward),
 *   alpha = 1/(sqrt(D) c); the guard flag and sink_scaled exactly as alg_attn_prepare
 *   (the guard's ||q_s||^2 and ||k||^2 maxima are taken over q_s and k_r).
 * q, k, v are read and q_s, k_r written in `layout`, the layout alg_attn_fwd / alg_attn_bwd
 * then take. Gains (D) f32 may be NULL (no gain); cos/sin (T, D/2) f32 may both be NULL
 * (no rotation); the tables are rounded to the input dtype before use, like the reference. */
int alg_attn_qk_prologue(alg_stream_t stream, int dtype, int layout, int B, int H, int T, int D,
                         const void* q, const void* k, const void* v,
                         const float* q_gain, const float* k_gain, const float* cos, const float* sin,
                         float eps, const float* sink_logit, int sink_count, float c, int n, int range_guard,
                         void* q_s, void* k_r, float* tau_q, float* tau_k, float* sink_scaled, int* guard_flag,
                         void* workspace, size_t workspace_bytes);

/* VJP of the fused prologue's normalisation and rotation (JAX autodiff of
 * algebraic.py:76-83 and 172-179): dq_r, dk_r (in `layout`) are the cotangents of the rotated
 * rows (alg_attn_bwd's dq with dq_scale = alpha, and its dk); out dq, dk in `layout` and the
 * gain gradients dq_gain, dk_gain (D) f32 (summed over all rows; NULL to skip). */
int alg_attn_qk_prologue_bwd(alg_stream_t stream, int dtype, int layout, int B, int H, int T, int D,
                             const void* q, const void* k, const float* q_gain, const float* k_gain,
                             const float* cos, const float* sin, const float* tau_q, const float* tau_k,
                             const void* dq_r, const void* dk_r, void* dq, void* dk,
                             float* dq_gain, float* dk_gain, void* workspace, size_t workspace_bytes);

/* Bytes of workspace for alg_head_fwd (pass 0), alg_head_bwd without a residual (pass 1),
 * alg_head_bwd with a residual (pass 2) and alg_head_eval (pass 3), for hidden states of
 * dtype ALG_DTYPE_BF16 or ALG_DTYPE_F32 (0 for f32 pass 2: the residual is bf16 only). */
size_t alg_head_workspace_size(int dtype, int N, int d, int V, int pass);

/* Bytes of the optional forward->backward residual: the token-major bf16 block
 * U = w*r (target entries (w_t - l) r_t) of Npad x Vp entries (U[tok, v] at tok * Vp + v,
 * Npad = N rounded up to 256, Vp = V rounded up to 8), then, at the next 256-byte boundary,
 * the row sums l (N floats). With it the backward needs no
 * logit recompute (3 products instead of 4); it has no counterpart in the reference, whose
 * residuals are (h, E, targets, stat) (fused_head.py:244). */
size_t alg_head_residual_size(int N, int d, int V);

/* Head forward, fused_head.py:72-117, 174-191, 219-229 (kind="alg_ce"):
 * in h (N,d) and E (V,d) of dtype ALG_DTYPE_BF16 or ALG_DTYPE_F32 (E already cast to h's
 * dtype, fused_head.py:168), targets (N) int32;
 * out stat (N) = l^(-1/n), zt (N) = target logits, pt (N) telemetry, obj (1) = mean(1-pt),
 * and, when residual is not NULL (bf16 only; ALG_ERR_UNSUPPORTED for f32), the residual for
 * alg_head_bwd. f32 runs the reference's computation in f32 throughout. The clamp
 * X = 1/4 (1e38/V)^(1/n) is derived from V and n. d must be a multiple of 8 and N at most 2^23. */
int alg_head_fwd(alg_stream_t stream, int dtype, int N, int d, int V,
                 const void* h, const void* E, const int32_t* targets, int n, float c,
                 float* stat, float* zt, float* pt, float* obj, void* residual,
                 void* workspace, size_t workspace_bytes);

/* Evaluation head, replacing the dense logits of the reference's scorer
 * (src/algebraic/benchmarking.py:178-188 with src/algebraic/evaluation.py:13-23, head
 * "alg_ce"): for h (N,d) and E (V,d) of dtype ALG_DTYPE_BF16 or ALG_DTYPE_F32 and targets
 * (N) int32, streams the vocabulary like
 * alg_head_fwd and writes logprob[n] = log_softmax(n asinh(z/c))[t_n] with no clamp (computed
 * as n (log rho(z_t/c) + log rho(-z_m/c)) - log sum_v (rho(z_v/c) rho(-z_m/c))^n, z_m the row's
 * largest logit, so no term overflows) and, if argmax is not NULL, argmax[n] = the first index
 * of the largest logit z_n (the first NaN if the row holds one, as jnp.argmax). No logits are
 * stored. */
int alg_head_eval(alg_stream_t stream, int dtype, int N, int d, int V,
                  const void* h, const void* E, const int32_t* targets, int n, float c,
                  float* logprob, int32_t* argmax, void* workspace, size_t workspace_bytes);

/* Row RMS norm with a learned gain, bf16 rows of d elements (d % 8 == 0, d <= 4096): the
 * model's final norm ahead of the head (model.py:208; rms_norm at algebraic.py:76-83).
 * Forward: tau[r] = 1/sqrt(mean(x_r^2) + eps), y = round((x tau) gain) (gain NULL: none).
 * Backward (JAX autodiff of the same expression): dx = round(a tau - x tau^3 sum(a x)/d) with
 * a = gain dy, and dgain (d) f32 = sum over rows of dy x tau (NULL to skip; then no workspace).
 * x, y, dy and dx are row-major and 16-byte aligned (ALG_ERR_INVALID otherwise). */
size_t alg_rms_norm_workspace_size(int rows, int d);
int alg_rms_norm_fwd(alg_stream_t stream, int rows, int d, const void* x, const float* gain, float eps,
                     void* y, float* tau);
int alg_rms_norm_bwd(alg_stream_t stream, int rows, int d, const void* x, const float* gain, const float* tau,
                     const void* dy, void* dx, float* dgain, void* workspace, size_t workspace_bytes);

/* ALU-GLU feed-forward (model.py:185-193, ffn = "alu_glu"; alu and its VJP algebraic.py:86-113),
 * bf16, d_ff = F a multiple of 128. Forward: for h2 (N, d) and w_gu = [w_g | w_u] (d, 2F),
 * gate = round(h2 w_g), up = round(h2 w_u), y = round(gate alu(up)) (alu with the negative-tail
 * form, beta its slope), all (N, F); y w_d is then a plain product. Backward: for the block
 * output's cotangent dout (N, dm) and w_d (F, dm), dy = round(dout w_d^T) and
 * d_gu = [round(dy alu(up)) | round(round(dy gate) alu'(up))] (N, 2F); dh2 = d_gu w_gu^T and
 * [dw_g | dw_u] = h2^T d_gu are then plain products. Every matrix is row-major, contiguous and
 * 16-byte aligned (ALG_ERR_INVALID otherwise). */
int alg_ffn_alu_glu_fwd(alg_stream_t stream, int N, int d, int F, const void* h2, const void* w_gu, float beta,
                        void* y, void* gate, void* up);
int alg_ffn_alu_glu_dy(alg_stream_t stream, int N, int dm, int F, const void* dout, const void* w_d,
                       const void* gate, const void* up, float beta, void* d_gu);

/* The block's plain products (the matmuls of model.py:185-193 that carry no activation: y w_d,
 * d_gu w_gu^T, h2^T d_gu, y^T dout; the reference leaves them to XLA): C (M, N) = A B in bf16,
 * one rounding of the f32 sum, C row-major with leading dimension ldc. A is (M, K) stored
 * row-major (a_trans = 0, lda >= K) or stored as its transpose, (K, M) row-major (a_trans = 1,
 * lda >= M); B is (K, N) stored row-major (b_trans = 0, ldb >= N) or as its transpose (N, K)
 * (b_trans = 1, ldb >= K). The stored rows' lengths (K, M or N as the layouts give), N and the
 * leading dimensions are multiples of 8 and A, B, C 16-byte aligned (ALG_ERR_INVALID
 * otherwise). When the last round of output tiles would leave CUs idle those tiles are split
 * over k into f32 workspace tiles summed in a fixed order: the workspace holds
 * alg_ffn_gemm_workspace_size(M, N, K) bytes (0 when there is no split). */
size_t alg_ffn_gemm_workspace_size(int M, int N, int K);
int alg_ffn_gemm(alg_stream_t stream, int M, int N, int K, const void* A, long lda, int a_trans, const void* B,
                 long ldb, int b_trans, void* C, long ldc, void* workspace, size_t workspace_bytes);

/* Head backward, fused_head.py:120-156, 194-216, 247-254:
 * in h, E (of dtype ALG_DTYPE_BF16 or ALG_DTYPE_F32), targets, stat, g (1) f32 on the device
 * (cotangent of obj) and optionally the forward's residual (bf16 only); out dh (N,d) in h's
 * dtype and dE (V,d) in dE_dtype (ALG_DTYPE_BF16 or ALG_DTYPE_F32). Without a residual the
 * logits are recomputed (the reference's schedule; f32 keeps dZ in f32 as the reference does
 * for f32 h). */
int alg_head_bwd(alg_stream_t stream, int dtype, int N, int d, int V,
                 const void* h, const void* E, const int32_t* targets, const float* stat,
                 const float* g, int n, float c, const void* residual, void* dh, void* dE, int dE_dtype,
                 void* workspace, size_t workspace_bytes);

/* Head backward with the vocabulary streamed, fused_head.py:120-156, 194-216, 247-254 without
 * the (N, V) logit-gradient block the reference writes (dz_ref, fused_head.py:145-146) and
 * feeds to XLA's dE product (:215). Arguments as alg_head_bwd without a residual (the forward
 * ran with residual NULL). The vocabulary is processed in chunks of vocab_chunk rows (0: the
 * default, enough rows for one chunk's dE product to fill the chip, 8192 at d = 2048; else a
 * positive multiple of 256, ALG_ERR_INVALID otherwise): per chunk the logits are recomputed,
 * the chunk's logit gradient is formed in the workspace, its dh product is accumulated in f32
 * and its rows of dE are written. Workspace: alg_head_streamed_workspace_size bytes, bounded
 * by the chunk (bf16: Npad x chunk bf16 + N x d f32 for the dh accumulator; f32: N x chunk f32)
 * instead of V. */
size_t alg_head_streamed_workspace_size(int dtype, int N, int d, int V, int vocab_chunk);
int alg_head_bwd_streamed(alg_stream_t stream, int dtype, int N, int d, int V,
                          const void* h, const void* E, const int32_t* targets, const float* stat,
                          const float* g, int n, float c, int vocab_chunk, void* dh, void* dE, int dE_dtype,
                          void* workspace, size_t workspace_bytes);

/* Measurement hook (no counterpart in the reference; for benchmarks and profilers):
 * while enabled, every kernel launch of this library records a HIP event pair on its
 * stream. alg_timer_report() waits for those events, writes a JSON object
 * {"kernel": {"launches": L, "mean_ms": M}, ...} into out (truncated to cap bytes, NUL
 * terminated), clears the records and returns the full length + 1. Not thread-safe with
 * concurrent timed launches. */
void alg_timer_enable(int on);
size_t alg_timer_report(char* out, size_t cap);

#ifdef __cplusplus
}
#endif

#endif /* ALGEBRAIC_HIP_H */
