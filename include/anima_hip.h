/*
 * anima_hip.h -- C-ABI of libanima_hip.so, the MI355X (gfx950) attention path
 * of the Anima 2B DiT.
 *
 * Part 1 is a drop-in for the anima_rt symbols that the torch-free NumpyDiT
 * host path binds through ctypes (anima_rt/scripts/anima_rt_ops.py:10-36,
 * scripts/phone_pipeline_nd.py:46-68): same names, same argument meaning,
 * host pointers, synchronous, bool result.  Part 2 adds device-pointer entry
 * points, the fused Q/K prologue, a one-call NumpyAttention core and the
 * cross-attention context K/V cache.
 *
 * Conventions
 *   - All tensors are row-major with the innermost axis contiguous.
 *   - A false return means nothing useful was written; the reason is
 *     available from anima_hip_last_error() (per calling thread).
 *   - Host-pointer entry points (Part 1, anima_hip_attention*,
 *     anima_hip_ctx_kv_create) copy to the GPU, run, copy back and return
 *     when the output is complete.  They are serialised by a library mutex.
 *     Copies of 4 MiB and more pass through pinned staging buffers, with
 *     the host memcpy split over the caller and up to 5 library threads.
 *   - "_dev" entry points take device pointers and a hipStream_t (passed as
 *     void*; NULL = HIP's default stream) and are asynchronous: they only
 *     enqueue work on that stream.
 *   - Stride arrays are int64[3] = {batch, head, sequence} element strides of
 *     a [B, H, S, D] view (D contiguous).  NULL means contiguous [B,H,S,D].
 *     A batch stride of 0 broadcasts batch entry 0 to every batch.
 */
#ifndef ANIMA_HIP_H
#define ANIMA_HIP_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ===================== Part 1: anima_rt drop-in ===================== */

/* Replaces anima_rt_init (anima_rt/src/anima_rt.cpp:13-20).  Binds the
 * current HIP device and creates the library's stream.  Idempotent; returns
 * false when no GPU is usable. */
bool anima_rt_init(void);

/* Replaces anima_rt_destroy (anima_rt.cpp:166-171).  Frees the workspace and
 * the stream; a later call to any entry point may initialise again. */
void anima_rt_destroy(void);

/* Replaces anima_rt_run_sdpa_flash (anima_rt.cpp:147-156).
 * Q,out: [BH, S_q, D]; K,V: [BH, S_kv, D]; fp32 host memory.
 * out = softmax(scale * Q K^T [masked j > i when is_causal]) V.
 * Like the reference, works without a prior anima_rt_init. */
bool anima_rt_run_sdpa_flash(const float *Q, const float *K, const float *V, float *out,
                             int BH, int S_q, int S_kv, int D, float scale, bool is_causal);

/* Replaces anima_rt_run_sdpa (anima_rt.cpp:78-141), the "math" entry.  The
 * reference scales both Q and K by `scale` (anima_rt.cpp:95-98), so it
 * computes softmax(scale^2 * Q K^T) V; this entry keeps that result so
 * existing callers see the same numbers.  Returns false unless
 * anima_rt_init() succeeded first (anima_rt.cpp:84). */
bool anima_rt_run_sdpa(const float *Q, const float *K, const float *V, float *out,
                       int BH, int S_q, int S_kv, int D, float scale, bool is_causal);

/* Replaces anima_rt_run_rmsnorm (anima_rt.cpp:45-50 -> rmsnorm_kernel,
 * anima_rt/include/cpu/rmsnorm_kernel.h:11-31).  x,out: [m, d]; w: [d] or
 * NULL.  Bit-identical to the reference.  Returns false unless anima_rt_init()
 * succeeded first (anima_rt.cpp:47). */
bool anima_rt_run_rmsnorm(const float *x, const float *w, float *out, int m, int d, float eps);

/* Replace anima_rt_run_gelu / anima_rt_run_silu (anima_rt.cpp:24-32 ->
 * gelu_kernel.h:13-23, exact erf form, and silu_kernel.h:9-17): out[i] =
 * f(x[i]) for i < n.  False (with a message) before anima_rt_init(), as the
 * reference without a backend; n <= 0 does nothing. */
bool anima_rt_run_gelu(const float *x, float *out, int n);
bool anima_rt_run_silu(const float *x, float *out, int n);

/* Replaces anima_rt_run_layernorm (anima_rt.cpp:36-43 -> layernorm_kernel.h:13-33):
 * LayerNorm without affine parameters over the rows of x [m, d].  False before
 * anima_rt_init(). */
bool anima_rt_run_layernorm(const float *x, float *out, int m, int d, float eps);

/* Replaces anima_rt_run_softmax (anima_rt.cpp:52-57 -> softmax_kernel.h:16-40):
 * softmax over the last axis of x [outer, dim].  False before anima_rt_init(). */
bool anima_rt_run_softmax(const float *x, float *out, int outer, int dim);

/* Replaces anima_rt_run_bias_add (gemm_backend.cpp:173-183): C[i][j] += bias[j]
 * on host memory C [M, N]; a NULL bias does nothing.  Needs no init, like the
 * reference. */
bool anima_rt_run_bias_add(float *C, const float *bias, int M, int N);

/* Replaces anima_rt_run_rope (anima_rt.cpp:160-164 -> rope_kernel,
 * anima_rt/include/cpu/rope_kernel.h:65-97).  t,out: [N, S, D];
 * freqs: [S, D/2, 2, 2].  Bit-identical to the reference. */
bool anima_rt_run_rope(const float *t, const float *freqs, float *out, int N, int S, int D);

/* Replaces anima_rt_run_gemm_fp32 (anima_rt/src/gemm_backend.cpp:140-148):
 * C[M,N] = A[M,K] . B[N,K]^T, f32 host arrays, f32 accumulation.  Off the
 * attention path; exported so the library can stand in for all of libanima_rt's
 * GEMM symbols. */
bool anima_rt_run_gemm_fp32(const float *A, const float *B, float *C, int M, int N, int K);

/* Replaces anima_rt_run_gemm_bf16 (gemm_backend.cpp:154-173):
 * C[M,N] = A[M,K] . W[N,K]^T with W as bf16 bit patterns (uint16), A and C
 * f32, f32 accumulation. */
bool anima_rt_run_gemm_bf16(const float *A, const uint16_t *W, float *C, int M, int N, int K);

/* ===================== Part 2: extensions ===================== */

/* Message describing the last failure on this thread ("" if none). */
const char *anima_hip_last_error(void);

/* ABI version of this header (major*100 + minor). */
int anima_hip_version(void);

/* Attention arithmetic modes. */
enum {
    ANIMA_HIP_F32 = 0,   /* f32 inputs, f32 MFMA, f32 accumulate            */
    ANIMA_HIP_BF16 = 1,  /* bf16 Q/K/V and P, f32 MFMA accumulate + softmax */
    ANIMA_HIP_F32X3 = 2  /* f32 inputs on bf16 MFMA: each operand as two bf16
                          * terms x = xh + xl (+ <= 2^-17 |x|), each product
                          * as xh*yh + xh*yl + xl*yh, f32 accumulate and
                          * softmax (D == 128)                               */
};

/* anima_rt_run_sdpa_flash with an arithmetic mode: host pointers, same
 * layouts and semantics; mode ANIMA_HIP_F32 is identical to the drop-in,
 * ANIMA_HIP_BF16 rounds Q, K, V (and P) to bf16 for the MFMAs, ANIMA_HIP_F32X3
 * takes them as bf16 term pairs (both D == 128). */
bool anima_hip_sdpa(const float *Q, const float *K, const float *V, float *out, int BH, int S_q,
                    int S_kv, int D, float scale, bool is_causal, int mode);

/* Flash attention on device f32 tensors (mode ANIMA_HIP_F32).  Same math as
 * anima_rt_run_sdpa_flash with strided [B,H,S,D] views. */
bool anima_hip_flash_f32_dev(const float *q, const float *k, const float *v, float *o,
                             int B, int H, int S_q, int S_kv, int D,
                             const int64_t *q_strides, const int64_t *k_strides,
                             const int64_t *v_strides, const int64_t *o_strides,
                             float scale, bool is_causal, void *stream);

/* Flash attention on device bf16 tensors (mode ANIMA_HIP_BF16): q, k are
 * bf16 [B,H,S,D] views (strides as above), vt is V packed by
 * anima_hip_pack_vt_dev, o is f32.  D must be 128 and scale > 0.  Scores,
 * softmax and accumulation are f32; Q, K, V and P enter the MFMAs as bf16.
 * vt_strides = {batch, head, d-row} (the d-row stride must equal
 * anima_hip_vt_padded_len(S_kv)); NULL = packed contiguous. */
bool anima_hip_flash_bf16_dev(const uint16_t *q, const uint16_t *k, const uint16_t *vt,
                              float *o, int B, int H, int S_q, int S_kv, int D,
                              const int64_t *q_strides, const int64_t *k_strides,
                              const int64_t *vt_strides, const int64_t *o_strides,
                              float scale, bool is_causal, void *stream);

/* Key count of one packed V^T row: S_kv rounded up to a multiple of 64. */
int64_t anima_hip_vt_padded_len(int S_kv);

/* Pack f32 V ([B,H,S_kv,D] view through v_strides, D = 128) into the bf16
 * V^T layout of anima_hip_flash_bf16_dev: per (batch, head) a
 * [D][anima_hip_vt_padded_len(S_kv)] matrix, zero-padded, with keys permuted
 * inside each group of 16 (offsets 4-7 and 8-11 swapped). */
bool anima_hip_pack_vt_dev(const float *v, uint16_t *vt, int B, int H, int S_kv, int D,
                           const int64_t *v_strides, const int64_t *vt_strides, void *stream);

/* Flash attention on device bf16 term tensors (mode ANIMA_HIP_F32X3): q, k
 * hold rows of 2*D bf16, [hi | lo] with hi = bf16(x) and lo = bf16(x - hi)
 * (anima_hip_qk_prologue_dev with flags & 4), the strides giving the row
 * starts (NULL: [B,H,S,2D] contiguous); vt is V packed by
 * anima_hip_pack_vt_terms_dev; o is f32.  D must be 128 and scale > 0.  Each
 * product runs as three bf16 MFMA products (hi*hi + hi*lo + lo*hi) with f32
 * accumulation; scores and softmax are f32, and P enters as two terms too. */
bool anima_hip_flash_x3_dev(const uint16_t *q, const uint16_t *k, const uint16_t *vt,
                            float *o, int B, int H, int S_q, int S_kv, int D,
                            const int64_t *q_strides, const int64_t *k_strides,
                            const int64_t *vt_strides, const int64_t *o_strides,
                            float scale, bool is_causal, void *stream);

/* anima_hip_flash_f32_dev with q given as raw f32 projection rows ([B,S_q,H,D]
 * through q_strides, NULL = contiguous; D == 128, 16-byte aligned rows): the
 * kernel applies the per-head RMSNorm (q_norm_w may be NULL) itself,
 * bit-identical to anima_hip_qk_prologue_dev (flags 1) followed by
 * anima_hip_flash_f32_dev.  No RoPE.  NumpyAttention.forward's cross-attention
 * q path (anima_rt/scripts/numpy_dit.py:285-286) and its attention in one
 * launch; the cross-attention entries use it on unsplit 8-wave grids. */
bool anima_hip_flash_f32_rawq_dev(const float *q, const float *q_norm_w, float eps,
                                  const float *k, const float *v, float *o, int B, int H,
                                  int S_q, int S_kv, int D, const int64_t *q_strides,
                                  const int64_t *k_strides, const int64_t *v_strides,
                                  const int64_t *o_strides, float scale, bool is_causal,
                                  void *stream);

/* anima_hip_flash_x3_dev with q given as raw f32 projection rows ([B,S_q,H,D]
 * through q_strides, NULL = contiguous; 16-byte aligned rows): the kernel
 * applies the per-head RMSNorm (q_norm_w may be NULL), the RoPE of freqs
 * ([S_q, D/2, 2, 2] or NULL) and the hi/lo term split itself, bit-identical to
 * anima_hip_qk_prologue_dev (flags 1 | 4) followed by anima_hip_flash_x3_dev.
 * NumpyAttention.forward's q path (anima_rt/scripts/numpy_dit.py:285-291)
 * and its attention in one launch; the cross-attention entries use it on
 * unsplit grids. */
bool anima_hip_flash_x3_rawq_dev(const float *q, const float *q_norm_w, const float *freqs,
                                 float eps, const uint16_t *k, const uint16_t *vt, float *o,
                                 int B, int H, int S_q, int S_kv, int D,
                                 const int64_t *q_strides, const int64_t *k_strides,
                                 const int64_t *vt_strides, const int64_t *o_strides,
                                 float scale, bool is_causal, void *stream);

/* anima_hip_flash_bf16_dev with q given as raw f32 projection rows
 * ([B,S_q,H,D] through q_strides, NULL = contiguous; 16-byte aligned rows):
 * the kernel applies the per-head RMSNorm (q_norm_w may be NULL) and the RoPE
 * of freqs ([S_q, D/2, 2, 2] or NULL) and rounds the rows to bf16 itself,
 * bit-identical to anima_hip_qk_prologue_dev (flags 1 | 2) followed by
 * anima_hip_flash_bf16_dev.  NumpyAttention.forward's q path
 * (anima_rt/scripts/numpy_dit.py:285-291) and its attention in one launch;
 * the bf16 cross-attention entries use it where the kernel runs two 4-wave
 * workgroups per CU (large grids over at most 1024 keys). */
bool anima_hip_flash_bf16_rawq_dev(const float *q, const float *q_norm_w, const float *freqs,
                                   float eps, const uint16_t *k, const uint16_t *vt, float *o,
                                   int B, int H, int S_q, int S_kv, int D,
                                   const int64_t *q_strides, const int64_t *k_strides,
                                   const int64_t *vt_strides, const int64_t *o_strides,
                                   float scale, bool is_causal, void *stream);

/* Pack f32 V into the term V^T layout of anima_hip_flash_x3_dev: per (batch,
 * head) the [D][anima_hip_vt_padded_len(S_kv)] hi matrix of
 * anima_hip_pack_vt_dev's layout followed by the same matrix of lo terms
 * bf16(v - bf16(v)).  vt_strides = {batch, head, d-row}; NULL = contiguous. */
bool anima_hip_pack_vt_terms_dev(const float *v, uint16_t *vt, int B, int H, int S_kv, int D,
                                 const int64_t *v_strides, const int64_t *vt_strides,
                                 void *stream);

/* Fused per-row prologue on device memory: for each row (b, s, h) of x,
 * optional RMSNorm (flags & 1; weight w may be NULL) followed by optional
 * rotate-half RoPE (freqs [S, D/2, 2, 2] or NULL), written through
 * out_strides as f32 or, with flags & 2, bf16 (round to nearest even), or,
 * with flags & 4, as bf16 terms: hi = bf16(y) at the row, lo = bf16(y - hi) D
 * elements after it (rows of [hi | lo], the q/k input of
 * anima_hip_flash_x3_dev).
 * This is NumpyAttention.forward's q/k path (anima_rt/scripts/numpy_dit.py:285-291):
 * RMSNorm (numpy_dit.py:285-286) -> RoPE (:288-289) -> transpose (:291). */
bool anima_hip_qk_prologue_dev(const float *x, void *out, const float *w, const float *freqs,
                               int B, int S, int H, int D,
                               const int64_t *x_strides, const int64_t *out_strides,
                               float eps, int flags, void *stream);

/* All three operands of a self-attention's flash call in one launch: the q
 * and k rows of anima_hip_qk_prologue_dev (RMSNorm with q_norm_w / k_norm_w,
 * NULL meaning weight 1, then RoPE with freqs [S, D/2, 2, 2] or NULL) and, in
 * the bf16 and f32x3 modes, V packed as anima_hip_pack_vt_dev /
 * anima_hip_pack_vt_terms_dev pack it.  This is NumpyAttention.forward's
 * q/k/v preparation (anima_rt/scripts/numpy_dit.py:283-291) for the
 * attention kernels.  q, k, v: [B, S, H, D] f32 views with token rows ld
 * elements apart (ld = 0: H*D; wider for column blocks of one fused
 * projection), batch entries S*ld apart; D == 128; 16-byte aligned.
 * Outputs, dense: qo, ko as [B, S, H, D] f32 (ANIMA_HIP_F32), [B, S, H, D]
 * bf16 (ANIMA_HIP_BF16) or [B, S, H, 2D] bf16 term rows (ANIMA_HIP_F32X3);
 * vt as [B, H, D (bf16) or 2D (terms), anima_hip_vt_padded_len(S)] (unused
 * and may be NULL in f32 mode).  Bit-identical to the separate entries. */
bool anima_hip_qkv_prologue_dev(const float *q, const float *k, const float *v, int64_t ld,
                                const float *q_norm_w, const float *k_norm_w,
                                const float *freqs, void *qo, void *ko, uint16_t *vt, int B,
                                int S, int H, int D, float eps, int mode, void *stream);

/* A self-attention's q/k/v projection and that prologue in one launch, for
 * the f32 modes at large token counts: x [B*S][ldx] f32 activations times
 * the stacked weights w_qkv [3*H*128][ldw] (bf16 bit patterns; q rows, then k,
 * then v: NumpyAttention.forward's q_proj, k_proj, v_proj,
 * anima_rt/scripts/numpy_dit.py:273-281) in anima_hip_linear_dev's exact
 * two-term product, whose epilogue writes the attention operands in place of
 * the projection: qo and ko as anima_hip_qkv_prologue_dev writes them (with
 * RMSNorm weights q_norm_w / k_norm_w, NULL meaning 1, and RoPE with freqs
 * [S, 64, 2, 2] or NULL) and vo as the term V^T (ANIMA_HIP_F32X3) or as
 * dense f32 V rows [B, S, H, 128] (ANIMA_HIP_F32).  Bit-identical to
 * anima_hip_linear_dev into [B*S][3*H*128] followed by
 * anima_hip_qkv_prologue_dev on its column blocks (whose f32-mode V is the
 * projection's v block itself).  Needs S a multiple of 64, H even, K a
 * multiple of 32, ldx % 4 == 0, ldw % 8 == 0, 16-byte aligned operands, and
 * (B*S/256) * (3*H/2) >= 256 (a grid that fills the GPU); other shapes are
 * refused with a message (use the two separate entries).  No counterpart in
 * the reference, whose projections and prologue are separate host steps. */
bool anima_hip_qkv_projection_dev(const float *x, int64_t ldx, const uint16_t *w_qkv,
                                  int64_t ldw, int K, const float *q_norm_w,
                                  const float *k_norm_w, const float *freqs, void *qo, void *ko,
                                  void *vo, int B, int S, int H, float eps, int mode,
                                  void *stream);

/* C[M,N] = A[M,K] . W[N,K]^T on device memory; W is bf16 bit patterns when
 * w_bf16 != 0, else f32; leading dimensions in elements. */
bool anima_hip_gemm_dev(const float *a, int64_t lda, const void *w, int w_bf16, int64_t ldw,
                        float *c, int64_t ldc, int M, int N, int K, void *stream);

/* Projection GEMM of the attention block on bf16 MFMA: C[M,N] = A[M,K] . W[N,K]^T
 * with f32 activations a, bf16 weights w (bit patterns, [out_features, in_features]
 * like the reference) and f32 output c, on device memory.  Replaces the
 * projections of NumpyAttention.forward (anima_rt/scripts/numpy_dit.py:273-281,
 * 294-296), computed there by anima_rt/vulkan/gemm_bf16.comp:25-57.
 *   mode ANIMA_HIP_F32 (and ANIMA_HIP_F32X3, the same here): a enters as two
 *                        bf16 terms hi + lo (per-element representation
 *                        error <= 2^-16 |a|), f32 accumulation;
 *   mode ANIMA_HIP_BF16: a is rounded to bf16 (<= 2^-8 |a|).
 * scratch: anima_hip_linear_scratch_bytes(M, K, mode) bytes of device memory,
 * 16-byte aligned; nothing is allocated.  At M <= 1024 with K a multiple of 64
 * (f32 modes, or bf16 mode with K >= 8192) the size includes 16 MiB for the
 * split-K partials of the hand-written small-M GEMM, which then runs instead
 * of the library GEMM; the partials are added in a fixed order, so results
 * are deterministic.  At large M (a grid of at least 256 tiles of 256 x 256
 * or 128 x 256, K a multiple of 32, 16-byte aligned A rows with lda % 4 == 0)
 * the f32 modes, and the bf16 mode where N and K are at most 2048, run a
 * kernel that stages the f32 rows of a and splits (or rounds) them in
 * registers (in the f32 modes bit-identical to the split pass followed by a
 * two-term product on the term rows).  Shapes without a
 * library solution (e.g. ldw not a multiple of 8) run the exact f32-MFMA
 * kernel instead. */
size_t anima_hip_linear_scratch_bytes(int M, int K, int mode);
bool anima_hip_linear_dev(const float *a, int64_t lda, const uint16_t *w, int64_t ldw, float *c,
                          int64_t ldc, int M, int N, int K, int mode, void *scratch,
                          size_t scratch_bytes, void *stream);

/* Device scratch needed by anima_hip_attention_dev for these sizes (bytes). */
size_t anima_hip_attention_scratch_bytes(int B, int S_q, int Bk, int S_kv, int H, int D,
                                         int mode);

/* Device-memory form of anima_hip_attention: q [B,S_q,H,D], k/v
 * [Bk,S_kv,H,D] f32 projections with Bk == B or Bk == 1 (one K/V batch shared
 * by every query batch); weights [D] and RoPE table [S_q,D/2,2,2] may be NULL;
 * out [B,S_q,H,D] f32.  `scratch` holds at least
 * anima_hip_attention_scratch_bytes() bytes; nothing is allocated. */
bool anima_hip_attention_dev(const float *q, const float *k, const float *v,
                             const float *q_norm_w, const float *k_norm_w, const float *freqs,
                             float *out, void *scratch, size_t scratch_bytes, int B, int S_q,
                             int Bk, int S_kv, int H, int D, float eps, int mode, void *stream);

/* anima_hip_attention_dev with O written as the bf16 terms of the input of a
 * bf16-MFMA projection of O instead of f32 (no counterpart in the
 * reference: NumpyAttention.forward hands O to output_proj as f32,
 * anima_rt/scripts/numpy_dit.py:294-296, and this form saves the pass that
 * splits it).  Token row t = b*S_q + s of out_terms is ld_terms bf16
 * elements long: hi = bf16(O) (round to nearest even) at column h*D + d and,
 * when lo_offset > 0, lo = bf16(O - hi) at lo_offset + h*D + d -- the terms
 * anima_hip_linear_dev forms from an f32 A (one term in ANIMA_HIP_BF16 mode,
 * two otherwise), bit for bit.  D must be 128; out_terms 16-byte aligned;
 * ld_terms and lo_offset multiples of 8, lo_offset >= H*D and
 * lo_offset + H*D <= ld_terms.  Same scratch as anima_hip_attention_dev. */
bool anima_hip_attention_terms_dev(const float *q, const float *k, const float *v,
                                   const float *q_norm_w, const float *k_norm_w,
                                   const float *freqs, uint16_t *out_terms, int64_t ld_terms,
                                   int64_t lo_offset, void *scratch, size_t scratch_bytes, int B,
                                   int S_q, int Bk, int S_kv, int H, int D, float eps, int mode,
                                   void *stream);

/* anima_hip_attention_dev without scratch and without any allocation.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops that forbid
 * hipMalloc).  Same arguments, kernels and results as
 * anima_hip_attention_dev; the scratch is a static device array of
 * ANIMA_HIP_STATIC_SCRATCH_BYTES that each GPU holds from the first call
 * made on it until the process ends (measured on MI355X: the library's
 * other entries leave it unreserved; free device memory drops by 194 MiB
 * at the first static call).  The array's device address is looked up once
 * per GPU, at that first call, and kept: resetting a device
 * (hipDeviceReset) while the library is loaded is not supported.  The first
 * call may itself be captured into a HIP graph.  A problem whose
 * anima_hip_attention_scratch_bytes() exceeds that size is rejected (false,
 * with a message) before anything is enqueued; 192 MiB covers the
 * 1024x1024 image's self-attention (B = 2, 4096 tokens, 16 x 128) in every
 * mode.  Every call on one GPU shares its array, so calls that overlap on
 * one GPU (other streams or threads) race: the caller serialises them.
 * Asynchronous on `stream`. */
#define ANIMA_HIP_STATIC_SCRATCH_BYTES (192u * 1024u * 1024u)
bool anima_hip_attention_static_dev(const float *q, const float *k, const float *v,
                                    const float *q_norm_w, const float *k_norm_w,
                                    const float *freqs, float *out, int B, int S_q, int Bk,
                                    int S_kv, int H, int D, float eps, int mode, void *stream);

/* One-call core of NumpyAttention.forward (numpy_dit.py:283-294) on host
 * memory: q [B,S_q,H,D], k/v [B,S_kv,H,D] (the projections), optional
 * per-head RMSNorm weights [D], optional RoPE table [S_q, D/2, 2, 2]
 * (self-attention only; requires S_q == S_kv), scale 1/sqrt(D), no mask.
 * Writes out [B,S_q,H,D], i.e. the [B*S_q, H*D] input of output_proj.
 * mode: ANIMA_HIP_F32, ANIMA_HIP_F32X3 or ANIMA_HIP_BF16 (the last two need
 * D == 128). */
bool anima_hip_attention(const float *q, const float *k, const float *v,
                         const float *q_norm_w, const float *k_norm_w, const float *freqs,
                         float *out, int B, int S_q, int S_kv, int H, int D, float eps,
                         int mode);

/* ---- Cross-attention over a cached text context ----
 * The context K/V of a cross-attention block depend only on the text context
 * and the block's weights, not on the latent or the denoise step
 * (anima_rt/scripts/sampling.py:121-138 feeds the same context every step;
 * numpy_dit.py:277-286 recomputes the projections and k_norm each call).  A
 * cache holds them on the GPU in the attention layout of `mode`:
 *   K = RMSNorm_head(ctx . Wk^T) (k_norm weight, eps), V = ctx . Wv^T.
 * ctx: [Bc, S_kv, C] f32 host; Wk, Wv: [H*D, C] bf16 bit patterns (the
 * safetensors [out_features, in_features] layout); k_norm_w: [D] or NULL.
 * Bc = 1 serves every query batch (both CFG branches share one context);
 * otherwise Bc must equal the query batch.  mode: ANIMA_HIP_F32,
 * ANIMA_HIP_F32X3 or ANIMA_HIP_BF16 (projections on exact hi+lo terms except
 * in bf16 mode).  Returns NULL on failure. */
typedef struct anima_hip_ctx_kv anima_hip_ctx_kv;

anima_hip_ctx_kv *anima_hip_ctx_kv_create(const float *ctx, const uint16_t *wk, const uint16_t *wv,
                                          const float *k_norm_w, int Bc, int S_kv, int C, int H,
                                          int D, float eps, int mode);
void anima_hip_ctx_kv_destroy(anima_hip_ctx_kv *kv);

/* Cross-attention of q [B, S_q, H, D] (q_proj output, f32 host) against the
 * cached context: q = RMSNorm_head(q) (q_norm_w [D] or NULL), no RoPE, no mask,
 * scale 1/sqrt(D).  out: [B, S_q, H, D] f32 host. */
bool anima_hip_cross_attention(const float *q, const float *q_norm_w, const anima_hip_ctx_kv *kv,
                               float *out, int B, int S_q, float eps);

/* Device scratch for anima_hip_cross_attention_dev (bytes). */
size_t anima_hip_cross_attention_scratch_bytes(const anima_hip_ctx_kv *kv, int B, int S_q);

/* Device-memory form of anima_hip_cross_attention (q, q_norm_w, out on the
 * device; nothing is allocated). */
bool anima_hip_cross_attention_dev(const float *q, const float *q_norm_w,
                                   const anima_hip_ctx_kv *kv, float *out, void *scratch,
                                   size_t scratch_bytes, int B, int S_q, float eps, void *stream);

/* anima_hip_cross_attention_dev writing O as the bf16 terms of the output
 * projection's input instead of f32 (no counterpart in the reference, like
 * anima_hip_attention_terms_dev, whose out_terms / ld_terms / lo_offset rules
 * it follows; D of the cache must be 128).  The DiT's cross-attention
 * sub-layer runs this form. */
bool anima_hip_cross_attention_terms_dev(const float *q, const float *q_norm_w,
                                         const anima_hip_ctx_kv *kv, uint16_t *out_terms,
                                         int64_t ld_terms, int64_t lo_offset, void *scratch,
                                         size_t scratch_bytes, int B, int S_q, float eps,
                                         void *stream);

/* One attention sub-block of a DiT block on the device-resident residual
 * stream (NumpyBlock.forward, anima_rt/scripts/numpy_dit.py:236-247):
 *   x += gate[b] * output_proj(attention(layernorm(x) * (1 + scale[b]) + shift[b]))
 * x: [B*S, Dm] f32, updated in place; mod: [B][3][Dm] f32 = (shift, scale,
 * gate), the three chunks of the block's AdaLN output (numpy_dit.py:218-228);
 * wq/wk/wv: [H*D, Dm], wo: [Dm, H*D] bf16 bit patterns like the reference's
 * weights.  kv == NULL: self-attention (k/v from the modulated x, RoPE with
 * freqs [S, D/2, 2, 2] or NULL).  kv != NULL: cross-attention over that
 * context cache (wk, wv, k_norm_w and freqs unused; H, D and mode must match
 * the cache).  LayerNorm has no affine parameters, as the reference calls it.
 * mode ANIMA_HIP_F32: projections on exact hi+lo bf16 terms and the f32
 * attention path; ANIMA_HIP_F32X3: the same projections and the f32x3
 * attention; ANIMA_HIP_BF16: bf16 activations throughout.  Dm and H*D
 * must be multiples of 8, Dm <= 4096.  scratch: device memory of
 * anima_hip_attention_block_scratch_bytes(kv, B, S, Dm, H, D, mode) bytes,
 * 16-byte aligned; nothing is allocated.  Asynchronous on `stream`. */
size_t anima_hip_attention_block_scratch_bytes(const anima_hip_ctx_kv *kv, int B, int S, int Dm,
                                               int H, int D, int mode);
bool anima_hip_attention_block_dev(float *x, const float *mod, const uint16_t *wq,
                                   const uint16_t *wk, const uint16_t *wv, const uint16_t *wo,
                                   const float *q_norm_w, const float *k_norm_w,
                                   const float *freqs, const anima_hip_ctx_kv *kv, int B, int S,
                                   int Dm, int H, int D, float eps, int mode, void *scratch,
                                   size_t scratch_bytes, void *stream);


/* ---- Model weights in the reference's on-disk format (safetensors) ----
 * The file the reference loads at scripts/phone_pipeline_nd.py:15-43 (read in
 * C++ by vulkan/safetensors_reader.h): u64 header length, JSON header of
 * {name: {dtype, shape, data_offsets}}, raw data.  Opened read-only and
 * memory-mapped; the header is validated (offsets inside the file, byte
 * counts matching dtype and shape).  Names match with or without the
 * reference's "net." prefix.  dtype codes: 0 = F32, 1 = F16, 2 = BF16 (the
 * codes of the reference's vk_weight_add, phone_pipeline_nd.py:31). */
typedef struct anima_hip_weights anima_hip_weights;
/* NULL on error (anima_hip_last_error() says why). */
anima_hip_weights *anima_hip_weights_open(const char *path);
/* Frees the device copies (after draining the device) and unmaps the file. */
void anima_hip_weights_close(anima_hip_weights *w);
int anima_hip_weights_count(const anima_hip_weights *w);
/* Name of tensor i without the "net." prefix; NULL when out of range. */
const char *anima_hip_weights_name(const anima_hip_weights *w, int i);
/* dtype code and up to max_ndim dimensions of a tensor; returns its rank,
 * or -1 when absent. */
int anima_hip_weights_info(const anima_hip_weights *w, const char *name, int *dtype,
                           int64_t *shape, int max_ndim);
/* Device copy of a tensor, uploaded on first request and resident until
 * close: as stored (as_f32 == 0; BF16 linear weights stay bit patterns, the
 * form anima_hip_linear_dev takes) or widened to f32 (BF16 bits << 16, F16
 * converted, as the reference widens its norm weights).  NULL on error. */
const void *anima_hip_weights_device(anima_hip_weights *w, const char *name, int as_f32);

/* dtype codes of weight tables (the codes above). */
#define ANIMA_HIP_DTYPE_F32 0
#define ANIMA_HIP_DTYPE_F16 1
#define ANIMA_HIP_DTYPE_BF16 2

/* ---- The whole DiT on the device (NumpyDiT, anima_rt/scripts/numpy_dit.py:67-130)
 * Shapes of the model; anima_hip_dit_default_config fills the Anima 2B values
 * (2048 wide, 28 blocks, 16 heads x 128, MLP 8192, text context 1024 wide,
 * 16 latent channels in and out, CFG batch 2).  The patch is 2 x 2 pixels of
 * one frame and the AdaLN hidden width 256, as in the reference. */
typedef struct anima_hip_dit_config {
    int dim;           /* model width D */
    int blocks;        /* DiT blocks */
    int heads;         /* attention heads */
    int head_dim;      /* per-head width */
    int mlp_hidden;    /* MLP hidden width */
    int ctx_dim;       /* text-context width */
    int in_channels;   /* latent channels (a zero padding-mask channel is appended) */
    int out_channels;  /* output channels */
    int max_batch;     /* largest forward batch, 1..4 (the CFG pair needs 2) */
} anima_hip_dit_config;

typedef struct anima_hip_dit anima_hip_dit;

void anima_hip_dit_default_config(anima_hip_dit_config *cfg);

/* A model over device-resident weights given as a table of n (name, device
 * pointer, dtype code, shape) entries; shapes holds two int64 per entry,
 * [out, in] for a matrix and [len, 0] for a vector, and every tensor is
 * checked against the configuration.  Names are the reference's checkpoint's, with or
 * without its "net." prefix (blocks.{i}.self_attn.q_proj.weight, ...,
 * x_embedder.proj.1.weight, t_embedder.1.linear_{1,2}.weight,
 * t_embedding_norm.weight, final_layer.adaln_modulation.{1,2}.weight,
 * final_layer.linear.weight).  Linear weights must be BF16 bit patterns
 * [out, in]; norm weights F32 or BF16 (widened like the reference).  The
 * pointers are borrowed and must stay valid for the model's life (the weight
 * store's anima_hip_weights_device copies do).  mode: ANIMA_HIP_F32 (f32
 * activations, exact hi+lo bf16 GEMM terms, f32 attention), ANIMA_HIP_F32X3
 * (the same with attention on bf16 term pairs; head_dim 128) or
 * ANIMA_HIP_BF16 (bf16 activations and attention inputs; head_dim 128).
 * NULL on error. */
anima_hip_dit *anima_hip_dit_create(const anima_hip_dit_config *cfg, const char *const *names,
                                    const void *const *ptrs, const int *dtypes,
                                    const int64_t *shapes, int n, int mode);
void anima_hip_dit_destroy(anima_hip_dit *dit);

/* Text context ctx [Bc, S_kv, ctx_dim] f32 on the device: every block's
 * cross-attention K = k_norm(ctx Wk^T) and V = ctx Wv^T are computed once here
 * and reused by every later forward (the reference recomputes them per call).
 * Bc = 1 serves every batch entry; the sampler needs Bc = 2 in the order
 * [unconditional, conditional] (sampling.py:127).  Allocates the caches. */
bool anima_hip_dit_set_context_dev(anima_hip_dit *dit, const float *ctx, int Bc, int S_kv,
                                   void *stream);

/* Device scratch of one forward on a [B, C, T, H, W] latent (bytes); query it
 * after the context is set. */
size_t anima_hip_dit_scratch_bytes(const anima_hip_dit *dit, int B, int T, int H, int W);

/* NumpyDiT.forward (numpy_dit.py:82-130) on device memory: x [B, C, T, H, W]
 * f32 with batch stride x_batch_stride elements (0: every batch entry reads
 * entry 0), sigma: B noise levels (host), freqs: the RoPE table [T*Hp*Wp, 64,
 * 2, 2] of the patch grid (Hp = ceil(H/2), Wp = ceil(W/2); the reference's
 * _generate_rope_freqs(Hp, Wp, T, head_dim)), out [B, out_channels, T, H, W].
 * Uses the context set last.  Nothing is allocated; asynchronous on stream;
 * calls on one model are not concurrent (they share its modulation vectors). */
bool anima_hip_dit_forward_dev(anima_hip_dit *dit, const float *x, int64_t x_batch_stride,
                               const float *sigma, int B, int T, int H, int W, const float *freqs,
                               float *out, void *scratch, size_t scratch_bytes, void *stream);

/* EulerSampler.sample (sampling.py:115-140) on the device: `steps` Euler
 * steps of the latent [C, H, W] (one frame, updated in place) over host
 * sigmas[steps + 1], each a B = 2 forward of the latent against the context
 * [unconditional, conditional] followed by v = v_u + cfg (v_c - v_u),
 * x += v (sigma_next - sigma).  scratch: anima_hip_dit_scratch_bytes(dit, 2,
 * 1, H, W).  Asynchronous on stream. */
bool anima_hip_dit_euler_dev(anima_hip_dit *dit, float *latent, const float *sigmas, int steps,
                             float cfg, int H, int W, const float *freqs, void *scratch,
                             size_t scratch_bytes, void *stream);

/* Timing hook: device time of the last completed host-pointer call (the
 * anima_rt_run_* drop-ins, anima_hip_sdpa, anima_hip_attention,
 * anima_hip_cross_attention), from HIP events on the library's streams:
 * kernel_ms between the end of its uploads and the start of its last
 * group's downloads (for a large call run as overlapped head or batch
 * groups, the kernel time that no copy hid), total_ms from the first upload
 * to the end of the last download (PCIe included).  Either pointer may be
 * NULL.  False before any such call. */
bool anima_hip_last_call_ms(float *kernel_ms, float *total_ms);

/* ---- Device memory for hosts without another HIP binding ---- */
void *anima_hip_malloc(size_t bytes);              /* NULL on error */
void anima_hip_free(void *p);
/* Synchronous copy; kind: 1 host->device, 2 device->host, 3 device->device. */
bool anima_hip_memcpy(void *dst, const void *src, size_t bytes, int kind);
bool anima_hip_synchronize(void);

#ifdef __cplusplus
}
#endif

#endif /* ANIMA_HIP_H */
