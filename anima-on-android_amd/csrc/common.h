// Shared declarations of libanima_hip: launch descriptors, error reporting
// and the kernel launchers each translation unit exports to the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <string>

namespace anima_hip {

// Record an error message for anima_hip_last_error(); always returns false so
// callers can `return fail(...)`.
bool fail(const std::string &msg);
// The library's device context exists (created on first use); false with the
// reason recorded otherwise.
bool device_ready();
// Check a HIP status; on error record "<what>: <hip error string>".
bool hip_ok(hipError_t e, const char *what);

// Element strides (in elements, not bytes) of a 4-D [B, H, S, D] view whose D
// axis is contiguous.  Stride 0 on the batch axis broadcasts one batch entry
// to every batch (used for a shared text context).
struct Strides {
    int64_t b, h, s;
};

// O of the D == 128 flash kernels written as the bf16 terms a bf16-MFMA
// projection of O reads, instead of f32: hi = bf16(O) (round to nearest even)
// at t + b*tb + h*th + q*ts + d and, when lo > 0, bf16(O - hi) lo elements
// after it.  These are the values split_kernel (linear.hip) writes from the
// f32 O, so the projection needs no split pass.  t == nullptr: f32 O.
// Offsets and strides are multiples of 8 elements and t is 16-byte aligned.
struct TermOut {
    uint16_t *t = nullptr;
    int64_t tb = 0, th = 0, ts = 0, lo = 0;
};

// Query rows handed to a flash kernel unprepared: f32 x, [B, S_q, H, 128]
// rows through strides s, 16-byte aligned.  The kernel applies the per-head
// RMSNorm (optional weight w), the rotate-half RoPE of table freqs
// ([S_q, 64, 2, 2], optional) and its own operand conversion, bit-identical to
// the row prologue followed by the kernel.  x == nullptr: q is prepared.
struct RawQ {
    const float *x = nullptr;
    Strides s{0, 0, 0};
    const float *w = nullptr;
    const float *freqs = nullptr;
    float eps = 1e-6f;
};

// Everything the attention kernels need; pointers are device pointers.
struct FlashProblem {
    const void *q, *k, *v;  // f32 or bf16 (see kernel)
    float *o;               // unused when ot.t is set
    Strides qs, ks, vs, os;
    int B, H, S_q, S_kv, D;
    float scale;       // softmax scale applied to q.k
    bool causal;       // mask key j > query i (top-left aligned, like anima_rt)
    TermOut ot;        // bf16 term output in place of o
    RawQ rq;           // f32x3, f32 and bf16 kernels: q given as raw projection rows
};
bool term_out_ok(const TermOut &t);  // alignment of a set term output

// Launch shape of the D == 128 flash kernels.  A grid of B*H*ceil(S_q/256)
// workgroups of 8 waves fills the GPU when it has at least one workgroup per
// CU.  Smaller problems (short sequences, few heads) use workgroups of 4
// waves and, when the caller provides scratch, split the key range over
// `splits` workgroups per query tile ("split-KV"): split s takes key tiles
// [s*tiles, (s+1)*tiles) (64 keys each) and writes its output normalised by
// its own row sum, plus that row's (max, sum), to scratch; flash_combine
// merges the splits into O.
struct FlashPlan {
    int waves = 8;
    int splits = 1;
    int tiles = 1 << 30;  // key tiles per split
    size_t bytes = 0;     // scratch for the partials (0 when unsplit)
};
// tile_us > 0: the kernel's time per 64-key tile in a 4-wave workgroup (us);
// the key range is then split only where the tiles a workgroup no longer
// walks are worth more than a split grid's fixed cost (kSplitCostUs: every
// split loads its query tile and writes f32 partials that the combine pass
// reads back).  tile_us == 0 always splits a small grid: the scratch size
// every mode's plan fits in.
FlashPlan flash_plan(int64_t BH, int S_q, int S_kv, int D, float tile_us = 0.0f);
// Measured on MI355X at 32 heads x 256 queries (unsplit 4-wave grids over
// 4 and 8 key tiles; split grids against them, combine included).
constexpr float kSplitCostUs = 13.0f;
constexpr float kTileUsF32 = 9.1f, kTileUsBF16 = 1.3f, kTileUsX3 = 2.5f;

// What a split workgroup writes (device view).  Partials are laid out
// [splits][BH][S_q][128] f32 and (max, sum) pairs [splits][BH][S_q] float2,
// the max in log2 units of the scaled scores.
struct FlashSplitArgs {
    int n = 1;
    int tiles = 1 << 30;
    int64_t BH = 0;
    float *part = nullptr;
    float2 *ml = nullptr;
};
// Split descriptor for plan `pl` over scratch `part` (nullptr or too small:
// unsplit).
FlashSplitArgs flash_split_args(const FlashPlan &pl, int64_t BH, int S_q, void *part,
                                size_t part_bytes);
// O[b,h,q,:] = sum_s w_s P_s[bh,q,:] / sum_s w_s, w_s = l_s * 2^(m_s - max_s m_s).
bool launch_flash_combine(const FlashProblem &p, const FlashSplitArgs &sa, hipStream_t st);

// f32 inputs, f32 MFMA (D == 128) or the generic kernel (any D <= 1024).
// `part` is optional split-KV scratch of flash_plan(...).bytes.
bool launch_flash_f32(const FlashProblem &p, hipStream_t st, void *part = nullptr,
                      size_t part_bytes = 0);
// True when launch_flash_f32 would take the MFMA path for this problem.
bool flash_f32_fast_path(const FlashProblem &p);

// bf16 inputs (Q, K row-major [.., S, D]; V transposed, layout below),
// bf16 MFMA with f32 accumulation and f32 softmax; D == 128 and scale > 0.
// `v` points at the packed V^T and `vs` holds its {batch, head, d-row}
// strides (the d-row stride is vt_padded_len(S_kv)).
bool launch_flash_bf16(const FlashProblem &p, hipStream_t st, void *part = nullptr,
                       size_t part_bytes = 0);
// True when launch_flash_bf16 runs this shape as two 4-wave workgroups per CU
// (large grids over short key ranges), where the kernel also takes raw query
// rows (FlashProblem::rq) at no cost: their larger load overlaps the other
// workgroup's tiles.
bool flash_bf16_raw_q(int64_t BH, int S_q, int S_kv);

// V^T layout of the bf16 path: per (batch, head) a [D][Sp] bf16 matrix with
// Sp = vt_padded_len(S_kv), zero beyond S_kv, and within every group of 16
// keys the key with offset c stored at position vt_key_pos(c) (bits 2 and 3
// of c swapped).  With this order one 16-byte LDS read yields the 8 keys
// that pair with the P values a lane holds in its MFMA accumulators.
constexpr int kVtTile = 64;
inline int64_t vt_padded_len(int64_t S_kv) { return (S_kv + kVtTile - 1) / kVtTile * kVtTile; }
__host__ __device__ inline int vt_key_pos(int c)
{
    return (c & ~12) | ((c & 4) << 1) | ((c & 8) >> 1);
}

// Pack V (f32, [B,H,S,D] view through `vs`, D == 128) into the V^T layout
// above at `vt` with strides {batch, head} = vts.b, vts.h (d-row stride Sp).
bool launch_vt_pack(const float *v, Strides vs, uint16_t *vt, Strides vts, int B, int H,
                    int S_kv, int D, hipStream_t st);

// f32-accurate attention on bf16 MFMA (flash_x3.hip): every f32 operand x as
// two bf16 terms xh = bf16(x), xl = bf16(x - xh), every product as
// xh*yh + xh*yl + xl*yh.  q, k: rows of 2*D bf16, [hi | lo], addressed
// through qs/ks (row starts); v: packed term V^T, per (batch, head) the D hi
// rows then the D lo rows of the V^T layout above, strides {batch, head,
// d-row = vt_padded_len(S_kv)}.  D == 128, scale > 0.
bool launch_flash_x3(const FlashProblem &p, hipStream_t st, void *part = nullptr,
                     size_t part_bytes = 0);
// Pack V (f32 view as for launch_vt_pack) into the term V^T layout above.
bool launch_vt_pack_terms(const float *v, Strides vs, uint16_t *vt, Strides vts, int B, int H,
                          int S_kv, int D, hipStream_t st);

// C[M,N] = A[M,K] . W[N,K]^T with f32 A/C and bf16 (w_bf16) or f32 W, f32
// accumulation; leading dimensions in elements.
bool launch_gemm(const float *a, int64_t lda, const void *w, bool w_bf16, int64_t ldw, float *c,
                 int64_t ldc, int M, int N, int K, hipStream_t st);

// Projection GEMM C[M,N] = A[M,K] . W[N,K]^T, f32 A/C, bf16 W, on bf16 MFMA
// (linear.hip).  exact: A enters as bf16 hi + lo terms (per-element error
// <= 2^-16 |a|); otherwise A is rounded to bf16.  Scratch holds the bf16
// terms: linear_scratch_bytes(M, K, exact) bytes, 16-byte aligned.
size_t linear_scratch_bytes(int M, int K, bool exact);
bool launch_linear(const float *a, int64_t lda, const uint16_t *w, int64_t ldw, float *c,
                   int64_t ldc, int M, int N, int K, bool exact, void *scratch,
                   size_t scratch_bytes, hipStream_t st);

// A split into [hi | lo] rows of 2*linear_terms_ld(K) bf16 (the product with
// a weight whose rows are [W | W], K' = 2 * linear_terms_ld(K), is then one
// GEMM: hi.W + lo.W accumulated in f32).  Scratch: linear_scratch_bytes(M, K,
// true).  Returns the terms.
uint16_t *launch_split_interleaved(const float *a, int64_t lda, int M, int K, void *scratch,
                                   size_t scratch_bytes, hipStream_t st);

// Large-M bf16 GEMM (gemm_large.hip): C[M,N] = a0 . W^T (+ a1 . W^T) with
// bf16 terms [M][lda] and weights [N][ldw], f32 accumulation, 256 x 256 (one
// term) or 128 x 256 (two terms) tiles of C.  Epilogue kGemmOutF32: C f32
// [M][ldc]; kGemmOutBf16: C bf16 (round to nearest even); kGemmOutResidual:
// c is the f32 residual x [M][ldc], x += gate[(m / S) * gate_stride + n] * C.
// gemm_large_supported says whether the shape, alignments and grid (at least
// 256 tiles) suit it; out_bytes is the output element size.
enum GemmOut { kGemmOutF32 = 0, kGemmOutBf16 = 1, kGemmOutResidual = 2 };
bool gemm_large_supported(int M, int N, int K, int terms, int64_t lda, int64_t ldw, int64_t ldc,
                          const void *a0, const void *a1, const void *w, const void *c,
                          int out_bytes);
bool launch_gemm_large(const uint16_t *a0, const uint16_t *a1, int64_t lda, const uint16_t *w,
                       int64_t ldw, void *c, int64_t ldc, int M, int N, int K, int epilogue,
                       const float *gate, int64_t gate_stride, int S, hipStream_t st);
// The two-term product on f32 activations a [M][lda] (lda % 4 == 0): the
// kernel splits a into hi = bf16(a), lo = bf16(a - hi) itself, so C (f32) is
// bit-identical to the split pass plus launch_gemm_large with both terms.
bool gemm_large_f32a_supported(int M, int N, int K, int64_t lda, int64_t ldw, int64_t ldc,
                               const float *a, const void *w, const void *c);
bool launch_gemm_large_f32a(const float *a, int64_t lda, const uint16_t *w, int64_t ldw, float *c,
                            int64_t ldc, int M, int N, int K, hipStream_t st);
// Large-M product on f32 activations in 256 x 256 tiles (gemm_f32a.hip): a
// [M][lda] (lda % 4 == 0, K % 32 == 0) split into bf16 hi + lo terms
// (two_terms) or rounded to bf16 in registers, C f32.  With two terms C is
// bit-identical to the split pass plus launch_gemm_large on the term rows.
bool gemm_f32a_supported(int M, int N, int K, int64_t lda, int64_t ldw, int64_t ldc,
                         const float *a, const void *w, const void *c);
bool launch_gemm_f32a(const float *a, int64_t lda, const uint16_t *w, int64_t ldw, float *c,
                      int64_t ldc, int M, int N, int K, bool two_terms, hipStream_t st);

// Small-M bf16 GEMM (gemm_bf16.hip): C[M,N] = a0 . W^T (+ a1 . W^T) with bf16
// activation terms a0 (a1 null for one term) [M][lda], bf16 W [N][ldw], f32
// C [M][ldc], for M <= 1024 and K a multiple of 64 (K per term), split over K
// into a workspace of gemm_bf16_workspace_bytes() (at most 16 MiB) and
// reduced in split order.
size_t gemm_bf16_workspace_bytes(int M, int N, int K);
constexpr size_t kGemmBf16MaxWorkspace = size_t(16) << 20;
bool gemm_bf16_supported(int M, int N, int K, int64_t lda, int64_t ldw, int64_t ldc,
                         const void *a0, const void *a1, const void *w, const void *c,
                         size_t ws_bytes);
bool launch_gemm_bf16(const uint16_t *a0, const uint16_t *a1, int64_t lda, const uint16_t *w,
                      int64_t ldw, float *c, int64_t ldc, int M, int N, int K, void *ws,
                      size_t ws_bytes, hipStream_t st);
// The same product left as *parts dense [M][N] planes at `planes` (at least
// gemm_bf16_workspace_bytes(M, N, K), and M*N*4, bytes), C their sum in
// plane order: the consumer adds them (one plane when K is not split).
bool launch_gemm_bf16_planes(const uint16_t *a0, const uint16_t *a1, int64_t lda,
                             const uint16_t *w, int64_t ldw, float *planes, size_t planes_bytes,
                             int M, int N, int K, int *parts, hipStream_t st);

// The same product on A already split into bf16 terms hi (and lo, or null for
// one term), rows of linear_terms_ld(K) elements zero-padded past K.
int64_t linear_terms_ld(int K);
bool linear_terms_supported(int M, int N, int K, const void *w, int64_t ldw, const float *c,
                            int64_t ldc);
// With a workspace of gemm_bf16_workspace_bytes(M, N, K) bytes, the shapes
// small_m_path() names run on the small-M kernel instead of the library GEMM.
bool small_m_path(int M, int K, bool two_terms);
bool launch_linear_terms(const uint16_t *hi, const uint16_t *lo, const uint16_t *w, int64_t ldw,
                         float *c, int64_t ldc, int M, int N, int K, hipStream_t st,
                         void *ws = nullptr, size_t ws_bytes = 0);
// C[M,N] = hi . W^T + lo . W^T on [hi | lo] rows (row stride ld_t, K
// elements each, ld_t == linear_terms_ld(2K) on the library path) and [W | W]
// weight rows: the small-M kernel's two-term product when it applies, else
// one library product over the doubled rows (K' = 2K).
bool launch_linear_pair(const uint16_t *terms, int64_t ld_t, int K, const uint16_t *w,
                        int64_t ldw, float *c, int64_t ldc, int M, int N, hipStream_t st,
                        void *ws = nullptr, size_t ws_bytes = 0);
// launch_linear_terms (lo null, K per row) or launch_linear_pair (pair: [hi |
// lo] rows of ld_t = 2K) into *parts dense [M][N] planes at `planes`
// (planes_bytes of room), C their sum in plane order: the small-M kernel's
// split-K partials left for the consumer, else one plane from the library.
bool launch_linear_planes(const uint16_t *terms, int64_t ld_t, int K, bool pair,
                          const uint16_t *w, int64_t ldw, float *planes, size_t planes_bytes,
                          int M, int N, int *parts, hipStream_t st);

// C[M,N] = hi . W^T rounded to bf16 (C bf16, ldc % 8 == 0): one product on
// activations already rounded to bf16.
bool launch_linear_terms_bf16out(const uint16_t *hi, const uint16_t *w, int64_t ldw, uint16_t *c,
                                 int64_t ldc, int M, int N, int K, hipStream_t st);

// x[b*S + s, :] += gate[b*gate_stride + :] (.) (bf16(a[b*S + s, :]) . W^T) for
// b < B: the output projection fused with the gated residual of a DiT block
// (the gate scales the N output channels).  Activations round to bf16 (the hi
// term of launch_linear; scratch: linear_scratch_bytes(B*S, K, false));
// linear_residual_supported says whether the library GEMM takes this shape
// with a per-channel scale.
bool linear_residual_supported(int S, int N, int K, const void *w, int64_t ldw, const float *x,
                               int64_t ldx);
bool launch_linear_residual(const float *a, int64_t lda, const uint16_t *w, int64_t ldw, float *x,
                            int64_t ldx, const float *gate, int64_t gate_stride, int B, int S, int N,
                            int K, void *scratch, size_t scratch_bytes, hipStream_t st);
// The same on activations already rounded to bf16: rows of linear_terms_ld(K).
bool launch_linear_residual_terms(const uint16_t *hi, const uint16_t *w, int64_t ldw, float *x,
                                  int64_t ldx, const float *gate, int64_t gate_stride, int B,
                                  int S, int N, int K, hipStream_t st);

// Per-row RMSNorm (+ optional RoPE) "prologue".
//   x:   rows indexed (b, s, h) through `xs` (D contiguous), f32
//   out: same indexing through `os`, f32 or bf16 (out_bf16)
//   w:   [D] weight or nullptr; freqs: [S, D/2, 2, 2] rotate-half table or nullptr
// Arithmetic follows the reference's serial order exactly (see prologue.hip).
struct RowProblem {
    const float *x;
    void *out;
    const float *w;
    const float *freqs;
    Strides xs, os;
    int B, S, H, D;
    float eps;
    bool norm;      // apply RMSNorm
    bool out_bf16;  // write bf16 (round to nearest even) instead of f32
    // With out_bf16: 0, or the element offset from each output row to a
    // second row receiving the lo terms bf16(y - bf16(y)).
    int64_t lo_off = 0;
};
bool launch_rows(const RowProblem &p, hipStream_t st);
// Both problems in one launch when both take the D == 128 float4 kernel, else
// two launches.
bool launch_rows_pair(const RowProblem &p1, const RowProblem &p2, hipStream_t st);

// ---- Composite attention core (attention.hip) ----
// Arithmetic of the attention kernels; the values of the public
// ANIMA_HIP_F32 / ANIMA_HIP_BF16 / ANIMA_HIP_F32X3.
enum AttnMode : int { kAttnF32 = 0, kAttnBF16 = 1, kAttnF32X3 = 2 };
// Prepared K/V layouts: f32 mode K and V f32 [Bk, S_kv, H, D]; bf16 mode K
// bf16 [Bk, S_kv, H, D] and V packed bf16 V^T [Bk, H, D, vt_padded_len(S_kv)];
// f32x3 mode K term rows [Bk, S_kv, H, 2D] ([hi | lo]) and V packed term V^T
// [Bk, H, 2D, vt_padded_len(S_kv)].
struct AttnInputs {
    const float *q = nullptr;         // [B, S_q, H, D] f32 projections
    const float *q_norm_w = nullptr;  // [D] or null
    const float *freqs = nullptr;     // [S_q, D/2, 2, 2] or null (self-attention)
    const float *k = nullptr;         // raw [Bk, S_kv, H, D] f32 (when not prepared)
    const float *v = nullptr;
    const float *k_norm_w = nullptr;
    const void *k_prep = nullptr;     // prepared K/V (context cache), or null
    const void *v_prep = nullptr;
    // Prepared Q rows in the mode's layout (with k_prep / v_prep): the
    // attention runs the flash kernel alone.
    const void *q_prep = nullptr;
    float *out = nullptr;             // [B, S_q, H, D] f32
    // Or O as bf16 projection terms (D == 128): token rows ld_t elements
    // apart, hi at column h*D + d, lo (when lo_t > 0) lo_t elements after it.
    uint16_t *out_t = nullptr;
    int64_t ld_t = 0, lo_t = 0;
    int B = 0, Bk = 0, S_q = 0, S_kv = 0, H = 0, D = 0;
    float eps = 1e-6f;
    AttnMode mode = kAttnF32;
    // Token-row strides (elements) of q and of the raw k/v: 0 means H*D
    // (dense); wider when they are column blocks of one fused projection.
    int64_t ld_q = 0, ld_kv = 0;
};
// A self-attention's three operands in one launch (prologue.hip): q and k
// [B, S, H, 128] f32 with token rows ld elements apart and batch entries
// S * ld apart, RMSNorm with w[0] / w[1] (null: weight 1) and RoPE with
// freqs (or null), written dense to qo / ko as f32 rows (kAttnF32), bf16
// rows (kAttnBF16) or [hi | lo] term rows (kAttnF32X3); in the last two
// modes v is also packed into vt as the flash kernel's V^T (contiguous
// [B][H][D or 2D][vt_padded_len(S)]).  Bit-identical to launch_rows +
// launch_vt_pack(_terms) on the same inputs.
struct PrepProblem {
    const float *q = nullptr, *k = nullptr, *v = nullptr;
    const float *w[2] = {nullptr, nullptr};
    const float *freqs = nullptr;
    void *qo = nullptr, *ko = nullptr;
    uint16_t *vt = nullptr;
    int64_t ld = 0;
    int B = 0, S = 0, H = 0, D = 0;
    float eps = 1e-6f;
    AttnMode mode = kAttnF32;
};
bool prep_qkv_supported(const PrepProblem &p);  // D == 128, 16-byte alignment
bool launch_prep_qkv(const PrepProblem &p, hipStream_t st);
// A self-attention's fused q/k/v projection with that one-launch prologue as
// its epilogue (gemm_f32a.hip): a [B*S][lda] f32 activations times the
// stacked bf16 weights w [3*H*128][ldw] (q rows, then k, then v), in the f32
// modes' exact two-term product.  Instead of the product's f32 columns the
// kernel writes the attention operands: qo / ko as launch_prep_qkv writes
// them (RMSNorm with w[0] / w[1], RoPE with freqs), and vo as the x3
// kernel's term V^T (kAttnF32X3) or dense f32 V rows [B, S, H, 128]
// (kAttnF32).  Bit-identical to launch_gemm_f32a (two terms) into [M][3HD]
// followed by launch_prep_qkv on its column blocks.  S % 64 == 0 (no V^T
// padding), H even (a 256-column tile holds two whole heads of one operand),
// and the f32a grid conditions.
struct QkvPrep {
    void *qo = nullptr, *ko = nullptr, *vo = nullptr;
    const float *w[2] = {nullptr, nullptr};
    const float *freqs = nullptr;
    int B = 0, S = 0, H = 0;
    float eps = 1e-6f;
    AttnMode mode = kAttnF32X3;
};
bool gemm_f32a_qkv_supported(const float *a, int64_t lda, const void *w, int64_t ldw, int K,
                             const QkvPrep &p);
bool launch_gemm_f32a_qkv(const float *a, int64_t lda, const uint16_t *w, int64_t ldw, int K,
                          const QkvPrep &p, hipStream_t st);
size_t prepared_k_bytes(int Bk, int S_kv, int H, int D, AttnMode mode);
size_t prepared_v_bytes(int Bk, int S_kv, int H, int D, AttnMode mode);
size_t attention_scratch_bytes(int B, int S_q, int Bk, int S_kv, int H, int D, AttnMode mode,
                               bool kv_prepared);
bool prepare_kv(const float *k, const float *v, const float *k_norm_w, const float *freqs,
                void *k_out, void *v_out, int Bk, int S_kv, int H, int D, float eps,
                AttnMode mode, hipStream_t st);
bool run_attention(const AttnInputs &in, void *scratch, hipStream_t st);

// ---- Attention sub-block of a DiT block on the resident residual stream
// (block.hip): x += gate[b] * output_proj(attention(LN(x)*(1+scale[b]) +
// shift[b])).  mod is [B][3][Dm] = (shift, scale, gate).  Self-attention when
// k_prep is null (q/k/v projections of the modulated x, RoPE with freqs);
// cross-attention over a prepared context cache otherwise (wk/wv unused).
struct BlockProblem {
    float *x = nullptr;         // [B*S, Dm] f32, updated in place
    const float *mod = nullptr;
    const uint16_t *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr;  // bf16 [out, in]
    const float *q_norm_w = nullptr, *k_norm_w = nullptr, *freqs = nullptr;
    const void *k_prep = nullptr, *v_prep = nullptr;  // context cache (cross-attention)
    int Bk = 0, S_kv = 0;
    int B = 0, S = 0, Dm = 0, H = 0, D = 0;
    float eps = 1e-6f;
    // Attention arithmetic; the projections take exact hi + lo bf16 terms of
    // their f32 activations unless the mode is bf16 (activations rounded).
    AttnMode mode = kAttnF32;
};
size_t attention_block_scratch_bytes(int B, int S, int Dm, int H, int D, int Bk, int S_kv,
                                     AttnMode mode, bool cross);
bool run_attention_block(const BlockProblem &p, void *scratch, size_t scratch_bytes, hipStream_t st);
// LayerNorm (no affine) + AdaLN modulation of rows of x, written as the bf16
// terms (hi, and lo unless null) of the projection GEMM's input.  Row r
// belongs to batch entry r / S, whose shift and scale are mod[b*mod_ld + :Dm]
// and mod[b*mod_ld + Dm : 2*Dm].
// res_y != null: first x += gate[b] * y (gate at res_gate + b*res_ld; y the
// sum of res_parts dense [M][Dm] planes at res_y, in plane order), written
// back to x (res_x must be x).  tld: term row stride in elements (0:
// linear_terms_ld(Dm)); [hi | lo] rows in one buffer use tld = 2 *
// linear_terms_ld(Dm) and lo = hi + linear_terms_ld(Dm).
// y_f32 != null: the modulated rows are written there as dense f32 [M][Dm]
// instead (hi and lo unused), the input of the f32-activation GEMMs.
bool launch_ln_modulate(const float *x, int64_t ldx, const float *mod, int64_t mod_ld,
                        uint16_t *hi, uint16_t *lo, int64_t M, int S, int Dm, float eps,
                        hipStream_t st, float *res_x = nullptr, const float *res_y = nullptr,
                        const float *res_gate = nullptr, int64_t res_ld = 0, int64_t tld = 0,
                        int res_parts = 1, float *y_f32 = nullptr);
// x += gate[b] * y for rows of S per batch entry.
bool launch_gate_residual(float *x, const float *y, const float *mod, int64_t M, int S, int Dm,
                          hipStream_t st);

// ---- Element-wise and row operators (ops.hip), device pointers ----
// GELU (exact erf form), SiLU, LayerNorm without affine over rows of D,
// softmax over rows of D, and C[i][j] += bias[j] for an M x N matrix.
bool launch_gelu(const float *x, float *y, int64_t n, hipStream_t st);
bool launch_silu(const float *x, float *y, int64_t n, hipStream_t st);
bool launch_layernorm_rows(const float *x, float *y, int64_t M, int D, float eps, hipStream_t st);
bool launch_softmax_rows(const float *x, float *y, int64_t M, int D, hipStream_t st);
bool launch_bias_add(float *c, const float *bias, int64_t M, int N, hipStream_t st);

}  // namespace anima_hip
