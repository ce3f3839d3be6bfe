// One attention sub-block of a DiT block on the device-resident residual
// stream, NumpyBlock.forward (anima_rt/scripts/numpy_dit.py:236-247):
//   x_n = layernorm(x)                       (anima_rt_run_layernorm, eps 1e-6)
//   x_m = x_n * (1 + scale[b]) + shift[b]    (AdaLN modulation)
//   a   = NumpyAttention(x_m [, ctx])        (projections, q/k RMSNorm, RoPE, SDPA)
//   x   = x + gate[b] * output_proj(a)
// with (shift, scale, gate) the three chunks of the block's AdaLN output
// (numpy_dit.py:218-228).  x stays in HBM across calls: the host sees
// nothing between the blocks of a denoise step.
//
// Kernels here:
//   ln_modulate_kernel  one wave per row: mean and variance by wave
//                       reductions (two passes over registers), then the
//                       modulated row written directly as the bf16 terms
//                       (hi, and lo in f32 mode) that the projection GEMM
//                       consumes, so no separate split pass runs;
//   gate_residual_kernel x += gate[b] * y, float4 per thread.
// The LayerNorm statistics are summed in a different order than the
// reference's serial Welford pass (layernorm_kernel.h:13-33), so x_n agrees
// to float32 rounding (~1e-7 relative), not bit for bit; the products
// and sums after it round like numpy's float32 expressions.
#include "common.h"

#include <cmath>

#pragma clang fp contract(off)

namespace anima_hip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

size_t round_up256(size_t n) { return (n + 255) / 256 * 256; }

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ unsigned int pack_pair(float x, float y)
{
    return __builtin_bit_cast(unsigned int, __builtin_convertvector(f32x2{x, y}, bf16x2));
}

struct LnArgs {
    const float *x;
    int64_t ldx;
    const float *mod;  // per batch entry b at mod + b*mod_ld: shift [Dm], scale [Dm], ...
    int64_t mod_ld;
    // Pending residual of the previous sub-layer, or null: before the norm,
    // x += gate[b] * y (gate at res_gate + b*res_ld), written back to x; y
    // is the sum of res_parts planes [M][Dm] res_plane floats apart, added
    // in plane order (a split-K GEMM's partials).
    const float *res_y;
    int res_parts;
    int64_t res_plane;
    const float *res_gate;
    int64_t res_ld;
    float *xw;  // x itself, writable (set with res_y)
    unsigned int *hi, *lo;  // [M][kp] bf16 (addressed as pairs); lo may be null
    float *yf;              // or, when set, the modulated rows as f32 [M][ldy]
    int64_t ldy;
    int64_t kp;
    int64_t tld;  // term row stride (elements): kp, or 2*kp for [hi | lo] rows
    int64_t M;
    int S, Dm;
    float eps;
};

// Row r of batch entry r / S, spread over WPR waves of the 4-wave block (4 /
// WPR rows per block): wave w takes the float4 columns c = 64 (w % WPR) +
// lane + 64 WPR i, i < VPL, so VPL float4 per lane cover Dm <= 256 WPR VPL.  Every load of the row (x, the
// pending residual's planes, the gate) is issued before the first store.
template <int VPL, int WPR>
__global__ __launch_bounds__(256) void ln_modulate_kernel(LnArgs a)
{
    constexpr int RPB = 4 / WPR;  // rows per block
    __shared__ float part[2][4];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int seg = wave % WPR;
    const int64_t row = int64_t(blockIdx.x) * RPB + wave / WPR;
    const bool live = row < a.M;  // uniform per row group (the barriers need every wave)
    const int64_t r = live ? row : 0;
    const int b = int(r / a.S);
    const float *x = a.x + r * a.ldx;
    const int n4 = a.Dm >> 2;
    f32x4 v[VPL];
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int c = 64 * seg + lane + 64 * WPR * i;
        v[i] = c < n4 && live ? *reinterpret_cast<const f32x4 *>(x + 4 * c)
                              : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if (a.res_y && live) {
        const float *yr = a.res_y + r * a.Dm;
        const float *gr = a.res_gate + b * a.res_ld;
        f32x4 y[VPL], g[VPL];
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int c = 64 * seg + lane + 64 * WPR * i;
            if (c < n4) {
                y[i] = *reinterpret_cast<const f32x4 *>(yr + 4 * c);
                g[i] = *reinterpret_cast<const f32x4 *>(gr + 4 * c);
            }
        }
        for (int p = 1; p < a.res_parts; ++p) {
#pragma unroll
            for (int i = 0; i < VPL; ++i) {
                const int c = 64 * seg + lane + 64 * WPR * i;
                if (c < n4)
                    y[i] += *reinterpret_cast<const f32x4 *>(yr + p * a.res_plane + 4 * c);
            }
        }
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int c = 64 * seg + lane + 64 * WPR * i;
            if (c < n4) {
                v[i] = v[i] + g[i] * y[i];
                *reinterpret_cast<f32x4 *>(a.xw + r * a.ldx + 4 * c) = v[i];
            }
        }
    }
#pragma unroll
    for (int i = 0; i < VPL; ++i)
        sum += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    // Row sums: the wave's, then the row's waves in order through LDS.
    auto row_sum = [&](float s, int k) {
        s = wave_sum(s);
        if (WPR == 1)
            return s;
        if (lane == 0)
            part[k][wave] = s;
        __syncthreads();
        const int w0 = wave - seg;
        float t = part[k][w0];
#pragma unroll
        for (int j = 1; j < WPR; ++j)
            t += part[k][w0 + j];
        return t;
    };
    const float mean = row_sum(sum, 0) / float(a.Dm);
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        if (64 * seg + lane + 64 * WPR * i < n4) {
            const f32x4 d = v[i] - mean;
            sq += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
        }
    }
    const float rstd = 1.0f / sqrtf(row_sum(sq, 1) / float(a.Dm) + a.eps);
    if (!live)
        return;
    const float *shift = a.mod + int64_t(b) * a.mod_ld;
    const float *scale = shift + a.Dm;
    if (a.yf) {
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int c = 64 * seg + lane + 64 * WPR * i;
            if (c < n4) {
                const f32x4 sc = *reinterpret_cast<const f32x4 *>(scale + 4 * c);
                const f32x4 sh = *reinterpret_cast<const f32x4 *>(shift + 4 * c);
                const f32x4 xn = (v[i] - mean) * rstd;
                *reinterpret_cast<f32x4 *>(a.yf + r * a.ldy + 4 * c) = xn * (1.0f + sc) + sh;
            }
        }
        return;
    }
    unsigned int *hrow = a.hi + r * (a.tld >> 1);
    unsigned int *lrow = a.lo ? a.lo + r * (a.tld >> 1) : nullptr;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int c = 64 * seg + lane + 64 * WPR * i;
        if (c < n4) {
            const f32x4 sc = *reinterpret_cast<const f32x4 *>(scale + 4 * c);
            const f32x4 sh = *reinterpret_cast<const f32x4 *>(shift + 4 * c);
            const f32x4 xn = (v[i] - mean) * rstd;
            const f32x4 y = xn * (1.0f + sc) + sh;
            const unsigned int h0 = pack_pair(y.x, y.y), h1 = pack_pair(y.z, y.w);
            *reinterpret_cast<uint2 *>(hrow + 2 * c) = uint2{h0, h1};
            if (lrow) {
                // y - hi is exact in f32 (hi holds the leading bits of y).
                const float r0 = y.x - __uint_as_float(h0 << 16);
                const float r1 = y.y - __uint_as_float(h0 & 0xFFFF0000u);
                const float r2 = y.z - __uint_as_float(h1 << 16);
                const float r3 = y.w - __uint_as_float(h1 & 0xFFFF0000u);
                *reinterpret_cast<uint2 *>(lrow + 2 * c) = uint2{pack_pair(r0, r1), pack_pair(r2, r3)};
            }
        }
    }
    // Dm % 8 == 4: the last four elements of the padded row are zero.
    if ((a.Dm & 7) == 4 && seg == 0 && lane == 0) {
        *reinterpret_cast<uint2 *>(hrow + 2 * n4) = uint2{0u, 0u};
        if (lrow)
            *reinterpret_cast<uint2 *>(lrow + 2 * n4) = uint2{0u, 0u};
    }
}

struct ResidualArgs {
    float *x;
    const float *y;
    const float *mod;
    int64_t n4;  // M * Dm / 4
    int S, Dm;
};

__global__ __launch_bounds__(256) void gate_residual_kernel(ResidualArgs a)
{
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= a.n4)
        return;
    const int64_t e = 4 * i;
    const int64_t row = e / a.Dm;
    const int d = int(e - row * a.Dm);
    const int b = int(row / a.S);
    const f32x4 g = *reinterpret_cast<const f32x4 *>(a.mod + (int64_t(b) * 3 + 2) * a.Dm + d);
    const f32x4 y = *reinterpret_cast<const f32x4 *>(a.y + e);
    f32x4 &x = *reinterpret_cast<f32x4 *>(a.x + e);
    x = x + g * y;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Scratch regions of one sub-block, 256-byte aligned, in order.
struct BlockScratch {
    size_t terms, q, k, v, o, y, attn, lin, total;
};

BlockScratch block_scratch(int B, int S, int Dm, int H, int D, int Bk, int S_kv, AttnMode mode,
                           bool cross)
{
    const bool bf16 = mode == kAttnBF16;
    const size_t M = size_t(B) * S, HD = size_t(H) * D;
    BlockScratch s{};
    s.terms = round_up256(M * size_t(linear_terms_ld(Dm)) * 2) * (bf16 ? 1 : 2);
    s.q = round_up256(M * HD * 4);
    s.k = cross ? 0 : s.q;
    s.v = cross ? 0 : s.q;
    s.o = s.q;
    s.y = round_up256(M * size_t(Dm) * 4);
    s.attn = round_up256(attention_scratch_bytes(B, S, Bk, S_kv, H, D, mode, cross));
    s.lin = round_up256(linear_scratch_bytes(int(M), int(HD), !bf16));
    s.total = s.terms + s.q + s.k + s.v + s.o + s.y + s.attn + s.lin;
    return s;
}

}  // namespace

size_t attention_block_scratch_bytes(int B, int S, int Dm, int H, int D, int Bk, int S_kv,
                                     AttnMode mode, bool cross)
{
    return block_scratch(B, S, Dm, H, D, Bk, S_kv, mode, cross).total;
}

bool launch_ln_modulate(const float *x, int64_t ldx, const float *mod, int64_t mod_ld,
                        uint16_t *hi, uint16_t *lo, int64_t M, int S, int Dm, float eps,
                        hipStream_t st, float *res_x, const float *res_y, const float *res_gate,
                        int64_t res_ld, int64_t tld, int res_parts, float *y_f32)
{
    if (M == 0)
        return true;
    if (Dm <= 0 || Dm % 4 || Dm > 256 * 16 || S <= 0)
        return fail("ln_modulate: the model width must be a positive multiple of 4, at most 4096");
    if (!aligned16(x) || ldx % 4 || !aligned16(mod) || mod_ld % 4 || !aligned16(hi) ||
        !aligned16(lo) || !aligned16(y_f32))
        return fail("ln_modulate: operands must be 16-byte aligned");
    if (res_y && (res_x != x || ldx != Dm || !aligned16(res_y) || !aligned16(res_gate) ||
                  res_ld % 4 || res_parts < 1))
        return fail("ln_modulate: the pending residual needs x itself, dense rows and 16-byte "
                    "alignment");
    LnArgs a;
    a.x = x;
    a.ldx = ldx;
    a.mod = mod;
    a.mod_ld = mod_ld;
    a.res_y = res_y;
    a.res_parts = res_parts;
    a.res_plane = M * Dm;
    a.res_gate = res_gate;
    a.res_ld = res_ld;
    a.xw = res_y ? res_x : nullptr;
    a.hi = reinterpret_cast<unsigned int *>(hi);
    a.lo = reinterpret_cast<unsigned int *>(lo);
    a.yf = y_f32;
    a.ldy = Dm;
    a.kp = linear_terms_ld(Dm);
    a.tld = tld > 0 ? tld : a.kp;
    if (a.tld < a.kp || a.tld % 8)
        return fail("ln_modulate: term rows must be at least the padded width, multiples of 8");
    a.M = M;
    a.S = S;
    a.Dm = Dm;
    a.eps = eps;
    // A block per row: the grid fills the chip even for a 256x256 image's
    // 512 tokens (measured as fast as a wave per row at 8192 tokens).
    constexpr int wpr = 4;
    const int64_t nblk = M;
    if (nblk > INT32_MAX)
        return fail("ln_modulate: too many rows");
    const int vpl = (Dm + 256 * wpr - 1) / (256 * wpr);
    const dim3 grid{unsigned(nblk)}, block{256};
    if (vpl <= 1)
        hipLaunchKernelGGL((ln_modulate_kernel<1, wpr>), grid, block, 0, st, a);
    else if (vpl <= 2)
        hipLaunchKernelGGL((ln_modulate_kernel<2, wpr>), grid, block, 0, st, a);
    else
        hipLaunchKernelGGL((ln_modulate_kernel<4, wpr>), grid, block, 0, st, a);
    return hip_ok(hipGetLastError(), "ln_modulate_kernel launch");
}

bool launch_gate_residual(float *x, const float *y, const float *mod, int64_t M, int S, int Dm,
                          hipStream_t st)
{
    if (M == 0)
        return true;
    if (Dm % 4 || !aligned16(x) || !aligned16(y) || !aligned16(mod))
        return fail("gate_residual: rows must be 16-byte aligned multiples of 4");
    ResidualArgs a;
    a.x = x;
    a.y = y;
    a.mod = mod;
    a.n4 = M * Dm / 4;
    a.S = S;
    a.Dm = Dm;
    const int64_t nblk = (a.n4 + 255) / 256;
    if (nblk > INT32_MAX)
        return fail("gate_residual: too many elements");
    hipLaunchKernelGGL(gate_residual_kernel, dim3(unsigned(nblk)), dim3(256), 0, st, a);
    return hip_ok(hipGetLastError(), "gate_residual_kernel launch");
}

bool run_attention_block(const BlockProblem &p, void *scratch, size_t scratch_bytes, hipStream_t st)
{
    const int B = p.B, S = p.S, Dm = p.Dm, H = p.H, D = p.D;
    const bool cross = p.k_prep != nullptr;
    const bool bf16 = p.mode == kAttnBF16;
    const int64_t M = int64_t(B) * S;
    const int HD = H * D;
    if (M == 0)
        return true;
    if (Dm % 8 || HD % 8)
        return fail("attention_block: the model width and H*D must be multiples of 8");
    if (!p.x || !p.mod || !p.wq || !p.wo || (!cross && (!p.wk || !p.wv)))
        return fail("attention_block: null pointer");
    const BlockScratch s = block_scratch(B, S, Dm, H, D, cross ? p.Bk : B, cross ? p.S_kv : S,
                                         p.mode, cross);
    if (!scratch || scratch_bytes < s.total || !aligned16(scratch))
        return fail("attention_block: scratch smaller than the size query or not 16-byte aligned");
    char *cur = static_cast<char *>(scratch);
    auto take = [&](size_t n) {
        char *r = cur;
        cur += n;
        return r;
    };
    uint16_t *hi = reinterpret_cast<uint16_t *>(take(s.terms));
    uint16_t *lo = bf16 ? nullptr : hi + (s.terms / 2) / sizeof(uint16_t);
    float *q = reinterpret_cast<float *>(take(s.q));
    float *k = reinterpret_cast<float *>(take(s.k));
    float *v = reinterpret_cast<float *>(take(s.v));
    float *o = reinterpret_cast<float *>(take(s.o));
    float *y = reinterpret_cast<float *>(take(s.y));
    void *attn = take(s.attn);
    void *lin = take(s.lin);

    // x_m as bf16 terms, then the projections of NumpyAttention.forward
    // (numpy_dit.py:273-281): q from x_m, and k/v from x_m (self) or the
    // cached context projections (cross).
    if (!launch_ln_modulate(p.x, Dm, p.mod, 3 * int64_t(Dm), hi, lo, M, S, Dm, p.eps, st))
        return false;
    if (!launch_linear_terms(hi, lo, p.wq, Dm, q, HD, int(M), HD, Dm, st))
        return false;
    if (!cross && (!launch_linear_terms(hi, lo, p.wk, Dm, k, HD, int(M), HD, Dm, st) ||
                   !launch_linear_terms(hi, lo, p.wv, Dm, v, HD, int(M), HD, Dm, st)))
        return false;

    AttnInputs in;
    in.q = q;
    in.q_norm_w = p.q_norm_w;
    in.freqs = cross ? nullptr : p.freqs;
    in.k = k;
    in.v = v;
    in.k_norm_w = p.k_norm_w;
    in.k_prep = p.k_prep;
    in.v_prep = p.v_prep;
    in.out = o;
    in.B = B;
    in.Bk = cross ? p.Bk : B;
    in.S_q = S;
    in.S_kv = cross ? p.S_kv : S;
    in.H = H;
    in.D = D;
    in.eps = p.eps;
    in.mode = p.mode;
    // With D == 128 the attention writes O straight into output_proj's bf16
    // terms, where launch_linear would split it: hi rows of
    // linear_terms_ld(HD) at lin and, in the f32 modes, the lo rows after
    // them (lo_t = the hi block's size).  Other head dims, or a shape the
    // library GEMM does not take (launch_linear's exact f32 fallback needs
    // O itself): f32 O at o.
    const bool terms_out = D == 128 && linear_terms_supported(int(M), Dm, HD, p.wo, HD, y, Dm);
    const int64_t kp = linear_terms_ld(HD);
    const size_t hi_bytes = round_up256(size_t(M) * size_t(kp) * 2);
    uint16_t *ohi = static_cast<uint16_t *>(lin);
    uint16_t *olo = bf16 ? nullptr : ohi + hi_bytes / 2;
    if (terms_out) {
        in.out = nullptr;
        in.out_t = ohi;
        in.ld_t = kp;
        in.lo_t = bf16 ? 0 : int64_t(hi_bytes / 2);
    }
    if (!run_attention(in, attn, st))
        return false;

    // output_proj (numpy_dit.py:294-296) and the gated residual.  bf16 mode:
    // one GEMM per batch entry whose per-channel scale is the gate and whose
    // C and D are the residual stream.  f32 mode (two terms, each pass would
    // read and write the residual again), or a shape the library GEMM does
    // not take with a per-channel scale: the projection into y, then a
    // residual pass.
    if (bf16 && linear_residual_supported(S, Dm, HD, p.wo, HD, p.x, Dm))
        return terms_out
                   ? launch_linear_residual_terms(ohi, p.wo, HD, p.x, Dm, p.mod + 2 * int64_t(Dm),
                                                  3 * int64_t(Dm), B, S, Dm, HD, st)
                   : launch_linear_residual(o, HD, p.wo, HD, p.x, Dm, p.mod + 2 * int64_t(Dm),
                                            3 * int64_t(Dm), B, S, Dm, HD, lin, s.lin, st);
    const size_t terms_bytes = hi_bytes * (bf16 ? 1 : 2);
    const bool ok =
        terms_out ? launch_linear_terms(ohi, olo, p.wo, HD, y, Dm, int(M), Dm, HD, st,
                                        static_cast<char *>(lin) + terms_bytes,
                                        s.lin - terms_bytes)
                  : launch_linear(o, HD, p.wo, HD, y, Dm, int(M), Dm, HD, !bf16, lin, s.lin, st);
    return ok && launch_gate_residual(p.x, y, p.mod, M, S, Dm, st);
}

}  // namespace anima_hip
