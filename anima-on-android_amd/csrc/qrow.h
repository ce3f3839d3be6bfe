// Query rows prepared inside the bf16-MFMA flash kernels (flash_x3.hip,
// flash_bf16.hip) from the raw f32 projection rows, with the row prologue's
// arithmetic (prologue.hip), so the q row pass can be skipped bit for bit.
#pragma once

#include "flash_tile.h"
#include "rowmath.h"

namespace anima_hip {
namespace flash_tile {

// Both halves of a query row at once: lo = v of lane l % 32, hi = v of lane
// 32 + l % 32 (one v_permlane32_swap).
__device__ __forceinline__ void row_halves(float v, float &lo, float &hi)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    lo = __uint_as_float(r[0]);
    hi = __uint_as_float(r[1]);
}

// The Q terms of one query row prepared from its raw f32 projection row, as
// the row prologue (prologue.hip) computes them for anima_rt's rmsnorm and
// rope kernels (anima_rt/include/cpu/rmsnorm_kernel.h:11-31,
// rope_kernel.h:65-97): y = x * inv_rms(sum x^2) [* w], then, with a table,
// for pair p
//     out[p] = c00 y[p] + c01 y[p+64],  out[p+64] = c10 y[p] + c11 y[p+64]
// (two products and one add, no contraction), split into hi = bf16(out) and
// lo = bf16(out - hi).  Lane half h owns d = 64h .. 64h+63 (the Q fragment
// layout).  The sum of squares keeps the reference's index order across the
// two halves: half 0 adds d < 64 from zero, half 1 continues from half 0's
// partial.  Every lane takes part in the exchanges; lanes whose row is not
// `valid` (past S_q) read nothing and end with zero terms.
// LO = false: the bf16 path's rows, hi terms only (ql is left untouched).
template <bool LO = true>
__device__ __forceinline__ void q_terms_from_raw(const float *xrow, const float *w,
                                                 const float *fq, float eps, bool valid,
                                                 int half, bf16x8 (&qh)[8], bf16x8 (&ql)[8])
{
#pragma clang fp contract(off)
    f32x4 x[16];
#pragma unroll
    for (int j = 0; j < 16; ++j)
        x[j] = valid ? *reinterpret_cast<const f32x4 *>(xrow + 64 * half + 4 * j)
                     : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
            ss = ss + x[j][e] * x[j][e];
    float ss0, unused;
    row_halves(ss, ss0, unused);
    float ss1 = ss0;  // half 1: half 0's partial, then its own squares in order
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
            ss1 = ss1 + x[j][e] * x[j][e];
    float total;
    row_halves(ss1, unused, total);
    const float inv = inv_rms(total, kD, eps);
    const f32x4 *wv = w ? reinterpret_cast<const f32x4 *>(w + 64 * half) : nullptr;
    const float *fh = fq ? fq + 2 * half : nullptr;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        unsigned hw[4], lw[4];
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
            unsigned short hb[2], lb[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int i = 8 * t + 2 * e2 + u;
                float y = x[i >> 2][i & 3] * inv;
                if (wv)
                    y = y * wv[i >> 2][i & 3];
                float out = y;
                if (fh) {
                    float ya, yb;
                    row_halves(y, ya, yb);
                    const float2 c = *reinterpret_cast<const float2 *>(fh + 4 * i);
                    out = c.x * ya + c.y * yb;
                }
                hb[u] = f32_to_bf16_rne(out);
                lb[u] = LO ? bf16_lo_term(out, hb[u]) : 0;
            }
            hw[e2] = valid ? unsigned(hb[0]) | (unsigned(hb[1]) << 16) : 0u;
            lw[e2] = valid ? unsigned(lb[0]) | (unsigned(lb[1]) << 16) : 0u;
        }
        qh[t] = __builtin_bit_cast(bf16x8, uint4{hw[0], hw[1], hw[2], hw[3]});
        if (LO)
            ql[t] = __builtin_bit_cast(bf16x8, uint4{lw[0], lw[1], lw[2], lw[3]});
    }
}

}  // namespace flash_tile
}  // namespace anima_hip
