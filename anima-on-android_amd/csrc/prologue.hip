// Row kernels: per-head RMSNorm, rotate-half RoPE, and the fused
// "norm + RoPE + relayout (+ bf16 cast)" prologue that feeds attention.
//
// Replaces, bit for bit on f32 output:
//   * anima_rt_run_rmsnorm (anima_rt/src/anima_rt.cpp:45-50) ->
//     rmsnorm_kernel (anima_rt/include/cpu/rmsnorm_kernel.h:11-31):
//       y = x * (1 / sqrt(sum(x*x) / D + eps)) [* w], serial fp32 sum;
//   * anima_rt_run_rope (anima_rt.cpp:160-164) -> rope_kernel
//     (anima_rt/include/cpu/rope_kernel.h:65-97) and NumpyDiT's _numpy_rope
//     (anima_rt/scripts/numpy_dit.py:33-37): pairs (p, p + D/2),
//       out[p]       = f00*y[p] + f01*y[p+D/2]
//       out[p + D/2] = f10*y[p] + f11*y[p+D/2]   (two products, one add);
//   * the RMSNorm -> RoPE -> transpose sequence of NumpyAttention.forward
//     (numpy_dit.py:285-291) in one pass over HBM.
// Output as f32, as bf16, or as two bf16 terms hi = bf16(y), lo = bf16(y - hi)
// (rows lo_off elements apart) for the f32-accurate bf16-MFMA attention.
//
// Bit-exactness: one thread owns each row's sum of squares and adds the
// squares in index order; floating-point contraction is switched off for this
// file (HIP's default -ffp-contract=fast would fuse x*x + s, and the header's
// round-to-nearest helpers are plain operators), and the f32 division and
// sqrt are rounded correctly by evaluating them in f64 and rounding once.
// Rows are staged through LDS so global loads and stores stay coalesced.
#include "common.h"
#include "rowmath.h"

#pragma clang fp contract(off)

namespace anima_hip {
namespace {

struct RowArgs {
    const float *x;
    void *out;
    const float *w;
    const float *freqs;
    int64_t xb, xh, xs, ob, oh, os;
    int64_t rows;      // B*S*H
    int64_t lo_off;    // bf16 output: offset of the lo-term row, or 0
    int S, H, D, rows_per_block;
    float eps;
    int norm, out_bf16;
};

// Four consecutive outputs as bf16 hi terms at ob and, when lo_off != 0, lo
// terms at ob + lo_off.
__device__ __forceinline__ void store_bf16x4(unsigned short *ob, int64_t lo_off, float v0,
                                             float v1, float v2, float v3)
{
    const unsigned short h0 = f32_to_bf16_rne(v0), h1 = f32_to_bf16_rne(v1),
                         h2 = f32_to_bf16_rne(v2), h3 = f32_to_bf16_rne(v3);
    *reinterpret_cast<uint2 *>(ob) = uint2{h0 | (unsigned(h1) << 16), h2 | (unsigned(h3) << 16)};
    if (lo_off)
        *reinterpret_cast<uint2 *>(ob + lo_off) =
            uint2{bf16_lo_term(v0, h0) | (unsigned(bf16_lo_term(v1, h1)) << 16),
                  bf16_lo_term(v2, h2) | (unsigned(bf16_lo_term(v3, h3)) << 16)};
}

// Row r (linear over (b, s, h) in that order) -> element offsets.
__device__ __forceinline__ void row_coords(const RowArgs &a, int64_t r, int64_t &xoff,
                                           int64_t &ooff, int &s)
{
    const int h = int(r % a.H);
    const int64_t bs = r / a.H;
    s = int(bs % a.S);
    const int64_t b = bs / a.S;
    xoff = b * a.xb + int64_t(h) * a.xh + int64_t(s) * a.xs;
    ooff = b * a.ob + int64_t(h) * a.oh + int64_t(s) * a.os;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Output element (row, d) from the staged row: y = x * inv [* w], then the
// rotate-half rotation when a table is given.  Contraction is off in this
// file, so every product and sum rounds like the reference's fp32 code.
__device__ __forceinline__ float norm_elem(const RowArgs &a, const float *row, float inv, int d)
{
    if (!a.norm)
        return row[d];
    float v = row[d] * inv;
    if (a.w)
        v = v * a.w[d];
    return v;
}

__device__ __forceinline__ float out_elem(const RowArgs &a, const float *row, float inv, int s,
                                          int d)
{
    if (!a.freqs)
        return norm_elem(a, row, inv, d);
    const int half = a.D >> 1;
    const bool lower = d < half;
    const int p = lower ? d : d - half;
    const float ya = norm_elem(a, row, inv, p);
    const float yb = norm_elem(a, row, inv, p + half);
    const float *fq = a.freqs + int64_t(s) * a.D * 2 + 4 * p + (lower ? 0 : 2);
    return fq[0] * ya + fq[1] * yb;
}

// Any D: rows staged in LDS with an odd pitch, per-row offsets computed once.
__global__ __launch_bounds__(256) void rows_kernel(RowArgs a)
{
    extern __shared__ float lds[];
    const int D = a.D;
    const int pitch = D + 1;  // odd pitch: serial per-row reads are conflict-free
    const int RB = a.rows_per_block;
    const int nwords = RB * pitch + 2 * RB;
    float *xs = lds;                                  // [RB][pitch]
    float *inv = lds + RB * pitch;                    // [RB]
    int *spos = reinterpret_cast<int *>(inv + RB);    // [RB]
    int64_t *offs = reinterpret_cast<int64_t *>(lds + nwords + (nwords & 1));  // [RB][2]
    const int64_t r0 = int64_t(blockIdx.x) * RB;
    const int nrows = int(min<int64_t>(RB, a.rows - r0));
    const int n = nrows * D;

    for (int rr = threadIdx.x; rr < nrows; rr += blockDim.x) {
        int64_t xo, oo;
        int s;
        row_coords(a, r0 + rr, xo, oo, s);
        offs[2 * rr] = xo;
        offs[2 * rr + 1] = oo;
        spos[rr] = s;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        const int rr = e / D, d = e - rr * D;
        xs[rr * pitch + d] = a.x[offs[2 * rr] + d];
    }
    __syncthreads();
    for (int rr = threadIdx.x; rr < nrows; rr += blockDim.x) {
        float f = 1.0f;
        if (a.norm) {
            const float *row = xs + rr * pitch;
            float ss = 0.0f;
            for (int d = 0; d < D; ++d)
                ss = ss + row[d] * row[d];
            f = inv_rms(ss, D, a.eps);
        }
        inv[rr] = f;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        const int rr = e / D, d = e - rr * D;
        const float v = out_elem(a, xs + rr * pitch, inv[rr], spos[rr], d);
        const int64_t oo = offs[2 * rr + 1] + d;
        if (a.out_bf16) {
            unsigned short *ob = static_cast<unsigned short *>(a.out);
            const unsigned short hi = f32_to_bf16_rne(v);
            ob[oo] = hi;
            if (a.lo_off)
                ob[oo + a.lo_off] = bf16_lo_term(v, hi);
        } else
            static_cast<float *>(a.out)[oo] = v;
    }
}

// D = 128 with 16-byte aligned rows: 32 rows per block (more blocks in
// flight per CU than with 64: 26.7 against 28.4 us for 128 Ki rows), float4
// traffic.
// LDS pitch 132 floats keeps float4 accesses aligned and makes the per-row
// float4 reads of the serial sum (lanes 528 bytes apart) bank-conflict free.
constexpr int kRows128 = 32;
constexpr int kPitch128 = 132;

// Rows [kRows128 * blk, kRows128 * (blk + 1)) of problem a.
__device__ __forceinline__ void rows_d128_block(const RowArgs &a, int64_t blk)
{
    __shared__ __attribute__((aligned(16))) float xs[kRows128 * kPitch128];
    __shared__ float inv[kRows128];
    __shared__ int spos[kRows128];
    __shared__ int64_t xoff[kRows128], ooff[kRows128];
    const int t = threadIdx.x;
    const int64_t r0 = blk * kRows128;
    const int nrows = int(min<int64_t>(kRows128, a.rows - r0));

    if (t < nrows) {
        int64_t xo, oo;
        int s;
        row_coords(a, r0 + t, xo, oo, s);
        xoff[t] = xo;
        ooff[t] = oo;
        spos[t] = s;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kRows128 / 8; ++i) {
        const int f = t + 256 * i;
        const int rr = f >> 5, c4 = f & 31;
        if (rr < nrows)
            *reinterpret_cast<f32x4 *>(&xs[rr * kPitch128 + 4 * c4]) =
                *reinterpret_cast<const f32x4 *>(a.x + xoff[rr] + 4 * c4);
    }
    __syncthreads();
    if (t < nrows) {
        float f = 1.0f;
        if (a.norm) {
            float ss = 0.0f;
            const float *row = xs + t * kPitch128;
#pragma unroll 8
            for (int j = 0; j < 32; ++j) {
                const f32x4 v = *reinterpret_cast<const f32x4 *>(row + 4 * j);
                ss = ss + v.x * v.x;
                ss = ss + v.y * v.y;
                ss = ss + v.z * v.z;
                ss = ss + v.w * v.w;
            }
            f = inv_rms(ss, 128, a.eps);
        }
        inv[t] = f;
    }
    __syncthreads();
    // Each thread owns the four rotation pairs (p, p+64), p = p0..p0+3, of
    // one row per iteration: the weights come once into registers, a row
    // needs one float4 of the RoPE table per pair, and both halves are
    // written as float4 (or 4 x bf16).
    const int p0 = 4 * (t & 15);
    f32x4 wl = f32x4{1.f, 1.f, 1.f, 1.f}, wh = wl;
    if (a.norm && a.w) {
        wl = *reinterpret_cast<const f32x4 *>(a.w + p0);
        wh = *reinterpret_cast<const f32x4 *>(a.w + 64 + p0);
    }
#pragma unroll
    for (int i = 0; i < kRows128 / 16; ++i) {
        const int rr = (t >> 4) + 16 * i;
        if (rr >= nrows)
            continue;
        const float *row = xs + rr * kPitch128;
        const float fi = inv[rr];
        f32x4 ya = *reinterpret_cast<const f32x4 *>(row + p0);
        f32x4 yb = *reinterpret_cast<const f32x4 *>(row + 64 + p0);
        if (a.norm) {
            ya = ya * fi;
            yb = yb * fi;
            if (a.w) {
                ya = ya * wl;
                yb = yb * wh;
            }
        }
        f32x4 lo = ya, hi = yb;
        if (a.freqs) {
            const f32x4 *fq = reinterpret_cast<const f32x4 *>(a.freqs + int64_t(spos[rr]) * 256 + 4 * p0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const f32x4 r = fq[e];  // [c00, c01, c10, c11] of pair p0 + e
                lo[e] = r.x * ya[e] + r.y * yb[e];
                hi[e] = r.z * ya[e] + r.w * yb[e];
            }
        }
        const int64_t oo = ooff[rr] + p0;
        if (a.out_bf16) {
            unsigned short *ob = static_cast<unsigned short *>(a.out) + oo;
            store_bf16x4(ob, a.lo_off, lo[0], lo[1], lo[2], lo[3]);
            store_bf16x4(ob + 64, a.lo_off, hi[0], hi[1], hi[2], hi[3]);
        } else {
            float *of = static_cast<float *>(a.out) + oo;
            *reinterpret_cast<f32x4 *>(of) = lo;
            *reinterpret_cast<f32x4 *>(of + 64) = hi;
        }
    }
}

__global__ __launch_bounds__(256) void rows_d128(RowArgs a) { rows_d128_block(a, blockIdx.x); }

// Two row problems in one launch: blocks [0, nblk_a) take a, the rest b.
__global__ __launch_bounds__(256) void rows_d128_pair(RowArgs a, RowArgs b, int64_t nblk_a)
{
    if (int64_t(blockIdx.x) < nblk_a)
        rows_d128_block(a, blockIdx.x);
    else
        rows_d128_block(b, int64_t(blockIdx.x) - nblk_a);
}

RowArgs row_args(const RowProblem &p)
{
    RowArgs a;
    a.x = p.x;
    a.out = p.out;
    a.w = p.w;
    a.freqs = p.freqs;
    a.xb = p.xs.b; a.xh = p.xs.h; a.xs = p.xs.s;
    a.ob = p.os.b; a.oh = p.os.h; a.os = p.os.s;
    a.rows = int64_t(p.B) * p.S * p.H;
    a.lo_off = p.out_bf16 ? p.lo_off : 0;
    a.S = p.S;
    a.H = p.H;
    a.D = p.D;
    a.eps = p.eps;
    a.norm = p.norm ? 1 : 0;
    a.out_bf16 = p.out_bf16 ? 1 : 0;
    a.rows_per_block = kRows128;
    return a;
}

// D = 128 with 16-byte aligned rows and operands: the float4 kernel.
bool d128_eligible(const RowProblem &p)
{
    const auto al = [](const void *ptr, unsigned m) {
        return (reinterpret_cast<uintptr_t>(ptr) & (m - 1)) == 0;
    };
    const auto st4 = [](const Strides &x) { return x.b % 4 == 0 && x.h % 4 == 0 && x.s % 4 == 0; };
    return p.D == 128 && al(p.x, 16) && al(p.out, p.out_bf16 ? 8 : 16) && st4(p.xs) &&
           st4(p.os) && (!p.w || al(p.w, 16)) && (!p.freqs || al(p.freqs, 16)) &&
           (!p.out_bf16 || p.lo_off % 4 == 0);
}


// ---- One launch for a self-attention's three operands ----
// Q rows and K rows (RMSNorm, RoPE, written dense as f32, bf16 or bf16 term
// rows) and, for the bf16-MFMA kernels, V packed as V^T (bf16 or hi/lo term
// rows; the layout of vt_pack_kernel / vt_pack_terms_kernel).  The work is a
// single grid of 32-key halves of V^T tiles, then 32-row groups of K, then
// of Q, so the three streams share one ramp and one tail instead of three,
// and every block keeps 16 KiB of loads in flight.  Row arithmetic is that of
// rows_d128_block (bit-identical outputs); q, k and v are [B, S, H, 128]
// views whose token rows are `ld` elements apart (column blocks of a fused
// projection allowed), batch entries S * ld apart.
constexpr int kPrepRows = 32;
constexpr int kPrepPitch = 132;                   // floats per staged row
// Row groups of 32 and V^T blocks of 32 keys (half a 64-key tile) keep the
// block at 20 KiB of LDS, eight blocks per CU: against 64-row groups and
// whole tiles (37 KiB, four blocks) 62.5 against 69.9 us (bf16) and 88.3
// against 89.7 us (f32x3) for 4096 tokens, B=2, H=16.
constexpr int kPrepVKeys = 32;                    // keys per V^T block (half a 64-key tile)
constexpr int kPrepTW = kPrepVKeys / 2 + 4;        // 32-bit words per transposed V^T row
constexpr int kPrepLds = 2 * 128 * kPrepTW;       // >= kPrepRows * kPrepPitch
static_assert(kPrepLds >= kPrepRows * kPrepPitch, "LDS union");
// RoPE table rows ([64 pairs][4] f32, 1 KiB per token) staged once per row
// group when its rows span at most this many tokens (H >= 16): read from L2
// per row instead, every table row would be fetched once per head
// (one-launch prologue 93 -> 89 us f32x3, 73 -> 70 us bf16 at 64-row groups).
constexpr int kPrepTabTokens = 2;
constexpr int kPrepTabFloats = kPrepTabTokens * 256;
// The LDS array: rows, table and 1/rms for Q/K groups, the two transposed
// V^T term blocks for V (20 KiB: eight blocks per CU).
constexpr int kPrepQKFloats = kPrepRows * kPrepPitch + kPrepTabFloats + kPrepRows;
constexpr int kPrepLdsAll = kPrepQKFloats > kPrepLds ? kPrepQKFloats : kPrepLds;

struct PrepArgs {
    const float *x[2];  // q, k
    void *out[2];       // dense rows: 128 f32, 128 bf16 or 256 bf16 (terms)
    const float *w[2];  // RMSNorm weights or null
    const float *freqs; // [S, 64, 2, 2] or null
    const float *v;
    unsigned short *vt; // [B*H][128 or 256 rows][sp]
    int64_t ld, sp;
    int rows;           // B*S*H (< 2^31, checked at launch)
    int qk_units;       // row groups per tensor
    int S, H, n_vtiles;
    int v_units;        // V^T blocks (0 in f32 mode); they come first in the grid
    float eps;
};

__device__ __forceinline__ unsigned pack_bf16x2(float a, float b)
{
    return unsigned(f32_to_bf16_rne(a)) | (unsigned(f32_to_bf16_rne(b)) << 16);
}

// A float4 of q, k or v, which this launch reads once: with NT, a
// nontemporal (streaming) load, so the inputs do not displace the outputs
// the attention kernel reads next from the caches (4096 tokens, B=2, H=16:
// 82.0 -> 75.4 us f32x3, 60.1 -> 59.3 us bf16; the f32 rows, which write
// less than they read, ran 49.2 -> 52.0 us and keep plain loads).
template <bool NT>
__device__ __forceinline__ f32x4 stream_load(const float *p)
{
    const f32x4 *q = reinterpret_cast<const f32x4 *>(p);
    return NT ? __builtin_nontemporal_load(q) : *q;
}

// OUT: 0 = f32 rows (no V), 1 = bf16 rows + bf16 V^T, 2 = term rows + term V^T.
template <int OUT>
__global__ __launch_bounds__(256) void prep_qkv_kernel(PrepArgs a)
{
    __shared__ __attribute__((aligned(16))) float lds[kPrepLdsAll];
    float *const inv = lds + kPrepRows * kPrepPitch + kPrepTabFloats;  // Q/K groups
    const int t = threadIdx.x;
    // Grid order: V^T blocks, then K row groups, then Q row groups, so the
    // rows the attention kernel reads first (Q) are the last written (and the
    // launch itself runs faster: 88.8 -> 81.3 us f32x3, 62.7 -> 60.3 us bf16
    // at 4096 tokens, B=2, H=16; the step 0.85 % and 0.6 % faster).
    const int u = int(blockIdx.x) - a.v_units;
    if (u >= 0) {
        const int p = u < a.qk_units ? 1 : 0;
        const int r0 = (p ? u : u - a.qk_units) * kPrepRows;
        const float *x = a.x[p];
        const int c4 = t & 31;
        // 32-bit row arithmetic (rows < 2^31): the token index r / H and the
        // head r % H of every row this thread loads.
#pragma unroll
        for (int i = 0; i < kPrepRows / 8; ++i) {
            const int rr = (t >> 5) + 8 * i;
            const int r = r0 + rr;
            if (r < a.rows) {
                const unsigned bs = unsigned(r) / unsigned(a.H);
                const int h = r - int(bs) * a.H;
                *reinterpret_cast<f32x4 *>(&lds[rr * kPrepPitch + 4 * c4]) =
                    stream_load<OUT != 0>(x + int64_t(bs) * a.ld + h * 128 + 4 * c4);
            }
        }
        // The RoPE table rows of the group's tokens bs0 .. bs1 (batch * S +
        // token), staged after the rows when there are at most
        // kPrepTabTokens of them: one 16-byte chunk (the 2x2 matrix of pair
        // c) per thread, stored at (c % 4) * 16 + c / 4 so that the 16
        // threads of a row, which read pairs 4i + e (i = 0..15) for one e at
        // a time, hit 16 consecutive chunks.
        const unsigned bs0 = unsigned(r0) / unsigned(a.H);
        const unsigned bs1 = unsigned(min(r0 + kPrepRows, a.rows) - 1) / unsigned(a.H);
        const bool tab_lds = a.freqs && bs1 - bs0 < unsigned(kPrepTabTokens);
        float *tab = lds + kPrepRows * kPrepPitch;
        if (tab_lds && (t >> 6) < kPrepTabTokens && bs0 + unsigned(t >> 6) <= bs1) {
            const int c = t & 63;
            *reinterpret_cast<f32x4 *>(&tab[(t >> 6) * 256 + 4 * ((c & 3) * 16 + (c >> 2))]) =
                *reinterpret_cast<const f32x4 *>(
                    a.freqs + int64_t((bs0 + unsigned(t >> 6)) % unsigned(a.S)) * 256 + 4 * c);
        }
        __syncthreads();
        if (t < kPrepRows) {
            // One thread per row: the sum of squares in index order.
            float ss = 0.0f;
            const float *row = lds + t * kPrepPitch;
#pragma unroll 8
            for (int j = 0; j < 32; ++j) {
                const f32x4 v = *reinterpret_cast<const f32x4 *>(row + 4 * j);
                ss = ss + v.x * v.x;
                ss = ss + v.y * v.y;
                ss = ss + v.z * v.z;
                ss = ss + v.w * v.w;
            }
            inv[t] = inv_rms(ss, 128, a.eps);
        }
        __syncthreads();
        const int p0 = 4 * (t & 15);
        f32x4 wl = f32x4{1.f, 1.f, 1.f, 1.f}, wh = wl;
        if (a.w[p]) {
            wl = *reinterpret_cast<const f32x4 *>(a.w[p] + p0);
            wh = *reinterpret_cast<const f32x4 *>(a.w[p] + 64 + p0);
        }
#pragma unroll
        for (int i = 0; i < kPrepRows / 16; ++i) {
            const int rr = (t >> 4) + 16 * i;
            const int r = r0 + rr;
            if (r >= a.rows)
                continue;
            const float *row = lds + rr * kPrepPitch;
            const float fi = inv[rr];
            f32x4 ya = *reinterpret_cast<const f32x4 *>(row + p0);
            f32x4 yb = *reinterpret_cast<const f32x4 *>(row + 64 + p0);
            ya = ya * fi;
            yb = yb * fi;
            if (a.w[p]) {
                ya = ya * wl;
                yb = yb * wh;
            }
            f32x4 lo = ya, hi = yb;
            if (a.freqs) {
                const unsigned bs = unsigned(r) / unsigned(a.H);
                const f32x4 *fq = reinterpret_cast<const f32x4 *>(
                    a.freqs + int64_t(bs % unsigned(a.S)) * 256 + 4 * p0);
                const f32x4 *fl =
                    reinterpret_cast<const f32x4 *>(tab + (bs - bs0) * 256 + 4 * (t & 15));
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // [c00, c01, c10, c11] of pair p0 + e
                    const f32x4 c = tab_lds ? fl[16 * e] : fq[e];
                    lo[e] = c.x * ya[e] + c.y * yb[e];
                    hi[e] = c.z * ya[e] + c.w * yb[e];
                }
            }
            if (OUT == 0) {
                float *of = static_cast<float *>(a.out[p]) + int64_t(r) * 128 + p0;
                *reinterpret_cast<f32x4 *>(of) = lo;
                *reinterpret_cast<f32x4 *>(of + 64) = hi;
            } else {
                unsigned short *ob = static_cast<unsigned short *>(a.out[p]) +
                                     int64_t(r) * (OUT == 2 ? 256 : 128) + p0;
                store_bf16x4(ob, OUT == 2 ? 128 : 0, lo[0], lo[1], lo[2], lo[3]);
                store_bf16x4(ob + 64, OUT == 2 ? 128 : 0, hi[0], hi[1], hi[2], hi[3]);
            }
        }
        return;
    }
    if (OUT == 0)
        return;
    // V block: kPrepVKeys keys of one (batch, head), transposed through LDS into rows
    // of V^T with keys in vt_key_pos order; adjacent key pairs share a word.
    const unsigned vu = blockIdx.x;
    const unsigned bh = vu / unsigned(a.n_vtiles);
    const int tile = int(vu - bh * unsigned(a.n_vtiles));
    const unsigned b = bh / unsigned(a.H);
    const int h = int(bh - b * unsigned(a.H));
    const int key0 = tile * kPrepVKeys;
    const float *vp = a.v + int64_t(b) * a.S * a.ld + h * 128;
    unsigned *Th = reinterpret_cast<unsigned *>(lds);
    unsigned *Tl = Th + 128 * kPrepTW;
#pragma unroll
    for (int i = 0; i < kPrepVKeys / 16; ++i) {
        const int f = t + 256 * i;  // (key pair, float4 column) of the tile
        const int pr = f >> 5, c4 = f & 31;
        const int k0 = key0 + 2 * pr, k1 = k0 + 1;
        const f32x4 x0 = k0 < a.S ? stream_load<true>(vp + int64_t(k0) * a.ld + 4 * c4)
                                  : f32x4{0.f, 0.f, 0.f, 0.f};
        const f32x4 x1 = k1 < a.S ? stream_load<true>(vp + int64_t(k1) * a.ld + 4 * c4)
                                  : f32x4{0.f, 0.f, 0.f, 0.f};
        const int wd = vt_key_pos(2 * pr) >> 1;  // word holding positions (2wd, 2wd+1)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const unsigned hw = pack_bf16x2(x0[e], x1[e]);
            Th[(4 * c4 + e) * kPrepTW + wd] = hw;
            if (OUT == 2) {
                const float h0 = __uint_as_float(hw << 16), h1 = __uint_as_float(hw & 0xFFFF0000u);
                Tl[(4 * c4 + e) * kPrepTW + wd] = pack_bf16x2(x0[e] - h0, x1[e] - h1);
            }
        }
    }
    __syncthreads();
    constexpr int vrows = OUT == 2 ? 256 : 128;
    unsigned short *tp = a.vt + int64_t(bh) * vrows * a.sp + key0;
#pragma unroll
    for (int i = 0; i < kPrepVKeys / 16; ++i) {
        const int f = t + 256 * i;  // 16-byte chunk: d row, 8 keys
        const int d = f / (kPrepVKeys / 8), c = f % (kPrepVKeys / 8);
        *reinterpret_cast<f32x4 *>(tp + d * a.sp + 8 * c) =
            *reinterpret_cast<const f32x4 *>(&Th[d * kPrepTW + 4 * c]);
        if (OUT == 2)
            *reinterpret_cast<f32x4 *>(tp + (128 + d) * a.sp + 8 * c) =
                *reinterpret_cast<const f32x4 *>(&Tl[d * kPrepTW + 4 * c]);
    }
}

}  // namespace

bool launch_rows_pair(const RowProblem &p1, const RowProblem &p2, hipStream_t st)
{
    const int64_t r1 = int64_t(p1.B) * p1.S * p1.H, r2 = int64_t(p2.B) * p2.S * p2.H;
    if (r1 == 0 || r2 == 0 || !d128_eligible(p1) || !d128_eligible(p2))
        return launch_rows(p1, st) && launch_rows(p2, st);
    const int64_t n1 = (r1 + kRows128 - 1) / kRows128, n2 = (r2 + kRows128 - 1) / kRows128;
    if (n1 + n2 > INT32_MAX)
        return fail("rows kernel: too many rows");
    hipLaunchKernelGGL(rows_d128_pair, dim3(unsigned(n1 + n2)), dim3(256), 0, st, row_args(p1),
                       row_args(p2), n1);
    return hip_ok(hipGetLastError(), "rows_d128_pair launch");
}

bool launch_rows(const RowProblem &p, hipStream_t st)
{
    const int64_t rows = int64_t(p.B) * p.S * p.H;
    if (rows == 0 || p.D == 0)
        return true;
    if (p.freqs && (p.D & 1))
        return fail("rope: head dim must be even");
    RowArgs a = row_args(p);
    if (d128_eligible(p)) {
        a.rows_per_block = kRows128;
        const int64_t nblk = (rows + kRows128 - 1) / kRows128;
        if (nblk > INT32_MAX)
            return fail("rows kernel: too many rows");
        hipLaunchKernelGGL(rows_d128, dim3(unsigned(nblk)), dim3(256), 0, st, a);
        return hip_ok(hipGetLastError(), "rows_d128 launch");
    }

    // Generic D: up to 64 rows per block within 48 KiB of LDS; at least one row.
    const int64_t budget = 48 * 1024 / 4;
    const int rb = int(std::min<int64_t>(64, budget / (p.D + 8)));
    if (rb < 1)
        return fail("rows kernel: D=" + std::to_string(p.D) + " exceeds the per-row LDS budget");
    const int64_t nblk = (rows + rb - 1) / rb;
    if (nblk > INT32_MAX)
        return fail("rows kernel: too many rows");
    a.rows_per_block = rb;
    // LDS: rows [rb][D+1] f32, inv [rb] f32, s [rb] i32, (pad to 8 bytes),
    // offsets [rb][2] i64 -- the layout rows_kernel computes.
    const size_t nwords = size_t(rb) * (p.D + 1) + 2 * size_t(rb);
    const size_t shm = 4 * (nwords + (nwords & 1)) + sizeof(int64_t) * 2 * size_t(rb);
    hipLaunchKernelGGL(rows_kernel, dim3(unsigned(nblk)), dim3(256), shm, st, a);
    return hip_ok(hipGetLastError(), "rows_kernel launch");
}


bool prep_qkv_supported(const PrepProblem &p)
{
    const auto al = [](const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    return p.D == 128 && p.ld % 4 == 0 && p.ld >= int64_t(p.H) * p.D && al(p.q) && al(p.k) &&
           al(p.qo) && al(p.ko) && (!p.w[0] || al(p.w[0])) && (!p.w[1] || al(p.w[1])) &&
           (!p.freqs || al(p.freqs)) && (p.mode == kAttnF32 || (al(p.v) && al(p.vt)));
}

bool launch_prep_qkv(const PrepProblem &p, hipStream_t st)
{
    const int64_t rows = int64_t(p.B) * p.S * p.H;
    if (rows == 0)
        return true;
    if (!prep_qkv_supported(p))
        return fail("prep_qkv: D must be 128 with 16-byte aligned operands and row strides");
    PrepArgs a;
    a.x[0] = p.q;
    a.x[1] = p.k;
    a.out[0] = p.qo;
    a.out[1] = p.ko;
    a.w[0] = p.w[0];
    a.w[1] = p.w[1];
    a.freqs = p.freqs;
    a.v = p.v;
    a.vt = p.vt;
    const int64_t sp = vt_padded_len(p.S);
    const int64_t nblk = 2 * ((rows + kPrepRows - 1) / kPrepRows) +
                         (p.mode == kAttnF32 ? 0 : int64_t(p.B) * p.H * (sp / kPrepVKeys));
    if (rows > INT32_MAX - kPrepRows || nblk > INT32_MAX)
        return fail("prep_qkv: problem too large for one launch");
    a.ld = p.ld;
    a.rows = int(rows);
    a.sp = sp;
    a.qk_units = int((rows + kPrepRows - 1) / kPrepRows);
    a.S = p.S;
    a.H = p.H;
    a.n_vtiles = int(sp / kPrepVKeys);
    a.v_units = p.mode == kAttnF32 ? 0 : int(int64_t(p.B) * p.H * (sp / kPrepVKeys));
    a.eps = p.eps;
    switch (p.mode) {
    case kAttnF32:
        hipLaunchKernelGGL(prep_qkv_kernel<0>, dim3(unsigned(nblk)), dim3(256), 0, st, a);
        break;
    case kAttnBF16:
        hipLaunchKernelGGL(prep_qkv_kernel<1>, dim3(unsigned(nblk)), dim3(256), 0, st, a);
        break;
    default:
        hipLaunchKernelGGL(prep_qkv_kernel<2>, dim3(unsigned(nblk)), dim3(256), 0, st, a);
        break;
    }
    return hip_ok(hipGetLastError(), "prep_qkv_kernel launch");
}

}  // namespace anima_hip
