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
//
// Bit-exactness: one thread owns each row's sum of squares and adds the
// squares in index order; floating-point contraction is switched off for this
// file (HIP's default -ffp-contract=fast would fuse x*x + s, and the header's
// round-to-nearest helpers are plain operators), and the f32 division and
// sqrt are rounded correctly by evaluating them in f64 and rounding once.
// Rows are staged through LDS so global loads and stores stay coalesced.
#include "common.h"

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
    int S, H, D, rows_per_block;
    float eps;
    int norm, out_bf16;
};

__device__ __forceinline__ unsigned short f32_to_bf16_rne(float f)
{
    unsigned int u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (unsigned short)(u >> 16);
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

__global__ __launch_bounds__(256) void rows_kernel(RowArgs a)
{
    extern __shared__ float lds[];
    const int D = a.D;
    const int pitch = D + 1;  // odd pitch: serial per-row reads are conflict-free
    const int RB = a.rows_per_block;
    float *xs = lds;                       // [RB][pitch]
    float *inv = lds + RB * pitch;         // [RB]
    const int64_t r0 = int64_t(blockIdx.x) * RB;
    const int nrows = int(min<int64_t>(RB, a.rows - r0));
    const int n = nrows * D;

    // Stage the rows (coalesced along D).
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        const int rr = e / D, d = e - rr * D;
        int64_t xo, oo;
        int s;
        row_coords(a, r0 + rr, xo, oo, s);
        xs[rr * pitch + d] = a.x[xo + d];
    }
    __syncthreads();

    // Serial sum of squares, one thread per row, index order.
    for (int rr = threadIdx.x; rr < nrows; rr += blockDim.x) {
        float f = 1.0f;
        if (a.norm) {
            const float *row = xs + rr * pitch;
            float ss = 0.0f;
            for (int d = 0; d < D; ++d)
                ss = ss + row[d] * row[d];
            // f32 divide and sqrt, each correctly rounded: evaluated in f64
            // and rounded once (exact for f32 operands), since the f32
            // device routines may differ from IEEE rounding by an ulp.
            const float ms = (float)((double)ss / (double)D);
            const float root = (float)sqrt((double)(ms + a.eps));
            f = (float)(1.0 / (double)root);
        }
        inv[rr] = f;
    }
    __syncthreads();

    const int halfD = D >> 1;
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
        const int rr = e / D, d = e - rr * D;
        int64_t xo, oo;
        int s;
        row_coords(a, r0 + rr, xo, oo, s);
        const float *row = xs + rr * pitch;
        const float f = inv[rr];
        auto y_at = [&](int dd) {
            if (!a.norm)
                return row[dd];
            float v = row[dd] * f;
            if (a.w)
                v = v * a.w[dd];
            return v;
        };
        float out;
        if (a.freqs) {
            const int p = d < halfD ? d : d - halfD;
            const float ya = y_at(p), yb = y_at(p + halfD);
            const float *fq = a.freqs + int64_t(s) * D * 2 + 4 * p + (d < halfD ? 0 : 2);
            out = fq[0] * ya + fq[1] * yb;
        } else {
            out = y_at(d);
        }
        if (a.out_bf16)
            static_cast<unsigned short *>(a.out)[oo + d] = f32_to_bf16_rne(out);
        else
            static_cast<float *>(a.out)[oo + d] = out;
    }
}

}  // namespace

bool launch_rows(const RowProblem &p, hipStream_t st)
{
    const int64_t rows = int64_t(p.B) * p.S * p.H;
    if (rows == 0 || p.D == 0)
        return true;
    if (p.freqs && (p.D & 1))
        return fail("rope: head dim must be even");
    // Up to 64 rows per block within 48 KiB of LDS; at least one row.
    const int64_t budget = 48 * 1024 / 4;
    int rb = int(std::min<int64_t>(64, budget / (p.D + 2)));
    if (rb < 1)
        return fail("rows kernel: D=" + std::to_string(p.D) + " exceeds the per-row LDS budget");
    const int64_t nblk = (rows + rb - 1) / rb;
    if (nblk > INT32_MAX)
        return fail("rows kernel: too many rows");
    RowArgs a;
    a.x = p.x;
    a.out = p.out;
    a.w = p.w;
    a.freqs = p.freqs;
    a.xb = p.xs.b; a.xh = p.xs.h; a.xs = p.xs.s;
    a.ob = p.os.b; a.oh = p.os.h; a.os = p.os.s;
    a.rows = rows;
    a.S = p.S;
    a.H = p.H;
    a.D = p.D;
    a.rows_per_block = rb;
    a.eps = p.eps;
    a.norm = p.norm ? 1 : 0;
    a.out_bf16 = p.out_bf16 ? 1 : 0;
    const size_t shm = sizeof(float) * (size_t(rb) * (p.D + 1) + rb);
    hipLaunchKernelGGL(rows_kernel, dim3(unsigned(nblk)), dim3(256), shm, st, a);
    return hip_ok(hipGetLastError(), "rows_kernel launch");
}

}  // namespace anima_hip
