// Element-wise and row operators of the anima_rt runtime that NumpyRT and
// anima_rt_ops.py call beside attention (anima_rt/src/anima_rt.cpp:24-60,
// gemm_backend.cpp:173-183): GELU (exact erf form), SiLU, LayerNorm without
// affine parameters, softmax over the last axis, and the bias add.
//   gelu/silu_kernel        one element per thread, HBM-bound;
//   layernorm_rows_kernel   one wave per row: mean, then the centred sum of
//                           squares (two passes over the row), then
//                           (x - mean) * rstd; the reference's Welford pass
//                           rounds differently, so rows agree to float32
//                           rounding, not bit for bit;
//   softmax_rows_kernel     one wave per row: max, sum of exp(x - max), then
//                           exp(x - max) * (1 / sum) as the reference does;
//   bias_add_kernel         C[i][j] += bias[j].
#include "common.h"

#include <cmath>

#pragma clang fp contract(off)

namespace anima_hip {
namespace {

__global__ __launch_bounds__(256) void gelu_kernel(const float *x, float *y, int64_t n)
{
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) {
        const float v = x[i];
        y[i] = v * 0.5f * (1.0f + erff(v * 0.70710678118654752440f));
    }
}

__global__ __launch_bounds__(256) void silu_kernel(const float *x, float *y, int64_t n)
{
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) {
        const float v = x[i];
        y[i] = v / (1.0f + expf(-v));
    }
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

__global__ __launch_bounds__(256) void layernorm_rows_kernel(const float *x, float *y, int64_t M,
                                                             int D, float eps)
{
    const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M)
        return;  // whole wave
    const float *xr = x + row * D;
    float *yr = y + row * D;
    float s = 0.0f;
    for (int j = lane; j < D; j += 64)
        s += xr[j];
    const float mean = wave_sum(s) / float(D);
    float q = 0.0f;
    for (int j = lane; j < D; j += 64) {
        const float d = xr[j] - mean;
        q += d * d;
    }
    const float rstd = 1.0f / sqrtf(wave_sum(q) / float(D) + eps);
    for (int j = lane; j < D; j += 64)
        yr[j] = (xr[j] - mean) * rstd;
}

__global__ __launch_bounds__(256) void softmax_rows_kernel(const float *x, float *y, int64_t M,
                                                           int D)
{
    const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M)
        return;  // whole wave
    const float *xr = x + row * D;
    float *yr = y + row * D;
    float m = -INFINITY;
    for (int j = lane; j < D; j += 64)
        m = fmaxf(m, xr[j]);
    m = wave_max(m);
    float s = 0.0f;
    for (int j = lane; j < D; j += 64)
        s += expf(xr[j] - m);
    const float inv = 1.0f / wave_sum(s);
    for (int j = lane; j < D; j += 64)
        yr[j] = expf(xr[j] - m) * inv;
}

__global__ __launch_bounds__(256) void bias_add_kernel(float *c, const float *bias, int64_t n,
                                                       int N)
{
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i < n)
        c[i] = c[i] + bias[i % N];
}

unsigned blocks_for(int64_t n, int64_t per_block) { return unsigned((n + per_block - 1) / per_block); }

bool too_big(int64_t blocks) { return blocks > INT32_MAX; }

}  // namespace

bool launch_gelu(const float *x, float *y, int64_t n, hipStream_t st)
{
    if (n <= 0)
        return true;
    if (too_big((n + 255) / 256))
        return fail("gelu: too many elements");
    hipLaunchKernelGGL(gelu_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, x, y, n);
    return hip_ok(hipGetLastError(), "gelu_kernel launch");
}

bool launch_silu(const float *x, float *y, int64_t n, hipStream_t st)
{
    if (n <= 0)
        return true;
    if (too_big((n + 255) / 256))
        return fail("silu: too many elements");
    hipLaunchKernelGGL(silu_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, x, y, n);
    return hip_ok(hipGetLastError(), "silu_kernel launch");
}

bool launch_layernorm_rows(const float *x, float *y, int64_t M, int D, float eps, hipStream_t st)
{
    if (M <= 0 || D <= 0)
        return true;
    if (too_big((M + 3) / 4))
        return fail("layernorm: too many rows");
    hipLaunchKernelGGL(layernorm_rows_kernel, dim3(blocks_for(M, 4)), dim3(256), 0, st, x, y, M,
                       D, eps);
    return hip_ok(hipGetLastError(), "layernorm_rows_kernel launch");
}

bool launch_softmax_rows(const float *x, float *y, int64_t M, int D, hipStream_t st)
{
    if (M <= 0 || D <= 0)
        return true;
    if (too_big((M + 3) / 4))
        return fail("softmax: too many rows");
    hipLaunchKernelGGL(softmax_rows_kernel, dim3(blocks_for(M, 4)), dim3(256), 0, st, x, y, M, D);
    return hip_ok(hipGetLastError(), "softmax_rows_kernel launch");
}

bool launch_bias_add(float *c, const float *bias, int64_t M, int N, hipStream_t st)
{
    const int64_t n = M * N;
    if (M <= 0 || N <= 0)
        return true;
    if (too_big((n + 255) / 256))
        return fail("bias_add: too many elements");
    hipLaunchKernelGGL(bias_add_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, c, bias, n, N);
    return hip_ok(hipGetLastError(), "bias_add_kernel launch");
}

}  // namespace anima_hip
