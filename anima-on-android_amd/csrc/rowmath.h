// Row arithmetic shared by the row prologue (prologue.hip) and the flash
// kernels that prepare their own query rows: bf16 rounding, the second bf16
// term of an f32 value, and the RMSNorm scale of anima_rt's rmsnorm_kernel
// (anima_rt/include/cpu/rmsnorm_kernel.h:11-31), 1 / sqrt(ss / D + eps) with
// the f32 divide and sqrt correctly rounded.
#pragma once

#include <hip/hip_runtime.h>

namespace anima_hip {

// f32 -> bf16, round to nearest even (bit pattern).
__device__ __forceinline__ unsigned short f32_to_bf16_rne(float f)
{
    unsigned int u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (unsigned short)(u >> 16);
}

// Second bf16 term of f: bf16(f - hi), hi = bf16(f) (f - hi is exact in f32).
__device__ __forceinline__ unsigned short bf16_lo_term(float f, unsigned short hi)
{
    return f32_to_bf16_rne(f - __uint_as_float(unsigned(hi) << 16));
}

__device__ __forceinline__ float inv_rms(float ss, int D, float eps)
{
    // f32 divide and sqrt, each correctly rounded: evaluated in f64 and
    // rounded once (exact for f32 operands).
    const float ms = (float)((double)ss / (double)D);
    const float root = (float)sqrt((double)(ms + eps));
    return (float)(1.0 / (double)root);
}

}  // namespace anima_hip
