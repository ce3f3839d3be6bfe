// Sustained bf16 MFMA rate of the GPU under the benchmark's conditions, for
// the measurement only (libanima_probe.so; not part of the attention
// library).  The published 2.5 PFLOP/s dense bf16 peak assumes the 2.4 GHz
// peak shader clock; under sustained MFMA load the MI355X lowers its clock
// to stay inside its power limit, and how far depends on the operands' bit
// activity.  This probe runs nothing but v_mfma_f32_32x32x16_bf16 -- one
// 8-wave workgroup per CU (two waves per SIMD, as the flash kernels run; each
// workgroup holds 96 KiB of LDS so that no CU gets two),
// each wave cycling 16 independent MFMAs over 8 A and 4 B fragments read
// from `src` once -- so its rate is the ceiling a kernel reaches on the same
// data with no other instruction beside its MFMAs.  Each wave also reads the
// shader-clock counter (s_memtime) and the 100 MHz real-time counter
// (s_memrealtime) around its loop, which gives the clock the GPU held.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kWaves = 8;
constexpr int kFrags = 12;  // 8 A + 4 B fragments per lane

// LDS held by each workgroup only so that two of them never share a CU.
constexpr int kLdsHold = 96 * 1024;

__global__ __launch_bounds__(kWaves * 64, 1) void mfma_probe_kernel(const bf16x8 *src, float *out,
                                                                    uint64_t *cyc, int iters)
{
    __shared__ float hold[kLdsHold / 4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    hold[threadIdx.x] = float(iters);
    const int gw = blockIdx.x * kWaves + wave;
    const bf16x8 *p = src + size_t(gw) * kFrags * 64 + lane;
    bf16x8 a[8], b[4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        a[i] = p[i * 64];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        b[i] = p[(8 + i) * 64];
    f32x16 acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
        acc[c] = f32x16{};
    const uint64_t t0 = clock64(), r0 = wall_clock64();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            acc[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i & 7], b[i >> 2], acc[i & 3],
                                                                 0, 0, 0);
    }
    const uint64_t t1 = clock64(), r1 = wall_clock64();
    __syncthreads();
    float s = hold[(threadIdx.x + 64) % (kWaves * 64)];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r)
            s += acc[c][r];
    out[size_t(gw) * 64 + lane] = s;
    if (lane == 0) {
        cyc[2 * gw] = t1 - t0;
        cyc[2 * gw + 1] = r1 - r0;
    }
}

}  // namespace

extern "C" {

// Bytes of `src` for a grid of `workgroups`: 12 bf16x8 fragments per lane.
size_t anima_probe_mfma_src_bytes(int workgroups)
{
    return workgroups > 0 ? size_t(workgroups) * kWaves * kFrags * 64 * sizeof(bf16x8) : 0;
}

// Runs `launches` back-to-back launches of `workgroups` 8-wave workgroups,
// `iters` loop iterations each (16 MFMAs per wave and iteration), on
// `stream`, after `warm_launches` untimed ones.  Writes the mean time per
// launch (HIP events on the stream), the executed bf16 MFMA TFLOP/s and the
// mean shader clock in GHz over the timed launches' waves.  src: device
// memory of anima_probe_mfma_src_bytes(workgroups) bytes (the operands).
// Returns false on a HIP error or bad arguments.  Synchronous.
bool anima_probe_mfma(const void *src, int workgroups, int iters, int warm_launches, int launches,
                      void *stream, float *ms_per_launch, double *tflops, double *clock_ghz)
{
    if (!src || workgroups <= 0 || iters <= 0 || launches <= 0 || warm_launches < 0 ||
        !ms_per_launch || !tflops || !clock_ghz)
        return false;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t nw = size_t(workgroups) * kWaves;
    float *out = nullptr;
    uint64_t *cyc = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    bool ok = hipMalloc(&out, nw * 64 * sizeof(float)) == hipSuccess &&
              hipMalloc(&cyc, nw * 2 * sizeof(uint64_t)) == hipSuccess &&
              hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess;
    if (ok) {
        const bf16x8 *s = static_cast<const bf16x8 *>(src);
        for (int i = 0; i < warm_launches; ++i)
            mfma_probe_kernel<<<workgroups, kWaves * 64, 0, st>>>(s, out, cyc, iters);
        ok = hipEventRecord(e0, st) == hipSuccess;
        for (int i = 0; ok && i < launches; ++i)
            mfma_probe_kernel<<<workgroups, kWaves * 64, 0, st>>>(s, out, cyc, iters);
        ok = ok && hipGetLastError() == hipSuccess && hipEventRecord(e1, st) == hipSuccess &&
             hipEventSynchronize(e1) == hipSuccess;
    }
    float ms = 0.f;
    ok = ok && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
    if (ok) {
        // Clock from the last launch's waves: shader cycles over real time.
        uint64_t *h = new uint64_t[nw * 2];
        ok = hipMemcpy(h, cyc, nw * 2 * sizeof(uint64_t), hipMemcpyDeviceToHost) == hipSuccess;
        double c = 0, r = 0;
        for (size_t i = 0; i < nw; ++i) {
            c += double(h[2 * i]);
            r += double(h[2 * i + 1]);
        }
        delete[] h;
        *ms_per_launch = ms / launches;
        const double flops = double(nw) * iters * 16 * (32.0 * 32.0 * 16.0 * 2.0);
        *tflops = flops / (double(*ms_per_launch) * 1e-3) / 1e12;
        *clock_ghz = r > 0 ? c / (r / 100e6) / 1e9 : 0.0;
    }
    if (e0)
        (void)hipEventDestroy(e0);
    if (e1)
        (void)hipEventDestroy(e1);
    if (cyc)
        (void)hipFree(cyc);
    if (out)
        (void)hipFree(out);
    return ok;
}

}  // extern "C"
