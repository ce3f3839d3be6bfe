// Linear layer GEMM: C[M,N] = A[M,K] . W[N,K]^T, A f32, W bf16 or f32, f32
// accumulation on v_mfma_f32_32x32x2_f32.
//
// Replaces anima_rt_run_gemm_bf16 / anima_rt_run_gemm_fp32
// (anima_rt/src/gemm_backend.cpp:140-173, row-major C = A @ W^T with W laid
// out [out_features, in_features]); used here for the cross-attention context
// projections k_proj / v_proj (anima_rt/scripts/numpy_dit.py:277-281), whose
// results the context K/V cache keeps for every denoise step.
//
// Block tile 128x128, K chunk 32, 4 waves in a 2x2 grid each owning 64x64
// (four 32x32 MFMA accumulators).  Operands are staged through LDS as f32
// (bf16 weights widened on the way in); every global access is bounds-checked
// so any M, N, K and any leading dimensions are accepted.
#include "common.h"

namespace anima_hip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 128, kBK = 32;
constexpr int kPitch = kBK + 4;  // floats per LDS row

struct GemmArgs {
    const float *a;
    const void *w;
    float *c;
    int64_t lda, ldw, ldc;
    int M, N, K, w_bf16, n_tiles_n;
};

__device__ __forceinline__ float load_w(const GemmArgs &g, int64_t idx)
{
    if (g.w_bf16) {
        const unsigned short bits = static_cast<const unsigned short *>(g.w)[idx];
        return __uint_as_float(unsigned(bits) << 16);
    }
    return static_cast<const float *>(g.w)[idx];
}

__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g)
{
    __shared__ __attribute__((aligned(16))) float As[kBM * kPitch];
    __shared__ __attribute__((aligned(16))) float Ws[kBN * kPitch];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, half = lane >> 5;
    const int tm = blockIdx.x / g.n_tiles_n, tn = blockIdx.x % g.n_tiles_n;
    const int m0 = tm * kBM, n0 = tn * kBN;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

    f32x16 acc[2][2] = {};
    for (int k0 = 0; k0 < g.K; k0 += kBK) {
        // 128 x 32 elements of each operand, 16 per thread, coalesced along K.
#pragma unroll 4
        for (int i = 0; i < 16; ++i) {
            const int e = tid + 256 * i;
            const int r = e >> 5, kk = e & 31;
            const int gm = m0 + r, gn = n0 + r, gk = k0 + kk;
            As[r * kPitch + kk] = (gm < g.M && gk < g.K) ? g.a[gm * g.lda + gk] : 0.0f;
            Ws[r * kPitch + kk] = (gn < g.N && gk < g.K) ? load_w(g, gn * g.ldw + gk) : 0.0f;
        }
        __syncthreads();
        // Lane half h contracts k = 16h + t (t = 0..15) of the chunk, for A
        // and W alike.
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
            f32x4 av[2], wv[2];
#pragma unroll
            for (int x = 0; x < 2; ++x) {
                av[x] = *reinterpret_cast<const f32x4 *>(
                    &As[(wm + 32 * x + col) * kPitch + 16 * half + 4 * t4]);
                wv[x] = *reinterpret_cast<const f32x4 *>(
                    &Ws[(wn + 32 * x + col) * kPitch + 16 * half + 4 * t4]);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int x = 0; x < 2; ++x)
#pragma unroll
                    for (int y = 0; y < 2; ++y)
                        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[x][e], wv[y][e],
                                                                         acc[x][y], 0, 0, 0);
        }
        __syncthreads();
    }
    // acc[x][y] register r, lane l: row 8(r/4) + 4h + (r%4), column l%32.
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int gm = m0 + wm + 32 * x + 8 * (r >> 2) + 4 * half + (r & 3);
                const int gn = n0 + wn + 32 * y + col;
                if (gm < g.M && gn < g.N)
                    g.c[gm * g.ldc + gn] = acc[x][y][r];
            }
}

}  // namespace

bool launch_gemm(const float *a, int64_t lda, const void *w, bool w_bf16, int64_t ldw, float *c,
                 int64_t ldc, int M, int N, int K, hipStream_t st)
{
    if (M < 0 || N < 0 || K < 0)
        return fail("gemm: negative dimension");
    if (M == 0 || N == 0)
        return true;  // K == 0 runs the kernel, which then stores zeros
    GemmArgs g;
    g.a = a;
    g.w = w;
    g.c = c;
    g.lda = lda;
    g.ldw = ldw;
    g.ldc = ldc;
    g.M = M;
    g.N = N;
    g.K = K;
    g.w_bf16 = w_bf16 ? 1 : 0;
    g.n_tiles_n = (N + kBN - 1) / kBN;
    const int64_t nblk = int64_t((M + kBM - 1) / kBM) * g.n_tiles_n;
    if (nblk > INT32_MAX)
        return fail("gemm: problem too large for one launch");
    hipLaunchKernelGGL(gemm_kernel, dim3(unsigned(nblk)), dim3(256), 0, st, g);
    return hip_ok(hipGetLastError(), "gemm_kernel launch");
}

}  // namespace anima_hip
