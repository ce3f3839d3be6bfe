// Projection GEMM of the DiT attention: C[M,N] = A[M,K] . W[N,K]^T with f32
// activations A, f32 output C and bf16 weights W, on bf16 MFMA.
//
// Replaces the reference's projection GEMM (anima_rt/vulkan/gemm_bf16.comp:25-57:
// f32 A, bf16 W widened to f32, f32 FMA accumulation; CPU form
// anima_rt/src/gemm_backend.cpp:140-173) as NumpyAttention.forward calls it for
// q/k/v_proj and output_proj (anima_rt/scripts/numpy_dit.py:273-281, 294-296),
// and for the text-context k/v_proj that feed the context K/V cache.
//
// W is bf16 already, so only A needs a representation the bf16 MFMA accepts.
// split_kernel writes it as bf16 terms with rows padded to 8 elements:
//   exact mode  A = hi + lo + r,  hi = bf16(A), lo = bf16(A - hi),
//               |r| <= 2^-16 |A| per element; C = hi.W^T + lo.W^T
//               (two products, f32 accumulation);
//   bf16 mode   hi only (|A - hi| <= 2^-8 |A|).
// The products are plain bf16 x bf16 -> f32 GEMMs: hipBLASLt, or the
// hand-written kernels where they measured faster (small M: gemm_bf16.hip;
// large M: gemm_large.hip on term planes and gemm_f32a.hip, which splits f32
// A in registers so the split pass does not run).  A shape without a
// hipBLASLt solution falls back to gemm_kernel (f32 MFMA on the exact f32
// values).
#include "common.h"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <memory>
#include <mutex>
#include <tuple>

namespace anima_hip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

size_t round_up256(size_t n) { return (n + 255) / 256 * 256; }
int64_t padded_k(int K) { return (int64_t(K) + 7) / 8 * 8; }

struct SplitArgs {
    const float *a;
    int64_t lda;
    unsigned int *hi, *lo;  // [M][Kp] bf16, addressed as bf16 pairs
    int64_t kp;             // padded row length (elements)
    int64_t rs;             // row stride of hi/lo (elements): kp, or 2*kp for [hi | lo] rows
    int M, K, vec;
    int64_t total;          // M * Kp / 8 chunks
};

__device__ __forceinline__ unsigned int pack_pair(float x, float y)
{
    return __builtin_bit_cast(unsigned int, __builtin_convertvector(f32x2{x, y}, bf16x2));
}

__device__ __forceinline__ float bf16_lo_value(unsigned int w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi_value(unsigned int w) { return __uint_as_float(w & 0xFFFF0000u); }

// One thread per 8 consecutive elements of a row: hi (and lo) as one
// 16-byte store each; elements k >= K are written as zero.
__global__ __launch_bounds__(256) void split_kernel(SplitArgs a)
{
    const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= a.total)
        return;
    const int64_t chunks = a.kp / 8;
    const int64_t m = idx / chunks;
    const int k0 = int(idx - m * chunks) * 8;
    const float *row = a.a + m * a.lda;
    float x[8];
    if (a.vec && k0 + 8 <= a.K) {
        const f32x4 u = *reinterpret_cast<const f32x4 *>(row + k0);
        const f32x4 v = *reinterpret_cast<const f32x4 *>(row + k0 + 4);
        x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w;
        x[4] = v.x; x[5] = v.y; x[6] = v.z; x[7] = v.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            x[e] = k0 + e < a.K ? row[k0 + e] : 0.0f;
    }
    unsigned int h[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        h[e] = pack_pair(x[2 * e], x[2 * e + 1]);
        // x - hi is exact in f32 (hi holds the leading bits of x).
        l[e] = pack_pair(x[2 * e] - bf16_lo_value(h[e]), x[2 * e + 1] - bf16_hi_value(h[e]));
    }
    const int64_t off = (m * a.rs + k0) / 2;
    *reinterpret_cast<uint4 *>(a.hi + off) = uint4{h[0], h[1], h[2], h[3]};
    if (a.lo)
        *reinterpret_cast<uint4 *>(a.lo + off) = uint4{l[0], l[1], l[2], l[3]};
}

// hipBLASLt plans per device and problem shape.  Row-major C[M,N] = A W^T is
// the column-major product C^T[N,M] = op_T(W_cm[K,N]) . A_cm[K,M].
struct LtPlan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t lw = nullptr, la = nullptr, lc = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    bool ok = false;
};

struct LtDevice {
    hipblasLtHandle_t handle = nullptr;
    std::map<std::tuple<int, int, int, int64_t, int64_t, int64_t, bool, bool>,
             std::unique_ptr<LtPlan>>
        plans;
};

std::mutex g_lt_mu;
std::map<int, std::unique_ptr<LtDevice>> g_lt;

// alpha_vec: alpha is a device vector over the N output channels (the rows of
// the column-major product), beta a host scalar.  out_bf16: C/D are bf16.
LtPlan *lt_plan(int M, int N, int K, int64_t lda, int64_t ldw, int64_t ldc, bool alpha_vec = false,
                bool out_bf16 = false)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        return nullptr;
    auto &slot = g_lt[dev];
    if (!slot) {
        slot.reset(new LtDevice);
        if (hipblasLtCreate(&slot->handle) != HIPBLAS_STATUS_SUCCESS) {
            slot->handle = nullptr;
            return nullptr;
        }
    }
    if (!slot->handle)
        return nullptr;
    auto &pp = slot->plans[std::make_tuple(M, N, K, lda, ldw, ldc, alpha_vec, out_bf16)];
    if (pp)
        return pp->ok ? pp.get() : nullptr;
    pp.reset(new LtPlan);
    LtPlan &p = *pp;
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    const int32_t pmode = alpha_vec ? HIPBLASLT_POINTER_MODE_ALPHA_DEVICE_VECTOR_BETA_HOST
                                    : HIPBLASLT_POINTER_MODE_HOST;
    uint64_t ws = 0;
    hipblasLtMatmulPreference_t pref = nullptr;
    hipblasLtMatmulHeuristicResult_t res[1];
    int n = 0;
    const bool built =
        hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) ==
            HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) ==
            HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_POINTER_MODE, &pmode,
                                        sizeof(pmode)) == HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatrixLayoutCreate(&p.lw, HIP_R_16BF, K, N, ldw) == HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, K, M, lda) == HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatrixLayoutCreate(&p.lc, out_bf16 ? HIP_R_16BF : HIP_R_32F, N, M, ldc) ==
            HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                              sizeof(ws)) == HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatmulAlgoGetHeuristic(slot->handle, p.desc, p.lw, p.la, p.lc, p.lc, pref, 1, res,
                                        &n) == HIPBLAS_STATUS_SUCCESS &&
        n > 0 && res[0].state == HIPBLAS_STATUS_SUCCESS;
    if (pref)
        hipblasLtMatmulPreferenceDestroy(pref);
    if (built) {
        p.algo = res[0].algo;
        p.ok = true;
    }
    return p.ok ? &p : nullptr;
}

bool lt_matmul(LtPlan *p, const void *w, const void *a, void *c, float beta, hipStream_t st,
               const float *alpha_vec = nullptr)
{
    int dev = 0;
    (void)hipGetDevice(&dev);
    const float alpha = 1.0f;
    const void *ap = alpha_vec ? static_cast<const void *>(alpha_vec) : &alpha;
    const hipblasStatus_t s = hipblasLtMatmul(g_lt[dev]->handle, p->desc, ap, w, p->lw, a, p->la,
                                              &beta, c, p->lc, c, p->lc, &p->algo, nullptr, 0, st);
    if (s != HIPBLAS_STATUS_SUCCESS)
        return fail("linear: hipblasLtMatmul failed with status " + std::to_string(int(s)));
    return true;
}

}  // namespace

int64_t linear_terms_ld(int K) { return padded_k(K); }

bool linear_terms_supported(int M, int N, int K, const void *w, int64_t ldw, const float *c,
                            int64_t ldc)
{
    if (M <= 0 || N <= 0 || K <= 0 || ldw < K || ldc < N || (ldw % 8) != 0 || (ldc % 4) != 0 ||
        (reinterpret_cast<uintptr_t>(w) & 15u) != 0 || (reinterpret_cast<uintptr_t>(c) & 15u) != 0)
        return false;
    std::lock_guard<std::mutex> g(g_lt_mu);
    return lt_plan(M, N, K, padded_k(K), ldw, ldc) != nullptr;
}

// The small-M kernel (gemm_bf16.hip) beats the library GEMM at M <= 1024 on
// two-term products (each W chunk staged once for both terms) and on one-term
// products with K >= 8192 (measured at M = 512); elsewhere the library runs.
bool small_m_path(int M, int K, bool two_terms)
{
    return M > 0 && M <= 1024 && K % 64 == 0 && (two_terms || K >= 8192);
}

bool launch_linear_terms(const uint16_t *hi, const uint16_t *lo, const uint16_t *w, int64_t ldw,
                         float *c, int64_t ldc, int M, int N, int K, hipStream_t st, void *ws,
                         size_t ws_bytes)
{
    if (ws && small_m_path(M, K, lo != nullptr) &&
        gemm_bf16_supported(M, N, K, padded_k(K), ldw, ldc, hi, lo, w, c, ws_bytes))
        return launch_gemm_bf16(hi, lo, padded_k(K), w, ldw, c, ldc, M, N, K, ws, ws_bytes, st);
    if (lo && gemm_large_supported(M, N, K, 2, padded_k(K), ldw, ldc, hi, lo, w, c, 4))
        return launch_gemm_large(hi, lo, padded_k(K), w, ldw, c, ldc, M, N, K, kGemmOutF32,
                                 nullptr, 0, 0, st);
    if (!linear_terms_supported(M, N, K, w, ldw, c, ldc))
        return fail("linear: no bf16 GEMM for this shape");
    if ((reinterpret_cast<uintptr_t>(hi) & 15u) != 0 || (reinterpret_cast<uintptr_t>(lo) & 15u) != 0)
        return fail("linear: bf16 terms must be 16-byte aligned");
    std::lock_guard<std::mutex> g(g_lt_mu);
    LtPlan *plan = lt_plan(M, N, K, padded_k(K), ldw, ldc);
    if (!lt_matmul(plan, w, hi, c, 0.0f, st))
        return false;
    return !lo || lt_matmul(plan, w, lo, c, 1.0f, st);
}

bool launch_linear_pair(const uint16_t *terms, int64_t ld_t, int K, const uint16_t *w,
                        int64_t ldw, float *c, int64_t ldc, int M, int N, hipStream_t st, void *ws,
                        size_t ws_bytes)
{
    if (ws && small_m_path(M, K, true) &&
        gemm_bf16_supported(M, N, K, ld_t, ldw, ldc, terms, terms + K, w, c, ws_bytes))
        return launch_gemm_bf16(terms, terms + K, ld_t, w, ldw, c, ldc, M, N, K, ws, ws_bytes, st);
    if (ld_t != padded_k(2 * K))
        return fail("linear: [hi | lo] rows must be 2K elements long");
    return launch_linear_terms(terms, nullptr, w, ldw, c, ldc, M, N, 2 * K, st);
}

bool launch_linear_planes(const uint16_t *terms, int64_t ld_t, int K, bool pair,
                          const uint16_t *w, int64_t ldw, float *planes, size_t planes_bytes,
                          int M, int N, int *parts, hipStream_t st)
{
    const uint16_t *lo = pair ? terms + K : nullptr;
    const int64_t lda = pair ? ld_t : padded_k(K);
    if ((pair || ld_t == padded_k(K)) && small_m_path(M, K, pair) &&
        gemm_bf16_supported(M, N, K, lda, ldw, N, terms, lo, w, planes, planes_bytes) &&
        planes_bytes >= size_t(M) * N * sizeof(float))
        return launch_gemm_bf16_planes(terms, lo, lda, w, ldw, planes, planes_bytes, M, N, K,
                                       parts, st);
    *parts = 1;
    return pair ? launch_linear_pair(terms, ld_t, K, w, ldw, planes, N, M, N, st)
                : launch_linear_terms(terms, nullptr, w, ldw, planes, N, M, N, K, st);
}

uint16_t *launch_split_interleaved(const float *a, int64_t lda, int M, int K, void *scratch,
                                   size_t scratch_bytes, hipStream_t st)
{
    const int64_t kp = padded_k(K);
    if (M <= 0 || K <= 0 || lda < K || !scratch ||
        scratch_bytes < size_t(M) * size_t(kp) * 4 ||
        (reinterpret_cast<uintptr_t>(scratch) & 15u) != 0) {
        fail("split: bad sizes or scratch smaller than 2 terms per element");
        return nullptr;
    }
    SplitArgs sa;
    sa.a = a;
    sa.lda = lda;
    sa.hi = static_cast<unsigned int *>(scratch);
    sa.lo = sa.hi + kp / 2;  // [hi | lo] in each row
    sa.kp = kp;
    sa.rs = 2 * kp;
    sa.M = M;
    sa.K = K;
    sa.vec = (reinterpret_cast<uintptr_t>(a) & 15u) == 0 && lda % 4 == 0;
    sa.total = int64_t(M) * kp / 8;
    const int64_t nblk = (sa.total + 255) / 256;
    if (nblk > INT32_MAX) {
        fail("split: problem too large for one launch");
        return nullptr;
    }
    hipLaunchKernelGGL(split_kernel, dim3(unsigned(nblk)), dim3(256), 0, st, sa);
    if (!hip_ok(hipGetLastError(), "split_kernel launch"))
        return nullptr;
    return static_cast<uint16_t *>(scratch);
}

bool launch_linear_terms_bf16out(const uint16_t *hi, const uint16_t *w, int64_t ldw, uint16_t *c,
                                 int64_t ldc, int M, int N, int K, hipStream_t st)
{
    if (M <= 0 || N <= 0 || K <= 0 || ldw < K || ldc < N || (ldw % 8) != 0 || (ldc % 8) != 0 ||
        (reinterpret_cast<uintptr_t>(w) & 15u) != 0 || (reinterpret_cast<uintptr_t>(c) & 15u) != 0 ||
        (reinterpret_cast<uintptr_t>(hi) & 15u) != 0)
        return fail("linear: bf16-output GEMM needs positive sizes and 16-byte aligned rows");
    std::lock_guard<std::mutex> g(g_lt_mu);
    LtPlan *plan = lt_plan(M, N, K, padded_k(K), ldw, ldc, false, true);
    if (!plan)
        return fail("linear: no bf16-output GEMM for this shape");
    return lt_matmul(plan, w, hi, c, 0.0f, st);
}

// Shapes of the small-M kernel also hold its split-K partials, after the terms.
size_t linear_scratch_bytes(int M, int K, bool exact)
{
    if (M <= 0 || K <= 0)
        return 0;
    return round_up256(size_t(M) * size_t(padded_k(K)) * 2) * (exact ? 2 : 1) +
           (small_m_path(M, K, exact) ? kGemmBf16MaxWorkspace : 0);
}

bool launch_linear(const float *a, int64_t lda, const uint16_t *w, int64_t ldw, float *c,
                   int64_t ldc, int M, int N, int K, bool exact, void *scratch,
                   size_t scratch_bytes, hipStream_t st)
{
    if (M < 0 || N < 0 || K < 0)
        return fail("linear: negative dimension");
    if (int64_t(M) * N == 0)
        return true;
    if (lda < K || ldw < K || ldc < N)
        return fail("linear: leading dimension smaller than the row length");
    const int64_t kp = padded_k(K);
    LtPlan *plan = nullptr;
    if (K > 0 && (ldw % 8) == 0 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0 &&
        (reinterpret_cast<uintptr_t>(c) & 15u) == 0 && (ldc % 4) == 0) {
        std::lock_guard<std::mutex> g(g_lt_mu);
        plan = lt_plan(M, N, K, kp, ldw, ldc);
    }
    if (!plan)  // exact f32 MFMA on the original values
        return launch_gemm(a, lda, w, true, ldw, c, ldc, M, N, K, st);
    if (!scratch || scratch_bytes < linear_scratch_bytes(M, K, exact) ||
        (reinterpret_cast<uintptr_t>(scratch) & 15u) != 0)
        return fail("linear: scratch smaller than linear_scratch_bytes() or not 16-byte aligned");
    // Large M, f32 modes: the kernel splits f32 A into its hi and lo terms in
    // registers, so the terms make no round trip through HBM; bit-identical to
    // the split + two-term product below.  256 x 256 tiles where they fill the
    // GPU, else 128 x 256.
    if (exact && gemm_f32a_supported(M, N, K, lda, ldw, ldc, a, w, c))
        return launch_gemm_f32a(a, lda, w, ldw, c, ldc, M, N, K, true, st);
    // One term (bf16 mode): the same kernel rounding A to bf16 in registers
    // beats the split pass + library product where N and K are at most 2048
    // (8192 x 2048 x 2048: 78.5 against 80.2 us, 8192 x 2048 x 1024: 45.4
    // against 50.0, 16384 x 2048 x 2048: 149.5 against 156.4).  Elsewhere the
    // split + library product stays: staging f32 rows doubles the A bytes,
    // and at larger N or K the kernel ran up to 34 % slower.
    if (!exact && N <= 2048 && K <= 2048 && gemm_f32a_supported(M, N, K, lda, ldw, ldc, a, w, c))
        return launch_gemm_f32a(a, lda, w, ldw, c, ldc, M, N, K, false, st);
    if (exact && gemm_large_f32a_supported(M, N, K, lda, ldw, ldc, a, w, c))
        return launch_gemm_large_f32a(a, lda, w, ldw, c, ldc, M, N, K, st);
    SplitArgs s;
    s.a = a;
    s.lda = lda;
    s.hi = static_cast<unsigned int *>(scratch);
    s.lo = exact ? reinterpret_cast<unsigned int *>(static_cast<char *>(scratch) +
                                                    round_up256(size_t(M) * kp * 2))
                 : nullptr;
    s.kp = kp;
    s.rs = kp;
    s.M = M;
    s.K = K;
    s.vec = (reinterpret_cast<uintptr_t>(a) & 15u) == 0 && lda % 4 == 0;
    s.total = int64_t(M) * kp / 8;
    const int64_t nblk = (s.total + 255) / 256;
    if (nblk > INT32_MAX)
        return fail("linear: problem too large for one launch");
    hipLaunchKernelGGL(split_kernel, dim3(unsigned(nblk)), dim3(256), 0, st, s);
    if (!hip_ok(hipGetLastError(), "split_kernel launch"))
        return false;
    // Small M: both terms in one product of the small-M kernel, its partials
    // after the terms in the scratch.
    const size_t terms = round_up256(size_t(M) * kp * 2) * (exact ? 2 : 1);
    if (small_m_path(M, K, exact)) {
        void *ws = static_cast<char *>(scratch) + terms;
        const size_t wsb = scratch_bytes - terms;
        const uint16_t *hi = reinterpret_cast<const uint16_t *>(s.hi);
        const uint16_t *lo = reinterpret_cast<const uint16_t *>(s.lo);
        if (gemm_bf16_supported(M, N, K, kp, ldw, ldc, hi, lo, w, c, wsb))
            return launch_gemm_bf16(hi, lo, kp, w, ldw, c, ldc, M, N, K, ws, wsb, st);
    }
    {
        const uint16_t *hi = reinterpret_cast<const uint16_t *>(s.hi);
        const uint16_t *lo = reinterpret_cast<const uint16_t *>(s.lo);
        if (exact && gemm_large_supported(M, N, K, 2, kp, ldw, ldc, hi, lo, w, c, 4))
            return launch_gemm_large(hi, lo, kp, w, ldw, c, ldc, M, N, K, kGemmOutF32, nullptr, 0,
                                     0, st);
    }
    std::lock_guard<std::mutex> g(g_lt_mu);
    if (!lt_matmul(plan, w, s.hi, c, 0.0f, st))
        return false;
    return !exact || lt_matmul(plan, w, s.lo, c, 1.0f, st);
}

bool linear_residual_supported(int S, int N, int K, const void *w, int64_t ldw, const float *x,
                               int64_t ldx)
{
    if (S <= 0 || N <= 0 || K <= 0 || ldw < K || ldx < N || (ldw % 8) != 0 || (ldx % 4) != 0 ||
        (reinterpret_cast<uintptr_t>(w) & 15u) != 0 || (reinterpret_cast<uintptr_t>(x) & 15u) != 0)
        return false;
    std::lock_guard<std::mutex> g(g_lt_mu);
    return lt_plan(S, N, K, padded_k(K), ldw, ldx, true) != nullptr;
}

bool launch_linear_residual(const float *a, int64_t lda, const uint16_t *w, int64_t ldw, float *x,
                            int64_t ldx, const float *gate, int64_t gate_stride, int B, int S, int N,
                            int K, void *scratch, size_t scratch_bytes, hipStream_t st)
{
    if (int64_t(B) * S * N == 0)
        return true;
    if (!linear_residual_supported(S, N, K, w, ldw, x, ldx))
        return fail("linear_residual: no bf16 GEMM with a per-channel scale for this shape");
    if ((reinterpret_cast<uintptr_t>(gate) & 3u) != 0)
        return fail("linear_residual: misaligned gate");
    const int M = B * S;
    const int64_t kp = padded_k(K);
    if (!scratch || scratch_bytes < linear_scratch_bytes(M, K, false) ||
        (reinterpret_cast<uintptr_t>(scratch) & 15u) != 0)
        return fail("linear_residual: scratch smaller than linear_scratch_bytes()");
    SplitArgs sa;
    sa.a = a;
    sa.lda = lda;
    sa.hi = static_cast<unsigned int *>(scratch);
    sa.lo = nullptr;
    sa.kp = kp;
    sa.rs = kp;
    sa.M = M;
    sa.K = K;
    sa.vec = (reinterpret_cast<uintptr_t>(a) & 15u) == 0 && lda % 4 == 0;
    sa.total = int64_t(M) * kp / 8;
    const int64_t nblk = (sa.total + 255) / 256;
    if (nblk > INT32_MAX)
        return fail("linear_residual: problem too large for one launch");
    hipLaunchKernelGGL(split_kernel, dim3(unsigned(nblk)), dim3(256), 0, st, sa);
    if (!hip_ok(hipGetLastError(), "split_kernel launch"))
        return false;
    return launch_linear_residual_terms(reinterpret_cast<const uint16_t *>(sa.hi), w, ldw, x, ldx,
                                        gate, gate_stride, B, S, N, K, st);
}

bool launch_linear_residual_terms(const uint16_t *hi, const uint16_t *w, int64_t ldw, float *x,
                                  int64_t ldx, const float *gate, int64_t gate_stride, int B,
                                  int S, int N, int K, hipStream_t st)
{
    if (int64_t(B) * S * N == 0)
        return true;
    if (!linear_residual_supported(S, N, K, w, ldw, x, ldx))
        return fail("linear_residual: no bf16 GEMM with a per-channel scale for this shape");
    if ((reinterpret_cast<uintptr_t>(gate) & 3u) != 0 || (reinterpret_cast<uintptr_t>(hi) & 15u) != 0)
        return fail("linear_residual: misaligned gate or terms");
    const int64_t kp = padded_k(K);
    std::lock_guard<std::mutex> g(g_lt_mu);
    LtPlan *plan = lt_plan(S, N, K, kp, ldw, ldx, true);
    // Per batch entry b: x_b = gate_b (.) (a_b W^T) + x_b, gate over the N
    // output channels.
    for (int b = 0; b < B; ++b) {
        const int64_t r0 = int64_t(b) * S;
        if (!lt_matmul(plan, w, hi + r0 * kp, x + r0 * ldx, 1.0f, st,
                       gate + int64_t(b) * gate_stride))
            return false;
    }
    return true;
}

}  // namespace anima_hip
