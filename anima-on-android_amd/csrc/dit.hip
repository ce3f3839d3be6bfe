// The Anima DiT around the attention path, on the device: NumpyDiT.forward
// (anima_rt/scripts/numpy_dit.py:82-130) with the residual stream resident in
// HBM from the patch embedding to the final layer, and the Euler flow-match
// sampler with classifier-free guidance (anima_rt/scripts/sampling.py:115-140)
// looping on the device.
//
// Per forward:
//   timestep_kernel   _numpy_timesteps (numpy_dit.py:39-46): [cos, sin] of
//                     sigma * exp(-ln(1e4) i / half), float32 like numpy;
//   gemv_kernel       every small-batch linear layer: the timestep MLP
//                     (numpy_dit.py:153-160) and all AdaLN modulation MLPs
//                     (numpy_dit.py:211-223, 171-180).  Their inputs depend on
//                     sigma only, so the 28 x 3 + 1 modulations run as two
//                     launches (first layers, then second layers plus the
//                     AdaLN-LoRA term) before the blocks;
//   launch_silu       anima_rt_run_silu (silu_kernel.h:9-17), from ops.hip;
//   patchify_kernel   _pad_to_patch_size + the zero padding-mask channel +
//                     _rearrange_patchify (numpy_dit.py:10-22, 92-95),
//                     written directly as the bf16 terms of the patch GEMM;
//   blocks            attention sub-layers (block.hip) and the MLP sub-layer
//                     below: LN + modulate -> layer1 -> GELU -> layer2 ->
//                     gated residual (numpy_dit.py:249-253, 304-317);
//   gelu_terms_kernel anima_rt_run_gelu (gelu_kernel.h:13-23, exact erf form)
//                     fused with the split of its output into GEMM terms;
//   final layer       LN + modulate (2 chunks) -> linear (numpy_dit.py:186-201);
//   unpatchify_kernel _rearrange_unpatchify + crop (numpy_dit.py:24-31, 128-129);
//   cfg_euler_kernel  sampler only: v = v_u + cfg (v_c - v_u), x += v dt.
// Linear layers over tokens run through linear.hip: the hand-written small-M
// kernel (gemm_bf16.hip) at M <= 1024, the large-M kernel (gemm_large.hip)
// for products of two term planes, hipBLASLt for the rest.  f32 mode feeds
// them exact hi + lo bf16 terms of the f32 activations, bf16 mode rounds the
// activations to bf16.  In the f32x3 mode at large M the self-attention's
// q/k/v product is the f32-activation kernel's fused form (gemm_f32a.hip),
// which writes the attention's prepared Q, K and V^T itself.
#include "common.h"

#include "anima_hip.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#pragma clang fp contract(off)

namespace anima_hip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kMaxBatch = 4;
constexpr int kPatch = 2;         // spatial patch (ps); one frame per patch (pt = 1)
constexpr int kAdaHidden = 256;   // hidden width of every AdaLN MLP (numpy_dit.py:176, 216)

size_t round_up256(size_t n) { return (n + 255) / 256 * 256; }
bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

__device__ __forceinline__ unsigned int pack_pair(float x, float y)
{
    return __builtin_bit_cast(unsigned int, __builtin_convertvector(f32x2{x, y}, bf16x2));
}

// hi/lo bf16 terms of 8 consecutive values (lo may be null).
__device__ __forceinline__ void store_terms8(const float (&v)[8], unsigned int *hi,
                                             unsigned int *lo)
{
    unsigned int h[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        h[e] = pack_pair(v[2 * e], v[2 * e + 1]);
        // v - hi is exact in f32 (hi holds the leading bits of v).
        l[e] = pack_pair(v[2 * e] - __uint_as_float(h[e] << 16),
                         v[2 * e + 1] - __uint_as_float(h[e] & 0xFFFF0000u));
    }
    *reinterpret_cast<uint4 *>(hi) = uint4{h[0], h[1], h[2], h[3]};
    if (lo)
        *reinterpret_cast<uint4 *>(lo) = uint4{l[0], l[1], l[2], l[3]};
}

// ---- timestep features -------------------------------------------------
struct TimestepArgs {
    float sigma[kMaxBatch];
    // When set, every batch entry takes sigma_dev[*step] instead (the
    // sampler's per-step value, read on the device so that one captured
    // step serves every step).
    const float *sigma_dev;
    const int *step;
    float *out;  // [B][D]
    int D;
};

__global__ __launch_bounds__(256) void timestep_kernel(TimestepArgs a)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int b = blockIdx.y;
    if (i >= a.D)
        return;
    const int half = a.D / 2;
    const int j = i < half ? i : i - half;
    // exponent = -log(10000) * arange(half, float32) / float(half), in float32.
    const float e = (-9.21034037197618f * float(j)) / float(half);
    const float sigma = a.sigma_dev ? a.sigma_dev[*a.step] : a.sigma[b];
    const float arg = sigma * expf(e);
    a.out[int64_t(b) * a.D + i] = i < half ? cosf(arg) : sinf(arg);
}

// ---- small-batch linear layers -------------------------------------------
// y[b][n] = sum_k x[b][k] W[n][k] (+ add[b][n]) for b < B <= kMaxBatch, one
// job per blockIdx.y.  L lanes share an output row: lane lr takes the 16-byte
// chunks lr, lr + L, ... of W's row, then the L partial sums combine by
// butterfly.  All jobs of a launch share K (a multiple of 8).
struct GemvJob {
    const uint16_t *w;  // [N][K] bf16 bits
    const float *x;     // row b at x + b*ldx
    float *y;           // row b at y + b*ldy
    const float *add;   // row b at add + b*ld_add, or null
    int64_t ldx, ldy, ld_add;
    int N;
};

template <int L>
__global__ __launch_bounds__(256) void gemv_kernel(const GemvJob *jobs, int B, int K)
{
    constexpr int R = 256 / L;
    const GemvJob j = jobs[blockIdx.y];
    const int r = threadIdx.x / L, lr = threadIdx.x % L;
    const int n = blockIdx.x * R + r;
    if (n >= j.N)
        return;  // whole L-lane group
    float acc[kMaxBatch] = {0.f, 0.f, 0.f, 0.f};
    const uint16_t *wr = j.w + int64_t(n) * K;
    for (int c = lr; c < K / 8; c += L) {
        const uint4 wv = *reinterpret_cast<const uint4 *>(wr + 8 * c);
        const float w8[8] = {__uint_as_float(wv.x << 16), __uint_as_float(wv.x & 0xFFFF0000u),
                             __uint_as_float(wv.y << 16), __uint_as_float(wv.y & 0xFFFF0000u),
                             __uint_as_float(wv.z << 16), __uint_as_float(wv.z & 0xFFFF0000u),
                             __uint_as_float(wv.w << 16), __uint_as_float(wv.w & 0xFFFF0000u)};
#pragma unroll
        for (int b = 0; b < kMaxBatch; ++b) {
            if (b < B) {
                const float *xb = j.x + b * j.ldx + 8 * c;
                const f32x4 x0 = *reinterpret_cast<const f32x4 *>(xb);
                const f32x4 x1 = *reinterpret_cast<const f32x4 *>(xb + 4);
                acc[b] += ((w8[0] * x0.x + w8[1] * x0.y) + (w8[2] * x0.z + w8[3] * x0.w)) +
                          ((w8[4] * x1.x + w8[5] * x1.y) + (w8[6] * x1.z + w8[7] * x1.w));
            }
        }
    }
#pragma unroll
    for (int off = L / 2; off > 0; off >>= 1) {
#pragma unroll
        for (int b = 0; b < kMaxBatch; ++b)
            acc[b] += __shfl_xor(acc[b], off);
    }
    if (lr == 0) {
#pragma unroll
        for (int b = 0; b < kMaxBatch; ++b) {
            if (b < B)
                j.y[b * j.ldy + n] = acc[b] + (j.add ? j.add[b * j.ld_add + n] : 0.0f);
        }
    }
}

// ---- GELU, written as GEMM terms ------------------------------------------
// g = x * 0.5 * (1 + erf(x / sqrt(2))) of h [M][N] (N % 8 == 0) into hi/lo
// rows of N bf16.
struct GeluArgs {
    const void *h;  // f32, or bf16 (H_BF16), rows of N
    unsigned int *hi, *lo;
    int64_t n8;     // M * N / 8
    int64_t row8;   // N / 8
    int64_t tld;    // term row stride (elements): N, or 2N for [hi | lo] rows
};

template <bool H_BF16>
__global__ __launch_bounds__(256) void gelu_terms_kernel(GeluArgs a)
{
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= a.n8)
        return;
    float x[8];
    if (H_BF16) {
        const uint4 v = reinterpret_cast<const uint4 *>(a.h)[i];
        const unsigned int w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[2 * e] = __uint_as_float(w4[e] << 16);
            x[2 * e + 1] = __uint_as_float(w4[e] & 0xFFFF0000u);
        }
    } else {
        const float *h = static_cast<const float *>(a.h);
        const f32x4 u = *reinterpret_cast<const f32x4 *>(h + 8 * i);
        const f32x4 w = *reinterpret_cast<const f32x4 *>(h + 8 * i + 4);
        x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w;
        x[4] = w.x; x[5] = w.y; x[6] = w.z; x[7] = w.w;
    }
    float g[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
        g[e] = x[e] * 0.5f * (1.0f + erff(x[e] * 0.70710678118654752440f));
    const int64_t m = i / a.row8;
    const int64_t off = (m * a.tld + 8 * (i - m * a.row8)) / 2;
    store_terms8(g, a.hi + off, a.lo ? a.lo + off : nullptr);
}

// ---- patch embedding input ------------------------------------------------
// Token m = ((b*T + t)*Hp + h)*Wp + w, feature k = ch*4 + 2*dy + dx (ch < C
// latent channels, ch == C the zero padding-mask channel), value
// x[b][ch][t][2h+dy][2w+dx], zero past the unpadded Hi x Wi.  Rows of kp
// (padded K) bf16 terms.
struct PatchArgs {
    const float *x;
    int64_t xb;  // batch stride of x (0: every batch entry reads entry 0)
    unsigned int *hi, *lo;
    int64_t kp, M;
    int C, T, Hi, Wi, Hp, Wp, K;
};

__global__ __launch_bounds__(256) void patchify_kernel(PatchArgs a)
{
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    const int64_t chunks = a.kp / 8;
    if (i >= a.M * chunks)
        return;
    const int64_t m = i / chunks;
    const int k0 = int(i - m * chunks) * 8;
    const int w = int(m % a.Wp);
    const int h = int((m / a.Wp) % a.Hp);
    const int t = int((m / (int64_t(a.Wp) * a.Hp)) % a.T);
    const int b = int(m / (int64_t(a.Wp) * a.Hp * a.T));
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int k = k0 + e;
        const int ch = k >> 2, y = 2 * h + ((k >> 1) & 1), xx = 2 * w + (k & 1);
        v[e] = (k < a.K && ch < a.C && y < a.Hi && xx < a.Wi)
                   ? a.x[b * a.xb + ((int64_t(ch) * a.T + t) * a.Hi + y) * a.Wi + xx]
                   : 0.0f;
    }
    store_terms8(v, a.hi + (m * a.kp + k0) / 2, a.lo ? a.lo + (m * a.kp + k0) / 2 : nullptr);
}

// ---- final-layer output -----------------------------------------------------
// out[b][c][t][y][x] = f[token(b, t, y/2, x/2)][((y%2)*2 + x%2)*Cout + c],
// cropped to Hi x Wi.
struct UnpatchArgs {
    const float *f;
    float *out;
    int64_t n;  // B*Cout*T*Hi*Wi
    int Cout, T, Hi, Wi, Hp, Wp;
};

__global__ __launch_bounds__(256) void unpatchify_kernel(UnpatchArgs a)
{
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= a.n)
        return;
    const int x = int(i % a.Wi);
    const int y = int((i / a.Wi) % a.Hi);
    const int t = int((i / (int64_t(a.Wi) * a.Hi)) % a.T);
    const int64_t bc = i / (int64_t(a.Wi) * a.Hi * a.T);
    const int c = int(bc % a.Cout);
    const int b = int(bc / a.Cout);
    const int64_t m = ((int64_t(b) * a.T + t) * a.Hp + (y >> 1)) * a.Wp + (x >> 1);
    a.out[i] = a.f[m * 4 * a.Cout + ((y & 1) * 2 + (x & 1)) * a.Cout + c];
}

// Sampler update of the latent x [C][Hi][Wi] from the two CFG branches'
// final-layer rows (batch entry 0 unconditional, 1 conditional).
struct EulerArgs {
    const float *f;
    float *x;
    int64_t n, S;  // C*Hi*Wi; tokens per branch
    int Cout, Hi, Wi, Wp;
    float cfg;
    // dt = sigmas[step + 1] - sigmas[step], rounded once from the exact
    // difference like the reference's float64 subtraction.
    const float *sigmas;
    const int *step;
};

__global__ __launch_bounds__(256) void cfg_euler_kernel(EulerArgs a)
{
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= a.n)
        return;
    const int x = int(i % a.Wi);
    const int y = int((i / a.Wi) % a.Hi);
    const int c = int(i / (int64_t(a.Wi) * a.Hi));
    const int64_t m = int64_t(y >> 1) * a.Wp + (x >> 1);
    const int col = ((y & 1) * 2 + (x & 1)) * a.Cout + c;
    const float vu = a.f[m * 4 * a.Cout + col];
    const float vc = a.f[(a.S + m) * 4 * a.Cout + col];
    const float v = vu + a.cfg * (vc - vu);
    const int st = *a.step;
    const float dt = float(double(a.sigmas[st + 1]) - double(a.sigmas[st]));
    a.x[i] = a.x[i] + v * dt;
}

// The sampler's device step counter: set to `value`, or advanced by one.
__global__ void step_kernel(int *step, int value, int advance)
{
    if (threadIdx.x == 0 && blockIdx.x == 0)
        *step = advance ? *step + 1 : value;
}

// bf16 bit patterns -> f32 (the reference's widening of norm weights).
__global__ __launch_bounds__(256) void widen_kernel(const uint16_t *in, float *out, int64_t n)
{
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i < n)
        out[i] = __uint_as_float(uint32_t(in[i]) << 16);
}

// dst row n = reps copies of src row n, each zero-padded from K to kp
// elements (kp % 8 == 0): one thread per 8 destination elements.
struct RepArgs {
    const uint16_t *src;
    uint16_t *dst;
    int64_t ld_src, ld_dst, rows;
    int K, kp, reps;
};

__global__ __launch_bounds__(256) void rep_rows_kernel(RepArgs a)
{
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    const int64_t per_row = int64_t(a.reps) * a.kp / 8;
    if (i >= a.rows * per_row)
        return;
    const int64_t n = i / per_row;
    const int col = int(i - n * per_row) * 8;
    const int k0 = col % a.kp;
    unsigned short v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
        v[e] = k0 + e < a.K ? a.src[n * a.ld_src + k0 + e] : 0;
    *reinterpret_cast<uint4 *>(a.dst + n * a.ld_dst + col) =
        uint4{v[0] | (unsigned(v[1]) << 16), v[2] | (unsigned(v[3]) << 16),
              v[4] | (unsigned(v[5]) << 16), v[6] | (unsigned(v[7]) << 16)};
}

unsigned grid1(int64_t n) { return unsigned((n + 255) / 256); }

bool launch_gemv(const GemvJob *jobs, int njobs, int maxN, int B, int K, hipStream_t st)
{
    if (njobs == 0)
        return true;
    if (K % 8 || B < 1 || B > kMaxBatch)
        return fail("gemv: K must be a multiple of 8 and the batch at most 4");
    const int L = K >= 512 ? 64 : K >= 256 ? 32 : K >= 128 ? 16 : 8;
    const unsigned gx = unsigned((int64_t(maxN) * L + 255) / 256);
    const dim3 grid(gx, unsigned(njobs));
    switch (L) {
    case 64: hipLaunchKernelGGL(gemv_kernel<64>, grid, dim3(256), 0, st, jobs, B, K); break;
    case 32: hipLaunchKernelGGL(gemv_kernel<32>, grid, dim3(256), 0, st, jobs, B, K); break;
    case 16: hipLaunchKernelGGL(gemv_kernel<16>, grid, dim3(256), 0, st, jobs, B, K); break;
    default: hipLaunchKernelGGL(gemv_kernel<8>, grid, dim3(256), 0, st, jobs, B, K); break;
    }
    return hip_ok(hipGetLastError(), "gemv_kernel launch");
}

}  // namespace

}  // namespace anima_hip

using namespace anima_hip;

namespace {

struct BlockWeights {
    const uint16_t *sa_q = nullptr, *sa_k = nullptr, *sa_v = nullptr, *sa_o = nullptr;
    const uint16_t *cx_q = nullptr, *cx_k = nullptr, *cx_v = nullptr, *cx_o = nullptr;
    const uint16_t *fc1 = nullptr, *fc2 = nullptr;
    const float *sa_qn = nullptr, *sa_kn = nullptr, *cx_qn = nullptr, *cx_kn = nullptr;
    const uint16_t *ada1[3] = {nullptr, nullptr, nullptr}, *ada2[3] = {nullptr, nullptr, nullptr};
    void *ctx_k = nullptr, *ctx_v = nullptr;  // cross-attention cache (owned)
    // GEMM-ready weights: q, k and v rows stacked into one [3*H*D] x ld_d
    // matrix (owned); in f32 mode every weight row repeated as [W | W] so a
    // layer is one product with [hi | lo] activation rows (owned), in bf16
    // mode the originals.
    const uint16_t *w_qkv = nullptr, *w_o = nullptr, *w_cq = nullptr, *w_co = nullptr;
    const uint16_t *w_fc1 = nullptr, *w_fc2 = nullptr;
};

}  // namespace

struct anima_hip_dit {
    anima_hip_dit_config cfg{};
    bool bf16 = false;          // activations of the linear layers rounded to bf16
    AttnMode attn = kAttnF32;   // attention arithmetic
    int device = 0;
    std::vector<BlockWeights> blk;
    const uint16_t *x_emb = nullptr;  // [D][kp_in] zero-padded copy (owned)
    const uint16_t *t1 = nullptr, *t2 = nullptr;
    const float *t_norm = nullptr;
    const uint16_t *fin_ada1 = nullptr, *fin_ada2 = nullptr, *fin_lin = nullptr;
    int kp_in = 0;                    // padded patch feature count
    int reps = 1;                     // activation terms per element: 2 (f32), 1 (bf16)
    int64_t ld_d = 0, ld_hd = 0, ld_hid = 0;  // term/weight row strides of D, H*D, hidden inputs
    // Per-forward vectors (sized for cfg.max_batch), owned.
    float *feat = nullptr, *h1 = nullptr, *h1s = nullptr, *emb = nullptr, *semb = nullptr;
    float *lora = nullptr, *m1 = nullptr, *mods = nullptr;
    GemvJob *jobs = nullptr;          // device table: t1, t2, layer-1 x n_ada, layer-2 x n_ada
    int n_ada = 0;
    std::vector<void *> owned;        // device allocations freed at destroy
    // Context caches: allocated for alloc_B x alloc_S; valid (a context is
    // set) only when ctx_B > 0, which set_context clears first and sets last.
    int alloc_B = 0, alloc_S = 0;
    int ctx_B = 0, ctx_S = 0;
    void *ctx_work = nullptr;
    size_t ctx_work_bytes = 0;
    // Sampler: the sigmas of a run on the device (capacity sig_cap), staged
    // through pinned host memory (reused once sig_ev has completed), the step
    // counter, and one captured Euler step (graph) for the buffers in
    // `graph_key`, replayed for every step after the first.
    float *sig_dev = nullptr, *sig_host = nullptr;
    int sig_cap = 0;
    hipEvent_t sig_ev = nullptr;
    // Recorded on the caller's stream after each run's last launch; the next
    // run's stream waits on it before it overwrites the sigmas and the step
    // counter, so runs on different streams follow one another on the device.
    hipEvent_t run_ev = nullptr;
    bool run_recorded = false;
    int *step_dev = nullptr;
    hipStream_t cap_stream = nullptr;
    hipGraphExec_t graph = nullptr;
    struct GraphKey {
        const void *latent, *freqs, *scratch, *sig;
        size_t scratch_bytes;
        int H, W;
        float cfg;
        unsigned gen;
        bool operator==(const GraphKey &o) const
        {
            return latent == o.latent && freqs == o.freqs && scratch == o.scratch &&
                   sig == o.sig && scratch_bytes == o.scratch_bytes && H == o.H && W == o.W &&
                   cfg == o.cfg && gen == o.gen;
        }
    } graph_key{};
    unsigned gen = 0;  // advanced whenever the context caches move
};

namespace {

void dit_free(anima_hip_dit *d)
{
    if (!d)
        return;
    (void)hipDeviceSynchronize();
    for (void *p : d->owned)
        (void)hipFree(p);
    for (auto &b : d->blk) {
        if (b.ctx_k)
            (void)hipFree(b.ctx_k);
        if (b.ctx_v)
            (void)hipFree(b.ctx_v);
    }
    if (d->ctx_work)
        (void)hipFree(d->ctx_work);
    if (d->graph)
        (void)hipGraphExecDestroy(d->graph);
    if (d->cap_stream)
        (void)hipStreamDestroy(d->cap_stream);
    if (d->sig_dev)
        (void)hipFree(d->sig_dev);
    if (d->sig_host)
        (void)hipHostFree(d->sig_host);
    if (d->sig_ev)
        (void)hipEventDestroy(d->sig_ev);
    if (d->run_ev)
        (void)hipEventDestroy(d->run_ev);
    delete d;
}

template <typename T>
bool dev_alloc(anima_hip_dit *d, T *&p, size_t bytes, const char *what)
{
    void *v = nullptr;
    if (!hip_ok(hipMalloc(&v, std::max<size_t>(bytes, 256)), what))
        return false;
    d->owned.push_back(v);
    p = static_cast<T *>(v);
    return true;
}

std::string strip_net(const char *n)
{
    std::string s(n ? n : "");
    if (s.rfind("net.", 0) == 0)
        s = s.substr(4);
    return s;
}

// Token count of one batch entry and the patch grid of a T x H x W latent.
void grid_of(int T, int H, int W, int &Hp, int &Wp, int64_t &S)
{
    Hp = (H + kPatch - 1) / kPatch;
    Wp = (W + kPatch - 1) / kPatch;
    S = int64_t(T) * Hp * Wp;
}

// Arena regions of one sub-layer (kind 0 self-attention, 1 cross-attention,
// 2 MLP), 256-byte aligned, in order: activation terms, then
//   self:  qkv [M][3HD] f32, o [M][HD] f32, attention scratch, o's terms;
//   cross: q [M][HD] f32,    o [M][HD] f32, attention scratch, o's terms;
//   mlp:   h [M][hidden] (f32, bf16 in bf16 mode), GELU terms [M][ld_hid].
struct SubLayout {
    size_t terms, a, b, attn, lin, ws, total;
};

SubLayout sub_layout(const anima_hip_dit *d, int B, int64_t S, int kind)
{
    const anima_hip_dit_config &c = d->cfg;
    const size_t M = size_t(B) * S, HD = size_t(c.heads) * c.head_dim;
    SubLayout l{};
    l.terms = round_up256(M * size_t(d->ld_d) * 2);
    if (kind == 2) {
        l.a = round_up256(M * c.mlp_hidden * (d->bf16 ? 2 : 4));
        l.b = round_up256(M * size_t(d->ld_hid) * 2);
    } else {
        l.a = round_up256(M * HD * 4 * (kind == 0 ? 3 : 1));
        l.b = round_up256(M * HD * 4);
        l.attn = round_up256(kind == 0 ? attention_scratch_bytes(B, int(S), B, int(S), c.heads,
                                                                 c.head_dim, d->attn, false)
                                       : attention_scratch_bytes(B, int(S), std::max(d->ctx_B, 1),
                                                                 std::max(d->ctx_S, 1), c.heads,
                                                                 c.head_dim, d->attn, true));
        l.lin = round_up256(M * size_t(linear_terms_ld(int(HD))) * 2 * d->reps);
    }
    // Split-K partials of the small-M GEMM, right after lin (the bf16 output
    // projection hands launch_linear both as one scratch).
    l.ws = M <= 1024 ? kGemmBf16MaxWorkspace : 0;
    l.total = l.terms + l.a + l.b + l.attn + l.lin + l.ws;
    return l;
}

// Scratch regions of one forward, 256-byte aligned, in order.
struct DitScratch {
    size_t x, y, patch, f, arena, total;
};

DitScratch dit_scratch(const anima_hip_dit *d, int B, int64_t S)
{
    const anima_hip_dit_config &c = d->cfg;
    const int64_t M = int64_t(B) * S;
    DitScratch s{};
    s.x = round_up256(size_t(M) * c.dim * 4);
    // The pending output projection: one [M][D] plane, or up to 16 MiB of
    // the small-M GEMM's split-K partial planes, added by the next LayerNorm.
    s.y = std::max(s.x, M <= 1024 ? kGemmBf16MaxWorkspace : size_t(0));
    s.patch = round_up256(size_t(M) * d->kp_in * 2) * 2;
    s.f = round_up256(size_t(M) * 4 * c.out_channels * 4);
    const SubLayout self = sub_layout(d, B, S, 0), cross = sub_layout(d, B, S, 1),
                    mlp = sub_layout(d, B, S, 2);
    size_t arena = std::max(self.total, std::max(cross.total, mlp.total));
    arena = std::max(arena, round_up256(size_t(M) * linear_terms_ld(c.dim) * 2) * 2);
    s.arena = round_up256(arena);
    s.total = s.x + s.y + s.patch + s.f + s.arena;
    return s;
}

bool check_cfg(const anima_hip_dit_config &c)
{
    if (c.dim <= 0 || c.dim % 8 || c.dim > 4096 || c.blocks < 0 || c.heads <= 0 ||
        c.head_dim <= 0 || (c.heads * c.head_dim) % 8 || c.mlp_hidden <= 0 ||
        c.mlp_hidden % 8 || c.ctx_dim <= 0 || c.ctx_dim % 8 || c.in_channels <= 0 ||
        c.out_channels <= 0 || c.max_batch < 1 || c.max_batch > kMaxBatch)
        return fail("dit: invalid configuration (widths multiples of 8, model width <= 4096, "
                    "max_batch 1..4)");
    return true;
}

// x += gate * y of the pending sub-layer (when pend_y; y the sum of
// pend_parts [M][D] planes), then LayerNorm + modulate into activation terms:
// [hi | lo] rows in f32 mode, hi rows in bf16 mode (row stride ld_d either
// way).
bool dit_norm(const anima_hip_dit *d, float *x, const float *mod, const float *pend_y,
              int pend_parts, const float *pend_mod, uint16_t *terms, int64_t M, int S,
              hipStream_t st)
{
    const int D = d->cfg.dim;
    uint16_t *lo = d->reps == 2 ? terms + linear_terms_ld(D) : nullptr;
    return launch_ln_modulate(x, D, mod, 3 * int64_t(D), terms, lo, M, S, D, 1e-6f, st, x, pend_y,
                              pend_y ? pend_mod + 2 * int64_t(D) : nullptr, 3 * int64_t(D),
                              d->ld_d, pend_parts);
}

// out [M][N] = terms . W^T for activation terms of row stride ld_t: [hi | lo]
// rows and [W | W] weight rows in f32 mode (a two-term product), hi rows in
// bf16 mode.  ws: the small-M GEMM's split-K partials.
bool dit_product(const anima_hip_dit *d, const uint16_t *terms, int64_t ld_t, const uint16_t *w,
                 int64_t ld_w, float *out, int N, int64_t M, void *ws, size_t ws_bytes,
                 hipStream_t st)
{
    if (d->reps == 2)
        return launch_linear_pair(terms, ld_t, int(ld_t / 2), w, ld_w, out, N, int(M), N, st, ws,
                                  ws_bytes);
    return launch_linear_terms(terms, nullptr, w, ld_w, out, N, int(M), N, int(ld_t), st, ws,
                               ws_bytes);
}

// The sub-layer's output projection y [M][N] = a . W^T for f32 activations a
// [M][K], left as *parts planes at y (y_bytes of room) for the next
// LayerNorm to add: split into terms in lin here, one product.  lin holds the
// terms and, right after them, ws_bytes of scratch.
bool dit_linear(const anima_hip_dit *d, const float *a, int K, const uint16_t *w, int64_t ld_w,
                float *y, size_t y_bytes, int *parts, int N, int64_t M, void *lin,
                size_t lin_bytes, size_t ws_bytes, hipStream_t st)
{
    if (d->reps == 2) {
        const uint16_t *t = launch_split_interleaved(a, K, int(M), K, lin, lin_bytes, st);
        return t && launch_linear_planes(t, 2 * linear_terms_ld(K), int(linear_terms_ld(K)), true,
                                         w, ld_w, y, y_bytes, int(M), N, parts, st);
    }
    *parts = 1;
    return launch_linear(a, K, w, ld_w, y, N, int(M), N, K, false, lin, lin_bytes + ws_bytes, st);
}

// The output projection of an attention sub-layer whose kernels wrote O as
// the projection's bf16 terms at t (attention_term_rows' layout), left as
// *parts planes at y like dit_linear's.
struct TermRows {
    int64_t ld, lo;  // row length and lo offset (0: hi only) in bf16 elements
};
TermRows attention_term_rows(const anima_hip_dit *d, int K)
{
    const int64_t kp = linear_terms_ld(K);
    return d->reps == 2 ? TermRows{2 * kp, kp} : TermRows{kp, 0};
}

bool dit_project_terms(const anima_hip_dit *d, const uint16_t *t, int K, const uint16_t *w,
                       int64_t ld_w, float *y, size_t y_bytes, int *parts, int N, int64_t M,
                       hipStream_t st)
{
    const TermRows tr = attention_term_rows(d, K);
    return launch_linear_planes(t, tr.ld, d->reps == 2 ? int(tr.lo) : K, d->reps == 2, w, ld_w,
                                y, y_bytes, int(M), N, parts, st);
}

// One sub-layer of block bw on the residual stream x (kind as sub_layout),
// after applying the pending residual (pend_parts planes at pend_y); its
// output projection goes to y as *y_parts planes (y_bytes of room).
bool dit_sublayer(const anima_hip_dit *d, const BlockWeights &bw, int kind, float *x,
                  const float *mod, const float *pend_y, int pend_parts, const float *pend_mod,
                  float *y, size_t y_bytes, int *y_parts, int B,
                  int64_t S, const float *freqs, void *arena, hipStream_t st)
{
    const anima_hip_dit_config &c = d->cfg;
    const int D = c.dim, HD = c.heads * c.head_dim;
    const int64_t M = int64_t(B) * S;
    const SubLayout l = sub_layout(d, B, S, kind);
    char *cur = static_cast<char *>(arena);
    uint16_t *terms = reinterpret_cast<uint16_t *>(cur);
    char *ra = cur + l.terms, *rb = ra + l.a, *rattn = rb + l.b, *rlin = rattn + l.attn;
    char *rws = rlin + l.lin;
    // Self-attention in the f32x3 mode where the 256 x 256 f32-activation
    // grid fills the GPU: LayerNorm + modulate leave f32 rows, and the fused
    // q/k/v product writes the attention's prepared Q, K and V itself (its
    // epilogue is the one-launch prologue), so no prologue pass reads the
    // projection back.  The three operands take the projection's region.
    // Against the library product on term rows plus the prologue this is
    // even in time (1024 x 1024 sampler step 67.41 / 67.49 -> 67.30 / 67.31
    // ms, interleaved): the hand-written product is slower than the library
    // by about what the prologue took.  In the f32 mode, whose prologue
    // writes f32 rows and no V^T (52 against 75 us), the steps measured even
    // within noise, and the library product stays.
    float *proj = reinterpret_cast<float *>(ra), *o = reinterpret_cast<float *>(rb);
    QkvPrep qp;
    const size_t op_bytes = size_t(M) * c.heads * c.head_dim * 4;
    const bool try_fused = kind == 0 && d->reps == 2 && d->attn == kAttnF32X3 &&
                           c.head_dim == 128;
    if (try_fused) {
        qp.qo = proj;
        qp.ko = reinterpret_cast<char *>(proj) + op_bytes;
        qp.vo = reinterpret_cast<char *>(proj) + 2 * op_bytes;
        qp.w[0] = bw.sa_qn;
        qp.w[1] = bw.sa_kn;
        qp.freqs = freqs;
        qp.B = B;
        qp.S = int(S);
        qp.H = c.heads;
        qp.mode = d->attn;
    }
    const bool fused_qkv = try_fused &&
                           gemm_f32a_qkv_supported(reinterpret_cast<const float *>(terms), D,
                                                   bw.w_qkv, d->ld_d, D, qp);
    if (fused_qkv) {
        if (!launch_ln_modulate(x, D, mod, 3 * int64_t(D), nullptr, nullptr, M, int(S), D, 1e-6f,
                                st, x, pend_y, pend_y ? pend_mod + 2 * int64_t(D) : nullptr,
                                3 * int64_t(D), 0, pend_parts, reinterpret_cast<float *>(terms)))
            return false;
    } else if (!dit_norm(d, x, mod, pend_y, pend_parts, pend_mod, terms, M, int(S), st)) {
        return false;
    }
    if (kind == 2) {  // NumpyMLP (numpy_dit.py:304-317)
        const int hid = c.mlp_hidden;
        const bool ok1 = d->bf16 ? launch_linear_terms_bf16out(terms, bw.w_fc1, d->ld_d,
                                                               reinterpret_cast<uint16_t *>(ra),
                                                               hid, int(M), hid, D, st)
                                 : dit_product(d, terms, d->ld_d, bw.w_fc1, d->ld_d,
                                               reinterpret_cast<float *>(ra), hid, M, rws, l.ws,
                                               st);
        if (!ok1)
            return false;
        GeluArgs ga;
        ga.h = ra;
        ga.hi = reinterpret_cast<unsigned int *>(rb);
        ga.lo = d->reps == 2 ? ga.hi + linear_terms_ld(hid) / 2 : nullptr;
        ga.n8 = M * hid / 8;
        ga.row8 = hid / 8;
        ga.tld = d->ld_hid;
        if (d->bf16)
            hipLaunchKernelGGL(gelu_terms_kernel<true>, dim3(grid1(ga.n8)), dim3(256), 0, st, ga);
        else
            hipLaunchKernelGGL(gelu_terms_kernel<false>, dim3(grid1(ga.n8)), dim3(256), 0, st, ga);
        return hip_ok(hipGetLastError(), "gelu_terms_kernel launch") &&
               launch_linear_planes(reinterpret_cast<const uint16_t *>(rb), d->ld_hid,
                                    int(d->ld_hid / d->reps), d->reps == 2, bw.w_fc2, d->ld_hid,
                                    y, y_bytes, int(M), D, y_parts, st);
    }
    // NumpyAttention.forward (numpy_dit.py:268-297): self-attention projects
    // q, k and v in one product; cross-attention projects q and reads the
    // block's context cache.
    AttnInputs in;
    in.B = B;
    in.S_q = int(S);
    in.H = c.heads;
    in.D = c.head_dim;
    in.eps = 1e-6f;
    in.mode = d->attn;
    in.out = o;
    if (fused_qkv) {
        if (!launch_gemm_f32a_qkv(reinterpret_cast<const float *>(terms), D, bw.w_qkv, d->ld_d, D,
                                  qp, st))
            return false;
        in.q_prep = qp.qo;
        in.k_prep = qp.ko;
        in.v_prep = qp.vo;
        in.Bk = B;
        in.S_kv = int(S);
    } else if (kind == 0) {
        if (!dit_product(d, terms, d->ld_d, bw.w_qkv, d->ld_d, proj, 3 * HD, M, rws, l.ws, st))
            return false;
        in.q = proj;
        in.k = proj + HD;
        in.v = proj + 2 * HD;
        in.ld_q = in.ld_kv = 3 * int64_t(HD);
        in.q_norm_w = bw.sa_qn;
        in.k_norm_w = bw.sa_kn;
        in.freqs = freqs;
        in.Bk = B;
        in.S_kv = int(S);
    } else {
        if (!dit_product(d, terms, d->ld_d, bw.w_cq, d->ld_d, proj, HD, M, rws, l.ws, st))
            return false;
        in.q = proj;
        in.q_norm_w = bw.cx_qn;
        in.k_prep = bw.ctx_k;
        in.v_prep = bw.ctx_v;
        in.Bk = d->ctx_B;
        in.S_kv = d->ctx_S;
    }
    const uint16_t *wo = kind == 0 ? bw.w_o : bw.w_co;
    if (c.head_dim != 128)  // the generic f32 kernel writes f32 O only
        return run_attention(in, rattn, st) &&
               dit_linear(d, o, HD, wo, d->ld_hd, y, y_bytes, y_parts, D, M, rlin, l.lin, l.ws,
                          st);
    // O straight into output_proj's bf16 terms: no split pass.
    const TermRows tr = attention_term_rows(d, HD);
    uint16_t *ot = reinterpret_cast<uint16_t *>(rlin);
    in.out = nullptr;
    in.out_t = ot;
    in.ld_t = tr.ld;
    in.lo_t = tr.lo;
    return run_attention(in, rattn, st) &&
           dit_project_terms(d, ot, HD, wo, d->ld_hd, y, y_bytes, y_parts, D, M, st);
}

// The forward pass on B batch entries of the latent x ([B][C][T][H][W] with
// batch stride xb) at noise levels sigma[B]; the final layer's token rows land
// in the `f` region of the scratch (returned through f_out).
bool dit_run(anima_hip_dit *d, const float *x, int64_t xb, const float *sigma, int B, int T,
             int H, int W, const float *freqs, void *scratch, size_t scratch_bytes,
             hipStream_t st, float **f_out, const float *sigma_dev = nullptr,
             const int *step_dev = nullptr)
{
    const anima_hip_dit_config &c = d->cfg;
    if (B < 1 || B > c.max_batch)
        return fail("dit: batch must be in 1..max_batch");
    if (T <= 0 || H <= 0 || W <= 0)
        return fail("dit: latent dimensions must be positive");
    if (!x || !sigma || (!freqs && c.blocks > 0))
        return fail("dit: null pointer");
    if (c.blocks > 0 && d->ctx_B == 0)
        return fail("dit: no text context set (anima_hip_dit_set_context_dev)");
    if (c.blocks > 0 && d->ctx_B != 1 && d->ctx_B != B)
        return fail("dit: the context batch must be 1 or the forward batch");
    int Hp, Wp;
    int64_t S;
    grid_of(T, H, W, Hp, Wp, S);
    const int64_t M = int64_t(B) * S;
    if (M > INT32_MAX / 8)
        return fail("dit: too many tokens");
    const DitScratch s = dit_scratch(d, B, S);
    if (!scratch || scratch_bytes < s.total || !aligned16(scratch))
        return fail("dit: scratch smaller than anima_hip_dit_scratch_bytes() or not 16-byte "
                    "aligned");
    char *base = static_cast<char *>(scratch);
    float *xr = reinterpret_cast<float *>(base);
    float *yp = reinterpret_cast<float *>(base + s.x);  // pending sub-layer output
    uint16_t *phi = reinterpret_cast<uint16_t *>(base + s.x + s.y);
    uint16_t *plo = d->bf16 ? nullptr : phi + (s.patch / 2) / 2;
    float *f = reinterpret_cast<float *>(base + s.x + s.y + s.patch);
    void *arena = base + s.x + s.y + s.patch + s.f;
    const int D = c.dim;

    // Timestep embedding, its MLP (the AdaLN-LoRA term), the normalised
    // embedding and every AdaLN modulation of this forward.
    TimestepArgs ta;
    for (int b = 0; b < kMaxBatch; ++b)
        ta.sigma[b] = b < B ? sigma[b] : 0.0f;
    ta.sigma_dev = sigma_dev;
    ta.step = step_dev;
    ta.out = d->feat;
    ta.D = D;
    hipLaunchKernelGGL(timestep_kernel, dim3(grid1(D), unsigned(B)), dim3(256), 0, st, ta);
    if (!hip_ok(hipGetLastError(), "timestep_kernel launch"))
        return false;
    RowProblem rp{};
    rp.x = d->feat;
    rp.out = d->emb;
    rp.w = d->t_norm;
    rp.xs = rp.os = Strides{D, D, D};
    rp.B = B;
    rp.S = 1;
    rp.H = 1;
    rp.D = D;
    rp.eps = 1e-6f;
    rp.norm = true;
    if (!launch_gemv(d->jobs, 1, D, B, D, st) || !launch_silu(d->h1, d->h1s, int64_t(B) * D, st) ||
        !launch_gemv(d->jobs + 1, 1, 3 * D, B, D, st) || !launch_rows(rp, st) ||
        !launch_silu(d->emb, d->semb, int64_t(B) * D, st) ||
        !launch_gemv(d->jobs + 2, d->n_ada, kAdaHidden, B, D, st) ||
        !launch_gemv(d->jobs + 2 + d->n_ada, d->n_ada, 3 * D, B, kAdaHidden, st))
        return false;

    // Patch embedding into the residual stream.
    PatchArgs pa;
    pa.x = x;
    pa.xb = xb;
    pa.hi = reinterpret_cast<unsigned int *>(phi);
    pa.lo = reinterpret_cast<unsigned int *>(plo);
    pa.kp = d->kp_in;
    pa.M = M;
    pa.C = c.in_channels;
    pa.T = T;
    pa.Hi = H;
    pa.Wi = W;
    pa.Hp = Hp;
    pa.Wp = Wp;
    pa.K = (c.in_channels + 1) * kPatch * kPatch;
    hipLaunchKernelGGL(patchify_kernel, dim3(grid1(M * (d->kp_in / 8))), dim3(256), 0, st, pa);
    if (!hip_ok(hipGetLastError(), "patchify_kernel launch") ||
        !launch_linear_terms(phi, plo, d->x_emb, d->kp_in, xr, D, int(M), D, d->kp_in, st))
        return false;

    // The blocks (numpy_dit.py:232-253).  Each sub-layer writes its output
    // projection to yp as one GEMM over all B*S rows; the next sub-layer's
    // (or the final layer's) LayerNorm pass applies x += gate * yp first.
    const int64_t mod_stride = int64_t(c.max_batch) * 3 * D;  // one modulation's rows
    const float *pend_mod = nullptr;                           // modulation owning yp
    int pend_parts = 1;                                        // planes of yp
    for (int i = 0; i < c.blocks; ++i) {
        for (int kind = 0; kind < 3; ++kind) {
            const float *mod = d->mods + (3 * i + kind) * mod_stride;
            int parts = 1;
            if (!dit_sublayer(d, d->blk[i], kind, xr, mod, pend_mod ? yp : nullptr, pend_parts,
                              pend_mod, yp, s.y, &parts, B, S, freqs, arena, st))
                return false;
            pend_mod = mod;
            pend_parts = parts;
        }
    }

    // Final layer: LN + modulate (shift, scale) and the output linear.
    uint16_t *thi = static_cast<uint16_t *>(arena);
    const size_t tbytes = round_up256(size_t(M) * linear_terms_ld(D) * 2);
    uint16_t *tlo = d->bf16 ? nullptr : thi + tbytes / 2;
    const float *fmod = d->mods + int64_t(3 * c.blocks) * mod_stride;
    if (!launch_ln_modulate(xr, D, fmod, 3 * int64_t(D), thi, tlo, M, int(S), D, 1e-6f, st, xr,
                            pend_mod ? yp : nullptr,
                            pend_mod ? pend_mod + 2 * int64_t(D) : nullptr, 3 * int64_t(D), 0,
                            pend_parts) ||
        !launch_linear_terms(thi, tlo, d->fin_lin, D, f, 4 * c.out_channels, int(M),
                             4 * c.out_channels, D, st))
        return false;
    *f_out = f;
    return true;
}

}  // namespace

extern "C" {

void anima_hip_dit_default_config(anima_hip_dit_config *cfg)
{
    if (!cfg)
        return;
    cfg->dim = 2048;
    cfg->blocks = 28;
    cfg->heads = 16;
    cfg->head_dim = 128;
    cfg->mlp_hidden = 8192;
    cfg->ctx_dim = 1024;
    cfg->in_channels = 16;
    cfg->out_channels = 16;
    cfg->max_batch = 2;
}

anima_hip_dit *anima_hip_dit_create(const anima_hip_dit_config *cfg, const char *const *names,
                                    const void *const *ptrs, const int *dtypes,
                                    const int64_t *shapes, int n, int mode)
{
    if (!cfg) {
        fail("dit_create: null configuration");
        return nullptr;
    }
    if (!check_cfg(*cfg))
        return nullptr;
    if (mode != ANIMA_HIP_F32 && mode != ANIMA_HIP_BF16 && mode != ANIMA_HIP_F32X3) {
        fail("dit_create: unknown mode " + std::to_string(mode));
        return nullptr;
    }
    if (mode != ANIMA_HIP_F32 && cfg->head_dim != 128) {
        fail("dit_create: the bf16 and f32x3 modes need head_dim 128");
        return nullptr;
    }
    if (n < 0 || (n > 0 && (!names || !ptrs || !dtypes || !shapes))) {
        fail("dit_create: null weight table");
        return nullptr;
    }
    if (!device_ready())
        return nullptr;
    auto *d = new anima_hip_dit;
    d->cfg = *cfg;
    d->bf16 = mode == ANIMA_HIP_BF16;
    d->attn = AttnMode(mode);
    (void)hipGetDevice(&d->device);
    const anima_hip_dit_config &c = d->cfg;
    const int D = c.dim, HD = c.heads * c.head_dim;
    const int K_in = (c.in_channels + 1) * kPatch * kPatch;
    d->blk.resize(c.blocks);
    const hipStream_t st = nullptr;

    // Look up every tensor the forward needs; linear weights must be bf16.
    auto find = [&](const std::string &name) -> int {
        for (int i = 0; i < n; ++i)
            if (strip_net(names[i]) == name)
                return i;
        return -1;
    };
    std::string err;
    auto shape_ok = [&](int i, const std::string &name, int64_t rows, int64_t cols) {
        if (shapes[2 * i] == rows && shapes[2 * i + 1] == cols)
            return true;
        if (err.empty())
            err = "dit_create: " + name + " has shape [" + std::to_string(shapes[2 * i]) + ", " +
                  std::to_string(shapes[2 * i + 1]) + "], expected [" + std::to_string(rows) +
                  ", " + std::to_string(cols) + "]";
        return false;
    };
    auto lin = [&](const std::string &name, int64_t rows, int64_t cols) -> const uint16_t * {
        const int i = find(name);
        if (i < 0 || !ptrs[i]) {
            if (err.empty())
                err = "dit_create: missing weight " + name;
            return nullptr;
        }
        if (!shape_ok(i, name, rows, cols))
            return nullptr;
        if (dtypes[i] != ANIMA_HIP_DTYPE_BF16) {
            if (err.empty())
                err = "dit_create: linear weight " + name + " must be BF16";
            return nullptr;
        }
        if (!aligned16(ptrs[i])) {
            if (err.empty())
                err = "dit_create: weight " + name + " is not 16-byte aligned";
            return nullptr;
        }
        return static_cast<const uint16_t *>(ptrs[i]);
    };
    auto norm = [&](const std::string &name, int len) -> const float * {
        const int i = find(name);
        if (i < 0 || !ptrs[i]) {
            if (err.empty())
                err = "dit_create: missing weight " + name;
            return nullptr;
        }
        if (!shape_ok(i, name, len, 0))
            return nullptr;
        if (dtypes[i] == ANIMA_HIP_DTYPE_F32) {
            if (!aligned16(ptrs[i])) {
                if (err.empty())
                    err = "dit_create: weight " + name + " is not 16-byte aligned";
                return nullptr;
            }
            return static_cast<const float *>(ptrs[i]);
        }
        if (dtypes[i] != ANIMA_HIP_DTYPE_BF16) {
            if (err.empty())
                err = "dit_create: norm weight " + name + " must be F32 or BF16";
            return nullptr;
        }
        float *w = nullptr;
        if (dev_alloc(d, w, size_t(len) * 4, "dit norm weight")) {
            hipLaunchKernelGGL(widen_kernel, dim3(grid1(len)), dim3(256), 0, st,
                               static_cast<const uint16_t *>(ptrs[i]), w, int64_t(len));
            if (hip_ok(hipGetLastError(), "widen_kernel launch"))
                return w;
        }
        if (err.empty())
            err = anima_hip_last_error();
        return nullptr;
    };
    static const char *kSub[3] = {"self_attn", "cross_attn", "mlp"};
    for (int i = 0; i < c.blocks; ++i) {
        BlockWeights &b = d->blk[i];
        const std::string p = "blocks." + std::to_string(i) + ".";
        b.sa_q = lin(p + "self_attn.q_proj.weight", HD, D);
        b.sa_k = lin(p + "self_attn.k_proj.weight", HD, D);
        b.sa_v = lin(p + "self_attn.v_proj.weight", HD, D);
        b.sa_o = lin(p + "self_attn.output_proj.weight", D, HD);
        b.sa_qn = norm(p + "self_attn.q_norm.weight", c.head_dim);
        b.sa_kn = norm(p + "self_attn.k_norm.weight", c.head_dim);
        b.cx_q = lin(p + "cross_attn.q_proj.weight", HD, D);
        b.cx_k = lin(p + "cross_attn.k_proj.weight", HD, c.ctx_dim);
        b.cx_v = lin(p + "cross_attn.v_proj.weight", HD, c.ctx_dim);
        b.cx_o = lin(p + "cross_attn.output_proj.weight", D, HD);
        b.cx_qn = norm(p + "cross_attn.q_norm.weight", c.head_dim);
        b.cx_kn = norm(p + "cross_attn.k_norm.weight", c.head_dim);
        b.fc1 = lin(p + "mlp.layer1.weight", c.mlp_hidden, D);
        b.fc2 = lin(p + "mlp.layer2.weight", D, c.mlp_hidden);
        for (int k = 0; k < 3; ++k) {
            b.ada1[k] = lin(p + "adaln_modulation_" + kSub[k] + ".1.weight", kAdaHidden, D);
            b.ada2[k] = lin(p + "adaln_modulation_" + kSub[k] + ".2.weight", 3 * D, kAdaHidden);
        }
    }
    const uint16_t *xe = lin("x_embedder.proj.1.weight", D, K_in);
    d->t1 = lin("t_embedder.1.linear_1.weight", D, D);
    d->t2 = lin("t_embedder.1.linear_2.weight", 3 * D, D);
    d->t_norm = norm("t_embedding_norm.weight", D);
    d->fin_ada1 = lin("final_layer.adaln_modulation.1.weight", kAdaHidden, D);
    d->fin_ada2 = lin("final_layer.adaln_modulation.2.weight", 2 * D, kAdaHidden);
    d->fin_lin = lin("final_layer.linear.weight", 4 * c.out_channels, D);
    if (!err.empty()) {
        fail(err);
        dit_free(d);
        return nullptr;
    }

    // x_embedder weight [D][K_in] copied into rows of kp_in zero-padded bf16.
    d->kp_in = int(linear_terms_ld(K_in));
    uint16_t *xp = nullptr;
    d->n_ada = 3 * c.blocks + 1;
    const int nj = 2 + 2 * d->n_ada;
    bool ok = dev_alloc(d, xp, size_t(D) * d->kp_in * 2, "dit x_embedder copy") &&
              hip_ok(hipMemsetAsync(xp, 0, size_t(D) * d->kp_in * 2, st), "hipMemset") &&
              hip_ok(hipMemcpy2DAsync(xp, size_t(d->kp_in) * 2, xe, size_t(K_in) * 2,
                                      size_t(K_in) * 2, size_t(D), hipMemcpyDeviceToDevice, st),
                     "x_embedder copy");
    d->x_emb = xp;
    const int MB = c.max_batch;
    ok = ok && dev_alloc(d, d->feat, size_t(MB) * D * 4, "dit vectors") &&
         dev_alloc(d, d->h1, size_t(MB) * D * 4, "dit vectors") &&
         dev_alloc(d, d->h1s, size_t(MB) * D * 4, "dit vectors") &&
         dev_alloc(d, d->emb, size_t(MB) * D * 4, "dit vectors") &&
         dev_alloc(d, d->semb, size_t(MB) * D * 4, "dit vectors") &&
         dev_alloc(d, d->lora, size_t(MB) * 3 * D * 4, "dit vectors") &&
         dev_alloc(d, d->m1, size_t(d->n_ada) * MB * kAdaHidden * 4, "dit vectors") &&
         dev_alloc(d, d->mods, size_t(d->n_ada) * MB * 3 * D * 4, "dit vectors") &&
         dev_alloc(d, d->jobs, size_t(nj) * sizeof(GemvJob), "dit job table") &&
         dev_alloc(d, d->step_dev, sizeof(int), "dit step counter");
    if (ok) {
        // The job table holds the batch strides of max_batch-sized buffers;
        // a forward on B <= max_batch rows uses the first B of each.
        std::vector<GemvJob> jobs(nj);
        jobs[0] = GemvJob{d->t1, d->feat, d->h1, nullptr, D, D, 0, D};
        jobs[1] = GemvJob{d->t2, d->h1s, d->lora, nullptr, D, 3 * D, 0, 3 * D};
        for (int a = 0; a < d->n_ada; ++a) {
            const bool fin = a == 3 * c.blocks;
            const uint16_t *w1 = fin ? d->fin_ada1 : d->blk[a / 3].ada1[a % 3];
            const uint16_t *w2 = fin ? d->fin_ada2 : d->blk[a / 3].ada2[a % 3];
            const int chunks = fin ? 2 : 3;
            // Modulation a: rows b of 3D floats at mods + (a * max_batch + b) * 3D,
            // i.e. the [B][3][D] (shift, scale, gate) layout of the sub-layers;
            // the final layer's two chunks fill the first 2D of each row.
            float *m1 = d->m1 + int64_t(a) * MB * kAdaHidden;
            float *mod = d->mods + int64_t(a) * MB * 3 * D;
            jobs[2 + a] = GemvJob{w1, d->semb, m1, nullptr, D, kAdaHidden, 0, kAdaHidden};
            jobs[2 + d->n_ada + a] =
                GemvJob{w2, m1, mod, d->lora, kAdaHidden, 3 * D, 3 * D, chunks * D};
        }
        ok = hip_ok(hipMemcpy(d->jobs, jobs.data(), jobs.size() * sizeof(GemvJob),
                              hipMemcpyHostToDevice),
                    "dit job table upload");
    }
    // GEMM-ready weights (see BlockWeights).
    const int kpD = int(linear_terms_ld(D)), kpHD = int(linear_terms_ld(HD));
    const int kpH = int(linear_terms_ld(c.mlp_hidden));
    d->reps = d->bf16 ? 1 : 2;
    d->ld_d = int64_t(d->reps) * kpD;
    d->ld_hd = int64_t(d->reps) * kpHD;
    d->ld_hid = int64_t(d->reps) * kpH;
    auto repeat = [&](const uint16_t *src, int64_t rows, int K, uint16_t *dst, int64_t ld_dst,
                      int kp) {
        RepArgs ra;
        ra.src = src;
        ra.dst = dst;
        ra.ld_src = K;
        ra.ld_dst = ld_dst;
        ra.rows = rows;
        ra.K = K;
        ra.kp = kp;
        ra.reps = d->reps;
        const int64_t n = rows * d->reps * kp / 8;
        hipLaunchKernelGGL(rep_rows_kernel, dim3(grid1(n)), dim3(256), 0, st, ra);
        return hip_ok(hipGetLastError(), "rep_rows_kernel launch");
    };
    auto prepared = [&](const uint16_t *src, int64_t rows, int K, int kp) -> const uint16_t * {
        if (d->reps == 1)
            return src;  // K == kp: the original rows are GEMM-ready
        uint16_t *w = nullptr;
        if (!dev_alloc(d, w, size_t(rows) * 2 * kp * 2, "dit repeated weight") ||
            !repeat(src, rows, K, w, 2 * int64_t(kp), kp))
            return nullptr;
        return w;
    };
    for (int i = 0; ok && i < c.blocks; ++i) {
        BlockWeights &b = d->blk[i];
        uint16_t *qkv = nullptr;
        ok = dev_alloc(d, qkv, size_t(3) * HD * d->ld_d * 2, "dit q/k/v weight") &&
             repeat(b.sa_q, HD, D, qkv, d->ld_d, kpD) &&
             repeat(b.sa_k, HD, D, qkv + int64_t(HD) * d->ld_d, d->ld_d, kpD) &&
             repeat(b.sa_v, HD, D, qkv + 2 * int64_t(HD) * d->ld_d, d->ld_d, kpD);
        b.w_qkv = qkv;
        b.w_o = ok ? prepared(b.sa_o, D, HD, kpHD) : nullptr;
        b.w_cq = b.w_o ? prepared(b.cx_q, HD, D, kpD) : nullptr;
        b.w_co = b.w_cq ? prepared(b.cx_o, D, HD, kpHD) : nullptr;
        b.w_fc1 = b.w_co ? prepared(b.fc1, c.mlp_hidden, D, kpD) : nullptr;
        b.w_fc2 = b.w_fc1 ? prepared(b.fc2, D, c.mlp_hidden, kpH) : nullptr;
        ok = ok && b.w_fc2;
    }
    ok = ok && hip_ok(hipStreamSynchronize(st), "dit_create");
    if (!ok) {
        dit_free(d);
        return nullptr;
    }
    return d;
}

void anima_hip_dit_destroy(anima_hip_dit *dit) { dit_free(dit); }

bool anima_hip_dit_set_context_dev(anima_hip_dit *d, const float *ctx, int Bc, int S_kv,
                                   void *stream)
{
    if (!d || !ctx)
        return fail("dit_set_context: null pointer");
    const anima_hip_dit_config &c = d->cfg;
    if (Bc < 1 || Bc > c.max_batch || S_kv <= 0)
        return fail("dit_set_context: context batch must be in 1..max_batch and S_kv positive");
    if (!aligned16(ctx))
        return fail("dit_set_context: context must be 16-byte aligned");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const int C = c.ctx_dim, H = c.heads, hd = c.head_dim, HD = H * hd;
    const int64_t M64 = int64_t(Bc) * S_kv;
    if (M64 > INT32_MAX / 8)
        return fail("dit_set_context: context too long");
    const int M = int(M64);
    // No context is valid until every block's cache is rebuilt.
    d->ctx_B = d->ctx_S = 0;
    if (Bc != d->alloc_B || S_kv != d->alloc_S) {
        // New cache shape: drain the device before the old caches go.
        if (!hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize"))
            return false;
        for (auto &b : d->blk) {
            if (b.ctx_k)
                (void)hipFree(b.ctx_k);
            if (b.ctx_v)
                (void)hipFree(b.ctx_v);
            b.ctx_k = b.ctx_v = nullptr;
        }
        d->alloc_B = d->alloc_S = 0;
        for (auto &b : d->blk) {
            if (!hip_ok(hipMalloc(&b.ctx_k, prepared_k_bytes(Bc, S_kv, H, hd, d->attn)),
                        "dit context K cache") ||
                !hip_ok(hipMalloc(&b.ctx_v, prepared_v_bytes(Bc, S_kv, H, hd, d->attn)),
                        "dit context V cache"))
                return false;
        }
        d->alloc_B = Bc;
        d->alloc_S = S_kv;
        ++d->gen;  // a captured sampler step holds the old cache addresses
    }
    const size_t proj = round_up256(size_t(M) * HD * 4);
    const size_t lin = round_up256(linear_scratch_bytes(M, C, !d->bf16));
    const size_t need = 2 * proj + lin;
    if (need > d->ctx_work_bytes) {
        if (!hip_ok(hipStreamSynchronize(st), "hipStreamSynchronize"))
            return false;
        if (d->ctx_work)
            (void)hipFree(d->ctx_work);
        d->ctx_work = nullptr;
        d->ctx_work_bytes = 0;
        if (!hip_ok(hipMalloc(&d->ctx_work, need), "dit context workspace"))
            return false;
        d->ctx_work_bytes = need;
    }
    float *kf = static_cast<float *>(d->ctx_work);
    float *vf = reinterpret_cast<float *>(static_cast<char *>(d->ctx_work) + proj);
    void *ls = static_cast<char *>(d->ctx_work) + 2 * proj;
    // Per block: K = k_norm(ctx Wk^T), V = ctx Wv^T (numpy_dit.py:277-286),
    // prepared once for every later forward.
    // f32 mode: K normalised in place in the cache, V projected straight
    // into it; bf16 / f32x3: projections in the workspace, then packed.
    const bool packed = d->attn != kAttnF32;
    for (auto &b : d->blk) {
        float *ko = packed ? kf : static_cast<float *>(b.ctx_k);
        float *vo = packed ? vf : static_cast<float *>(b.ctx_v);
        if (!launch_linear(ctx, C, b.cx_k, C, ko, HD, M, HD, C, !d->bf16, ls, lin, st) ||
            !launch_linear(ctx, C, b.cx_v, C, vo, HD, M, HD, C, !d->bf16, ls, lin, st))
            return false;
        const bool ok = packed ? prepare_kv(kf, vf, b.cx_kn, nullptr, b.ctx_k, b.ctx_v, Bc, S_kv,
                                            H, hd, 1e-6f, d->attn, st)
                               : prepare_kv(ko, nullptr, b.cx_kn, nullptr, b.ctx_k, nullptr, Bc,
                                            S_kv, H, hd, 1e-6f, kAttnF32, st);
        if (!ok)
            return false;
    }
    d->ctx_B = Bc;
    d->ctx_S = S_kv;
    return true;
}

size_t anima_hip_dit_scratch_bytes(const anima_hip_dit *d, int B, int T, int H, int W)
{
    if (!d || B < 0 || T < 0 || H < 0 || W < 0)
        return 0;
    int Hp, Wp;
    int64_t S;
    grid_of(T, H, W, Hp, Wp, S);
    return dit_scratch(d, B, S).total;
}

bool anima_hip_dit_forward_dev(anima_hip_dit *d, const float *x, int64_t x_batch_stride,
                               const float *sigma, int B, int T, int H, int W, const float *freqs,
                               float *out, void *scratch, size_t scratch_bytes, void *stream)
{
    if (!d || !out)
        return fail("dit_forward: null pointer");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    float *f = nullptr;
    if (!dit_run(d, x, x_batch_stride, sigma, B, T, H, W, freqs, scratch, scratch_bytes, st, &f))
        return false;
    int Hp, Wp;
    int64_t S;
    grid_of(T, H, W, Hp, Wp, S);
    UnpatchArgs ua;
    ua.f = f;
    ua.out = out;
    ua.Cout = d->cfg.out_channels;
    ua.T = T;
    ua.Hi = H;
    ua.Wi = W;
    ua.Hp = Hp;
    ua.Wp = Wp;
    ua.n = int64_t(B) * ua.Cout * T * H * W;
    hipLaunchKernelGGL(unpatchify_kernel, dim3(grid1(ua.n)), dim3(256), 0, st, ua);
    return hip_ok(hipGetLastError(), "unpatchify_kernel launch");
}

bool anima_hip_dit_euler_dev(anima_hip_dit *d, float *latent, const float *sigmas, int steps,
                             float cfg, int H, int W, const float *freqs, void *scratch,
                             size_t scratch_bytes, void *stream)
{
    if (!d || !latent || !sigmas)
        return fail("dit_euler: null pointer");
    if (steps < 0)
        return fail("dit_euler: negative step count");
    if (d->cfg.max_batch < 2 || d->ctx_B != 2)
        return fail("dit_euler: needs max_batch >= 2 and a context of 2 entries "
                    "(unconditional, conditional)");
    if (d->cfg.in_channels != d->cfg.out_channels)
        return fail("dit_euler: the latent needs as many output channels as input channels");
    if (steps == 0)
        return true;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    int Hp, Wp;
    int64_t S;
    grid_of(1, H, W, Hp, Wp, S);

    // The run's sigmas to the device, through pinned staging that the
    // previous run's copy has finished reading.
    const int n_sig = steps + 1;
    if (d->sig_ev && !hip_ok(hipEventSynchronize(d->sig_ev), "hipEventSynchronize"))
        return false;
    if (n_sig > d->sig_cap) {
        if (!hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize"))
            return false;
        if (d->sig_dev)
            (void)hipFree(d->sig_dev);
        if (d->sig_host)
            (void)hipHostFree(d->sig_host);
        d->sig_dev = d->sig_host = nullptr;
        d->sig_cap = 0;
        const int cap = std::max(n_sig, 64);
        if (!hip_ok(hipMalloc(&d->sig_dev, size_t(cap) * 4), "dit sigma buffer") ||
            !hip_ok(hipHostMalloc(&d->sig_host, size_t(cap) * 4, hipHostMallocDefault),
                    "dit sigma staging"))
            return false;
        d->sig_cap = cap;
        ++d->gen;  // the captured step holds the old sigma buffer
    }
    if (!d->sig_ev && !hip_ok(hipEventCreateWithFlags(&d->sig_ev, hipEventDisableTiming),
                              "hipEventCreate"))
        return false;
    if (!d->run_ev && !hip_ok(hipEventCreateWithFlags(&d->run_ev, hipEventDisableTiming),
                              "hipEventCreate"))
        return false;
    // The previous run (possibly on another stream) still reads the sigma
    // buffer and the step counter until its last replay ends.
    if (d->run_recorded && !hip_ok(hipStreamWaitEvent(st, d->run_ev, 0), "hipStreamWaitEvent"))
        return false;
    // From the upload on, every exit marks the end of this run's work on st.
    struct RunEnd {
        anima_hip_dit *d;
        hipStream_t st;
        ~RunEnd() { d->run_recorded = hipEventRecord(d->run_ev, st) == hipSuccess; }
    } run_end{d, st};
    std::copy(sigmas, sigmas + n_sig, d->sig_host);
    if (!hip_ok(hipMemcpyAsync(d->sig_dev, d->sig_host, size_t(n_sig) * 4,
                               hipMemcpyHostToDevice, st),
                "sigma upload") ||
        !hip_ok(hipEventRecord(d->sig_ev, st), "hipEventRecord"))
        return false;

    // One Euler step on stream s: the CFG batch [uncond, cond] of the same
    // latent at sigmas[step] (sampling.py:124-130), the update, and the
    // counter advanced for the next step.
    const float unused[2] = {0.0f, 0.0f};
    auto step = [&](hipStream_t s) {
        float *f = nullptr;
        if (!dit_run(d, latent, 0, unused, 2, 1, H, W, freqs, scratch, scratch_bytes, s, &f,
                     d->sig_dev, d->step_dev))
            return false;
        EulerArgs ea;
        ea.f = f;
        ea.x = latent;
        ea.S = S;
        ea.Cout = d->cfg.out_channels;
        ea.Hi = H;
        ea.Wi = W;
        ea.Wp = Wp;
        ea.n = int64_t(ea.Cout) * H * W;
        ea.cfg = cfg;
        ea.sigmas = d->sig_dev;
        ea.step = d->step_dev;
        hipLaunchKernelGGL(cfg_euler_kernel, dim3(grid1(ea.n)), dim3(256), 0, s, ea);
        hipLaunchKernelGGL(step_kernel, dim3(1), dim3(64), 0, s, d->step_dev, 0, 1);
        return hip_ok(hipGetLastError(), "cfg_euler_kernel launch");
    };
    hipLaunchKernelGGL(step_kernel, dim3(1), dim3(64), 0, st, d->step_dev, 0, 0);
    // The first step runs directly (it also creates every GEMM plan the
    // step needs); the rest replay one captured step, recorded on the
    // model's own stream, then launched on the caller's.
    if (!step(st))
        return false;
    if (steps == 1)
        return true;
    const anima_hip_dit::GraphKey key{latent, freqs, scratch, d->sig_dev, scratch_bytes, H, W,
                                      cfg, d->gen};
    if (!(d->graph && d->graph_key == key)) {
        if (d->graph) {
            if (!hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize"))
                return false;
            (void)hipGraphExecDestroy(d->graph);
            d->graph = nullptr;
        }
        if (!d->cap_stream &&
            !hip_ok(hipStreamCreateWithFlags(&d->cap_stream, hipStreamNonBlocking),
                    "hipStreamCreate"))
            return false;
        hipGraph_t g = nullptr;
        if (!hip_ok(hipStreamBeginCapture(d->cap_stream, hipStreamCaptureModeThreadLocal),
                    "hipStreamBeginCapture"))
            return false;
        const bool recorded = step(d->cap_stream);
        const hipError_t e = hipStreamEndCapture(d->cap_stream, &g);
        bool ok = recorded && hip_ok(e, "hipStreamEndCapture");
        // Only kernel launches may be replayed: a library call that recorded
        // a memset or copy node leaves the remaining steps to run directly.
        bool kernels_only = ok;
        if (ok) {
            size_t n = 0;
            ok = hip_ok(hipGraphGetNodes(g, nullptr, &n), "hipGraphGetNodes");
            std::vector<hipGraphNode_t> nodes(n);
            ok = ok && hip_ok(hipGraphGetNodes(g, nodes.data(), &n), "hipGraphGetNodes");
            for (size_t i = 0; ok && i < n; ++i) {
                hipGraphNodeType t;
                ok = hip_ok(hipGraphNodeGetType(nodes[i], &t), "hipGraphNodeGetType");
                kernels_only = kernels_only && t == hipGraphNodeTypeKernel;
            }
            kernels_only = kernels_only && ok;
        }
        if (ok && kernels_only)
            ok = hip_ok(hipGraphInstantiate(&d->graph, g, nullptr, nullptr, 0),
                        "hipGraphInstantiate");
        if (g)
            (void)hipGraphDestroy(g);
        if (!ok) {
            d->graph = nullptr;
            return false;
        }
        if (!kernels_only) {
            for (int i = 1; i < steps; ++i)
                if (!step(st))
                    return false;
            return true;
        }
        d->graph_key = key;
    }
    for (int i = 1; i < steps; ++i)
        if (!hip_ok(hipGraphLaunch(d->graph, st), "hipGraphLaunch"))
            return false;
    return true;
}

}  // extern "C"
