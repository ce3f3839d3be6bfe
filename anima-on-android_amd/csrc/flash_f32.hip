// Non-causal / causal flash attention on f32 inputs with f32 MFMA (gfx950).
//
// Replaces anima::cpu::flash_attention (anima_rt/include/cpu/flash_attention.h:55-208),
// the body of anima_rt_run_sdpa_flash (anima_rt/src/anima_rt.cpp:147-156):
//   O = softmax(scale * Q K^T) V   per (batch, head), fp32 accumulation,
//   optional causal mask "key j > query i" (top-left aligned).
//
// Kernel shape (D = 128):
//   * one workgroup = NW waves, each wave owns 32 query rows (BM = 32*NW);
//   * K/V tiles of 64 keys are staged through LDS, double-buffered: the next
//     tile's V, then its K, is fetched into registers while the current tile
//     feeds the MFMAs, so one barrier per tile suffices;
//   * scores are computed transposed, S^T = K Q^T, with
//     v_mfma_f32_32x32x2_f32: lane l then holds query row (l % 32) in every
//     accumulator, so the online-softmax max/sum are lane-local except for a
//     single exchange with lane l^32 per tile;
//   * the output is accumulated transposed, O^T += V^T P^T: the B operand of
//     that MFMA is exactly the S^T accumulator (after exp2), so P never moves
//     between lanes, and the per-row rescale factor is lane-local too;
//   * exp is evaluated as exp2(s * scale*log2(e) - m) on v_exp_f32, with the
//     running max m updated lazily (only when a tile max exceeds it by more
//     than 8 in log2 units), so the O rescale is almost never executed.
// The contraction index d is permuted (lane half h walks d = 64h + t) so each
// lane reads K and Q as contiguous float4s; the permutation is applied to Q
// and K alike, so the dot products are unchanged.
#include "common.h"
#include "flash_tile.h"
#include "rowmath.h"

#include <cmath>

namespace anima_hip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kD = 128;
constexpr int kBN = 64;          // keys per K/V tile
constexpr int kKStride = kD + 4; // LDS row pitch of K (floats): 16-byte skew per row
constexpr int kVStride = kD;     // LDS row pitch of V: rows are read whole
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kVmcnt0 = 0x0F70;  // s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15)
constexpr float kRescaleLog2 = 8.0f;  // lazy-rescale threshold: p <= 2^8

struct F32Args {
    const float *q, *k, *v;
    float *o;
    int64_t qb, qh, qs, kb, kh, ks, vb, vh, vs, ob, oh, os;
    int H, S_q, S_kv, n_qtiles;
    float c;     // scale * log2(e)
    int causal;
    FlashSplitArgs split;  // n == 1: write O; n > 1: write this split's partial
    TermOut ot;            // n == 1 and ot.t set: O as bf16 terms
    // q holds raw projection rows (RawQ, no RoPE): the kernel applies the
    // per-head RMSNorm (weight qw, optional) itself.
    int raw_q;
    const float *qw;
    float eps;
};

// RMSNorm of one query row held as the f32 kernel's Q fragment (lane half h
// owns d = 64h .. 64h+63), as the row prologue (prologue.hip) computes it for
// anima_rt's rmsnorm_kernel (anima_rt/include/cpu/rmsnorm_kernel.h:11-31):
// y = x * inv_rms(sum x^2) [* w], no contraction.  The sum of squares keeps
// the reference's index order across the halves: half 0 adds d < 64 from
// zero, half 1 continues from half 0's partial (one v_permlane32_swap each
// way).  Every lane takes part; a zero row stays zero.
__device__ __forceinline__ void rms_norm_fragment(float (&x)[64], const float *w, float eps,
                                                  int half)
{
#pragma clang fp contract(off)
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 64; ++i)
        ss = ss + x[i] * x[i];
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false,
                                                    false);
    float ss1 = __uint_as_float(a[0]);  // half 0's partial
#pragma unroll
    for (int i = 0; i < 64; ++i)
        ss1 = ss1 + x[i] * x[i];
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss1), __float_as_uint(ss1),
                                                    false, false);
    const float inv = inv_rms(__uint_as_float(b[1]), kD, eps);  // half 1's total
    const f32x4 *wv = w ? reinterpret_cast<const f32x4 *>(w + 64 * half) : nullptr;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const f32x4 wj = wv ? wv[j] : f32x4{1.0f, 1.0f, 1.0f, 1.0f};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float y = x[4 * j + e] * inv;
            x[4 * j + e] = wv ? y * wj[e] : y;
        }
    }
}

__device__ __forceinline__ f32x16 mfma32(float a, float b, f32x16 c)
{
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Row index inside a 32x32 MFMA accumulator: register r of lane half h.
// Max of v over the two lanes l and l^32 (the two halves of a query row) with
// one v_permlane32_swap: r[0] holds the low half in both halves, r[1] the
// high half.
__device__ __forceinline__ float row_pair_max(float v)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ int acc_row(int r, int h)
{
    return 8 * (r >> 2) + 4 * h + (r & 3);
}

template <int NW>
__global__ __launch_bounds__(NW * 64, 1) void flash_f32_d128(F32Args a)
{
    constexpr int NT = NW * 64;
    constexpr int BM = NW * 32;
    constexpr int F4_PER_TILE = kBN * kD / 4;
    constexpr int LD = F4_PER_TILE / NT;  // float4 per thread per tile (K and V each)
    static_assert(F4_PER_TILE % NT == 0, "tile must split evenly over the workgroup");

    __shared__ __attribute__((aligned(16))) float Ks[2][kBN * kKStride];
    __shared__ __attribute__((aligned(16))) float Vs[2][kBN * kVStride];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int col = lane & 31;
    const int half = lane >> 5;

    // XCD-major order: the query tiles of one (batch, head) run on one XCD
    // and read its K/V through that XCD's L2 (the dispatcher's round-robin
    // order had every XCD fetch every head's K/V: 1.21 GB per launch at
    // 4096 tokens, B = 2, against 268 MB of algorithmic bytes).
    const int blk = flash_tile::xcd_major_block();
    const int sp = blk % a.split.n;
    const int qt = (blk / a.split.n) % a.n_qtiles;
    const int bh = (blk / a.split.n) / a.n_qtiles;
    const int b = bh / a.H;
    const int h = bh - b * a.H;
    const int q_tile0 = qt * BM;
    const int qrow = q_tile0 + wave * 32 + col;

    const float *qp = a.q + b * a.qb + h * a.qh;
    const float *kp = a.k + b * a.kb + h * a.kh;
    const float *vp = a.v + b * a.vb + h * a.vh;

    // Q fragment of this lane: Q[qrow][64*half + t], t = 0..63.
    float qf[64];
    if (qrow < a.S_q) {
        const f32x4 *src = reinterpret_cast<const f32x4 *>(qp + qrow * a.qs + 64 * half);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const f32x4 t = src[i];
            qf[4 * i + 0] = t.x;
            qf[4 * i + 1] = t.y;
            qf[4 * i + 2] = t.z;
            qf[4 * i + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 64; ++i)
            qf[i] = 0.0f;
    }
    if (a.raw_q)
        rms_norm_fragment(qf, a.qw, a.eps, half);
    // Retire the Q loads here.  Otherwise the compiler still counts them as
    // outstanding inside the tile loop and waits for vmcnt(0) before the
    // first MFMAs, which also waits for the next tile's prefetch.
    __builtin_amdgcn_s_waitcnt(kVmcnt0);

    int kv_end = a.S_kv;
    if (a.causal) {
        const int last_row = min(a.S_q, q_tile0 + BM);
        kv_end = min(kv_end, last_row);
    }
    // Key tiles [j0, j1) of this split (all of them when unsplit).
    const int j0 = sp * a.split.tiles;
    const int j1 = min((kv_end + kBN - 1) / kBN, j0 + a.split.tiles);

    // Next-tile staging registers, used for V then for K so only one
    // half-tile is held at a time.
    f32x4 stg[LD];
    auto gload = [&](const float *base, int64_t row_stride, int key0) {
#pragma unroll
        for (int i = 0; i < LD; ++i) {
            const int f = tid + i * NT;
            const int r = f >> 5;
            const int c4 = f & 31;
            const int key = key0 + r;
            stg[i] = key < a.S_kv
                         ? *reinterpret_cast<const f32x4 *>(base + key * row_stride + 4 * c4)
                         : f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };
    auto lstore = [&](float *dst, int pitch) {
#pragma unroll
        for (int i = 0; i < LD; ++i) {
            const int f = tid + i * NT;
            const int r = f >> 5;
            const int c4 = f & 31;
            *reinterpret_cast<f32x4 *>(dst + r * pitch + 4 * c4) = stg[i];
        }
    };

    f32x16 o0 = {}, o1 = {}, o2 = {}, o3 = {};
    float m = -INFINITY;  // running max of scaled logits (log2 domain)
    float l = 0.0f;       // running partial sum of this lane's keys

    if (j0 < j1) {
        gload(kp, a.ks, j0 * kBN);
        lstore(Ks[0], kKStride);
        gload(vp, a.vs, j0 * kBN);
        lstore(Vs[0], kVStride);
    }
    __syncthreads();

    for (int j = j0; j < j1; ++j) {
        const int buf = (j - j0) & 1;
        const bool more = j + 1 < j1;
        if (more)
            gload(vp, a.vs, (j + 1) * kBN);

        // S^T for keys [64j, 64j+32) (s0) and [64j+32, 64j+64) (s1).
        f32x16 s0 = {}, s1 = {};
        const float *kr0 = &Ks[buf][col * kKStride + 64 * half];
        const float *kr1 = kr0 + 32 * kKStride;
#pragma unroll
        for (int t4 = 0; t4 < 16; ++t4) {
            const f32x4 k0 = *reinterpret_cast<const f32x4 *>(kr0 + 4 * t4);
            const f32x4 k1 = *reinterpret_cast<const f32x4 *>(kr1 + 4 * t4);
            s0 = mfma32(k0.x, qf[4 * t4 + 0], s0);
            s1 = mfma32(k1.x, qf[4 * t4 + 0], s1);
            s0 = mfma32(k0.y, qf[4 * t4 + 1], s0);
            s1 = mfma32(k1.y, qf[4 * t4 + 1], s1);
            s0 = mfma32(k0.z, qf[4 * t4 + 2], s0);
            s1 = mfma32(k1.z, qf[4 * t4 + 2], s1);
            s0 = mfma32(k0.w, qf[4 * t4 + 3], s0);
            s1 = mfma32(k1.w, qf[4 * t4 + 3], s1);
        }

        // Scale into the log2 domain, mask, tile max.
        const int key0 = j * kBN;
        const bool need_mask = (key0 + kBN > a.S_kv) || a.causal;
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float x0 = s0[r] * a.c;
            float x1 = s1[r] * a.c;
            if (need_mask) {
                const int k0i = key0 + acc_row(r, half);
                const int k1i = k0i + 32;
                if (k0i >= a.S_kv || (a.causal && k0i > qrow))
                    x0 = -INFINITY;
                if (k1i >= a.S_kv || (a.causal && k1i > qrow))
                    x1 = -INFINITY;
            }
            s0[r] = x0;
            s1[r] = x1;
            mx = fmaxf(mx, fmaxf(x0, x1));
        }
        mx = row_pair_max(mx);
        // Lazy rescale: the reference max m (log2 domain) moves only when some
        // row of the wave sees a tile max above m + kRescaleLog2, and then for
        // the whole wave at once; otherwise the exponentials stay <= 2^8 and
        // O, l keep accumulating against the same m (exact, since the final
        // O / l shares it).  The O rescale is therefore almost never run.
        if (__any(mx > m + kRescaleLog2)) {
            const float m_new = fmaxf(m, mx);
            const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - m_new);
            m = m_new;
            l *= alpha;
            o0 *= alpha;
            o1 *= alpha;
            o2 *= alpha;
            o3 *= alpha;
        }
        const float m_use = (m == -INFINITY) ? 0.0f : m;

        float psum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s0[r] = __builtin_amdgcn_exp2f(s0[r] - m_use);
            s1[r] = __builtin_amdgcn_exp2f(s1[r] - m_use);
            psum += s0[r] + s1[r];
        }
        l += psum;
        // V of the next tile goes to the other buffer (last read before the
        // previous barrier), then K of the next tile is fetched.
        if (more) {
            lstore(Vs[buf ^ 1], kVStride);
            gload(kp, a.ks, (j + 1) * kBN);
        }

        // O^T[d][q] += V^T P^T.  Output block c holds d = 4*i + c, so one
        // float4 read of a V row feeds the four blocks.
        const float *vr = &Vs[buf][4 * col];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = acc_row(r, half);
            const f32x4 va = *reinterpret_cast<const f32x4 *>(vr + key * kVStride);
            const f32x4 vb = *reinterpret_cast<const f32x4 *>(vr + (key + 32) * kVStride);
            o0 = mfma32(va.x, s0[r], o0);
            o1 = mfma32(va.y, s0[r], o1);
            o2 = mfma32(va.z, s0[r], o2);
            o3 = mfma32(va.w, s0[r], o3);
            o0 = mfma32(vb.x, s1[r], o0);
            o1 = mfma32(vb.y, s1[r], o1);
            o2 = mfma32(vb.z, s1[r], o2);
            o3 = mfma32(vb.w, s1[r], o3);
        }

        if (more)
            lstore(Ks[buf ^ 1], kKStride);
        __syncthreads();
    }

    l += __shfl_xor(l, 32);
    // Every score of the row masked or NaN (the max never left -inf): zeros,
    // as the reference leaves such rows (flash_attention.h:148-152, 194-201).
    const bool dead = m == -INFINITY;
    const float inv = dead ? 0.0f : l > 0.0f ? 1.0f / l : 0.0f;
    if (qrow < a.S_q) {
        float *op = a.o + b * a.ob + h * a.oh + qrow * a.os;
        uint16_t *tp = a.ot.t ? a.ot.t + b * a.ot.tb + h * a.ot.th + qrow * a.ot.ts : nullptr;
        if (a.split.n > 1) {
            const int64_t prow = (int64_t(sp) * a.split.BH + bh) * a.S_q + qrow;
            op = a.split.part + prow * kD;
            tp = nullptr;
            if (half == 0)
                a.split.ml[prow] = make_float2(m, dead ? 0.0f : l);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int d0 = 4 * acc_row(r, half);
            flash_tile::store_out4(dead ? f32x4{0.f, 0.f, 0.f, 0.f}
                                        : f32x4{o0[r] * inv, o1[r] * inv, o2[r] * inv,
                                                o3[r] * inv},
                                   op, tp, a.ot.lo, d0);
        }
    }
}

// Generic flash attention for any head dim up to 64*DPL: one wave per query
// row, lanes split the head dim, one key per step with a wave-wide reduction.
// Correct for every shape the C-ABI accepts; used when D != 128 or the
// operands are not 16-byte aligned.
struct GenArgs {
    const float *q, *k, *v;
    float *o;
    int64_t qb, qh, qs, kb, kh, ks, vb, vh, vs, ob, oh, os;
    int H, S_q, S_kv, D;
    float c;
    int causal;
};

template <int DPL>
__global__ __launch_bounds__(64) void flash_f32_generic(GenArgs a)
{
    const int lane = threadIdx.x;
    const int qrow = blockIdx.x;
    const int bh = blockIdx.y;
    const int b = bh / a.H;
    const int h = bh - b * a.H;
    const float *qp = a.q + b * a.qb + h * a.qh + qrow * a.qs;
    const float *kp = a.k + b * a.kb + h * a.kh;
    const float *vp = a.v + b * a.vb + h * a.vh;

    float qv[DPL], ov[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
        const int d = lane + 64 * i;
        qv[i] = d < a.D ? qp[d] : 0.0f;
        ov[i] = 0.0f;
    }
    const int nk = a.causal ? min(a.S_kv, qrow + 1) : a.S_kv;
    float m = -INFINITY, l = 0.0f;
    for (int j = 0; j < nk; ++j) {
        const float *kr = kp + j * a.ks;
        float part = 0.0f;
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
            const int d = lane + 64 * i;
            if (d < a.D)
                part += qv[i] * kr[d];
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
            part += __shfl_xor(part, off);
        const float x = part * a.c;
        const float m_new = fmaxf(m, x);
        const float alpha = __builtin_amdgcn_exp2f(m - m_new);
        const float p = __builtin_amdgcn_exp2f(x - m_new);
        l = l * alpha + p;
        const float *vr = vp + j * a.vs;
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
            const int d = lane + 64 * i;
            ov[i] = ov[i] * alpha + (d < a.D ? p * vr[d] : 0.0f);
        }
        m = m_new;
    }
    const bool dead = m == -INFINITY;  // every score NaN: zeros, as the reference
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    float *op = a.o + b * a.ob + h * a.oh + qrow * a.os;
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
        const int d = lane + 64 * i;
        if (d < a.D)
            op[d] = dead ? 0.0f : ov[i] * inv;
    }
}

template <typename T>
void fill_common(T &g, const FlashProblem &p)
{
    g.q = static_cast<const float *>(p.q);
    g.k = static_cast<const float *>(p.k);
    g.v = static_cast<const float *>(p.v);
    g.o = p.o;
    g.qb = p.qs.b; g.qh = p.qs.h; g.qs = p.qs.s;
    g.kb = p.ks.b; g.kh = p.ks.h; g.ks = p.ks.s;
    g.vb = p.vs.b; g.vh = p.vs.h; g.vs = p.vs.s;
    g.ob = p.os.b; g.oh = p.os.h; g.os = p.os.s;
    g.H = p.H;
    g.S_q = p.S_q;
    g.S_kv = p.S_kv;
    g.c = p.scale * kLog2e;
    g.causal = p.causal ? 1 : 0;
}

bool aligned16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }
bool stride4(const Strides &s) { return s.b % 4 == 0 && s.h % 4 == 0 && s.s % 4 == 0; }

template <int NW>
bool launch_d128(const F32Args &a, int64_t BH, hipStream_t st)
{
    constexpr int BM = NW * 32;
    F32Args g = a;
    g.n_qtiles = (g.S_q + BM - 1) / BM;
    const int64_t nblk = BH * g.n_qtiles * g.split.n;
    if (nblk > INT32_MAX)
        return fail("flash_f32: problem too large for one launch");
    hipLaunchKernelGGL(flash_f32_d128<NW>, dim3(unsigned(nblk)), dim3(NW * 64), 0, st, g);
    return hip_ok(hipGetLastError(), "flash_f32_d128 launch");
}

}  // namespace

bool flash_f32_fast_path(const FlashProblem &p)
{
    return p.D == kD && aligned16(p.q) && aligned16(p.k) && aligned16(p.v) && aligned16(p.o) &&
           stride4(p.qs) && stride4(p.ks) && stride4(p.vs) && stride4(p.os);
}

bool launch_flash_f32(const FlashProblem &p, hipStream_t st, void *part, size_t part_bytes)
{
    const int64_t BH = int64_t(p.B) * p.H;
    if (BH == 0 || p.S_q == 0)
        return true;
    // Raw query rows (RMSNorm, no RoPE) are read like prepared f32 rows, by
    // the D == 128 kernel only.
    const bool raw_q = p.rq.x != nullptr;
    FlashProblem f = p;
    if (raw_q) {
        f.q = p.rq.x;
        f.qs = p.rq.s;
        if (p.rq.freqs || !flash_f32_fast_path(f) || (p.rq.w && !aligned16(p.rq.w)))
            return fail("flash_f32: raw query rows need D == 128, 16-byte aligned rows and "
                        "strides, and no RoPE table");
    }
    if (f.ot.t && !(flash_f32_fast_path(f) && term_out_ok(f.ot)))
        return fail("flash_f32: term output needs D == 128, 16-byte aligned operands and an "
                    "16-byte aligned output with strides of 8 elements");
    if (flash_f32_fast_path(f)) {
        F32Args a;
        fill_common(a, f);
        a.ot = f.ot;
        a.raw_q = raw_q ? 1 : 0;
        a.qw = p.rq.w;
        a.eps = p.rq.eps;
        const FlashPlan pl = flash_plan(BH, p.S_q, p.S_kv, p.D, kTileUsF32);
        a.split = flash_split_args(pl, BH, p.S_q, part, part_bytes);
        if (!(pl.waves == 4 ? launch_d128<4>(a, BH, st) : launch_d128<8>(a, BH, st)))
            return false;
        return a.split.n == 1 || launch_flash_combine(p, a.split, st);
    }
    if (p.D > 1024)
        return fail("flash_f32: head dim " + std::to_string(p.D) + " > 1024 is not supported");
    if (BH > 65535)
        return fail("flash_f32 generic path: B*H > 65535 is not supported");
    GenArgs g;
    fill_common(g, p);
    g.D = p.D;
    const dim3 grid(unsigned(p.S_q), unsigned(BH));
    const int dpl = (p.D + 63) / 64;
    if (dpl <= 1)
        hipLaunchKernelGGL(flash_f32_generic<1>, grid, dim3(64), 0, st, g);
    else if (dpl <= 2)
        hipLaunchKernelGGL(flash_f32_generic<2>, grid, dim3(64), 0, st, g);
    else if (dpl <= 4)
        hipLaunchKernelGGL(flash_f32_generic<4>, grid, dim3(64), 0, st, g);
    else if (dpl <= 8)
        hipLaunchKernelGGL(flash_f32_generic<8>, grid, dim3(64), 0, st, g);
    else
        hipLaunchKernelGGL(flash_f32_generic<16>, grid, dim3(64), 0, st, g);
    return hip_ok(hipGetLastError(), "flash_f32_generic launch");
}

}  // namespace anima_hip
