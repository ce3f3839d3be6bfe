// Split-KV support of the D == 128 flash kernels: the launch plan for
// problems too small to fill the GPU, and the kernel that merges the
// per-split partial outputs.
//
// Merging follows from the online-softmax identity the flash kernels already
// use between key tiles (anima_rt/include/cpu/flash_attention.h:145-178 rescales
// the running sum and output when a later key block raises the max): with
// split s holding O_s = sum_j p_j v_j / l_s, p_j = 2^(x_j - m_s), l_s = sum_j p_j,
//   O = sum_s l_s 2^(m_s - M) O_s / sum_s l_s 2^(m_s - M),  M = max_s m_s.
#include "common.h"
#include "flash_tile.h"

#include <cmath>

namespace anima_hip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;
constexpr int kBN = 64;            // keys per tile of the flash kernels
constexpr int kTargetBlocks = 256; // one flash workgroup per CU of an MI355X (256 CUs)

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
size_t round_up256(size_t n) { return (n + 255) / 256 * 256; }

struct CombineArgs {
    float *o;
    int64_t ob, oh, os;
    int H, S_q;
    FlashSplitArgs sa;
    TermOut ot;     // set: O as bf16 terms instead of f32 at o
    int64_t total;  // BH * S_q * 32 float4 columns
};

// One thread per (row, float4 of the head dim).
__global__ __launch_bounds__(256) void flash_combine_kernel(CombineArgs a)
{
    const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= a.total)
        return;
    const int64_t row = idx >> 5;  // bh * S_q + q
    const int c4 = int(idx & 31);
    const int64_t plane = a.sa.BH * a.S_q;
    // Groups of kU splits: all loads of a group are issued before any use,
    // so the merge costs a few memory latencies rather than one per split.
    constexpr int kU = 8;
    float mx = -INFINITY;
    for (int s0 = 0; s0 < a.sa.n; s0 += kU) {
        float2 v[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u)
            v[u] = s0 + u < a.sa.n ? a.sa.ml[(s0 + u) * plane + row] : make_float2(0.f, 0.f);
        // A split with l == 0 saw no key (causal) or only masked or NaN
        // scores; a NaN l (a NaN score among finite ones) joins and makes
        // the row NaN, as in the reference.
#pragma unroll
        for (int u = 0; u < kU; ++u)
            if (v[u].y != 0.0f)
                mx = fmaxf(mx, v[u].x);
    }
    float lsum = 0.0f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < a.sa.n; s0 += kU) {
        float2 v[kU];
        f32x4 x[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const bool in = s0 + u < a.sa.n;
            const int64_t prow = (s0 + u) * plane + row;
            v[u] = in ? a.sa.ml[prow] : make_float2(0.f, 0.f);
            x[u] = in ? *reinterpret_cast<const f32x4 *>(a.sa.part + prow * kD + 4 * c4)
                      : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            if (v[u].y != 0.0f) {
                const float w = v[u].y * exp2f(v[u].x - mx);
                lsum += w;
                acc += w * x[u];
            }
        }
    }
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    const int64_t bh = row / a.S_q;
    const int q = int(row - bh * a.S_q);
    const int b = int(bh / a.H), h = int(bh - int64_t(b) * a.H);
    flash_tile::store_out4(acc * inv, a.o + b * a.ob + h * a.oh + q * a.os,
                           a.ot.t ? a.ot.t + b * a.ot.tb + h * a.ot.th + q * a.ot.ts : nullptr,
                           a.ot.lo, 4 * c4);
}

}  // namespace

bool term_out_ok(const TermOut &t)
{
    return (reinterpret_cast<uintptr_t>(t.t) & 15u) == 0 && t.tb % 8 == 0 && t.th % 8 == 0 &&
           t.ts % 8 == 0 && t.lo % 8 == 0 && t.lo >= 0;
}

FlashPlan flash_plan(int64_t BH, int S_q, int S_kv, int D, float tile_us)
{
    FlashPlan pl;
    if (D != kD || BH <= 0 || S_q <= 0 || BH * ceil_div(S_q, 256) >= kTargetBlocks)
        return pl;
    pl.waves = 4;
    const int64_t units = BH * ceil_div(S_q, 128);
    const int64_t ntiles = ceil_div(S_kv, kBN);
    const int64_t want = ceil_div(kTargetBlocks, units);
    if (want < 2 || ntiles < 2)
        return pl;
    const int64_t tiles = ceil_div(ntiles, std::min(want, ntiles));
    const int64_t splits = ceil_div(ntiles, tiles);
    if (splits < 2 || (tile_us > 0.0f && double(ntiles - tiles) * tile_us < kSplitCostUs))
        return pl;
    pl.splits = int(splits);
    pl.tiles = int(tiles);
    const size_t rows = size_t(splits) * size_t(BH) * size_t(S_q);
    pl.bytes = round_up256(rows * kD * sizeof(float)) + rows * sizeof(float2);
    return pl;
}

FlashSplitArgs flash_split_args(const FlashPlan &pl, int64_t BH, int S_q, void *part,
                                size_t part_bytes)
{
    FlashSplitArgs sa;
    if (pl.splits < 2 || !part || part_bytes < pl.bytes ||
        (reinterpret_cast<uintptr_t>(part) & 15u) != 0)
        return sa;
    const size_t rows = size_t(pl.splits) * size_t(BH) * size_t(S_q);
    sa.n = pl.splits;
    sa.tiles = pl.tiles;
    sa.BH = BH;
    sa.part = static_cast<float *>(part);
    sa.ml = reinterpret_cast<float2 *>(static_cast<char *>(part) +
                                       round_up256(rows * kD * sizeof(float)));
    return sa;
}

bool launch_flash_combine(const FlashProblem &p, const FlashSplitArgs &sa, hipStream_t st)
{
    CombineArgs a;
    a.o = p.o;
    a.ob = p.os.b;
    a.oh = p.os.h;
    a.os = p.os.s;
    a.H = p.H;
    a.S_q = p.S_q;
    a.sa = sa;
    a.ot = p.ot;
    a.total = sa.BH * p.S_q * (kD / 4);
    const int64_t nblk = ceil_div(a.total, 256);
    if (nblk > INT32_MAX)
        return fail("flash_combine: problem too large for one launch");
    hipLaunchKernelGGL(flash_combine_kernel, dim3(unsigned(nblk)), dim3(256), 0, st, a);
    return hip_ok(hipGetLastError(), "flash_combine_kernel launch");
}

}  // namespace anima_hip
