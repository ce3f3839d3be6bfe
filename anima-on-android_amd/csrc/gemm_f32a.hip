// Large-M projection GEMM on f32 activations: C[M,N] = A[M,K] . W[N,K]^T
// with f32 A, bf16 weights W and f32 C, on bf16 MFMA with f32 accumulation.
// The f32 A is split in registers, as linear.hip's split pass would write it:
//   two terms (f32 modes): hi = bf16(a), lo = bf16(a - hi), C = hi W^T + lo W^T
//                          (|a - hi - lo| <= 2^-16 |a|);
//   one term (bf16 mode):  hi only.
// The projections are the reference's (numpy_dit.py:273-281, 294-296,
// 304-317; anima_rt/vulkan/gemm_bf16.comp:25-57 computes them with f32 FMAs
// on f32 activations and bf16 weights, and anima_rt_run_gemm_bf16,
// gemm_backend.cpp:154-173, is this product's drop-in entry).
//
// Why f32 rows: the split pass reads f32 A and writes the terms, which the
// product reads back; staging the f32 rows themselves moves the same bytes
// through L2 as the hi and lo rows would, and the pass and its HBM round trip
// go away.  Shape of the kernel:
//   * 256 x 256 tiles of C, 32-element K chunks: a stage is 256 f32 A rows
//     (128 bytes each) + 256 W rows (64 bytes), 48 KiB; three stages (144
//     KiB), so a chunk's copies have two chunks' time to land;
//   * 8 waves as 8 (M) x 1 (N): a wave owns 32 rows of C and all 256
//     columns (8 accumulators of v_mfma_f32_32x32x16_bf16), so each A row is
//     read and split by one wave only, and per 16-element K step a wave does
//     8 MFMAs per term on 2 A reads (32 bytes per lane, split in registers)
//     and 8 W reads; two terms need 24 B/clk of L2 -> LDS at the full MFMA
//     rate (inside the ~35 B/clk a CU takes), one term 48;
//   * every wave copies 4 A windows and 2 W windows of each chunk (1 KiB
//     global_load_lds each); 16-byte pieces are XOR-swizzled (A rows by
//     (row & 7) ^ ((row >> 3) & 1), W rows by (row >> 2) & 3) so each 16-lane
//     quarter of a fragment read touches 16 distinct bank groups;
//   * one barrier per chunk, between its two K steps, after every wave has
//     read all of the chunk; the freed stage then takes the chunk three
//     ahead, one copy after each accumulator's products of the second K step
//     (issued together after the barrier, the 48 copies of a CU stalled the
//     issuing waves; spread out, 8192 x 2048 x 2048 two-term 0.1179 ->
//     0.1135 ms and 8192 x 2048 x 8192 0.469 -> 0.436 ms);
//   * XCD-major workgroup order with the N tiles of one M tile consecutive.
// Per element of C the hi and lo products of each K step accumulate in that
// order, K steps ascending: the order of the two-term kernel on term rows
// (gemm_large.hip), so C is bit-identical to the split pass plus that kernel.
#include "flash_tile.h"

#include <algorithm>

namespace anima_hip {
namespace {

using namespace flash_tile;

constexpr int kFaBK = 32;      // K elements per chunk
constexpr int kFaBM = 256;     // rows of C (and f32 A rows) per tile
constexpr int kFaBN = 256;     // columns of C (W rows) per tile
constexpr int kFaWaves = 8;
constexpr int kFaStages = 3;
constexpr int kFaAEl = kFaBM * kFaBK * 2;        // 16-bit slots of the f32 A part (32 KiB)
constexpr int kFaWEl = kFaBN * kFaBK;            // 16-bit slots of the W part (16 KiB)
constexpr int kFaStage = kFaAEl + kFaWEl;        // 48 KiB
constexpr int kFaACopies = kFaAEl / 512 / kFaWaves;  // 1 KiB windows per wave: 4
constexpr int kFaWCopies = kFaWEl / 512 / kFaWaves;  // 2
constexpr int kFaNB = kFaBN / 32;                // accumulator blocks per wave

struct FaArgs {
    const float *a;   // [M][lda]
    const u16 *w;     // [N][ldw]
    float *c;         // [M][ldc]
    int64_t lda, ldw, ldc;
    int M, N, tiles_n, chunks;
};

__device__ __forceinline__ int fa_swz_a(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int fa_swz_w(int row) { return (row >> 2) & 3; }

template <int TERMS>
__global__ __launch_bounds__(kFaWaves * 64, 1) void gemm_f32a_kernel(FaArgs g)
{
    __shared__ __attribute__((aligned(16))) u16 smem[kFaStages * kFaStage];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, half = lane >> 5;

    const int blk = xcd_major_block();
    const int tn = blk % g.tiles_n, tm = blk / g.tiles_n;
    const int row0 = tm * kFaBM, col0 = tn * kFaBN;

    // Copies.  A window i of wave w is window 4w + i of the A part (8 rows
    // of 128 bytes): lane l fills slot l & 7 of row (64 win + l) >> 3 with
    // the row's piece slot ^ fa_swz_a(row).  W window i is window 2w + i of
    // the W part (16 rows of 64 bytes), slot l & 3 of row (64 win + l) >> 2
    // with piece slot ^ fa_swz_w(row).  Rows past M or N re-read the last
    // row (their results are not stored).  Byte offsets from the tile's first
    // row at the chunk's first column.
    unsigned aoff[kFaACopies], woff[kFaWCopies];
#pragma unroll
    for (int i = 0; i < kFaACopies; ++i) {
        const int f = (wave * kFaACopies + i) * 64 + lane;
        const int r = f >> 3, pc = (f & 7) ^ fa_swz_a(r);
        const int rr = min(row0 + r, g.M - 1) - row0;
        aoff[i] = unsigned(int64_t(rr) * g.lda * 4 + 16 * pc);
    }
#pragma unroll
    for (int i = 0; i < kFaWCopies; ++i) {
        const int f = (wave * kFaWCopies + i) * 64 + lane;
        const int r = f >> 2, pc = (f & 3) ^ fa_swz_w(r);
        const int rr = min(col0 + r, g.N - 1) - col0;
        woff[i] = unsigned(int64_t(rr) * g.ldw * 2 + 16 * pc);
    }
    const char *asrc = reinterpret_cast<const char *>(g.a + int64_t(row0) * g.lda);
    const char *wsrc = reinterpret_cast<const char *>(g.w + int64_t(col0) * g.ldw);
    // Copy i (0 .. kCopies - 1) of this wave for chunk c into `stage`: the
    // A windows first, then the W windows.
    auto dma_one = [&](int c, int stage, int i) {
        u16 *st = smem + stage * kFaStage;
        if (i < kFaACopies)
            dma16s(asrc + int64_t(c) * kFaBK * 4, aoff[i], st + (wave * kFaACopies + i) * 512);
        else
            dma16s(wsrc + int64_t(c) * kFaBK * 2, woff[i - kFaACopies],
                   st + kFaAEl + (wave * kFaWCopies + i - kFaACopies) * 512);
    };
    auto dma = [&](int c, int stage) {
#pragma unroll
        for (int i = 0; i < kFaACopies + kFaWCopies; ++i)
            dma_one(c, stage, i);
    };

    // Fragments of K step t (elements 16t .. 16t + 15 of the chunk): this
    // lane's 8 elements 8 (2t + half) .. of A row wave * 32 + col (two
    // 16-byte pieces of f32) and of W rows 32 nb + col (one piece of bf16).
    const int arow = wave * 32 + col;
    const int aswz = fa_swz_a(arow);
    auto frags = [&](const u16 *st, int t, bf16x8 (&af)[2], bf16x8 (&wf)[kFaNB]) {
        const int p0 = 2 * (2 * t + half);
        const f32x4 x0 = *reinterpret_cast<const f32x4 *>(st + arow * 64 + 8 * (p0 ^ aswz));
        const f32x4 x1 = *reinterpret_cast<const f32x4 *>(st + arow * 64 + 8 * ((p0 + 1) ^ aswz));
#pragma unroll
        for (int nb = 0; nb < kFaNB; ++nb) {
            const int r = 32 * nb + col;
            wf[nb] = *reinterpret_cast<const bf16x8 *>(st + kFaAEl + r * kFaBK +
                                                       8 * ((2 * t + half) ^ fa_swz_w(r)));
        }
        uint2 h0, l0, h1, l1;
        split_terms4(x0, h0, l0);
        split_terms4(x1, h1, l1);
        af[0] = __builtin_bit_cast(bf16x8, uint4{h0.x, h0.y, h1.x, h1.y});
        if (TERMS == 2)
            af[1] = __builtin_bit_cast(bf16x8, uint4{l0.x, l0.y, l1.x, l1.y});
    };

    f32x16 acc[kFaNB];
#pragma unroll
    for (int nb = 0; nb < kFaNB; ++nb)
        acc[nb] = f32x16{};
    bf16x8 af[2][2], wf[2][kFaNB];
    // Per accumulator the hi product, then the lo product.
    auto mfmas = [&](int set) {
#pragma unroll
        for (int nb = 0; nb < kFaNB; ++nb) {
            acc[nb] = mfma_bf16(af[set][0], wf[set][nb], acc[nb]);
            if (TERMS == 2)
                acc[nb] = mfma_bf16(af[set][1], wf[set][nb], acc[nb]);
        }
    };

    const int total = g.chunks;
    constexpr int kCopies = kFaACopies + kFaWCopies;  // per wave and chunk
    dma(0, 0);
    if (total > 1)
        dma(1, 1);
    if (total > 2)
        dma(2, 2);
    // Chunk 0's copies landed: the later chunks' may still be in flight.
    if (total > 2)
        wait_vmcnt<2 * kCopies>();
    else if (total > 1)
        wait_vmcnt<kCopies>();
    else
        wait_vmcnt<0>();
    ring_barrier();
    frags(smem, 0, af[0], wf[0]);
    for (int c = 0; c < total; ++c) {
        const u16 *st = smem + (c % kFaStages) * kFaStage;
        frags(st, 1, af[1], wf[1]);
        mfmas(0);
        __builtin_amdgcn_sched_barrier(0);
        const bool more = c + 1 < total;
        if (more) {
            // Chunk c + 1's copies landed (c + 2's may still fly).  After the
            // barrier every wave sees them and has read all of chunk c (its
            // step-1 fragments above; the barrier waits for those reads), so
            // chunk c's stage takes chunk c + 3 while the step-1 MFMAs run.
            if (c + 2 < total)
                wait_vmcnt<kCopies>();
            else
                wait_vmcnt<0>();
            ring_barrier();
        }
        // Step 1's MFMAs with chunk c + 3's copies between them, one after
        // each accumulator's products: copies issued in one burst stall the
        // issuing waves at the memory pipe, while spread out they wait behind
        // the MFMAs.
        const bool copies = c + 3 < total;
#pragma unroll
        for (int nb = 0; nb < kFaNB; ++nb) {
            acc[nb] = mfma_bf16(af[1][0], wf[1][nb], acc[nb]);
            if (TERMS == 2)
                acc[nb] = mfma_bf16(af[1][1], wf[1][nb], acc[nb]);
            __builtin_amdgcn_sched_barrier(0);
            if (copies && nb < kCopies)
                dma_one(c + 3, c % kFaStages, nb);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (more)
            frags(smem + ((c + 1) % kFaStages) * kFaStage, 0, af[0], wf[0]);
    }

    // Lane (col, half) of accumulator nb holds C[m][n] for n = col0 + 32 nb +
    // col and m = row0 + wave * 32 + acc_row(r, half): for one register, 32
    // lanes cover 128 consecutive bytes of a row.  Nontemporal (streaming)
    // stores: C goes to the next kernel through HBM, and the stores of one
    // round of tiles then overlap the next round's loads better (8192 x 8192
    // x 2048: 0.498 -> 0.480 ms, 8192 x 2048 x 2048 0.1203 -> 0.1188 ms on one
    // box).
    const bool full = row0 + kFaBM <= g.M && col0 + kFaBN <= g.N;
#pragma unroll
    for (int nb = 0; nb < kFaNB; ++nb) {
        const int n = col0 + 32 * nb + col;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = row0 + wave * 32 + acc_row(r, half);
            if (!full && (m >= g.M || n >= g.N))
                continue;
            __builtin_nontemporal_store(acc[nb][r], g.c + int64_t(m) * g.ldc + n);
        }
    }
}

}  // namespace

// Shapes the kernel takes: K a multiple of 32, 16-byte aligned A and W rows,
// byte offsets of a tile's rows within 32 bits, and at least one full round
// of workgroups (256 tiles of 256 x 256).
bool gemm_f32a_supported(int M, int N, int K, int64_t lda, int64_t ldw, int64_t ldc,
                         const float *a, const void *w, const void *c)
{
    const auto al = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (M <= 0 || N <= 0 || K <= 0 || K % kFaBK)
        return false;
    const int64_t tiles = int64_t((M + kFaBM - 1) / kFaBM) * ((N + kFaBN - 1) / kFaBN);
    return tiles >= 256 && tiles < (int64_t(1) << 31) && lda >= K && ldw >= K && ldc >= N &&
           lda % 4 == 0 && ldw % 8 == 0 && al(a) && al(w) &&
           (reinterpret_cast<uintptr_t>(c) & 3) == 0 &&
           int64_t(kFaBM) * lda * 4 < (int64_t(1) << 31) &&
           int64_t(kFaBN) * ldw * 2 < (int64_t(1) << 31);
}

bool launch_gemm_f32a(const float *a, int64_t lda, const uint16_t *w, int64_t ldw, float *c,
                      int64_t ldc, int M, int N, int K, bool two_terms, hipStream_t st)
{
    if (!gemm_f32a_supported(M, N, K, lda, ldw, ldc, a, w, c))
        return fail("gemm_f32a: unsupported shape or alignment");
    FaArgs g;
    g.a = a;
    g.w = w;
    g.c = c;
    g.lda = lda;
    g.ldw = ldw;
    g.ldc = ldc;
    g.M = M;
    g.N = N;
    g.tiles_n = (N + kFaBN - 1) / kFaBN;
    g.chunks = K / kFaBK;
    const dim3 grid(unsigned(((M + kFaBM - 1) / kFaBM) * g.tiles_n)), block(kFaWaves * 64);
    if (two_terms)
        hipLaunchKernelGGL(gemm_f32a_kernel<2>, grid, block, 0, st, g);
    else
        hipLaunchKernelGGL(gemm_f32a_kernel<1>, grid, block, 0, st, g);
    return hip_ok(hipGetLastError(), "gemm_f32a_kernel launch");
}

}  // namespace anima_hip
