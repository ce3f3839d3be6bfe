// Large-M projection GEMM on bf16 MFMA: C[M,N] = sum_t A_t[M,K] . W[N,K]^T
// with bf16 activation terms A_t (one term, or the hi and lo terms of f32
// activations), bf16 weights W (the reference's [out_features, in_features]
// bit patterns) and f32 accumulation, for the token counts of the 1024x1024
// image (M = 8192 for the CFG pair) and above.
//
// The reference computes these projections with f32 FMAs in its Vulkan GEMM
// (anima_rt/vulkan/gemm_bf16.comp:25-57; numpy_dit.py:273-281, 294-296,
// 304-317).  A compute unit takes about 35 bytes per clock from L2 into LDS
// (global_load_lds, measured), and its four MFMA pipes at full rate need
// 4096 (BM_rows + BN) / (BM_rows BN) bytes per clock for a tile whose staged
// A rows number BM_rows; so the tile is as large as LDS allows:
//   * one term: 256 x 256 tiles of C; two terms: 128 x 256 tiles, every K
//     chunk of W staged once and multiplied by both terms (the hi and lo
//     rows of the tile, 256 staged A rows either way).  Per 64-element K
//     chunk a stage is 256 A rows + 256 W rows of 128 bytes = 64 KiB, i.e.
//     32 bytes per clock at the full MFMA rate;
//   * 8 waves as 2 (M) x 4 (N): a wave owns 64 W rows and 128 staged A rows
//     (one term: 128 rows of C as 4 x 2 v_mfma_f32_32x32x16_bf16
//     accumulators; two terms: 64 rows of C as 2 x 2 accumulators, each
//     taking the hi and the lo product), 8 MFMAs per 16-element K step
//     either way;
//   * chunks reach LDS by DMA (global_load_lds) through two stages; 128-byte
//     rows whose 16-byte pieces are XOR-swizzled by (row & 7) ^
//     ((row >> 3) & 1), so every ds_read_b128 quarter touches 16 distinct
//     bank groups; fragments of K step t + 1 are read while the MFMAs of step
//     t run;
//   * one barrier per chunk, after its last K step's MFMAs are issued: by
//     then every wave has read all of the chunk, so its stage takes the
//     chunk after next while those MFMAs run.  The waves copying A rows
//     issue those copies right after the barrier, the waves copying W rows
//     after the next chunk's first K step, so the two waves of a SIMD do not
//     stall at copy issue together (8192 x 2048 x 8192 with two terms:
//     428 -> 411 us);
//   * workgroups in XCD-major order with the N tiles of one M tile
//     consecutive: the workgroups of one XCD share W chunks and A chunks
//     through its L2.
// Epilogues: C as f32, C as bf16 (round to nearest even), both through
// nontemporal (streaming) stores, or x[m][n] += gate[m / S][n] * C[m][n] (the
// gated residual of a DiT block).
//
// f32 activations (F32A): the two-term tile stages the 128 f32 rows of A
// themselves (256 bytes per row and chunk, the bytes of the hi and lo rows
// together, 16-byte pieces XOR-swizzled by row & 15) and every wave splits
// its fragments into hi = bf16(a) and lo = bf16(a - hi) in registers, the
// split pass's arithmetic (linear.hip), so C is bit-identical to the split
// pass followed by the two-term product and the pass's HBM round trip of the
// terms is gone.
#include "flash_tile.h"
#include "rowmath.h"

#include <algorithm>

namespace anima_hip {
namespace {

using namespace flash_tile;

constexpr int kLgBK = 64;     // K elements per chunk (128-byte rows)
constexpr int kLgBN = 256;    // W rows (N) per tile
constexpr int kLgRows = 256;  // staged A rows per tile (BM * terms)
constexpr int kLgWaves = 8;
constexpr int kLgStage = (kLgRows + kLgBN) * kLgBK;  // bf16 elements (64 KiB)
constexpr int kLgCopies = kLgStage / 512 / kLgWaves;  // 1 KiB windows per wave per chunk

constexpr int kLgF32 = kGemmOutF32, kLgBf16 = kGemmOutBf16, kLgResidual = kGemmOutResidual;

struct LargeArgs {
    const u16 *a0, *a1;  // activation terms [M][lda]; a1 null for one term
    const float *af;     // F32A: f32 activations [M][lda] (a0, a1 unused)
    const u16 *w;        // [N][ldw]
    void *c;             // f32 or bf16 [M][ldc]; the residual x for kLgResidual
    const float *gate;   // kLgResidual: gate[b * gate_stride + n], b = m / S
    int64_t lda, ldw, ldc, gate_stride;
    int M, N, S;
    int tiles_n, chunks;
};

__device__ __forceinline__ int lg_swizzle(int row) { return (row & 7) ^ ((row >> 3) & 1); }

template <int TERMS, int EPI, bool F32A>
__global__ __launch_bounds__(kLgWaves * 64, 1) void gemm_large_kernel(LargeArgs g)
{
    static_assert(!F32A || TERMS == 2, "f32 activations take the two-term tile");
    constexpr int BM = kLgRows / TERMS;        // rows of C per tile
    // Waves as WM x WN over the tile: 2 x 4 (a wave owns BM / 2 rows of C and
    // 64 columns), or with F32A 4 x 2 (32 rows, 128 columns), so that each
    // row block of A is split in registers by two waves instead of four.
    constexpr int WM = F32A ? 4 : 2, WN = kLgWaves / WM;
    constexpr int MB = F32A ? 1 : 4 / TERMS;   // 32-row accumulator blocks per wave
    constexpr int NB = kLgBN / WN / 32;        // 32-column accumulator blocks per wave
    constexpr int A_EL = kLgRows * kLgBK;      // A part of a stage
    __shared__ __attribute__((aligned(16))) u16 smem[2 * kLgStage];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, half = lane >> 5;
    const int wm = wave % WM, wn = wave / WM;

    const int blk = xcd_major_block();
    const int tn = blk % g.tiles_n, tm = blk / g.tiles_n;
    const int row0 = tm * BM, col0 = tn * kLgBN;

    // Copies: window i of wave w is window 8w + i of the stage (8 rows of one
    // operand): windows 0..31 hold the A rows (term-major: term t's BM rows
    // at staged rows t * BM ..; F32A: 4 f32 rows of 256 bytes per window),
    // 32..63 the W rows.  Waves 0-3 copy A, 4-7 copy W, so a wave's source
    // operand and term are uniform.  Rows past M or N re-read the last row
    // (their results are not stored).  Byte offsets from the operand's tile
    // row at the chunk's first column.
    const bool copies_a = wave < 4;
    const int term = copies_a && !F32A ? (wave * kLgCopies * 8) / BM : 0;
    unsigned off_b[kLgCopies];
#pragma unroll
    for (int i = 0; i < kLgCopies; ++i) {
        const int win = (wave & 3) * kLgCopies + i;  // window within the operand
        const int f = win * 64 + lane;
        if (F32A && copies_a) {
            const int r = f >> 4, lc = (f & 15) ^ (r & 15);
            const int rr = min(row0 + r, g.M - 1) - row0;
            off_b[i] = unsigned(int64_t(rr) * g.lda * 4 + 16 * lc);
            continue;
        }
        const int r = f >> 3, lc = (f & 7) ^ lg_swizzle(r);
        int rr;
        if (copies_a)
            rr = min(row0 + (r % BM), g.M - 1) - row0;
        else
            rr = min(col0 + r, g.N - 1) - col0;
        off_b[i] = unsigned(int64_t(rr) * (copies_a ? g.lda : g.ldw) * 2 + 16 * lc);
    }
    const char *src0 =
        F32A && copies_a ? reinterpret_cast<const char *>(g.af + int64_t(row0) * g.lda)
        : copies_a       ? reinterpret_cast<const char *>((term ? g.a1 : g.a0) + int64_t(row0) * g.lda)
                         : reinterpret_cast<const char *>(g.w + int64_t(col0) * g.ldw);
    const int64_t chunk_bytes = int64_t(kLgBK) * (F32A && copies_a ? 4 : 2);
    u16 *dst0 = smem + (copies_a ? 0 : A_EL) + (wave & 3) * kLgCopies * 512;
    auto dma = [&](int c, int stage) {
        const char *src = src0 + int64_t(c) * chunk_bytes;
#pragma unroll
        for (int i = 0; i < kLgCopies; ++i)
            dma16s(src, off_b[i], dst0 + stage * kLgStage + i * 512);
    };

    // Fragments of K step t from a stage: A blocks b (staged rows
    // wm * 128 + 32 b for one term; term b / 2, rows wm * 64 + 32 (b % 2) for
    // two), W blocks nb (rows wn * 64 + 32 nb), piece 2t + half of row col.
    const int sw = lg_swizzle(col);
    auto frags = [&](const u16 *st, int t, bf16x8 (&af)[4], bf16x8 (&wf)[NB]) {
        const int pc = ((2 * t + half) ^ sw) * 8;
        // W first: the step's first MFMA takes W block 0 and A block 0.
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            wf[nb] = *reinterpret_cast<const bf16x8 *>(st + A_EL +
                                                       (wn * 32 * NB + 32 * nb + col) * kLgBK + pc);
        if (F32A) {
            // The 8 f32 of the wave's row block: pieces 2 (2t + half) and the
            // next of its 256-byte row, split into the hi (af[0]) and lo
            // (af[1]) fragments.
            const int srow = wm * 32 + col;
            const int p0 = 2 * (2 * t + half);
            const f32x4 x0 =
                *reinterpret_cast<const f32x4 *>(st + srow * 128 + 8 * (p0 ^ (srow & 15)));
            const f32x4 x1 =
                *reinterpret_cast<const f32x4 *>(st + srow * 128 + 8 * ((p0 + 1) ^ (srow & 15)));
            uint2 h0, l0, h1, l1;
            split_terms4(x0, h0, l0);
            split_terms4(x1, h1, l1);
            af[0] = __builtin_bit_cast(bf16x8, uint4{h0.x, h0.y, h1.x, h1.y});
            af[1] = __builtin_bit_cast(bf16x8, uint4{l0.x, l0.y, l1.x, l1.y});
            return;
        }
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int srow = TERMS == 1 ? wm * 128 + 32 * b : (b >> 1) * BM + wm * 64 + 32 * (b & 1);
            af[b] = *reinterpret_cast<const bf16x8 *>(st + (srow + col) * kLgBK + pc);
        }
    };

    f32x16 acc[MB][NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            acc[mb][nb] = f32x16{};
    const int total = g.chunks;
    dma(0, 0);
    if (total > 1) {
        dma(1, 1);
        wait_vmcnt<kLgCopies>();
    } else {
        wait_vmcnt<0>();
    }
    ring_barrier();
    bf16x8 af[2][4], wf[2][NB];
    frags(smem, 0, af[0], wf[0]);
    // The 8 MFMAs of one K step on fragment set `set`.
    auto mfmas = [&](int set) {
        if (F32A) {
            // Per accumulator the hi product, then the lo product (the order
            // of the two-term kernel on term rows, so C is bit-identical).
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                acc[0][nb] = mfma_bf16(af[set][0], wf[set][nb], acc[0][nb]);
                acc[0][nb] = mfma_bf16(af[set][1], wf[set][nb], acc[0][nb]);
            }
            return;
        }
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
                acc[b % MB][nb] = mfma_bf16(af[set][b], wf[set][nb], acc[b % MB][nb]);
    };
    // Waves 0-3 (A rows) issue chunk c + 2's copies right after the barrier
    // that frees its stage, waves 4-7 (W rows) after the next chunk's first
    // K step, so the two waves of a SIMD do not stall at copy issue together.
    const bool late_copies = !copies_a;
    for (int c = 0; c < total; ++c) {
        const u16 *st = smem + (c & 1) * kLgStage;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            frags(st, j + 1, af[(j + 1) & 1], wf[(j + 1) & 1]);
            mfmas(j & 1);
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            if (j == 0 && late_copies && c >= 1 && c + 1 < total) {
                __builtin_amdgcn_sched_barrier(0);
                dma(c + 1, (c + 1) & 1);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        mfmas(1);
        __builtin_amdgcn_sched_barrier(0);
        if (c + 1 < total) {
            wait_vmcnt<0>();
            ring_barrier();
            if (c + 2 < total && !late_copies)
                dma(c + 2, c & 1);
            frags(smem + ((c + 1) & 1) * kLgStage, 0, af[0], wf[0]);
        }
    }

    // Lane (col, half) of accumulator (mb, nb) holds C[m][n] for n = col0 +
    // wn * 32 NB + 32 nb + col and m = row0 + wm * 32 MB + 32 mb + 8 (r >> 2)
    // + 4 half + (r & 3): for one register, 32 lanes cover 128 consecutive
    // bytes of a row.
    const int mw = row0 + wm * (32 * MB);
    const bool full = row0 + BM <= g.M && col0 + kLgBN <= g.N;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        // The 32 rows of block mb meet at most one batch boundary when S >= 32
        // (the gated residual's gate row is that of the batch entry m / S).
        const int mbase = mw + 32 * mb;
        const int b_lo = EPI == kLgResidual ? mbase / g.S : 0;
        const int bnd = (b_lo + 1) * g.S;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const int n = col0 + wn * 32 * NB + 32 * nb + col;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = mbase + acc_row(r, half);
                if (!full && (m >= g.M || n >= g.N))
                    continue;
                const float v = acc[mb][nb][r];
                const int64_t o = int64_t(m) * g.ldc + n;
                if (EPI == kLgF32) {
                    __builtin_nontemporal_store(v, static_cast<float *>(g.c) + o);
                } else if (EPI == kLgBf16) {
                    __builtin_nontemporal_store(f32_to_bf16_rne(v), static_cast<u16 *>(g.c) + o);
                } else {
                    const int b = g.S >= 32 ? (m >= bnd ? b_lo + 1 : b_lo) : m / g.S;
                    const float gv = g.gate[int64_t(b) * g.gate_stride + n];
                    float *x = static_cast<float *>(g.c) + o;
                    *x = gv * v + *x;
                }
            }
        }
    }
}

}  // namespace

// Shapes the kernel takes: K a multiple of 64, 16-byte aligned operands,
// row pitches that keep a tile's byte offsets in 32 bits, and at least one
// full round of workgroups (256) -- below that the library's smaller tiles
// or the small-M kernel keep more compute units busy.
bool gemm_large_supported(int M, int N, int K, int terms, int64_t lda, int64_t ldw,
                          int64_t ldc, const void *a0, const void *a1, const void *w,
                          const void *c, int out_bytes)
{
    const auto al = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (M <= 0 || N <= 0 || K <= 0 || K % kLgBK || (terms != 1 && terms != 2) ||
        (terms == 2) != (a1 != nullptr))
        return false;
    const int64_t bm = kLgRows / terms;
    const int64_t tiles = ((M + bm - 1) / bm) * ((N + kLgBN - 1) / kLgBN);
    return tiles >= 256 && tiles < (int64_t(1) << 31) && lda >= K && ldw >= K && ldc >= N &&
           lda % 8 == 0 && ldw % 8 == 0 && al(a0) && (!a1 || al(a1)) && al(w) &&
           (reinterpret_cast<uintptr_t>(c) & (out_bytes - 1)) == 0 &&
           int64_t(kLgRows) * std::max(lda, ldw) * 2 < (int64_t(1) << 31);
}

bool gemm_large_f32a_supported(int M, int N, int K, int64_t lda, int64_t ldw, int64_t ldc,
                               const float *a, const void *w, const void *c)
{
    const auto al = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (M <= 0 || N <= 0 || K <= 0 || K % kLgBK)
        return false;
    const int64_t tiles = ((M + 127) / 128) * int64_t((N + kLgBN - 1) / kLgBN);
    return tiles >= 256 && tiles < (int64_t(1) << 31) && lda >= K && ldw >= K && ldc >= N &&
           lda % 4 == 0 && ldw % 8 == 0 && al(a) && al(w) &&
           (reinterpret_cast<uintptr_t>(c) & 3) == 0 &&
           int64_t(128) * lda * 4 < (int64_t(1) << 31) &&
           int64_t(kLgBN) * ldw * 2 < (int64_t(1) << 31);
}

bool launch_gemm_large_f32a(const float *a, int64_t lda, const uint16_t *w, int64_t ldw, float *c,
                            int64_t ldc, int M, int N, int K, hipStream_t st)
{
    if (!gemm_large_f32a_supported(M, N, K, lda, ldw, ldc, a, w, c))
        return fail("gemm_large_f32a: unsupported shape or alignment");
    LargeArgs g;
    g.a0 = g.a1 = nullptr;
    g.af = a;
    g.w = w;
    g.c = c;
    g.gate = nullptr;
    g.lda = lda;
    g.ldw = ldw;
    g.ldc = ldc;
    g.gate_stride = 0;
    g.M = M;
    g.N = N;
    g.S = M;
    g.tiles_n = (N + kLgBN - 1) / kLgBN;
    g.chunks = K / kLgBK;
    const dim3 grid(unsigned(((M + 127) / 128) * g.tiles_n)), block(kLgWaves * 64);
    hipLaunchKernelGGL((gemm_large_kernel<2, kLgF32, true>), grid, block, 0, st, g);
    return hip_ok(hipGetLastError(), "gemm_large_kernel (f32 activations) launch");
}

bool launch_gemm_large(const uint16_t *a0, const uint16_t *a1, int64_t lda, const uint16_t *w,
                       int64_t ldw, void *c, int64_t ldc, int M, int N, int K, int epilogue,
                       const float *gate, int64_t gate_stride, int S, hipStream_t st)
{
    const int terms = a1 ? 2 : 1;
    if (!gemm_large_supported(M, N, K, terms, lda, ldw, ldc, a0, a1, w, c,
                              epilogue == kLgBf16 ? 2 : 4))
        return fail("gemm_large: unsupported shape or alignment");
    if (epilogue == kLgResidual && (!gate || S <= 0))
        return fail("gemm_large: the gated residual needs the gate and the tokens per batch entry");
    LargeArgs g;
    g.a0 = a0;
    g.a1 = a1;
    g.af = nullptr;
    g.w = w;
    g.c = c;
    g.gate = gate;
    g.lda = lda;
    g.ldw = ldw;
    g.ldc = ldc;
    g.gate_stride = gate_stride;
    g.M = M;
    g.N = N;
    g.S = S > 0 ? S : M;
    const int bm = kLgRows / terms;
    const int tiles_m = (M + bm - 1) / bm;
    g.tiles_n = (N + kLgBN - 1) / kLgBN;
    g.chunks = K / kLgBK;
    const dim3 grid(unsigned(tiles_m * g.tiles_n)), block(kLgWaves * 64);
#define ANIMA_LG_LAUNCH(T, E) \
    hipLaunchKernelGGL((gemm_large_kernel<T, E, false>), grid, block, 0, st, g)
    if (terms == 1) {
        if (epilogue == kLgBf16)
            ANIMA_LG_LAUNCH(1, kLgBf16);
        else if (epilogue == kLgResidual)
            ANIMA_LG_LAUNCH(1, kLgResidual);
        else
            ANIMA_LG_LAUNCH(1, kLgF32);
    } else {
        if (epilogue == kLgResidual)
            ANIMA_LG_LAUNCH(2, kLgResidual);
        else if (epilogue == kLgBf16)
            ANIMA_LG_LAUNCH(2, kLgBf16);
        else
            ANIMA_LG_LAUNCH(2, kLgF32);
    }
#undef ANIMA_LG_LAUNCH
    return hip_ok(hipGetLastError(), "gemm_large_kernel launch");
}

}  // namespace anima_hip
