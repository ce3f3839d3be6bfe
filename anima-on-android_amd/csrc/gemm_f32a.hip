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
//
// The QKV form (launch_gemm_f32a_qkv) is a self-attention's stacked q/k/v
// projection whose epilogue writes the attention's prepared operands instead
// of C: q and k rows after RMSNorm and RoPE with the one-launch prologue's
// arithmetic, and the packed V^T, so no prologue pass reads the projection
// back (4096 tokens, B = 2, H = 16: 363-367 us against 338-345 + 74-75 us
// for this kernel's plain form plus the prologue; the epilogue costs about
// 24 us, 10 of them the RoPE table's loads, and is latency-bound: the
// hardware bf16 conversion in place of the prologue's integer rounding,
// which takes a third of its VALU work, did not change its time).
#include "flash_tile.h"
#include "rowmath.h"

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

// The attention operands written in place of C by the fused q/k/v
// projection (launch_gemm_f32a_qkv): columns [0, HD) are q, [HD, 2HD) k,
// [2HD, 3HD) v, HD = H * 128, so a 256-column tile holds two whole heads of
// one of them.
struct FaQkv {
    void *qo, *ko, *vo;  // q / k rows; term V^T (terms) or f32 V rows
    const float *w[2];   // RMSNorm weights of q / k, or null
    const float *freqs;  // [S, 64, 2, 2] or null
    int64_t sp;          // V^T row length (= S)
    int S, H, HD;
    float eps;
    int terms;           // 1: [hi | lo] term rows and term V^T; 0: f32 rows
};

struct FaArgs {
    const float *a;   // [M][lda]
    const u16 *w;     // [N][ldw]
    float *c;         // [M][ldc]
    int64_t lda, ldw, ldc;
    int M, N, tiles_n, chunks;
    FaQkv qkv;        // QKV kernels only
};

constexpr int kQkvPitch = 132;  // floats per staged row of a head block (128 + 4 against conflicts)
static_assert(kFaWaves * 32 * kQkvPitch * 4 <= kFaStages * kFaStage * 2,
              "a head block per wave fits the rings");

__device__ __forceinline__ int fa_swz_a(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int fa_swz_w(int row) { return (row >> 2) & 3; }

// Wait for this wave's LDS accesses; the compiler moves no memory access
// across (rows written by other lanes of the wave are read next).
__device__ __forceinline__ void wave_lds_fence()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("" ::: "memory");
}

// Epilogue of the fused q/k/v projection: this wave's 32 token rows of the
// tile's two heads, in place of C.  Accumulators 4 hh .. 4 hh + 3 hold head
// hh: lane (col, half) has column d = 32 (nb % 4) + col of the rows
// acc_row(r, half).
//   q, k: RMSNorm, RoPE and the row layout of prep_qkv_kernel (prologue.hip)
//     with its arithmetic (no contraction): each head block goes through an
//     LDS region of the wave; one lane per row sums the squares in index
//     order, then 16 lanes per row take four rotation pairs each.  The bf16
//     terms come from the hardware conversion (split_terms4), which rounds
//     to nearest even like the prologue's integer form: the same bits for
//     every finite value and for the quiet NaNs that arithmetic produces;
//   v, terms: the term V^T straight from the accumulators.  In the key order
//     vt_key_pos (bits 2 and 3 of the key swapped) the keys of registers
//     8i .. 8i + 7 are positions 8 (2i + half) .. + 7 of the wave's 32-key
//     block: one 16-byte chunk per term and register group;
//   v, f32: dense V rows.
// M and S are multiples of 32, so a wave's 32 rows lie in one batch entry
// and are all inside or all past M (those write nothing).
__device__ __forceinline__ void qkv_epilogue(const FaQkv &e, f32x16 (&acc)[kFaNB], float *lds,
                                             int M, int row0, int col0, int wave, int lane)
{
#pragma clang fp contract(off)
    const int col = lane & 31, half = lane >> 5;
    const int mw = row0 + wave * 32;
    const int part = col0 / e.HD;                // 0 q, 1 k, 2 v (uniform per workgroup)
    const int head0 = (col0 - part * e.HD) / kD;  // the tile's first head
    const int bb = mw / e.S, s0 = mw - bb * e.S;
    if (part == 2) {
        if (mw >= M)
            return;
        if (!e.terms) {
            float *vo = static_cast<float *>(e.vo);
#pragma unroll
            for (int nb = 0; nb < kFaNB; ++nb) {
                const int n = (head0 + (nb >> 2)) * kD + 32 * (nb & 3) + col;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    vo[int64_t(mw + acc_row(r, half)) * e.HD + n] = acc[nb][r];
            }
            return;
        }
        u16 *vt = static_cast<u16 *>(e.vo);
#pragma unroll
        for (int nb = 0; nb < kFaNB; ++nb) {
            const int d = 32 * (nb & 3) + col;
            u16 *vrow = vt + (int64_t(bb) * e.H + head0 + (nb >> 2)) * (2 * kD) * e.sp +
                        int64_t(d) * e.sp + s0;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                uint2 h0, l0, h1, l1;
                split_terms4(f32x4{acc[nb][8 * i], acc[nb][8 * i + 1], acc[nb][8 * i + 2],
                                   acc[nb][8 * i + 3]},
                             h0, l0);
                split_terms4(f32x4{acc[nb][8 * i + 4], acc[nb][8 * i + 5], acc[nb][8 * i + 6],
                                   acc[nb][8 * i + 7]},
                             h1, l1);
                u16 *dst = vrow + 8 * (2 * i + half);
                *reinterpret_cast<u32x4 *>(dst) = u32x4{h0.x, h0.y, h1.x, h1.y};
                *reinterpret_cast<u32x4 *>(dst + kD * e.sp) = u32x4{l0.x, l0.y, l1.x, l1.y};
            }
        }
        return;
    }
    // Every wave has read its last fragments: the rings are free.
    __syncthreads();
    if (mw >= M)
        return;
    float *stg = lds + wave * (32 * kQkvPitch);
    const float *w = e.w[part];
    const int p0 = 4 * (lane & 15);
    f32x4 wl = f32x4{1.f, 1.f, 1.f, 1.f}, wh = wl;
    if (w) {
        wl = *reinterpret_cast<const f32x4 *>(w + p0);
        wh = *reinterpret_cast<const f32x4 *>(w + 64 + p0);
    }
    // The RoPE table entries of two of this lane's rows at a time, loaded
    // together (the first two while the sums of squares run) instead of
    // paying the load latency row by row; four rows at a time no longer fit
    // the registers beside the second head's accumulators.
    f32x4 tab[2][4];
    auto load_tab = [&](int it0) {
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const f32x4 *fq = reinterpret_cast<const f32x4 *>(
                e.freqs + int64_t(s0 + (lane >> 4) + 4 * (it0 + it)) * 256 + 4 * p0);
#pragma unroll
            for (int ee = 0; ee < 4; ++ee)
                tab[it][ee] = fq[ee];
        }
    };
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                stg[acc_row(r, half) * kQkvPitch + 32 * q + col] = acc[4 * hh + q][r];
        wave_lds_fence();
        if (e.freqs)
            load_tab(0);
        float inv = 0.0f;
        if (lane < 32) {
            float ss = 0.0f;
            const float *row = stg + lane * kQkvPitch;
#pragma unroll 8
            for (int j = 0; j < 32; ++j) {
                const f32x4 v = *reinterpret_cast<const f32x4 *>(row + 4 * j);
                ss = ss + v.x * v.x;
                ss = ss + v.y * v.y;
                ss = ss + v.z * v.z;
                ss = ss + v.w * v.w;
            }
            inv = inv_rms(ss, kD, e.eps);
        }
        const int64_t h = head0 + hh;
#pragma unroll
        for (int it = 0; it < 8; ++it) {
            if (it % 2 == 0 && it > 0 && e.freqs)
                load_tab(it);
            const int rr = (lane >> 4) + 4 * it;
            const float fi = __shfl(inv, rr);
            const float *row = stg + rr * kQkvPitch;
            f32x4 ya = *reinterpret_cast<const f32x4 *>(row + p0);
            f32x4 yb = *reinterpret_cast<const f32x4 *>(row + 64 + p0);
            ya = ya * fi;
            yb = yb * fi;
            if (w) {
                ya = ya * wl;
                yb = yb * wh;
            }
            f32x4 lo = ya, hi = yb;
            if (e.freqs) {
#pragma unroll
                for (int ee = 0; ee < 4; ++ee) {
                    const f32x4 c = tab[it & 1][ee];  // [c00, c01, c10, c11] of pair p0 + ee
                    lo[ee] = c.x * ya[ee] + c.y * yb[ee];
                    hi[ee] = c.z * ya[ee] + c.w * yb[ee];
                }
            }
            const int64_t orow = int64_t(mw + rr) * e.H + h;
            void *out = part == 0 ? e.qo : e.ko;
            if (e.terms) {
                u16 *ob = static_cast<u16 *>(out) + orow * (2 * kD) + p0;
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    uint2 th, tl;
                    split_terms4(k ? hi : lo, th, tl);
                    *reinterpret_cast<uint2 *>(ob + 64 * k) = th;
                    *reinterpret_cast<uint2 *>(ob + 64 * k + kD) = tl;
                }
            } else {
                float *of = static_cast<float *>(out) + orow * kD + p0;
                *reinterpret_cast<f32x4 *>(of) = lo;
                *reinterpret_cast<f32x4 *>(of + 64) = hi;
            }
        }
        // This wave's reads of the block are done before the next head's
        // block overwrites it.
        wave_lds_fence();
    }
}

template <int TERMS, bool QKV>
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

    if (QKV) {
        qkv_epilogue(g.qkv, acc, reinterpret_cast<float *>(smem), g.M, row0, col0, wave, lane);
        return;
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
        hipLaunchKernelGGL((gemm_f32a_kernel<2, false>), grid, block, 0, st, g);
    else
        hipLaunchKernelGGL((gemm_f32a_kernel<1, false>), grid, block, 0, st, g);
    return hip_ok(hipGetLastError(), "gemm_f32a_kernel launch");
}

bool gemm_f32a_qkv_supported(const float *a, int64_t lda, const void *w, int64_t ldw, int K,
                             const QkvPrep &p)
{
    const auto al = [](const void *x) { return (reinterpret_cast<uintptr_t>(x) & 15) == 0; };
    if ((p.mode != kAttnF32 && p.mode != kAttnF32X3) || p.B <= 0 || p.S <= 0 || p.H <= 0 ||
        p.H % 2 || p.S % 64)
        return false;
    const int64_t M = int64_t(p.B) * p.S, HD = int64_t(p.H) * 128;
    if (M > INT32_MAX || 3 * HD > INT32_MAX)
        return false;
    return p.qo && p.ko && p.vo && al(p.qo) && al(p.ko) && al(p.vo) && (!p.w[0] || al(p.w[0])) &&
           (!p.w[1] || al(p.w[1])) && (!p.freqs || al(p.freqs)) &&
           gemm_f32a_supported(int(M), int(3 * HD), K, lda, ldw, 3 * HD, a, w, p.qo);
}

bool launch_gemm_f32a_qkv(const float *a, int64_t lda, const uint16_t *w, int64_t ldw, int K,
                          const QkvPrep &p, hipStream_t st)
{
    if (!gemm_f32a_qkv_supported(a, lda, w, ldw, K, p))
        return fail("gemm_f32a_qkv: unsupported mode, shape or alignment (f32 or f32x3 mode, "
                    "S a multiple of 64, an even head count, 16-byte aligned operands, a grid "
                    "of at least 256 tiles)");
    FaArgs g{};
    g.a = a;
    g.w = w;
    g.lda = lda;
    g.ldw = ldw;
    g.M = p.B * p.S;
    g.N = 3 * p.H * 128;
    g.tiles_n = g.N / kFaBN;
    g.chunks = K / kFaBK;
    g.qkv.qo = p.qo;
    g.qkv.ko = p.ko;
    g.qkv.vo = p.vo;
    g.qkv.w[0] = p.w[0];
    g.qkv.w[1] = p.w[1];
    g.qkv.freqs = p.freqs;
    g.qkv.sp = p.S;
    g.qkv.S = p.S;
    g.qkv.H = p.H;
    g.qkv.HD = p.H * 128;
    g.qkv.eps = p.eps;
    g.qkv.terms = p.mode == kAttnF32X3 ? 1 : 0;
    const dim3 grid(unsigned(((g.M + kFaBM - 1) / kFaBM) * g.tiles_n)), block(kFaWaves * 64);
    hipLaunchKernelGGL((gemm_f32a_kernel<2, true>), grid, block, 0, st, g);
    return hip_ok(hipGetLastError(), "gemm_f32a_kernel (q/k/v) launch");
}

}  // namespace anima_hip
