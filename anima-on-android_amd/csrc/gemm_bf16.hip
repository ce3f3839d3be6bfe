// Small-M projection GEMM on bf16 MFMA: C[M,N] = sum_t A_t[M,K] . W[N,K]^T with
// bf16 activation terms A_t (one term, or hi and lo of f32 activations), bf16
// weights W (the reference's [out_features, in_features] bit patterns) and f32
// output, for the token counts of a 256x256 image's CFG pair (M = 512) and
// below.
//
// The reference computes these projections with f32 FMAs in its Vulkan GEMM
// (anima_rt/vulkan/gemm_bf16.comp:25-57, numpy_dit.py:273-281, 294-296,
// 304-317).  What bounds them on MI355X at M = 512 is the L2 -> LDS stream of
// A and W rows: a compute unit takes about 35 bytes per clock from L2 (probed
// with global_load_lds), while its four MFMA pipes need 4096 (BM + BN) /
// (BM BN) bytes per clock.  So:
//   * each workgroup takes a 128 x 128 tile of C and a slice of K ("split-K":
//     about 256 workgroups even when M*N holds only 64 tiles); the f32
//     partial tiles go to a workspace and a second kernel adds them in split
//     order (deterministic, no atomics);
//   * with two activation terms (hi + lo of the f32 activations, the exact
//     f32 mode) each K chunk of W is staged once and multiplied by both
//     terms into the same accumulators: 1.5 times the MFMA work per staged
//     byte of a one-term product;
//   * 8 waves: 2 x 2 waves, each a 64 x 64 block of C as 2 x 2
//     v_mfma_f32_32x32x16_bf16 accumulators, times two waves splitting every
//     chunk's four K steps (t = 0, 2 and t = 1, 3), whose sums are added
//     through LDS at the end; two waves per SIMD hide the LDS latency;
//   * A and W chunks of 64 K-elements reach LDS by DMA (global_load_lds)
//     through a ring of 4 stages (3 with two terms); rows of 128 bytes whose
//     16-byte pieces are XOR-swizzled by (row & 7) ^ ((row >> 3) & 1), so the
//     16 lanes of every ds_read_b128 quarter touch 16 distinct bank groups
//     (conflict-free at the 256-byte-per-clock LDS width);
//   * one barrier per chunk, placed before the chunk's last MFMA step so the
//     wait overlaps MFMAs in flight, and the next chunk's first fragments
//     load under that step.
#include "flash_tile.h"

#include <algorithm>

namespace anima_hip {
namespace {

using namespace flash_tile;

constexpr int kGemmBK = 64;      // K-elements per chunk (128 bytes per row)
constexpr int kGemmTile = 128;   // BM = BN
constexpr int kGemmWaves = 8;    // 2 x 2 output blocks x 2 K halves
constexpr int kGemmMaxM = 1024;  // larger M goes to the library GEMM
constexpr int kGemmTargetBlocks = 256;
constexpr int kGemmMinChunks = 8;  // shortest K slice of a split
constexpr int kGemmMaxSplits = 16;

struct GemmArgs {
    const u16 *a0, *a1;  // activation terms [M][lda]; a1 null for one term
    const u16 *w;        // [N][ldw]
    float *out;          // C [M][ldo]: ldc when splits == 1, else partials [splits][M][N]
    int64_t lda, ldw, ldo;
    int M, N;
    int tiles_m, tiles_n, splits;
    int chunks;          // K chunks per split
};

// s_waitcnt vmcnt(n) for n < 64 (the count's high bits live in bits 15:14).
template <int N>
__device__ __forceinline__ void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Wait until at most n chunks of COPIES copies each remain in flight
// (0 <= n <= 2; a negative n means nothing is in flight).
template <int COPIES>
__device__ __forceinline__ void wait_chunks(int n)
{
    if (n >= 2)
        wait_vm<2 * COPIES>();
    else if (n == 1)
        wait_vm<COPIES>();
    else
        wait_vm<0>();
}

__device__ __forceinline__ int gemm_swizzle(int row) { return (row & 7) ^ ((row >> 3) & 1); }

template <bool PAIR>
__global__ __launch_bounds__(kGemmWaves * 64, 1) void gemm_bf16_kernel(GemmArgs g)
{
    constexpr int NA = PAIR ? 2 : 1;           // activation terms per chunk
    constexpr int STAGES = PAIR ? 3 : 4;
    constexpr int BM = kGemmTile, BN = kGemmTile;
    constexpr int TERM_EL = BM * kGemmBK;      // one term's rows of a chunk
    constexpr int A_EL = NA * TERM_EL, STAGE = A_EL + BN * kGemmBK;
    constexpr int TERM_WIN = TERM_EL / 512, A_WIN = A_EL / 512;  // 1 KiB windows
    constexpr int COPIES = STAGE / 512 / kGemmWaves;  // 16-byte copies per lane
    static_assert(STAGE / 512 % kGemmWaves == 0, "stage splits evenly over the waves");
    __shared__ __attribute__((aligned(16))) u16 smem[STAGES * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, half = lane >> 5;
    const int wm = wave & 1, wn = (wave >> 1) & 1, ks = wave >> 2;

    // Tile order: consecutive ids (one XCD) share the split and the A rows.
    const int blk = xcd_major_block();
    const int tn = blk % g.tiles_n;
    const int rest = blk / g.tiles_n;
    const int tm = rest % g.tiles_m;
    const int sp = rest / g.tiles_m;
    const int row0 = tm * BM, col0 = tn * BN;
    const int total = g.chunks;

    // Copy i of the wave fills LDS window wave*COPIES + i of the stage; a
    // window holds 8 rows of one operand (term 0 rows, term 1 rows, then W
    // rows), so its source base is wave-uniform.  Rows past M or N re-read
    // the last row (their results are discarded).  Byte offsets from the
    // operand's first tile row at the chunk's first column.
    unsigned off_b[COPIES];
#pragma unroll
    for (int i = 0; i < COPIES; ++i) {
        const int win = wave * COPIES + i;
        const bool ra = win < A_WIN;
        const int ff = (ra ? win % TERM_WIN : win - A_WIN) * 64 + lane;
        const int r = ff >> 3, lc = (ff & 7) ^ gemm_swizzle(r);
        const int rr = ra ? min(row0 + r, g.M - 1) - row0 : min(col0 + r, g.N - 1) - col0;
        off_b[i] = unsigned(int64_t(rr) * (ra ? g.lda : g.ldw) * 2 + 16 * lc);
    }
    auto dma = [&](int c, int stage) {
        const int64_t k0 = (int64_t(sp) * g.chunks + c) * kGemmBK;
        const u16 *abase = g.a0 + int64_t(row0) * g.lda + k0;
        const u16 *lbase = PAIR ? g.a1 + int64_t(row0) * g.lda + k0 : abase;
        const u16 *wbase = g.w + int64_t(col0) * g.ldw + k0;
#pragma unroll
        for (int i = 0; i < COPIES; ++i) {
            const int win = wave * COPIES + i;
            const u16 *src = win >= A_WIN ? wbase : win >= TERM_WIN ? lbase : abase;
            dma16s(src, off_b[i], &smem[stage * STAGE + win * 512]);
        }
    };

    f32x16 acc[2][2] = {};
    // Fragments of K step t: this wave's A row blocks (per term) and W row
    // blocks, piece 2t + half of their rows (row & 15 == col & 15).
    const int sw = gemm_swizzle(col);
    auto frags = [&](const u16 *st, int t, bf16x8 (&af)[2 * NA], bf16x8 (&wf)[2]) {
        const int pc = ((2 * t + half) ^ sw) * 8;
#pragma unroll
        for (int b = 0; b < 2 * NA; ++b)
            af[b] = *reinterpret_cast<const bf16x8 *>(
                st + (b >> 1) * TERM_EL + (wm * 64 + 32 * (b & 1) + col) * kGemmBK + pc);
#pragma unroll
        for (int b = 0; b < 2; ++b)
            wf[b] = *reinterpret_cast<const bf16x8 *>(st + A_EL + (wn * 64 + 32 * b + col) *
                                                                       kGemmBK + pc);
    };

    // Every stage filled up front.  The barrier of chunk c sits between its
    // two K steps' MFMAs: by then every wave has read all of chunk c, so its
    // slot takes chunk c + STAGES, and chunk c+1 (whose copies each wave has
    // waited for) is visible for the next fragments.
    const int pre = min(STAGES, total);
    for (int c = 0; c < pre; ++c)
        dma(c, c);
    wait_chunks<COPIES>(pre - 1);
    ring_barrier();
    bf16x8 af[2][2 * NA], wf[2][2];
    frags(smem, ks, af[0], wf[0]);
    for (int c = 0; c < total; ++c) {
        const u16 *st = smem + (c % STAGES) * STAGE;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if (j == 0) {
                frags(st, ks + 2, af[1], wf[1]);
            } else if (c + 1 < total) {
                wait_chunks<COPIES>(min(total - 1, c + STAGES - 1) - (c + 1));
                ring_barrier();
                if (c + STAGES < total)
                    dma(c + STAGES, c % STAGES);
                frags(smem + ((c + 1) % STAGES) * STAGE, ks, af[0], wf[0]);
            }
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    acc[mb][nb] = mfma_bf16(af[j][mb], wf[j][nb], acc[mb][nb]);
                    if (PAIR)
                        acc[mb][nb] = mfma_bf16(af[j][2 + mb], wf[j][nb], acc[mb][nb]);
                }
        }
    }

    // The second K half's sums join the first through LDS (the ring is idle:
    // every copy has landed and, after the barrier, every read is done).
    float *slot = reinterpret_cast<float *>(smem) + (wm + 2 * wn) * (4 * 16 * 64) + lane;
    ring_barrier();
    if (ks == 1) {
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                slot[(b * 16 + r) * 64] = acc[b >> 1][b & 1][r];
    }
    ring_barrier();
    if (ks == 1)
        return;
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r)
            acc[b >> 1][b & 1][r] += slot[(b * 16 + r) * 64];

    // Lane (col, half) holds C[m = acc_row(r, half)][n = col] of each block:
    // for a fixed register, 32 lanes write 32 consecutive floats of a row
    // (whole 128-byte lines; 16-byte pieces of four columns measured slower).
    // Register r's row offset 8 (r >> 2) + (r & 3) is a compile-time
    // multiple of the uniform row stride; the lane adds 4 half rows + col.
    float *out = g.splits > 1 ? g.out + int64_t(sp) * g.M * g.N : g.out;
    const int mw = row0 + wm * 64, nw = col0 + wn * 64;
    const int lane_off = 4 * half * int(g.ldo) + col;
    if (row0 + BM <= g.M && col0 + BN <= g.N) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float *row = out + int64_t(mw + 32 * mb + 8 * (r >> 2) + (r & 3)) * g.ldo +
                                 nw + 32 * nb;
                    row[lane_off] = acc[mb][nb][r];
                }
    } else {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                const int n = nw + 32 * nb + col;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = mw + 32 * mb + acc_row(r, half);
                    if (m < g.M && n < g.N)
                        out[int64_t(m) * g.ldo + n] = acc[mb][nb][r];
                }
            }
    }
}

struct ReduceArgs {
    const float *part;
    float *c;
    int64_t ldc;
    int M, N, splits;
};

// C[m][n] = sum_s part[s][m][n], s in order; four columns per thread, every
// split's load issued before the adds.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(ReduceArgs r)
{
    const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
    const int n4 = r.N / 4;
    if (idx >= int64_t(r.M) * n4)
        return;
    const int m = int(idx / n4), n = int(idx - int64_t(m) * n4) * 4;
    const int64_t plane = int64_t(r.M) * r.N;
    const float *p = r.part + int64_t(m) * r.N + n;
    f32x4 v[kGemmMaxSplits];
#pragma unroll
    for (int s = 0; s < kGemmMaxSplits; ++s)
        if (s < r.splits)
            v[s] = *reinterpret_cast<const f32x4 *>(p + s * plane);
    f32x4 sum = v[0];
#pragma unroll
    for (int s = 1; s < kGemmMaxSplits; ++s)
        if (s < r.splits)
            sum += v[s];
    *reinterpret_cast<f32x4 *>(r.c + int64_t(m) * r.ldc + n) = sum;
}

struct GemmPlan {
    int tiles_m = 0, tiles_n = 0, splits = 1, chunks = 0;
};

// Splits of the K range: the largest divisor of the chunk count that keeps
// the grid at most kGemmTargetBlocks and every split at least kGemmMinChunks
// chunks long.  The partials then take at most kGemmTargetBlocks tiles of
// 64 KiB (16 MiB).
GemmPlan plan_of(int M, int N, int K)
{
    GemmPlan p;
    p.tiles_m = (M + kGemmTile - 1) / kGemmTile;
    p.tiles_n = (N + kGemmTile - 1) / kGemmTile;
    const int chunks = K / kGemmBK;
    const int tiles = p.tiles_m * p.tiles_n;
    const int want = std::min(kGemmMaxSplits, std::max(1, kGemmTargetBlocks / std::max(tiles, 1)));
    int best = 1;
    for (int s = 1; s <= want && s * kGemmMinChunks <= chunks; ++s)
        if (chunks % s == 0)
            best = s;
    p.splits = best;
    p.chunks = chunks / best;
    return p;
}

bool eligible(int M, int N, int K, int64_t lda, int64_t ldw, const void *a0, const void *a1,
              const void *w)
{
    const auto al = [](const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    return M > 0 && M <= kGemmMaxM && N > 0 && N % 4 == 0 && K > 0 && K % kGemmBK == 0 &&
           lda >= K && ldw >= K && lda % 8 == 0 && ldw % 8 == 0 && al(a0) && (!a1 || al(a1)) &&
           al(w) && int64_t(kGemmTile) * std::max(lda, ldw) * 2 < (int64_t(1) << 31);
}

}  // namespace

size_t gemm_bf16_workspace_bytes(int M, int N, int K)
{
    if (M <= 0 || M > kGemmMaxM || N <= 0 || K <= 0 || K % kGemmBK)
        return 0;
    const GemmPlan p = plan_of(M, N, K);
    return p.splits > 1 ? size_t(p.splits) * M * N * sizeof(float) : 0;
}

bool gemm_bf16_supported(int M, int N, int K, int64_t lda, int64_t ldw, int64_t ldc,
                         const void *a0, const void *a1, const void *w, const void *c,
                         size_t ws_bytes)
{
    return eligible(M, N, K, lda, ldw, a0, a1, w) && ldc >= N && ldc % 4 == 0 &&
           4 * ldc < (int64_t(1) << 28) && (reinterpret_cast<uintptr_t>(c) & 15) == 0 &&
           ws_bytes >= gemm_bf16_workspace_bytes(M, N, K);
}

namespace {

// The product as partial planes at g.out ([splits][M][N], or C itself with
// stride ldo when not split); returns the plan.
bool launch_parts(const uint16_t *a0, const uint16_t *a1, int64_t lda, const uint16_t *w,
                  int64_t ldw, float *out, int64_t ldo, int M, int N, const GemmPlan &p,
                  hipStream_t st)
{
    GemmArgs g;
    g.a0 = a0;
    g.a1 = a1;
    g.w = w;
    g.lda = lda;
    g.ldw = ldw;
    g.M = M;
    g.N = N;
    g.tiles_m = p.tiles_m;
    g.tiles_n = p.tiles_n;
    g.splits = p.splits;
    g.chunks = p.chunks;
    g.out = out;
    g.ldo = ldo;
    const int nblk = p.tiles_m * p.tiles_n * p.splits;
    if (a1)
        hipLaunchKernelGGL(gemm_bf16_kernel<true>, dim3(unsigned(nblk)), dim3(kGemmWaves * 64), 0,
                           st, g);
    else
        hipLaunchKernelGGL(gemm_bf16_kernel<false>, dim3(unsigned(nblk)), dim3(kGemmWaves * 64), 0,
                           st, g);
    return hip_ok(hipGetLastError(), "gemm_bf16_kernel launch");
}

}  // namespace

bool launch_gemm_bf16(const uint16_t *a0, const uint16_t *a1, int64_t lda, const uint16_t *w,
                      int64_t ldw, float *c, int64_t ldc, int M, int N, int K, void *ws,
                      size_t ws_bytes, hipStream_t st)
{
    if (!gemm_bf16_supported(M, N, K, lda, ldw, ldc, a0, a1, w, c, ws_bytes))
        return fail("gemm_bf16: unsupported shape, alignment or workspace");
    const GemmPlan p = plan_of(M, N, K);
    if (p.splits > 1 && (!ws || (reinterpret_cast<uintptr_t>(ws) & 15) != 0))
        return fail("gemm_bf16: split-K needs a 16-byte aligned workspace");
    if (!launch_parts(a0, a1, lda, w, ldw, p.splits > 1 ? static_cast<float *>(ws) : c,
                      p.splits > 1 ? N : ldc, M, N, p, st))
        return false;
    if (p.splits == 1)
        return true;
    ReduceArgs r;
    r.part = static_cast<const float *>(ws);
    r.c = c;
    r.ldc = ldc;
    r.M = M;
    r.N = N;
    r.splits = p.splits;
    const int64_t n = int64_t(M) * (N / 4);
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, r);
    return hip_ok(hipGetLastError(), "gemm_reduce_kernel launch");
}

bool launch_gemm_bf16_planes(const uint16_t *a0, const uint16_t *a1, int64_t lda,
                             const uint16_t *w, int64_t ldw, float *planes, size_t planes_bytes,
                             int M, int N, int K, int *parts, hipStream_t st)
{
    if (!parts || planes_bytes < size_t(M) * N * sizeof(float) ||
        !gemm_bf16_supported(M, N, K, lda, ldw, N, a0, a1, w, planes, planes_bytes))
        return fail("gemm_bf16: unsupported shape, alignment or room for the planes");
    const GemmPlan p = plan_of(M, N, K);
    *parts = p.splits;
    return launch_parts(a0, a1, lda, w, ldw, planes, N, M, N, p, st);
}

}  // namespace anima_hip
