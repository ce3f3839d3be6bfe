// Flash attention to f32 accuracy on bf16 MFMA (gfx950).
//
// Same computation as anima_rt_run_sdpa_flash (anima_rt/src/anima_rt.cpp:147-156 ->
// anima_rt/include/cpu/flash_attention.h:55-208) on f32 Q, K, V.  Both products
// run on v_mfma_f32_32x32x16_bf16, which is 16x faster than the f32 MFMA, with
// every f32 operand x split into two bf16 terms
//     xh = bf16(x),  xl = bf16(x - xh),   |x - xh - xl| <= 2^-17 |x|,
// and every product x*y taken as xh*yh + xh*yl + xl*yh (bf16 products are exact
// in f32; the dropped xl*yl and the residuals leave <= ~3 * 2^-17 relative per
// product), accumulated in f32:
//     S^T = K Q^T         as Kh Qh + Kh Ql + Kl Qh,
//     O^T += V^T P^T      as Vh Ph + Vh Pl + Vl Ph,  P = exp2(s*c - m) split
//                         the same way after the f32 softmax arithmetic;
// the row sum l adds the terms Ph + Pl the MFMAs consume.
//
// Layouts (bf16 bit patterns): Q and K rows of [hi(128) | lo(128)] per (batch,
// token, head), written by the row prologue; V^T per (batch, head) as
// [2 * 128 d-rows][Sp keys]: the 128 hi rows, then the 128 lo rows, keys in
// vt_key_pos order, zero past S_kv (vt_pack_terms_kernel below).
//
// Kernel shape (D = 128), per workgroup NW waves x 32 query rows, as the bf16
// kernel: transposed products (lane l holds query row l%32 in every
// accumulator), lane-local online softmax with one exchange between lanes l
// and l^32, lazy rescale of the running max.  Then:
//   * K tiles [64 keys][256] and V^T tiles [256][64 keys] (32 KiB each) reach
//     LDS by DMA through rings of two stages, one tile ahead, one barrier per
//     tile (128 KiB of LDS); XOR-swizzled like the bf16 kernel so fragment
//     reads are bank-conflict free;
//   * per tile and wave, 48 score MFMAs, then the softmax pipelined inside the
//     tile: the exponentials and term split of key chunk i+1 (16 keys) run on
//     the VALU between the 12 P.V MFMAs of chunk i.  The MFMA work of a tile
//     is about 2.4x its VALU work, and the second wave of each SIMD fills the
//     remaining issue gaps.
#include "qrow.h"

#include <cmath>

namespace anima_hip {
namespace {

using namespace flash_tile;

constexpr int kRow = 2 * kD;          // bf16 per Q/K term row: [hi | lo]
constexpr int kTile = kBN * kRow;     // bf16 per K or V^T tile (32 KiB)
static_assert(kTile == 2 * kD * kBN, "K and V^T tiles have the same size");

struct X3Args {
    const u16 *q, *k, *vt;
    float *o;
    int64_t qb, qh, qs, kb, kh, ks, vb, vh, vd, ob, oh, os;
    int H, S_q, S_kv, n_qtiles;
    float c;  // scale * log2(e), > 0
    int causal;
    int dma32;  // K/V^T tile rows fit 32-bit byte offsets from the tile start
    FlashSplitArgs split;  // n == 1: write O; n > 1: write this split's partial
    TermOut ot;            // n == 1 and ot.t set: O as bf16 terms
    // Raw query rows (RawQ) in place of q's term rows when qx is set.
    const float *qx, *qw, *qf;
    int64_t rqb, rqh, rqs;
    float eps;
};

template <int NW>
__global__ __launch_bounds__(NW * 64, 1) void flash_x3_d128(X3Args a)
{
    constexpr int NT = NW * 64;
    constexpr int BM = NW * 32;
    constexpr int DMA = kTile / 8 / NT;  // 16-byte copies per thread per tile
    static_assert(kTile / 8 % NT == 0, "tiles must split evenly");

    // K ring, then V^T ring, in one array: the epilogue reuses it whole.
    __shared__ __attribute__((aligned(16))) u16 smem[4 * kTile];
    u16 (*const Ks)[kTile] = reinterpret_cast<u16 (*)[kTile]>(smem);
    u16 (*const Vs)[kTile] = reinterpret_cast<u16 (*)[kTile]>(smem + 2 * kTile);
    static_assert(NW * kOWaveFloats * 4 <= int(sizeof(smem)), "O staging fits the rings");

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31;
    const int half = lane >> 5;

    const int blk = xcd_major_block();
    const int sp = blk % a.split.n;
    const int qt = (blk / a.split.n) % a.n_qtiles;
    const int bh = (blk / a.split.n) / a.n_qtiles;
    const int b = bh / a.H;
    const int h = bh - b * a.H;
    const int q_tile0 = qt * BM;
    const int qrow = q_tile0 + wave * 32 + col;

    const u16 *qp = a.q + b * a.qb + h * a.qh;
    const u16 *kp = a.k + b * a.kb + h * a.kh;
    const u16 *vp = a.vt + b * a.vb + h * a.vh;

    int kv_end = a.S_kv;
    if (a.causal)
        kv_end = min(kv_end, min(a.S_q, q_tile0 + BM));
    // Key tiles [j0, j0 + ntiles) of this split (all of them when unsplit).
    const int j0 = sp * a.split.tiles;
    const int ntiles = max(0, min((kv_end + kBN - 1) / kBN - j0, a.split.tiles));

    // LDS layouts, unpadded, XOR-swizzled (16-byte chunks):
    //   K   [64 keys][256]: chunk c (0..31; hi 0..15, lo 16..31) of key row r
    //       at c ^ (r & 15);
    //   V^T [256 rows][64 keys] (hi d-rows 0..127, lo 128..255): chunk c of
    //       row r at c ^ ((r >> 1) & 7).
    // Copy i of wave w fills physical chunks f = i*NT + 64w + lane of the
    // tile: K row f >> 5 = i*NT/32 + 2w + half, chunk col ^ (row & 15); V^T
    // row f >> 3 = i*NT/8 + 8w + lane/8.  With NT a multiple of 256 the V^T
    // swizzle term does not depend on i and the K term only on i's parity, so
    // a lane's source offset is one register (two for K) plus a uniform step
    // per copy (247 -> 231 VGPRs at NW = 8).
    const int krl = 2 * wave + half;  // K row of copy 0
    unsigned koff_b[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = col ^ ((i * (NT / 32) + krl) & 15);
        koff_b[i] = unsigned(krl * a.ks + 8 * c) * 2u;
    }
    const int vrl = 8 * wave + (lane >> 3);  // V^T row of copy 0
    const int vcl = (lane & 7) ^ ((vrl >> 1) & 7);
    const unsigned voff_b = unsigned(vrl * a.vd + 8 * vcl) * 2u;
    static_assert(NT % 256 == 0, "copy offsets assume whole 256-thread groups");
    auto dma_k = [&](int t, int stage) {
        const int key0 = (j0 + t) * kBN;
        if (a.dma32 && key0 + kBN <= a.S_kv) {
            const u16 *base = kp + int64_t(key0) * a.ks;
#pragma unroll
            for (int i = 0; i < DMA; ++i)
                dma16s(base + int64_t(i * (NT / 32)) * a.ks, koff_b[i & 1],
                       &Ks[stage][(i * NT + 64 * wave) * 8]);
        } else {
            // Keys past S_kv copy row S_kv - 1; their scores are masked.
#pragma unroll
            for (int i = 0; i < DMA; ++i) {
                const int r = i * (NT / 32) + krl;
                const int key = min(key0 + r, a.S_kv - 1);
                dma16(kp + key * a.ks + 8 * (col ^ (r & 15)), &Ks[stage][(i * NT + 64 * wave) * 8]);
            }
        }
    };
    auto dma_v = [&](int t, int stage) {
        // V^T is zero-padded in HBM to whole tiles.
        const int key0 = (j0 + t) * kBN;
        if (a.dma32) {
            const u16 *base = vp + key0;
#pragma unroll
            for (int i = 0; i < DMA; ++i)
                dma16s(base + int64_t(i * (NT / 8)) * a.vd, voff_b,
                       &Vs[stage][(i * NT + 64 * wave) * 8]);
        } else {
#pragma unroll
            for (int i = 0; i < DMA; ++i)
                dma16(vp + (i * (NT / 8) + vrl) * a.vd + key0 + 8 * vcl,
                      &Vs[stage][(i * NT + 64 * wave) * 8]);
        }
    };
    // Fragments: K key row col + 32*kb, term chunk 16*term + 8*half + t;
    // V^T row 128*term + 32*blk + col, keys [16i, 16i+16) (chunk half + 2i).
    const int ksw = col & 15, vsw = (col >> 1) & 7;
    auto kfrag = [&](const u16 *kst, int t, int kb, int term) {
        return *reinterpret_cast<const bf16x8 *>(
            kst + (col + 32 * kb) * kRow + 8 * (16 * term + (((half << 3) | t) ^ ksw)));
    };
    auto vfrag = [&](const u16 *vst, int blk, int i, int term) {
        return *reinterpret_cast<const bf16x8 *>(
            vst + (128 * term + 32 * blk + col) * kBN + 8 * ((half + 2 * i) ^ vsw));
    };

    f32x16 o0 = {}, o1 = {}, o2 = {}, o3 = {};
    float m = -INFINITY;
    float l = 0.0f, l2 = 0.0f;  // row sums of the hi and lo P terms
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};

    // Q terms: hi Q[qrow][64*half + 8t .. +7], lo 128 elements further.
    bf16x8 qh[8], ql[8];
    if (!a.qx) {
        if (qrow < a.S_q) {
            const bf16x8 *src = reinterpret_cast<const bf16x8 *>(qp + qrow * a.qs + 64 * half);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                qh[t] = src[t];
                ql[t] = src[kD / 8 + t];
            }
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t)
                qh[t] = ql[t] = bf16x8{};
        }
        // Retire the Q loads before the loop, whose vmcnt waits count only
        // copies.
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
    }
    if (ntiles > 0) {
        dma_k(0, 0);
        dma_v(0, 0);
    }
    // Raw query rows are prepared while the first tile's copies are in
    // flight (issued first, so the two latencies overlap).  Prepared rows
    // load first: copies first cost a small 4-wave grid (256 x 512 keys,
    // B = 2, H = 16) 3 %.
    if (a.qx) {
        const int r = min(qrow, a.S_q - 1);
        q_terms_from_raw(a.qx + b * a.rqb + h * a.rqh + int64_t(r) * a.rqs, a.qw,
                         a.qf ? a.qf + int64_t(r) * 4 * kD / 2 : nullptr, a.eps, qrow < a.S_q,
                         half, qh, ql);
    }
    wait_vmcnt<0>();
    ring_barrier();

    for (int j = 0; j < ntiles; ++j) {
        const int st = j & 1;
        // Tile j+1 into the other stage, read by every wave in iteration j-1
        // (before the barrier that ended it).  A copy instruction holds its
        // wave at issue for about a hundred cycles, so the two waves of a
        // SIMD (w and w + 4, waves being placed round-robin on the four
        // SIMDs) do not issue theirs together: waves 0-3 right after the
        // barrier, waves 4-7 after their score MFMAs (1.0-1.4 % faster at
        // 4096 tokens than all waves at the top of the tile).
        const bool late_copies = (wave >> 2) & 1;
        const bool copy_next = j + 1 < ntiles;
        if (copy_next && !late_copies) {
            dma_k(j + 1, st ^ 1);
            dma_v(j + 1, st ^ 1);
        }
        const u16 *kst = Ks[st];
        const u16 *vst = Vs[st];

        // ---- Scores S^T of keys [0,32) in s0, [32,64) in s1; the K fragments
        // of step t+1 are read while the MFMAs of step t run.
        f32x16 s0 = {}, s1 = {};
        bf16x8 kf[2][4];
        auto read_k = [&](int t) {
            kf[t & 1][0] = kfrag(kst, t, 0, 0);
            kf[t & 1][1] = kfrag(kst, t, 1, 0);
            kf[t & 1][2] = kfrag(kst, t, 0, 1);
            kf[t & 1][3] = kfrag(kst, t, 1, 1);
        };
        // V^T fragments (hi, lo) of P.V step n = 4*chunk + blk, two steps ahead.
        bf16x8 vh[3], vl[3];
        auto read_v = [&](int n) {
            vh[n % 3] = vfrag(vst, n & 3, n >> 2, 0);
            vl[n % 3] = vfrag(vst, n & 3, n >> 2, 1);
        };
        read_k(0);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            if (t < 7)
                read_k(t + 1);
            else {
                read_v(0);
                read_v(1);
            }
            const bf16x8 *k = kf[t & 1];
            s0 = mfma_bf16(k[0], qh[t], s0);
            s1 = mfma_bf16(k[1], qh[t], s1);
            s0 = mfma_bf16(k[0], ql[t], s0);
            s1 = mfma_bf16(k[1], ql[t], s1);
            s0 = mfma_bf16(k[2], qh[t], s0);
            s1 = mfma_bf16(k[3], qh[t], s1);
            __builtin_amdgcn_sched_barrier(0);
        }

        if (copy_next && late_copies) {
            dma_k(j + 1, st ^ 1);
            dma_v(j + 1, st ^ 1);
        }

        // ---- Mask (tail tile, causal), tile max, lazy rescale.
        const int key0 = (j0 + j) * kBN;
        if ((key0 + kBN > a.S_kv) || a.causal) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int k0i = key0 + acc_row(r, half);
                const int k1i = k0i + 32;
                if (k0i >= a.S_kv || (a.causal && k0i > qrow))
                    s0[r] = -INFINITY;
                if (k1i >= a.S_kv || (a.causal && k1i > qrow))
                    s1[r] = -INFINITY;
            }
        }
        float mx0 = -INFINITY, mx1 = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
            mx0 = fmaxf(mx0, fmaxf(s0[r], s0[r + 1]));
            mx1 = fmaxf(mx1, fmaxf(s1[r], s1[r + 1]));
        }
        // Raw-score max (c > 0, so it commutes with the scaling).  The
        // reference max m (log2 units) moves only when some row of the wave
        // exceeds it by more than kRescaleLog2, for the whole wave at once;
        // otherwise p <= 2^kRescaleLog2 and O, l keep accumulating against
        // the same m (exact, since the final O / l shares it).
        const float cand = row_pair_max(fmaxf(mx0, mx1)) * a.c;
        if (__any(cand > m + kRescaleLog2)) {
            const float m_new = fmaxf(m, cand);
            const float alpha =
                m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - m_new);
            m = m_new;
            l *= alpha;
            l2 *= alpha;
            o0 *= alpha;
            o1 *= alpha;
            o2 *= alpha;
            o3 *= alpha;
        }
        const float neg_m = (m == -INFINITY) ? 0.0f : -m;

        // ---- P terms of key chunk i (keys [16i, 16i+16): accumulator
        // registers 8*(i&1) .. +7 of s0 for i < 2, of s1 otherwise), pair q
        // (registers 2q, 2q+1 of those 8), into ph/pl; the row sums add the
        // terms.
        bf16x8 ph[2], pl[2];
        // This tile's row sums start from zero and join l, l2 once per tile:
        // over millions of keys a running sum fed one pair at a time rounds
        // away its smallest terms.
        float t = 0.0f, t2 = 0.0f;
        auto p_pair = [&](int i, int q) {
            const f32x16 &s = i < 2 ? s0 : s1;
            const int r = 8 * (i & 1) + 2 * q;
            const float e0 = __builtin_amdgcn_exp2f(fmaf(s[r], a.c, neg_m));
            const float e1 = __builtin_amdgcn_exp2f(fmaf(s[r + 1], a.c, neg_m));
            const bf16x2 hi = __builtin_convertvector(f32x2{e0, e1}, bf16x2);
            const bf16x2 lo =
                __builtin_convertvector(f32x2{e0 - float(hi[0]), e1 - float(hi[1])}, bf16x2);
            ph[i & 1][2 * q] = hi[0];
            ph[i & 1][2 * q + 1] = hi[1];
            pl[i & 1][2 * q] = lo[0];
            pl[i & 1][2 * q + 1] = lo[1];
            t = __builtin_amdgcn_fdot2_f32_bf16(hi, one, t, false);
            t2 = __builtin_amdgcn_fdot2_f32_bf16(lo, one, t2, false);
        };
#pragma unroll
        for (int q = 0; q < 4; ++q)
            p_pair(0, q);

        // ---- P.V: step n = 4*i + blk issues the three MFMAs of d block blk
        // and key chunk i, reads the V^T fragments of step n+2 and computes
        // one pair of chunk i+1's P terms.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int blk = 0; blk < 4; ++blk) {
                const int n = 4 * i + blk;
                if (n + 2 < 16)
                    read_v(n + 2);
                f32x16 &ob = blk == 0 ? o0 : blk == 1 ? o1 : blk == 2 ? o2 : o3;
                ob = mfma_bf16(vh[n % 3], ph[i & 1], ob);
                ob = mfma_bf16(vh[n % 3], pl[i & 1], ob);
                ob = mfma_bf16(vl[n % 3], ph[i & 1], ob);
                if (i < 3)
                    p_pair(i + 1, blk);
                __builtin_amdgcn_sched_barrier(0);
            }
        }

        l += t;
        l2 += t2;

        // Tile j+1's copies (this iteration's) complete, then visible to all.
        wait_vmcnt<0>();
        ring_barrier();
    }

    l += l2;
    l += __shfl_xor(l, 32);
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    // Every score of the row masked or NaN: the reference leaves zeros.
    const bool dead = m == -INFINITY;
    const int row0 = q_tile0 + wave * 32;
    float *op = a.o + b * a.ob + h * a.oh + row0 * a.os;
    int64_t ostride = a.os;
    u16 *tp = a.ot.t ? a.ot.t + b * a.ot.tb + h * a.ot.th + row0 * a.ot.ts : nullptr;
    if (a.split.n > 1) {
        tp = nullptr;
        const int64_t prow0 = (int64_t(sp) * a.split.BH + bh) * a.S_q + row0;
        op = a.split.part + prow0 * kD;
        ostride = kD;
        if (half == 0 && qrow < a.S_q)
            a.split.ml[prow0 + col] = make_float2(m, dead ? 0.0f : l);
    }
    // Every wave has passed the loop's last barrier: the rings are free.
    store_o_rows(reinterpret_cast<float *>(smem) + wave * kOWaveFloats, o0, o1, o2, o3, inv, dead,
                 op, ostride, a.S_q - row0, tp, a.ot.ts, a.ot.lo);
}

// V (f32, [B,H,S,D] view, D = 128) -> packed bf16 term V^T [B,H][2D][Sp]:
// rows d hold bf16(v), rows D + d hold bf16(v - bf16(v)).  One block per
// (batch*head, 64-key tile): coalesced float4 reads of the V rows, transpose
// through LDS (each thread converts a pair of adjacent keys, which
// vt_key_pos keeps adjacent, into one 32-bit LDS word per term), 16-byte
// coalesced writes along the key axis.
struct PackArgs {
    const float *v;
    u16 *vt;
    int64_t vb, vh, vs, tb, th;
    int H, S_kv, n_tiles;
    int64_t sp;
};

constexpr int kTPitchW = (kBN + 8) / 2;  // 32-bit words per LDS row of a transposed tile

__global__ __launch_bounds__(256) void vt_pack_terms_kernel(PackArgs a)
{
    __shared__ __attribute__((aligned(16))) unsigned int Th[kD * kTPitchW];
    __shared__ __attribute__((aligned(16))) unsigned int Tl[kD * kTPitchW];
    const int tile = blockIdx.x % a.n_tiles;
    const int bh = blockIdx.x / a.n_tiles;
    const int b = bh / a.H, h = bh - b * a.H;
    const int key0 = tile * kBN;
    const float *vp = a.v + b * a.vb + h * a.vh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int f = threadIdx.x + 256 * i;  // (key pair, float4 column) of the tile
        const int pr = f >> 5, c4 = f & 31;
        const int k0 = key0 + 2 * pr, k1 = k0 + 1;
        const f32x4 x0 = k0 < a.S_kv ? *reinterpret_cast<const f32x4 *>(vp + k0 * a.vs + 4 * c4)
                                     : f32x4{0.f, 0.f, 0.f, 0.f};
        const f32x4 x1 = k1 < a.S_kv ? *reinterpret_cast<const f32x4 *>(vp + k1 * a.vs + 4 * c4)
                                     : f32x4{0.f, 0.f, 0.f, 0.f};
        const int w = vt_key_pos(2 * pr) >> 1;  // word holding positions (2w, 2w+1)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const bf16x2 hi = __builtin_convertvector(f32x2{x0[e], x1[e]}, bf16x2);
            const bf16x2 lo =
                __builtin_convertvector(f32x2{x0[e] - float(hi[0]), x1[e] - float(hi[1])}, bf16x2);
            Th[(4 * c4 + e) * kTPitchW + w] = __builtin_bit_cast(unsigned int, hi);
            Tl[(4 * c4 + e) * kTPitchW + w] = __builtin_bit_cast(unsigned int, lo);
        }
    }
    __syncthreads();
    u16 *tp = a.vt + b * a.tb + h * a.th + key0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int f = threadIdx.x + 256 * i;  // 16-byte chunk: d row, 8 keys
        const int d = f >> 3, c = f & 7;
        *reinterpret_cast<f32x4 *>(tp + d * a.sp + 8 * c) =
            *reinterpret_cast<const f32x4 *>(&Th[d * kTPitchW + 4 * c]);
        *reinterpret_cast<f32x4 *>(tp + (kD + d) * a.sp + 8 * c) =
            *reinterpret_cast<const f32x4 *>(&Tl[d * kTPitchW + 4 * c]);
    }
}

template <int NW>
bool launch_d128(const X3Args &a, int64_t BH, hipStream_t st)
{
    constexpr int BM = NW * 32;
    X3Args g = a;
    g.n_qtiles = (g.S_q + BM - 1) / BM;
    const int64_t nblk = BH * g.n_qtiles * g.split.n;
    if (nblk > INT32_MAX)
        return fail("flash_x3: problem too large for one launch");
    hipLaunchKernelGGL(flash_x3_d128<NW>, dim3(unsigned(nblk)), dim3(NW * 64), 0, st, g);
    return hip_ok(hipGetLastError(), "flash_x3_d128 launch");
}

}  // namespace

bool launch_flash_x3(const FlashProblem &p, hipStream_t st, void *part, size_t part_bytes)
{
    const int64_t BH = int64_t(p.B) * p.H;
    if (BH == 0 || p.S_q == 0)
        return true;
    if (p.D != kD)
        return fail("flash_x3: head dim must be 128 (got " + std::to_string(p.D) + ")");
    if (!(p.scale > 0.0f) || !std::isfinite(p.scale))
        return fail("flash_x3: scale must be positive");
    const int64_t sp = vt_padded_len(p.S_kv);
    if (p.vs.s != sp)
        return fail("flash_x3: V^T row stride must equal the padded key count");
    // Every Q/K row is read as 2*D elements ([hi | lo]): a row stride below
    // that (e.g. a dense row of D values) would read past the tensor's end.
    const auto rows_fit = [](const Strides &x) {
        for (const int64_t v : {x.b, x.h, x.s})
            if (v != 0 && (v < 0 || v < kRow))
                return false;
        return true;
    };
    const bool raw_q = p.rq.x != nullptr;  // q's term rows unused
    if ((!raw_q && !rows_fit(p.qs)) || !rows_fit(p.ks))
        return fail("flash_x3: q/k strides must leave 2*D = 256 elements per row (hi | lo terms)");
    // Each (batch, head) of the term V^T holds 2*D rows of Sp keys.
    for (const int64_t v : {p.vs.b, p.vs.h})
        if (v != 0 && (v < 0 || v < int64_t(2 * kD) * vt_padded_len(p.S_kv)))
            return fail("flash_x3: V^T batch/head strides must leave 2*D rows of the padded key "
                        "count per head");
    const auto s8 = [](const Strides &x) { return x.b % 8 == 0 && x.h % 8 == 0 && x.s % 8 == 0; };
    if ((!raw_q && (!aligned(p.q, 16) || !s8(p.qs))) || !aligned(p.k, 16) || !aligned(p.v, 16) ||
        !aligned(p.o, 16) || !s8(p.ks) || !s8(p.vs) || p.os.b % 4 || p.os.h % 4 || p.os.s % 4)
        return fail("flash_x3: operands must be 16-byte aligned with 16-byte row strides");
    if (raw_q) {
        const Strides &x = p.rq.s;
        if (!aligned(p.rq.x, 16) || x.b % 4 || x.h % 4 || x.s % 4 ||
            (p.rq.w && !aligned(p.rq.w, 16)) || (p.rq.freqs && !aligned(p.rq.freqs, 16)))
            return fail("flash_x3: raw query rows must be 16-byte aligned with 16-byte strides");
    }
    if (p.ot.t && !term_out_ok(p.ot))
        return fail("flash_x3: term output must be 16-byte aligned with strides of 8 elements");
    X3Args a;
    a.q = static_cast<const u16 *>(p.q);
    a.k = static_cast<const u16 *>(p.k);
    a.vt = static_cast<const u16 *>(p.v);
    a.o = p.o;
    a.qb = p.qs.b; a.qh = p.qs.h; a.qs = p.qs.s;
    a.kb = p.ks.b; a.kh = p.ks.h; a.ks = p.ks.s;
    a.vb = p.vs.b; a.vh = p.vs.h; a.vd = sp;
    a.ob = p.os.b; a.oh = p.os.h; a.os = p.os.s;
    a.ot = p.ot;
    a.H = p.H;
    a.S_q = p.S_q;
    a.S_kv = p.S_kv;
    a.c = p.scale * kLog2e;
    a.causal = p.causal ? 1 : 0;
    // Byte offsets of a tile's rows from its first row: K rows r < 64 at
    // r*ks, V^T rows r < 256 at r*Sp, plus one row of 512 bytes.
    a.dma32 = (int64_t(kBN) * p.ks.s * 2 + 512 < (int64_t(1) << 31)) &&
              (int64_t(2 * kD) * sp * 2 + 512 < (int64_t(1) << 31));
    a.qx = p.rq.x;
    a.qw = p.rq.w;
    a.qf = p.rq.freqs;
    a.rqb = p.rq.s.b; a.rqh = p.rq.s.h; a.rqs = p.rq.s.s;
    a.eps = p.rq.eps;
    const FlashPlan pl = flash_plan(BH, p.S_q, p.S_kv, p.D, kTileUsX3);
    a.split = flash_split_args(pl, BH, p.S_q, part, part_bytes);
    if (!(pl.waves == 4 ? launch_d128<4>(a, BH, st) : launch_d128<8>(a, BH, st)))
        return false;
    return a.split.n == 1 || launch_flash_combine(p, a.split, st);
}

bool launch_vt_pack_terms(const float *v, Strides vs, uint16_t *vt, Strides vts, int B, int H,
                          int S_kv, int D, hipStream_t st)
{
    const int64_t BH = int64_t(B) * H;
    if (BH == 0 || S_kv == 0)
        return true;
    if (D != kD)
        return fail("vt_pack_terms: head dim must be 128");
    if (!aligned(v, 16) || !aligned(vt, 16) || vs.b % 4 || vs.h % 4 || vs.s % 4 || vts.b % 8 ||
        vts.h % 8)
        return fail("vt_pack_terms: operands must be 16-byte aligned");
    PackArgs a;
    a.v = v;
    a.vt = vt;
    a.vb = vs.b; a.vh = vs.h; a.vs = vs.s;
    a.tb = vts.b; a.th = vts.h;
    a.H = H;
    a.S_kv = S_kv;
    a.sp = vt_padded_len(S_kv);
    a.n_tiles = int(a.sp / kBN);
    const int64_t nblk = BH * a.n_tiles;
    if (nblk > INT32_MAX)
        return fail("vt_pack_terms: problem too large for one launch");
    hipLaunchKernelGGL(vt_pack_terms_kernel, dim3(unsigned(nblk)), dim3(256), 0, st, a);
    return hip_ok(hipGetLastError(), "vt_pack_terms_kernel launch");
}

}  // namespace anima_hip
