// Flash attention with bf16 inputs, bf16 MFMA and f32 accumulation (gfx950).
//
// Same computation as anima_rt_run_sdpa_flash (anima_rt/src/anima_rt.cpp:147-156 ->
// anima_rt/include/cpu/flash_attention.h:55-208) with Q, K, V and the softmax
// probabilities P rounded to bf16 before the two products; scores, the
// online max/sum and the output accumulate in f32.
//
// Kernel shape (D = 128), per workgroup NW waves x 32 query rows:
//   * S^T = K Q^T with v_mfma_f32_32x32x16_bf16; lane l holds query row l%32
//     in every accumulator (lane-local softmax, one exchange with lane l^32);
//   * O^T += V^T P^T with the same instruction: P's B operand is the S^T
//     accumulator converted to bf16 in place (8 consecutive accumulator
//     registers = 8 keys); V^T's A operand is one 16-byte LDS read thanks to
//     the key order of the packed V^T (vt_key_pos);
//   * K tiles [64 keys][128 d] and V^T tiles [128 d][64 keys] reach LDS by
//     DMA (global_load_lds) through rings of three stages, one barrier per
//     tile; rows are unpadded and XOR-swizzled in 16-byte chunks so the
//     per-lane 16-byte fragment reads are bank-conflict free;
//   * software-pipelined per wave: the MFMAs computing the scores of tile
//     j+1 are interleaved (sched_barrier) with the VALU softmax of tile j,
//     then P.V of tile j follows, so the MFMA pipe and the VALU overlap
//     inside every wave; LDS fragments are read two MFMA pairs ahead of use
//     and the compute section runs at raised wave priority (s_setprio);
//   * the row sum l accumulates the bf16-rounded P that the P.V MFMAs use;
//   * the softmax scale is folded into the exponent: p = exp2(s*c - m) with
//     c = scale*log2(e) > 0, so the tile max is taken on raw scores; the
//     running max m is updated lazily (only when a tile max exceeds it by
//     more than 8 in log2 units), so the O rescale is usually skipped.
// Also here: the V -> packed V^T conversion kernel of this path.
#include "qrow.h"

#include <cmath>

namespace anima_hip {
namespace {

using namespace flash_tile;

constexpr int kTileElems = kBN * kD;  // bf16 per K or V^T tile (16 KiB)
// Short key ranges (cross-attention over a 512-token context: 8 tiles per
// workgroup) on grids of at least one 8-wave workgroup per CU run as 4-wave
// workgroups with two-stage rings (64 KiB of LDS, at most 256 VGPRs), two
// per CU: one workgroup's query load and output stores, which a workgroup of
// 8 tiles cannot hide behind its own MFMA work, overlap the other's tiles.
constexpr int kPairMaxTiles = 16;

struct Bf16Args {
    const u16 *q, *k, *vt;
    float *o;
    int64_t qb, qh, qs, kb, kh, ks, vb, vh, vd, ob, oh, os;
    int H, S_q, S_kv, n_qtiles;
    float c;  // scale * log2(e), > 0
    int causal;
    int dma32;  // K/V^T tile rows fit 32-bit byte offsets from the tile start
    FlashSplitArgs split;  // n == 1: write O; n > 1: write this split's partial
    TermOut ot;            // n == 1 and ot.t set: O as bf16 terms
    // Raw query rows (RawQ) in place of q's bf16 rows when qx is set.
    const float *qx, *qw, *qf;
    int64_t rqb, rqh, rqs;
    float eps;
};

// NW waves x 32 query rows per workgroup, K/V^T rings of ST stages.  The
// two-stage form is held to two waves per SIMD (256 VGPRs), so that two
// 4-wave workgroups share a CU.
template <int NW, int ST>
__global__ __launch_bounds__(NW * 64, ST == 2 ? 2 : 1) void flash_bf16_d128(Bf16Args a)
{
    constexpr int NT = NW * 64;
    constexpr int BM = NW * 32;
    constexpr int DMA = kTileElems / 8 / NT;  // 16-byte copies per thread per tile
    static_assert(kTileElems / 8 % NT == 0, "tiles must split evenly");
    static_assert(ST == 2 || ST == 3, "two- or three-stage rings");

    // K ring, then V^T ring, in one array: the epilogue reuses it whole.
    __shared__ __attribute__((aligned(16))) u16 smem[2 * ST * kTileElems];
    u16 (*const Ks)[kTileElems] = reinterpret_cast<u16 (*)[kTileElems]>(smem);
    u16 (*const Vs)[kTileElems] = reinterpret_cast<u16 (*)[kTileElems]>(smem + ST * kTileElems);
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

    // Q fragment: Q[qrow][64*half + 8t .. +7], t = 0..7.
    bf16x8 qf[8];
    if (!a.qx) {
        if (qrow < a.S_q) {
            const bf16x8 *src = reinterpret_cast<const bf16x8 *>(qp + qrow * a.qs + 64 * half);
#pragma unroll
            for (int t = 0; t < 8; ++t)
                qf[t] = src[t];
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t)
                qf[t] = bf16x8{};
        }
        // Retire the Q loads here.  Otherwise the compiler still counts them
        // as outstanding inside the tile loop and waits for vmcnt(0) before
        // the first MFMAs, which also waits for the next tile's prefetch.
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
    }

    int kv_end = a.S_kv;
    if (a.causal)
        kv_end = min(kv_end, min(a.S_q, q_tile0 + BM));
    // Key tiles [j0, j0 + ntiles) of this split (all of them when unsplit).
    const int j0 = sp * a.split.tiles;
    const int ntiles = max(0, min((kv_end + kBN - 1) / kBN - j0, a.split.tiles));

    // K and V^T tiles reach LDS by DMA through rings of ST buffers: tile t
    // lives in stage t % ST.  Iteration j reads K(j+1) (scores of the next
    // tile) and V^T(j) (P.V of this tile) and starts the copies of K(j+ST) and
    // V^T(j+ST-1): with three stages they have two iterations to land, with
    // two stages one.
    // Layouts, unpadded, XOR-swizzled so every 16-lane group of a fragment
    // read hits distinct banks:
    //   K   [64 keys][128 d]: 16-byte chunk c of key row r at chunk c ^ (r & 15);
    //   V^T [128 d][64 keys]: chunk c of d row r at chunk c ^ ((r >> 1) & 7).
    // Keys past S_kv copy row S_kv - 1 (their scores are masked); V^T is
    // zero-padded in HBM to whole tiles.
    // This lane's source chunks: window w = wave*DMA + i of a tile, chunk
    // slot f = 64w + lane; byte offsets from the tile's first row (whole
    // tiles, with dma32) or the row index for the clamped path.
    unsigned koff_b[DMA], voff_b[DMA];
    int krow[DMA], kchk[DMA];
#pragma unroll
    for (int i = 0; i < DMA; ++i) {
        const int f = (wave * DMA + i) * 64 + lane;
        const int r = f >> 4, c = (f & 15) ^ (r & 15);
        krow[i] = r;
        kchk[i] = c;
        koff_b[i] = unsigned(r * a.ks + 8 * c) * 2u;
        const int rv = f >> 3, cv = (f & 7) ^ ((rv >> 1) & 7);
        voff_b[i] = unsigned(rv * a.vd + 8 * cv) * 2u;
    }
    auto dma_k = [&](int t, int stage) {
        const int key0 = (j0 + t) * kBN;
        if (a.dma32 && key0 + kBN <= a.S_kv) {
            const u16 *base = kp + int64_t(key0) * a.ks;
#pragma unroll
            for (int i = 0; i < DMA; ++i)
                dma16s(base, koff_b[i], &Ks[stage][(wave * DMA + i) * 512]);
        } else {
#pragma unroll
            for (int i = 0; i < DMA; ++i) {
                const int key = min(key0 + krow[i], a.S_kv - 1);
                dma16(kp + key * a.ks + 8 * kchk[i], &Ks[stage][(wave * DMA + i) * 512]);
            }
        }
    };
    auto dma_v = [&](int t, int stage) {
        const int key0 = (j0 + t) * kBN;
        if (a.dma32) {
            const u16 *base = vp + key0;
#pragma unroll
            for (int i = 0; i < DMA; ++i)
                dma16s(base, voff_b[i], &Vs[stage][(wave * DMA + i) * 512]);
        } else {
#pragma unroll
            for (int i = 0; i < DMA; ++i) {
                const int f = (wave * DMA + i) * 64 + lane;
                const int r = f >> 3, c = (f & 7) ^ ((r >> 1) & 7);
                dma16(vp + r * a.vd + key0 + 8 * c, &Vs[stage][(wave * DMA + i) * 512]);
            }
        }
    };
    // Element offsets of this lane's fragments inside a stage: K rows col and
    // col + 32, chunk 8*half + t; V^T rows col + 32*blk, chunk half + 2i.
    const int ksw = col & 15, vsw = (col >> 1) & 7;
    auto koff = [&](int t) { return col * kD + 8 * (((half << 3) | t) ^ ksw); };
    auto voff = [&](int i) { return col * kBN + 8 * ((half + 2 * i) ^ vsw); };
    // S^T of one 64-key tile from K stage `stage`: keys [0,32) in s0,
    // [32,64) in s1.
    auto scores = [&](int stage, f32x16 &s0, f32x16 &s1) {
        s0 = f32x16{};
        s1 = f32x16{};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const bf16x8 k0 = *reinterpret_cast<const bf16x8 *>(&Ks[stage][koff(t)]);
            const bf16x8 k1 = *reinterpret_cast<const bf16x8 *>(&Ks[stage][koff(t) + 32 * kD]);
            s0 = mfma_bf16(k0, qf[t], s0);
            s1 = mfma_bf16(k1, qf[t], s1);
        }
    };

    f32x16 o0 = {}, o1 = {}, o2 = {}, o3 = {};
    float m = -INFINITY;
    float l = 0.0f, l2 = 0.0f;  // two running row sums (chains of v_dot2)
    // Scores of two consecutive tiles; the loop below is unrolled by two so
    // the pair being consumed and the pair being produced swap roles without
    // register copies.
    f32x16 sa0 = {}, sa1 = {}, sb0 = {}, sb1 = {};

    if (ntiles > 0) {
        dma_k(0, 0);
        if (ntiles > 1)
            dma_k(1, 1);
        dma_v(0, 0);
    }
    // Raw query rows are prepared while the first tiles' copies are in
    // flight.
    if (a.qx) {
        const int r = min(qrow, a.S_q - 1);
        bf16x8 unused[8];
        q_terms_from_raw<false>(a.qx + b * a.rqb + h * a.rqh + int64_t(r) * a.rqs, a.qw,
                                a.qf ? a.qf + int64_t(r) * 4 * kD / 2 : nullptr, a.eps,
                                qrow < a.S_q, half, qf, unused);
    }
    wait_vmcnt<0>();
    ring_barrier();
    if (ntiles > 0)
        scores(0, sa0, sa1);
    if (ST == 3) {
        if (ntiles > 2)
            dma_k(2, 2);
        if (ntiles > 1)
            dma_v(1, 1);
    }
    ring_barrier();  // K stage 0 is rewritten in the first iteration

    // Raw-score tile max over a lane's 32 scores, combined across the two
    // lanes of the row (c > 0, so the max commutes with the scaling).
    auto tile_max = [&](const f32x16 &s0, const f32x16 &s1) {
        float a0 = -INFINITY, a1 = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
            a0 = fmaxf(a0, fmaxf(s0[r], s0[r + 1]));
            a1 = fmaxf(a1, fmaxf(s1[r], s1[r + 1]));
        }
        return row_pair_max(fmaxf(a0, a1));
    };
    // Max of the unmasked scores of the tile consumed next; the pipelined
    // section computes it for tile j+1 while the P.V MFMAs of tile j run.
    float mx_next = ntiles > 0 ? tile_max(sa0, sa1) : -INFINITY;

    // Tile j: consumes the scores sc0/sc1 of tile j, produces sn0/sn1 of
    // tile j+1.
    auto tile = [&](const int j, f32x16 &sc0, f32x16 &sc1, f32x16 &sn0, f32x16 &sn1) {
        const int sv = j % ST, sk = (j + 1) % ST;  // stages of V^T(j), K(j+1)
        const bool dk = j + ST < ntiles, dv = j + ST - 1 < ntiles;
        if (dk)
            dma_k(j + ST, sv);
        if (dv)
            dma_v(j + ST - 1, (j + ST - 1) % ST);

        float mx = mx_next;
        const int key0 = (j0 + j) * kBN;
        if ((key0 + kBN > a.S_kv) || a.causal) {
            // Tail tile or causal: mask, then take the max again.
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int k0i = key0 + acc_row(r, half);
                const int k1i = k0i + 32;
                if (k0i >= a.S_kv || (a.causal && k0i > qrow))
                    sc0[r] = -INFINITY;
                if (k1i >= a.S_kv || (a.causal && k1i > qrow))
                    sc1[r] = -INFINITY;
            }
            mx = tile_max(sc0, sc1);
        }

        // Lazy rescale: the reference max m (log2 domain) moves only when some
        // row of the wave sees a tile max above m + kRescaleLog2, and then for
        // the whole wave at once; otherwise exp2 values stay <= 2^kRescaleLog2
        // and O, l keep accumulating against the same m (exact, since the
        // final O / l shares it).  The rare rescale happens here, before the
        // branch-free pipelined section below.
        const float cand = mx * a.c;
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

        // ---- Pipelined section, one basic block, hand-interleaved.  Step t
        // issues the K reads of step t+2, one score MFMA of tile j+1, two
        // exponentials of tile j, the other score MFMA and two more
        // exponentials; the last two steps also read the V^T fragments of the
        // first P.V block.  sched_barrier keeps the steps in this order so the
        // MFMA pipe and the VALU work side by side and every LDS read has two
        // MFMA pairs to land.  (On the last tile the next K buffer holds stale
        // data; those scores are never used.)  The wave runs this section at
        // raised priority, so a wave still storing tiles or waiting at the
        // barrier yields issue slots to it.
        const u16 *kst = Ks[sk];
        const u16 *vst = Vs[sv];
        bf16x8 kf0[8], kf1[8], vf[4][4];
        auto read_k = [&](int t) {
            kf0[t] = *reinterpret_cast<const bf16x8 *>(kst + koff(t));
            kf1[t] = *reinterpret_cast<const bf16x8 *>(kst + koff(t) + 32 * kD);
        };
        auto read_v = [&](int blk, int i) {  // d block blk, keys [16i, 16i+16)
            vf[blk][i] = *reinterpret_cast<const bf16x8 *>(vst + voff(i) + 32 * blk * kBN);
        };
        __builtin_amdgcn_s_setprio(1);
        sn0 = f32x16{};
        sn1 = f32x16{};
        read_k(0);
        read_k(1);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            if (t < 6)
                read_k(t + 2);
            if (t >= 6) {
                read_v(0, 2 * (t - 6));
                read_v(0, 2 * (t - 6) + 1);
            }
            sn0 = mfma_bf16(kf0[t], qf[t], sn0);
            sc0[2 * t] = __builtin_amdgcn_exp2f(fmaf(sc0[2 * t], a.c, neg_m));
            sc0[2 * t + 1] = __builtin_amdgcn_exp2f(fmaf(sc0[2 * t + 1], a.c, neg_m));
            sn1 = mfma_bf16(kf1[t], qf[t], sn1);
            sc1[2 * t] = __builtin_amdgcn_exp2f(fmaf(sc1[2 * t], a.c, neg_m));
            sc1[2 * t + 1] = __builtin_amdgcn_exp2f(fmaf(sc1[2 * t + 1], a.c, neg_m));
            __builtin_amdgcn_sched_barrier(0);
        }
        const bf16x8 p00 = pack8(sc0, 0), p01 = pack8(sc0, 8);
        const bf16x8 p10 = pack8(sc1, 0), p11 = pack8(sc1, 8);
        // Row sum of the bf16 probabilities the P.V MFMAs consume, two per
        // v_dot2_f32_bf16.
        l = row_sum8(p10, row_sum8(p00, l));
        l2 = row_sum8(p11, row_sum8(p01, l2));

        // P.V of tile j, reading the V^T fragments of block blk+1 ahead;
        // meanwhile the VALU takes the max of tile j+1.
        float a0 = -INFINITY, a1 = -INFINITY;
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) {
            if (blk < 3) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    read_v(blk + 1, i);
            }
            f32x16 &ob = blk == 0 ? o0 : blk == 1 ? o1 : blk == 2 ? o2 : o3;
            ob = mfma_bf16(vf[blk][0], p00, ob);
            a0 = fmaxf(a0, fmaxf(sn0[4 * blk], sn0[4 * blk + 1]));
            ob = mfma_bf16(vf[blk][1], p01, ob);
            a0 = fmaxf(a0, fmaxf(sn0[4 * blk + 2], sn0[4 * blk + 3]));
            ob = mfma_bf16(vf[blk][2], p10, ob);
            a1 = fmaxf(a1, fmaxf(sn1[4 * blk], sn1[4 * blk + 1]));
            ob = mfma_bf16(vf[blk][3], p11, ob);
            a1 = fmaxf(a1, fmaxf(sn1[4 * blk + 2], sn1[4 * blk + 3]));
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_setprio(0);
        mx_next = row_pair_max(fmaxf(a0, a1));

        // The next iteration reads K(j+2) and V^T(j+1).  With three stages
        // they were started one iteration ago: wait until only this
        // iteration's copies are outstanding.  With two stages they are this
        // iteration's: wait for all.  Then let every wave see them.
        const int inflight = ST == 3 ? DMA * (int(dk) + int(dv)) : 0;
        if (inflight == 2 * DMA)
            wait_vmcnt<2 * DMA>();
        else if (inflight == DMA)
            wait_vmcnt<DMA>();
        else
            wait_vmcnt<0>();
        ring_barrier();
    };
    int j = 0;
    for (; j + 1 < ntiles; j += 2) {
        tile(j, sa0, sa1, sb0, sb1);
        tile(j + 1, sb0, sb1, sa0, sa1);
    }
    if (j < ntiles)
        tile(j, sa0, sa1, sb0, sb1);

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

// V (f32, [B,H,S,D] view, D = 128) -> packed bf16 V^T [B,H][D][Sp].  One block
// per (batch*head, 64-key tile): coalesced float4 reads of the V rows,
// transpose through LDS, 16-byte coalesced writes along the key axis.  Each
// thread converts a pair of adjacent keys (2p, 2p+1), which vt_key_pos keeps
// adjacent, and writes them as one 32-bit LDS word: lanes never share an LDS
// dword within one store.
struct PackArgs {
    const float *v;
    u16 *vt;
    int64_t vb, vh, vs, tb, th;
    int H, S_kv, n_tiles;
    int64_t sp;
};

constexpr int kTPitchW = (kBN + 8) / 2;  // 32-bit words per LDS row of the transposed tile

__global__ __launch_bounds__(256) void vt_pack_kernel(PackArgs a)
{
    __shared__ __attribute__((aligned(16))) unsigned int T[kD * kTPitchW];
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
            const bf16x2 pair = __builtin_convertvector(f32x2{x0[e], x1[e]}, bf16x2);
            T[(4 * c4 + e) * kTPitchW + w] = __builtin_bit_cast(unsigned int, pair);
        }
    }
    __syncthreads();
    u16 *tp = a.vt + b * a.tb + h * a.th + key0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int f = threadIdx.x + 256 * i;  // 16-byte chunk: d row, 8 keys
        const int d = f >> 3, c = f & 7;
        *reinterpret_cast<f32x4 *>(tp + d * a.sp + 8 * c) =
            *reinterpret_cast<const f32x4 *>(&T[d * kTPitchW + 4 * c]);
    }
}

template <int NW, int ST>
bool launch_d128(const Bf16Args &a, int64_t BH, hipStream_t st)
{
    constexpr int BM = NW * 32;
    Bf16Args g = a;
    g.n_qtiles = (g.S_q + BM - 1) / BM;
    const int64_t nblk = BH * g.n_qtiles * g.split.n;
    if (nblk > INT32_MAX)
        return fail("flash_bf16: problem too large for one launch");
    hipLaunchKernelGGL((flash_bf16_d128<NW, ST>), dim3(unsigned(nblk)), dim3(NW * 64), 0, st, g);
    return hip_ok(hipGetLastError(), "flash_bf16_d128 launch");
}

// Two 4-wave workgroups per CU with two-stage rings: large unsplit grids over
// at most kPairMaxTiles key tiles.
bool paired_plan(const FlashPlan &pl, int S_kv)
{
    return pl.waves == 8 && pl.splits == 1 && (S_kv + kBN - 1) / kBN <= kPairMaxTiles;
}

}  // namespace

bool flash_bf16_raw_q(int64_t BH, int S_q, int S_kv)
{
    return paired_plan(flash_plan(BH, S_q, S_kv, kD, kTileUsBF16), S_kv);
}

bool launch_flash_bf16(const FlashProblem &p, hipStream_t st, void *part, size_t part_bytes)
{
    const int64_t BH = int64_t(p.B) * p.H;
    if (BH == 0 || p.S_q == 0)
        return true;
    if (p.D != kD)
        return fail("flash_bf16: head dim must be 128 (got " + std::to_string(p.D) + ")");
    if (!(p.scale > 0.0f) || !std::isfinite(p.scale))
        return fail("flash_bf16: scale must be positive");
    const int64_t sp = vt_padded_len(p.S_kv);
    if (p.vs.s != sp)
        return fail("flash_bf16: V^T row stride must equal the padded key count");
    const auto s8 = [](const Strides &x) { return x.b % 8 == 0 && x.h % 8 == 0 && x.s % 8 == 0; };
    const bool raw_q = p.rq.x != nullptr;  // q's bf16 rows unused
    if ((!raw_q && (!aligned(p.q, 16) || !s8(p.qs))) || !aligned(p.k, 16) || !aligned(p.v, 16) ||
        !aligned(p.o, 16) || !s8(p.ks) || !s8(p.vs) || p.os.b % 4 || p.os.h % 4 || p.os.s % 4)
        return fail("flash_bf16: operands must be 16-byte aligned with 16-byte row strides");
    if (raw_q) {
        const Strides &x = p.rq.s;
        if (!aligned(p.rq.x, 16) || x.b % 4 || x.h % 4 || x.s % 4 ||
            (p.rq.w && !aligned(p.rq.w, 16)) || (p.rq.freqs && !aligned(p.rq.freqs, 16)))
            return fail("flash_bf16: raw query rows must be 16-byte aligned with 16-byte strides");
    }
    if (p.ot.t && !term_out_ok(p.ot))
        return fail("flash_bf16: term output must be 16-byte aligned with strides of 8 elements");
    Bf16Args a;
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
    // r*ks, V^T d-rows r < 128 at r*Sp, plus 256 bytes.
    a.dma32 = (int64_t(kBN) * p.ks.s * 2 + 256 < (int64_t(1) << 31)) &&
              (int64_t(kD) * sp * 2 + 256 < (int64_t(1) << 31));
    a.qx = p.rq.x;
    a.qw = p.rq.w;
    a.qf = p.rq.freqs;
    a.rqb = p.rq.s.b; a.rqh = p.rq.s.h; a.rqs = p.rq.s.s;
    a.eps = p.rq.eps;
    const FlashPlan pl = flash_plan(BH, p.S_q, p.S_kv, p.D, kTileUsBF16);
    a.split = flash_split_args(pl, BH, p.S_q, part, part_bytes);
    const bool ok = paired_plan(pl, p.S_kv) ? launch_d128<4, 2>(a, BH, st)
                    : pl.waves == 4        ? launch_d128<4, 3>(a, BH, st)
                                           : launch_d128<8, 3>(a, BH, st);
    if (!ok)
        return false;
    return a.split.n == 1 || launch_flash_combine(p, a.split, st);
}

bool launch_vt_pack(const float *v, Strides vs, uint16_t *vt, Strides vts, int B, int H,
                    int S_kv, int D, hipStream_t st)
{
    const int64_t BH = int64_t(B) * H;
    if (BH == 0 || S_kv == 0)
        return true;
    if (D != kD)
        return fail("vt_pack: head dim must be 128");
    if (!aligned(v, 16) || !aligned(vt, 16) || vs.b % 4 || vs.h % 4 || vs.s % 4 || vts.b % 8 ||
        vts.h % 8)
        return fail("vt_pack: operands must be 16-byte aligned");
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
        return fail("vt_pack: problem too large for one launch");
    hipLaunchKernelGGL(vt_pack_kernel, dim3(unsigned(nblk)), dim3(256), 0, st, a);
    return hip_ok(hipGetLastError(), "vt_pack_kernel launch");
}

}  // namespace anima_hip
