// Device helpers shared by the bf16-MFMA flash kernels (flash_bf16.hip,
// flash_x3.hip): the global -> LDS DMA copy, ring synchronisation, the
// 32x32x16 bf16 MFMA, and the per-row reductions of the transposed
// formulation, where lane l of a wave holds query row l % 32 in every
// accumulator register and the two lanes l, l^32 share a row.
#pragma once

#include "common.h"

namespace anima_hip {
namespace flash_tile {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16;

constexpr int kD = 128;               // head dim of these kernels
constexpr int kBN = 64;               // keys per tile (== kVtTile)
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kVmcnt0 = 0x0F70;       // s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15)
constexpr float kRescaleLog2 = 8.0f;  // lazy-rescale threshold: p <= 2^8
static_assert(kBN == kVtTile, "V^T padding must match the key tile");

// One 16-byte global -> LDS copy per lane (global_load_lds_dwordx4): lane i
// of the wave writes bytes [16i, 16i + 16) of the wave-uniform 1 KiB LDS
// window `lds` (through M0); no VGPRs hold the data.  Completion is counted
// by vmcnt and waited for explicitly (wait_vmcnt).  Issued from inline asm so
// that the compiler, which cannot tell ring stages apart, does not put a
// vmcnt(0) in front of every LDS read of another stage.
// M0 is declared clobbered; nothing else in these kernels keeps a value in
// M0 (checked in the generated assembly), so the reserved-register warning
// does not apply.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const u16 *src, u16 *lds)
{
    const unsigned m0 = static_cast<unsigned>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void *)lds));
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(m0), "v"(src)
                 : "memory", "m0");
}
// The same copy addressed as a wave-uniform 64-bit base (SGPRs) plus this
// lane's 32-bit byte offset, so no per-lane 64-bit address arithmetic runs.
__device__ __forceinline__ void dma16s(const void *base, unsigned voff, u16 *lds)
{
    const unsigned m0 = static_cast<unsigned>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void *)lds));
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(m0), "v"(voff), "s"(base)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt unconstrained).
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 16, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

// Workgroup barrier for the LDS rings: this wave's LDS reads are complete
// (lgkmcnt(0)), copies still in flight stay in flight (no vmcnt wait, unlike
// __syncthreads), and the compiler moves no memory access across it.
__device__ __forceinline__ void ring_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ f32x16 mfma_bf16(bf16x8 a, bf16x8 b, f32x16 c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Max of v over the two lanes l and l^32 (the two halves of a query row) with
// one v_permlane32_swap: r[0] holds the low half in both halves, r[1] the
// high half.
__device__ __forceinline__ float row_pair_max(float v)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Key (within a 32-key block) of accumulator register r of a lane in half h
// (lanes 32h .. 32h+31) of a 32x32 MFMA result.
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// Adds the 8 bf16 values of a P operand to the running sum acc, in f32
// (v_dot2_f32_bf16 with a vector of ones).
__device__ __forceinline__ float row_sum8(const bf16x8 &p, float acc)
{
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
    for (int i = 0; i < 8; i += 2)
        acc = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{p[i], p[i + 1]}, one, acc, false);
    return acc;
}

// Accumulator registers base .. base+7 as one bf16 MFMA operand (round to
// nearest even, v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16x8 pack8(const f32x16 &s, int base)
{
    bf16x8 r;
    const bf16x2 p0 = __builtin_convertvector(f32x2{s[base + 0], s[base + 1]}, bf16x2);
    const bf16x2 p1 = __builtin_convertvector(f32x2{s[base + 2], s[base + 3]}, bf16x2);
    const bf16x2 p2 = __builtin_convertvector(f32x2{s[base + 4], s[base + 5]}, bf16x2);
    const bf16x2 p3 = __builtin_convertvector(f32x2{s[base + 6], s[base + 7]}, bf16x2);
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

// hi = bf16(v) and lo = bf16(v - hi), both rounded to nearest even, as two
// bf16 pairs each: split_kernel's arithmetic (linear.hip), so a term output
// equals the split of the f32 output bit for bit.  v - hi is exact in f32.
__device__ __forceinline__ void split_terms4(const f32x4 &v, uint2 &hi, uint2 &lo)
{
    const bf16x2 h0 = __builtin_convertvector(f32x2{v.x, v.y}, bf16x2);
    const bf16x2 h1 = __builtin_convertvector(f32x2{v.z, v.w}, bf16x2);
    const bf16x2 l0 =
        __builtin_convertvector(f32x2{v.x - float(h0[0]), v.y - float(h0[1])}, bf16x2);
    const bf16x2 l1 =
        __builtin_convertvector(f32x2{v.z - float(h1[0]), v.w - float(h1[1])}, bf16x2);
    hi = uint2{__builtin_bit_cast(unsigned, h0), __builtin_bit_cast(unsigned, h1)};
    lo = uint2{__builtin_bit_cast(unsigned, l0), __builtin_bit_cast(unsigned, l1)};
}

// Four f32 values of an output row at d (a multiple of 4): as f32 at o + d,
// or, when t is set, as bf16 terms at t + d (and t + lo + d when lo > 0).
__device__ __forceinline__ void store_out4(const f32x4 &v, float *o, u16 *t, int64_t lo, int d)
{
    if (t) {
        uint2 h, l;
        split_terms4(v, h, l);
        *reinterpret_cast<uint2 *>(t + d) = h;
        if (lo > 0)
            *reinterpret_cast<uint2 *>(t + lo + d) = l;
    } else {
        *reinterpret_cast<f32x4 *>(o + d) = v;
    }
}

// Epilogue of the transposed bf16-MFMA kernels.  A wave holds O^T of its 32
// query rows in four 32x32 accumulators (o_blk: d = 32 blk + acc_row(r,
// half)), so a direct store writes 16 bytes of 32 rows 8 KiB apart per
// instruction and fills each 128-byte line over four instructions.  Staged
// through an LDS region of the wave instead, in two passes over d, every store
// instruction writes four whole 256-byte half rows.
// Rows r >= nrows are not written.  A dead row (its running max never left
// -inf: every score was masked or NaN) is written as zeros, which is what the
// reference's flash attention leaves there (flash_attention.h:148-152 skips
// such rows and :194-201 divides only positive sums of a zero-filled output).
// With trow0 set, the rows go out as bf16 terms (split_terms4) at trow0 +
// r * tstride instead of f32 at row0 + r * stride, in 16-byte stores.  The
// stores are nontemporal (streaming): this kernel never reads O back
// (4096 tokens, B=2, H=16: step 0.6779 -> 0.6745 ms f32x3, 4096 x 512
// cross-attention 109.9 -> 108.1 us f32x3 and 68.1 -> 67.2 us bf16).
// The caller guarantees no other wave uses `lds` (kOWaveFloats floats).
constexpr int kOPitch = 68;  // floats per staged half row: 64 d + 4 against bank conflicts
constexpr int kOWaveFloats = 32 * kOPitch;

__device__ __forceinline__ void store_o_rows(float *lds, const f32x16 &o0, const f32x16 &o1,
                                             const f32x16 &o2, const f32x16 &o3, float inv,
                                             bool dead, float *row0, int64_t stride, int nrows,
                                             u16 *trow0, int64_t tstride, int64_t tlo)
{
    const int lane = threadIdx.x & 63, col = lane & 31, half = lane >> 5;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
#pragma unroll
        for (int bb = 0; bb < 2; ++bb) {
            const f32x16 &ob = p == 0 ? (bb == 0 ? o0 : o1) : (bb == 0 ? o2 : o3);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                f32x4 v = f32x4{ob[4 * g] * inv, ob[4 * g + 1] * inv, ob[4 * g + 2] * inv,
                                ob[4 * g + 3] * inv};
                if (dead)
                    v = f32x4{0.f, 0.f, 0.f, 0.f};
                *reinterpret_cast<f32x4 *>(lds + col * kOPitch + 32 * bb + acc_row(4 * g, half)) =
                    v;
            }
        }
        // The rows were written by other lanes of this wave: wait for the LDS
        // writes, and keep the compiler from moving reads above them.
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        asm volatile("" ::: "memory");
        if (trow0) {
            // Terms: 8 values per lane, so each term goes out as one 16-byte
            // store and an instruction writes 8 whole 128-byte half rows.
            const int c = lane & 7;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 8 * i + (lane >> 3);
                const float *src = lds + r * kOPitch + 8 * c;
                uint2 h0, l0, h1, l1;
                split_terms4(*reinterpret_cast<const f32x4 *>(src), h0, l0);
                split_terms4(*reinterpret_cast<const f32x4 *>(src + 4), h1, l1);
                u16 *dst = trow0 + r * tstride + 64 * p + 8 * c;
                if (r < nrows) {
                    __builtin_nontemporal_store(u32x4{h0.x, h0.y, h1.x, h1.y},
                                                reinterpret_cast<u32x4 *>(dst));
                    if (tlo > 0)
                        __builtin_nontemporal_store(u32x4{l0.x, l0.y, l1.x, l1.y},
                                                    reinterpret_cast<u32x4 *>(dst + tlo));
                }
            }
        } else {
            const int c = lane & 15;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int r = 4 * i + (lane >> 4);
                const f32x4 v = *reinterpret_cast<const f32x4 *>(lds + r * kOPitch + 4 * c);
                if (r < nrows)
                    __builtin_nontemporal_store(
                        v, reinterpret_cast<f32x4 *>(row0 + r * stride + 64 * p + 4 * c));
            }
        }
        // This pass's reads complete before the next pass overwrites the rows.
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xC07F);
        asm volatile("" ::: "memory");
    }
}

// Logical id of this workgroup, XCD-major.  The dispatcher hands workgroup i
// to XCD i % 8, so consecutive ids land on different XCDs and every XCD ends
// up streaming every (batch, head)'s K/V from HBM.  Renumbered so that the
// workgroups of one XCD take one contiguous range of ids, the query tiles of
// a (batch, head), which read the same K/V tiles at about the same time, run
// on one XCD and share its L2.  A bijection on [0, gridDim.x) for every grid
// size (the first n % 8 XCDs take one id more), so only locality depends on
// the dispatch order, never the result.
constexpr unsigned kXcds = 8;
__device__ __forceinline__ int xcd_major_block()
{
    const unsigned n = gridDim.x, i = blockIdx.x, x = i % kXcds;
    const unsigned q = n / kXcds, r = n % kXcds;
    return int(x * q + (x < r ? x : r) + i / kXcds);
}

inline bool aligned(const void *ptr, unsigned m)
{
    return (reinterpret_cast<uintptr_t>(ptr) & (m - 1)) == 0;
}

}  // namespace flash_tile
}  // namespace anima_hip
