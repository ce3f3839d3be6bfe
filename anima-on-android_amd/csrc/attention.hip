// Device-side composition of the attention core of NumpyAttention.forward
// (anima_rt/scripts/numpy_dit.py:283-294) on [B, S, H, D] projections:
//   q' = RoPE?(RMSNorm_head(q)), k' = RoPE?(RMSNorm_head(k)), O = SDPA(q', k', v)
// with the output written straight into [B, S_q, H, D] (the [B*S, H*D] input
// of output_proj), so none of the reference's transposes/copies
// (numpy_dit.py:291-294, phone_pipeline_nd.py:63-65) exist here.
//
// K/V are either raw projections (prepared per call) or already prepared by
// prepare_kv (the cross-attention context cache).  A K/V batch of 1 is
// broadcast to every query batch (stride 0), which is how one text context
// serves both CFG branches.
#include "common.h"

#include <cmath>

namespace anima_hip {

namespace {
constexpr size_t kAlign = 256;
size_t round_up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

// [B, S, H, D] view whose token rows are ld elements apart (ld = H*D when
// dense; wider when q/k/v are column blocks of one [B*S, 3*H*D] projection).
Strides bshd(int S, int H, int D, bool broadcast, int64_t ld = 0)
{
    const int64_t row = ld > 0 ? ld : int64_t(H) * D;
    return Strides{broadcast ? 0 : int64_t(S) * row, int64_t(D), row};
}

// Q/K rows of the attention kernels of `mode` in [B, S, H, D] order: f32 or
// bf16 rows of D, or [hi | lo] term rows of 2D (f32x3).
Strides bshd_mode(int S, int H, int D, bool broadcast, AttnMode mode)
{
    return mode == kAttnF32X3 ? bshd(S, H, 2 * D, broadcast) : bshd(S, H, D, broadcast);
}

// Packed V^T strides {batch, head, d-row} of the bf16 / f32x3 layouts.
Strides vt_strides(int S_kv, int H, int D, bool broadcast, AttnMode mode)
{
    const int64_t sp = vt_padded_len(S_kv), rows = mode == kAttnF32X3 ? 2 * int64_t(D) : D;
    return Strides{broadcast ? 0 : int64_t(H) * rows * sp, rows * sp, sp};
}

// Bytes per Q/K element in the layout of `mode`: f32, one bf16, or two bf16 terms.
size_t qk_elem_bytes(AttnMode mode) { return mode == kAttnBF16 ? 2 : 4; }
}  // namespace

size_t prepared_k_bytes(int Bk, int S_kv, int H, int D, AttnMode mode)
{
    return size_t(Bk) * S_kv * H * D * qk_elem_bytes(mode);
}

size_t prepared_v_bytes(int Bk, int S_kv, int H, int D, AttnMode mode)
{
    if (mode == kAttnF32)
        return size_t(Bk) * S_kv * H * D * 4;
    return size_t(Bk) * H * D * vt_padded_len(S_kv) * (mode == kAttnF32X3 ? 4 : 2);
}

size_t attention_scratch_bytes(int B, int S_q, int Bk, int S_kv, int H, int D, AttnMode mode,
                               bool kv_prepared)
{
    size_t n = round_up(size_t(B) * S_q * H * D * qk_elem_bytes(mode));
    if (!kv_prepared) {
        n += round_up(prepared_k_bytes(Bk, S_kv, H, D, mode));
        if (mode != kAttnF32)
            n += round_up(prepared_v_bytes(Bk, S_kv, H, D, mode));
    }
    return n + round_up(flash_plan(int64_t(B) * H, S_q, S_kv, D).bytes);
}

namespace {

// The Q or K row problem: RMSNorm (+ RoPE) of [B, S, H, D] rows ld apart,
// written in the Q/K layout of `mode`.
RowProblem qk_rows(const float *x, const float *norm_w, const float *freqs, void *out, int B,
                   int S, int H, int D, float eps, AttnMode mode, int64_t ld = 0)
{
    RowProblem p;
    p.x = x;
    p.out = out;
    p.w = norm_w;
    p.freqs = freqs;
    p.xs = bshd(S, H, D, false, ld);
    p.os = bshd_mode(S, H, D, false, mode);
    p.B = B;
    p.S = S;
    p.H = H;
    p.D = D;
    p.eps = eps;
    p.norm = true;
    p.out_bf16 = mode != kAttnF32;
    p.lo_off = mode == kAttnF32X3 ? D : 0;
    return p;
}

// V's part of prepare_kv: packed (term) V^T, or a copy (f32) unless in place.
bool prepare_v(const float *v, void *v_out, int Bk, int S_kv, int H, int D, AttnMode mode,
               hipStream_t st, int64_t ld = 0)
{
    if (mode != kAttnF32) {
        const Strides vs = bshd(S_kv, H, D, false, ld);
        const Strides vts = vt_strides(S_kv, H, D, false, mode);
        uint16_t *vt = static_cast<uint16_t *>(v_out);
        return mode == kAttnF32X3 ? launch_vt_pack_terms(v, vs, vt, vts, Bk, H, S_kv, D, st)
                                  : launch_vt_pack(v, vs, vt, vts, Bk, H, S_kv, D, st);
    }
    if (v_out && v_out != v) {
        if (ld > 0 && ld != int64_t(H) * D)
            return fail("prepare_kv: a strided V cannot be copied into a dense cache");
        return hip_ok(hipMemcpyAsync(v_out, v, prepared_v_bytes(Bk, S_kv, H, D, kAttnF32),
                                     hipMemcpyDeviceToDevice, st),
                      "V copy");
    }
    return true;
}

}  // namespace

bool prepare_kv(const float *k, const float *v, const float *k_norm_w, const float *freqs,
                void *k_out, void *v_out, int Bk, int S_kv, int H, int D, float eps,
                AttnMode mode, hipStream_t st)
{
    if (mode != kAttnF32 && D != 128)
        return fail("prepare_kv: the bf16 and f32x3 modes need D == 128");
    return launch_rows(qk_rows(k, k_norm_w, freqs, k_out, Bk, S_kv, H, D, eps, mode), st) &&
           prepare_v(v, v_out, Bk, S_kv, H, D, mode, st);
}

bool run_attention(const AttnInputs &in, void *scratch, hipStream_t st)
{
    const int B = in.B, S_q = in.S_q, S_kv = in.S_kv, H = in.H, D = in.D;
    const AttnMode mode = in.mode;
    if (int64_t(B) * S_q * H * D == 0)
        return true;
    if (in.Bk != B && in.Bk != 1)
        return fail("attention: K/V batch must be 1 (broadcast) or equal to the query batch");
    if (mode != kAttnF32 && D != 128)
        return fail("attention: the bf16 and f32x3 modes need D == 128");
    if (in.freqs && S_q != S_kv)
        return fail("attention: RoPE needs S_q == S_kv (self-attention)");
    const bool prepared = in.k_prep != nullptr;
    const bool q_ready = in.q_prep != nullptr;
    if (q_ready && (!prepared || !in.v_prep))
        return fail("attention: prepared Q rows need prepared K and V");
    char *cur = static_cast<char *>(scratch);
    void *qn = q_ready ? const_cast<void *>(in.q_prep) : static_cast<void *>(cur);
    cur += round_up(size_t(B) * S_q * H * D * qk_elem_bytes(mode));

    const void *kp = in.k_prep, *vp = in.v_prep;
    RowProblem pk{};
    const int64_t ld_q = in.ld_q > 0 ? in.ld_q : int64_t(H) * D;
    const int64_t ld_kv = in.ld_kv > 0 ? in.ld_kv : int64_t(H) * D;
    // Self-attention with q, k, v of one shape and row stride (the usual
    // case, and the fused projection's column blocks): one launch prepares
    // all three operands.
    PrepProblem pp;
    bool fused = !prepared && in.Bk == B && S_q == S_kv && ld_q == ld_kv;
    if (fused) {
        void *kn = cur;
        void *vt = mode != kAttnF32 ? cur + round_up(prepared_k_bytes(B, S_kv, H, D, mode))
                                    : nullptr;
        pp.q = in.q;
        pp.k = in.k;
        pp.v = in.v;
        pp.w[0] = in.q_norm_w;
        pp.w[1] = in.k_norm_w;
        pp.freqs = in.freqs;
        pp.qo = qn;
        pp.ko = kn;
        pp.vt = static_cast<uint16_t *>(vt);
        pp.ld = ld_q;
        pp.B = B;
        pp.S = S_q;
        pp.H = H;
        pp.D = D;
        pp.eps = in.eps;
        pp.mode = mode;
        fused = prep_qkv_supported(pp);
    }
    if (fused) {
        cur += round_up(prepared_k_bytes(B, S_kv, H, D, mode));
        if (mode != kAttnF32)
            cur += round_up(prepared_v_bytes(B, S_kv, H, D, mode));
        if (!launch_prep_qkv(pp, st))
            return false;
        kp = pp.ko;
        vp = mode != kAttnF32 ? static_cast<const void *>(pp.vt) : static_cast<const void *>(in.v);
    } else if (!prepared) {
        void *kn = cur;
        cur += round_up(prepared_k_bytes(in.Bk, S_kv, H, D, mode));
        void *vt = mode != kAttnF32 ? static_cast<void *>(cur) : nullptr;
        pk = qk_rows(in.k, in.k_norm_w, in.freqs, kn, in.Bk, S_kv, H, D, in.eps, mode, in.ld_kv);
        if (!prepare_v(in.v, vt, in.Bk, S_kv, H, D, mode, st, in.ld_kv))
            return false;
        kp = kn;
        vp = mode != kAttnF32 ? vt : static_cast<const void *>(in.v);
        if (mode != kAttnF32)
            cur += round_up(prepared_v_bytes(in.Bk, S_kv, H, D, mode));
    }
    // Split-KV partials (small problems only).
    void *part = cur;
    const size_t part_bytes = flash_plan(int64_t(B) * H, S_q, S_kv, D).bytes;

    // Cross-attention (K/V prepared, no RoPE) in f32x3 on a grid of at least
    // one 8-wave workgroup per CU: the flash kernel prepares its own query
    // rows from the raw projection (RawQ), one pass over HBM fewer.  The
    // kernel reads the same bytes for a raw f32 row as for a [hi | lo] term
    // row (4096 x 512, B = 2: 119.9 -> 108.9 us).  Smaller grids keep the row
    // pass (256 x 512: 28.0 against 28.9 us on the raw path, whose copies go
    // out ahead of Q), and split grids would repeat it per split.
    // Self-attention keeps it too, where the RoPE table's reads at each
    // workgroup's start cost more than the pass.
    // The f32 kernel, which reads Q as f32 rows anyway, does the same (RMSNorm
    // only: its rows carry no terms; 4096 x 512: 307.5 -> 286.5 us).  The
    // bf16 kernel does it where it runs two 4-wave workgroups per CU (short
    // key ranges, flash_bf16_raw_q): there the doubled Q read at a
    // workgroup's start overlaps the other workgroup's tiles.  With one
    // 8-wave workgroup per CU it measured the same as the row pass (4096 x
    // 512, B = 2: 65.7 against 65.9 us, bit-identical).
    const auto a16 = [](const void *x) { return (reinterpret_cast<uintptr_t>(x) & 15u) == 0; };
    const FlashPlan raw_plan = flash_plan(int64_t(B) * H, S_q, S_kv, D,
                                          mode == kAttnF32X3 ? kTileUsX3 : kTileUsF32);
    const bool raw_kernel =
        mode == kAttnBF16 ? flash_bf16_raw_q(int64_t(B) * H, S_q, S_kv)
                          : raw_plan.waves == 8 && raw_plan.splits == 1;
    const bool raw_q = !q_ready && prepared && !in.freqs && D == 128 && a16(in.q) &&
                       ld_q % 4 == 0 && (!in.q_norm_w || a16(in.q_norm_w)) && raw_kernel;

    // Q rows, and K rows unless prepared, in one launch.
    const RowProblem pq =
        qk_rows(in.q, in.q_norm_w, in.freqs, qn, B, S_q, H, D, in.eps, mode, in.ld_q);
    if (!fused && !raw_q && !q_ready &&
        !(prepared ? launch_rows(pq, st) : launch_rows_pair(pk, pq, st)))
        return false;

    const bool bcast = in.Bk == 1 && B > 1;
    FlashProblem p;
    p.q = qn;
    p.k = kp;
    p.v = vp;
    p.o = in.out;
    p.qs = bshd_mode(S_q, H, D, false, mode);
    p.os = bshd(S_q, H, D, false);
    p.ks = bshd_mode(S_kv, H, D, bcast, mode);
    if (mode != kAttnF32)
        p.vs = vt_strides(S_kv, H, D, bcast, mode);
    else
        p.vs = prepared ? bshd(S_kv, H, D, bcast) : bshd(S_kv, H, D, bcast, in.ld_kv);
    p.B = B;
    p.H = H;
    p.S_q = S_q;
    p.S_kv = S_kv;
    p.D = D;
    p.scale = float(1.0 / std::sqrt(double(D)));
    p.causal = false;
    if (raw_q) {
        p.q = nullptr;
        p.rq.x = in.q;
        p.rq.s = bshd(S_q, H, D, false, in.ld_q);
        p.rq.w = in.q_norm_w;
        p.rq.eps = in.eps;
    }
    if (in.out_t) {
        p.o = nullptr;
        p.os = Strides{0, 0, 0};
        p.ot.t = in.out_t;
        p.ot.tb = int64_t(S_q) * in.ld_t;
        p.ot.th = D;
        p.ot.ts = in.ld_t;
        p.ot.lo = in.lo_t;
    }
    switch (mode) {
    case kAttnBF16:
        return launch_flash_bf16(p, st, part, part_bytes);
    case kAttnF32X3:
        return launch_flash_x3(p, st, part, part_bytes);
    default:
        return launch_flash_f32(p, st, part, part_bytes);
    }
}

}  // namespace anima_hip
