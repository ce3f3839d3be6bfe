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
}  // namespace

size_t prepared_k_bytes(int Bk, int S_kv, int H, int D, bool bf16)
{
    return size_t(Bk) * S_kv * H * D * (bf16 ? 2 : 4);
}

size_t prepared_v_bytes(int Bk, int S_kv, int H, int D, bool bf16)
{
    return bf16 ? size_t(Bk) * H * D * vt_padded_len(S_kv) * 2 : size_t(Bk) * S_kv * H * D * 4;
}

size_t attention_scratch_bytes(int B, int S_q, int Bk, int S_kv, int H, int D, bool bf16,
                               bool kv_prepared)
{
    size_t n = round_up(size_t(B) * S_q * H * D * (bf16 ? 2 : 4));
    if (!kv_prepared) {
        n += round_up(prepared_k_bytes(Bk, S_kv, H, D, bf16));
        if (bf16)
            n += round_up(prepared_v_bytes(Bk, S_kv, H, D, true));
    }
    return n + round_up(flash_plan(int64_t(B) * H, S_q, S_kv, D).bytes);
}

namespace {

// The K row problem of prepare_kv: RMSNorm (+ RoPE) of [Bk, S_kv, H, D] K.
RowProblem k_rows(const float *k, const float *k_norm_w, const float *freqs, void *k_out, int Bk,
                  int S_kv, int H, int D, float eps, bool bf16, int64_t ld = 0)
{
    RowProblem pk;
    pk.x = k;
    pk.out = k_out;
    pk.w = k_norm_w;
    pk.freqs = freqs;
    pk.xs = bshd(S_kv, H, D, false, ld);
    pk.os = bshd(S_kv, H, D, false);
    pk.B = Bk;
    pk.S = S_kv;
    pk.H = H;
    pk.D = D;
    pk.eps = eps;
    pk.norm = true;
    pk.out_bf16 = bf16;
    return pk;
}

// V's part of prepare_kv: packed bf16 V^T, or a copy (f32) unless in place.
bool prepare_v(const float *v, void *v_out, int Bk, int S_kv, int H, int D, bool bf16,
               hipStream_t st, int64_t ld = 0)
{
    if (bf16) {
        const int64_t sp = vt_padded_len(S_kv);
        const Strides vts{int64_t(H) * D * sp, int64_t(D) * sp, sp};
        return launch_vt_pack(v, bshd(S_kv, H, D, false, ld), static_cast<uint16_t *>(v_out), vts, Bk,
                              H, S_kv, D, st);
    }
    if (v_out && v_out != v) {
        if (ld > 0 && ld != int64_t(H) * D)
            return fail("prepare_kv: a strided V cannot be copied into a dense cache");
        return hip_ok(hipMemcpyAsync(v_out, v, prepared_v_bytes(Bk, S_kv, H, D, false),
                                     hipMemcpyDeviceToDevice, st),
                      "V copy");
    }
    return true;
}

}  // namespace

bool prepare_kv(const float *k, const float *v, const float *k_norm_w, const float *freqs,
                void *k_out, void *v_out, int Bk, int S_kv, int H, int D, float eps, bool bf16,
                hipStream_t st)
{
    return launch_rows(k_rows(k, k_norm_w, freqs, k_out, Bk, S_kv, H, D, eps, bf16), st) &&
           prepare_v(v, v_out, Bk, S_kv, H, D, bf16, st);
}

bool run_attention(const AttnInputs &in, void *scratch, hipStream_t st)
{
    const int B = in.B, S_q = in.S_q, S_kv = in.S_kv, H = in.H, D = in.D;
    if (int64_t(B) * S_q * H * D == 0)
        return true;
    if (in.Bk != B && in.Bk != 1)
        return fail("attention: K/V batch must be 1 (broadcast) or equal to the query batch");
    if (in.bf16 && D != 128)
        return fail("attention: the bf16 mode needs D == 128");
    if (in.freqs && S_q != S_kv)
        return fail("attention: RoPE needs S_q == S_kv (self-attention)");
    const bool prepared = in.k_prep != nullptr;
    char *cur = static_cast<char *>(scratch);
    void *qn = cur;
    cur += round_up(size_t(B) * S_q * H * D * (in.bf16 ? 2 : 4));

    const void *kp = in.k_prep, *vp = in.v_prep;
    RowProblem pk{};
    if (!prepared) {
        void *kn = cur;
        cur += round_up(prepared_k_bytes(in.Bk, S_kv, H, D, in.bf16));
        void *vt = in.bf16 ? static_cast<void *>(cur) : nullptr;
        pk = k_rows(in.k, in.k_norm_w, in.freqs, kn, in.Bk, S_kv, H, D, in.eps, in.bf16,
                    in.ld_kv);
        if (!prepare_v(in.v, vt, in.Bk, S_kv, H, D, in.bf16, st, in.ld_kv))
            return false;
        kp = kn;
        vp = in.bf16 ? vt : static_cast<const void *>(in.v);
        if (in.bf16)
            cur += round_up(prepared_v_bytes(in.Bk, S_kv, H, D, true));
    }
    // Split-KV partials (small problems only).
    void *part = cur;
    const size_t part_bytes = flash_plan(int64_t(B) * H, S_q, S_kv, D).bytes;

    RowProblem pq;
    pq.x = in.q;
    pq.out = qn;
    pq.w = in.q_norm_w;
    pq.freqs = in.freqs;
    pq.xs = bshd(S_q, H, D, false, in.ld_q);
    pq.os = bshd(S_q, H, D, false);
    pq.B = B;
    pq.S = S_q;
    pq.H = H;
    pq.D = D;
    pq.eps = in.eps;
    pq.norm = true;
    pq.out_bf16 = in.bf16;
    // Q rows, and K rows unless prepared, in one launch.
    if (!(prepared ? launch_rows(pq, st) : launch_rows_pair(pk, pq, st)))
        return false;

    const bool bcast = in.Bk == 1 && B > 1;
    FlashProblem p;
    p.q = qn;
    p.k = kp;
    p.v = vp;
    p.o = in.out;
    p.qs = p.os = bshd(S_q, H, D, false);
    p.ks = bshd(S_kv, H, D, bcast);
    if (in.bf16) {
        const int64_t sp = vt_padded_len(S_kv);
        p.vs = Strides{bcast ? 0 : int64_t(H) * D * sp, int64_t(D) * sp, sp};
    } else {
        p.vs = prepared ? bshd(S_kv, H, D, bcast) : bshd(S_kv, H, D, bcast, in.ld_kv);
    }
    p.B = B;
    p.H = H;
    p.S_q = S_q;
    p.S_kv = S_kv;
    p.D = D;
    p.scale = float(1.0 / std::sqrt(double(D)));
    p.causal = false;
    return in.bf16 ? launch_flash_bf16(p, st, part, part_bytes)
                   : launch_flash_f32(p, st, part, part_bytes);
}

}  // namespace anima_hip
