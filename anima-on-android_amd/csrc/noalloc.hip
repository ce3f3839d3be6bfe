// Allocation-free form of anima_hip_attention_dev: the same attention core
// (RMSNorm + RoPE prologue, flash attention, split-KV partials) on device
// memory, with its scratch in a static device array instead of a caller
// workspace, for callers that cannot allocate (code under HIP graph capture,
// serving loops that forbid hipMalloc).
//
// The array `scratch` below exists once per GPU, at an address of that GPU.
// In host code its name is only a stand-in for the symbol, so the device
// address is looked up with hipGetSymbolAddress once per device, on the first
// call made while that device is current, and only that address is handed to
// the kernels.  Every call on a GPU shares the array: calls that overlap on
// one GPU (other streams, other threads) race and must be serialised by the
// caller.  The kernels write every scratch byte they later read (the Q/K
// rows, the padded V^T including its zero tail, and each split's partial
// rows), so nothing needs clearing between calls.
#include "common.h"

#include "anima_hip.h"

#include <mutex>
#include <string>

static __device__ __align__(256) unsigned char scratch[ANIMA_HIP_STATIC_SCRATCH_BYTES];

namespace {

constexpr size_t kStaticScratchBytes = size_t(ANIMA_HIP_STATIC_SCRATCH_BYTES);
constexpr int kMaxDevices = 64;

std::mutex g_mu;
void *g_scratch[kMaxDevices] = {};

// Device address of this GPU's `scratch`, looked up once per device.
bool static_scratch(void **out)
{
    using anima_hip::fail;
    using anima_hip::hip_ok;
    int dev = -1;
    if (!hip_ok(hipGetDevice(&dev), "attention_static_dev: hipGetDevice"))
        return false;
    if (dev < 0 || dev >= kMaxDevices)
        return fail("attention_static_dev: device ordinal " + std::to_string(dev) +
                    " beyond the supported " + std::to_string(kMaxDevices));
    std::lock_guard<std::mutex> g(g_mu);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        if (!hip_ok(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                    "attention_static_dev: hipGetSymbolAddress(scratch)"))
            return false;
        if (!p)
            return fail("attention_static_dev: hipGetSymbolAddress returned no address");
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return true;
}

}  // namespace

extern "C" {

bool anima_hip_attention_static_dev(const float *q, const float *k, const float *v,
                                    const float *q_norm_w, const float *k_norm_w,
                                    const float *freqs, float *out, int B, int S_q, int Bk,
                                    int S_kv, int H, int D, float eps, int mode, void *stream)
{
    using namespace anima_hip;
    if (B < 0 || H < 0 || S_q < 0 || S_kv < 0 || D < 0 || Bk < 0)
        return fail("attention_static_dev: negative dimension");
    if (mode != ANIMA_HIP_F32 && mode != ANIMA_HIP_BF16 && mode != ANIMA_HIP_F32X3)
        return fail("attention_static_dev: unknown mode " + std::to_string(mode));
    if (mode != ANIMA_HIP_F32 && D != 128)
        return fail("attention_static_dev: the bf16 and f32x3 modes need D == 128");
    if (int64_t(B) * S_q * H * D == 0)
        return true;
    if (!q || !out || (S_kv > 0 && (!k || !v)))
        return fail("attention_static_dev: null pointer");
    const AttnMode am = AttnMode(mode);
    const size_t need = attention_scratch_bytes(B, S_q, Bk, S_kv, H, D, am, false);
    if (need > kStaticScratchBytes)
        return fail("attention_static_dev: the problem needs " + std::to_string(need) +
                    " bytes of scratch, more than the static " +
                    std::to_string(kStaticScratchBytes) +
                    "; use anima_hip_attention_dev with caller scratch");
    void *ws = nullptr;
    if (!static_scratch(&ws))
        return false;
    AttnInputs in;
    in.q = q;
    in.q_norm_w = q_norm_w;
    in.freqs = freqs;
    in.k = k;
    in.v = v;
    in.k_norm_w = k_norm_w;
    in.out = out;
    in.B = B;
    in.Bk = Bk;
    in.S_q = S_q;
    in.S_kv = S_kv;
    in.H = H;
    in.D = D;
    in.eps = eps;
    in.mode = am;
    return run_attention(in, ws, static_cast<hipStream_t>(stream));
}

}  // extern "C"
