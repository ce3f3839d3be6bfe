"""Write tests/golden/dit_ref_vectors.npz with the reference's own DiT code.

What only the reference's Python pins: the composition of NumpyDiT.forward
(patch order, padding-mask channel, timestep features, AdaLN chunk order and
LoRA term, block order, final layer, unpatchify and crop) and of
EulerSampler.sample with ZImageScheduler.  This script runs that code
(anima_rt/scripts/numpy_dit.py and sampling.py, imported from the reference
tree in this container only) on a small-width model and stores inputs and
outputs; the weights are regenerated from the seed by dit_weights.py.

The reference classes take their runtime (rt) and GEMM engine (vk) as
constructor arguments (numpy_dit.py:67-80).  Here rt is the reference runtime
compiled from its own sources (oracle/_ref), called through the same methods
as NumpyRT (scripts/phone_pipeline_nd.py:46-68); vk is that runtime's bf16
GEMM (fp32 activations x bf16 weights, fp32 accumulation), standing in for
the phone's Vulkan GEMM of the same arithmetic.  NumpyDiT.forward itself
(numpy_dit.py:82-130) runs unchanged: its first statements reset the Vulkan
descriptor pool through the phone-only module vk_ops (numpy_dit.py:87-88),
which this script provides as a stub whose reset does nothing.
NumpyDiT.__init__ fixes the full model's sizes (numpy_dit.py:68-79), so the
small model's instance is assembled from the reference's own sub-module
classes with the same attribute names and then driven through that method.

Model: width 2048 (NumpyPatchEmbed fixes it), 2 blocks, 2 heads x 128, MLP
512, text context 64 wide, 16 latent channels; latent 7 x 10 (odd height:
exercises padding and crop).

Run:  python tests/golden/make_dit_golden.py   (needs oracle/_ref built)
"""
import os
import sys
import types

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF_SCRIPTS = "/root/reference/anima_rt/scripts"
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, HERE)

import oracle  # noqa: E402
import dit_weights  # noqa: E402

OUT = os.path.join(HERE, "dit_ref_vectors.npz")
CFG = dict(dim=2048, blocks=2, heads=2, head_dim=128, mlp_hidden=512, ctx_dim=64)
WEIGHT_SEED = 7101


class RefRT:
    """The reference runtime behind NumpyRT's methods."""

    def __init__(self, norm_weights):
        self._nw = norm_weights

    def run_layernorm(self, x, D):
        return oracle.ref_layernorm(np.ascontiguousarray(x, np.float32).reshape(-1, D), 1e-6)

    def run_rmsnorm(self, x, key):
        *b, D = x.shape
        out = oracle.ref_rmsnorm(np.ascontiguousarray(x, np.float32).reshape(-1, D),
                                 self._nw[key + ".weight"], 1e-6)
        return out.reshape(*b, D)

    def run_gelu(self, x):
        return oracle.ref_gelu(x)

    def run_silu(self, x):
        return oracle.ref_silu(x)

    def run_sdpa(self, q, k, v):
        B, H, Sq, D = q.shape
        Skv = k.shape[2]
        o = oracle.ref_flash_sdpa(np.ascontiguousarray(q, np.float32).reshape(B * H, Sq, D),
                                  np.ascontiguousarray(k, np.float32).reshape(B * H, Skv, D),
                                  np.ascontiguousarray(v, np.float32).reshape(B * H, Skv, D),
                                  1.0 / np.sqrt(D), False)
        return o.reshape(B, H, Sq, D)


class RefVK:
    """vk_run_gemm(name, x, out, M, N, K): out = x . W[name]^T."""

    def __init__(self, linear_weights):
        self._w = linear_weights

    def vk_run_gemm(self, name, x, out, M, N, K):
        w = self._w[name]
        assert w.shape == (N, K), (name, w.shape, (N, K))
        out[...] = oracle.ref_gemm_bf16(np.ascontiguousarray(x, np.float32).reshape(M, K), w)


def main():
    if not oracle.ref_available():
        raise SystemExit("oracle/_ref/libanima_rt_ref.so missing: run `make -C oracle ref`")
    sys.path.insert(0, REF_SCRIPTS)
    import numpy_dit as nd
    import sampling

    w = dit_weights.make(WEIGHT_SEED, **CFG)
    rt = RefRT({k: v for k, v in w.items() if v.ndim == 1})
    vk = RefVK({k: v for k, v in w.items() if v.ndim == 2})
    D, heads, hd = CFG["dim"], CFG["heads"], CFG["head_dim"]
    blocks = [nd.NumpyBlock(i, D, CFG["ctx_dim"], heads, hd, CFG["mlp_hidden"], vk, rt)
              for i in range(CFG["blocks"])]
    x_embedder = nd.NumpyPatchEmbed(vk)
    t_embedder = nd.NumpyTimestepEmbedding(D, vk, rt)
    final_layer = nd.NumpyFinalLayer(D, vk, rt)

    # The phone's Vulkan module, reached only for its pool reset.
    vk_ops = types.ModuleType("vk_ops")
    vk_ops._lib = types.SimpleNamespace(vk_reset_pool=lambda: None)
    sys.modules["vk_ops"] = vk_ops
    model = object.__new__(nd.NumpyDiT)
    model._vk, model._rt = vk, rt
    model.D, model.num_blocks, model.num_heads = D, CFG["blocks"], heads
    model.head_dim, model.mlp_hidden = hd, CFG["mlp_hidden"]
    model.ps, model.pt, model.out_ch = 2, 1, 16
    model.x_embedder, model.t_embedder, model.final_layer = x_embedder, t_embedder, final_layer
    model.blocks = blocks
    reference_forward = model.forward

    rng = np.random.default_rng(7102)
    vec = {"weight_seed": np.array(WEIGHT_SEED)}
    for k, v in CFG.items():
        vec["cfg_" + k] = np.array(v)
    x = rng.standard_normal((2, 16, 1, 7, 10), dtype=np.float32)
    sigma = np.array([0.9, 0.35], np.float32)
    ctx = rng.standard_normal((2, 8, CFG["ctx_dim"]), dtype=np.float32) * np.float32(0.5)
    vec["fwd_x"], vec["fwd_sigma"], vec["fwd_ctx"] = x, sigma, ctx
    vec["fwd_out"] = reference_forward(x, sigma, ctx)
    print("forward done", flush=True)

    noise = rng.standard_normal((1, 16, 7, 10), dtype=np.float32)
    ctx_c = rng.standard_normal((1, 8, CFG["ctx_dim"]), dtype=np.float32) * np.float32(0.5)
    ctx_u = rng.standard_normal((1, 8, CFG["ctx_dim"]), dtype=np.float32) * np.float32(0.5)
    sigmas = sampling.ZImageScheduler().get_sigmas(2, 1.0)
    vec["smp_noise"], vec["smp_ctx_cond"], vec["smp_ctx_uncond"] = noise, ctx_c, ctx_u
    vec["smp_sigmas"], vec["smp_cfg"] = sigmas, np.array(5.0, np.float32)
    vec["smp_out"] = sampling.EulerSampler().sample(model, noise, sigmas, ctx_c, ctx_u, 5.0,
                                                    0).astype(np.float32)
    print("sampler done", flush=True)
    np.savez_compressed(OUT, **vec)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(vec)} arrays)")


if __name__ == "__main__":
    main()
