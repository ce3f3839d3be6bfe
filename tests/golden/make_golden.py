"""Write tests/golden/anima_rt_ref_vectors.npz from the reference runtime.

The expected outputs come from anima_rt compiled from its own sources
(oracle/_ref/libanima_rt_ref.so, built by `make -C oracle ref` where the
reference tree exists), called through its C-ABI exactly as its ctypes
callers do (anima_rt/scripts/anima_rt_ops.py:28-31).  Inputs are seeded
numpy draws; both inputs and outputs are stored, so the fixture stands on its
own where the reference is absent.

Cases
  flash_*  anima_rt_run_sdpa_flash: short tiles, a causal case, and one that
           crosses the reference's qSplit=64 / kvSplit=512 tile boundaries
  math_*   anima_rt_run_sdpa (effective logit scale = scale^2)
  rms_*    anima_rt_run_rmsnorm: the shapes of
           anima_rt/scripts/tests/verify_kernels.py:92-115 (4x128 weighted,
           64x2048 weighted, 4x128 without weight at eps 1e-5)
  rope_*   anima_rt_run_rope on a 4x4 token grid, and the D=4 known-answer
           input of scripts/test_rope_debug.py:17-34
  gemm_*   anima_rt_run_gemm_bf16 (fp32 activations x bf16 weights)
  ln_*, silu_*, gelu_*, softmax_*  anima_rt_run_layernorm / _silu / _gelu / _softmax

Run:  python tests/golden/make_golden.py
"""
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "anima-on-android_amd"))

import oracle  # noqa: E402
from anima_hip.rope import generate_rope_freqs  # noqa: E402

OUT = os.path.join(HERE, "anima_rt_ref_vectors.npz")


def normal(rng, *shape, sigma=1.0):
    return (rng.standard_normal(shape) * sigma).astype(np.float32)


def main():
    if not oracle.ref_available():
        raise SystemExit("oracle/_ref/libanima_rt_ref.so missing: run `make -C oracle ref`")
    rng = np.random.default_rng(20240601)
    vec = {}

    flash_cases = {
        "flash_small": (3, 37, 70, 128, False),
        "flash_causal": (2, 50, 50, 64, True),
        "flash_tiles": (1, 200, 600, 128, False),
        "flash_d80": (2, 29, 41, 80, False),
    }
    for name, (bh, sq, sk, d, causal) in flash_cases.items():
        q, k, v = normal(rng, bh, sq, d), normal(rng, bh, sk, d), normal(rng, bh, sk, d)
        vec[f"{name}_q"], vec[f"{name}_k"], vec[f"{name}_v"] = q, k, v
        vec[f"{name}_causal"] = np.array(causal)
        vec[f"{name}_out"] = oracle.ref_flash_sdpa(q, k, v, 1.0 / math.sqrt(d), causal)

    q, k, v = normal(rng, 2, 33, 128), normal(rng, 2, 47, 128), normal(rng, 2, 47, 128)
    vec["math_q"], vec["math_k"], vec["math_v"] = q, k, v
    vec["math_out"] = oracle.ref_math_sdpa(q, k, v, 1.0 / math.sqrt(128), False)

    x4 = normal(rng, 4, 128)
    w4 = normal(rng, 128)
    x64 = normal(rng, 64, 2048)
    w64 = normal(rng, 2048)
    vec["rms_x4"], vec["rms_w4"] = x4, w4
    vec["rms_out4"] = oracle.ref_rmsnorm(x4, w4, 1e-6)
    vec["rms_x64"], vec["rms_w64"] = x64, w64
    vec["rms_out64"] = oracle.ref_rmsnorm(x64, w64, 1e-6)
    vec["rms_out4_nw"] = oracle.ref_rmsnorm(x4, None, 1e-5)

    t = normal(rng, 2, 16, 128)
    fr = generate_rope_freqs(4, 4, 1, 128)
    vec["rope_t"], vec["rope_freqs"] = t, fr
    vec["rope_out"] = oracle.ref_rope(t, fr)
    kat_t = np.array([[[1.0, 2.0, 3.0, 4.0]]], np.float32)
    kat_f = np.array([[[[0.5, -0.866], [0.866, 0.5]], [[0.0, -1.0], [1.0, 0.0]]]], np.float32)
    vec["rope_kat_t"], vec["rope_kat_freqs"] = kat_t, kat_f
    vec["rope_kat_out"] = oracle.ref_rope(kat_t, kat_f)

    a = normal(rng, 8, 32)
    wb = oracle.f32_to_bf16_bits(normal(rng, 16, 32, sigma=0.02))
    vec["gemm_a"], vec["gemm_w_bf16"] = a, wb
    vec["gemm_out"] = oracle.ref_gemm_bf16(a, wb)

    # LayerNorm (no affine, eps 1e-6 as NumpyRT calls it) on DiT-width rows
    # with an offset mean, and SiLU over a range that includes large |x|.
    ln_x = normal(rng, 6, 2048, sigma=2.0) + np.float32(0.75)
    vec["ln_x"] = ln_x
    vec["ln_out"] = oracle.ref_layernorm(ln_x, 1e-6)
    silu_x = np.concatenate([normal(rng, 1000, sigma=4.0),
                             np.array([0.0, -0.0, 1e-8, -1e-8, 30.0, -30.0, 88.0, -88.0,
                                       -100.0], np.float32)]).astype(np.float32)
    vec["silu_x"] = silu_x
    vec["silu_out"] = oracle.ref_silu(silu_x)
    # GELU (exact erf form) over the MLP's activation range and its tails.
    gelu_x = np.concatenate([normal(rng, 1000, sigma=3.0),
                             np.array([0.0, -0.0, 1e-8, -1e-8, 5.0, -5.0, 10.0, -10.0, 40.0,
                                       -40.0], np.float32)]).astype(np.float32)
    vec["gelu_x"] = gelu_x
    vec["gelu_out"] = oracle.ref_gelu(gelu_x)
    # Softmax rows: ordinary, a large offset, a row with a dominant entry and
    # a constant row.
    sm_x = normal(rng, 5, 77, sigma=3.0)
    sm_x[1] += np.float32(500.0)
    sm_x[2, 13] = np.float32(60.0)
    sm_x[3] = np.float32(-2.5)
    vec["softmax_x"] = sm_x
    vec["softmax_out"] = oracle.ref_softmax(sm_x)

    np.savez_compressed(OUT, **vec)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(vec)} arrays)")


if __name__ == "__main__":
    main()
