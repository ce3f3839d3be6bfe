"""Parity of the bf16-input / f32-accumulate attention path with the oracle.

Stated tolerance of this path: relative 2e-2, measured normwise as
max|out - ref| <= 2e-2 * max|ref| against anima_rt's f32 flash attention
(the oracle) on identical seeded inputs.  Q, K, V and the probabilities P
are rounded to bf16 before the MFMAs; scores, softmax and accumulation stay
f32.  The observed error is also reported against fp64 brute force.
"""
import math
import os

import numpy as np
import pytest

import oracle
from anima_hip import AnimaHipError, rt
from anima_hip.rope import generate_rope_freqs

pytestmark = pytest.mark.gpu

REL = 2e-2
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "anima_rt_ref_vectors.npz")


def randn(rng, *shape):
    return rng.standard_normal(shape, dtype=np.float32)


def rel_err(out, ref):
    return float(np.abs(out - ref).max() / np.abs(ref).max())


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


@pytest.mark.parametrize("name", ["flash_small", "flash_tiles"])
def test_bf16_golden(name):
    g = np.load(GOLDEN)
    q, k, v = g[f"{name}_q"], g[f"{name}_k"], g[f"{name}_v"]
    out = rt.sdpa(q, k, v, 1.0 / math.sqrt(128), False, mode=rt.BF16)
    err = rel_err(out, g[f"{name}_out"])
    print(f"bf16 {name}: rel err {err:.3e}", flush=True)
    assert err <= REL


@pytest.mark.parametrize("sq,sk,causal", [(1, 1, False), (77, 77, False), (129, 513, False),
                                          (1000, 511, False), (256, 4097, False),
                                          (300, 300, True), (520, 100, True)])
def test_bf16_shapes(sq, sk, causal):
    rng = np.random.default_rng(sq * 13 + sk)
    q, k, v = randn(rng, 3, sq, 128), randn(rng, 3, sk, 128), randn(rng, 3, sk, 128)
    print(f"bf16 case sq={sq} sk={sk} causal={causal}", flush=True)
    out = rt.sdpa(q, k, v, is_causal=causal, mode=rt.BF16)
    ref = oracle.flash_sdpa(q, k, v, is_causal=causal, threads=3)
    assert rel_err(out, ref) <= REL


def test_bf16_rejects_other_head_dims():
    rng = np.random.default_rng(0)
    q = randn(rng, 1, 8, 64)
    with pytest.raises(AnimaHipError, match="D == 128"):
        rt.sdpa(q, q, q, mode=rt.BF16)


def test_bf16_self_attention_256_and_fp64():
    rng = np.random.default_rng(1001)
    B, S, H, D = 1, 256, 16, 128
    q, k, v = randn(rng, B, S, H, D), randn(rng, B, S, H, D), randn(rng, B, S, H, D)
    f = generate_rope_freqs(16, 16)
    ones = np.ones(D, np.float32)
    out = rt.attention(q, k, v, ones, ones, f, mode=rt.BF16)
    ref = oracle.attention_dataflow(q, k, v, ones, ones, f)
    err = rel_err(out, ref)
    print(f"bf16 256 tokens rel err {err:.3e}", flush=True)
    assert err <= REL


def test_bf16_self_attention_4096_all_heads():
    """B=2, H=16, S=4096: full problem on the GPU, all 32 slices vs the oracle."""
    import fullsize
    q, k, v, f = fullsize.self_case(4096, (64, 64), 3003)
    ones = np.ones(128, np.float32)
    out = rt.attention(q, k, v, ones, ones, f, mode=rt.BF16)
    fullsize.check_all_slices(out, fullsize.self_ref(4096, (64, 64), 3003), rt.BF16,
                              "bf16 self-attention 4096 tokens")


def test_bf16_deterministic():
    rng = np.random.default_rng(5)
    q, k, v = randn(rng, 2, 700, 128), randn(rng, 2, 900, 128), randn(rng, 2, 900, 128)
    a = rt.sdpa(q, k, v, mode=rt.BF16)
    np.testing.assert_array_equal(a, rt.sdpa(q, k, v, mode=rt.BF16))
