"""Parity of the HIP f32 attention path with the oracle, through the C-ABI.

Tolerance: max-abs 1e-4 against anima_rt's CPU flash attention (the
oracle restatement, itself bit-identical to the reference) on identical
seeded inputs.  RMSNorm and RoPE are bit-exact.
"""
import math
import os

import numpy as np
import pytest

import oracle
from anima_hip import rt
from anima_hip.rope import generate_rope_freqs

pytestmark = pytest.mark.gpu

TOL = 1e-4
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "anima_rt_ref_vectors.npz")


def randn(rng, *shape):
    return rng.standard_normal(shape, dtype=np.float32)


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()
    yield


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN)


@pytest.mark.parametrize("name", ["flash_small", "flash_causal", "flash_tiles", "flash_d80"])
def test_flash_golden(gold, name):
    q, k, v = gold[f"{name}_q"], gold[f"{name}_k"], gold[f"{name}_v"]
    causal = bool(gold[f"{name}_causal"])
    print(f"case {name} q{q.shape} k{k.shape} causal={causal}", flush=True)
    out = rt.sdpa_flash(q, k, v, 1.0 / math.sqrt(q.shape[-1]), causal)
    assert np.abs(out - gold[f"{name}_out"]).max() <= TOL


def test_math_sdpa_golden(gold):
    out = rt.sdpa_math(gold["math_q"], gold["math_k"], gold["math_v"], 1.0 / math.sqrt(128))
    assert np.abs(out - gold["math_out"]).max() <= TOL


def test_rmsnorm_bit_exact(gold):
    np.testing.assert_array_equal(rt.rmsnorm(gold["rms_x4"], gold["rms_w4"], 1e-6),
                                  gold["rms_out4"])
    np.testing.assert_array_equal(rt.rmsnorm(gold["rms_x64"], gold["rms_w64"], 1e-6),
                                  gold["rms_out64"])
    np.testing.assert_array_equal(rt.rmsnorm(gold["rms_x4"], None, 1e-5), gold["rms_out4_nw"])
    rng = np.random.default_rng(1)
    x = randn(rng, 4099, 128) * 3
    w = randn(rng, 128)
    np.testing.assert_array_equal(rt.rmsnorm(x, w), oracle.rmsnorm(x, w))


def test_rope_bit_exact(gold):
    np.testing.assert_array_equal(rt.rope(gold["rope_t"], gold["rope_freqs"]), gold["rope_out"])
    np.testing.assert_array_equal(rt.rope(gold["rope_kat_t"], gold["rope_kat_freqs"]),
                                  gold["rope_kat_out"])
    rng = np.random.default_rng(2)
    t = randn(rng, 3, 6144, 128)
    f = generate_rope_freqs(96, 64)
    np.testing.assert_array_equal(rt.rope(t, f), oracle.rope(t, f))


@pytest.mark.parametrize("sq,sk", [(1, 1), (77, 77), (129, 513), (1000, 511), (300, 77),
                                   (64, 4097), (256, 1)])
def test_flash_tails(sq, sk):
    rng = np.random.default_rng(sq * 31 + sk)
    bh = 3
    q, k, v = randn(rng, bh, sq, 128), randn(rng, bh, sk, 128), randn(rng, bh, sk, 128)
    print(f"tail case sq={sq} sk={sk}", flush=True)
    out = rt.sdpa_flash(q, k, v)
    ref = oracle.flash_sdpa(q, k, v, threads=3)
    assert np.abs(out - ref).max() <= TOL


@pytest.mark.parametrize("sq,sk", [(300, 300), (40, 200), (520, 100)])
def test_flash_causal(sq, sk):
    rng = np.random.default_rng(sq + sk)
    q, k, v = randn(rng, 2, sq, 128), randn(rng, 2, sk, 128), randn(rng, 2, sk, 128)
    out = rt.sdpa_flash(q, k, v, is_causal=True)
    ref = oracle.flash_sdpa(q, k, v, is_causal=True, threads=2)
    assert np.abs(out - ref).max() <= TOL


@pytest.mark.parametrize("d", [16, 64, 100, 256])
def test_flash_generic_head_dims(d):
    rng = np.random.default_rng(d)
    q, k, v = randn(rng, 2, 70, d), randn(rng, 2, 90, d), randn(rng, 2, 90, d)
    out = rt.sdpa_flash(q, k, v)
    ref = oracle.flash_sdpa(q, k, v, threads=2)
    assert np.abs(out - ref).max() <= TOL


def test_self_attention_256_tokens():
    """B=1, H=16, S=256 (16x16 grid), N(0,1) q/k/v, RMSNorm(w=1) + RoPE."""
    rng = np.random.default_rng(1001)
    B, S, H, D = 1, 256, 16, 128
    q, k, v = randn(rng, B, S, H, D), randn(rng, B, S, H, D), randn(rng, B, S, H, D)
    f = generate_rope_freqs(16, 16)
    ones = np.ones(D, np.float32)
    ref = oracle.attention_dataflow(q, k, v, ones, ones, f)
    out = rt.attention(q, k, v, ones, ones, f)
    assert np.abs(out - ref).max() <= TOL
    # Same through the drop-in SDPA on the reference's own pre-processed inputs.
    qn = oracle.numpy_rope(oracle.rmsnorm(q, ones), f).transpose(0, 2, 1, 3).reshape(16, S, D)
    kn = oracle.numpy_rope(oracle.rmsnorm(k, ones), f).transpose(0, 2, 1, 3).reshape(16, S, D)
    vt = v.transpose(0, 2, 1, 3).reshape(16, S, D)
    o2 = rt.sdpa_flash(qn, kn, vt)
    assert np.abs(o2 - oracle.flash_sdpa(qn, kn, vt)).max() <= TOL
    assert np.abs(o2 - oracle.sdpa_fp64(qn, kn, vt)).max() <= TOL


def test_attention_prologue_bit_exact_pieces():
    """The fused path's RMSNorm+RoPE equals the oracle's bit for bit: checked
    by feeding V = identity-like rows so the output exposes nothing else; here
    simply compare the drop-in rmsnorm+rope composition to the oracle."""
    rng = np.random.default_rng(5)
    B, S, H, D = 2, 64, 4, 128
    x = randn(rng, B, S, H, D)
    w = randn(rng, D)
    f = generate_rope_freqs(8, 8)
    xn = rt.rmsnorm(x, w)
    np.testing.assert_array_equal(xn, oracle.rmsnorm(x, w))
    r = rt.AnimaRT()
    np.testing.assert_array_equal(r.run_rope(xn, f), oracle.numpy_rope(xn, f))


def test_self_attention_4096_tokens_all_heads():
    """Config 3, B=2, H=16, S=4096 (64x64 grid): the whole problem on the GPU,
    every one of the 32 (batch, head) slices against the oracle; outputs lie
    within the per-dim range of V (softmax weights are a convex combination)."""
    import fullsize
    q, k, v, f = fullsize.self_case(4096, (64, 64), 3003)
    ones = np.ones(128, np.float32)
    out = rt.attention(q, k, v, ones, ones, f)
    assert np.all(out <= v.max(axis=1, keepdims=True) + 1e-5)
    assert np.all(out >= v.min(axis=1, keepdims=True) - 1e-5)
    fullsize.check_all_slices(out, fullsize.self_ref(4096, (64, 64), 3003), rt.F32,
                              "self-attention 4096 tokens")


def test_deterministic():
    rng = np.random.default_rng(77)
    q, k, v = randn(rng, 4, 700, 128), randn(rng, 4, 900, 128), randn(rng, 4, 900, 128)
    np.testing.assert_array_equal(rt.sdpa_flash(q, k, v), rt.sdpa_flash(q, k, v))
