"""The oracle against the reference runtime compiled from its sources.

oracle/_ref/libanima_rt_ref.so exists where `make -C oracle ref` ran next to
the reference tree; elsewhere these tests skip and the golden vectors of
tests/test_oracle.py carry the same check.
"""
import math

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")


@pytest.mark.parametrize("bh,sq,sk,d,causal", [
    (2, 256, 256, 128, False),   # config-1 tile choice qSplit=64
    (1, 800, 520, 128, False),   # qSplit=256, two kv blocks (512 + 8)
    (3, 31, 77, 64, True),
    (1, 1, 1, 128, False),
    (2, 70, 9, 100, True),
])
def test_flash_bitwise_vs_reference(bh, sq, sk, d, causal):
    rng = np.random.default_rng(sq * 7 + sk)
    q = rng.standard_normal((bh, sq, d)).astype(np.float32)
    k = rng.standard_normal((bh, sk, d)).astype(np.float32)
    v = rng.standard_normal((bh, sk, d)).astype(np.float32)
    s = 1.0 / math.sqrt(d)
    np.testing.assert_array_equal(oracle.flash_sdpa(q, k, v, s, causal),
                                  oracle.ref_flash_sdpa(q, k, v, s, causal))


@pytest.mark.parametrize("causal", [False, True])
def test_math_bitwise_vs_reference(causal):
    rng = np.random.default_rng(4)
    q = rng.standard_normal((2, 40, 128)).astype(np.float32)
    k = rng.standard_normal((2, 40, 128)).astype(np.float32)
    v = rng.standard_normal((2, 40, 128)).astype(np.float32)
    np.testing.assert_array_equal(oracle.math_sdpa(q, k, v, 0.088, causal),
                                  oracle.ref_math_sdpa(q, k, v, 0.088, causal))


def test_rmsnorm_rope_gemm_bitwise_vs_reference():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((257, 128)).astype(np.float32)
    w = rng.standard_normal(128).astype(np.float32)
    np.testing.assert_array_equal(oracle.rmsnorm(x, w), oracle.ref_rmsnorm(x, w))
    np.testing.assert_array_equal(oracle.rmsnorm(x, None, 1e-5), oracle.ref_rmsnorm(x, None, 1e-5))
    t = rng.standard_normal((4, 96, 128)).astype(np.float32)
    f = oracle.rope_freqs(12, 8)
    np.testing.assert_array_equal(oracle.rope(t, f), oracle.ref_rope(t, f))
    a = rng.standard_normal((5, 64)).astype(np.float32)
    wb = oracle.f32_to_bf16_bits(rng.standard_normal((9, 64)).astype(np.float32))
    np.testing.assert_array_equal(oracle.gemm_bf16(a, wb), oracle.ref_gemm_bf16(a, wb))


def test_layernorm_silu_bitwise_vs_reference():
    rng = np.random.default_rng(44)
    x = (rng.standard_normal((33, 2048)) * 5 - 2).astype(np.float32)
    np.testing.assert_array_equal(oracle.layernorm(x), oracle.ref_layernorm(x))
    np.testing.assert_array_equal(oracle.layernorm(x[:, :77], 1e-5), oracle.ref_layernorm(x[:, :77], 1e-5))
    np.testing.assert_array_equal(oracle.silu(x), oracle.ref_silu(x))
    np.testing.assert_array_equal(oracle.gelu(x), oracle.ref_gelu(x))
    np.testing.assert_array_equal(oracle.softmax(x[:, :300]), oracle.ref_softmax(x[:, :300]))


@pytest.mark.parametrize("where", ["q_row", "k_row", "v_elem"])
def test_flash_nan_pattern_vs_reference(where):
    # The reference's NaN behaviour, which the GPU kernels reproduce: a query
    # row whose scores are all NaN is skipped and stays zero
    # (flash_attention.h:148-152, 194-201); a NaN key makes every row of its
    # head NaN; a NaN value element makes its column NaN.  The oracle matches
    # the compiled reference bit for bit, NaN positions included.
    rng = np.random.default_rng(17)
    q, k, v = (rng.standard_normal((2, 600, 128)).astype(np.float32) for _ in range(3))
    {"q_row": q, "k_row": k, "v_elem": v}[where][0, 40, 7 if where == "v_elem" else 3] = np.nan
    out = oracle.flash_sdpa(q, k, v, 0.088)
    np.testing.assert_array_equal(out, oracle.ref_flash_sdpa(q, k, v, 0.088))
    if where == "q_row":
        assert np.all(out[0, 40] == 0) and np.isfinite(np.delete(out[0], 40, axis=0)).all()
    elif where == "k_row":
        assert np.isnan(out[0]).all() and np.isfinite(out[1]).all()
    else:
        assert np.isnan(out[0, :, 7]).all() and np.isfinite(np.delete(out[0], 7, axis=1)).all()
