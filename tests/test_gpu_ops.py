"""The reference runtime's remaining operators through the drop-in C-ABI
(anima_rt_run_gelu/_silu/_layernorm/_softmax/_bias_add) and the NumpyDiT
host-object mirrors (AnimaRT's run_layernorm/run_gelu/run_silu, AnimaVK's
vk_run_gemm) against the oracle, which is bit-identical to the reference.

Tolerances: GELU and SiLU within 4 float32 ulp of the result plus one ulp of
erf/exp times |x| (device erf/exp against glibc's); LayerNorm relative 2e-6
(another summation order over the row); softmax 1e-5 against the reference
and 2e-6 against fp64; bias_add exact; the bf16-weight GEMM's f32 mode
1e-5 of the output scale.
"""
import numpy as np
import pytest

import oracle
from anima_hip import rt

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


def _ulp_close(a, b, x, n=4):
    """|a - b| <= n ulp(b) + 1.2e-7 |x|: a few ulp of the result, plus one ulp
    of erf/exp carried by the factor x (where erf(x/sqrt 2) is +-1 to within
    an ulp, GELU's exact result is 0 or x but an ulp of erf gives |x| 6e-8)."""
    tol = n * np.spacing(np.abs(b).astype(np.float32)) + np.float32(1.2e-7) * np.abs(x)
    assert np.all(np.abs(a - b) <= tol), float(np.max(np.abs(a - b) - tol))


def test_gelu_silu_vs_oracle():
    rng = np.random.default_rng(81)
    x = np.concatenate([rng.standard_normal(100003).astype(np.float32) * 4,
                        np.array([0.0, -0.0, 1e-30, -1e-30, 9.0, -9.0, 40.0, -40.0, 88.0, -88.0],
                                 np.float32)])
    print("gelu/silu", x.size, flush=True)
    _ulp_close(rt.gelu(x), oracle.gelu(x), x)
    _ulp_close(rt.silu(x), oracle.silu(x), x)


@pytest.mark.parametrize("m,d", [(1, 1), (7, 77), (33, 2048), (5, 3000)])
def test_layernorm_vs_oracle(m, d):
    rng = np.random.default_rng(82 + d)
    x = (rng.standard_normal((m, d)) * 3 + 0.5).astype(np.float32)
    print(f"layernorm {m}x{d}", flush=True)
    got, ref = rt.layernorm(x), oracle.layernorm(x)
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("m,d", [(1, 1), (3, 77), (64, 512), (2, 4097)])
def test_softmax_vs_oracle(m, d):
    rng = np.random.default_rng(83 + d)
    x = (rng.standard_normal((m, d)) * 5).astype(np.float32)
    x[0] += np.float32(300.0)
    print(f"softmax {m}x{d}", flush=True)
    got, ref = rt.softmax(x), oracle.softmax(x)
    # The reference sums the row's exponentials serially in float32, which
    # drifts ~sqrt(d) 2^-24 relative; the device sums pairwise.  Against the
    # reference 1e-5, against fp64 2e-6.
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-12)
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    np.testing.assert_allclose(got, e / e.sum(axis=1, keepdims=True), rtol=2e-6, atol=1e-12)
    np.testing.assert_allclose(got.sum(axis=1), 1.0, rtol=1e-5)


def test_bias_add():
    rng = np.random.default_rng(84)
    c = rng.standard_normal((9, 33)).astype(np.float32)
    b = rng.standard_normal(33).astype(np.float32)
    ref = c + b
    rt.bias_add(c, b)
    np.testing.assert_array_equal(c, ref)


def test_numpyrt_mirror_methods():
    """AnimaRT's run_layernorm / run_gelu / run_silu take NumpyRT's arguments
    (phone_pipeline_nd.py:50-60): [M, D] rows and flat vectors."""
    rng = np.random.default_rng(85)
    x = rng.standard_normal((12, 256)).astype(np.float32)
    r = rt.AnimaRT({})
    np.testing.assert_allclose(r.run_layernorm(x, 256), oracle.layernorm(x), rtol=2e-6,
                               atol=2e-6)
    _ulp_close(r.run_gelu(x.reshape(-1)), oracle.gelu(x).reshape(-1), x.reshape(-1))
    _ulp_close(r.run_silu(x.reshape(-1)), oracle.silu(x).reshape(-1), x.reshape(-1))


def test_anima_vk_gemm_from_checkpoint(tmp_path):
    """AnimaVK.vk_run_gemm(name, x, out, M, N, K) on a bf16 weight from a
    safetensors file equals the reference's GEMM to f32-mode precision."""
    import safetensors_file
    rng = np.random.default_rng(86)
    w = oracle.f32_to_bf16_bits(rng.standard_normal((96, 200)).astype(np.float32) * 0.02)
    path = tmp_path / "w.safetensors"
    safetensors_file.write(path, {"net.blocks.0.mlp.layer1.weight": ("BF16", w)})
    x = rng.standard_normal((37, 200)).astype(np.float32)
    out = np.zeros((37, 96), np.float32)
    with rt.Weights(path) as store:
        rt.AnimaVK(store).vk_run_gemm("blocks.0.mlp.layer1.weight", x, out, 37, 96, 200)
        with pytest.raises(RuntimeError, match="expected BF16"):
            rt.AnimaVK(store).vk_run_gemm("blocks.0.mlp.layer1.weight", x, out, 37, 96, 100)
    ref = oracle.gemm_bf16(x, w)
    assert np.abs(out - ref).max() <= 1e-5 * np.abs(ref).max()


def test_timing_hook_reports_the_last_host_call():
    """anima_hip_last_call_ms: device time of the last host-pointer call, the
    kernels between its uploads and downloads inside the whole call."""
    rng = np.random.default_rng(87)
    q = rng.standard_normal((16, 1024, 128)).astype(np.float32)
    rt.sdpa_flash(q, q, q)
    k_ms, t_ms = rt.last_call_ms()
    print(f"sdpa 16x1024^2: kernels {k_ms:.3f} ms of {t_ms:.3f} ms", flush=True)
    assert 0.0 < k_ms < t_ms < 1e4
    rt.softmax(q[0])
    k2, t2 = rt.last_call_ms()
    assert 0.0 < k2 <= t2 and (k2, t2) != (k_ms, t_ms)


def test_numpyrt_sdpa_and_rmsnorm_on_numpy_attention_views():
    """AnimaRT.run_rmsnorm / run_sdpa called the way NumpyAttention.forward
    calls NumpyRT (numpy_dit.py:283-292, phone_pipeline_nd.py:53-68): the
    per-head RMSNorm on [B,S,H,D] projections, one of them a column block of
    a fused [B*S, 3*H*D] projection (a strided view), then SDPA on the
    non-contiguous q/k/v.transpose(0,2,1,3) views.  The result must equal the
    reference's marshaling (ascontiguousarray of the [B*H,S,D] reshape, flash
    attention with scale 1/sqrt(D)) as the oracle computes it."""
    B, S, H, D = 2, 96, 4, 128
    rng = np.random.default_rng(88)
    fused = rng.standard_normal((B * S, 3 * H * D)).astype(np.float32)
    q = fused[:, :H * D].reshape(B, S, H, D)          # a strided view
    k = np.ascontiguousarray(fused[:, H * D:2 * H * D]).reshape(B, S, H, D)
    v = np.ascontiguousarray(fused[:, 2 * H * D:]).reshape(B, S, H, D)
    qw = rng.uniform(0.5, 1.5, D).astype(np.float32)
    r = rt.AnimaRT({"blk.q_norm.weight": qw, "blk.k_norm.weight": np.ones(D, np.float32)})
    qn = r.run_rmsnorm(q, "blk.q_norm")
    kn = r.run_rmsnorm(k, "blk.k_norm")
    np.testing.assert_array_equal(qn, oracle.rmsnorm(np.ascontiguousarray(q), qw))
    np.testing.assert_array_equal(kn, oracle.rmsnorm(k, np.ones(D, np.float32)))

    qs, ks, vs = (t.transpose(0, 2, 1, 3) for t in (qn, kn, v))
    assert not qs.flags.c_contiguous
    out = r.run_sdpa(qs, ks, vs)
    assert out.shape == (B, H, S, D)
    ref = oracle.flash_sdpa(*(np.ascontiguousarray(t.reshape(B * H, S, D)) for t in (qs, ks, vs)))
    assert np.abs(out.reshape(B * H, S, D) - ref).max() <= 1e-4
    # The caller's arrays are left as they were.
    np.testing.assert_array_equal(qs, qn.transpose(0, 2, 1, 3))
