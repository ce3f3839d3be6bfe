"""Cross-attention with the cached text-context K/V, the projection GEMM, and
the rectangular high-resolution configuration, against the oracle.

Tolerances: max-abs 1e-4 for the f32 path; normwise relative 2e-2
(max|out-ref| <= 2e-2 max|ref|) for the bf16-input path.
"""
import os

import numpy as np
import pytest

import oracle
from anima_hip import AnimaHipError, rt
from anima_hip.rope import generate_rope_freqs

pytestmark = pytest.mark.gpu

TOL = 1e-4
REL = 2e-2
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "anima_rt_ref_vectors.npz")


def randn(rng, *shape, sigma=1.0):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma)).astype(np.float32)


def rel_err(out, ref):
    return float(np.abs(out - ref).max() / np.abs(ref).max())


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


def test_gemm_bf16_golden_and_shapes():
    g = np.load(GOLDEN)
    c = rt.gemm_bf16(g["gemm_a"], g["gemm_w_bf16"])
    assert np.abs(c - g["gemm_out"]).max() <= 1e-5 * max(1.0, np.abs(g["gemm_out"]).max())
    rng = np.random.default_rng(4)
    for M, N, K in [(37, 130, 77), (1, 1, 1), (300, 257, 1024), (5, 9, 0)]:
        a = randn(rng, M, K)
        w = oracle.f32_to_bf16_bits(randn(rng, N, K, sigma=0.02))
        ref = oracle.gemm_bf16(a, w) if K else np.zeros((M, N), np.float32)
        out = rt.gemm_bf16(a, w)
        assert np.abs(out - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max()), (M, N, K)
    a, b = randn(rng, 64, 96), randn(rng, 40, 96)
    np.testing.assert_allclose(rt.gemm_fp32(a, b), a.astype(np.float64) @ b.T.astype(np.float64),
                               atol=2e-5)


def _cross_256x512(seed=2002, Bc=1):
    """B=2 CFG, Sq=256 latent tokens, Sk=512 context tokens, 16 heads x 128.
    x ~ N(0,1) [2,256,2048]; ctx ~ N(0,0.5) [Bc,512,1024]; Wq/Wk/Wv bf16 ~ N(0,0.02)."""
    rng = np.random.default_rng(seed)
    x = randn(rng, 2, 256, 2048)
    ctx = randn(rng, Bc, 512, 1024, sigma=0.5)
    wq = oracle.f32_to_bf16_bits(randn(rng, 2048, 2048, sigma=0.02))
    wk = oracle.f32_to_bf16_bits(randn(rng, 2048, 1024, sigma=0.02))
    wv = oracle.f32_to_bf16_bits(randn(rng, 2048, 1024, sigma=0.02))
    return x, ctx, wq, wk, wv


@pytest.mark.parametrize("Bc", [1, 2])
def test_cross_attention_256x512_cached_kv(Bc):
    x, ctx, wq, wk, wv = _cross_256x512(Bc=Bc)
    ones = np.ones(128, np.float32)
    # Oracle: projections with anima_rt's bf16 GEMM, then NumpyAttention's
    # norm -> SDPA dataflow (no RoPE for cross-attention).
    q_ref = oracle.gemm_bf16(x.reshape(-1, 2048), wq).reshape(2, 256, 16, 128)
    k_ref = np.stack([oracle.gemm_bf16(ctx[b], wk) for b in range(Bc)]).reshape(Bc, 512, 16, 128)
    v_ref = np.stack([oracle.gemm_bf16(ctx[b], wv) for b in range(Bc)]).reshape(Bc, 512, 16, 128)
    kb = np.broadcast_to(k_ref, (2, 512, 16, 128))
    vb = np.broadcast_to(v_ref, (2, 512, 16, 128))
    ref = oracle.attention_dataflow(q_ref, kb, vb, ones, ones, None,
                                    sdpa=lambda a, b, c: oracle.flash_sdpa(a, b, c, threads=8))

    q = rt.gemm_bf16(x.reshape(-1, 2048), wq).reshape(2, 256, 16, 128)
    assert np.abs(q - q_ref).max() <= 1e-4
    cache = rt.ContextKV(ctx, wk, wv, ones, heads=16, head_dim=128)
    try:
        out = cache.attend(q, ones)
        err = float(np.abs(out - ref).max())
        print(f"cross 256x512 Bc={Bc} f32 max_abs={err:.3e}", flush=True)
        assert err <= TOL
        # The cache is reused: a second call (next denoise step) is identical.
        np.testing.assert_array_equal(cache.attend(q, ones), out)
    finally:
        cache.close()

    cache = rt.ContextKV(ctx, wk, wv, ones, heads=16, head_dim=128, mode=rt.BF16)
    try:
        out = cache.attend(q, ones)
        err = rel_err(out, ref)
        print(f"cross 256x512 Bc={Bc} bf16 rel={err:.3e}", flush=True)
        assert err <= REL
    finally:
        cache.close()

    cache = rt.ContextKV(ctx, wk, wv, ones, heads=16, head_dim=128, mode=rt.F32X3)
    try:
        out = cache.attend(q, ones)
        err = float(np.abs(out - ref).max())
        print(f"cross 256x512 Bc={Bc} f32x3 max_abs={err:.3e}", flush=True)
        assert err <= TOL
    finally:
        cache.close()


def test_cross_attention_errors():
    rng = np.random.default_rng(1)
    ctx = randn(rng, 3, 16, 32)
    w = oracle.f32_to_bf16_bits(randn(rng, 2 * 64, 32, sigma=0.02))
    cache = rt.ContextKV(ctx, w, w, None, heads=2, head_dim=64)
    try:
        with pytest.raises(AnimaHipError, match="batch"):
            cache.attend(randn(rng, 2, 8, 2, 64))  # Bc=3 cannot serve B=2
        out = cache.attend(randn(rng, 3, 8, 2, 64))  # generic head dim path
        assert np.isfinite(out).all()
    finally:
        cache.close()
    for mode in (rt.BF16, rt.F32X3):
        with pytest.raises(AnimaHipError, match="D == 128"):
            rt.ContextKV(ctx, w, w, None, heads=2, head_dim=64, mode=mode)


@pytest.mark.parametrize("mode", [rt.F32, rt.F32X3, rt.BF16])
def test_rectangular_96x64_grid_6144_tokens_all_heads(mode):
    """Config 5: B=2, H=16, S=6144 (96x64 grid, rectangular RoPE)
    self-attention, and the 6144 x 512 cross-attention through the context
    K/V cache (ContextKV) of a [2, 512, 1024] context; all 32 (batch, head)
    slices of both against the oracle, in every arithmetic mode.  (6144 is a
    multiple of every tile; the ragged tails are covered by the tail tests.)"""
    import fullsize
    q, k, v, f = fullsize.self_case(6144, (96, 64), 5005)
    ones = np.ones(128, np.float32)
    out = rt.attention(q, k, v, ones, ones, f, mode=mode)
    fullsize.check_all_slices(out, fullsize.self_ref(6144, (96, 64), 5005), mode,
                              "self-attention 6144 tokens")
    ctx, wk, wv = fullsize.context_case(5006)
    cache = rt.ContextKV(ctx, wk, wv, ones, heads=16, head_dim=128, mode=mode)
    try:
        out = cache.attend(fullsize.cross_q(6144, 5007), ones)
    finally:
        cache.close()
    fullsize.check_all_slices(out, fullsize.cross_ref(6144, 5007, 5006), mode,
                              "cross-attention 6144x512 (cached context)")


@pytest.mark.parametrize("mode", [rt.F32X3, rt.F32])
def test_broadcast_context_4096_tokens_equals_repeated_context(mode):
    """One context (Bc = 1) serving both CFG entries at 4096 query tokens, the
    grid on which f32x3 prepares its raw query rows inside the flash kernel,
    with a norm weight on q: equal bit for bit to the same context repeated
    (Bc = 2), and two slices within the f32 tolerance of the oracle."""
    import fullsize
    ctx, wk, wv = fullsize.context_case(6006, Bc=1)
    rng = np.random.default_rng(6007)
    qw = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    kw = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    q = fullsize.cross_q(4096, 6008)
    outs = []
    for c in (ctx, np.concatenate([ctx, ctx])):
        cache = rt.ContextKV(c, wk, wv, kw, heads=16, head_dim=128, mode=mode)
        try:
            print(f"cross 4096x512 Bc={c.shape[0]} mode={mode}", flush=True)
            outs.append(cache.attend(q, qw))
        finally:
            cache.close()
    np.testing.assert_array_equal(outs[0], outs[1])
    k = oracle.gemm_bf16(ctx[0], wk).reshape(1, 512, 16, 128)
    v = oracle.gemm_bf16(ctx[0], wv).reshape(1, 512, 16, 128)
    for b, h in ((0, 2), (1, 13)):
        ref = oracle.attention_dataflow(q[b:b + 1, :, h:h + 1], k[:, :, h:h + 1],
                                        v[:, :, h:h + 1], qw, kw, None)[0, :, 0]
        err = float(np.abs(outs[0][b, :, h] - ref).max())
        print(f"cross 4096x512 broadcast mode={mode} b={b} h={h}: max-abs {err:.3e}", flush=True)
        assert err <= 1e-4


@pytest.mark.parametrize("mode", [rt.F32X3, rt.BF16, rt.F32])
def test_host_call_batch_groups_equal_per_batch_calls(mode):
    """anima_hip_cross_attention (host pointers) at B = 2, 4096 query tokens
    runs as two batch groups, each reading its own entry of a Bc = 2 context
    cache while the other group's copies run; equal bit for bit to B = 1 calls
    on caches of each context entry alone."""
    import fullsize
    ctx, wk, wv = fullsize.context_case(7007)
    rng = np.random.default_rng(7008)
    qw = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    kw = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    q = fullsize.cross_q(4096, 7009)
    print(f"cross host groups mode={mode}", flush=True)
    cache = rt.ContextKV(ctx, wk, wv, kw, heads=16, head_dim=128, mode=mode)
    try:
        full = cache.attend(q, qw)
    finally:
        cache.close()
    for b in range(2):
        one = rt.ContextKV(ctx[b:b + 1], wk, wv, kw, heads=16, head_dim=128, mode=mode)
        try:
            np.testing.assert_array_equal(full[b:b + 1], one.attend(q[b:b + 1], qw))
        finally:
            one.close()
