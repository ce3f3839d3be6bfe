"""Pins the CPU oracle (no GPU needed).

Every oracle function is checked against something other than itself:
the golden vectors written by the reference runtime (tests/golden), the
reference compiled from source where present (oracle/_ref), fp64 closed
forms, and invariants that a dropped term, a wrong index or a transposed
operand would break.
"""
import math
import os

import numpy as np
import pytest

import oracle
from anima_hip.rope import generate_rope_freqs

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "anima_rt_ref_vectors.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN)


# ----------------------------------------------------------- golden vectors

@pytest.mark.parametrize("name", ["flash_small", "flash_causal", "flash_tiles", "flash_d80"])
def test_flash_matches_reference_vectors_bitwise(gold, name):
    q, k, v = gold[f"{name}_q"], gold[f"{name}_k"], gold[f"{name}_v"]
    causal = bool(gold[f"{name}_causal"])
    out = oracle.flash_sdpa(q, k, v, 1.0 / math.sqrt(q.shape[-1]), causal)
    np.testing.assert_array_equal(out, gold[f"{name}_out"])


def test_flash_threads_bitwise_equal_single(gold):
    q, k, v = gold["flash_tiles_q"], gold["flash_tiles_k"], gold["flash_tiles_v"]
    q = np.concatenate([q, q[:, ::-1]], 0)
    k = np.concatenate([k, k], 0)
    v = np.concatenate([v, v[:, ::-1]], 0)
    np.testing.assert_array_equal(oracle.flash_sdpa(q, k, v, threads=2),
                                  oracle.flash_sdpa(q, k, v, threads=1))


def test_math_sdpa_matches_reference_vectors(gold):
    out = oracle.math_sdpa(gold["math_q"], gold["math_k"], gold["math_v"], 1.0 / math.sqrt(128))
    np.testing.assert_array_equal(out, gold["math_out"])


def test_rmsnorm_matches_reference_vectors(gold):
    np.testing.assert_array_equal(oracle.rmsnorm(gold["rms_x4"], gold["rms_w4"], 1e-6),
                                  gold["rms_out4"])
    np.testing.assert_array_equal(oracle.rmsnorm(gold["rms_x64"], gold["rms_w64"], 1e-6),
                                  gold["rms_out64"])
    np.testing.assert_array_equal(oracle.rmsnorm(gold["rms_x4"], None, 1e-5),
                                  gold["rms_out4_nw"])


def test_rope_matches_reference_vectors(gold):
    np.testing.assert_array_equal(oracle.rope(gold["rope_t"], gold["rope_freqs"]),
                                  gold["rope_out"])
    np.testing.assert_array_equal(oracle.rope(gold["rope_kat_t"], gold["rope_kat_freqs"]),
                                  gold["rope_kat_out"])


def test_rope_known_answer():
    # scripts/test_rope_debug.py:17-34: t=[1,2,3,4], pair 0 rotated by 60 deg
    # (cos .5, sin .866), pair 1 by 90 deg -> [-2.098, -4.0, 2.366, 2.0].
    t = np.array([[[1.0, 2.0, 3.0, 4.0]]], np.float32)
    f = np.array([[[[0.5, -0.866], [0.866, 0.5]], [[0.0, -1.0], [1.0, 0.0]]]], np.float32)
    np.testing.assert_allclose(oracle.rope(t, f)[0, 0], [-2.098, -4.0, 2.366, 2.0], atol=1e-6)
    # The [B,S,H,D] numpy form computes the same products and sums.
    np.testing.assert_array_equal(oracle.numpy_rope(t[:, :, None, :], f)[:, :, 0, :],
                                  oracle.rope(t, f))


def test_gemm_bf16_matches_reference_vectors(gold):
    np.testing.assert_array_equal(oracle.gemm_bf16(gold["gemm_a"], gold["gemm_w_bf16"]),
                                  gold["gemm_out"])


# ------------------------------------------------------------- fp64 / math

@pytest.mark.parametrize("bh,sq,sk,d,causal", [(2, 17, 33, 128, False), (1, 64, 64, 32, True),
                                               (2, 5, 600, 128, False), (1, 300, 7, 16, False)])
def test_flash_vs_fp64(bh, sq, sk, d, causal):
    rng = np.random.default_rng(bh * 1000 + sq)
    q = rng.standard_normal((bh, sq, d)).astype(np.float32)
    k = rng.standard_normal((bh, sk, d)).astype(np.float32)
    v = rng.standard_normal((bh, sk, d)).astype(np.float32)
    out = oracle.flash_sdpa(q, k, v, is_causal=causal)
    ref = oracle.sdpa_fp64(q, k, v, is_causal=causal)
    assert np.abs(out - ref).max() < 2e-6


def test_math_sdpa_is_scale_squared():
    rng = np.random.default_rng(7)
    q, k, v = (rng.standard_normal((2, 20, 128)).astype(np.float32) for _ in range(3))
    s = 1.0 / math.sqrt(128)
    out = oracle.math_sdpa(q, k, v, s)
    assert np.abs(out - oracle.sdpa_fp64(q, k, v, scale=s * s)).max() < 2e-6
    assert np.abs(out - oracle.sdpa_fp64(q, k, v, scale=s)).max() > 1e-2


def test_flash_invariants():
    rng = np.random.default_rng(3)
    v = rng.standard_normal((2, 40, 128)).astype(np.float32)
    k = rng.standard_normal((2, 40, 128)).astype(np.float32)
    # Q = 0 -> uniform weights -> mean of V.
    out = oracle.flash_sdpa(np.zeros((2, 9, 128), np.float32), k, v)
    np.testing.assert_allclose(out, np.broadcast_to(v.mean(1, keepdims=True), out.shape),
                               atol=2e-6)
    # One key -> output is that V row.
    out1 = oracle.flash_sdpa(rng.standard_normal((2, 9, 128)).astype(np.float32), k[:, :1],
                             v[:, :1])
    np.testing.assert_array_equal(out1, np.broadcast_to(v[:, :1], out1.shape))
    # Convex combination: every output lies within the per-dim range of V.
    q = rng.standard_normal((2, 9, 128)).astype(np.float32)
    o = oracle.flash_sdpa(q, k, v)
    assert np.all(o <= v.max(1, keepdims=True) + 1e-6)
    assert np.all(o >= v.min(1, keepdims=True) - 1e-6)
    # Key permutation invariance.
    perm = rng.permutation(40)
    np.testing.assert_allclose(oracle.flash_sdpa(q, k[:, perm], v[:, perm]), o, atol=2e-6)


def test_rmsnorm_vs_fp64():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((300, 128)).astype(np.float32) * 3
    w = rng.standard_normal(128).astype(np.float32)
    np.testing.assert_allclose(oracle.rmsnorm(x, w), oracle.rmsnorm_fp64(x, w), rtol=2e-6,
                               atol=2e-6)


def test_rope_norm_preserving():
    rng = np.random.default_rng(5)
    t = rng.standard_normal((3, 64, 128)).astype(np.float32)
    f = oracle.rope_freqs(8, 8)
    y = oracle.rope(t, f)
    pairs_in = t[..., :64] ** 2 + t[..., 64:] ** 2
    pairs_out = y[..., :64] ** 2 + y[..., 64:] ** 2
    np.testing.assert_allclose(pairs_out, pairs_in, rtol=3e-6, atol=1e-6)


# ---------------------------------------------------------------- RoPE table

@pytest.mark.parametrize("H,W,T", [(16, 16, 1), (96, 64, 1), (5, 3, 2)])
def test_rope_table_closed_form(H, W, T):
    got = oracle.rope_freqs(H, W, T)
    exp = oracle.rope_freqs_fp64(H, W, T)
    assert got.shape == (T * H * W, 64, 2, 2)
    # float32 angle rounding: |error| <= ~ulp(angle) with angles up to ~95 rad.
    np.testing.assert_allclose(got, exp, atol=2e-5)
    # Entry layout [cos, -sin; sin, cos].
    np.testing.assert_array_equal(got[..., 0, 0], got[..., 1, 1])
    np.testing.assert_array_equal(got[..., 0, 1], -got[..., 1, 0])


def test_rope_table_axes():
    H, W = 6, 4
    f = oracle.rope_freqs(H, W, 1)
    # T=1: the 22 temporal pairs are the identity rotation.
    np.testing.assert_array_equal(f[:, :22, 0, 0], 1.0)
    np.testing.assert_array_equal(f[:, :22, 1, 0], 0.0)
    grid = f.reshape(H, W, 64, 2, 2)
    # Height pairs depend only on the row, width pairs only on the column.
    assert np.all(grid[:, :1, 22:43] == grid[:, :, 22:43])
    assert np.all(grid[:1, :, 43:] == grid[:, :, 43:])
    # Pair 22 (first height pair) has frequency 1: angle == row index.
    np.testing.assert_allclose(np.arcsin(grid[:2, 0, 22, 1, 0]), [0.0, 1.0], atol=1e-6)


def test_product_rope_table_equals_oracle():
    # The host table builder shipped with the library computes the same numpy
    # float32 expression; both are pinned by the closed form above.
    for H, W, T in [(16, 16, 1), (96, 64, 1), (3, 5, 2)]:
        np.testing.assert_array_equal(generate_rope_freqs(H, W, T), oracle.rope_freqs(H, W, T))


def test_attention_dataflow_vs_fp64():
    rng = np.random.default_rng(9)
    B, S, H, D = 2, 16, 3, 128
    q, k, v = (rng.standard_normal((B, S, H, D)).astype(np.float32) for _ in range(3))
    f = oracle.rope_freqs(4, 4)
    out = oracle.attention_dataflow(q, k, v, freqs=f)
    qn = oracle.rmsnorm_fp64(q)
    kn = oracle.rmsnorm_fp64(k)
    f64 = oracle.rope_freqs_fp64(4, 4)[:, None]

    def rot(x):
        a, b = x[..., :64], x[..., 64:]
        return np.concatenate([f64[..., 0, 0] * a + f64[..., 0, 1] * b,
                               f64[..., 1, 0] * a + f64[..., 1, 1] * b], -1)

    qt = rot(qn).transpose(0, 2, 1, 3).reshape(B * H, S, D)
    kt = rot(kn).transpose(0, 2, 1, 3).reshape(B * H, S, D)
    vt = v.transpose(0, 2, 1, 3).reshape(B * H, S, D)
    ref = oracle.sdpa_fp64(qt, kt, vt).reshape(B, H, S, D).transpose(0, 2, 1, 3)
    assert np.abs(out - ref).max() < 5e-6


# ---------------------------------------------------- block-level pieces

def test_layernorm_and_silu_match_reference_vectors(gold):
    np.testing.assert_array_equal(oracle.layernorm(gold["ln_x"], 1e-6), gold["ln_out"])
    np.testing.assert_array_equal(oracle.silu(gold["silu_x"]), gold["silu_out"])


def test_layernorm_vs_fp64_two_pass():
    rng = np.random.default_rng(21)
    x = (rng.standard_normal((16, 2048)) * 3 + 1.5).astype(np.float32)
    xd = x.astype(np.float64)
    mu = xd.mean(-1, keepdims=True)
    ref = (xd - mu) / np.sqrt(((xd - mu) ** 2).mean(-1, keepdims=True) + 1e-6)
    assert np.abs(oracle.layernorm(x) - ref).max() < 2e-5
    # A constant row has zero variance: y = 0 exactly.
    np.testing.assert_array_equal(oracle.layernorm(np.full((1, 64), 3.25, np.float32)), 0.0)


def test_silu_vs_fp64():
    x = np.linspace(-40, 40, 4001, dtype=np.float32)
    ref = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.abs(oracle.silu(x) - ref).max() <= 4 * np.spacing(np.abs(ref).astype(np.float32)).max()


def test_modulate_and_gate_residual():
    rng = np.random.default_rng(22)
    xn = rng.standard_normal((2, 5, 64), dtype=np.float32)
    sc, sh, g = (rng.standard_normal((2, 64), dtype=np.float32) for _ in range(3))
    out = rng.standard_normal((2, 5, 64), dtype=np.float32)
    # Closed cases: zero scale/shift is the identity, zero gate keeps x.
    z = np.zeros((2, 64), np.float32)
    np.testing.assert_array_equal(oracle.modulate(xn, z, z), xn)
    np.testing.assert_array_equal(oracle.gate_residual(xn, z, out), xn)
    # Each operation rounds to float32 once: matches fp64 to a few ulps.
    m = oracle.modulate(xn, sc, sh)
    md = xn.astype(np.float64) * (1.0 + sc[:, None].astype(np.float64)) + sh[:, None]
    assert np.abs(m - md).max() <= 4 * np.spacing(np.abs(md).max().astype(np.float32))
    r = oracle.gate_residual(xn, g, out)
    rd = xn.astype(np.float64) + g[:, None].astype(np.float64) * out
    assert np.abs(r - rd).max() <= 4 * np.spacing(np.abs(rd).max().astype(np.float32))
    # And the float32 order is the numpy one: (x_n * (1 + scale)) + shift.
    np.testing.assert_array_equal(m, xn * (np.float32(1.0) + sc[:, None]) + sh[:, None])
    np.testing.assert_array_equal(r, xn + g[:, None] * out)


@pytest.mark.parametrize("cross", [False, True])
def test_attention_block_vs_fp64(cross):
    """The composed sub-block against the same dataflow in float64: LayerNorm,
    modulate, bf16-weight projections, per-head RMSNorm, RoPE (self only),
    softmax attention, output projection, gated residual."""
    rng = np.random.default_rng(23 + cross)
    B, S, Dm, H, D, Sk, C = 2, 16, 256, 2, 128, 24, 64
    x = rng.standard_normal((B, S, Dm), dtype=np.float32)
    mod = (rng.standard_normal((B, 3, Dm)) * 0.5).astype(np.float32)
    ctx = rng.standard_normal((1, Sk, C), dtype=np.float32) if cross else None
    kin = C if cross else Dm
    wq, wk, wv = (oracle.f32_to_bf16_bits(rng.standard_normal((H * D, n), dtype=np.float32)
                                          * 0.05) for n in (Dm, kin, kin))
    wo = oracle.f32_to_bf16_bits(rng.standard_normal((Dm, H * D), dtype=np.float32) * 0.05)
    qw, kw = (rng.uniform(0.5, 1.5, D).astype(np.float32) for _ in range(2))
    f = None if cross else generate_rope_freqs(4, 4)
    got = oracle.attention_block(x, mod, wq, wk, wv, wo, qw, kw, f, ctx, heads=H, head_dim=D)

    d64 = lambda a: np.asarray(a, np.float64)
    wf = lambda bits: d64(oracle.bf16_bits_to_f32(bits))
    xd = d64(x)
    mu = xd.mean(-1, keepdims=True)
    xn = (xd - mu) / np.sqrt(((xd - mu) ** 2).mean(-1, keepdims=True) + 1e-6)
    xm = xn * (1 + d64(mod[:, 1])[:, None]) + d64(mod[:, 0])[:, None]
    src = np.broadcast_to(d64(ctx), (B, Sk, C)) if cross else xm
    q = (xm @ wf(wq).T).reshape(B, S, H, D)
    k = (src @ wf(wk).T).reshape(B, -1, H, D)
    v = (src @ wf(wv).T).reshape(B, -1, H, D)
    q, k = oracle.rmsnorm_fp64(q, qw), oracle.rmsnorm_fp64(k, kw)
    if not cross:
        fd = d64(f).reshape(S, D // 2, 2, 2)
        rot = lambda t: np.concatenate(
            [fd[None, :, None, :, 0, 0] * t[..., :D // 2] + fd[None, :, None, :, 0, 1] * t[..., D // 2:],
             fd[None, :, None, :, 1, 0] * t[..., :D // 2] + fd[None, :, None, :, 1, 1] * t[..., D // 2:]],
            axis=-1)
        q, k = rot(q), rot(k)
    qt, kt, vt = (t.transpose(0, 2, 1, 3).reshape(B * H, -1, D) for t in (q, k, v))
    o = oracle.sdpa_fp64(qt, kt, vt).reshape(B, H, S, D).transpose(0, 2, 1, 3).reshape(B, S, H * D)
    ref = xd + d64(mod[:, 2])[:, None] * (o @ wf(wo).T)
    assert np.abs(got - ref).max() < 2e-5 * max(1.0, np.abs(ref).max())
