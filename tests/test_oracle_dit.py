"""Pins the oracle's DiT pieces around the attention path (no GPU needed).

The composition (patch order, padding-mask channel, timestep features, AdaLN
chunk order and LoRA term, MLP, final layer, unpatchify, Euler/CFG sampler)
is checked bit for bit against tests/golden/dit_ref_vectors.npz, which the
reference's own numpy_dit.py / sampling.py wrote (make_dit_golden.py); GELU
against the reference runtime's vectors; the pieces also against fp64 closed
forms and permutation identities.
"""
import math
import os

import numpy as np
import pytest

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "anima_rt_ref_vectors.npz")
DIT_GOLDEN = os.path.join(HERE, "golden", "dit_ref_vectors.npz")


@pytest.fixture(scope="module")
def dit_gold():
    g = np.load(DIT_GOLDEN)
    import sys
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import dit_weights
    cfg = {k[4:]: int(g[k]) for k in g.files if k.startswith("cfg_")}
    return g, cfg, dit_weights.make(int(g["weight_seed"]), **cfg)


def test_gelu_matches_reference_vectors():
    gold = np.load(GOLDEN)
    np.testing.assert_array_equal(oracle.gelu(gold["gelu_x"]), gold["gelu_out"])


def test_softmax_matches_reference_vectors_and_fp64():
    gold = np.load(GOLDEN)
    x = gold["softmax_x"]
    y = oracle.softmax(x)
    np.testing.assert_array_equal(y, gold["softmax_out"])
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    np.testing.assert_allclose(y, e / e.sum(axis=1, keepdims=True), rtol=2e-6, atol=1e-9)
    np.testing.assert_allclose(y.sum(axis=1), 1.0, rtol=2e-6)
    np.testing.assert_allclose(y[3], 1.0 / 77, rtol=1e-6)  # constant row


def test_gelu_vs_fp64_and_identities():
    x = np.linspace(-8, 8, 4001).astype(np.float32)
    ref = np.array([v * 0.5 * (1 + math.erf(v / math.sqrt(2))) for v in x.astype(np.float64)])
    g = oracle.gelu(x)
    assert np.abs(g - ref).max() <= 4 * np.spacing(np.float32(8))
    assert g[2000] == 0.0  # GELU(0)
    # GELU(x) - GELU(-x) = x (Phi(x) + Phi(-x) = 1)
    np.testing.assert_allclose(g - g[::-1], x, atol=2e-6)


def test_timesteps_closed_form():
    sig = np.array([0.0, 0.3, 1.0], np.float32)
    t = oracle.timesteps(sig, 64)
    half = 32
    f = np.exp(-math.log(10000) * np.arange(half) / half)
    ref = np.concatenate([np.cos(sig[:, None].astype(np.float64) * f),
                          np.sin(sig[:, None].astype(np.float64) * f)], axis=1)
    assert t.shape == (3, 64) and t.dtype == np.float32
    np.testing.assert_allclose(t, ref, atol=1e-6)
    np.testing.assert_array_equal(t[0, :half], 1.0)  # sigma 0: cos 1, sin 0
    np.testing.assert_array_equal(t[0, half:], 0.0)


def test_patchify_unpatchify_round_trip_and_order():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 3, 1, 5, 6)).astype(np.float32)
    tok = oracle.patchify(x)
    assert tok.shape == (2, 1, 3, 3, 16)
    # feature (c*2 + dy)*2 + dx of token (h, w) is x[c, 2h+dy, 2w+dx]; c = 3 is
    # the zero padding-mask channel; row 5 (padding) is zero.
    b, h, w, c, dy, dx = 1, 1, 2, 2, 1, 0
    assert tok[b, 0, h, w, (c * 2 + dy) * 2 + dx] == x[b, c, 0, 2 * h + dy, 2 * w + dx]
    assert np.all(tok[..., 12:] == 0.0)
    assert np.all(tok[:, :, 2, :, [2, 3, 6, 7, 10, 11]] == 0.0)
    # The final layer's feature layout (dy*2 + dx)*C + c inverts onto the
    # latent grid: build those features from x and get x back, cropped.
    C = 3
    f = np.zeros((2, 1, 3, 3, 4 * C), np.float32)
    for dy in range(2):
        for dx in range(2):
            for c in range(C):
                xp = np.zeros((2, 6, 6), np.float32)
                xp[:, :5, :6] = x[:, c, 0]
                f[:, 0, :, :, (dy * 2 + dx) * C + c] = xp[:, dy::2, dx::2]
    np.testing.assert_array_equal(oracle.unpatchify(f, C, 5, 6), x)


def test_sigmas_match_reference_scheduler(dit_gold):
    g, _, _ = dit_gold
    np.testing.assert_array_equal(oracle.z_image_sigmas(2), g["smp_sigmas"])
    s = oracle.z_image_sigmas(8)
    assert s[0] == 1.0 and s[-1] == 0.0 and np.all(np.diff(s) < 0)


def test_dit_forward_matches_reference_code_bitwise(dit_gold):
    g, cfg, w = dit_gold
    out = oracle.dit_forward(g["fwd_x"], g["fwd_sigma"], g["fwd_ctx"], w, cfg["blocks"],
                             cfg["heads"], cfg["head_dim"])
    assert out.shape == g["fwd_out"].shape == (2, 16, 1, 7, 10)
    np.testing.assert_array_equal(out, g["fwd_out"])


def test_euler_sampler_matches_reference_code_bitwise(dit_gold):
    g, cfg, w = dit_gold

    def fwd(x, s, c):
        return oracle.dit_forward(x, s, c, w, cfg["blocks"], cfg["heads"], cfg["head_dim"])

    out = oracle.euler_sample(fwd, g["smp_noise"], g["smp_sigmas"], g["smp_ctx_cond"],
                              g["smp_ctx_uncond"], float(g["smp_cfg"]))
    np.testing.assert_array_equal(out, g["smp_out"])


def test_dit_forward_sensitivity(dit_gold):
    """A plausible mistake shows: swapping the two batch entries' sigmas or
    dropping the AdaLN-LoRA term changes the output beyond rounding."""
    g, cfg, w = dit_gold
    base = g["fwd_out"]
    out = oracle.dit_forward(g["fwd_x"], g["fwd_sigma"][::-1].copy(), g["fwd_ctx"], w,
                             cfg["blocks"], cfg["heads"], cfg["head_dim"])
    assert np.abs(out - base).max() > 1e-3
    w2 = dict(w)
    w2["t_embedder.1.linear_2.weight"] = np.zeros_like(w["t_embedder.1.linear_2.weight"])
    out = oracle.dit_forward(g["fwd_x"], g["fwd_sigma"], g["fwd_ctx"], w2, cfg["blocks"],
                             cfg["heads"], cfg["head_dim"])
    assert np.abs(out - base).max() > 1e-3


def test_product_weight_names_match_reference_layout():
    """The model's tensor table (anima_hip.dit.weight_shapes) is the one the
    reference's code consumed when it wrote the fixture (dit_weights.shapes,
    every matrix shape asserted by the GEMM engine of make_dit_golden.py)."""
    import sys
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import dit_weights
    from anima_hip.dit import DiTConfig, weight_shapes
    for blocks, heads, hidden, ctx in ((2, 2, 512, 64), (28, 16, 8192, 1024)):
        cfg = DiTConfig.anima_2b(blocks=blocks, heads=heads, mlp_hidden=hidden, ctx_dim=ctx)
        assert weight_shapes(cfg) == dit_weights.shapes(2048, blocks, heads, 128, hidden, ctx)


@pytest.mark.parametrize("grid", [(16, 16), (64, 64), (96, 64)])
def test_rope_tables_match_reference_builder_bitwise(grid):
    # Tables written by the reference's own _generate_rope_freqs
    # (numpy_dit.py:48-60; tests/golden/make_rope_golden.py): the library's
    # host builder (anima_hip/rope.py) and the oracle's reproduce them bit for
    # bit at the grids of configs 1, 3 and 5, the 96x64 one rectangular.
    import hashlib

    from anima_hip.rope import generate_rope_freqs
    g = np.load(os.path.join(HERE, "golden", "rope_ref_tables.npz"))
    H, W = grid
    key = f"{H}x{W}"
    for table in (generate_rope_freqs(H, W), oracle.rope_freqs(H, W)):
        assert table.dtype == np.float32 and table.shape == (H * W, 64, 2, 2)
        t5 = table.reshape(H, W, 64, 2, 2)
        np.testing.assert_array_equal(t5[:, 0], g[f"col0_{key}"])
        np.testing.assert_array_equal(t5[0, :], g[f"row0_{key}"])
        if f"table_{key}" in g.files:
            np.testing.assert_array_equal(table, g[f"table_{key}"])
        digest = hashlib.sha256(np.ascontiguousarray(table).tobytes()).hexdigest()
        assert digest == str(g[f"sha256_{key}"])


@pytest.mark.parametrize("cross", [False, True])
def test_float64_block_checker_matches_oracle_composition(cross):
    """fullsize.block_ref (float64 projections, used by the full-size block
    tests where the scalar bf16 GEMM would take minutes) against the oracle's
    own composition of the sub-layer (oracle.attention_block, anima_rt's
    float32-accumulating bf16 GEMM) at 64 tokens: the two differ only by the
    projections' accumulation rounding."""
    import fullsize
    rng = np.random.default_rng(4403 + cross)
    B, S, Dm, H, D = 2, 64, 2048, 16, 128
    x = rng.standard_normal((B, S, Dm), dtype=np.float32)
    mod = (rng.standard_normal((B, 3, Dm)) * 0.5).astype(np.float32)

    def w(n, k):
        return oracle.f32_to_bf16_bits(rng.standard_normal((n, k), dtype=np.float32) * 0.02)

    wq, wo = w(H * D, Dm), w(Dm, H * D)
    qw, kw = (rng.uniform(0.5, 1.5, D).astype(np.float32) for _ in range(2))
    if cross:
        ctx = (rng.standard_normal((1, 96, 1024)) * 0.5).astype(np.float32)
        wk, wv, f = w(H * D, 1024), w(H * D, 1024), None
    else:
        ctx, wk, wv, f = None, w(H * D, Dm), w(H * D, Dm), oracle.rope_freqs(8, 8)
    ours = fullsize.block_ref(x, mod, wq, wk, wv, wo, qw, kw, f, ctx)
    theirs = oracle.attention_block(x, mod, wq, wk, wv, wo, qw, kw, f, ctx, heads=H, head_dim=D)
    d_ours, d_theirs = ours - x, theirs - x
    err = np.abs(d_ours - d_theirs).max() / np.abs(d_theirs).max()
    assert err <= 1e-5, err
    # A dropped term is far outside that: the gate alone moves the update by its own size.
    assert np.abs(d_theirs).max() > 0.05
