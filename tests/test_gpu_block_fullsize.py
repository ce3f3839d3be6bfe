"""Config 4's attention sub-layers at full size: one DiT block at 1024x1024
output (B=2 CFG pair, S=4096 latent tokens on the 64x64 grid, d_model 2048,
16 heads x 128), hidden states ~ N(0,1) through seeded bf16 projection
weights ~ N(0,0.02), as NumpyBlock.forward runs them
(anima_rt/scripts/numpy_dit.py:230-253, NumpyAttention.forward 268-297):

  self:  x += gate * output_proj(SDPA(RoPE(q_norm(x_m Wq^T)),
                                      RoPE(k_norm(x_m Wk^T)), x_m Wv^T))
  cross: x += gate * output_proj(SDPA(q_norm(x_m Wq^T), k_norm(ctx Wk^T),
                                      ctx Wv^T))
  x_m = LayerNorm(x) * (1 + scale) + shift

with the cross-attention's context K/V cached once ([2, 512, 1024] context
~ N(0, 0.5)), through anima_hip_attention_block_dev in every arithmetic
mode.  This is the composition the 28-block step of the bench times: the
M = 8192 projection products, the LayerNorm/modulate term writer, the
one-launch Q/K/V prologue, the flash kernels on 8-wave grids (for the
cross sub-layer in the f32 and f32x3 modes: query rows normalised inside
the kernel) and the attention's output written as the output projection's
bf16 terms.

The checker (fullsize.block_ref) runs on the host: LayerNorm and modulate
through the oracle, every projection as a float64 product of the f32
activations and the bf16-decoded weights (the exact mathematics of
anima_rt's bf16 GEMM, gemm_backend.cpp:117-131, without its float32
accumulation rounding), q/k RMSNorm and RoPE through the oracle, and
attention on all 32 (batch, head) slices through the oracle's flash
attention (flash_attention.h:55-208) on host threads.
test_oracle_dit.py checks that checker against the oracle's own
composition (oracle.attention_block) at a small size.  The residual x
passes through unchanged, so the update x_out - x is compared: max-abs 1e-4
of its scale in the f32 and f32x3 modes, 2e-2 in bf16 mode.
"""
import functools

import pytest

import fullsize
import oracle
from anima_hip import rt
from anima_hip.rope import generate_rope_freqs
from test_gpu_block import D, H, _check, _inputs, _run_block, _weights

pytestmark = pytest.mark.gpu

B, S, GRID, S_CTX, C = 2, 4096, (64, 64), 512, 1024


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


@functools.lru_cache(maxsize=None)
def _self_case():
    _, x, mod, w, qw, kw = _inputs(4401, B, S)
    ref = fullsize.block_ref(x, mod, *w, qw, kw, oracle.rope_freqs(*GRID), None)
    return x, mod, w, qw, kw, ref


@functools.lru_cache(maxsize=None)
def _cross_case():
    rng, x, mod, w, qw, kw = _inputs(4402, B, S)
    ctx = fullsize.randn(rng, B, S_CTX, C, sigma=0.5)
    wk, wv = _weights(rng, H * D, C), _weights(rng, H * D, C)
    ws = [w[0], wk, wv, w[3]]
    ref = fullsize.block_ref(x, mod, *ws, qw, kw, None, ctx)
    return x, mod, ws, qw, kw, ctx, ref


@pytest.mark.parametrize("mode", [rt.F32, rt.F32X3, rt.BF16])
def test_self_attention_block_4096(mode):
    x, mod, w, qw, kw, ref = _self_case()
    print(f"self-attention block B={B} S={S} mode={mode}", flush=True)
    out = _run_block(x, mod, w, qw, kw, generate_rope_freqs(*GRID), None, mode)
    _check(out, ref, x, mode)


@pytest.mark.parametrize("mode", [rt.F32, rt.F32X3, rt.BF16])
def test_cross_attention_block_4096(mode):
    x, mod, ws, qw, kw, ctx, ref = _cross_case()
    print(f"cross-attention block B={B} S={S} x {S_CTX} mode={mode}", flush=True)
    kv = rt.ContextKV(ctx, ws[1], ws[2], kw, heads=H, head_dim=D, mode=mode)
    try:
        out = _run_block(x, mod, ws, qw, kw, None, kv, mode)
    finally:
        kv.close()
    _check(out, ref, x, mode)
