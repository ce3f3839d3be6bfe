"""Inputs and oracle outputs of the full-size configurations, computed once
per test session and shared by the GPU tests of every arithmetic mode.

Every (batch, head) slice of these problems is independent, so the oracle
runs anima_rt's flash attention (oracle.flash_sdpa, a restatement of
flash_attention.h:55-208) over all 32 slices on up to 16 host threads.

  config 3: self-attention, B=2, H=16, S=4096 (64x64 grid), q/k/v ~ N(0,1),
            RMSNorm (weight 1, eps 1e-6) + 3D RoPE, scale 1/sqrt(128).
  config 4: per block, that self-attention plus cross-attention of 4096
            query tokens over a cached [2, 512, 1024] context ~ N(0, 0.5)
            projected by bf16 weights ~ N(0, 0.02) (K = k_norm(ctx Wk^T),
            V = ctx Wv^T, no RoPE, no mask).
  config 5: self-attention at 6144 tokens (96x64 grid, rectangular RoPE)
            and cross-attention 6144 x 512 over a cached context.

block_ref restates one attention sub-layer of NumpyBlock.forward
(numpy_dit.py:236-247) with float64 projections, for the full-size block
tests.
"""
import functools
import os

import numpy as np

import oracle

H, D, S_KV, C = 16, 128, 512, 1024
THREADS = max(1, min(16, os.cpu_count() or 1))
ONES = np.ones(D, np.float32)


def randn(rng, *shape, sigma=1.0):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma)).astype(np.float32)


def threaded_sdpa(q, k, v):
    return oracle.flash_sdpa(q, k, v, threads=THREADS)


@functools.lru_cache(maxsize=None)
def self_case(S, grid, seed):
    """q, k, v [2, S, 16, 128] ~ N(0,1) and the RoPE table of `grid` built by
    the library's host code (anima_hip.rope, the product's table builder)."""
    from anima_hip.rope import generate_rope_freqs
    rng = np.random.default_rng(seed)
    q, k, v = (randn(rng, 2, S, H, D) for _ in range(3))
    return q, k, v, generate_rope_freqs(*grid)


@functools.lru_cache(maxsize=None)
def self_ref(S, grid, seed):
    """NumpyAttention's norm -> RoPE -> SDPA dataflow on self_case's inputs,
    with the oracle's own RoPE table, all slices."""
    q, k, v, _ = self_case(S, grid, seed)
    return oracle.attention_dataflow(q, k, v, ONES, ONES, oracle.rope_freqs(*grid),
                                     sdpa=threaded_sdpa)


@functools.lru_cache(maxsize=None)
def context_case(seed, Bc=2):
    """ctx [Bc, 512, 1024] ~ N(0, 0.5); Wk, Wv [2048, 1024] bf16 bits ~ N(0, 0.02)."""
    rng = np.random.default_rng(seed)
    ctx = randn(rng, Bc, S_KV, C, sigma=0.5)
    wk = oracle.f32_to_bf16_bits(randn(rng, H * D, C, sigma=0.02))
    wv = oracle.f32_to_bf16_bits(randn(rng, H * D, C, sigma=0.02))
    return ctx, wk, wv


@functools.lru_cache(maxsize=None)
def context_kv_ref(seed, Bc=2):
    """The context's K and V projections [Bc, 512, 16, 128] with anima_rt's
    bf16 GEMM (gemm_backend.cpp:117-131); k_norm is applied by the dataflow."""
    ctx, wk, wv = context_case(seed, Bc)
    k = np.stack([oracle.gemm_bf16(ctx[b], wk) for b in range(Bc)]).reshape(Bc, S_KV, H, D)
    v = np.stack([oracle.gemm_bf16(ctx[b], wv) for b in range(Bc)]).reshape(Bc, S_KV, H, D)
    return k, v


@functools.lru_cache(maxsize=None)
def cross_q(S, seed):
    return randn(np.random.default_rng(seed), 2, S, H, D)


@functools.lru_cache(maxsize=None)
def cross_ref(S, q_seed, ctx_seed):
    """Cross-attention of cross_q(S, q_seed) over context ctx_seed: q_norm and
    k_norm with weight 1, no RoPE (numpy_dit.py:277-291), all slices."""
    q = cross_q(S, q_seed)
    k, v = context_kv_ref(ctx_seed)
    return oracle.attention_dataflow(q, k, v, ONES, ONES, None, sdpa=threaded_sdpa)


def check_all_slices(out, ref, mode, what, f32_tol=1e-4, bf16_rel=2e-2):
    """Every (batch, head) slice within the mode's tolerance: max-abs 1e-4 in
    the f32 and f32x3 modes, normwise max|out-ref| <= 2e-2 max|ref| per slice
    in the bf16 mode.  Returns the worst slice's error."""
    from anima_hip import rt
    assert out.shape == ref.shape
    assert np.isfinite(out).all(), what
    worst = 0.0
    for b in range(out.shape[0]):
        for h in range(out.shape[2]):
            o, r = out[b, :, h], ref[b, :, h]
            err = float(np.abs(o - r).max())
            if mode == rt.BF16:
                err /= float(np.abs(r).max())
            worst = max(worst, err)
            assert err <= (bf16_rel if mode == rt.BF16 else f32_tol), (what, b, h, err)
    print(f"{what} mode={mode}: worst slice {'normwise' if mode == rt.BF16 else 'max_abs'} "
          f"{worst:.3e} over {out.shape[0] * out.shape[2]} slices", flush=True)
    return worst


def proj_f64(a, w_bits):
    """a[M, K] . W[N, K]^T as a float64 product of the f32 activations and
    the bf16-decoded weights, rounded to f32: the exact mathematics of
    anima_rt's bf16 GEMM (gemm_backend.cpp:117-131) without its float32
    accumulation rounding, fast enough for M = 8192 on the host."""
    w = oracle.bf16_bits_to_f32(w_bits).astype(np.float64)
    return (np.asarray(a, np.float64) @ w.T).astype(np.float32)


def block_ref(x, mod, wq, wk, wv, wo, qw, kw, freqs, ctx, heads=H, head_dim=D):
    """One attention sub-layer of NumpyBlock.forward (numpy_dit.py:236-247,
    NumpyAttention.forward 268-297) on the host:
    x + gate * output_proj(attention(LayerNorm(x) * (1 + scale) + shift)).
    LayerNorm, modulate, q/k RMSNorm, RoPE and flash attention (all slices,
    THREADS host threads) through the oracle; the projections through
    proj_f64.  Self-attention when ctx is None (K/V from the modulated x,
    RoPE with freqs), else K/V projected from ctx [Bc, S_kv, C], no RoPE."""
    B, S, Dm = x.shape
    shift, scale, gate = (np.ascontiguousarray(mod[:, i]) for i in range(3))
    xm = oracle.modulate(oracle.layernorm(x, 1e-6), scale, shift).reshape(B * S, Dm)
    q = proj_f64(xm, wq).reshape(B, S, heads, head_dim)
    src = xm.reshape(B, S, Dm) if ctx is None else np.asarray(ctx, np.float32)
    k = np.stack([proj_f64(s, wk) for s in src]).reshape(len(src), -1, heads, head_dim)
    v = np.stack([proj_f64(s, wv) for s in src]).reshape(len(src), -1, heads, head_dim)
    if len(src) != B:
        k = np.broadcast_to(k, (B,) + k.shape[1:])
        v = np.broadcast_to(v, (B,) + v.shape[1:])
    attn = oracle.attention_dataflow(q, k, v, qw, kw, freqs if ctx is None else None, 1e-6,
                                     sdpa=threaded_sdpa)
    out = proj_f64(attn.reshape(B * S, heads * head_dim), wo).reshape(B, S, Dm)
    return oracle.gate_residual(x, gate, out)
