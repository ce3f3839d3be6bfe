"""The attention sub-block of a DiT block on the resident residual stream
(anima_hip_attention_block_dev) against the oracle's composition of
NumpyBlock.forward's pieces: LayerNorm, AdaLN modulate, bf16-weight
projections, q/k RMSNorm, RoPE (self), SDPA, output projection, gated
residual.

The residual x itself passes through unchanged, so the checks compare the
update x_out - x_in with the oracle's: max-abs 1e-4 of its scale in the f32
and f32x3 modes, normwise relative 2e-2 in bf16 mode.
"""
import ctypes as ct

import numpy as np
import pytest

import oracle
from anima_hip import _lib, rt
from anima_hip.rope import generate_rope_freqs

pytestmark = pytest.mark.gpu

S, DM, H, D = 256, 2048, 16, 128


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


def _weights(rng, n_out, n_in):
    return oracle.f32_to_bf16_bits(rng.standard_normal((n_out, n_in), dtype=np.float32) * 0.02)


def _inputs(seed, B, S=S):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, S, DM), dtype=np.float32)
    mod = (rng.standard_normal((B, 3, DM)) * 0.5).astype(np.float32)
    w = [_weights(rng, H * D, DM) for _ in range(3)] + [_weights(rng, DM, H * D)]
    qw, kw = (rng.uniform(0.5, 1.5, D).astype(np.float32) for _ in range(2))
    return rng, x, mod, w, qw, kw


def _run_block(x, mod, w, qw, kw, freqs, kv, mode):
    from devmem import DevBuf
    lib = _lib.load()
    B, S = x.shape[:2]
    bufs = {name: DevBuf.of(a) for name, a in
            (("x", x), ("mod", mod), ("wq", w[0]), ("wk", w[1]), ("wv", w[2]), ("wo", w[3]),
             ("qw", qw), ("kw", kw))}
    fr = DevBuf.of(freqs) if freqs is not None else None
    handle = kv.handle if kv is not None else None
    n = lib.anima_hip_attention_block_scratch_bytes(handle, B, S, DM, H, D, mode)
    scratch = DevBuf(n)
    ok = lib.anima_hip_attention_block_dev(
        bufs["x"].addr, bufs["mod"].addr, bufs["wq"].addr, bufs["wk"].addr, bufs["wv"].addr,
        bufs["wo"].addr, bufs["qw"].addr, bufs["kw"].addr, fr.addr if fr else None, handle,
        B, S, DM, H, D, ct.c_float(1e-6), mode, scratch.addr, n, None)
    _lib.check(ok, "attention_block_dev")
    return bufs["x"].get(x.shape)


def _check(out, ref, x, mode):
    d_out, d_ref = out - x, ref - x
    scale = np.abs(d_ref).max()
    err = np.abs(d_out - d_ref).max() / scale
    print(f"  mode {mode}: update scale {scale:.3e}, rel err {err:.3e}", flush=True)
    assert np.isfinite(out).all()
    assert err <= (2e-2 if mode == rt.BF16 else 1e-4)


# B=2: the gate and the residual rows differ per batch entry.
@pytest.mark.parametrize("B", [1, 2])
@pytest.mark.parametrize("mode", [rt.F32, rt.BF16, rt.F32X3])
def test_self_attention_block(mode, B):
    rng, x, mod, w, qw, kw = _inputs(606 + mode + 10 * B, B)
    f = generate_rope_freqs(16, 16)
    print(f"self-attention block mode={mode} B={B}", flush=True)
    out = _run_block(x, mod, w, qw, kw, f, None, mode)
    ref = oracle.attention_block(x, mod, *w, qw, kw, f, None, heads=H, head_dim=D,
                                 sdpa=lambda a, b, c: oracle.flash_sdpa(a, b, c, threads=8))
    _check(out, ref, x, mode)


@pytest.mark.parametrize("B", [1, 2])
@pytest.mark.parametrize("mode", [rt.F32, rt.BF16, rt.F32X3])
def test_cross_attention_block(mode, B):
    rng, x, mod, w, qw, kw = _inputs(707 + mode + 10 * B, B)
    ctx = (rng.standard_normal((B, 512, 1024)) * 0.5).astype(np.float32)
    wk, wv = _weights(rng, H * D, 1024), _weights(rng, H * D, 1024)
    print(f"cross-attention block mode={mode} B={B}", flush=True)
    kv = rt.ContextKV(ctx, wk, wv, kw, heads=H, head_dim=D, mode=mode)
    try:
        out = _run_block(x, mod, [w[0], wk, wv, w[3]], qw, kw, None, kv, mode)
        # Twice in a row on the same inputs: identical (the cache is reused).
        np.testing.assert_array_equal(_run_block(x, mod, [w[0], wk, wv, w[3]], qw, kw, None, kv,
                                                 mode), out)
    finally:
        kv.close()
    ref = oracle.attention_block(x, mod, w[0], wk, wv, w[3], qw, kw, None, ctx, heads=H,
                                 head_dim=D,
                                 sdpa=lambda a, b, c: oracle.flash_sdpa(a, b, c, threads=8))
    _check(out, ref, x, mode)


def test_block_argument_errors():
    lib = _lib.load()
    z = np.zeros(16, np.float32)
    ok = lib.anima_hip_attention_block_dev(z.ctypes.data, None, None, None, None, None, None, None,
                                           None, None, 1, 4, 64, 1, 64, ct.c_float(1e-6), 0, None,
                                           0, None)
    assert not ok and "null" in _lib.last_error()
    ok = lib.anima_hip_attention_block_dev(None, None, None, None, None, None, None, None, None,
                                           None, 1, 4, 64, 1, 64, ct.c_float(1e-6), 9, None, 0,
                                           None)
    assert not ok and "mode" in _lib.last_error()
    # Widths that are not multiples of 8 are refused with a reason.
    assert lib.anima_hip_attention_block_scratch_bytes(None, 1, 4, 60, 1, 64, 0) > 0
