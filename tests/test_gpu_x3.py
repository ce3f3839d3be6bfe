"""Parity of the f32x3 attention path (f32 operands as bf16 term pairs on bf16
MFMA) with the oracle.

The path is held to the f32 path's stated tolerance, max-abs 1e-4 against
anima_rt's f32 flash attention (the oracle, bit-identical to the reference)
on identical seeded inputs.  Its error model: every operand x enters as
xh + xl with |x - xh - xl| <= 2^-17 |x| and every product drops xl*yl, so
scores and outputs carry ~1e-5 of their scale; the tighter relative bound
REL_X3 (normwise, max|out - ref| / max|ref|) checks that model, and the
error is also reported against fp64 brute force.
"""
import ctypes as ct
import math
import os

import numpy as np
import pytest

import oracle
from anima_hip import AnimaHipError, _lib, rt
from anima_hip.rope import generate_rope_freqs
from devmem import DevBuf

pytestmark = pytest.mark.gpu

TOL = 1e-4      # the f32 path's max-abs tolerance
REL_X3 = 5e-5   # normwise, the term-split error model
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "anima_rt_ref_vectors.npz")


def randn(rng, *shape):
    return rng.standard_normal(shape, dtype=np.float32)


def check(out, ref, what):
    err = float(np.abs(out - ref).max())
    rel = err / float(np.abs(ref).max())
    print(f"x3 {what}: max-abs {err:.3e} rel {rel:.3e}", flush=True)
    assert err <= TOL and rel <= REL_X3


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


@pytest.mark.parametrize("name", ["flash_small", "flash_tiles"])
def test_x3_golden(name):
    g = np.load(GOLDEN)
    q, k, v = g[f"{name}_q"], g[f"{name}_k"], g[f"{name}_v"]
    out = rt.sdpa(q, k, v, 1.0 / math.sqrt(128), False, mode=rt.F32X3)
    check(out, g[f"{name}_out"], name)


@pytest.mark.parametrize("sq,sk,causal", [(1, 1, False), (77, 77, False), (129, 513, False),
                                          (1000, 511, False), (256, 4097, False),
                                          (300, 300, True), (520, 100, True)])
def test_x3_shapes(sq, sk, causal):
    """Tails (keys not a multiple of the 64-key tile), split-KV plans (few
    rows, many keys), causal masking."""
    rng = np.random.default_rng(sq * 17 + sk)
    q, k, v = randn(rng, 3, sq, 128), randn(rng, 3, sk, 128), randn(rng, 3, sk, 128)
    print(f"x3 case sq={sq} sk={sk} causal={causal}", flush=True)
    out = rt.sdpa(q, k, v, is_causal=causal, mode=rt.F32X3)
    check(out, oracle.flash_sdpa(q, k, v, is_causal=causal, threads=3), f"{sq}x{sk}")


def test_x3_rejects_other_head_dims():
    rng = np.random.default_rng(0)
    q = randn(rng, 1, 8, 64)
    with pytest.raises(AnimaHipError, match="D == 128"):
        rt.sdpa(q, q, q, mode=rt.F32X3)


def test_x3_self_attention_256_against_reference_and_fp64():
    """B=1, H=16, S=256, N(0,1) q/k/v after RMSNorm(w=1) + RoPE (16x16 grid)."""
    rng = np.random.default_rng(1001)
    B, S, H, D = 1, 256, 16, 128
    q, k, v = randn(rng, B, S, H, D), randn(rng, B, S, H, D), randn(rng, B, S, H, D)
    f = generate_rope_freqs(16, 16)
    ones = np.ones(D, np.float32)
    qn = oracle.numpy_rope(oracle.rmsnorm(q, ones), f).transpose(0, 2, 1, 3).reshape(H, S, D)
    kn = oracle.numpy_rope(oracle.rmsnorm(k, ones), f).transpose(0, 2, 1, 3).reshape(H, S, D)
    vt = v.transpose(0, 2, 1, 3).reshape(H, S, D)
    out = rt.sdpa(qn, kn, vt, mode=rt.F32X3)
    check(out, oracle.flash_sdpa(qn, kn, vt), "256 tokens vs reference")
    check(out, oracle.sdpa_fp64(qn, kn, vt), "256 tokens vs fp64")


def test_x3_error_scales_with_v():
    """The term split is relative: V scaled by 2^10 gives the same relative
    error (the absolute 1e-4 bound is for N(0,1)-scale data)."""
    rng = np.random.default_rng(77)
    q, k, v = randn(rng, 2, 300, 128), randn(rng, 2, 300, 128), randn(rng, 2, 300, 128)
    a = rt.sdpa(q, k, v, mode=rt.F32X3)
    b = rt.sdpa(q, k, v * np.float32(1024.0), mode=rt.F32X3)
    # Power-of-two scaling commutes with every bf16/f32 rounding.
    np.testing.assert_array_equal(b, a * np.float32(1024.0))


def test_x3_device_entries_match_host_path():
    """anima_hip_qk_prologue_dev (flags 4: term rows) + anima_hip_pack_vt_terms_dev
    + anima_hip_flash_x3_dev on device buffers: the term rows hold hi = bf16(x),
    lo = bf16(x - hi) exactly, and the output meets the tolerance (the
    host-pointer path splits the key range of this small problem over
    workgroups, the device entry without scratch does not, so the two differ
    in summation order only)."""
    lib = _lib.load()
    rng = np.random.default_rng(91)
    B, H, S, D = 2, 3, 200, 128
    q, k, v = randn(rng, B, H, S, D), randn(rng, B, H, S, D), randn(rng, B, H, S, D)
    dq, dk, dv = DevBuf.of(q), DevBuf.of(k), DevBuf.of(v)
    tq, tk = DevBuf(q.size * 4), DevBuf(k.size * 4)
    sp = lib.anima_hip_vt_padded_len(S)
    tv = DevBuf(B * H * 2 * D * sp * 2)
    o = DevBuf(q.size * 4)
    terms = _lib.strides([H * S * 2 * D, S * 2 * D, 2 * D])
    for x, t in ((dq, tq), (dk, tk)):
        ok = lib.anima_hip_qk_prologue_dev(x.addr, t.addr, None, None, B, S, H, D, None, terms,
                                           ct.c_float(0.0), 4, None)
        _lib.check(ok, "qk_prologue terms")
    _lib.check(lib.anima_hip_pack_vt_terms_dev(dv.addr, tv.addr, B, H, S, D, None, None, None),
               "pack_vt_terms")
    _lib.check(lib.anima_hip_flash_x3_dev(tq.addr, tk.addr, tv.addr, o.addr, B, H, S, S, D,
                                          None, None, None, None, ct.c_float(1 / math.sqrt(D)),
                                          False, None), "flash_x3_dev")
    out = o.get(q.shape)
    host = rt.sdpa(q.reshape(B * H, S, D), k.reshape(B * H, S, D), v.reshape(B * H, S, D),
                   mode=rt.F32X3).reshape(q.shape)
    check(out, oracle.flash_sdpa(q.reshape(B * H, S, D), k.reshape(B * H, S, D),
                                 v.reshape(B * H, S, D), threads=3).reshape(q.shape), "device entries")
    np.testing.assert_allclose(out, host, rtol=0, atol=2e-5)
    rows = tq.get((B, H, S, 2 * D), np.uint16)
    hi = oracle.f32_to_bf16_bits(q)
    np.testing.assert_array_equal(rows[..., :D], hi)
    rest = q - (hi.astype(np.uint32) << 16).view(np.float32)
    np.testing.assert_array_equal(rows[..., D:], oracle.f32_to_bf16_bits(rest))
    vt = tv.get((B, H, 2 * D, sp), np.uint16)
    vhi = oracle.f32_to_bf16_bits(v)
    vlo = oracle.f32_to_bf16_bits(v - (vhi.astype(np.uint32) << 16).view(np.float32))
    pos = np.array([(c & ~12) | ((c & 4) << 1) | ((c & 8) >> 1) for c in range(16)])
    perm = (np.arange(sp) // 16) * 16 + pos[np.arange(sp) % 16]  # key -> position
    full_hi = np.zeros((B, H, D, sp), np.uint16)
    full_lo = np.zeros_like(full_hi)
    full_hi[..., perm[:S]] = vhi.transpose(0, 1, 3, 2)
    full_lo[..., perm[:S]] = vlo.transpose(0, 1, 3, 2)
    np.testing.assert_array_equal(vt[:, :, :D], full_hi)
    np.testing.assert_array_equal(vt[:, :, D:], full_lo)


def test_x3_device_entry_rejects_dense_row_strides():
    """Term rows hold 2*D values; strides of dense D-value rows are refused
    before any launch (the lo half would be read past the tensor's end)."""
    lib = _lib.load()
    B, H, S, D = 1, 2, 64, 128
    buf = DevBuf(B * H * S * 2 * D * 2)
    o = DevBuf(B * H * S * D * 4)
    sp = lib.anima_hip_vt_padded_len(S)
    vt = DevBuf(B * H * 2 * D * sp * 2)
    dense = _lib.strides([H * S * D, S * D, D])
    ok = lib.anima_hip_flash_x3_dev(buf.addr, buf.addr, vt.addr, o.addr, B, H, S, S, D, dense,
                                    None, None, None, ct.c_float(0.1), False, None)
    assert not ok and "256 elements per row" in _lib.last_error()
    terms = _lib.strides([H * S * 2 * D, S * 2 * D, 2 * D])
    bf16_vt = _lib.strides([H * D * sp, D * sp, sp])  # the bf16 layout: D rows per head
    ok = lib.anima_hip_flash_x3_dev(buf.addr, buf.addr, vt.addr, o.addr, B, H, S, S, D, terms,
                                    terms, bf16_vt, None, ct.c_float(0.1), False, None)
    assert not ok and "2*D rows" in _lib.last_error()


def test_x3_deterministic():
    rng = np.random.default_rng(5)
    q, k, v = randn(rng, 2, 700, 128), randn(rng, 2, 900, 128), randn(rng, 2, 900, 128)
    a = rt.sdpa(q, k, v, mode=rt.F32X3)
    np.testing.assert_array_equal(a, rt.sdpa(q, k, v, mode=rt.F32X3))


def test_x3_attention_core_256_and_4096_tokens_all_heads():
    """The fused attention core (anima_hip_attention: RMSNorm + RoPE prologue
    writing term rows, term V^T pack, f32x3 flash) at 256 tokens and at the
    4096-token, B=2, H=16 workload; every (batch, head) slice of the latter
    against the oracle."""
    ones = np.ones(128, np.float32)
    rng = np.random.default_rng(1001)
    q, k, v = randn(rng, 1, 256, 16, 128), randn(rng, 1, 256, 16, 128), randn(rng, 1, 256, 16, 128)
    f = generate_rope_freqs(16, 16)
    out = rt.attention(q, k, v, ones, ones, f, mode=rt.F32X3)
    check(out, oracle.attention_dataflow(q, k, v, ones, ones, f), "attention 256 tokens")

    import fullsize
    q, k, v, f = fullsize.self_case(4096, (64, 64), 3003)
    out = rt.attention(q, k, v, ones, ones, f, mode=rt.F32X3)
    fullsize.check_all_slices(out, fullsize.self_ref(4096, (64, 64), 3003), rt.F32X3,
                              "f32x3 attention core 4096 tokens")
