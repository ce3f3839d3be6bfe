"""The flash kernels given raw query rows against the two-pass form they
replace, bit for bit:

- f32x3, anima_hip_flash_x3_rawq_dev (RMSNorm, RoPE and the hi/lo term split
  of q inside the kernel) against anima_hip_qk_prologue_dev (flags 1 | 4) +
  anima_hip_flash_x3_dev: dense and fused-projection layouts, with and
  without norm weights and RoPE, ragged query and key tiles, causal masking,
  cross-attention shapes, the 4-wave grid of small problems, NaN / infinity;
- f32, anima_hip_flash_f32_rawq_dev (RMSNorm inside the kernel) against
  anima_hip_qk_prologue_dev (flags 1) + anima_hip_flash_f32_dev, with NaN and
  infinity rows.

The prologue is itself pinned bit for bit to the reference's RMSNorm and RoPE
(tests/test_gpu_flash.py), and the composed attention to the oracle
(tests/test_gpu_x3.py, test_gpu_flash.py), so equality here carries both.  The
cross-attention entries take these kernels on unsplit 8-wave grids;
tests/test_gpu_cross.py holds them to the oracle at configs 2, 4 and 5."""
import ctypes as ct
import math

import numpy as np
import pytest

from anima_hip import _lib, rt
from anima_hip.rope import generate_rope_freqs
from devmem import DevBuf

pytestmark = pytest.mark.gpu
D = 128


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


def _ptr(b):
    return b.addr if b is not None else None


def _bits(x):
    return np.ascontiguousarray(x).view(np.uint32)


CASES = [  # B, S_q, S_kv, H, grid (None: no RoPE), fused projection layout, weights, causal
    (2, 4096, 4096, 16, (64, 64), False, True, False),
    (2, 77, 77, 3, (7, 11), True, True, False),
    (1, 1000, 1000, 16, None, False, False, False),
    (3, 64, 64, 2, (8, 8), False, True, True),
    (2, 300, 512, 16, None, False, True, False),
    (1, 520, 100, 4, None, True, False, True),
]


@pytest.mark.parametrize("B,S_q,S_kv,H,grid,fused,weights,causal", CASES)
def test_rawq_matches_prologue_then_flash(B, S_q, S_kv, H, grid, fused, weights, causal):
    lib = _lib.load()
    rng = np.random.default_rng(B * 7919 + S_q * 31 + S_kv + H)
    print(f"rawq case B={B} S_q={S_q} S_kv={S_kv} H={H} grid={grid} fused={fused} "
          f"weights={weights} causal={causal}", flush=True)
    ld = 3 * H * D if fused else H * D
    qraw = rng.standard_normal((B, S_q, ld), dtype=np.float32)
    qraw[0, S_q // 3, :D] *= 40.0  # one large row: a wide range inside the sum of squares
    qb = DevBuf.of(qraw)
    k = DevBuf.of(rng.standard_normal((B, S_kv, H, D), dtype=np.float32))
    v = DevBuf.of(rng.standard_normal((B, S_kv, H, D), dtype=np.float32))
    wq = DevBuf.of(rng.uniform(0.5, 1.5, D).astype(np.float32)) if weights else None
    wk = DevBuf.of(rng.uniform(0.5, 1.5, D).astype(np.float32)) if weights else None
    fr = DevBuf.of(generate_rope_freqs(*grid)) if grid else None
    eps = ct.c_float(1e-6)
    scale = ct.c_float(1.0 / math.sqrt(D))
    sp = lib.anima_hip_vt_padded_len(S_kv)
    row = 2 * D
    qx_s = _lib.strides([S_q * ld, D, ld])
    q_terms = DevBuf(B * S_q * H * row * 2)
    k_terms = DevBuf(B * S_kv * H * row * 2)
    vt = DevBuf(B * H * row * sp * 2)
    qts = _lib.strides([S_q * H * row, row, H * row])
    kts = _lib.strides([S_kv * H * row, row, H * row])
    kvs = _lib.strides([S_kv * H * D, D, H * D])
    os_ = _lib.strides([S_q * H * D, D, H * D])
    _lib.check(lib.anima_hip_qk_prologue_dev(qb.addr, q_terms.addr, _ptr(wq), _ptr(fr), B, S_q,
                                             H, D, qx_s, qts, eps, 1 | 4, None), "q prologue")
    _lib.check(lib.anima_hip_qk_prologue_dev(k.addr, k_terms.addr, _ptr(wk),
                                             _ptr(fr) if S_q == S_kv else None, B, S_kv, H, D,
                                             kvs, kts, eps, 1 | 4, None), "k prologue")
    _lib.check(lib.anima_hip_pack_vt_terms_dev(v.addr, vt.addr, B, H, S_kv, D, kvs, None, None),
               "pack_vt_terms_dev")
    o_ref, o_raw = DevBuf(B * S_q * H * D * 4), DevBuf(B * S_q * H * D * 4)
    _lib.check(lib.anima_hip_flash_x3_dev(q_terms.addr, k_terms.addr, vt.addr, o_ref.addr, B, H,
                                          S_q, S_kv, D, qts, kts, None, os_, scale, causal,
                                          None), "flash_x3_dev")
    _lib.check(lib.anima_hip_flash_x3_rawq_dev(qb.addr, _ptr(wq), _ptr(fr), eps, k_terms.addr,
                                               vt.addr, o_raw.addr, B, H, S_q, S_kv, D, qx_s,
                                               kts, None, os_, scale, causal, None),
               "flash_x3_rawq_dev")
    ref = o_ref.get((B, S_q, H, D))
    out = o_raw.get((B, S_q, H, D))
    assert np.isfinite(out).all()
    assert np.array_equal(_bits(out), _bits(ref))


def test_rawq_nan_and_inf_rows_match():
    """A NaN and an infinity in two raw rows: the kernel's preparation
    propagates them exactly as the row prologue does."""
    lib = _lib.load()
    rng = np.random.default_rng(404)
    B, S, H = 1, 256, 4
    qraw = rng.standard_normal((B, S, H, D), dtype=np.float32)
    qraw[0, 5, 1, 70] = np.nan
    qraw[0, 9, 2, 3] = np.inf
    qb = DevBuf.of(qraw)
    kv = rng.standard_normal((2, B, S, H, D), dtype=np.float32)
    fr = DevBuf.of(generate_rope_freqs(16, 16))
    eps = ct.c_float(1e-6)
    scale = ct.c_float(1.0 / math.sqrt(D))
    sp = lib.anima_hip_vt_padded_len(S)
    xs = _lib.strides([S * H * D, D, H * D])
    ts = _lib.strides([S * H * 2 * D, 2 * D, H * 2 * D])
    qt, kt = DevBuf(B * S * H * 2 * D * 2), DevBuf(B * S * H * 2 * D * 2)
    k, v = DevBuf.of(kv[0]), DevBuf.of(kv[1])
    vt = DevBuf(B * H * 2 * D * sp * 2)
    for x, o in ((qb, qt), (k, kt)):
        _lib.check(lib.anima_hip_qk_prologue_dev(x.addr, o.addr, None, fr.addr, B, S, H, D, xs,
                                                 ts, eps, 1 | 4, None), "prologue")
    _lib.check(lib.anima_hip_pack_vt_terms_dev(v.addr, vt.addr, B, H, S, D, xs, None, None),
               "pack")
    o_ref, o_raw = DevBuf(B * S * H * D * 4), DevBuf(B * S * H * D * 4)
    _lib.check(lib.anima_hip_flash_x3_dev(qt.addr, kt.addr, vt.addr, o_ref.addr, B, H, S, S, D,
                                          ts, ts, None, xs, scale, False, None), "flash")
    _lib.check(lib.anima_hip_flash_x3_rawq_dev(qb.addr, None, fr.addr, eps, kt.addr, vt.addr,
                                               o_raw.addr, B, H, S, S, D, xs, ts, None, xs,
                                               scale, False, None), "flash rawq")
    ref, out = o_ref.get((B, S, H, D)), o_raw.get((B, S, H, D))
    assert np.isfinite(ref[0, 6]).all()
    assert np.array_equal(_bits(out), _bits(ref))


F32_CASES = [  # B, S_q, S_kv, H, fused projection layout, weights, causal
    (2, 4096, 512, 16, False, True, False),
    (2, 77, 77, 3, True, True, False),
    (1, 1000, 1000, 16, False, False, True),
    (2, 256, 512, 16, True, False, False),
]


@pytest.mark.parametrize("B,S_q,S_kv,H,fused,weights,causal", F32_CASES)
def test_f32_rawq_matches_prologue_then_flash(B, S_q, S_kv, H, fused, weights, causal):
    """anima_hip_flash_f32_rawq_dev (q RMSNorm inside the f32 kernel) against
    anima_hip_qk_prologue_dev (flags 1, f32 rows) + anima_hip_flash_f32_dev,
    bit for bit; one row carries a NaN and one an infinity."""
    lib = _lib.load()
    rng = np.random.default_rng(B * 104729 + S_q * 17 + S_kv + H)
    print(f"f32 rawq case B={B} S_q={S_q} S_kv={S_kv} H={H} fused={fused} weights={weights} "
          f"causal={causal}", flush=True)
    ld = 3 * H * D if fused else H * D
    qraw = rng.standard_normal((B, S_q, ld), dtype=np.float32)
    qraw[0, S_q // 3, :D] *= 40.0
    qraw[B - 1, S_q // 2, 5] = np.nan
    qraw[0, S_q - 1, D + 7 if H > 1 else 7] = np.inf
    qb = DevBuf.of(qraw)
    k = DevBuf.of(rng.standard_normal((B, S_kv, H, D), dtype=np.float32))
    v = DevBuf.of(rng.standard_normal((B, S_kv, H, D), dtype=np.float32))
    wq = DevBuf.of(rng.uniform(0.5, 1.5, D).astype(np.float32)) if weights else None
    eps = ct.c_float(1e-6)
    scale = ct.c_float(1.0 / math.sqrt(D))
    qx_s = _lib.strides([S_q * ld, D, ld])
    qs = _lib.strides([S_q * H * D, D, H * D])
    kvs = _lib.strides([S_kv * H * D, D, H * D])
    qn = DevBuf(B * S_q * H * D * 4)
    _lib.check(lib.anima_hip_qk_prologue_dev(qb.addr, qn.addr, _ptr(wq), None, B, S_q, H, D,
                                             qx_s, qs, eps, 1, None), "q prologue")
    o_ref, o_raw = DevBuf(B * S_q * H * D * 4), DevBuf(B * S_q * H * D * 4)
    _lib.check(lib.anima_hip_flash_f32_dev(qn.addr, k.addr, v.addr, o_ref.addr, B, H, S_q, S_kv,
                                           D, qs, kvs, kvs, qs, scale, causal, None),
               "flash_f32_dev")
    _lib.check(lib.anima_hip_flash_f32_rawq_dev(qb.addr, _ptr(wq), eps, k.addr, v.addr,
                                                o_raw.addr, B, H, S_q, S_kv, D, qx_s, kvs, kvs,
                                                qs, scale, causal, None), "flash_f32_rawq_dev")
    ref = o_ref.get((B, S_q, H, D))
    out = o_raw.get((B, S_q, H, D))
    assert np.isfinite(ref[0, 1]).all()
    assert np.array_equal(_bits(out), _bits(ref))


BF16_CASES = [  # B, S_q, S_kv, H, grid (None: no RoPE), fused projection layout, weights, causal
    (2, 4096, 512, 16, None, False, True, False),     # two 4-wave workgroups per CU
    (2, 4096, 700, 16, None, True, True, False),      # the same with a ragged key tile
    (2, 4096, 4096, 16, (64, 64), False, True, False),  # 8-wave grid, RoPE
    (1, 520, 100, 4, None, True, False, True),        # 4-wave grid, causal
    (2, 77, 77, 3, (7, 11), True, True, False),
]


@pytest.mark.parametrize("B,S_q,S_kv,H,grid,fused,weights,causal", BF16_CASES)
def test_bf16_rawq_matches_prologue_then_flash(B, S_q, S_kv, H, grid, fused, weights, causal):
    """anima_hip_flash_bf16_rawq_dev (q RMSNorm, RoPE and bf16 rounding
    inside the bf16 kernel) against anima_hip_qk_prologue_dev (flags 1 | 2,
    bf16 rows) + anima_hip_flash_bf16_dev, bit for bit; one row carries a NaN
    and one an infinity."""
    lib = _lib.load()
    rng = np.random.default_rng(B * 15485863 + S_q * 13 + S_kv + H)
    print(f"bf16 rawq case B={B} S_q={S_q} S_kv={S_kv} H={H} grid={grid} fused={fused} "
          f"weights={weights} causal={causal}", flush=True)
    ld = 3 * H * D if fused else H * D
    qraw = rng.standard_normal((B, S_q, ld), dtype=np.float32)
    qraw[0, S_q // 3, :D] *= 40.0
    qraw[B - 1, S_q // 2, 5] = np.nan
    qraw[0, S_q - 1, D + 7 if H > 1 else 7] = np.inf
    qb = DevBuf.of(qraw)
    k = DevBuf.of(rng.standard_normal((B, S_kv, H, D), dtype=np.float32))
    v = DevBuf.of(rng.standard_normal((B, S_kv, H, D), dtype=np.float32))
    wq = DevBuf.of(rng.uniform(0.5, 1.5, D).astype(np.float32)) if weights else None
    wk = DevBuf.of(rng.uniform(0.5, 1.5, D).astype(np.float32)) if weights else None
    fr = DevBuf.of(generate_rope_freqs(*grid)) if grid else None
    eps = ct.c_float(1e-6)
    scale = ct.c_float(1.0 / math.sqrt(D))
    sp = lib.anima_hip_vt_padded_len(S_kv)
    qx_s = _lib.strides([S_q * ld, D, ld])
    qs = _lib.strides([S_q * H * D, D, H * D])
    kvs = _lib.strides([S_kv * H * D, D, H * D])
    qn, kn = DevBuf(B * S_q * H * D * 2), DevBuf(B * S_kv * H * D * 2)
    vt = DevBuf(B * H * D * sp * 2)
    _lib.check(lib.anima_hip_qk_prologue_dev(qb.addr, qn.addr, _ptr(wq), _ptr(fr), B, S_q, H, D,
                                             qx_s, qs, eps, 1 | 2, None), "q prologue")
    _lib.check(lib.anima_hip_qk_prologue_dev(k.addr, kn.addr, _ptr(wk),
                                             _ptr(fr) if S_q == S_kv else None, B, S_kv, H, D,
                                             kvs, kvs, eps, 1 | 2, None), "k prologue")
    _lib.check(lib.anima_hip_pack_vt_dev(v.addr, vt.addr, B, H, S_kv, D, kvs, None, None), "pack")
    o_ref, o_raw = DevBuf(B * S_q * H * D * 4), DevBuf(B * S_q * H * D * 4)
    _lib.check(lib.anima_hip_flash_bf16_dev(qn.addr, kn.addr, vt.addr, o_ref.addr, B, H, S_q,
                                            S_kv, D, qs, kvs, None, qs, scale, causal, None),
               "flash_bf16_dev")
    _lib.check(lib.anima_hip_flash_bf16_rawq_dev(qb.addr, _ptr(wq), _ptr(fr), eps, kn.addr,
                                                 vt.addr, o_raw.addr, B, H, S_q, S_kv, D, qx_s,
                                                 kvs, None, qs, scale, causal, None),
               "flash_bf16_rawq_dev")
    ref = o_ref.get((B, S_q, H, D))
    out = o_raw.get((B, S_q, H, D))
    assert np.isfinite(ref[0, 1]).all()
    assert np.array_equal(_bits(out), _bits(ref))


def test_bf16_paired_workgroups_equal_three_stage_rings():
    """The 4096 x 512 cross-attention shape (B=2, H=16) runs as two 4-wave
    workgroups per CU with two-stage K/V rings; each (batch, head) called on
    its own is a small grid that runs 4-wave workgroups with three-stage
    rings.  Every query row's arithmetic is the same, so the outputs agree
    bit for bit."""
    lib = _lib.load()
    rng = np.random.default_rng(2718)
    B, S_q, S_kv, H = 2, 4096, 512, 16
    q = rng.standard_normal((B, S_q, H, D), dtype=np.float32)
    k = rng.standard_normal((B, S_kv, H, D), dtype=np.float32)
    v = rng.standard_normal((B, S_kv, H, D), dtype=np.float32)
    bits16 = lambda x: ((x.view(np.uint32).astype(np.uint64) + 0x7FFF +
                         ((x.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16)
    qd, kd = DevBuf.of(bits16(q)), DevBuf.of(bits16(k))
    sp = lib.anima_hip_vt_padded_len(S_kv)
    vd, vt = DevBuf.of(v), DevBuf(B * H * D * sp * 2)
    kvs = _lib.strides([S_kv * H * D, D, H * D])
    qs = _lib.strides([S_q * H * D, D, H * D])
    _lib.check(lib.anima_hip_pack_vt_dev(vd.addr, vt.addr, B, H, S_kv, D, kvs, None, None), "pack")
    scale = ct.c_float(1.0 / math.sqrt(D))
    o_all, o_one = DevBuf(B * S_q * H * D * 4), DevBuf(B * S_q * H * D * 4)
    _lib.check(lib.anima_hip_flash_bf16_dev(qd.addr, kd.addr, vt.addr, o_all.addr, B, H, S_q,
                                            S_kv, D, qs, kvs, None, qs, scale, False, None),
               "flash all heads")
    vts = _lib.strides([H * D * sp, D * sp, sp])
    for b in range(B):
        for h in range(H):
            off = (b * S_q * H + h) * D  # element offset of (b, 0, h, 0)
            koff = (b * S_kv * H + h) * D
            _lib.check(lib.anima_hip_flash_bf16_dev(
                qd.addr + 2 * off, kd.addr + 2 * koff, vt.addr + 2 * (b * H + h) * D * sp,
                o_one.addr + 4 * off, 1, 1, S_q, S_kv, D, qs, kvs, vts, qs, scale, False, None),
                "flash one head")
    assert np.array_equal(_bits(o_all.get((B, S_q, H, D))), _bits(o_one.get((B, S_q, H, D))))
