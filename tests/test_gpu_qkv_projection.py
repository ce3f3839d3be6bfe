"""anima_hip_qkv_projection_dev, a self-attention's q/k/v projection whose
epilogue is the attention prologue, against the two entries it fuses, bit for
bit: anima_hip_linear_dev (f32 mode, the same exact two-term product) into
[B*S][3*H*128] f32, then anima_hip_qkv_prologue_dev on its column blocks
(RMSNorm with and without weights, RoPE with and without a table).  In the
f32x3 mode the outputs are [hi | lo] term rows and the term V^T; in the f32
mode f32 rows and the projection's v block as dense V rows.  The cases take
the full-width q/k/v product (H = 16, K = 2048) at 4096 tokens, a shorter K,
and three batch entries of 1088 tokens, whose last 256-row tile is ragged
(rows past M) and whose 32-row groups meet batch boundaries inside a tile,
and activations holding NaN and infinities.  The two separate entries are pinned against the oracle elsewhere
(tests/test_gpu_linear.py, tests/test_gpu_prep.py, tests/test_gpu_flash.py).
"""
import ctypes as ct

import numpy as np
import pytest

import oracle
from anima_hip import _lib, rt
from anima_hip.rope import generate_rope_freqs

pytestmark = pytest.mark.gpu
D = 128


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


CASES = [  # B, S, H, K, RMSNorm weights, RoPE grid (H x W = S) or None
    (2, 2048, 16, 2048, True, (32, 64)),
    (2, 2048, 16, 1024, False, None),
    (3, 1088, 16, 2048, True, (32, 34)),
]


@pytest.mark.parametrize("mode", [rt.F32, rt.F32X3])
@pytest.mark.parametrize("B,S,H,K,weights,grid", CASES)
def test_fused_projection_equals_linear_then_prologue(mode, B, S, H, K, weights, grid):
    from devmem import DevBuf
    lib = _lib.load()
    HD, M = H * D, B * S
    N = 3 * HD
    print(f"qkv projection B={B} S={S} H={H} K={K} mode={mode}", flush=True)
    rng = np.random.default_rng(B * S + K + mode)
    x = DevBuf.of(rng.standard_normal((M, K), dtype=np.float32))
    w = DevBuf.of(oracle.f32_to_bf16_bits(rng.standard_normal((N, K), dtype=np.float32)
                                          * np.float32(0.02)))
    keep = []

    def opt(a):
        if a is None:
            return None
        d = DevBuf.of(a)
        keep.append(d)
        return d.addr

    wq = opt(rng.uniform(0.5, 1.5, D).astype(np.float32) if weights else None)
    wk = opt(rng.uniform(0.5, 1.5, D).astype(np.float32) if weights else None)
    fr = opt(generate_rope_freqs(*grid) if grid else None)
    eps = ct.c_float(1e-6)

    # The two separate entries.
    c = DevBuf(M * N * 4)
    sb = lib.anima_hip_linear_scratch_bytes(M, K, rt.F32)
    scratch = DevBuf(max(sb, 256))
    _lib.check(lib.anima_hip_linear_dev(x.addr, K, w.addr, K, c.addr, N, M, N, K, rt.F32,
                                        scratch.addr, sb, None), "linear_dev")
    row_bytes = M * HD * 4  # q or k rows, f32 or [hi | lo] terms; also the term V^T
    q0, k0 = DevBuf(row_bytes), DevBuf(row_bytes)
    vt0 = DevBuf(row_bytes) if mode == rt.F32X3 else None
    _lib.check(lib.anima_hip_qkv_prologue_dev(c.addr, c.addr + HD * 4, c.addr + 2 * HD * 4, N,
                                              wq, wk, fr, q0.addr, k0.addr,
                                              vt0.addr if vt0 else None, B, S, H, D, eps, mode,
                                              None), "qkv_prologue_dev")

    # The fused entry.
    q1, k1, v1 = DevBuf(row_bytes), DevBuf(row_bytes), DevBuf(row_bytes)
    _lib.check(lib.anima_hip_qkv_projection_dev(x.addr, K, w.addr, K, K, wq, wk, fr, q1.addr,
                                                k1.addr, v1.addr, B, S, H, eps, mode, None),
               "qkv_projection_dev")

    n = row_bytes // 4
    for a, b in ((q0, q1), (k0, k1)):
        np.testing.assert_array_equal(a.get((n,), np.uint32), b.get((n,), np.uint32))
    if mode == rt.F32X3:
        np.testing.assert_array_equal(vt0.get((n,), np.uint32), v1.get((n,), np.uint32))
    else:
        v_ref = c.get((M, N))[:, 2 * HD:]
        np.testing.assert_array_equal(v_ref.view(np.uint32), v1.get((M, HD)).view(np.uint32))


@pytest.mark.parametrize("mode", [rt.F32, rt.F32X3])
def test_fused_projection_with_nan_and_inf_activations(mode):
    """Rows whose activations hold NaN or infinity: the NaNs that reach the
    outputs (whole q/k rows through RMSNorm, single columns of V) carry the
    same bits as on the two-entry path."""
    from devmem import DevBuf
    lib = _lib.load()
    B, S, H, K = 2, 2048, 16, 1024
    HD, M = H * D, B * S
    N = 3 * HD
    rng = np.random.default_rng(99 + mode)
    xa = rng.standard_normal((M, K), dtype=np.float32)
    xa[5, :] = np.nan
    xa[17, 3] = np.inf
    xa[4000, 100] = -np.inf
    x = DevBuf.of(xa)
    w = DevBuf.of(oracle.f32_to_bf16_bits(rng.standard_normal((N, K), dtype=np.float32)
                                          * np.float32(0.02)))
    fr = DevBuf.of(generate_rope_freqs(32, 64))
    eps = ct.c_float(1e-6)
    c = DevBuf(M * N * 4)
    sb = lib.anima_hip_linear_scratch_bytes(M, K, rt.F32)
    scratch = DevBuf(max(sb, 256))
    _lib.check(lib.anima_hip_linear_dev(x.addr, K, w.addr, K, c.addr, N, M, N, K, rt.F32,
                                        scratch.addr, sb, None), "linear_dev")
    row_bytes = M * HD * 4
    q0, k0, v0 = DevBuf(row_bytes), DevBuf(row_bytes), DevBuf(row_bytes)
    _lib.check(lib.anima_hip_qkv_prologue_dev(c.addr, c.addr + HD * 4, c.addr + 2 * HD * 4, N,
                                              None, None, fr.addr, q0.addr, k0.addr,
                                              v0.addr if mode == rt.F32X3 else None, B, S, H, D,
                                              eps, mode, None), "qkv_prologue_dev")
    q1, k1, v1 = DevBuf(row_bytes), DevBuf(row_bytes), DevBuf(row_bytes)
    _lib.check(lib.anima_hip_qkv_projection_dev(x.addr, K, w.addr, K, K, None, None, fr.addr,
                                                q1.addr, k1.addr, v1.addr, B, S, H, eps, mode,
                                                None), "qkv_projection_dev")
    n = row_bytes // 4
    proj = c.get((M, N))
    assert np.isnan(proj[5]).all() and np.isnan(proj).sum() > N  # NaN rows and columns exercised
    for a, b in ((q0, q1), (k0, k1)):
        np.testing.assert_array_equal(a.get((n,), np.uint32), b.get((n,), np.uint32))
    if mode == rt.F32X3:
        np.testing.assert_array_equal(v0.get((n,), np.uint32), v1.get((n,), np.uint32))
    else:
        np.testing.assert_array_equal(np.ascontiguousarray(proj[:, 2 * HD:]).view(np.uint32),
                                      v1.get((M, HD)).view(np.uint32))


def test_fused_projection_refuses_unsupported_shapes():
    from devmem import DevBuf
    lib = _lib.load()
    eps = ct.c_float(1e-6)
    buf = DevBuf(4096 * 16 * D * 4 * 3)
    a = buf.addr
    # bf16 mode, S not a multiple of 64, an odd head count, too small a grid.
    for args, msg in (((2, 2048, 16, rt.BF16), "f32 and f32x3"),
                      ((2, 2000, 16, rt.F32X3), "unsupported"),
                      ((2, 2048, 15, rt.F32X3), "unsupported"),
                      ((1, 256, 16, rt.F32X3), "unsupported")):
        B, S, H, mode = args
        ok = lib.anima_hip_qkv_projection_dev(a, 2048, a, 2048, 2048, None, None, None, a, a, a,
                                              B, S, H, eps, mode, None)
        assert not ok and msg in _lib.last_error()
