"""anima_hip_qkv_prologue_dev, the one-launch preparation of a
self-attention's q rows, k rows and packed V^T, against the separate entries
it replaces (anima_hip_qk_prologue_dev twice and anima_hip_pack_vt_dev /
anima_hip_pack_vt_terms_dev): bit for bit, in every mode, with and without
RMSNorm weights and RoPE, on dense [B, S, H, D] inputs and on column blocks
of one fused [B*S, 3*H*D] projection (row stride 3*H*D, as the DiT's q/k/v),
including ragged key tiles.  The separate entries are themselves pinned bit
for bit to the reference's RMSNorm and RoPE (tests/test_gpu_flash.py).  The
attention core through anima_hip_attention_dev, which now takes this path,
is checked against the oracle by the other GPU tests."""
import ctypes as ct

import numpy as np
import pytest

from anima_hip import _lib, rt
from anima_hip.rope import generate_rope_freqs

pytestmark = pytest.mark.gpu
D = 128


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


CASES = [  # B, S, H, grid (None: no RoPE), fused projection layout, norm weights
    (2, 4096, 16, (64, 64), False, False),
    (2, 77, 3, (7, 11), True, True),
    (1, 1000, 16, None, True, True),
    (3, 64, 2, (8, 8), False, True),
    # RoPE table rows staged in LDS per 32-row group (H >= 16): a last group
    # holding one token (1 * 77 * 16 rows), and one token per group (H = 32).
    (1, 77, 16, (7, 11), True, True),
    (2, 64, 32, (8, 8), False, True),
]


@pytest.mark.parametrize("mode", [rt.F32, rt.BF16, rt.F32X3])
@pytest.mark.parametrize("B,S,H,grid,fused,weights", CASES)
def test_qkv_prologue_matches_separate_entries(mode, B, S, H, grid, fused, weights):
    from devmem import DevBuf
    lib = _lib.load()
    rng = np.random.default_rng(B * 1000 + S + H + mode)
    ld = 3 * H * D if fused else H * D
    print(f"qkv prologue mode={mode} B={B} S={S} H={H} grid={grid} ld={ld}", flush=True)
    if fused:  # q, k, v are column blocks of one [B*S, 3*H*D] buffer
        proj = rng.standard_normal((B, S, 3 * H * D), dtype=np.float32)
        buf = DevBuf.of(proj)
        q, k, v = buf.addr, buf.addr + 4 * H * D, buf.addr + 8 * H * D
    else:
        bufs = [DevBuf.of(rng.standard_normal((B, S, H, D), dtype=np.float32)) for _ in range(3)]
        q, k, v = (b.addr for b in bufs)
    wq = DevBuf.of(rng.uniform(0.5, 1.5, D).astype(np.float32)) if weights else None
    wk = DevBuf.of(rng.uniform(0.5, 1.5, D).astype(np.float32)) if weights else None
    fr = DevBuf.of(generate_rope_freqs(*grid)) if grid else None
    ptr = (lambda b: b.addr if b is not None else None)

    terms = mode == rt.F32X3
    row = 2 * D if terms else D
    ebytes = 4 if mode == rt.F32 else 2
    qk_bytes = B * S * H * row * ebytes
    sp = lib.anima_hip_vt_padded_len(S)
    vt_bytes = B * H * row * sp * 2
    outs = {n: DevBuf(qk_bytes) for n in ("q0", "k0", "q1", "k1")}
    vts = {n: DevBuf(vt_bytes) for n in ("v0", "v1")}

    # The separate entries.
    xs = _lib.strides([S * ld, D, ld])
    os_ = _lib.strides([S * H * row, row, H * row])
    flags = 1 | (2 if mode == rt.BF16 else 4 if terms else 0)
    eps = ct.c_float(1e-6)
    for x, w, o in ((q, wq, outs["q0"]), (k, wk, outs["k0"])):
        _lib.check(lib.anima_hip_qk_prologue_dev(x, o.addr, ptr(w), ptr(fr), B, S, H, D, xs, os_,
                                                 eps, flags, None), "qk_prologue_dev")
    if mode == rt.BF16:
        _lib.check(lib.anima_hip_pack_vt_dev(v, vts["v0"].addr, B, H, S, D, xs, None, None),
                   "pack_vt_dev")
    elif terms:
        _lib.check(lib.anima_hip_pack_vt_terms_dev(v, vts["v0"].addr, B, H, S, D, xs, None,
                                                   None), "pack_vt_terms_dev")
    # One launch.
    _lib.check(lib.anima_hip_qkv_prologue_dev(q, k, v, ld if fused else 0, ptr(wq), ptr(wk),
                                              ptr(fr), outs["q1"].addr, outs["k1"].addr,
                                              vts["v1"].addr if mode != rt.F32 else None, B, S,
                                              H, D, eps, mode, None), "qkv_prologue_dev")
    dt = np.float32 if mode == rt.F32 else np.uint16
    n = qk_bytes // ebytes
    for a, b in (("q0", "q1"), ("k0", "k1")):
        np.testing.assert_array_equal(outs[a].get((n,), dt), outs[b].get((n,), dt))
    if mode != rt.F32:
        np.testing.assert_array_equal(vts["v0"].get((vt_bytes // 2,), np.uint16),
                                      vts["v1"].get((vt_bytes // 2,), np.uint16))


def test_qkv_prologue_argument_errors():
    lib = _lib.load()
    eps = ct.c_float(1e-6)
    ok = lib.anima_hip_qkv_prologue_dev(None, None, None, 0, None, None, None, None, None, None,
                                        1, 4, 1, 64, eps, rt.F32X3, None)
    assert not ok and "D == 128" in _lib.last_error()
    ok = lib.anima_hip_qkv_prologue_dev(None, None, None, 0, None, None, None, None, None, None,
                                        1, 4, 1, 128, eps, rt.F32X3, None)
    assert not ok and "null pointer" in _lib.last_error()
    ok = lib.anima_hip_qkv_prologue_dev(None, None, None, 64, None, None, None, None, None, None,
                                        1, 4, 1, 128, eps, rt.F32, None)
    assert not ok and "row stride" in _lib.last_error()
