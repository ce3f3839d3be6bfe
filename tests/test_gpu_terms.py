"""anima_hip_attention_terms_dev, the attention core writing O as the bf16
terms of the next projection's input, against anima_hip_attention_dev's f32
O split on the host: hi = bf16(O) and lo = bf16(O - hi), both rounded to
nearest even (oracle.f32_to_bf16_bits, the reference's rounding,
gemm_backend.cpp:77-85) -- the terms anima_hip_linear_dev forms from an f32
activation.  The same kernels run in both calls, so the terms must equal the
split of the f32 output bit for bit, in every arithmetic mode and on every
launch shape the attention takes: 8-wave grids, 4-wave grids, split-KV with
the combine pass, ragged query tiles and a K/V batch broadcast to both
query batches.  Columns outside the hi and lo blocks of a row keep what the
buffer held.  The f32 output is itself checked against the oracle by the
other GPU tests."""
import ctypes as ct

import numpy as np
import pytest

import oracle
from anima_hip import _lib, rt
from anima_hip.rope import generate_rope_freqs

pytestmark = pytest.mark.gpu

H, D = 16, 128
HD = H * D
SENTINEL = 0xFFFF  # a bf16 NaN pattern no finite output produces


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


CASES = [  # B, S_q, Bk, S_kv, RoPE grid; the launch shape it takes
    (2, 2048, 2, 2048, (32, 64)),  # 8-wave grid, no split
    (2, 2000, 2, 2000, None),      # 8-wave grid, ragged last query tile
    (2, 256, 2, 256, (16, 16)),    # 4-wave grid; 4-way split-KV + combine in f32
    (1, 256, 1, 2048, None),       # 4-wave grid, 8-way split-KV + combine
    (2, 1024, 1, 512, None),       # cross-attention shape: broadcast K/V, 4-wave grid
    (2, 300, 2, 64, None),         # 4-wave grid, one key tile, no split
]


def _split_terms(o):
    hi = oracle.f32_to_bf16_bits(o)
    lo = oracle.f32_to_bf16_bits(o - oracle.bf16_bits_to_f32(hi))
    return hi, lo


@pytest.mark.parametrize("mode", [rt.F32, rt.BF16, rt.F32X3])
@pytest.mark.parametrize("B,S_q,Bk,S_kv,grid", CASES)
def test_term_output_is_the_split_of_the_f32_output(mode, B, S_q, Bk, S_kv, grid):
    from devmem import DevBuf
    lib = _lib.load()
    rng = np.random.default_rng(B * 7 + S_q + S_kv + mode)
    q = rng.standard_normal((B, S_q, H, D), dtype=np.float32)
    k = rng.standard_normal((Bk, S_kv, H, D), dtype=np.float32)
    v = rng.standard_normal((Bk, S_kv, H, D), dtype=np.float32)
    qw, kw = (rng.uniform(0.5, 1.5, D).astype(np.float32) for _ in range(2))
    bufs = [DevBuf.of(x) for x in (q, k, v, qw, kw)]
    fr = DevBuf.of(generate_rope_freqs(*grid)) if grid else None
    n = lib.anima_hip_attention_scratch_bytes(B, S_q, Bk, S_kv, H, D, mode)
    scratch = DevBuf(n)
    eps = ct.c_float(1e-6)
    args = [b.addr for b in bufs] + [fr.addr if fr else None]
    print(f"attention terms B={B} S_q={S_q} Bk={Bk} S_kv={S_kv} mode={mode}", flush=True)

    out = DevBuf(q.nbytes)
    _lib.check(lib.anima_hip_attention_dev(*args, out.addr, scratch.addr, n, B, S_q, Bk, S_kv,
                                           H, D, eps, mode, None), "attention_dev")
    o = out.get((B * S_q, HD), np.float32)
    hi, lo = _split_terms(o)

    # Two-term rows with a gap after each block, and hi-only rows.
    for ld, lo_off in ((2 * HD + 16, HD + 8), (HD + 8, 0)):
        rows = np.full((B * S_q, ld), SENTINEL, np.uint16)
        t = DevBuf.of(rows)
        _lib.check(lib.anima_hip_attention_terms_dev(*args, t.addr, ld, lo_off, scratch.addr, n,
                                                     B, S_q, Bk, S_kv, H, D, eps, mode, None),
                   "attention_terms_dev")
        got = t.get((B * S_q, ld), np.uint16)
        np.testing.assert_array_equal(got[:, :HD], hi)
        if lo_off:
            np.testing.assert_array_equal(got[:, lo_off:lo_off + HD], lo)
            rest = np.concatenate([got[:, HD:lo_off], got[:, lo_off + HD:]], axis=1)
        else:
            rest = got[:, HD:]
        assert np.all(rest == SENTINEL)
        t.close()
    out.close()
    scratch.close()


def test_term_output_argument_errors():
    lib = _lib.load()
    eps = ct.c_float(1e-6)

    def call(ld, lo, d=D):
        return lib.anima_hip_attention_terms_dev(None, None, None, None, None, None, None, ld, lo,
                                                 None, 0, 1, 4, 1, 4, H, d, eps, rt.F32, None)

    assert not call(HD, 0, d=64) and "D == 128" in _lib.last_error()
    assert not call(HD - 4, 0) and "hi block" in _lib.last_error()
    assert not call(2 * HD, HD - 8) and "lo block" in _lib.last_error()
    assert not call(2 * HD, HD + 8) and "lo block" in _lib.last_error()
    assert not call(2 * HD + 4, HD) and "multiples of 8" in _lib.last_error()
    assert not call(2 * HD, HD) and "null pointer" in _lib.last_error()


# Cross-attention over a cached 512-token context at the 1024x1024 image's
# 4096 query tokens (B = 2): an 8-wave grid, so in the f32 and f32x3 modes the
# flash kernel normalises the raw query rows itself and writes the terms --
# the combination the DiT's cross-attention sub-layer runs.  Also a 4-wave
# grid (256 query tokens) with a broadcast context, and a ragged tile.
@pytest.mark.parametrize("mode", [rt.F32, rt.F32X3, rt.BF16])
@pytest.mark.parametrize("B,S_q,Bc", [(2, 4096, 2), (2, 256, 1), (2, 2000, 2)])
def test_cross_term_output_is_the_split_of_the_f32_output(mode, B, S_q, Bc):
    from devmem import DevBuf
    lib = _lib.load()
    rng = np.random.default_rng(9100 + S_q + Bc + mode)
    q = rng.standard_normal((B, S_q, H, D), dtype=np.float32)
    qw = rng.uniform(0.5, 1.5, D).astype(np.float32)
    ctx = (rng.standard_normal((Bc, 512, 1024)) * 0.5).astype(np.float32)
    wk, wv = (oracle.f32_to_bf16_bits(rng.standard_normal((HD, 1024), dtype=np.float32) * 0.02)
              for _ in range(2))
    kv = rt.ContextKV(ctx, wk, wv, None, heads=H, head_dim=D, mode=mode)
    print(f"cross attention terms B={B} S_q={S_q} Bc={Bc} mode={mode}", flush=True)
    try:
        dq, dw = DevBuf.of(q), DevBuf.of(qw)
        n = lib.anima_hip_cross_attention_scratch_bytes(kv.handle, B, S_q)
        scratch = DevBuf(n)
        eps = ct.c_float(1e-6)
        out = DevBuf(q.nbytes)
        _lib.check(lib.anima_hip_cross_attention_dev(dq.addr, dw.addr, kv.handle, out.addr,
                                                     scratch.addr, n, B, S_q, eps, None),
                   "cross_attention_dev")
        o = out.get((B * S_q, HD), np.float32)
        hi, lo = _split_terms(o)
        ld, lo_off = 2 * HD + 16, HD + 8
        t = DevBuf.of(np.full((B * S_q, ld), SENTINEL, np.uint16))
        _lib.check(lib.anima_hip_cross_attention_terms_dev(dq.addr, dw.addr, kv.handle, t.addr,
                                                           ld, lo_off, scratch.addr, n, B, S_q,
                                                           eps, None),
                   "cross_attention_terms_dev")
        got = t.get((B * S_q, ld), np.uint16)
        np.testing.assert_array_equal(got[:, :HD], hi)
        np.testing.assert_array_equal(got[:, lo_off:lo_off + HD], lo)
        assert np.all(got[:, HD:lo_off] == SENTINEL) and np.all(got[:, lo_off + HD:] == SENTINEL)
        if S_q == 4096:
            # One (batch, head) slice of the f32 output against the oracle.
            k, v = (np.stack([oracle.gemm_bf16(ctx[b], w) for b in range(Bc)])
                    .reshape(Bc, 512, H, D) for w in (wk, wv))
            ref = oracle.attention_dataflow(q[1:2, :, 5:6], k[1:2, :, 5:6], v[1:2, :, 5:6],
                                            qw, None, None)
            err = np.abs(o.reshape(B, S_q, H, D)[1:2, :, 5:6] - ref).max()
            if mode == rt.BF16:
                err /= np.abs(ref).max()
            print(f"  slice (1, 5) error {err:.3e}", flush=True)
            assert err <= (2e-2 if mode == rt.BF16 else 1e-4)
    finally:
        kv.close()


def test_cross_term_output_argument_errors():
    lib = _lib.load()
    eps = ct.c_float(1e-6)
    assert not lib.anima_hip_cross_attention_terms_dev(None, None, None, None, HD, 0, None, 0, 1,
                                                       4, eps, None)
    assert "null cache handle" in _lib.last_error()
