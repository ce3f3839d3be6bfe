"""Bounds of the attention epilogues: with a ragged last query tile, no
kernel writes past the last row of O.

The one-call attention (anima_hip_attention_dev) and the cached-context
cross-attention (anima_hip_cross_attention_dev) write O as [B, S_q, H, D]
rows.  Here O lives at the start of a larger buffer whose tail holds a
sentinel pattern; after the call the tail must be unchanged and O must equal
the result written into an exactly sized buffer, bit for bit.  The shapes
take the 4-wave grid (few query tiles) and the 8-wave grid, with S_q not a
multiple of the 128- or 256-row query tile.
"""
import ctypes as ct

import numpy as np
import pytest

from anima_hip import _lib, rt
from anima_hip.rope import generate_rope_freqs

pytestmark = pytest.mark.gpu

H, D = 16, 128
TAIL_ROWS = 300
SENTINEL = np.float32(-3.75)


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


@pytest.mark.parametrize("mode", [rt.F32, rt.BF16, rt.F32X3])
@pytest.mark.parametrize("B,S,grid", [(1, 200, (10, 20)), (2, 3000, (50, 60))])
def test_attention_writes_no_row_past_o(mode, B, S, grid):
    from devmem import DevBuf
    lib = _lib.load()
    rng = np.random.default_rng(S + 10 * mode)
    q, k, v = (rng.standard_normal((B, S, H, D), dtype=np.float32) for _ in range(3))
    bufs = [DevBuf.of(x) for x in (q, k, v)]
    ones = DevBuf.of(np.ones(D, np.float32))
    fr = DevBuf.of(generate_rope_freqs(*grid))
    n = lib.anima_hip_attention_scratch_bytes(B, S, B, S, H, D, mode)
    scratch = DevBuf(n)
    rows = B * S * H
    print(f"attention guard B={B} S={S} mode={mode}", flush=True)

    def run(out):
        _lib.check(lib.anima_hip_attention_dev(bufs[0].addr, bufs[1].addr, bufs[2].addr,
                                               ones.addr, ones.addr, fr.addr, out.addr,
                                               scratch.addr, n, B, S, B, S, H, D,
                                               ct.c_float(1e-6), mode, None), "attention_dev")

    exact = DevBuf(rows * D * 4)
    run(exact)
    ref = exact.get((rows, D))
    big = DevBuf.of(np.full((rows + TAIL_ROWS, D), SENTINEL))
    run(big)
    got = big.get((rows + TAIL_ROWS, D))
    assert np.array_equal(got[:rows].view(np.uint32), ref.view(np.uint32))
    assert np.all(got[rows:] == SENTINEL)


@pytest.mark.parametrize("mode", [rt.F32, rt.BF16, rt.F32X3])
@pytest.mark.parametrize("B,S", [(2, 200), (2, 3000)])
def test_cross_attention_writes_no_row_past_o(mode, B, S):
    from devmem import DevBuf
    lib = _lib.load()
    rng = np.random.default_rng(7 * S + mode)
    ctx = rng.standard_normal((B, 512, 1024), dtype=np.float32) * np.float32(0.5)
    w = rng.standard_normal((2, H * D, 1024), dtype=np.float32) * np.float32(0.02)
    u = w.view(np.uint32).astype(np.uint64)
    bits = (((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF) >> 16).astype(np.uint16)
    cache = rt.ContextKV(ctx, bits[0], bits[1], np.ones(D, np.float32), heads=H, head_dim=D,
                         mode=mode)
    try:
        q = DevBuf.of(rng.standard_normal((B, S, H, D), dtype=np.float32))
        qw = DevBuf.of(np.ones(D, np.float32))
        n = lib.anima_hip_cross_attention_scratch_bytes(cache.handle, B, S)
        scratch = DevBuf(max(n, 256))
        rows = B * S * H
        print(f"cross-attention guard B={B} S={S} mode={mode}", flush=True)

        def run(out):
            _lib.check(lib.anima_hip_cross_attention_dev(q.addr, qw.addr, cache.handle,
                                                         out.addr, scratch.addr, n, B, S,
                                                         ct.c_float(1e-6), None),
                       "cross_attention_dev")

        exact = DevBuf(rows * D * 4)
        run(exact)
        ref = exact.get((rows, D))
        big = DevBuf.of(np.full((rows + TAIL_ROWS, D), SENTINEL))
        run(big)
        got = big.get((rows + TAIL_ROWS, D))
        assert np.array_equal(got[:rows].view(np.uint32), ref.view(np.uint32))
        assert np.all(got[rows:] == SENTINEL)
    finally:
        cache.close()
