"""Launch shapes of the D=128 flash kernels, each checked against the oracle.

* Split-KV: problems whose B*H*ceil(S_q/256) grid is below one workgroup per
  CU split the key range over several workgroups and merge the partials
  (host entries and the attention entries, which carry scratch).
* Workgroups of 4 waves without splitting: the device-pointer flash entries,
  which take no scratch.
* Workgroups of 8 waves: grids of at least 256 workgroups, with ragged
  query and key tails.

Tolerances are those of the two paths: max-abs 1e-4 (f32) and normwise
relative 2e-2 (bf16) against anima_rt's flash attention.
"""
import ctypes as ct

import numpy as np
import pytest

import oracle
from anima_hip import _lib, rt

pytestmark = pytest.mark.gpu

TOL = 1e-4
REL = 2e-2


def randn(rng, *shape):
    return rng.standard_normal(shape, dtype=np.float32)


def rel_err(out, ref):
    return float(np.abs(out - ref).max() / np.abs(ref).max())


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


def _inputs(seed, bh, sq, sk):
    rng = np.random.default_rng(seed)
    return randn(rng, bh, sq, 128), randn(rng, bh, sk, 128), randn(rng, bh, sk, 128)


# (BH, S_q, S_kv, causal): 32 splits of 2 tiles; one query row over 65 splits
# of one tile (the last one ragged); causal splits that are empty for the
# early query rows; the 256-token self-attention shape and a 3-tile key range
# (4 and 3 splits in f32; unsplit 4-wave grids in bf16, whose tiles are too
# cheap for a split to repay its fixed cost).
SPLIT_CASES = [(4, 256, 4096, False), (1, 1, 4097, False), (2, 300, 1000, True),
               (16, 256, 256, False), (3, 77, 129, False)]


@pytest.mark.parametrize("bh,sq,sk,causal", SPLIT_CASES)
def test_split_kv_f32(bh, sq, sk, causal):
    q, k, v = _inputs(bh * 1000 + sq + sk, bh, sq, sk)
    print(f"split f32 bh={bh} sq={sq} sk={sk} causal={causal}", flush=True)
    out = rt.sdpa_flash(q, k, v, is_causal=causal)
    ref = oracle.flash_sdpa(q, k, v, is_causal=causal, threads=min(bh, 8))
    assert np.abs(out - ref).max() <= TOL


@pytest.mark.parametrize("bh,sq,sk,causal", SPLIT_CASES)
def test_split_kv_bf16(bh, sq, sk, causal):
    q, k, v = _inputs(bh * 1000 + sq + sk + 1, bh, sq, sk)
    print(f"split bf16 bh={bh} sq={sq} sk={sk} causal={causal}", flush=True)
    out = rt.sdpa(q, k, v, is_causal=causal, mode=rt.BF16)
    ref = oracle.flash_sdpa(q, k, v, is_causal=causal, threads=min(bh, 8))
    assert rel_err(out, ref) <= REL


@pytest.mark.parametrize("bh,sq,sk,causal", [(256, 200, 77, False), (256, 300, 300, True)])
@pytest.mark.parametrize("mode", [rt.F32, rt.BF16])
def test_eight_wave_grid_tails(bh, sq, sk, causal, mode):
    q, k, v = _inputs(bh + sq + sk + mode, bh, sq, sk)
    print(f"8-wave grid mode={mode} bh={bh} sq={sq} sk={sk} causal={causal}", flush=True)
    out = rt.sdpa(q, k, v, is_causal=causal, mode=mode)
    ref = oracle.flash_sdpa(q, k, v, is_causal=causal, threads=8)
    if mode == rt.F32:
        assert np.abs(out - ref).max() <= TOL
    else:
        assert rel_err(out, ref) <= REL


def test_device_entries_without_scratch():
    """The _dev flash entries run small problems unsplit on 4-wave groups."""
    from devmem import DevBuf
    lib = _lib.load()
    bh, sq, sk = 3, 300, 700
    q, k, v = _inputs(4242, bh, sq, sk)
    ref = oracle.flash_sdpa(q, k, v, threads=3)
    dq, dk, dv = DevBuf.of(q), DevBuf.of(k), DevBuf.of(v)
    o = DevBuf(q.nbytes)
    scale = ct.c_float(128 ** -0.5)
    print("dev f32 unsplit", flush=True)
    ok = lib.anima_hip_flash_f32_dev(dq.addr, dk.addr, dv.addr, o.addr, 1, bh, sq, sk, 128, None,
                                     None, None, None, scale, False, None)
    _lib.check(ok, "flash_f32_dev")
    assert np.abs(o.get(q.shape) - ref).max() <= TOL

    print("dev bf16 unsplit", flush=True)
    qb, kb = DevBuf(q.nbytes // 2), DevBuf(k.nbytes // 2)
    sp = int(lib.anima_hip_vt_padded_len(sk))
    vt = DevBuf(bh * 128 * sp * 2)
    # [BH, S, D] seen as B=1, S, H=BH rows: {batch, head, seq} element strides.
    for src, dst, s in ((dq, qb, sq), (dk, kb, sk)):
        st = _lib.strides([bh * s * 128, s * 128, 128])
        ok = lib.anima_hip_qk_prologue_dev(src.addr, dst.addr, None, None, 1, s, bh, 128, st, st,
                                           ct.c_float(1e-6), 2, None)
        _lib.check(ok, "qk_prologue_dev")
    ok = lib.anima_hip_pack_vt_dev(dv.addr, vt.addr, 1, bh, sk, 128, None, None, None)
    _lib.check(ok, "pack_vt_dev")
    o2 = DevBuf(q.nbytes)
    vts = _lib.strides([bh * 128 * sp, 128 * sp, sp])
    ok = lib.anima_hip_flash_bf16_dev(qb.addr, kb.addr, vt.addr, o2.addr, 1, bh, sq, sk, 128, None,
                                      None, vts, None, scale, False, None)
    _lib.check(ok, "flash_bf16_dev")
    assert rel_err(o2.get(q.shape), ref) <= REL


@pytest.mark.parametrize("mode", [rt.F32, rt.BF16])
def test_empty_key_set_and_zero_sizes(mode):
    """S_kv = 0 gives O = 0 (no visible key; anima_rt's flash_attention divides
    by zero computing its key-slice count there, flash_attention.h:66-70, so the
    oracle is not called), and zero-size problems are no-ops."""
    q = np.ones((2, 5, 128), np.float32)
    empty = np.zeros((2, 0, 128), np.float32)
    out = np.full((2, 5, 128), np.nan, np.float32)  # must be overwritten with zeros
    ok = _lib.load().anima_hip_sdpa(q.ctypes.data, empty.ctypes.data, empty.ctypes.data,
                                    out.ctypes.data, 2, 5, 0, 128, ct.c_float(128 ** -0.5), False,
                                    int(mode))
    _lib.check(ok, "anima_hip_sdpa")
    assert not np.isnan(out).any() and not out.any()
    assert rt.sdpa(np.zeros((2, 0, 128), np.float32), q, q, mode=mode).shape == (2, 0, 128)
    none = np.zeros((0, 5, 128), np.float32)
    assert rt.sdpa(none, empty[:0], empty[:0], mode=mode).shape == (0, 5, 128)


@pytest.mark.parametrize("mode", [rt.F32, rt.BF16])
def test_long_sequence_32768_sampled_rows(mode):
    """S_q = S_kv = 32768 (8x the 1024x1024 latent), two heads: 64 query rows
    (first, last, random) against the oracle over all 32768 keys; query rows
    are independent, so the oracle runs on the sampled rows only."""
    rng = np.random.default_rng(32768 + mode)
    bh, S = 2, 32768
    q, k, v = randn(rng, bh, S, 128), randn(rng, bh, S, 128), randn(rng, bh, S, 128)
    print(f"long sequence mode={mode} S={S}", flush=True)
    out = rt.sdpa(q, k, v, mode=mode)
    assert np.isfinite(out).all()
    rows = np.unique(np.concatenate([[0, 1, S - 2, S - 1], rng.integers(0, S, 60)]))
    ref = oracle.flash_sdpa(np.ascontiguousarray(q[:, rows]), k, v, threads=2)
    if mode == rt.F32:
        assert np.abs(out[:, rows] - ref).max() <= TOL
    else:
        assert rel_err(out[:, rows], ref) <= REL
