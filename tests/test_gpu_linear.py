"""Projection GEMM on bf16 MFMA (anima_hip_linear_dev) against the oracle's
anima_rt GEMM (f32 activations x bf16 weights, f32 accumulation).

Stated accuracy, normwise (max|out - ref| / max|ref|):
* mode F32  (activations as bf16 hi + lo terms): <= 2e-5;
* mode BF16 (activations rounded to bf16):        <= 1e-2.
The F32 mode must also be far closer than the BF16 mode on the same data,
which fails if the lo term were dropped.
"""
import ctypes as ct

import numpy as np
import pytest

import oracle
from anima_hip import _lib, rt

pytestmark = pytest.mark.gpu

REL_F32 = 2e-5
REL_BF16 = 1e-2


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


def rel_err(out, ref):
    return float(np.abs(out - ref).max() / np.abs(ref).max())


def run_linear(a, w_bits, mode, lda=None):
    """C = A W^T through anima_hip_linear_dev; `lda` > K places the rows of A
    in a wider buffer."""
    from devmem import DevBuf
    lib = _lib.load()
    M, K = a.shape
    N = w_bits.shape[0]
    lda = lda or K
    abuf = np.zeros((M, lda), np.float32)
    abuf[:, :K] = a
    da, dw, dc = DevBuf.of(abuf), DevBuf.of(w_bits), DevBuf(M * N * 4)
    sb = lib.anima_hip_linear_scratch_bytes(M, K, mode)
    scratch = DevBuf(max(sb, 256))
    ok = lib.anima_hip_linear_dev(da.addr, lda, dw.addr, K, dc.addr, N, M, N, K, mode,
                                  scratch.addr, sb, None)
    _lib.check(ok, "linear_dev")
    return dc.get((M, N))


def _data(seed, M, N, K):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((M, K), dtype=np.float32)
    w = oracle.f32_to_bf16_bits(rng.standard_normal((N, K), dtype=np.float32) * 0.02)
    return a, w


# (M, N, K, lda): ragged M/N, the text-context K/V projection (Bc=1 and 2),
# the 256-token q projection, K not a multiple of 8 (no library solution:
# exact f32-MFMA fallback), and A rows inside a wider buffer.
CASES = [(300, 200, 136, None), (512, 2048, 1024, None), (1024, 2048, 1024, None),
         (512, 2048, 2048, None), (37, 64, 77, None), (200, 256, 512, 520)]


@pytest.mark.parametrize("M,N,K,lda", CASES)
def test_linear_modes(M, N, K, lda):
    a, w = _data(M + N + K, M, N, K)
    ref = oracle.gemm_bf16(a, w)
    print(f"linear M={M} N={N} K={K} lda={lda}", flush=True)
    e32 = rel_err(run_linear(a, w, rt.F32, lda), ref)
    e16 = rel_err(run_linear(a, w, rt.BF16, lda), ref)
    print(f"  rel err f32-split {e32:.2e}  bf16 {e16:.2e}", flush=True)
    assert e32 <= REL_F32
    assert e16 <= REL_BF16
    if K % 8 == 0:
        assert e32 * 20 < e16


# Shapes of the small-M kernel (M <= 1024, K a multiple of 64; split over K
# with a deterministic reduction): the 256x256 image's fc2 (K = 8192, the
# f32 mode's two terms doubling it), q/k/v and output projections at M = 512,
# and ragged M and N (tails clamped).  Rows are sampled for the oracle.
SMALL_M = [(512, 2048, 8192), (512, 6144, 2048), (512, 2048, 2048), (77, 300, 512),
           (1000, 2052, 4096), (8, 128, 64), (512, 2048, 16384), (256, 384, 576),
           (640, 1024, 1536)]


@pytest.mark.parametrize("M,N,K", SMALL_M)
def test_small_m_kernel_vs_oracle(M, N, K):
    a, w = _data(M * 7 + N + K, M, N, K)
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M).integers(0, M, 14)]))
    ref = oracle.gemm_bf16(np.ascontiguousarray(a[rows]), w)
    print(f"small-M linear M={M} N={N} K={K}", flush=True)
    e = {}
    for mode, tol in ((rt.F32, REL_F32), (rt.BF16, REL_BF16)):
        out = run_linear(a, w, mode)
        assert np.isfinite(out).all()
        e[mode] = rel_err(out[rows], ref)
        print(f"  mode {mode}: rel err {e[mode]:.2e} on {len(rows)} rows", flush=True)
        assert e[mode] <= tol
        # Deterministic: the split partials are added in a fixed order.
        np.testing.assert_array_equal(run_linear(a, w, mode), out)
    assert e[rt.F32] * 20 < e[rt.BF16]


def test_linear_projection_8192x2048x2048_sampled_rows():
    """The per-block projection at 4096 tokens, B=2: [8192, 2048] x [2048, 2048]^T;
    64 rows (first, last and random) are checked against the oracle."""
    M, N, K = 8192, 2048, 2048
    a, w = _data(8192, M, N, K)
    rows = np.unique(np.concatenate([[0, 1, 4095, 4096, M - 1],
                                     np.random.default_rng(5).integers(0, M, 59)]))
    ref = oracle.gemm_bf16(a[rows], w)
    for mode, tol in ((rt.F32, REL_F32), (rt.BF16, REL_BF16)):
        out = run_linear(a, w, mode)
        assert np.isfinite(out).all()
        err = rel_err(out[rows], ref)
        print(f"  mode {mode}: rel err {err:.2e} on {len(rows)} rows", flush=True)
        assert err <= tol


# Shapes of the large-M kernel (at least 256 output tiles of 256 x 256, or
# of 128 x 256 with two terms): the 1024x1024 image's projections at
# M = 8192 -- q/k/v/o (N = 2048), the fused q/k/v (N = 6144), fc1 (N = 8192)
# and fc2 (K = 8192) -- and ragged M and N with the last rows and columns
# of the tile clamped.  Rows are sampled for the oracle, including both ends
# of every ragged edge.
LARGE_M = [(8192, 6144, 2048), (8192, 8192, 2048), (8192, 2048, 8192), (8000, 2100, 512),
           (8200, 2048, 1024),
           # the f32-activation kernel's 32-element K chunks: one, three and five
           # chunks (prologue only; the three-stage ring filled; copies in the loop)
           (8192, 2048, 32), (8192, 2048, 96), (8192, 2048, 160)]


@pytest.mark.parametrize("M,N,K", LARGE_M)
def test_large_m_kernel_vs_oracle(M, N, K):
    a, w = _data(M * 3 + N + K, M, N, K)
    rows = np.unique(np.concatenate([[0, 1, 255, 256, M - 257, M - 256, M - 2, M - 1],
                                     np.random.default_rng(M + N).integers(0, M, 24)]))
    ref = oracle.gemm_bf16(np.ascontiguousarray(a[rows]), w)
    print(f"large-M linear M={M} N={N} K={K}", flush=True)
    e = {}
    for mode, tol in ((rt.F32, REL_F32), (rt.BF16, REL_BF16)):
        out = run_linear(a, w, mode)
        assert np.isfinite(out).all()
        e[mode] = rel_err(out[rows], ref)
        print(f"  mode {mode}: rel err {e[mode]:.2e} on {len(rows)} rows", flush=True)
        assert e[mode] <= tol
    assert e[rt.F32] * 20 < e[rt.BF16]


@pytest.mark.parametrize("M,N,K", [(8192, 2048, 2048), (8000, 2100, 512), (8200, 2048, 1024),
                                   (8192, 6144, 64), (4096, 2048, 512), (4000, 2100, 128)])
def test_large_m_f32_activations_equal_split_path(M, N, K):
    """F32 mode at large M with 16-byte aligned A rows: the product kernels
    split the f32 activations into hi/lo bf16 terms in registers (256 x 256
    tiles where they fill the GPU, 128 x 256 at 4096 rows).  The same values
    with a row stride of K + 2 floats take the split pass and the two-term
    kernel on its term rows; the outputs agree bit for bit (ragged M and N,
    and K of one to two chunks, included)."""
    a, w = _data(M + 7 * N + K, M, N, K)
    print(f"f32-activation large-M linear M={M} N={N} K={K}", flush=True)
    fused = run_linear(a, w, rt.F32)
    split = run_linear(a, w, rt.F32, lda=K + 2)
    assert np.isfinite(fused).all()
    assert np.array_equal(fused.view(np.uint32), split.view(np.uint32))


@pytest.mark.parametrize("M,N,K,lda", [(8192, 2048, 512, 516), (4096, 2048, 256, 260)])
def test_large_m_f32_activations_wide_rows(M, N, K, lda):
    """The in-register split on A rows inside a wider buffer (row stride K + 4
    floats, still 16-byte aligned), 256 x 256 and 128 x 256 tiles: the same
    bits as the split path (row stride K + 2, which the kernels do not take)."""
    a, w = _data(M + N + lda, M, N, K)
    print(f"f32-activation large-M linear M={M} N={N} K={K} lda={lda}", flush=True)
    fused = run_linear(a, w, rt.F32, lda=lda)
    split = run_linear(a, w, rt.F32, lda=K + 2)
    assert np.array_equal(fused.view(np.uint32), split.view(np.uint32))


@pytest.mark.parametrize("M,N,K", [(8192, 2048, 256), (4096, 2048, 256), (8192, 2048, 128)])
@pytest.mark.parametrize("mode", [rt.F32, rt.BF16])
def test_large_m_output_rows_in_a_wider_buffer(M, N, K, mode):
    """C rows with a pitch of N + 64 floats: the same values as packed rows,
    and the 64 columns past N of every row keep the caller's bytes (the large-M
    epilogues store no column past N)."""
    from devmem import DevBuf
    lib = _lib.load()
    a, w = _data(M + N + K + mode, M, N, K)
    ldc = N + 64
    da, dw = DevBuf.of(a), DevBuf.of(w)
    sentinel = np.full((M, ldc), np.float32(-7.25))
    dc = DevBuf.of(sentinel)
    sb = lib.anima_hip_linear_scratch_bytes(M, K, mode)
    scratch = DevBuf(max(sb, 256))
    print(f"large-M linear into rows of {ldc} floats, M={M} N={N} K={K} mode {mode}", flush=True)
    _lib.check(lib.anima_hip_linear_dev(da.addr, K, dw.addr, K, dc.addr, ldc, M, N, K, mode,
                                        scratch.addr, sb, None), "linear_dev")
    wide = dc.get((M, ldc))
    packed = run_linear(a, w, mode)
    assert np.array_equal(wide[:, :N].view(np.uint32), packed.view(np.uint32))
    assert np.array_equal(wide[:, N:], sentinel[:, N:])


def test_linear_drop_in_gemm_bf16_is_split_path():
    """anima_rt_run_gemm_bf16 (host drop-in) runs the F32 split mode on shapes
    the library GEMM supports, within the drop-in's 1e-5 bound."""
    a, w = _data(11, 256, 512, 1024)
    ref = oracle.gemm_bf16(a, w)
    out = rt.gemm_bf16(a, w)
    assert np.abs(out - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


def test_linear_errors():
    lib = _lib.load()
    assert not lib.anima_hip_linear_dev(None, 8, None, 8, None, 8, 4, 4, 8, 7, None, 0, None)
    assert "mode" in _lib.last_error()
    assert lib.anima_hip_linear_scratch_bytes(0, 8, rt.F32) == 0
    assert (lib.anima_hip_linear_scratch_bytes(10, 9, rt.F32)
            == 2 * lib.anima_hip_linear_scratch_bytes(10, 9, rt.BF16))
