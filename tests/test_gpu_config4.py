"""Config 4: one DiT denoise step's attention at 1024x1024 output.  Per block
a self-attention over 4096 latent tokens (B=2 CFG pair, H=16, D=128, q/k
RMSNorm + 3D RoPE on the 64x64 grid) and a cross-attention of 4096 query
tokens over that block's cached text-context K/V (a [2, 512, 1024] context
~ N(0, 0.5) through bf16 k/v weights ~ N(0, 0.02), k_norm, no RoPE), as
NumpyBlock runs them (anima_rt/scripts/numpy_dit.py:230-253) with the
context fixed across the step's blocks and the sampler's steps
(anima_rt/scripts/sampling.py:121-130).

* One block: both attentions through the device entry points
  (anima_hip_attention_dev, anima_hip_cross_attention_dev on a ContextKV),
  all 32 (batch, head) slices of each against the oracle.
* The 28-block step: 28 distinct blocks (inputs, contexts, weights) run back
  to back on one stream with one shared scratch buffer, as the bench times
  it; every block's two outputs must equal a standalone call of that block
  bit for bit, and one slice of the last block is checked against the
  oracle.

Tolerances: max-abs 1e-4 (f32, f32x3), normwise 2e-2 per slice (bf16).
"""
import ctypes as ct

import numpy as np
import pytest

import fullsize
import oracle
from anima_hip import _lib, rt

pytestmark = pytest.mark.gpu

B, S, H, D = 2, 4096, 16, 128
BLOCKS = 28
EPS = ct.c_float(1e-6)
ONES = np.ones(D, np.float32)
MODES = [rt.F32, rt.F32X3, rt.BF16]


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


def _scratch_bytes(lib, cache, mode):
    return max(lib.anima_hip_attention_scratch_bytes(B, S, B, S, H, D, mode),
               lib.anima_hip_cross_attention_scratch_bytes(cache.handle, B, S))


def _self(lib, q, k, v, ones, freqs, out, scratch, n, mode):
    ok = lib.anima_hip_attention_dev(q, k, v, ones, ones, freqs, out, scratch, n, B, S, B, S, H,
                                     D, EPS, mode, None)
    _lib.check(ok, "attention_dev")


def _cross(lib, q, ones, cache, out, scratch, n):
    ok = lib.anima_hip_cross_attention_dev(q, ones, cache.handle, out, scratch, n, B, S, EPS,
                                           None)
    _lib.check(ok, "cross_attention_dev")


@pytest.mark.parametrize("mode", MODES)
def test_config4_block_all_slices(mode):
    from devmem import DevBuf
    lib = _lib.load()
    q, k, v, f = fullsize.self_case(S, (64, 64), 3003)
    qx = fullsize.cross_q(S, 4004)
    ctx, wk, wv = fullsize.context_case(4005)
    print(f"config 4 block mode={mode}: device self + cached cross", flush=True)
    cache = rt.ContextKV(ctx, wk, wv, ONES, heads=H, head_dim=D, mode=mode)
    try:
        dq, dk, dv, dqx = (DevBuf.of(a) for a in (q, k, v, qx))
        ones, fr = DevBuf.of(ONES), DevBuf.of(f)
        o_self, o_cross = DevBuf(q.nbytes), DevBuf(q.nbytes)
        n = _scratch_bytes(lib, cache, mode)
        scratch = DevBuf(n)
        _self(lib, dq.addr, dk.addr, dv.addr, ones.addr, fr.addr, o_self.addr, scratch.addr, n,
              mode)
        _cross(lib, dqx.addr, ones.addr, cache, o_cross.addr, scratch.addr, n)
        out_self, out_cross = o_self.get(q.shape), o_cross.get(q.shape)
    finally:
        cache.close()
    fullsize.check_all_slices(out_self, fullsize.self_ref(S, (64, 64), 3003), mode,
                              "config 4 block, self-attention 4096x4096")
    fullsize.check_all_slices(out_cross, fullsize.cross_ref(S, 4004, 4005), mode,
                              "config 4 block, cross-attention 4096x512")


def _check_slice(out, ref, mode, what):
    err = float(np.abs(out - ref).max())
    if mode == rt.BF16:
        err /= float(np.abs(ref).max())
    print(f"  {what} mode={mode}: {err:.3e}", flush=True)
    assert err <= (2e-2 if mode == rt.BF16 else 1e-4), (what, err)


@pytest.mark.parametrize("mode", MODES)
def test_config4_28_blocks_equal_standalone_calls(mode):
    from anima_hip.rope import generate_rope_freqs
    from devmem import DevBuf
    lib = _lib.load()
    rng = np.random.default_rng(4400 + mode)
    n_el = B * S * H * D
    # Per-block inputs are windows of one N(0,1) pool at distinct offsets of
    # 7 tokens and 3 heads (a multiple of 16 bytes): q, k, v and the cross
    # query of block i start at (4i + j) * DELTA elements.
    DELTA = 7 * H * D + 3 * D
    pool = fullsize.randn(rng, n_el + 4 * BLOCKS * DELTA)
    ctx_el, w_el = 2 * 512 * 1024, H * D * 1024
    DC, DW = 5 * 1024 + 16, 3 * 1024 + 8
    ctx_pool = fullsize.randn(rng, ctx_el + BLOCKS * DC, sigma=0.5)
    w_pool = oracle.f32_to_bf16_bits(fullsize.randn(rng, w_el + 2 * BLOCKS * DW, sigma=0.02))

    def ctx_of(i):
        return ctx_pool[i * DC:i * DC + ctx_el].reshape(2, 512, 1024)

    def w_of(i, j):  # j = 0: Wk, 1: Wv
        o = (2 * i + j) * DW
        return w_pool[o:o + w_el].reshape(H * D, 1024)

    print(f"config 4, 28 blocks mode={mode}: building {BLOCKS} context caches", flush=True)
    caches = [rt.ContextKV(ctx_of(i), w_of(i, 0), w_of(i, 1), ONES, heads=H, head_dim=D,
                           mode=mode) for i in range(BLOCKS)]
    try:
        dpool = DevBuf.of(pool)
        ones, fr = DevBuf.of(ONES), DevBuf.of(generate_rope_freqs(64, 64))
        n = _scratch_bytes(lib, caches[0], mode)
        scratch = DevBuf(n)

        def at(i, j):
            return dpool.addr + 4 * (4 * i + j) * DELTA

        outs = [(DevBuf(4 * n_el), DevBuf(4 * n_el)) for _ in range(BLOCKS)]
        print("  the step: 28 x (self + cross), one stream, one scratch", flush=True)
        for i in range(BLOCKS):
            _self(lib, at(i, 0), at(i, 1), at(i, 2), ones.addr, fr.addr, outs[i][0].addr,
                  scratch.addr, n, mode)
            _cross(lib, at(i, 3), ones.addr, caches[i], outs[i][1].addr, scratch.addr, n)
        print("  standalone calls per block", flush=True)
        tmp, scratch2 = DevBuf(4 * n_el), DevBuf(n)
        last = {}
        for i in range(BLOCKS):
            for j, name in enumerate(("self", "cross")):
                in_step = outs[i][j].get((B, S, H, D))
                if j == 0:
                    _self(lib, at(i, 0), at(i, 1), at(i, 2), ones.addr, fr.addr, tmp.addr,
                          scratch2.addr, n, mode)
                else:
                    _cross(lib, at(i, 3), ones.addr, caches[i], tmp.addr, scratch2.addr, n)
                alone = tmp.get((B, S, H, D))
                assert np.isfinite(in_step).all(), (i, name)
                assert np.array_equal(in_step, alone), f"block {i} {name}: step != standalone"
                if i == BLOCKS - 1:
                    last[name] = in_step
        # One slice of the last block against the oracle.
        b, h = 1, 15
        off = lambda j: (4 * (BLOCKS - 1) + j) * DELTA  # noqa: E731
        win = [pool[off(j):off(j) + n_el].reshape(B, S, H, D)[b:b + 1, :, h:h + 1]
               for j in range(4)]
        ref = oracle.attention_dataflow(win[0], win[1], win[2], ONES, ONES,
                                        oracle.rope_freqs(64, 64))
        _check_slice(last["self"][b, :, h], ref[0, :, 0], mode, "block 27 self slice (1, 15)")
        rows = slice(h * D, (h + 1) * D)
        kx = oracle.gemm_bf16(ctx_of(BLOCKS - 1)[b], np.ascontiguousarray(w_of(BLOCKS - 1, 0)[rows]))
        vx = oracle.gemm_bf16(ctx_of(BLOCKS - 1)[b], np.ascontiguousarray(w_of(BLOCKS - 1, 1)[rows]))
        ref = oracle.attention_dataflow(win[3], kx.reshape(1, 512, 1, D), vx.reshape(1, 512, 1, D),
                                        ONES, ONES, None)
        _check_slice(last["cross"][b, :, h], ref[0, :, 0], mode, "block 27 cross slice (1, 15)")
    finally:
        for c in caches:
            c.close()
