"""The host-pointer calls' group pipeline: group g+1 uploads while group g
computes on the compute stream, and group g's output comes back on the
download stream while later groups upload.

At 32 (batch, head) slices of 4096 tokens the call runs as two groups of 16
(64 slices: four groups of 16); a call on 16 slices alone runs as one group
with the same launch plan per slice, so the pipelined call must equal the
per-group calls bit for bit.  Slices of each group are also checked against
the oracle (anima_rt's flash attention, bit-identical to the reference) at
the stated tolerances.
"""
import numpy as np
import pytest

import oracle
from anima_hip import rt

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


@pytest.mark.parametrize("mode", [rt.F32, rt.F32X3, rt.BF16])
def test_two_group_call_equals_the_half_calls(mode):
    BH, S, D = 32, 4096, 128
    rng = np.random.default_rng(32 + mode)
    q, k, v = (rng.standard_normal((BH, S, D), dtype=np.float32) for _ in range(3))
    print(f"pipeline case BH={BH} S={S} mode={mode}", flush=True)
    full = rt.sdpa(q, k, v, mode=mode)
    halves = np.concatenate([rt.sdpa(q[:16], k[:16], v[:16], mode=mode),
                             rt.sdpa(q[16:], k[16:], v[16:], mode=mode)])
    np.testing.assert_array_equal(full, halves)
    for h in (5, 27):
        ref = oracle.flash_sdpa(q[h:h + 1], k[h:h + 1], v[h:h + 1], threads=4)[0]
        err = float(np.abs(full[h] - ref).max())
        print(f"pipeline mode={mode} head {h}: max-abs {err:.3e}", flush=True)
        if mode == rt.BF16:
            assert err <= 2e-2 * float(np.abs(ref).max())
        else:
            assert err <= 1e-4


def _check_slices(out, q, k, v, heads, mode, what):
    for h in heads:
        ref = oracle.flash_sdpa(q[h:h + 1], k[h:h + 1], v[h:h + 1], threads=4)[0]
        err = float(np.abs(out[h] - ref).max())
        print(f"{what} mode={mode} head {h}: max-abs {err:.3e}", flush=True)
        if mode == rt.BF16:
            assert err <= 2e-2 * float(np.abs(ref).max())
        else:
            assert err <= 1e-4


@pytest.mark.parametrize("mode", [rt.F32X3, rt.BF16])
def test_four_group_call_equals_the_group_calls(mode):
    """64 slices of 4096 tokens: four groups of 16, the first groups'
    downloads overlapping the later groups' uploads."""
    BH, S, D = 64, 4096, 128
    rng = np.random.default_rng(96 + mode)
    q, k, v = (rng.standard_normal((BH, S, D), dtype=np.float32) for _ in range(3))
    print(f"pipeline case BH={BH} S={S} mode={mode}", flush=True)
    full = rt.sdpa(q, k, v, mode=mode)
    for g in range(4):
        sl = slice(16 * g, 16 * g + 16)
        np.testing.assert_array_equal(full[sl], rt.sdpa(q[sl], k[sl], v[sl], mode=mode))
    _check_slices(full, q, k, v, (2, 63), mode, "four groups")


@pytest.mark.parametrize("mode", [rt.F32, rt.F32X3])
def test_two_group_call_with_ragged_chunks(mode):
    """4000 query and 1000 key tokens: every copy ends in a partial 16 MiB
    staging chunk, and the K/V pieces differ in size from the Q/O pieces."""
    BH, Sq, Sk, D = 32, 4000, 1000, 128
    rng = np.random.default_rng(128 + mode)
    q = rng.standard_normal((BH, Sq, D), dtype=np.float32)
    k, v = (rng.standard_normal((BH, Sk, D), dtype=np.float32) for _ in range(2))
    print(f"pipeline case BH={BH} Sq={Sq} Sk={Sk} mode={mode}", flush=True)
    full = rt.sdpa(q, k, v, mode=mode)
    halves = np.concatenate([rt.sdpa(q[:16], k[:16], v[:16], mode=mode),
                             rt.sdpa(q[16:], k[16:], v[16:], mode=mode)])
    np.testing.assert_array_equal(full, halves)
    _check_slices(full, q, k, v, (0, 31), mode, "ragged groups")
    # The same call again: staging slots and events carry over between calls.
    np.testing.assert_array_equal(rt.sdpa(q, k, v, mode=mode), full)


@pytest.mark.parametrize("mode", [rt.F32, rt.F32X3, rt.BF16])
def test_attention_two_batch_groups_equal_the_single_batch_calls(mode):
    """anima_hip_attention at B=2, 4096 tokens, H=16 (RMSNorm + 3D RoPE)
    runs as two batch groups; each must equal a B=1 call bit for bit."""
    from anima_hip.rope import generate_rope_freqs
    B, S, H, D = 2, 4096, 16, 128
    rng = np.random.default_rng(64 + mode)
    q, k, v = (rng.standard_normal((B, S, H, D), dtype=np.float32) for _ in range(3))
    wq = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    wk = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    f = generate_rope_freqs(64, 64)
    print(f"pipeline attention case B={B} S={S} mode={mode}", flush=True)
    full = rt.attention(q, k, v, wq, wk, f, mode=mode)
    for b in range(B):
        one = rt.attention(q[b:b + 1], k[b:b + 1], v[b:b + 1], wq, wk, f, mode=mode)
        np.testing.assert_array_equal(full[b:b + 1], one)
    for b, h in ((0, 3), (1, 12)):
        ref = oracle.attention_dataflow(q[b:b + 1, :, h:h + 1], k[b:b + 1, :, h:h + 1],
                                        v[b:b + 1, :, h:h + 1], wq, wk, f)[0, :, 0]
        err = float(np.abs(full[b, :, h] - ref).max())
        print(f"pipeline attention mode={mode} b={b} h={h}: max-abs {err:.3e}", flush=True)
        if mode == rt.BF16:
            assert err <= 2e-2 * float(np.abs(ref).max())
        else:
            assert err <= 1e-4


def test_attention_four_batch_groups_equal_the_single_batch_calls():
    """anima_hip_attention at B=4, 4096 tokens, H=16 (RMSNorm + 3D RoPE) runs
    as four batch groups; each must equal a B=1 call bit for bit (f32x3)."""
    from anima_hip.rope import generate_rope_freqs
    B, S, H, D = 4, 4096, 16, 128
    mode = rt.F32X3
    rng = np.random.default_rng(256)
    q, k, v = (rng.standard_normal((B, S, H, D), dtype=np.float32) for _ in range(3))
    wq = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    wk = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    f = generate_rope_freqs(64, 64)
    print(f"pipeline attention case B={B} S={S} mode={mode}", flush=True)
    full = rt.attention(q, k, v, wq, wk, f, mode=mode)
    for b in range(B):
        one = rt.attention(q[b:b + 1], k[b:b + 1], v[b:b + 1], wq, wk, f, mode=mode)
        np.testing.assert_array_equal(full[b:b + 1], one)
    ref = oracle.attention_dataflow(q[3:4, :, 9:10], k[3:4, :, 9:10], v[3:4, :, 9:10], wq, wk,
                                    f)[0, :, 0]
    err = float(np.abs(full[3, :, 9] - ref).max())
    print(f"pipeline attention four groups b=3 h=9: max-abs {err:.3e}", flush=True)
    assert err <= 1e-4
