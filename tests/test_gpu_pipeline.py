"""The host-pointer SDPA's two-group pipeline (the second half of the heads
uploads while the first half computes on a second stream).

At 32 (batch, head) slices of 4096 tokens the call runs as two groups of 16;
a call on 16 slices alone runs as one group with the same launch plan per
slice, so the pipelined call must equal the two half calls bit for bit.  One
slice of each group is also checked against the oracle (anima_rt's flash
attention, bit-identical to the reference) at the stated tolerances.
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
