"""Seeded sweep of random attention shapes through the drop-in SDPA in every
arithmetic mode, against the oracle (anima_rt's flash attention restated,
bit-identical to the reference).

Shapes mix short and tile-crossing lengths (1 .. 900 keys, 1 .. 700 queries),
1 .. 6 (batch, head) slices, causal and not; the f32 mode also takes head
dims other than 128 (its generic kernel).  Tolerances are the stated ones:
max-abs 1e-4 for the f32 and f32x3 paths, normwise 2e-2 for bf16 inputs.
"""
import numpy as np
import pytest

import oracle
from anima_hip import rt

pytestmark = pytest.mark.gpu

N_CASES = 12


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


def _cases(seed, any_d):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(N_CASES):
        bh = int(rng.integers(1, 7))
        sq = int(rng.choice([1, 31, 64, 65, 200, 333, 700]))
        sk = int(rng.choice([1, 17, 64, 100, 257, 513, 900]))
        d = int(rng.choice([32, 80, 128, 160])) if any_d else 128
        out.append((bh, sq, sk, d, bool(rng.integers(0, 2)), int(rng.integers(1 << 30))))
    return out


@pytest.mark.parametrize("mode,seed,any_d", [(rt.F32, 9101, True), (rt.F32X3, 9102, False),
                                             (rt.BF16, 9103, False)])
def test_random_shapes(mode, seed, any_d):
    for bh, sq, sk, d, causal, s in _cases(seed, any_d):
        rng = np.random.default_rng(s)
        q = rng.standard_normal((bh, sq, d), dtype=np.float32)
        k = rng.standard_normal((bh, sk, d), dtype=np.float32)
        v = rng.standard_normal((bh, sk, d), dtype=np.float32)
        print(f"sweep mode={mode} bh={bh} sq={sq} sk={sk} d={d} causal={causal}", flush=True)
        out = rt.sdpa(q, k, v, is_causal=causal, mode=mode)
        ref = oracle.flash_sdpa(q, k, v, is_causal=causal, threads=4)
        assert np.isfinite(out).all()
        err = float(np.abs(out - ref).max())
        if mode == rt.BF16:
            assert err <= 2e-2 * float(np.abs(ref).max()), err
        else:
            assert err <= 1e-4, err
