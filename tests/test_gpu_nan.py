"""NaN inputs: the GPU kernels reproduce the reference's pattern.

anima_rt's flash attention (flash_attention.h:145-201) skips a query row
whose every score is NaN (its max test `s > row_max` never passes), so that
row keeps the zeros the output was filled with; a NaN key makes every score
of its head's rows NaN-tainted, so the whole head becomes NaN; a NaN value
element taints its column.  The oracle restates this bit for bit against the
compiled reference (tests/test_oracle_ref.py).  Here each arithmetic mode,
on the split-KV launch shape (few heads) and on the 8-wave grid (many
heads), must produce NaN exactly where the oracle does, zeros where it
does, and agree elsewhere within the mode's tolerance (max-abs 1e-4 for f32
and f32x3, normwise 2e-2 for bf16).
"""
import numpy as np
import pytest

import oracle
from anima_hip import rt

pytestmark = pytest.mark.gpu

SCALE = 0.088


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


def _case(where, bh, s, d, seed):
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal((bh, s, d)).astype(np.float32) for _ in range(3))
    t = {"q_row": q, "k_row": k, "v_elem": v}[where]
    t[0, 40, 7] = np.nan
    t[bh - 1, s - 3, d - 1] = np.nan
    return q, k, v


@pytest.mark.parametrize("where", ["q_row", "k_row", "v_elem"])
@pytest.mark.parametrize("bh,s,d,modes", [
    (2, 1000, 128, (rt.F32, rt.F32X3, rt.BF16)),   # split-KV partials + combine
    (256, 300, 128, (rt.F32, rt.F32X3, rt.BF16)),  # 8-wave grid, ragged tail
    (3, 130, 80, (rt.F32,)),                      # generic kernel (D != 128)
])
def test_nan_pattern_matches_reference(where, bh, s, d, modes):
    q, k, v = _case(where, bh, s, d, bh + s + d)
    ref = oracle.flash_sdpa(q, k, v, SCALE, threads=8)
    nan = np.isnan(ref)
    if where == "q_row":  # the two all-NaN rows are zeros, nothing is NaN
        assert not nan.any() and np.all(ref[0, 40] == 0) and np.all(ref[bh - 1, s - 3] == 0)
    else:
        assert nan.any()
    for mode in modes:
        print(f"NaN in {where}: bh={bh} s={s} d={d} mode={mode}", flush=True)
        out = rt.sdpa(q, k, v, scale=SCALE, mode=mode)
        np.testing.assert_array_equal(np.isnan(out), nan)
        np.testing.assert_array_equal(out[ref == 0], 0.0)
        if nan.all():  # NaN keys in every head
            continue
        err = float(np.abs(out[~nan] - ref[~nan]).max())
        if mode == rt.BF16:
            err /= float(np.abs(ref[~nan]).max())
        assert err <= (2e-2 if mode == rt.BF16 else 1e-4), (mode, err)
