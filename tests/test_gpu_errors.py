"""Error paths of the host-pointer entries on a GPU: an allocation failure,
injected through ANIMA_HIP_FAIL_ALLOC, makes the C-ABI return false with a
message and the Python layer raise AnimaHipError instead of returning the
zeros that NumpyRT.run_sdpa would leave (scripts/phone_pipeline_nd.py:67
ignores the result); once the failure is gone the same calls succeed and
match the oracle (max-abs 1e-4)."""
import os

import numpy as np
import pytest

import oracle
from anima_hip import AnimaHipError, rt

pytestmark = pytest.mark.gpu


@pytest.fixture()
def fresh_runtime():
    rt.destroy()  # frees the workspace, so the next call must allocate
    yield
    os.environ.pop("ANIMA_HIP_FAIL_ALLOC", None)
    rt.init()


def test_injected_allocation_failure_raises_then_recovers(fresh_runtime):
    rng = np.random.default_rng(99)
    q, k, v = (rng.standard_normal((4, 77, 128), dtype=np.float32) for _ in range(3))
    x = rng.standard_normal((3, 128), dtype=np.float32)
    rt.init()
    os.environ["ANIMA_HIP_FAIL_ALLOC"] = "1"
    print("injected allocation failure: sdpa_flash, sdpa(f32x3), rmsnorm", flush=True)
    with pytest.raises(AnimaHipError, match="injected"):
        rt.sdpa_flash(q, k, v)
    with pytest.raises(AnimaHipError, match="injected"):
        rt.sdpa(q, k, v, mode=rt.F32X3)
    with pytest.raises(AnimaHipError, match="injected"):
        rt.rmsnorm(x)
    del os.environ["ANIMA_HIP_FAIL_ALLOC"]
    print("recovery after the failure", flush=True)
    ref = oracle.flash_sdpa(q, k, v, threads=4)
    for mode in (rt.F32, rt.F32X3):
        out = rt.sdpa(q, k, v, mode=mode)
        assert np.abs(out - ref).max() <= 1e-4
    np.testing.assert_array_equal(rt.rmsnorm(x), oracle.rmsnorm(x, None, 1e-6))
