"""Host <-> device copies of the host-pointer entries, which go through pinned
staging from 4 MiB up (16 MiB chunks, 4 pinned slots, a pool of host copy
threads).

RoPE with the identity table (cos 1, sin 0) returns its input bit for bit,
so anima_rt_run_rope checks every byte of an upload and a download.  Sizes
sit below, at and across the chunk and slot boundaries (the largest spans
six chunks, more than the four slots), include byte counts that are not
multiples of 64, and each runs twice with other data, so a slot that still
held an earlier call's bytes would show.
"""
import numpy as np
import pytest

from anima_hip import rt

pytestmark = pytest.mark.gpu

MiB = 1 << 20


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


def identity_freqs(D):
    f = np.zeros((1, D // 2, 2, 2), np.float32)
    f[..., 0, 0] = f[..., 1, 1] = 1.0
    f[..., 0, 1] = -0.0
    return f


@pytest.mark.parametrize("nbytes,D", [(4 * MiB - 512, 128), (4 * MiB + 512, 128),
                                      (16 * MiB + 512, 128), (80 * MiB + 512, 128),
                                      (8 * MiB + 24, 2)])
def test_staged_round_trip_is_bit_exact(nbytes, D):
    N = nbytes // (4 * D)
    assert N * 4 * D == nbytes
    f = identity_freqs(D)
    for seed in (1, 2):
        x = np.random.default_rng(seed * 1000 + D).standard_normal((N, 1, D), dtype=np.float32)
        x[x == 0] = 1.0  # x*1 + y*(-0) == x holds for every non-zero x
        print(f"staging case bytes={nbytes} D={D} seed={seed}", flush=True)
        np.testing.assert_array_equal(rt.rope(x, f), x)
