"""The drop-in's host-pointer entries called from several threads at once.

The reference library is single-threaded (anima_rt.cpp keeps one global
backend), and its binding is called from one Python thread.  The replacement
promises thread-safe initialisation and serialises its shared staging behind
a lock, so concurrent callers must each get exactly the result of the same
call made alone (the kernels are deterministic: no atomics, fixed split
orders).  ctypes releases the GIL for the duration of each foreign call, so
the threads below really overlap inside the library.
"""
import threading

import numpy as np
import pytest

from anima_hip import rt
from anima_hip.rope import generate_rope_freqs

pytestmark = pytest.mark.gpu

N_THREADS = 6
ROUNDS = 3


def _calls():
    """A mix of host entries on small seeded inputs: name -> zero-argument call."""
    rng = np.random.default_rng(2024)
    bh, s, d = 8, 384, 128
    q, k, v = (rng.standard_normal((bh, s, d), dtype=np.float32) for _ in range(3))
    B, S, H = 1, 256, 4
    qa, ka, va = (rng.standard_normal((B, S, H, d), dtype=np.float32) for _ in range(3))
    freqs = generate_rope_freqs(16, 16)
    x = rng.standard_normal((512, d), dtype=np.float32)
    w = rng.standard_normal(d, dtype=np.float32)
    ctx = rng.standard_normal((1, 64, 256), dtype=np.float32) * np.float32(0.5)
    wk = rng.standard_normal((H * d, 256), dtype=np.float32) * np.float32(0.02)
    wv = rng.standard_normal((H * d, 256), dtype=np.float32) * np.float32(0.02)

    def bits(a):
        u = a.view(np.uint32).astype(np.uint64)
        return (((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF) >> 16).astype(np.uint16)

    cache = rt.ContextKV(ctx, bits(wk), bits(wv), np.ones(d, np.float32), heads=H, head_dim=d,
                         mode=rt.F32X3)
    calls = {
        "sdpa_flash": lambda: rt.sdpa_flash(q, k, v),
        "sdpa_flash_causal": lambda: rt.sdpa_flash(q, k, v, is_causal=True),
        "sdpa_bf16": lambda: rt.sdpa(q, k, v, mode=rt.BF16),
        "sdpa_f32x3": lambda: rt.sdpa(q, k, v, mode=rt.F32X3),
        "attention_rope_f32x3": lambda: rt.attention(qa, ka, va, freqs=freqs, mode=rt.F32X3),
        "rmsnorm": lambda: rt.rmsnorm(x, w),
        "cross_f32x3": lambda: cache.attend(qa),
    }
    return calls, cache


def test_concurrent_host_calls_equal_calls_made_alone():
    # Initialisation itself from several threads at once.
    inits = [threading.Thread(target=rt.init) for _ in range(N_THREADS)]
    for t in inits:
        t.start()
    for t in inits:
        t.join()
    calls, cache = _calls()
    try:
        alone = {name: fn() for name, fn in calls.items()}
        names = list(calls)
        errors, mismatches = [], []

        def worker(tid):
            try:
                for r in range(ROUNDS):
                    # Each thread walks the calls in its own rotation, so
                    # different entries overlap.
                    for i in range(len(names)):
                        name = names[(i + tid + r) % len(names)]
                        out = calls[name]()
                        if not np.array_equal(out.view(np.uint32), alone[name].view(np.uint32)):
                            mismatches.append((tid, r, name))
            except Exception as e:  # reported below, not swallowed
                errors.append((tid, repr(e)))

        threads = [threading.Thread(target=worker, args=(t,)) for t in range(N_THREADS)]
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=120)
        assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
        assert not errors, errors
        assert not mismatches, mismatches[:5]
    finally:
        cache.close()
