"""Write tests/golden/rope_ref_tables.npz with the reference's own RoPE table
builder, numpy_dit._generate_rope_freqs (anima_rt/scripts/numpy_dit.py:48-60),
imported from the reference tree in this container only.

The table's float32 bits depend on numpy's float32 pow, cos and sin inside
that function, which no closed form pins bit for bit.  Stored per grid
(T=1, head_dim 128): the 16x16 table whole (256 tokens, config 1), and for
the 64x64 (config 3, 4096 tokens) and 96x64 (config 5, 6144 tokens) tables,
which are 4 and 6 MiB, their SHA-256 digest plus the rows of tokens
(h, 0) and (0, w), which carry every distinct height and width angle.

Run:  python tests/golden/make_rope_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "rope_ref_tables.npz")
REF_SCRIPTS = "/root/reference/anima_rt/scripts"
GRIDS = [(16, 16), (64, 64), (96, 64)]


def main():
    sys.path.insert(0, REF_SCRIPTS)
    import numpy_dit as nd

    vec = {}
    for H, W in GRIDS:
        t = np.ascontiguousarray(nd._generate_rope_freqs(H, W, 1, 128), np.float32)
        assert t.shape == (H * W, 64, 2, 2)
        key = f"{H}x{W}"
        vec[f"sha256_{key}"] = np.array(hashlib.sha256(t.tobytes()).hexdigest())
        vec[f"col0_{key}"] = t.reshape(H, W, 64, 2, 2)[:, 0]   # tokens (h, 0)
        vec[f"row0_{key}"] = t.reshape(H, W, 64, 2, 2)[0, :]   # tokens (0, w)
        if H * W <= 256:
            vec[f"table_{key}"] = t
    np.savez_compressed(OUT, **vec)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(vec)} arrays)")


if __name__ == "__main__":
    main()
