"""Seeded synthetic weights for DiT tests, named like the reference's checkpoint.

The golden DiT fixture (dit_ref_vectors.npz, written by make_dit_golden.py)
stores only inputs and outputs; the weights are regenerated from the seed by
this module, identically wherever numpy's PCG64 stream is the same.

Every tensor the forward needs (numpy_dit.py:67-80, 145-317):
linear weights as bf16 bit patterns [out, in] drawn N(0, 0.02) in float32 and
rounded to nearest even; norm weights as bf16-representable float32 vectors
around 1 (1 + N(0, 0.1)), stored here as float32 like the reference's widened
norm weights.
"""
import numpy as np

ADA_HIDDEN = 256


def shapes(dim, blocks, heads, head_dim, mlp_hidden, ctx_dim, in_ch=16, out_ch=16):
    """Ordered {name: shape} of the model's tensors."""
    hd = heads * head_dim
    s = {"x_embedder.proj.1.weight": (dim, (in_ch + 1) * 4),
         "t_embedder.1.linear_1.weight": (dim, dim),
         "t_embedder.1.linear_2.weight": (3 * dim, dim),
         "t_embedding_norm.weight": (dim,)}
    for i in range(blocks):
        p = f"blocks.{i}."
        for a, kv_in in (("self_attn", dim), ("cross_attn", ctx_dim)):
            s[p + a + ".q_proj.weight"] = (hd, dim)
            s[p + a + ".k_proj.weight"] = (hd, kv_in)
            s[p + a + ".v_proj.weight"] = (hd, kv_in)
            s[p + a + ".output_proj.weight"] = (dim, hd)
            s[p + a + ".q_norm.weight"] = (head_dim,)
            s[p + a + ".k_norm.weight"] = (head_dim,)
        s[p + "mlp.layer1.weight"] = (mlp_hidden, dim)
        s[p + "mlp.layer2.weight"] = (dim, mlp_hidden)
        for sub in ("self_attn", "cross_attn", "mlp"):
            s[p + f"adaln_modulation_{sub}.1.weight"] = (ADA_HIDDEN, dim)
            s[p + f"adaln_modulation_{sub}.2.weight"] = (3 * dim, ADA_HIDDEN)
    s["final_layer.adaln_modulation.1.weight"] = (ADA_HIDDEN, dim)
    s["final_layer.adaln_modulation.2.weight"] = (2 * dim, ADA_HIDDEN)
    s["final_layer.linear.weight"] = (4 * out_ch, dim)
    return s


def _bf16_bits(x):
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFFFFFF
    return (b >> 16).astype(np.uint16)


def make(seed, **cfg):
    """{name: array}: uint16 bf16 bits for matrices, float32 for vectors."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shp in shapes(**cfg).items():
        if len(shp) == 1:
            v = np.float32(1.0) + rng.standard_normal(shp, dtype=np.float32) * np.float32(0.1)
            out[name] = (_bf16_bits(v).astype(np.uint32) << 16).view(np.float32)
        else:
            out[name] = _bf16_bits(rng.standard_normal(shp, dtype=np.float32) * np.float32(0.02))
    return out
