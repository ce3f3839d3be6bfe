"""Host-side 3D RoPE table for the DiT's self-attention.

Builds the [T*H*W, head_dim/2, 2, 2] rotation table the attention prologue
consumes, exactly as NumpyDiT's host code does
(anima_rt/scripts/numpy_dit.py:48-60, which mirrors
VideoRopePosition3DEmb.generate_embeddings, src/position_embedding.py:100-163):

  * head_dim splits into a temporal block of dim_t = head_dim - 2*dim_h
    channels and two spatial blocks of dim_h = dim_w = head_dim//6*2;
  * frequencies base^(-2j/dim) with base 1e4 for time and
    1e4 * 4^(dim/(dim-2)) (NTK extrapolation ratio 4) for height and width;
  * entry [cos a, -sin a, sin a, cos a] with a = position * frequency;
  * token order (t, h, w) row-major -- the rectangular H x W grid is honoured
    (no square-grid assumption).
All arithmetic is numpy float32, as in the reference's host code, so the
table matches it element for element.
"""
from __future__ import annotations

import numpy as np


def _axis_freqs(base: float, dim: int) -> np.ndarray:
    exponents = np.arange(0, dim, 2, dtype=np.float32)[: dim // 2] / dim
    return 1.0 / (base ** exponents)


def _rotation(angles: np.ndarray) -> np.ndarray:
    c = np.cos(angles)
    s = np.sin(angles)
    return np.stack([c, -s, s, c], axis=-1)


def generate_rope_freqs(H: int, W: int, T: int = 1, head_dim: int = 128) -> np.ndarray:
    """Rotation table [T*H*W, head_dim/2, 2, 2] float32 for a T x H x W token grid."""
    if head_dim % 2:
        raise ValueError("head_dim must be even")
    dim_h = head_dim // 6 * 2
    dim_t = head_dim - 2 * dim_h
    spatial_base = 10000.0 * 4.0 ** (dim_h / (dim_h - 2))
    blocks = [
        (_rotation(np.outer(np.arange(T, dtype=np.float32), _axis_freqs(10000.0, dim_t))), 0),
        (_rotation(np.outer(np.arange(H, dtype=np.float32), _axis_freqs(spatial_base, dim_h))), 1),
        (_rotation(np.outer(np.arange(W, dtype=np.float32), _axis_freqs(spatial_base, dim_h))), 2),
    ]
    parts = []
    for rot, axis in blocks:
        shape = [1, 1, 1, rot.shape[1], 4]
        shape[axis] = rot.shape[0]
        parts.append(np.broadcast_to(rot.reshape(shape), (T, H, W, rot.shape[1], 4)))
    table = np.concatenate(parts, axis=3).astype(np.float32, copy=False)
    return np.ascontiguousarray(table.reshape(T * H * W, head_dim // 2, 2, 2))
