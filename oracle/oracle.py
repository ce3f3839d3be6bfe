"""CPU oracle for the Anima DiT attention hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker.  The product (``anima_hip`` + ``libanima_hip.so``) never imports it
and has no CPU fallback.

Contents
  * ctypes wrappers over ``liboracle.so`` (``anima_oracle.c``): the plain-C
    restatement of anima_rt's flash SDPA, math SDPA, RMSNorm, RoPE, bf16
    GEMM, LayerNorm and SiLU, bit-identical to the reference runtime, and the
    float32 AdaLN modulate / gated residual of NumpyBlock.forward.
  * ctypes wrappers over ``_ref/libanima_rt_ref.so``: the reference runtime
    itself, compiled from its sources (present only where it was built).
  * numpy restatements of the NumpyDiT host pieces: the 3D RoPE table
    (anima_rt/scripts/numpy_dit.py:48-60), the rotate-half application
    (numpy_dit.py:33-37) and the attention dataflow of
    NumpyAttention.forward (numpy_dit.py:268-297).
  * fp64 brute-force SDPA / RMSNorm / RoPE used to pin the above.

Pinning status (each function is checked by something other than itself):
  flash_sdpa, math_sdpa, rmsnorm, rope -- bit-identical to the compiled
      reference (tests/test_oracle_ref.py) and to fp64 closed forms.
  rope_freqs -- closed form in fp64 (angle = pos * theta^(-2j/dim)), the
      [cos,-sin,sin,cos] entry layout, identity on temporal pairs for T=1,
      and the reference's D=4 known-answer test; bit-for-bit equality with
      numpy_dit.py's float32 rounding is "parity unpinned" (would need an
      import of the reference) and is covered only to 1 ulp-level tolerance.
  numpy_rope -- same arithmetic as rope (checked bit-identical against it).
  layernorm, silu, gelu, softmax -- bit-identical to the compiled reference
      and the golden vectors it wrote; fp64 two-pass moments, x/(1+exp(-x)),
      x*Phi(x), exp(x - max)/sum.
  timesteps, patchify, unpatchify, adaln, mlp_block, dit_forward,
  z_image_sigmas, euler_sample -- bit-identical to the reference's own
      numpy_dit.py / sampling.py on tests/golden/dit_ref_vectors.npz; closed
      forms and index identities.
  modulate, gate_residual -- fp64 evaluation within float32 rounding, and
      closed cases (scale = shift = 0 is identity, gate = 0 keeps x).
  attention_block -- composition of the pinned pieces above.
"""
from __future__ import annotations

import ctypes as _ct
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libanima_rt_ref.so")

_P = _ct.c_void_p
_I = _ct.c_int
_F = _ct.c_float


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _f32c(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


_oracle_lib = None
_ref_lib = None


def oracle_lib():
    """Load liboracle.so (built by `make -C oracle`)."""
    global _oracle_lib
    if _oracle_lib is None:
        if not os.path.exists(ORACLE_SO):
            raise FileNotFoundError(f"{ORACLE_SO} missing: run `make -C oracle`")
        lib = _ct.CDLL(ORACLE_SO)
        sig = [_P] * 4 + [_I] * 4 + [_F, _I]
        lib.oracle_flash_attention.argtypes = sig
        lib.oracle_flash_attention.restype = _I
        lib.oracle_flash_attention_mt.argtypes = sig + [_I]
        lib.oracle_flash_attention_mt.restype = _I
        lib.oracle_sdpa_math.argtypes = sig
        lib.oracle_sdpa_math.restype = _I
        lib.oracle_rmsnorm.argtypes = [_P, _P, _P, _ct.c_int64, _ct.c_int64, _F]
        lib.oracle_rmsnorm.restype = None
        lib.oracle_rope.argtypes = [_P, _P, _P, _I, _I, _I]
        lib.oracle_rope.restype = None
        lib.oracle_gemm_bf16.argtypes = [_P, _P, _P, _I, _I, _I]
        lib.oracle_gemm_bf16.restype = None
        lib.oracle_f32_to_bf16.argtypes = [_F]
        lib.oracle_f32_to_bf16.restype = _ct.c_uint16
        lib.oracle_layernorm.argtypes = [_P, _P, _ct.c_int64, _ct.c_int64, _F]
        lib.oracle_layernorm.restype = None
        lib.oracle_silu.argtypes = [_P, _P, _ct.c_int64]
        lib.oracle_silu.restype = None
        lib.oracle_gelu.argtypes = [_P, _P, _ct.c_int64]
        lib.oracle_gelu.restype = None
        lib.oracle_softmax.argtypes = [_P, _P, _ct.c_int64, _ct.c_int64]
        lib.oracle_softmax.restype = None
        lib.oracle_modulate.argtypes = [_P, _P, _P, _P, _I, _ct.c_int64, _ct.c_int64]
        lib.oracle_modulate.restype = None
        lib.oracle_gate_residual.argtypes = [_P, _P, _P, _I, _ct.c_int64, _ct.c_int64]
        lib.oracle_gate_residual.restype = None
        _oracle_lib = lib
    return _oracle_lib


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref_lib():
    """Load the reference runtime compiled from its own sources (oracle/_ref)."""
    global _ref_lib
    if _ref_lib is None:
        lib = _ct.CDLL(REF_SO)
        sig = [_P] * 4 + [_I] * 4 + [_F, _ct.c_bool]
        lib.anima_rt_init.restype = _ct.c_bool
        lib.anima_rt_run_sdpa_flash.argtypes = sig
        lib.anima_rt_run_sdpa_flash.restype = _ct.c_bool
        lib.anima_rt_run_sdpa.argtypes = sig
        lib.anima_rt_run_sdpa.restype = _ct.c_bool
        lib.anima_rt_run_rmsnorm.argtypes = [_P, _P, _P, _I, _I, _F]
        lib.anima_rt_run_rmsnorm.restype = _ct.c_bool
        lib.anima_rt_run_rope.argtypes = [_P, _P, _P, _I, _I, _I]
        lib.anima_rt_run_rope.restype = _ct.c_bool
        lib.anima_rt_run_gemm_bf16.argtypes = [_P, _P, _P, _I, _I, _I]
        lib.anima_rt_run_gemm_bf16.restype = _ct.c_bool
        lib.anima_rt_run_layernorm.argtypes = [_P, _P, _I, _I, _F]
        lib.anima_rt_run_layernorm.restype = _ct.c_bool
        lib.anima_rt_run_silu.argtypes = [_P, _P, _I]
        lib.anima_rt_run_silu.restype = _ct.c_bool
        lib.anima_rt_run_gelu.argtypes = [_P, _P, _I]
        lib.anima_rt_run_gelu.restype = _ct.c_bool
        lib.anima_rt_run_softmax.argtypes = [_P, _P, _I, _I]
        lib.anima_rt_run_softmax.restype = _ct.c_bool
        if not lib.anima_rt_init():
            raise RuntimeError("reference anima_rt_init failed")
        _ref_lib = lib
    return _ref_lib


# ---------------------------------------------------------------- C oracle

def flash_sdpa(q, k, v, scale=None, is_causal=False, threads=1):
    """anima_rt flash SDPA restated (flash_attention.h:55-208).

    q: [BH,Sq,D], k/v: [BH,Sk,D] float32.  Returns [BH,Sq,D] float32."""
    q, k, v = _f32c(q), _f32c(k), _f32c(v)
    BH, Sq, D = q.shape
    Sk = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    o = np.zeros((BH, Sq, D), np.float32)
    lib = oracle_lib()
    if threads > 1:
        ok = lib.oracle_flash_attention_mt(_ptr(q), _ptr(k), _ptr(v), _ptr(o), BH, Sq, Sk,
                                           D, scale, int(is_causal), int(threads))
    else:
        ok = lib.oracle_flash_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(o), BH, Sq, Sk, D,
                                        scale, int(is_causal))
    if not ok:
        raise MemoryError("oracle_flash_attention failed")
    return o


def math_sdpa(q, k, v, scale=None, is_causal=False):
    """anima_rt math SDPA restated (anima_rt.cpp:78-141): softmax(scale^2 QK^T) V."""
    q, k, v = _f32c(q), _f32c(k), _f32c(v)
    BH, Sq, D = q.shape
    Sk = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    o = np.zeros((BH, Sq, D), np.float32)
    if not oracle_lib().oracle_sdpa_math(_ptr(q), _ptr(k), _ptr(v), _ptr(o), BH, Sq, Sk, D,
                                         scale, int(is_causal)):
        raise MemoryError("oracle_sdpa_math failed")
    return o


def rmsnorm(x, w=None, eps=1e-6):
    """RMSNorm over the last axis restated (rmsnorm_kernel.h:11-31)."""
    x = _f32c(x)
    D = x.shape[-1]
    M = x.size // D
    y = np.empty_like(x)
    wp = None
    if w is not None:
        w = _f32c(w)
        wp = _ptr(w)
    oracle_lib().oracle_rmsnorm(_ptr(x), wp, _ptr(y), M, D, eps)
    return y


def layernorm(x, eps=1e-6):
    """LayerNorm without affine over the last axis restated
    (anima_rt_run_layernorm -> layernorm_kernel.h:13-33, welford.h:15-31)."""
    x = _f32c(x)
    D = x.shape[-1]
    y = np.empty_like(x)
    oracle_lib().oracle_layernorm(_ptr(x), _ptr(y), x.size // D, D, eps)
    return y


def silu(x):
    """SiLU restated (silu_kernel.h:11-20)."""
    x = _f32c(x)
    y = np.empty_like(x)
    oracle_lib().oracle_silu(_ptr(x), _ptr(y), x.size)
    return y


def gelu(x):
    """GELU, exact erf form, restated (gelu_kernel.h:13-23)."""
    x = _f32c(x)
    y = np.empty_like(x)
    oracle_lib().oracle_gelu(_ptr(x), _ptr(y), x.size)
    return y


def softmax(x):
    """Softmax over the last axis restated (softmax_kernel.h:16-40)."""
    x = _f32c(x)
    D = x.shape[-1]
    y = np.empty_like(x)
    oracle_lib().oracle_softmax(_ptr(x), _ptr(y), x.size // D, D)
    return y


def modulate(xn, scale, shift):
    """x_n*(1.0 + scale) + shift in float32 (numpy_dit.py:238); xn [B,S,D],
    scale/shift [B,D]."""
    xn, scale, shift = _f32c(xn), _f32c(scale), _f32c(shift)
    B, S, D = xn.shape
    y = np.empty_like(xn)
    oracle_lib().oracle_modulate(_ptr(xn), _ptr(scale), _ptr(shift), _ptr(y), B, S, D)
    return y


def gate_residual(x, gate, out):
    """x + gate*out in float32 (numpy_dit.py:240); x/out [B,S,D], gate [B,D]."""
    x = _f32c(x).copy()
    gate, out = _f32c(gate), _f32c(out)
    B, S, D = x.shape
    oracle_lib().oracle_gate_residual(_ptr(x), _ptr(gate), _ptr(out), B, S, D)
    return x


def attention_block(x, mod, wq, wk, wv, wo, q_norm_w, k_norm_w, freqs=None, ctx=None,
                    heads=16, head_dim=128, eps=1e-6, sdpa=None):
    """One attention sub-block of NumpyBlock.forward (numpy_dit.py:236-247):
    x + gate * output_proj(attention(layernorm(x)*(1+scale) + shift)).
    x [B,S,Dm]; mod [B,3,Dm] = (shift, scale, gate); w* bf16 bit patterns
    [out, in]; self-attention when ctx is None (K/V from the modulated x,
    RoPE with freqs), else cross-attention with K/V projected from ctx
    [Bc,Sk,C] (Bc 1 broadcasts over the batch) and no RoPE."""
    x = _f32c(x)
    B, S, Dm = x.shape
    shift, scale, gate = (np.ascontiguousarray(mod[:, i]) for i in range(3))
    xm = modulate(layernorm(x, eps), scale, shift)
    HD = heads * head_dim
    q = gemm_bf16(xm.reshape(B * S, Dm), wq).reshape(B, S, heads, head_dim)
    if ctx is None:
        k = gemm_bf16(xm.reshape(B * S, Dm), wk).reshape(B, S, heads, head_dim)
        v = gemm_bf16(xm.reshape(B * S, Dm), wv).reshape(B, S, heads, head_dim)
    else:
        ctx = _f32c(ctx)
        Bc, Sk, C = ctx.shape
        k = np.stack([gemm_bf16(ctx[b], wk) for b in range(Bc)]).reshape(Bc, Sk, heads, head_dim)
        v = np.stack([gemm_bf16(ctx[b], wv) for b in range(Bc)]).reshape(Bc, Sk, heads, head_dim)
        k = np.broadcast_to(k, (B, Sk, heads, head_dim))
        v = np.broadcast_to(v, (B, Sk, heads, head_dim))
    attn = attention_dataflow(q, k, v, q_norm_w, k_norm_w, freqs if ctx is None else None,
                              eps, sdpa)
    out = gemm_bf16(attn.reshape(B * S, HD), wo).reshape(B, S, Dm)
    return gate_residual(x, gate, out)


def rope(t, freqs):
    """Rotate-half RoPE restated (rope_kernel.h:65-97). t: [N,S,D], freqs: [S,D/2,2,2]."""
    t = _f32c(t)
    N, S, D = t.shape
    f = _f32c(freqs).reshape(S, D // 2, 2, 2)
    out = np.empty_like(t)
    oracle_lib().oracle_rope(_ptr(t), _ptr(f), _ptr(out), N, S, D)
    return out


def f32_to_bf16_bits(x) -> np.ndarray:
    """Round fp32 to bf16 (nearest-even), returning the uint16 bit patterns
    (gemm_backend.cpp:77-85), vectorised."""
    b = _f32c(x).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFFFFFF
    return (b >> 16).astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    """bf16 bits -> fp32 by a 16-bit shift (phone_pipeline_nd.py:38-40)."""
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def gemm_bf16(a, w_bits):
    """C = A . W^T with bf16 W (gemm_backend.cpp:117-131)."""
    a = _f32c(a)
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    M, K = a.shape
    N = w_bits.shape[0]
    c = np.empty((M, N), np.float32)
    oracle_lib().oracle_gemm_bf16(_ptr(a), _ptr(w_bits), _ptr(c), M, N, K)
    return c


# ------------------------------------------------------- reference runtime

def ref_flash_sdpa(q, k, v, scale=None, is_causal=False):
    q, k, v = _f32c(q), _f32c(k), _f32c(v)
    BH, Sq, D = q.shape
    Sk = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    o = np.zeros((BH, Sq, D), np.float32)
    assert ref_lib().anima_rt_run_sdpa_flash(_ptr(q), _ptr(k), _ptr(v), _ptr(o), BH, Sq, Sk,
                                             D, scale, bool(is_causal))
    return o


def ref_math_sdpa(q, k, v, scale=None, is_causal=False):
    q, k, v = _f32c(q), _f32c(k), _f32c(v)
    BH, Sq, D = q.shape
    Sk = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    o = np.zeros((BH, Sq, D), np.float32)
    assert ref_lib().anima_rt_run_sdpa(_ptr(q), _ptr(k), _ptr(v), _ptr(o), BH, Sq, Sk, D,
                                       scale, bool(is_causal))
    return o


def ref_layernorm(x, eps=1e-6):
    x = _f32c(x)
    D = x.shape[-1]
    y = np.zeros_like(x)
    assert ref_lib().anima_rt_run_layernorm(_ptr(x), _ptr(y), x.size // D, D, eps)
    return y


def ref_silu(x):
    x = _f32c(x)
    y = np.zeros_like(x)
    assert ref_lib().anima_rt_run_silu(_ptr(x), _ptr(y), x.size)
    return y


def ref_gelu(x):
    x = _f32c(x)
    y = np.zeros_like(x)
    assert ref_lib().anima_rt_run_gelu(_ptr(x), _ptr(y), x.size)
    return y


def ref_softmax(x):
    x = _f32c(x)
    D = x.shape[-1]
    y = np.zeros_like(x)
    assert ref_lib().anima_rt_run_softmax(_ptr(x), _ptr(y), x.size // D, D)
    return y


def ref_rmsnorm(x, w=None, eps=1e-6):
    x = _f32c(x)
    D = x.shape[-1]
    M = x.size // D
    y = np.zeros_like(x)
    wp = None
    if w is not None:
        w = _f32c(w)
        wp = _ptr(w)
    assert ref_lib().anima_rt_run_rmsnorm(_ptr(x), wp, _ptr(y), M, D, eps)
    return y


def ref_rope(t, freqs):
    t = _f32c(t)
    N, S, D = t.shape
    f = _f32c(freqs)
    out = np.zeros_like(t)
    assert ref_lib().anima_rt_run_rope(_ptr(t), _ptr(f), _ptr(out), N, S, D)
    return out


def ref_gemm_bf16(a, w_bits):
    a = _f32c(a)
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    M, K = a.shape
    N = w_bits.shape[0]
    c = np.zeros((M, N), np.float32)
    assert ref_lib().anima_rt_run_gemm_bf16(_ptr(a), _ptr(w_bits), _ptr(c), M, N, K)
    return c


# --------------------------------------------------------- numpy host side

def rope_freqs(H: int, W: int, T: int = 1, head_dim: int = 128) -> np.ndarray:
    """3D RoPE table [T*H*W, head_dim/2, 2, 2] as NumpyDiT builds it
    (anima_rt/scripts/numpy_dit.py:48-60, mirroring
    src/position_embedding.py:100-163).

    Pair ranges: the first dim_t/2 pairs rotate with the frame index, the next
    dim_h/2 with the row index and the last dim_w/2 with the column index,
    where dim_h = dim_w = head_dim//6*2 and dim_t = head_dim - 2*dim_h.  The
    spatial bases are 1e4 * 4^(dim/(dim-2)) (NTK extrapolation ratio 4), the
    temporal base 1e4.  Every entry is [cos a, -sin a, sin a, cos a] with
    a = position * base^(-2j/dim).  Token order is (t, h, w) row-major.
    All arithmetic is numpy float32 like the reference's host code."""
    dh = head_dim // 6 * 2
    dw = dh
    dt = head_dim - 2 * dh
    ntk_h = 4.0 ** (dh / (dh - 2))
    ntk_w = 4.0 ** (dw / (dw - 2))

    def inv_freq(base, dim):
        expo = np.arange(0, dim, 2, dtype=np.float32)[: dim // 2] / dim
        return 1.0 / (base ** expo)

    fh = inv_freq(10000.0 * ntk_h, dh)
    fw = inv_freq(10000.0 * ntk_w, dw)
    ft = inv_freq(10000.0, dt)

    def rot(angle):
        c, s = np.cos(angle), np.sin(angle)
        return np.stack([c, -s, s, c], axis=-1)

    ang_t = np.outer(np.arange(T, dtype=np.float32), ft)
    ang_h = np.outer(np.arange(H, dtype=np.float32), fh)
    ang_w = np.outer(np.arange(W, dtype=np.float32), fw)
    npair = head_dim // 2
    table = np.empty((T, H, W, npair, 4), np.float32)
    nt, nh = dt // 2, dh // 2
    table[:, :, :, :nt] = rot(ang_t)[:, None, None]
    table[:, :, :, nt:nt + nh] = rot(ang_h)[None, :, None]
    table[:, :, :, nt + nh:] = rot(ang_w)[None, None, :]
    return table.reshape(T * H * W, npair, 2, 2)


def numpy_rope(x, freqs):
    """Rotate-half RoPE on [..., S, H, D] activations with an [S, D/2, 2, 2]
    table, float32, products then one add per output
    (numpy_dit.py:33-37 == predict2.apply_rotary_pos_emb)."""
    x = np.asarray(x, np.float32)
    D = x.shape[-1]
    h = D // 2
    S = x.shape[-3]
    f = np.asarray(freqs, np.float32).reshape(S, h, 2, 2)[:, None]  # [S,1,h,2,2]
    a, b = x[..., :h], x[..., h:]
    out = np.empty_like(x)
    out[..., :h] = f[..., 0, 0] * a + f[..., 0, 1] * b
    out[..., h:] = f[..., 1, 0] * a + f[..., 1, 1] * b
    return out


def attention_dataflow(q, k, v, q_norm_w=None, k_norm_w=None, freqs=None, eps=1e-6,
                       sdpa=None):
    """The middle of NumpyAttention.forward (numpy_dit.py:283-294) on
    [B,S,H,D] projections: per-head RMSNorm of q and k (weights optional),
    RoPE on both when a table is given (self-attention only), transpose to
    [B,H,S,D], flash SDPA with scale 1/sqrt(D), transpose back.
    Returns [B,Sq,H,D] float32."""
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    qn = rmsnorm(q, q_norm_w, eps)
    kn = rmsnorm(k, k_norm_w, eps)
    if freqs is not None:
        qn = numpy_rope(qn, freqs)
        kn = numpy_rope(kn, freqs)
    qt = qn.transpose(0, 2, 1, 3).reshape(B * H, Sq, D)
    kt = kn.transpose(0, 2, 1, 3).reshape(B * H, Sk, D)
    vt = v.transpose(0, 2, 1, 3).reshape(B * H, Sk, D)
    run = sdpa or flash_sdpa
    o = run(qt, kt, vt)
    return o.reshape(B, H, Sq, D).transpose(0, 2, 1, 3).copy()


# ------------------------------------------------------------ fp64 checks

def sdpa_fp64(q, k, v, scale=None, is_causal=False):
    """Textbook softmax(scale*QK^T)V in float64 (independent of the tiling)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    D = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    s = np.einsum("bqd,bkd->bqk", q, k) * scale
    if is_causal:
        Sq, Sk = s.shape[1:]
        mask = np.arange(Sk)[None, :] > np.arange(Sq)[:, None]
        s = np.where(mask[None], -np.inf, s)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("bqk,bkd->bqd", p, v)


def rmsnorm_fp64(x, w=None, eps=1e-6):
    x = np.asarray(x, np.float64)
    y = x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    if w is not None:
        y = y * np.asarray(w, np.float64)
    return y


def rope_freqs_fp64(H: int, W: int, T: int = 1, head_dim: int = 128) -> np.ndarray:
    """The RoPE table from the closed form in float64: per pair j of each
    axis block, angle = pos * base^(-2j/dim)."""
    dh = head_dim // 6 * 2
    dt = head_dim - 2 * dh
    tab = np.empty((T, H, W, head_dim // 2), np.float64)
    bases = [(dt, 10000.0), (dh, 10000.0 * 4.0 ** (dh / (dh - 2))),
             (dh, 10000.0 * 4.0 ** (dh / (dh - 2)))]
    col = 0
    for axis, (dim, base) in enumerate(bases):
        for j in range(dim // 2):
            fr = base ** (-(2.0 * j) / dim)
            pos = [np.arange(T), np.arange(H), np.arange(W)][axis].astype(np.float64)
            shape = [1, 1, 1]
            shape[axis] = -1
            tab[..., col] = pos.reshape(shape) * fr
            col += 1
    c, s = np.cos(tab), np.sin(tab)
    return np.stack([c, -s, s, c], axis=-1).reshape(T * H * W, head_dim // 2, 2, 2)


# ------------------------------------------------- the DiT around the path
# numpy restatements of NumpyDiT's host pieces and of the Euler/CFG sampler
# (anima_rt/scripts/numpy_dit.py, anima_rt/scripts/sampling.py), composed from
# the C restatements above.  Weights are a dict name -> array: linear weights
# as bf16 bit patterns [out, in] (uint16), norm weights as float32 vectors.

PATCH = 2  # spatial patch; one frame per patch


def timesteps(sigma, dim):
    """Sinusoidal timestep features, _numpy_timesteps (numpy_dit.py:39-46):
    [cos(sigma f_i), sin(sigma f_i)] with f_i = exp(-ln(1e4) i / half), every
    operation in float32."""
    half = dim // 2
    exponent = (np.float32(-math.log(10000)) * np.arange(half, dtype=np.float32)
                / np.float32(half))
    freqs = np.exp(exponent)
    s = np.atleast_1d(np.asarray(sigma, np.float32)).reshape(-1, 1)
    arg = s * freqs.reshape(1, -1)
    return np.concatenate([np.cos(arg), np.sin(arg)], axis=-1).astype(np.float32)


def patchify(x):
    """Pad H and W to the patch, append the zero padding-mask channel and cut
    2x2 patches (numpy_dit.py:10-22, 92-95): [B,C,T,H,W] -> [B,T,Hp,Wp,(C+1)*4]
    with feature index (c*2 + dy)*2 + dx."""
    x = _f32c(x)
    B, C, T, H, W = x.shape
    Hp, Wp = -(-H // PATCH), -(-W // PATCH)
    xp = np.zeros((B, C + 1, T, Hp * PATCH, Wp * PATCH), np.float32)
    xp[:, :C, :, :H, :W] = x
    t = xp.reshape(B, C + 1, T, Hp, PATCH, Wp, PATCH).transpose(0, 2, 3, 5, 1, 4, 6)
    return np.ascontiguousarray(t.reshape(B, T, Hp, Wp, (C + 1) * PATCH * PATCH))


def unpatchify(f, out_ch, H, W):
    """Inverse patch rearrangement and crop (numpy_dit.py:24-31, 128-129):
    [B,T,Hp,Wp,4*out_ch] with feature (dy*2 + dx)*out_ch + c -> [B,out_ch,T,H,W]."""
    B, T, Hp, Wp, _ = f.shape
    o = f.reshape(B, T, Hp, Wp, PATCH, PATCH, out_ch).transpose(0, 6, 1, 2, 4, 3, 5)
    o = o.reshape(B, out_ch, T, Hp * PATCH, Wp * PATCH)
    return np.ascontiguousarray(o[:, :, :, :H, :W]).astype(np.float32)


def adaln(emb, w1, w2, lora, n_chunks):
    """AdaLN modulation (NumpyBlock._adaln, numpy_dit.py:211-223; the final
    layer's, :171-180): one SiLU, two bias-free linears D -> 256 -> n*D, plus
    the first n*D entries of the AdaLN-LoRA term.  Returns n chunks [B, D]."""
    emb = _f32c(emb)
    D = emb.shape[-1]
    m2 = gemm_bf16(gemm_bf16(silu(emb), w1), w2)
    m2 = (m2 + _f32c(lora)[:, :n_chunks * D]).astype(np.float32)
    return [np.ascontiguousarray(m2[:, i * D:(i + 1) * D]) for i in range(n_chunks)]


def mlp_block(x, mod, w1, w2, eps=1e-6):
    """MLP sub-layer of NumpyBlock.forward with NumpyMLP (numpy_dit.py:249-253,
    304-317): x + gate * layer2(gelu(layer1(layernorm(x)*(1+scale) + shift)))."""
    x = _f32c(x)
    B, S, D = x.shape
    shift, scale, gate = (np.ascontiguousarray(mod[:, i]) for i in range(3))
    xm = modulate(layernorm(x, eps), scale, shift)
    h = gelu(gemm_bf16(xm.reshape(B * S, D), w1))
    return gate_residual(x, gate, gemm_bf16(h, w2).reshape(B, S, D))


def dit_forward(x, sigma, ctx, w, blocks, heads, head_dim, out_ch=16, eps=1e-6, sdpa=None):
    """NumpyDiT.forward (numpy_dit.py:82-130) on latent x [B,C,T,H,W], noise
    levels sigma [B] and text context ctx [B,S_kv,ctx_dim]; returns
    [B,out_ch,T,H,W]."""
    x = _f32c(x)
    B, C, T, H, W = x.shape
    tok = patchify(x)
    _, _, Hp, Wp, K = tok.shape
    S = T * Hp * Wp
    xr = gemm_bf16(tok.reshape(B * S, K), w["x_embedder.proj.1.weight"])
    D = xr.shape[-1]
    xr = xr.reshape(B, S, D)
    freqs = rope_freqs(Hp, Wp, T, head_dim)
    feat = timesteps(sigma, D)
    lora = gemm_bf16(silu(gemm_bf16(feat, w["t_embedder.1.linear_1.weight"])),
                     w["t_embedder.1.linear_2.weight"])
    emb = rmsnorm(feat, w["t_embedding_norm.weight"], 1e-6)
    for i in range(blocks):
        p = f"blocks.{i}."

        def mods(sub):
            return np.stack(adaln(emb, w[p + f"adaln_modulation_{sub}.1.weight"],
                                  w[p + f"adaln_modulation_{sub}.2.weight"], lora, 3), axis=1)

        a = p + "self_attn."
        xr = attention_block(xr, mods("self_attn"), w[a + "q_proj.weight"], w[a + "k_proj.weight"],
                             w[a + "v_proj.weight"], w[a + "output_proj.weight"],
                             w[a + "q_norm.weight"], w[a + "k_norm.weight"], freqs, None,
                             heads, head_dim, eps, sdpa)
        a = p + "cross_attn."
        xr = attention_block(xr, mods("cross_attn"), w[a + "q_proj.weight"],
                             w[a + "k_proj.weight"], w[a + "v_proj.weight"],
                             w[a + "output_proj.weight"], w[a + "q_norm.weight"],
                             w[a + "k_norm.weight"], None, ctx, heads, head_dim, eps, sdpa)
        xr = mlp_block(xr, mods("mlp"), w[p + "mlp.layer1.weight"], w[p + "mlp.layer2.weight"],
                       eps)
    shift, scale = adaln(emb, w["final_layer.adaln_modulation.1.weight"],
                         w["final_layer.adaln_modulation.2.weight"], lora, 2)
    xm = modulate(layernorm(xr, eps), scale, shift)
    f = gemm_bf16(xm.reshape(B * S, D), w["final_layer.linear.weight"])
    return unpatchify(f.reshape(B, T, Hp, Wp, -1), out_ch, H, W)


def z_image_sigmas(steps, denoise=1.0, shift=3.0):
    """ZImageScheduler.get_sigmas (sampling.py:74-83): linspace from denoise
    to 0 in float32, then shift*s / (1 + (shift-1)*s)."""
    s = np.linspace(denoise, 0.0, steps + 1, dtype=np.float32)
    return (shift * s / (1.0 + (shift - 1.0) * s)).astype(np.float32)


def euler_sample(forward, noise, sigmas, ctx_cond, ctx_uncond, cfg):
    """EulerSampler.sample (sampling.py:115-140): per step one forward of the
    CFG pair [uncond, cond], v = v_u + cfg (v_c - v_u), x += v (s_next - s)."""
    x = _f32c(noise)
    ctx_b = np.concatenate([ctx_uncond, ctx_cond], axis=0)
    for i in range(len(sigmas) - 1):
        s, s_next = float(sigmas[i]), float(sigmas[i + 1])
        x_b = np.tile(np.expand_dims(x, 2), (2, 1, 1, 1, 1))
        v = forward(x_b, np.array([s, s], np.float32), ctx_b)
        v_cfg = v[0:1] + cfg * (v[1:2] - v[0:1])
        x = x + v_cfg[:, :, 0] * (s_next - s)
    return x
