"""Torch-free host interface of the attention path, on numpy buffers.

`AnimaRT` is a drop-in for the ``rt`` object NumpyDiT calls
(``NumpyRT`` in scripts/phone_pipeline_nd.py:46-68) and `AnimaVK` for its
GEMM engine ``vk`` (NumpyVK, :69-72): the same method names, argument
meanings and array layouts, backed by libanima_hip.so on the GPU.
One deliberate difference: a false return from the library raises
`AnimaHipError` (the reference's ``run_sdpa`` ignores the return value,
phone_pipeline_nd.py:67, and would hand back zeros).
"""
from __future__ import annotations

import ctypes as ct
import math

import numpy as np

from . import _lib

F32 = 0
BF16 = 1
F32X3 = 2  # f32 operands as bf16 term pairs on bf16 MFMA (three products each)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    return None if a is None else a.ctypes.data


def init() -> None:
    """anima_rt_init (anima_rt/src/anima_rt.cpp:13-20)."""
    _lib.check(_lib.load().anima_rt_init(), "anima_rt_init")


def destroy() -> None:
    """anima_rt_destroy (anima_rt.cpp:166-171)."""
    _lib.load().anima_rt_destroy()


def last_call_ms():
    """(kernel_ms, total_ms) of the last host-pointer call: device time between
    its uploads and downloads, and from the first upload to the last download
    (anima_hip_last_call_ms)."""
    k, t = ct.c_float(), ct.c_float()
    _lib.check(_lib.load().anima_hip_last_call_ms(ct.byref(k), ct.byref(t)),
               "anima_hip_last_call_ms")
    return k.value, t.value


def sdpa_flash(q, k, v, scale=None, is_causal=False) -> np.ndarray:
    """anima_rt_run_sdpa_flash on [BH,S,D] arrays (anima_rt.cpp:147-156)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    BH, Sq, D = q.shape
    Sk = k.shape[1]
    if k.shape != (BH, Sk, D) or v.shape != (BH, Sk, D):
        raise ValueError(f"sdpa shapes q{q.shape} k{k.shape} v{v.shape}")
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    o = np.zeros((BH, Sq, D), np.float32)
    ok = _lib.load().anima_rt_run_sdpa_flash(_p(q), _p(k), _p(v), _p(o), BH, Sq, Sk, D,
                                             ct.c_float(scale), ct.c_bool(is_causal))
    _lib.check(ok, "anima_rt_run_sdpa_flash")
    return o


def sdpa(q, k, v, scale=None, is_causal=False, mode=F32) -> np.ndarray:
    """anima_hip_sdpa: sdpa_flash with an arithmetic mode (F32, BF16 or F32X3)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    BH, Sq, D = q.shape
    Sk = k.shape[1]
    if k.shape != (BH, Sk, D) or v.shape != (BH, Sk, D):
        raise ValueError(f"sdpa shapes q{q.shape} k{k.shape} v{v.shape}")
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    o = np.zeros((BH, Sq, D), np.float32)
    ok = _lib.load().anima_hip_sdpa(_p(q), _p(k), _p(v), _p(o), BH, Sq, Sk, D, ct.c_float(scale),
                                    ct.c_bool(is_causal), int(mode))
    _lib.check(ok, "anima_hip_sdpa")
    return o


def sdpa_math(q, k, v, scale=None, is_causal=False) -> np.ndarray:
    """anima_rt_run_sdpa (anima_rt.cpp:78-141): the reference's math entry,
    whose effective logit scale is scale**2.  Needs init() first."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    BH, Sq, D = q.shape
    Sk = k.shape[1]
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    o = np.zeros((BH, Sq, D), np.float32)
    ok = _lib.load().anima_rt_run_sdpa(_p(q), _p(k), _p(v), _p(o), BH, Sq, Sk, D,
                                       ct.c_float(scale), ct.c_bool(is_causal))
    _lib.check(ok, "anima_rt_run_sdpa")
    return o


def rmsnorm(x, w=None, eps=1e-6) -> np.ndarray:
    """anima_rt_run_rmsnorm over the last axis (anima_rt.cpp:45-50). Needs init()."""
    x = _f32(x)
    D = x.shape[-1]
    M = x.size // D if D else 0
    w = None if w is None else _f32(w)
    out = np.zeros_like(x)
    ok = _lib.load().anima_rt_run_rmsnorm(_p(x), _p(w), _p(out), M, D, ct.c_float(eps))
    _lib.check(ok, "anima_rt_run_rmsnorm")
    return out


def _unary(name, x, *extra):
    x = _f32(x)
    out = np.zeros_like(x)
    _lib.check(getattr(_lib.load(), "anima_rt_run_" + name)(_p(x), _p(out), *extra),
               "anima_rt_run_" + name)
    return out


def gelu(x) -> np.ndarray:
    """anima_rt_run_gelu, exact erf form (anima_rt.cpp:24-27). Needs init()."""
    return _unary("gelu", x, int(np.size(x)))


def silu(x) -> np.ndarray:
    """anima_rt_run_silu (anima_rt.cpp:29-32). Needs init()."""
    return _unary("silu", x, int(np.size(x)))


def layernorm(x, eps=1e-6) -> np.ndarray:
    """anima_rt_run_layernorm over the last axis, no affine (anima_rt.cpp:36-43).
    Needs init()."""
    x = _f32(x)
    D = x.shape[-1]
    return _unary("layernorm", x, x.size // D if D else 0, D, ct.c_float(eps))


def softmax(x) -> np.ndarray:
    """anima_rt_run_softmax over the last axis (anima_rt.cpp:52-57). Needs init()."""
    x = _f32(x)
    D = x.shape[-1]
    return _unary("softmax", x, x.size // D if D else 0, D)


def bias_add(c, bias) -> np.ndarray:
    """anima_rt_run_bias_add (gemm_backend.cpp:173-183): c[i, :] += bias, in
    place on a C-contiguous float32 matrix; returns c."""
    if c.dtype != np.float32 or not c.flags.c_contiguous or c.ndim != 2:
        raise ValueError("bias_add: c must be a C-contiguous float32 matrix")
    b = None if bias is None else _f32(bias)
    if b is not None and b.shape != (c.shape[1],):
        raise ValueError("bias_add: bias must have one entry per column")
    _lib.check(_lib.load().anima_rt_run_bias_add(_p(c), _p(b), c.shape[0], c.shape[1]),
               "anima_rt_run_bias_add")
    return c


def rope(t, freqs) -> np.ndarray:
    """anima_rt_run_rope on t [N,S,D] with freqs [S,D/2,2,2] (anima_rt.cpp:160-164)."""
    t = _f32(t)
    N, S, D = t.shape
    f = _f32(freqs)
    if f.size != S * D * 2:
        raise ValueError(f"freqs has {f.size} values, expected S*D*2 = {S * D * 2}")
    out = np.zeros_like(t)
    ok = _lib.load().anima_rt_run_rope(_p(t), _p(f), _p(out), N, S, D)
    _lib.check(ok, "anima_rt_run_rope")
    return out


def attention(q, k, v, q_norm_w=None, k_norm_w=None, freqs=None, eps=1e-6,
              mode=F32) -> np.ndarray:
    """One call for the middle of NumpyAttention.forward
    (anima_rt/scripts/numpy_dit.py:283-294): per-head RMSNorm of q and k,
    RoPE when `freqs` is given (self-attention), SDPA with scale 1/sqrt(D),
    on [B,S,H,D] projections.  Returns [B,S_q,H,D] float32, i.e. the
    [B*S_q, H*D] input of output_proj without any host transposes."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    if k.shape != (B, Sk, H, D) or v.shape != (B, Sk, H, D):
        raise ValueError(f"attention shapes q{q.shape} k{k.shape} v{v.shape}")
    qw = None if q_norm_w is None else _f32(q_norm_w)
    kw = None if k_norm_w is None else _f32(k_norm_w)
    f = None if freqs is None else _f32(freqs)
    out = np.zeros((B, Sq, H, D), np.float32)
    ok = _lib.load().anima_hip_attention(_p(q), _p(k), _p(v), _p(qw), _p(kw), _p(f), _p(out),
                                         B, Sq, Sk, H, D, ct.c_float(eps), int(mode))
    _lib.check(ok, "anima_hip_attention")
    return out


def gemm_fp32(a, b) -> np.ndarray:
    """anima_rt_run_gemm_fp32: C = A . B^T (gemm_backend.cpp:140-148)."""
    a, b = _f32(a), _f32(b)
    M, K = a.shape
    N = b.shape[0]
    if b.shape != (N, K):
        raise ValueError(f"gemm shapes a{a.shape} b{b.shape}")
    c = np.zeros((M, N), np.float32)
    _lib.check(_lib.load().anima_rt_run_gemm_fp32(_p(a), _p(b), _p(c), M, N, K),
               "anima_rt_run_gemm_fp32")
    return c


def gemm_bf16(a, w_bits) -> np.ndarray:
    """anima_rt_run_gemm_bf16: C = A . W^T with W as bf16 bit patterns
    (uint16 [N, K], gemm_backend.cpp:154-173)."""
    a = _f32(a)
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    M, K = a.shape
    N = w.shape[0]
    if w.shape != (N, K):
        raise ValueError(f"gemm shapes a{a.shape} w{w.shape}")
    c = np.zeros((M, N), np.float32)
    _lib.check(_lib.load().anima_rt_run_gemm_bf16(_p(a), _p(w), _p(c), M, N, K),
               "anima_rt_run_gemm_bf16")
    return c


DTYPES = {0: "F32", 1: "F16", 2: "BF16"}


class Weights:
    """A model file in the reference's safetensors format
    (scripts/phone_pipeline_nd.py:15-43), memory-mapped and validated by the
    library.  ``device(name)`` uploads a tensor once and returns its device
    pointer, resident until ``close()``: BF16 linear weights as bit patterns
    (the form ``anima_hip_linear_dev`` takes), or widened to f32 with
    ``as_f32=True`` (what the reference does for its norm weights).  Names
    match with or without the reference's ``net.`` prefix."""

    def __init__(self, path):
        self._lib = _lib.load()
        h = self._lib.anima_hip_weights_open(str(path).encode())
        if not h:
            raise _lib.AnimaHipError(f"anima_hip_weights_open failed: {_lib.last_error()}")
        self._h = h

    @property
    def handle(self):
        return self._h

    def names(self) -> list:
        n = self._lib.anima_hip_weights_count(self._h)
        return [self._lib.anima_hip_weights_name(self._h, i).decode() for i in range(n)]

    def info(self, name):
        """(dtype string, shape tuple) of a tensor."""
        dt = ct.c_int()
        shape = (ct.c_int64 * 8)()
        nd = self._lib.anima_hip_weights_info(self._h, name.encode(), ct.byref(dt), shape, 8)
        if nd < 0:
            raise KeyError(name)
        return DTYPES[dt.value], tuple(shape[i] for i in range(min(nd, 8)))

    def device(self, name, as_f32=False) -> int:
        p = self._lib.anima_hip_weights_device(self._h, name.encode(), int(bool(as_f32)))
        if not p:
            raise _lib.AnimaHipError(f"anima_hip_weights_device({name}) failed: "
                                     f"{_lib.last_error()}")
        return p

    def close(self):
        if self._h:
            self._lib.anima_hip_weights_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def load_context(path) -> np.ndarray:
    """Text-context embeddings as the reference stores them
    (context_cond.npy / context_uncond.npy, phone_pipeline_nd.py:79-85):
    float32 [batch, tokens, 1024].  Loaded without pickle support."""
    ctx = np.load(path, allow_pickle=False)
    if ctx.ndim == 2:
        ctx = ctx[None]
    if ctx.ndim != 3:
        raise ValueError(f"context {path}: expected [batch, tokens, dim], got {ctx.shape}")
    return np.ascontiguousarray(ctx, dtype=np.float32)


class ContextKV:
    """Cross-attention K/V of one text context, kept on the GPU
    (anima_hip_ctx_kv_create).  K = RMSNorm_head(ctx . Wk^T), V = ctx . Wv^T,
    computed once; every denoise step and both CFG branches reuse them.

    ctx: [S_kv, C] or [Bc, S_kv, C] float32; wk_bits / wv_bits: bf16 bit
    patterns [H*D, C] (uint16); k_norm_w: [D] or None."""

    def __init__(self, ctx, wk_bits, wv_bits, k_norm_w=None, heads=16, head_dim=128, eps=1e-6,
                 mode=F32):
        ctx = _f32(ctx)
        if ctx.ndim == 2:
            ctx = ctx[None]
        Bc, S, C = ctx.shape
        wk = np.ascontiguousarray(wk_bits, dtype=np.uint16)
        wv = np.ascontiguousarray(wv_bits, dtype=np.uint16)
        if wk.shape != (heads * head_dim, C) or wv.shape != wk.shape:
            raise ValueError(f"weights must be [{heads * head_dim}, {C}]")
        kw = None if k_norm_w is None else _f32(k_norm_w)
        self.batch, self.tokens, self.heads, self.head_dim = Bc, S, heads, head_dim
        self.mode = mode
        h = _lib.load().anima_hip_ctx_kv_create(_p(ctx), _p(wk), _p(wv), _p(kw), Bc, S, C, heads,
                                                head_dim, ct.c_float(eps), int(mode))
        if not h:
            raise _lib.AnimaHipError(f"anima_hip_ctx_kv_create failed: {_lib.last_error()}")
        self._h = ct.c_void_p(h)

    @property
    def handle(self):
        return self._h

    def attend(self, q, q_norm_w=None, eps=1e-6) -> np.ndarray:
        """Cross-attention of q [B, S_q, H, D] (q_proj output) against the
        cached context; returns [B, S_q, H, D] float32."""
        if self._h is None:
            raise _lib.AnimaHipError("context cache already closed")
        q = _f32(q)
        B, Sq, H, D = q.shape
        if (H, D) != (self.heads, self.head_dim):
            raise ValueError(f"q heads/dim {H}x{D} != cache {self.heads}x{self.head_dim}")
        qw = None if q_norm_w is None else _f32(q_norm_w)
        out = np.zeros_like(q)
        ok = _lib.load().anima_hip_cross_attention(_p(q), _p(qw), self._h, _p(out), B, Sq,
                                                   ct.c_float(eps))
        _lib.check(ok, "anima_hip_cross_attention")
        return out

    def close(self):
        if getattr(self, "_h", None) is not None:
            _lib.load().anima_hip_ctx_kv_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class AnimaRT:
    """Drop-in for NumpyDiT's ``rt`` (NumpyRT, scripts/phone_pipeline_nd.py:46-68).

    ``norm_weights`` maps '<prefix>.weight' to float32 arrays, like NumpyRT's
    ``nw``; ``run_rmsnorm(x, key)`` looks the weight up by key prefix.
    """

    def __init__(self, norm_weights=None):
        init()
        self._nw = dict(norm_weights or {})

    def _w(self, key):
        w = self._nw.get(key + ".weight")
        return None if w is None else _f32(w)

    def run_rmsnorm(self, x, key, eps=1e-6):
        x = np.asarray(x, np.float32)
        return rmsnorm(x, self._w(key), eps)

    def run_layernorm(self, x, D):
        """[M, D] rows, eps 1e-6, no affine (NumpyRT.run_layernorm)."""
        return layernorm(np.asarray(x, np.float32).reshape(-1, D), 1e-6)

    def run_gelu(self, x):
        return gelu(np.asarray(x, np.float32).reshape(-1))

    def run_silu(self, x):
        return silu(np.asarray(x, np.float32).reshape(-1))

    def run_sdpa(self, q, k, v):
        """[B,H,S,D] q/k/v -> [B,H,S_q,D], scale 1/sqrt(D), non-causal."""
        B, H, Sq, D = q.shape
        Sk = k.shape[2]
        o = sdpa_flash(np.asarray(q).reshape(B * H, Sq, D), np.asarray(k).reshape(B * H, Sk, D),
                       np.asarray(v).reshape(B * H, Sk, D), scale=1.0 / math.sqrt(D))
        return o.reshape(B, H, Sq, D)

    def run_rope(self, t, freqs):
        """[B,S,H,D] activations with an [S,D/2,2,2] table (rotate-half)."""
        t = np.asarray(t, np.float32)
        B, S, H, D = t.shape
        flat = np.ascontiguousarray(t.transpose(0, 2, 1, 3)).reshape(B * H, S, D)
        return rope(flat, freqs).reshape(B, H, S, D).transpose(0, 2, 1, 3)

    def run_attention(self, q, k, v, prefix, rope_emb=None, mode=F32):
        """NumpyAttention.forward's norm -> RoPE -> SDPA core for block `prefix`
        on [B,S,H,D] projections (numpy_dit.py:283-294)."""
        freqs = None if rope_emb is None else np.asarray(rope_emb, np.float32).reshape(
            q.shape[1], q.shape[3] // 2, 2, 2)
        return attention(q, k, v, self._w(f"{prefix}.q_norm"), self._w(f"{prefix}.k_norm"),
                         freqs, mode=mode)


class AnimaVK:
    """Drop-in for NumpyDiT's GEMM engine ``vk`` (NumpyVK,
    scripts/phone_pipeline_nd.py:69-72, over vk_run_gemm of
    vulkan/hybrid_engine.cpp): ``vk_run_gemm(name, x, out, M, N, K)`` writes
    out[M, N] = x[M, K] . W[name]^T with the named bf16 weight resident on the
    GPU (a ``Weights`` store).  mode F32 feeds x as exact hi + lo bf16 terms,
    BF16 rounds it.  Raises RuntimeError on failure, like NumpyVK."""

    def __init__(self, weights, mode=F32):
        from .dit import DeviceArray
        self._w = weights
        self._mode = int(mode)
        self._lib = _lib.load()
        self._dev = DeviceArray
        self._bufs = {}

    def _buf(self, role, nbytes):
        b = self._bufs.get(role)
        if b is None or b.nbytes < nbytes:
            if b is not None:
                b.close()
            b = self._bufs[role] = self._dev(max(int(nbytes), 256))
        return b

    def vk_run_gemm(self, name, x, out, M, N, K):
        dt, shape = self._w.info(name)
        if dt != "BF16" or tuple(shape) != (N, K):
            raise RuntimeError(f"vk_run_gemm({name}) failed: weight is {dt} {shape}, "
                               f"expected BF16 ({N}, {K})")
        x = _f32(x).reshape(M, K)
        if out.dtype != np.float32 or out.size != M * N or not out.flags.c_contiguous:
            raise RuntimeError(f"vk_run_gemm({name}) failed: out must be float32 [{M}, {N}]")
        xd = self._buf("x", x.nbytes)
        xd.upload(x)
        od = self._buf("out", out.nbytes)
        n = self._lib.anima_hip_linear_scratch_bytes(M, K, self._mode)
        sd = self._buf("scratch", n)
        ok = self._lib.anima_hip_linear_dev(xd.ptr, K, self._w.device(name), K, od.ptr, N, M, N,
                                            K, self._mode, sd.ptr, n, None)
        if not ok:
            raise RuntimeError(f"vk_run_gemm({name}) failed: {_lib.last_error()}")
        out.reshape(-1)[:] = od.download((M * N,))
