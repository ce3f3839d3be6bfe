"""The whole Anima DiT on the GPU behind the reference's model interface.

``AnimaDiT.forward(x_np, sigma, ctx_np)`` takes and returns numpy arrays like
NumpyDiT.forward (anima_rt/scripts/numpy_dit.py:82-130), so the reference's
EulerSampler / run_ksampler (anima_rt/scripts/sampling.py:115-140, 179-209)
drive it unchanged.  ``AnimaDiT.sample`` runs that sampler's whole loop on the
device instead: the latent, the residual stream and the per-block text-context
K/V stay in HBM for every step, and only the final latent comes back.

Weights come from the reference's safetensors file (``rt.Weights``) or from a
table of device tensors; the library checks every shape against the model
configuration.  Compute is libanima_hip only: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as ct

import numpy as np

from . import _lib
from .rope import generate_rope_freqs
from .rt import BF16, F32, F32X3

DTYPE_CODES = {"F32": 0, "F16": 1, "BF16": 2}
ADA_HIDDEN = 256  # hidden width of every AdaLN modulation MLP


class DiTConfig(ct.Structure):
    """anima_hip_dit_config (include/anima_hip.h)."""
    _fields_ = [(n, ct.c_int) for n in ("dim", "blocks", "heads", "head_dim", "mlp_hidden",
                                          "ctx_dim", "in_channels", "out_channels",
                                          "max_batch")]

    @classmethod
    def anima_2b(cls, **overrides):
        """The Anima 2B shapes (anima_hip_dit_default_config) with overrides."""
        c = cls()
        _lib.load().anima_hip_dit_default_config(ct.byref(c))
        for k, v in overrides.items():
            setattr(c, k, int(v))
        return c


def weight_shapes(config: DiTConfig) -> dict:
    """{name: shape} of every tensor the model reads, in the reference
    checkpoint's names (without the "net." prefix) and [out, in] layout
    (numpy_dit.py:145-317)."""
    c = config
    D, hd = c.dim, c.heads * c.head_dim
    s = {"x_embedder.proj.1.weight": (D, (c.in_channels + 1) * 4),
         "t_embedder.1.linear_1.weight": (D, D),
         "t_embedder.1.linear_2.weight": (3 * D, D),
         "t_embedding_norm.weight": (D,)}
    for i in range(c.blocks):
        p = f"blocks.{i}."
        for a, kv_in in (("self_attn", D), ("cross_attn", c.ctx_dim)):
            s[p + a + ".q_proj.weight"] = (hd, D)
            s[p + a + ".k_proj.weight"] = (hd, kv_in)
            s[p + a + ".v_proj.weight"] = (hd, kv_in)
            s[p + a + ".output_proj.weight"] = (D, hd)
            s[p + a + ".q_norm.weight"] = (c.head_dim,)
            s[p + a + ".k_norm.weight"] = (c.head_dim,)
        s[p + "mlp.layer1.weight"] = (c.mlp_hidden, D)
        s[p + "mlp.layer2.weight"] = (D, c.mlp_hidden)
        for sub in ("self_attn", "cross_attn", "mlp"):
            s[p + f"adaln_modulation_{sub}.1.weight"] = (ADA_HIDDEN, D)
            s[p + f"adaln_modulation_{sub}.2.weight"] = (3 * D, ADA_HIDDEN)
    s["final_layer.adaln_modulation.1.weight"] = (ADA_HIDDEN, D)
    s["final_layer.adaln_modulation.2.weight"] = (2 * D, ADA_HIDDEN)
    s["final_layer.linear.weight"] = (4 * c.out_channels, D)
    return s


def _norm_weight(name):
    return name.endswith("_norm.weight") or name == "t_embedding_norm.weight"


class DeviceArray:
    """Device memory from libanima_hip (anima_hip_malloc), freed on close."""

    def __init__(self, nbytes):
        self._lib = _lib.load()
        self.nbytes = int(nbytes)
        self.ptr = self._lib.anima_hip_malloc(max(self.nbytes, 1))
        if not self.ptr:
            raise _lib.AnimaHipError(f"anima_hip_malloc failed: {_lib.last_error()}")

    @classmethod
    def of(cls, a):
        a = np.ascontiguousarray(a)
        d = cls(a.nbytes)
        d.upload(a)
        return d

    def upload(self, a):
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError("array larger than the device buffer")
        _lib.check(self._lib.anima_hip_memcpy(self.ptr, a.ctypes.data, a.nbytes, 1), "memcpy")

    def download(self, shape, dtype=np.float32):
        out = np.empty(shape, dtype)
        if out.nbytes > self.nbytes:
            raise ValueError("requested more than the device buffer holds")
        _lib.check(self._lib.anima_hip_memcpy(out.ctypes.data, self.ptr, out.nbytes, 2),
                   "memcpy")
        return out

    def close(self):
        if self.ptr:
            self._lib.anima_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class AnimaDiT:
    """Device-resident Anima DiT.

    weights: an ``rt.Weights`` store (device copies are made on demand: linear
    weights as bf16 bits, norm weights widened to f32), or a dict
    name -> (device pointer, dtype string, shape) of tensors already on the
    device, which must outlive the model.  mode: ``rt.F32`` (f32 MFMA attention), ``rt.F32X3``
    (attention on bf16 term pairs, the same f32 tolerance) or ``rt.BF16``; the linear layers take
    exact hi + lo bf16 terms except in ``rt.BF16``."""

    def __init__(self, weights, config: DiTConfig | None = None, mode=F32):
        self._lib = _lib.load()
        self.config = config if config is not None else DiTConfig.anima_2b()
        self.mode = int(mode)
        table = self._table(weights)
        n = len(table)
        names = (ct.c_char_p * n)(*[k.encode() for k in table])
        ptrs = (ct.c_void_p * n)(*[v[0] for v in table.values()])
        dtypes = (ct.c_int * n)(*[DTYPE_CODES[v[1]] for v in table.values()])
        shp = []
        for _, _, s in table.values():
            shp += [int(s[0]), int(s[1]) if len(s) > 1 else 0]
        shapes = (ct.c_int64 * (2 * n))(*shp)
        h = self._lib.anima_hip_dit_create(ct.byref(self.config), names, ptrs, dtypes, shapes, n,
                                           self.mode)
        if not h:
            raise _lib.AnimaHipError(f"anima_hip_dit_create failed: {_lib.last_error()}")
        self._h = h
        self._weights = weights  # keeps a store's device copies alive
        self._bufs = {}
        self._ctx_host = None
        self._freqs_key = None

    @staticmethod
    def _table(weights):
        if isinstance(weights, dict):
            return {k: (int(p), dt, tuple(s)) for k, (p, dt, s) in weights.items()}
        table = {}
        for name in weights.names():
            dt, shape = weights.info(name)
            if len(shape) == 1 and _norm_weight(name):
                table[name] = (weights.device(name, as_f32=True), "F32", shape)
            elif len(shape) == 2:
                table[name] = (weights.device(name), dt, shape)
        return table

    @property
    def handle(self):
        return self._h

    # ---- device buffers (grow-only, by role) ----
    def _buf(self, role, nbytes):
        b = self._bufs.get(role)
        if b is None or b.nbytes < nbytes:
            if b is not None:
                b.close()
            b = self._bufs[role] = DeviceArray(nbytes)
        return b

    def _freqs(self, T, H, W):
        Hp, Wp = -(-H // 2), -(-W // 2)
        key = (T, Hp, Wp)
        if self._freqs_key != key:
            f = generate_rope_freqs(Hp, Wp, T, self.config.head_dim)
            self._buf("freqs", f.nbytes).upload(f)
            self._freqs_key = key
        return self._bufs["freqs"].ptr

    def set_context(self, ctx):
        """Text context [Bc, S_kv, ctx_dim] (host): recomputes every block's
        cross-attention K/V on the device; skipped when ctx equals the last one."""
        ctx = np.ascontiguousarray(ctx, dtype=np.float32)
        if ctx.ndim == 2:
            ctx = ctx[None]
        if self._ctx_host is not None and self._ctx_host.shape == ctx.shape and \
                np.array_equal(self._ctx_host, ctx):
            return
        self._ctx_host = None  # the device holds no valid context until this succeeds
        d = self._buf("ctx", ctx.nbytes)
        d.upload(ctx)
        _lib.check(self._lib.anima_hip_dit_set_context_dev(self._h, d.ptr, ctx.shape[0],
                                                           ctx.shape[1], None),
                   "dit_set_context_dev")
        self._ctx_host = ctx.copy()

    def _scratch(self, B, T, H, W):
        n = self._lib.anima_hip_dit_scratch_bytes(self._h, B, T, H, W)
        return self._buf("scratch", n), n

    def forward(self, x_np, sigma, ctx_np):
        """NumpyDiT.forward: x [B,C,T,H,W], sigma scalar or [B], ctx [B,N,ctx_dim]
        -> [B,out_channels,T,H,W] float32."""
        x = np.ascontiguousarray(x_np, dtype=np.float32)
        B, C, T, H, W = x.shape
        sig = np.atleast_1d(np.asarray(sigma, dtype=np.float32))
        if sig.shape[0] == 1 and B > 1:
            sig = np.repeat(sig, B)
        if sig.shape[0] != B:
            raise ValueError("sigma must have one entry per batch entry")
        self.set_context(ctx_np)
        xd = self._buf("x", x.nbytes)
        xd.upload(x)
        out_shape = (B, self.config.out_channels, T, H, W)
        od = self._buf("out", int(np.prod(out_shape)) * 4)
        scr, n = self._scratch(B, T, H, W)
        sig_c = (ct.c_float * B)(*sig.tolist())
        _lib.check(self._lib.anima_hip_dit_forward_dev(
            self._h, xd.ptr, C * T * H * W, sig_c, B, T, H, W, self._freqs(T, H, W), od.ptr,
            scr.ptr, n, None), "dit_forward_dev")
        return od.download(out_shape)

    def sample(self, noise, sigmas, ctx_cond, ctx_uncond, cfg):
        """EulerSampler.sample with the loop on the device: noise [1,C,H,W],
        sigmas [steps+1], contexts [1,N,ctx_dim] -> latent [1,C,H,W]."""
        x = np.ascontiguousarray(noise, dtype=np.float32)
        if x.ndim != 4 or x.shape[0] != 1:
            raise ValueError("noise must be [1, C, H, W]")
        _, C, H, W = x.shape
        self.set_context(np.concatenate([np.asarray(ctx_uncond, np.float32),
                                         np.asarray(ctx_cond, np.float32)], axis=0))
        sig = np.ascontiguousarray(sigmas, dtype=np.float32)
        steps = sig.shape[0] - 1
        xd = self._buf("latent", x.nbytes)
        xd.upload(x)
        scr, n = self._scratch(2, 1, H, W)
        _lib.check(self._lib.anima_hip_dit_euler_dev(
            self._h, xd.ptr, sig.ctypes.data, steps, ct.c_float(cfg), H, W,
            self._freqs(1, H, W), scr.ptr, n, None), "dit_euler_dev")
        return xd.download(x.shape)

    def close(self):
        if getattr(self, "_h", None):
            self._lib.anima_hip_dit_destroy(self._h)
            self._h = None
        for b in self._bufs.values():
            b.close()
        self._bufs = {}

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


__all__ = ["AnimaDiT", "DiTConfig", "DeviceArray", "weight_shapes", "F32", "F32X3", "BF16"]
