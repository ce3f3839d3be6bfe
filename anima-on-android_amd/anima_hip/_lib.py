"""ctypes binding of libanima_hip.so (declarations mirror include/anima_hip.h).

The library is the only compute path: when it cannot be loaded this module
raises instead of falling back to any CPU implementation.
"""
from __future__ import annotations

import ctypes as ct
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libanima_hip.so")

_P = ct.c_void_p
_I = ct.c_int
_F = ct.c_float
_B = ct.c_bool
_I64P = ct.POINTER(ct.c_int64)

# name -> (restype, argtypes); every symbol declared in include/anima_hip.h.
SIGNATURES = {
    "anima_rt_init": (_B, []),
    "anima_rt_destroy": (None, []),
    "anima_rt_run_sdpa_flash": (_B, [_P] * 4 + [_I] * 4 + [_F, _B]),
    "anima_rt_run_sdpa": (_B, [_P] * 4 + [_I] * 4 + [_F, _B]),
    "anima_rt_run_rmsnorm": (_B, [_P, _P, _P, _I, _I, _F]),
    "anima_rt_run_rope": (_B, [_P, _P, _P, _I, _I, _I]),
    "anima_rt_run_gelu": (_B, [_P, _P, _I]),
    "anima_rt_run_silu": (_B, [_P, _P, _I]),
    "anima_rt_run_layernorm": (_B, [_P, _P, _I, _I, _F]),
    "anima_rt_run_softmax": (_B, [_P, _P, _I, _I]),
    "anima_rt_run_bias_add": (_B, [_P, _P, _I, _I]),
    "anima_rt_run_gemm_fp32": (_B, [_P] * 3 + [_I] * 3),
    "anima_rt_run_gemm_bf16": (_B, [_P] * 3 + [_I] * 3),
    "anima_hip_last_error": (ct.c_char_p, []),
    "anima_hip_version": (_I, []),
    "anima_hip_sdpa": (_B, [_P] * 4 + [_I] * 4 + [_F, _B, _I]),
    "anima_hip_flash_f32_dev": (_B, [_P] * 4 + [_I] * 5 + [_I64P] * 4 + [_F, _B, _P]),
    "anima_hip_flash_bf16_dev": (_B, [_P] * 4 + [_I] * 5 + [_I64P] * 4 + [_F, _B, _P]),
    "anima_hip_flash_x3_dev": (_B, [_P] * 4 + [_I] * 5 + [_I64P] * 4 + [_F, _B, _P]),
    "anima_hip_flash_f32_rawq_dev": (_B, [_P, _P, _F] + [_P] * 3 + [_I] * 5 + [_I64P] * 4
                                     + [_F, _B, _P]),
    "anima_hip_flash_x3_rawq_dev": (_B, [_P] * 3 + [_F] + [_P] * 3 + [_I] * 5 + [_I64P] * 4
                                    + [_F, _B, _P]),
    "anima_hip_flash_bf16_rawq_dev": (_B, [_P] * 3 + [_F] + [_P] * 3 + [_I] * 5 + [_I64P] * 4
                                      + [_F, _B, _P]),
    "anima_hip_pack_vt_terms_dev": (_B, [_P, _P] + [_I] * 4 + [_I64P] * 2 + [_P]),
    "anima_hip_vt_padded_len": (ct.c_int64, [_I]),
    "anima_hip_pack_vt_dev": (_B, [_P, _P] + [_I] * 4 + [_I64P] * 2 + [_P]),
    "anima_hip_qk_prologue_dev": (_B, [_P] * 4 + [_I] * 4 + [_I64P] * 2 + [_F, _I, _P]),
    "anima_hip_qkv_prologue_dev": (_B, [_P] * 3 + [ct.c_int64] + [_P] * 6 + [_I] * 4
                                   + [_F, _I, _P]),
    "anima_hip_qkv_projection_dev": (_B, [_P, ct.c_int64, _P, ct.c_int64, _I] + [_P] * 6
                                     + [_I] * 3 + [_F, _I, _P]),
    "anima_hip_attention": (_B, [_P] * 7 + [_I] * 5 + [_F, _I]),
    "anima_hip_gemm_dev": (_B, [_P, ct.c_int64, _P, _I, ct.c_int64, _P, ct.c_int64] + [_I] * 3
                           + [_P]),
    "anima_hip_attention_block_scratch_bytes": (ct.c_size_t, [_P] + [_I] * 6),
    "anima_hip_attention_block_dev": (_B, [_P] * 10 + [_I] * 5 + [_F, _I, _P, ct.c_size_t, _P]),
    "anima_hip_weights_open": (_P, [ct.c_char_p]),
    "anima_hip_weights_close": (None, [_P]),
    "anima_hip_weights_count": (_I, [_P]),
    "anima_hip_weights_name": (ct.c_char_p, [_P, _I]),
    "anima_hip_weights_info": (_I, [_P, ct.c_char_p, ct.POINTER(_I), _I64P, _I]),
    "anima_hip_weights_device": (_P, [_P, ct.c_char_p, _I]),
    "anima_hip_linear_scratch_bytes": (ct.c_size_t, [_I, _I, _I]),
    "anima_hip_linear_dev": (_B, [_P, ct.c_int64, _P, ct.c_int64, _P, ct.c_int64] + [_I] * 4
                             + [_P, ct.c_size_t, _P]),
    "anima_hip_attention_scratch_bytes": (ct.c_size_t, [_I] * 7),
    "anima_hip_attention_dev": (_B, [_P] * 8 + [ct.c_size_t] + [_I] * 6 + [_F, _I, _P]),
    "anima_hip_attention_static_dev": (_B, [_P] * 7 + [_I] * 6 + [_F, _I, _P]),
    "anima_hip_attention_terms_dev": (_B, [_P] * 7 + [ct.c_int64] * 2 + [_P, ct.c_size_t]
                                      + [_I] * 6 + [_F, _I, _P]),
    "anima_hip_dit_default_config": (None, [_P]),
    "anima_hip_dit_create": (_P, [_P, _P, _P, ct.POINTER(_I), _I64P, _I, _I]),
    "anima_hip_dit_destroy": (None, [_P]),
    "anima_hip_dit_set_context_dev": (_B, [_P, _P, _I, _I, _P]),
    "anima_hip_dit_scratch_bytes": (ct.c_size_t, [_P] + [_I] * 4),
    "anima_hip_dit_forward_dev": (_B, [_P, _P, ct.c_int64, _P] + [_I] * 4
                                  + [_P, _P, _P, ct.c_size_t, _P]),
    "anima_hip_dit_euler_dev": (_B, [_P, _P, _P, _I, _F, _I, _I, _P, _P, ct.c_size_t, _P]),
    "anima_hip_last_call_ms": (_B, [ct.POINTER(_F), ct.POINTER(_F)]),
    "anima_hip_malloc": (_P, [ct.c_size_t]),
    "anima_hip_free": (None, [_P]),
    "anima_hip_memcpy": (_B, [_P, _P, ct.c_size_t, _I]),
    "anima_hip_synchronize": (_B, []),
    "anima_hip_ctx_kv_create": (_P, [_P] * 4 + [_I] * 5 + [_F, _I]),
    "anima_hip_ctx_kv_destroy": (None, [_P]),
    "anima_hip_cross_attention": (_B, [_P] * 4 + [_I] * 2 + [_F]),
    "anima_hip_cross_attention_scratch_bytes": (ct.c_size_t, [_P, _I, _I]),
    "anima_hip_cross_attention_dev": (_B, [_P] * 5 + [ct.c_size_t] + [_I] * 2 + [_F, _P]),
    "anima_hip_cross_attention_terms_dev": (_B, [_P] * 4 + [ct.c_int64] * 2 + [_P, ct.c_size_t]
                                            + [_I] * 2 + [_F, _P]),
}


class AnimaHipError(RuntimeError):
    """A libanima_hip entry point returned false."""


_lib = None


def load() -> ct.CDLL:
    """Load libanima_hip.so once and declare every entry point."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise AnimaHipError(
                f"{LIB_PATH} is missing; build it with `make -C anima-on-android_amd` "
                "(or __graft_entry__.build())")
        lib = ct.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error() -> str:
    msg = load().anima_hip_last_error()
    return msg.decode() if msg else ""


def check(ok: bool, what: str) -> None:
    if not ok:
        raise AnimaHipError(f"{what} failed: {last_error()}")


def strides(s) -> object:
    """int64[3] {batch, head, seq} element strides, or None for contiguous."""
    if s is None:
        return None
    return (ct.c_int64 * 3)(*[int(x) for x in s])
