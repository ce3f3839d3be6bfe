"""The C-ABI library without a GPU: it loads, exports every declared symbol,
and reports errors instead of returning silently (no compute is launched)."""
import ctypes as ct
import os
import re
import subprocess

import numpy as np
import pytest

import anima_hip
from anima_hip import _lib, rt

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "anima_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(anima_(?:rt|hip)_\w+)\s*\(", text)))


def test_library_built_and_loads():
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build()"
    _lib.load()


def test_every_declared_symbol_is_exported_and_bound():
    names = declared_functions()
    assert "anima_rt_run_sdpa_flash" in names and len(names) >= 10
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [n for n in names if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    assert sorted(_lib.SIGNATURES) == names, "ctypes declarations out of sync with the header"


def _prototypes():
    """name -> (return type, [parameter types]) parsed from the header."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    text = "\n".join(ln for ln in text.splitlines() if not ln.lstrip().startswith("#"))
    protos = {}
    for m in re.finditer(r"^([\w ]+?\**)\s*\b(anima_(?:rt|hip)_\w+)\s*\(([^)]*)\)\s*;", text,
                         flags=re.M):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
        plist = [] if params in ("", "void") else [p.strip() for p in params.split(",")]
        types = []
        for prm in plist:
            prm = re.sub(r"\b\w+$", "", prm).strip() if not prm.endswith("*") else prm
            types.append(" ".join(prm.split()))
        protos[name] = (" ".join(ret.split()), types)
    return protos


def _ctype_of(c):
    import ctypes as ct
    c = c.replace("const ", "").strip()
    if c.endswith("*"):
        base = c[:-1].strip()
        return {"int64_t": "int64*", "int": "int*", "char": "char*", "float": "float*"}.get(
            base, "ptr")
    return {"bool": ct.c_bool, "int": ct.c_int, "float": ct.c_float, "size_t": ct.c_size_t,
            "int64_t": ct.c_int64, "void": None}[c]


def test_ctypes_declarations_match_header_prototypes():
    import ctypes as ct
    protos = _prototypes()
    assert set(protos) == set(_lib.SIGNATURES)
    for name, (ret, params) in protos.items():
        res, args = _lib.SIGNATURES[name]
        assert len(args) == len(params), f"{name}: {len(args)} ctypes args, header has {len(params)}"
        for i, (c, py) in enumerate(zip(params, args)):
            want = _ctype_of(c)
            if want == "ptr":
                assert py is ct.c_void_p, f"{name} arg {i}: {c}"
            elif want == "int64*":
                assert py is ct.POINTER(ct.c_int64), f"{name} arg {i}: {c}"
            elif want == "int*":
                assert py is ct.POINTER(ct.c_int), f"{name} arg {i}: {c}"
            elif want == "char*":
                assert py is ct.c_char_p, f"{name} arg {i}: {c}"
            elif want == "float*":
                assert py in (ct.POINTER(ct.c_float), ct.c_void_p), f"{name} arg {i}: {c}"
            else:
                assert py is want, f"{name} arg {i}: {c} vs {py}"
        rwant = _ctype_of(ret)
        if rwant in ("ptr", "char*"):
            assert res in (ct.c_void_p, ct.c_char_p), name
        else:
            assert res is rwant, f"{name} return {ret} vs {res}"


def test_reference_drop_in_signatures():
    # The ctypes argtypes the reference's binding uses (anima_rt_ops.py:28-34).
    import ctypes as ct
    sig = _lib.SIGNATURES
    assert sig["anima_rt_run_sdpa_flash"][1] == [ct.c_void_p] * 4 + [ct.c_int] * 4 + [
        ct.c_float, ct.c_bool]
    assert sig["anima_rt_run_sdpa"][1] == sig["anima_rt_run_sdpa_flash"][1]
    assert sig["anima_rt_run_rmsnorm"][1] == [ct.c_void_p] * 3 + [ct.c_int] * 2 + [ct.c_float]
    assert sig["anima_rt_run_rope"][1] == [ct.c_void_p] * 3 + [ct.c_int] * 3
    for name in ("anima_rt_init", "anima_rt_run_sdpa_flash", "anima_rt_run_sdpa",
                 "anima_rt_run_rmsnorm", "anima_rt_run_rope"):
        assert sig[name][0] is ct.c_bool


# The symbols and ctypes argument types the reference's own binding declares
# at import time (anima_rt/scripts/anima_rt_ops.py:11-34); a library missing
# any of them cannot be loaded in its place.
_P, _I, _F = ct.c_void_p, ct.c_int, ct.c_float
REFERENCE_BINDING = {
    "anima_rt_run_gelu": [_P, _P, _I],
    "anima_rt_run_silu": [_P, _P, _I],
    "anima_rt_run_layernorm": [_P, _P, _I, _I, _F],
    "anima_rt_run_rmsnorm": [_P, _P, _P, _I, _I, _F],
    "anima_rt_run_softmax": [_P, _P, _I, _I],
    "anima_rt_run_gemm_fp32": [_P, _P, _P, _I, _I, _I],
    "anima_rt_run_gemm_bf16": [_P, _P, _P, _I, _I, _I],
    "anima_rt_run_sdpa": [_P] * 4 + [_I] * 4 + [_F, ct.c_bool],
    "anima_rt_run_sdpa_flash": [_P] * 4 + [_I] * 4 + [_F, ct.c_bool],
    "anima_rt_run_rope": [_P, _P, _P, _I, _I, _I],
}


def test_reference_binding_loads_against_this_library():
    lib = ct.CDLL(_lib.LIB_PATH)
    lib.anima_rt_init.restype = ct.c_bool
    for name, args in REFERENCE_BINDING.items():
        fn = getattr(lib, name)  # AttributeError if the symbol were missing
        fn.argtypes = args
        fn.restype = ct.c_bool
        assert _lib.SIGNATURES[name] == (ct.c_bool, args), name
    assert _lib.SIGNATURES["anima_rt_run_bias_add"] == (ct.c_bool, [_P, _P, _I, _I])


def test_rmsnorm_and_math_sdpa_require_init():
    # anima_rt.cpp:47 and :84 return false before anima_rt_init(); so does the
    # drop-in, and the Python layer turns that into an exception.
    rt.destroy()
    lib = _lib.load()
    x = np.ones((2, 8), np.float32)
    out = np.zeros_like(x)
    assert not lib.anima_rt_run_rmsnorm(x.ctypes.data, None, out.ctypes.data, 2, 8, 1e-6)
    assert "anima_rt_init" in _lib.last_error()
    with pytest.raises(anima_hip.AnimaHipError):
        rt.rmsnorm(x)
    q = np.ones((1, 4, 8), np.float32)
    with pytest.raises(anima_hip.AnimaHipError, match="anima_rt_init"):
        rt.sdpa_math(q, q, q)
    # anima_rt.cpp:25, :30, :38, :54: the activations, LayerNorm and softmax
    # need the backend too.
    for fn in (rt.gelu, rt.silu, rt.layernorm, rt.softmax):
        with pytest.raises(anima_hip.AnimaHipError, match="anima_rt_init"):
            fn(x)
    # bias_add with a null bias does nothing and needs no init
    # (gemm_backend.cpp:176); zero-sized inputs succeed after init-free checks.
    c = np.ones((2, 3), np.float32)
    assert lib.anima_rt_run_bias_add(c.ctypes.data, None, 2, 3)
    assert np.all(c == 1.0)
    # The timing hook has nothing to report until a host call completes.
    assert not lib.anima_hip_last_call_ms(None, None)
    assert "no host-pointer call" in _lib.last_error()


def test_python_shape_validation():
    q = np.zeros((2, 4, 8), np.float32)
    with pytest.raises(ValueError):
        rt.sdpa_flash(q, np.zeros((2, 5, 9), np.float32), np.zeros((2, 5, 9), np.float32))
    with pytest.raises(ValueError):
        rt.rope(q, np.zeros((3, 4, 2, 2), np.float32))


@pytest.mark.parametrize("entry", ["anima_hip_flash_bf16_dev", "anima_hip_flash_x3_dev"])
@pytest.mark.parametrize("scale", [float("nan"), 0.0, -0.088, float("inf")])
def test_bf16_and_x3_entries_refuse_a_bad_scale_before_any_device_work(entry, scale):
    # These kernels fold the scale into exp2's argument and take the row max
    # on raw scores, so they need a positive finite scale.  The check runs on
    # the host before the device context is touched (no GPU needed here).
    lib = _lib.load()
    fn = getattr(lib, entry)
    ok = fn(None, None, None, None, 1, 1, 1, 1, 128, None, None, None, None, ct.c_float(scale),
            False, None)
    assert not ok
    assert "scale must be positive and finite" in _lib.last_error()


def test_linear_scratch_holds_the_small_m_partials_only_where_that_kernel_runs():
    # anima_hip_linear_scratch_bytes: the bf16 terms (two for the f32 modes),
    # plus 16 MiB of split-K partials where the hand-written small-M GEMM
    # replaces the library: M <= 1024, K a multiple of 64, and two terms or
    # K >= 8192 (pure host arithmetic, no GPU).
    lib = _lib.load()
    part = 16 << 20
    terms = lambda M, K, n: -(-(M * (-(-K // 8) * 8) * 2) // 256) * 256 * n  # noqa: E731
    for M, K, mode, extra in [(512, 2048, rt.F32, True), (512, 2048, rt.F32X3, True),
                              (512, 2048, rt.BF16, False), (512, 8192, rt.BF16, True),
                              (1024, 4096, rt.F32, True), (1025, 4096, rt.F32, False),
                              (512, 2056, rt.F32, False), (77, 64, rt.F32, True)]:
        n = 1 if mode == rt.BF16 else 2
        want = terms(M, K, n) + (part if extra else 0)
        assert lib.anima_hip_linear_scratch_bytes(M, K, mode) == want, (M, K, mode)
