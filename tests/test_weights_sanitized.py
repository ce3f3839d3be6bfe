"""The library's safetensors header parser (csrc/safetensors_header.h) under
AddressSanitizer and UndefinedBehaviorSanitizer on the CPU.

tests/native/st_header_check.cpp compiles the same header the library
compiles into weights.hip.  Every malformed-file case of the weight-store
tests, plus hostile nesting and size-overflow headers, must be either
accepted with consistent entries or refused with a message; a bounded fuzz
of mutated headers must raise no sanitizer error and accept no header whose
entries break the invariants (inside the data region, byte count = dtype
size x element count).  The reference's own reader
(vulkan/safetensors_reader.h:33-70) checks none of this.
"""
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

from safetensors_file import write

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "native", "st_header_check.cpp")
INC = os.path.join(ROOT, "anima-on-android_amd", "csrc")

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("st") / "st_header_check")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-Wall", "-Werror",
           "-I", INC, SRC, "-o", exe]
    subprocess.run(cmd, check=True)
    return exe


def _run(exe, *args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    return subprocess.run([exe, *args], capture_output=True, text=True, env=env, timeout=300)


def _cases(d):
    a = np.arange(8, dtype=np.float32)
    paths = {}

    def put(name, **kw):
        p = d / f"{name}.safetensors"
        write(p, kw.pop("tensors", {"a": ("F32", a)}), **kw)
        paths[name] = p

    put("good", metadata={"format": "pt", "nested": {"x": [1, [2, [3]]]}})
    put("bad_json",
        header_override='{"a": {"dtype": "F32", "shape": [8], "data_offsets": [0, 32]')
    put("offsets_out",
        header_override='{"a": {"dtype": "F32", "shape": [8], "data_offsets": [0, 64]}}')
    put("size_mismatch",
        header_override='{"a": {"dtype": "F32", "shape": [7], "data_offsets": [0, 32]}}')
    put("bad_dtype",
        header_override='{"a": {"dtype": "I8", "shape": [32], "data_offsets": [0, 32]}}')
    put("missing_field", header_override='{"a": {"dtype": "F32", "data_offsets": [0, 32]}}')
    put("trailing", header_override='{"a": {"dtype": "F32", "shape": [8], '
                                    '"data_offsets": [0, 32]}} {}')
    put("deep_metadata", header_override='{"__metadata__": ' + "[" * 300000 + "}")
    put("deep_field", header_override='{"a": {"dtype": "F32", "shape": [8], '
                                      '"data_offsets": [0, 32], "x": ' + "{\"k\": " * 100000
        + "1" + "}" * 100000 + "}}")
    put("shape_wraps", header_override='{"w": {"dtype": "F32", "shape": [4611686018427387904],'
                                       ' "data_offsets": [0, 0]}}')
    put("shape_product_wraps", header_override='{"w": {"dtype": "BF16", "shape": '
                                               '[4294967296, 4294967296], '
                                               '"data_offsets": [0, 0]}}')
    put("huge_offsets", header_override='{"w": {"dtype": "F32", "shape": [1], "data_offsets": '
                                        '[9223372036854775800, 9223372036854775804]}}')
    p = d / "truncated.safetensors"
    p.write_bytes(b"\x10\x00\x00")
    paths["truncated"] = p
    p = d / "header_too_long.safetensors"
    p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    paths["header_too_long"] = p
    return paths


def test_malformed_headers_under_sanitizers(checker, tmp_path):
    paths = _cases(tmp_path)
    r = _run(checker, *[str(p) for p in paths.values()])
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = {os.path.basename(ln.split(":")[0]).split(".")[0]: ln
             for ln in r.stdout.splitlines() if ln}
    assert ": ok 1" in lines["good"]
    for name in paths:
        if name != "good":
            assert "refused" in lines[name], lines[name]
    assert "nesting deeper than" in lines["deep_metadata"]
    assert "too large" in lines["shape_wraps"] or "bad shape" in lines["shape_wraps"]


def test_fuzzed_headers_under_sanitizers(checker):
    r = _run(checker, "--fuzz", "20261202", "30000")
    print(r.stdout[-2000:], r.stderr[-4000:])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "fuzz ok" in r.stdout
