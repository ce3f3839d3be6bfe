"""The safetensors weight store without a GPU: header parsing, the "net."
prefix, dtypes and shapes, and refusal of malformed files."""
import struct

import numpy as np
import pytest

from anima_hip import AnimaHipError, rt
from safetensors_file import write


def _sample(rng):
    return {
        "net.blocks.0.self_attn.q_proj.weight": ("BF16", rng.integers(0, 65535, (32, 16), dtype=np.uint16)),
        "net.blocks.0.self_attn.q_norm.weight": ("BF16", rng.integers(0, 65535, (16,), dtype=np.uint16)),
        "net.x_embedder.bias": ("F32", rng.standard_normal(7).astype(np.float32)),
        "net.t_embedder.half": ("F16", rng.standard_normal((2, 3)).astype(np.float16).view(np.uint16)),
        "scalar": ("F32", np.array(3.5, np.float32)),
    }


def test_parse_names_dtypes_shapes(tmp_path):
    rng = np.random.default_rng(0)
    p = tmp_path / "m.safetensors"
    t = _sample(rng)
    write(p, t, metadata={"format": "pt", "note": "x, {y}: [z]"})
    with rt.Weights(p) as w:
        names = w.names()
        assert sorted(names) == sorted(n[4:] if n.startswith("net.") else n for n in t)
        for n, (dt, a) in t.items():
            assert w.info(n) == (dt, a.shape)
            short = n[4:] if n.startswith("net.") else n
            assert w.info(short) == (dt, a.shape)
        with pytest.raises(KeyError):
            w.info("missing.weight")


def test_empty_header_and_zero_size_tensor(tmp_path):
    p = tmp_path / "e.safetensors"
    write(p, {})
    with rt.Weights(p) as w:
        assert w.names() == []
    p2 = tmp_path / "z.safetensors"
    write(p2, {"empty": ("F32", np.zeros((0, 4), np.float32))})
    with rt.Weights(p2) as w:
        assert w.info("empty") == ("F32", (0, 4))


@pytest.mark.parametrize("case", ["truncated", "bad_json", "offsets_out", "size_mismatch",
                                  "bad_dtype", "header_too_long", "missing_field", "trailing",
                                  "deep_metadata", "deep_field", "shape_wraps"])
def test_malformed_files_are_refused(tmp_path, case):
    p = tmp_path / f"{case}.safetensors"
    a = np.arange(8, dtype=np.float32)
    if case == "truncated":
        p.write_bytes(b"\x10\x00\x00")
    elif case == "bad_json":
        write(p, {}, header_override='{"a": {"dtype": "F32", "shape": [8], "data_offsets": [0, 32]')
    elif case == "offsets_out":
        write(p, {"a": ("F32", a)}, header_override='{"a": {"dtype": "F32", "shape": [8], "data_offsets": [0, 64]}}')
    elif case == "size_mismatch":
        write(p, {"a": ("F32", a)}, header_override='{"a": {"dtype": "F32", "shape": [7], "data_offsets": [0, 32]}}')
    elif case == "bad_dtype":
        write(p, {"a": ("F32", a)}, header_override='{"a": {"dtype": "I8", "shape": [32], "data_offsets": [0, 32]}}')
    elif case == "header_too_long":
        p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    elif case == "missing_field":
        write(p, {"a": ("F32", a)}, header_override='{"a": {"dtype": "F32", "data_offsets": [0, 32]}}')
    elif case == "trailing":
        write(p, {"a": ("F32", a)}, header_override='{"a": {"dtype": "F32", "shape": [8], "data_offsets": [0, 32]}} {}')
    elif case == "deep_metadata":
        # Nesting far past the parser's cap of 64 levels: refused, not a stack overflow.
        write(p, {"a": ("F32", a)}, header_override='{"__metadata__": ' + "[" * 300000 + "}")
    elif case == "deep_field":
        write(p, {"a": ("F32", a)}, header_override='{"a": {"dtype": "F32", "shape": [8], "data_offsets": [0, 32], "x": '
              + '{"k": ' * 100000 + "1" + "}" * 100000 + "}}")
    elif case == "shape_wraps":
        # 2^62 F32 elements: the byte count wraps to 0 in 64 bits and would
        # match data_offsets [0, 0] without the overflow check.
        write(p, {}, header_override='{"w": {"dtype": "F32", "shape": [4611686018427387904], "data_offsets": [0, 0]}}')
    with pytest.raises(AnimaHipError):
        rt.Weights(p)


def test_nesting_within_the_cap_is_accepted(tmp_path):
    p = tmp_path / "nested.safetensors"
    a = np.arange(8, dtype=np.float32)
    meta = "[" * 64 + "]" * 64
    write(p, {"a": ("F32", a)},
          header_override='{"__metadata__": ' + meta + ', "a": {"dtype": "F32", "shape": [8], '
                          '"data_offsets": [0, 32]}}')
    with rt.Weights(p) as w:
        assert w.info("a") == ("F32", (8,))
    write(p, {"a": ("F32", a)}, header_override='{"__metadata__": ' + "[" + meta + "]" + "}")
    with pytest.raises(AnimaHipError, match="nesting deeper than 64"):
        rt.Weights(p)


def test_missing_file():
    with pytest.raises(AnimaHipError, match="cannot open"):
        rt.Weights("/nonexistent/model.safetensors")


def test_load_context(tmp_path):
    ctx = np.random.default_rng(1).standard_normal((1, 512, 1024)).astype(np.float32)
    np.save(tmp_path / "context_cond.npy", ctx)
    np.testing.assert_array_equal(rt.load_context(tmp_path / "context_cond.npy"), ctx)
    np.save(tmp_path / "c2.npy", ctx[0])
    assert rt.load_context(tmp_path / "c2.npy").shape == (1, 512, 1024)
    np.save(tmp_path / "obj.npy", np.array([{"a": 1}], dtype=object), allow_pickle=True)
    with pytest.raises(ValueError):
        rt.load_context(tmp_path / "obj.npy")
