"""Weights from a safetensors file on the device: the copies hold exactly the
file's bytes (or their f32 widening), stay resident, and drive the attention
sub-block like the same weights passed as arrays."""
import ctypes as ct

import numpy as np
import pytest

import oracle
from anima_hip import _lib, rt
from safetensors_file import write

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


def _download(ptr, nbytes, dtype, shape):
    import devmem
    out = np.empty(shape, dtype)
    assert out.nbytes == nbytes
    assert devmem.hip().hipDeviceSynchronize() == 0
    assert devmem.hip().hipMemcpy(out.ctypes.data, ptr, nbytes, 2) == 0
    return out


def test_device_copies_exact(tmp_path):
    rng = np.random.default_rng(5)
    bf = rng.integers(0, 0x7F80, (64, 48), dtype=np.uint16)  # finite bf16 patterns
    f16 = rng.standard_normal((5, 7)).astype(np.float16)
    f32 = rng.standard_normal(33).astype(np.float32)
    p = tmp_path / "w.safetensors"
    write(p, {"net.a.weight": ("BF16", bf), "net.b": ("F16", f16.view(np.uint16)), "c": ("F32", f32)})
    with rt.Weights(p) as w:
        d = w.device("a.weight")
        assert w.device("net.a.weight") == d  # uploaded once, resident
        np.testing.assert_array_equal(_download(d, bf.nbytes, np.uint16, bf.shape), bf)
        wide = _download(w.device("a.weight", as_f32=True), bf.size * 4, np.float32, bf.shape)
        np.testing.assert_array_equal(wide, oracle.bf16_bits_to_f32(bf))
        np.testing.assert_array_equal(
            _download(w.device("b", as_f32=True), f16.size * 4, np.float32, f16.shape),
            f16.astype(np.float32))
        np.testing.assert_array_equal(_download(w.device("c"), f32.nbytes, np.float32, f32.shape), f32)
        with pytest.raises(Exception):
            w.device("nope")


def test_block_from_file_weights(tmp_path):
    """Self-attention sub-block with wq/wk/wv/wo and q/k norm weights read from
    a file (names as in the reference's checkpoint) equals the same call with
    the arrays uploaded directly."""
    from devmem import DevBuf
    rng = np.random.default_rng(9)
    B, S, DM, H, D = 1, 64, 256, 2, 128
    pre = "net.blocks.0.self_attn."
    ws = {n: oracle.f32_to_bf16_bits(rng.standard_normal(shape, dtype=np.float32) * 0.05)
          for n, shape in (("q_proj", (H * D, DM)), ("k_proj", (H * D, DM)),
                           ("v_proj", (H * D, DM)), ("output_proj", (DM, H * D)))}
    norms = {n: oracle.f32_to_bf16_bits(rng.uniform(0.5, 1.5, D).astype(np.float32))
             for n in ("q_norm", "k_norm")}
    p = tmp_path / "block.safetensors"
    write(p, {**{pre + n + ".weight": ("BF16", a) for n, a in ws.items()},
              **{pre + n + ".weight": ("BF16", a) for n, a in norms.items()}})
    x = rng.standard_normal((B * S, DM), dtype=np.float32)
    mod = (rng.standard_normal((B, 3, DM)) * 0.5).astype(np.float32)
    lib = _lib.load()
    n = lib.anima_hip_attention_block_scratch_bytes(None, B, S, DM, H, D, rt.F32)
    scratch = DevBuf(n)
    dmod = DevBuf.of(mod)

    def run(ptrs):
        dx = DevBuf.of(x)
        ok = lib.anima_hip_attention_block_dev(dx.addr, dmod.addr, *ptrs, None, None, B, S, DM,
                                               H, D, ct.c_float(1e-6), rt.F32, scratch.addr, n,
                                               None)
        _lib.check(ok, "attention_block_dev")
        return dx.get(x.shape)

    arrays = [DevBuf.of(ws[k]) for k in ("q_proj", "k_proj", "v_proj", "output_proj")]
    arrays += [DevBuf.of(oracle.bf16_bits_to_f32(norms[k])) for k in ("q_norm", "k_norm")]
    ref = run([a.addr for a in arrays])
    with rt.Weights(p) as w:
        ptrs = [w.device(f"blocks.0.self_attn.{k}.weight")
                for k in ("q_proj", "k_proj", "v_proj", "output_proj")]
        ptrs += [w.device(f"blocks.0.self_attn.{k}.weight", as_f32=True) for k in ("q_norm", "k_norm")]
        out = run(ptrs)
    np.testing.assert_array_equal(out, ref)
    assert np.abs(out - x).max() > 0  # the block did update the stream
