"""The whole DiT on the device (anima_hip_dit_*) against the reference.

Small-width model of tests/golden/dit_ref_vectors.npz (written by the
reference's own numpy_dit.py / sampling.py on its compiled runtime): forward
and the Euler/CFG sampler, both arithmetic modes.  A full-width block (2048
wide, 16 heads x 128, MLP 8192) against the oracle's composition, which is
bit-identical to the reference's on the fixture.

Tolerances, normwise over the output (max |out - ref| / max |ref|):
  f32 mode  1e-4 (every linear layer runs on exact hi+lo bf16 terms, per
            element <= 2^-16 relative; LayerNorm sums in another order;
            device exp/erf/cos/sin round within a few ulp); the same for the
            f32x3 mode, whose attention takes its f32 operands as bf16 term
            pairs (~1e-5 relative);
  bf16 mode 3e-2 (activations rounded to bf16 before every linear layer and
            attention, as the 2e-2 attention path tolerance compounds over
            the blocks).
"""
import os
import sys

import numpy as np
import pytest

import oracle
from anima_hip import _lib, rt
from anima_hip.dit import AnimaDiT, DeviceArray, DiTConfig

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import dit_weights  # noqa: E402

TOL = {rt.F32: 1e-4, rt.BF16: 3e-2, rt.F32X3: 1e-4}


@pytest.fixture(scope="module", autouse=True)
def _init():
    rt.init()


@pytest.fixture(scope="module")
def gold():
    g = np.load(os.path.join(HERE, "golden", "dit_ref_vectors.npz"))
    cfg = {k[4:]: int(g[k]) for k in g.files if k.startswith("cfg_")}
    return g, cfg, dit_weights.make(int(g["weight_seed"]), **cfg)


def _device_table(w, norm_bf16=False):
    """Upload every tensor; returns (table for AnimaDiT, buffers to keep)."""
    table, keep = {}, []
    for name, a in w.items():
        if a.ndim == 2:
            d, dt = DeviceArray.of(a), "BF16"
        elif norm_bf16:
            d, dt = DeviceArray.of(oracle.f32_to_bf16_bits(a)), "BF16"
        else:
            d, dt = DeviceArray.of(a), "F32"
        keep.append(d)
        table[name] = (d.ptr, dt, a.shape)
    return table, keep


def _config(cfg):
    return DiTConfig.anima_2b(dim=cfg["dim"], blocks=cfg["blocks"], heads=cfg["heads"],
                              head_dim=cfg["head_dim"], mlp_hidden=cfg["mlp_hidden"],
                              ctx_dim=cfg["ctx_dim"])


def _err(out, ref):
    assert out.shape == ref.shape and np.isfinite(out).all()
    return float(np.abs(out - ref).max() / np.abs(ref).max())


@pytest.mark.parametrize("mode", [rt.F32, rt.BF16, rt.F32X3])
def test_forward_matches_reference(gold, mode):
    g, cfg, w = gold
    print(f"dit forward mode={mode} cfg={cfg}", flush=True)
    table, keep = _device_table(w, norm_bf16=(mode == rt.BF16))
    with AnimaDiT(table, _config(cfg), mode) as m:
        out = m.forward(g["fwd_x"], g["fwd_sigma"], g["fwd_ctx"])
        again = m.forward(g["fwd_x"], g["fwd_sigma"], g["fwd_ctx"])
    err = _err(out, g["fwd_out"])
    print(f"  normwise error {err:.3e}", flush=True)
    assert err <= TOL[mode]
    np.testing.assert_array_equal(again, out)  # deterministic, cache reused


@pytest.mark.parametrize("mode", [rt.F32, rt.BF16, rt.F32X3])
def test_sampler_matches_reference(gold, mode):
    g, cfg, w = gold
    print(f"dit euler mode={mode}", flush=True)
    table, keep = _device_table(w)
    with AnimaDiT(table, _config(cfg), mode) as m:
        out = m.sample(g["smp_noise"], g["smp_sigmas"], g["smp_ctx_cond"], g["smp_ctx_uncond"],
                       float(g["smp_cfg"]))
        # The reference's own loop shape (host loop over model.forward) on the
        # same model gives the same latent: the device loop only moves it.
        host = oracle.euler_sample(m.forward, g["smp_noise"], g["smp_sigmas"],
                                   g["smp_ctx_cond"], g["smp_ctx_uncond"], float(g["smp_cfg"]))
    err = _err(out, g["smp_out"])
    print(f"  normwise error {err:.3e}", flush=True)
    assert err <= TOL[mode]
    np.testing.assert_array_equal(out, host)


@pytest.mark.parametrize("mode", [rt.F32X3, rt.BF16])
def test_sampler_graph_replays_match_host_loop(gold, mode):
    """anima_hip_dit_euler_dev runs its first step directly and replays one
    captured step (a HIP graph) for the rest.  Every replay must equal the
    reference's host loop over forward: runs of 5 and 3 steps with different
    sigmas (the second replays the cached graph), then a run whose longer
    context moves the caches (the step is captured again), with direct
    forwards and host synchronisation in between."""
    g, cfg, w = gold
    table, keep = _device_table(w)
    noise, c_c, c_u = g["smp_noise"], g["smp_ctx_cond"], g["smp_ctx_uncond"]
    # The third run's context is 3 tokens longer: its caches move, so the
    # captured step must be recorded again.
    longer = [np.concatenate([c, c[:, :3]], axis=1) for c in (c_c, c_u)]
    with AnimaDiT(table, _config(cfg), mode) as m:
        for n, shift, (cc, cu) in ((5, 1.0, (c_c, c_u)), (3, 3.0, (c_c, c_u)),
                                   (3, 2.0, longer)):
            sig = oracle.z_image_sigmas(n, 1.0, shift)
            print(f"dit graph mode={mode} steps={n} ctx={cc.shape[1]}", flush=True)
            dev = m.sample(noise, sig, cc, cu, 5.0)
            host = oracle.euler_sample(m.forward, noise, sig, cc, cu, 5.0)
            np.testing.assert_array_equal(dev, host)
            assert np.isfinite(dev).all() and not np.array_equal(dev, noise)


def test_sampler_graph_at_4096_tokens_matches_host_loop():
    """The device sampler loop at the Anima 2B widths on a 16 x 128 x 64
    latent (the CFG pair: 2 x 2048 tokens), where the f32x3 self-attention
    runs the fused q/k/v product inside the captured step: three steps (the
    first direct, two replays) equal the host loop over forward bit for bit."""
    cfg = dict(dim=2048, blocks=1, heads=16, head_dim=128, mlp_hidden=8192, ctx_dim=1024)
    w = dit_weights.make(7401, **cfg)
    rng = np.random.default_rng(7402)
    noise = rng.standard_normal((1, 16, 128, 64), dtype=np.float32)
    c_c, c_u = (rng.standard_normal((1, 32, 1024), dtype=np.float32) * np.float32(0.5)
                for _ in range(2))
    table, keep = _device_table(w)
    sig = oracle.z_image_sigmas(3, 1.0, 3.0)
    print("dit graph f32x3, 2 x 2048 tokens", flush=True)
    with AnimaDiT(table, DiTConfig.anima_2b(blocks=1), rt.F32X3) as m:
        dev = m.sample(noise, sig, c_c, c_u, 5.0)
        host = oracle.euler_sample(m.forward, noise, sig, c_c, c_u, 5.0)
    np.testing.assert_array_equal(dev, host)
    assert np.isfinite(dev).all() and not np.array_equal(dev, noise)


def test_context_batch_one_broadcasts(gold):
    g, cfg, w = gold
    table, keep = _device_table(w)
    ctx1 = g["fwd_ctx"][:1]
    with AnimaDiT(table, _config(cfg), rt.F32) as m:
        a = m.forward(g["fwd_x"], g["fwd_sigma"], ctx1)
        b = m.forward(g["fwd_x"], g["fwd_sigma"], np.concatenate([ctx1, ctx1]))
    assert _err(a, b) <= 1e-6


def test_full_width_block_vs_oracle():
    """One block at the Anima 2B widths on a 2 x 6 x 8 latent (12 tokens per
    entry) against the oracle's composition."""
    cfg = dict(dim=2048, blocks=1, heads=16, head_dim=128, mlp_hidden=8192, ctx_dim=1024)
    w = dit_weights.make(7201, **cfg)
    rng = np.random.default_rng(7202)
    x = rng.standard_normal((2, 16, 1, 6, 8), dtype=np.float32)
    sigma = np.array([0.7, 0.7], np.float32)
    ctx = rng.standard_normal((2, 24, 1024), dtype=np.float32) * np.float32(0.5)
    print("dit full-width block", flush=True)
    ref = oracle.dit_forward(x, sigma, ctx, w, 1, 16, 128,
                             sdpa=lambda a, b, c: oracle.flash_sdpa(a, b, c, threads=8))
    table, keep = _device_table(w)
    for mode in (rt.F32, rt.BF16, rt.F32X3):
        with AnimaDiT(table, DiTConfig.anima_2b(blocks=1), mode) as m:
            err = _err(m.forward(x, sigma, ctx), ref)
        print(f"  mode {mode}: normwise error {err:.3e}", flush=True)
        assert err <= TOL[mode]


def test_full_width_block_at_4096_tokens_vs_oracle(monkeypatch):
    """One block at the Anima 2B widths on a 2 x 16 x 128 x 64 latent (2048
    tokens per entry, M = 4096): the whole DiT's large-M paths, i.e. in the
    f32x3 mode the fused q/k/v product whose epilogue writes the attention's
    prepared operands (anima_hip_qkv_projection_dev's kernel), in the f32 mode
    the library product on term rows plus the one-launch prologue, in bf16 the
    bf16 ones; the 8-wave flash grids.  Against the oracle's composition with
    its bf16 GEMMs taken as float64 products of the decoded weights
    (tests/fullsize.py proj_f64: the same mathematics, rounded once) so that it
    finishes in seconds, and its attention on host threads."""
    import fullsize
    monkeypatch.setattr(oracle, "gemm_bf16", fullsize.proj_f64)
    cfg = dict(dim=2048, blocks=1, heads=16, head_dim=128, mlp_hidden=8192, ctx_dim=1024)
    w = dit_weights.make(7301, **cfg)
    rng = np.random.default_rng(7302)
    x = rng.standard_normal((2, 16, 1, 128, 64), dtype=np.float32)
    sigma = np.array([0.9, 0.6], np.float32)
    ctx = rng.standard_normal((2, 64, 1024), dtype=np.float32) * np.float32(0.5)
    print("dit full-width block, 4096 tokens", flush=True)
    ref = oracle.dit_forward(x, sigma, ctx, w, 1, 16, 128, sdpa=fullsize.threaded_sdpa)
    table, keep = _device_table(w)
    for mode in (rt.F32X3, rt.F32, rt.BF16):
        with AnimaDiT(table, DiTConfig.anima_2b(blocks=1), mode) as m:
            err = _err(m.forward(x, sigma, ctx), ref)
        print(f"  mode {mode}: normwise error {err:.3e}", flush=True)
        assert err <= TOL[mode]


def test_create_and_call_errors(gold):
    g, cfg, w = gold
    table, keep = _device_table(w)
    bad = dict(table)
    del bad["blocks.1.mlp.layer2.weight"]
    with pytest.raises(_lib.AnimaHipError, match="missing weight blocks.1.mlp.layer2"):
        AnimaDiT(bad, _config(cfg))
    bad = dict(table)
    p, dt, s = bad["blocks.0.self_attn.q_proj.weight"]
    bad["blocks.0.self_attn.q_proj.weight"] = (p, dt, (s[0], s[1] // 2))
    with pytest.raises(_lib.AnimaHipError, match="expected"):
        AnimaDiT(bad, _config(cfg))
    bad = dict(table)
    p, dt, s = bad["final_layer.linear.weight"]
    bad["final_layer.linear.weight"] = (p, "F32", s)
    with pytest.raises(_lib.AnimaHipError, match="must be BF16"):
        AnimaDiT(bad, _config(cfg))
    with pytest.raises(_lib.AnimaHipError, match="configuration"):
        AnimaDiT(table, DiTConfig.anima_2b(max_batch=5))
    lib = _lib.load()
    with AnimaDiT(table, _config(cfg)) as m:
        x = DeviceArray.of(g["fwd_x"])
        out = DeviceArray(g["fwd_x"].nbytes)
        sig = (np.ctypeslib.as_ctypes(g["fwd_sigma"]))
        ok = lib.anima_hip_dit_forward_dev(m.handle, x.ptr, 16 * 70, sig, 2, 1, 7, 10, x.ptr,
                                           out.ptr, x.ptr, 1 << 30, None)
        assert not ok and "context" in _lib.last_error()
        ok = lib.anima_hip_dit_euler_dev(m.handle, x.ptr, sig, 1, 5.0, 7, 10, x.ptr, x.ptr, 0,
                                         None)
        assert not ok and "context of 2 entries" in _lib.last_error()
        m.set_context(g["fwd_ctx"])
        ok = lib.anima_hip_dit_forward_dev(m.handle, x.ptr, 16 * 70, sig, 2, 1, 7, 10, x.ptr,
                                           out.ptr, x.ptr, 64, None)
        assert not ok and "scratch" in _lib.last_error()
        ok = lib.anima_hip_dit_forward_dev(m.handle, x.ptr, 16 * 70, sig, 3, 1, 7, 10, x.ptr,
                                           out.ptr, x.ptr, 1 << 30, None)
        assert not ok and "batch" in _lib.last_error()


def test_model_from_checkpoint_file(gold, tmp_path):
    """The reference's on-disk format: safetensors with the "net." prefix,
    BF16 linear and norm weights (as the checkpoint stores them) and a tensor
    the model does not read; AnimaDiT(Weights(path)) computes exactly what the
    device-table model with the same values does."""
    import safetensors_file
    g, cfg, w = gold
    tensors = {"net." + k: ("BF16", a if a.ndim == 2 else oracle.f32_to_bf16_bits(a))
               for k, a in w.items()}
    tensors["net.pos_embedder.seq"] = ("F32", np.arange(8, dtype=np.float32))
    path = tmp_path / "dit.safetensors"
    safetensors_file.write(path, tensors, metadata={"format": "pt"})
    print("dit from file", flush=True)
    with rt.Weights(path) as store:
        with AnimaDiT(store, _config(cfg), rt.F32) as m:
            a = m.forward(g["fwd_x"], g["fwd_sigma"], g["fwd_ctx"])
    table, keep = _device_table(w)
    with AnimaDiT(table, _config(cfg), rt.F32) as m:
        b = m.forward(g["fwd_x"], g["fwd_sigma"], g["fwd_ctx"])
    np.testing.assert_array_equal(a, b)
    assert _err(a, g["fwd_out"]) <= TOL[rt.F32]
