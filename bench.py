#!/usr/bin/env python3
"""Attention throughput of the Anima DiT hot path on one MI355X.

Workload (the configuration the headline metric is quoted on): self-attention
at 1024x1024 output, B=2 (CFG cond+uncond), H=16, S_q=S_kv=4096 tokens
(64x64 patch grid), head_dim 128.  Inputs are seeded N(0,1) q/k/v projections
in NumpyDiT's [B,S,H,D] layout, already resident in HBM.

One step = the whole device-resident hot path over that batch:
  prologue(q) + prologue(k)   per-head RMSNorm (w=1, eps 1e-6) + 3D RoPE
  flash attention             softmax(QK^T/sqrt(D)) V, output in [B,S,H,D]
FLOPs per step = 4*B*H*S_q*S_kv*D (softmax and prologue not counted).

Prints ONE JSON line on stdout (progress goes to stderr).  `roofline` covers
the flash kernel alone: its average duration is measured with HIP events
recorded on the stream it is launched on, around every launch in the timed
region.  `cpu_baseline` times anima_rt's own flash attention (the reference
built from source in oracle/_ref when present, else the bit-identical C
restatement) on a bounded sample of the same heads on this host's CPU.
"""
import argparse
import ctypes as ct
import json
import math
import os
import sys
import threading
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "anima-on-android_amd"))

PEAK_TFLOPS = {"f32": 157.3, "bf16": 2516.6}  # MI355X dense MFMA peaks
HBM_GBPS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "flash_traffic.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--variant", choices=["f32", "bf16"], default="f32",
                    help="f32: f32 MFMA on f32 inputs; bf16: bf16 inputs, f32 accumulate")
    ap.add_argument("--cpu-heads", type=int, default=8,
                    help="(batch, head) slices timed single-core for cpu_baseline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    return ap.parse_args()


def traffic_for(kernel, workload):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE,
    WRITE_SIZE), scaled by a copy-kernel calibration; None until measured."""
    try:
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f).get(kernel)
    except (OSError, ValueError):
        return None
    if not rec or rec.get("workload") != workload:
        return None
    return rec.get("bytes_per_launch")


def cpu_baseline(qn, kn, v, B, H, S, D, heads):
    """anima_rt flash attention on `heads` (b, h) slices, one core, plus the
    same per-head work spread over this host's cores."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle

    kind = "reference" if oracle.ref_available() else "port"
    fn = oracle.ref_flash_sdpa if kind == "reference" else oracle.flash_sdpa
    scale = 1.0 / math.sqrt(D)

    def slice_heads(x, n):  # [B,S,H,D] device -> n contiguous [S,D] f32 host slices
        sl = []
        for i in range(n):
            b, h = divmod(i, H)
            sl.append(x[b, :, h, :].float().contiguous().cpu().numpy())
        return sl

    n1 = max(1, min(heads, B * H))
    qs, ks, vs = slice_heads(qn, n1), slice_heads(kn, n1), slice_heads(v, n1)
    log(f"[bench] cpu baseline: {n1} head(s) of {S}x{S}, 1 core ({kind})")
    t0 = time.perf_counter()
    fn(np.stack(qs), np.stack(ks), np.stack(vs), scale)
    dt = time.perf_counter() - t0
    flops = 4.0 * n1 * S * S * D
    single = {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": kind,
              "sample": f"{n1} of {B * H} (batch,head) slices of the 4096x4096 self-attention, "
                        f"anima_rt flash_attention, {dt:.2f} s wall",
              "seconds": dt}

    threads = max(1, min(16, os.cpu_count() or 1, B * H))
    if threads > 1:
        qs, ks, vs = slice_heads(qn, threads), slice_heads(kn, threads), slice_heads(v, threads)
        log(f"[bench] cpu baseline: {threads} heads on {threads} threads")

        def work(i):
            fn(qs[i][None], ks[i][None], vs[i][None], scale)

        ts = [threading.Thread(target=work, args=(i,)) for i in range(threads)]
        t0 = time.perf_counter()
        for t in ts:
            t.start()
        for t in ts:
            t.join()
        dtm = time.perf_counter() - t0
        multi = {"value": 4.0 * threads * S * S * D / dtm / 1e12, "unit": "TFLOP/s",
                 "cores": threads, "kind": kind,
                 "sample": f"{threads} slices, one per thread (heads are independent)",
                 "seconds": dtm}
    else:
        multi = None
    return single, multi


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this attention path runs on a single MI355X "
              "(the 32 (batch, head) slices shard across GPUs with no exchange; "
              "multi-GPU runs are not part of this build).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from anima_hip import _lib
    from anima_hip.rope import generate_rope_freqs

    B, H, S, D = 2, 16, 4096, 128
    workload = "self-attention 4096x4096, B=2 H=16 D=128 (64x64 grid, RMSNorm+3D RoPE)"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = _lib.load()
    _lib.check(lib.anima_rt_init(), "anima_rt_init")

    log("[bench] generating inputs")
    rng = np.random.default_rng(3003)
    host = [rng.standard_normal((B, S, H, D), dtype=np.float32) for _ in range(3)]
    q, k, v = (torch.from_numpy(x).to(dev) for x in host)
    bf16 = args.variant == "bf16"
    qn = torch.empty(q.shape, dtype=torch.bfloat16 if bf16 else torch.float32, device=dev)
    kn = torch.empty_like(qn)
    o = torch.empty_like(q)
    sp = lib.anima_hip_vt_padded_len(S)
    vt = torch.empty((B, H, D, sp), dtype=torch.bfloat16, device=dev) if bf16 else None
    freqs = torch.from_numpy(generate_rope_freqs(64, 64)).to(dev)
    ones = torch.ones(D, device=dev)
    st = torch.cuda.Stream(device=dev)
    stp = ct.c_void_p(st.cuda_stream)
    bshd = _lib.strides([S * H * D, D, H * D])  # [B,S,H,D] viewed as [B,H,S,D]
    scale = ct.c_float(1.0 / math.sqrt(D))

    def prologue(x, y):
        flags = 1 | (2 if bf16 else 0)  # RMSNorm (+ bf16 output)
        ok = lib.anima_hip_qk_prologue_dev(x.data_ptr(), y.data_ptr(), ones.data_ptr(),
                                           freqs.data_ptr(), B, S, H, D, bshd, bshd,
                                           ct.c_float(1e-6), flags, stp)
        _lib.check(ok, "qk_prologue")

    def flash():
        if bf16:
            ok = lib.anima_hip_flash_bf16_dev(qn.data_ptr(), kn.data_ptr(), vt.data_ptr(),
                                              o.data_ptr(), B, H, S, S, D, bshd, bshd, None,
                                              bshd, scale, False, stp)
        else:
            ok = lib.anima_hip_flash_f32_dev(qn.data_ptr(), kn.data_ptr(), v.data_ptr(),
                                             o.data_ptr(), B, H, S, S, D, bshd, bshd, bshd,
                                             bshd, scale, False, stp)
        _lib.check(ok, f"flash_{args.variant}")

    def step(ev=None):
        prologue(q, qn)
        prologue(k, kn)
        if bf16:
            _lib.check(lib.anima_hip_pack_vt_dev(v.data_ptr(), vt.data_ptr(), B, H, S, D, bshd,
                                                 None, stp), "pack_vt")
        if ev is not None:
            ev[0].record(st)
        flash()
        if ev is not None:
            ev[1].record(st)

    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        for _ in range(args.warmup):
            step()
    torch.cuda.synchronize()
    log(f"[bench] warmup done ({args.warmup} steps); timing {args.steps} steps")

    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        t_start.record(st)
        for i in range(args.steps):
            step(evs[i])
        t_end.record(st)
    torch.cuda.synchronize()
    ms_step = t_start.elapsed_time(t_end) / args.steps
    ms_flash = sum(a.elapsed_time(b) for a, b in evs) / args.steps
    if not torch.isfinite(o).all():
        raise RuntimeError("non-finite attention output")
    log(f"[bench] step {ms_step:.3f} ms, flash kernel {ms_flash:.3f} ms")

    flops = 4.0 * B * H * S * S * D
    value = flops / (ms_step * 1e-3) / 1e12
    achieved = flops / (ms_flash * 1e-3) / 1e12
    peak = PEAK_TFLOPS[args.variant]
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak,
                "unit": "TFLOP/s", "frac": round(achieved / peak, 4),
                "traffic": traffic_for(f"flash_{args.variant}", workload),
                "kernel": f"flash_{args.variant}_d128", "avg_launch_ms": round(ms_flash, 4)}

    cpu = multi = None
    if not args.no_cpu_baseline:
        cpu, multi = cpu_baseline(qn, kn, v, B, H, S, D, args.cpu_heads)

    line = {
        "metric": "attention TFLOP/s + % MFMA peak at 4096 tok B=2 H16 D128; speedup vs host CPU",
        "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": args.variant,
        "data": "synthetic (seeded N(0,1) q/k/v, unit RMSNorm weights)",
        "config": {"workload": workload, "B": B, "H": H, "S_q": S, "S_kv": S, "D": D,
                   "step": "qk prologue (RMSNorm+RoPE) x2 " + ("+ V^T bf16 pack " if bf16 else "")
                           + "+ flash attention",
                   "mfma": "v_mfma_f32_32x32x16_bf16" if bf16 else "v_mfma_f32_32x32x2_f32"},
        "pct_mfma_peak": round(100.0 * value / peak, 2),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_baseline_multicore": multi,
        "speedup_vs_cpu": None if cpu is None else round(value / cpu["value"], 1),
        "speedup_vs_cpu_multicore": None if multi is None else round(value / multi["value"], 1),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
