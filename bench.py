#!/usr/bin/env python3
"""Benchmark of the MI355X GQA flash-attention hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--all] [--no-cpu]

A step is one forward + backward of the headline Gemma4 global layer: B=1, Hq=32, Hkv=4
(GQA 8:1), N=16384, D=512, full causal, bf16, synthetic N(0,1) inputs from a seeded CPU
generator, resident in HBM before timing starts. Besides the headline ``value``
(fwd+bwd TFLOPS) the line carries forward TFLOPS, the D=256 sliding-window layer
(16:8, W=1024, N=16384) and per-kernel times of the forward, dQ and dK/dV kernels.

FLOP charge (the reference's convention, /root/reference/benchmarks/run_final_benchmark.py
217-224): causal fwd 2*B*Hq*N^2*D, fwd+bwd 7*B*Hq*N^2*D. Sliding window: with
P = W(W+1)/2 + W(N-W) attended pairs, fwd 4*B*Hq*D*P and fwd+bwd 14*B*Hq*D*P.
Percentages are of MI355X dense fp16/bf16 MFMA peak, 2516.6 TFLOP/s.

Prints exactly one JSON line on stdout.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_TFLOPS = 2516.6  # MI355X dense bf16/fp16 MFMA
METRIC = "fwd & fwd+bwd TFLOPS (D=512 causal, D=256 SWA) at N=16K; % of MFMA peak"
H100_FWDBWD_TFLOPS = 117.1  # reference, D=512 causal 32:4 N=16384 fwd+bwd (attn_only_all_n.json:200-210)

WORKLOADS = {
    "d512_causal_gqa8_n16k": dict(B=1, Hq=32, Hkv=4, N=16384, D=512, causal=True, window=0, dtype="bf16", amp=1.0),
    "d256_swa1024_gqa2_n16k": dict(B=1, Hq=16, Hkv=8, N=16384, D=256, causal=True, window=1024, dtype="bf16", amp=1.0),
    "c2_d512_causal_gqa8_n8k": dict(B=1, Hq=32, Hkv=4, N=8192, D=512, causal=True, window=0, dtype="bf16", amp=1.0),
    "c4_d512_causal_gqa8_n32k": dict(B=1, Hq=16, Hkv=2, N=32768, D=512, causal=True, window=0, dtype="fp16", amp=0.5),
}


def charged_flops(w, passes):
    B, Hq, N, D, W = w["B"], w["Hq"], w["N"], w["D"], w["window"]
    if w["causal"] and 0 < W < N:
        P = W * (W + 1) / 2 + W * (N - W)
        return (4 if passes == "fwd" else 14) * B * Hq * D * P
    if w["causal"]:
        return (2 if passes == "fwd" else 7) * B * Hq * N * N * D
    return (4 if passes == "fwd" else 14) * B * Hq * N * N * D


def kernel_flops(w):
    """Algorithmic flops per launch of each kernel: 2*D per pair-product per attended
    (query, key) pair; forward 2 products, dQ 3 (S, dP, dQ), dKV 4 (S, dP, dV, dK)."""
    unit = charged_flops(w, "fwd") / 2.0  # = 2*D*pairs (causal convention)
    return {"fwd": 2 * unit, "dq": 3 * unit, "dkv": 4 * unit}


def make_inputs(w, device):
    import torch

    dt = {"bf16": torch.bfloat16, "fp16": torch.float16}[w["dtype"]]
    g = torch.Generator().manual_seed(0)
    shapes = [(w["B"], w["Hq"], w["N"], w["D"]), (w["B"], w["Hkv"], w["N"], w["D"]),
              (w["B"], w["Hkv"], w["N"], w["D"]), (w["B"], w["Hq"], w["N"], w["D"])]
    return [(torch.randn(*s, generator=g) * w["amp"]).to(device=device, dtype=dt) for s in shapes]


def time_loop(fn, iters, warmup):
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters


def bench_workload(name, w, steps, warmup, device, kernels=True):
    import torch

    import gemma_triton_flash_attn_amd as gfa
    from gemma_triton_flash_attn_amd import _lib
    from gemma_triton_flash_attn_amd.attention import _backward, _forward

    print(f"[bench] {name}: {w}", file=sys.stderr, flush=True)
    q, k, v, do = make_inputs(w, device)
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
    scale = w["D"] ** -0.5

    def fwd():
        return gfa.flash_attn_gqa_train(qg, kg, vg, causal=w["causal"], slide_size=w["window"])

    def fwd_bwd():
        qg.grad = kg.grad = vg.grad = None
        o = fwd()
        o.backward(do)

    res = {}
    with torch.no_grad():
        ms_fwd = time_loop(lambda: fwd(), steps, warmup)
    ms_fb = time_loop(fwd_bwd, steps, warmup)
    res["ms_fwd"] = ms_fwd
    res["ms_fwd_bwd"] = ms_fb
    res["tflops_fwd"] = charged_flops(w, "fwd") / ms_fwd / 1e9
    res["tflops_fwd_bwd"] = charged_flops(w, "fwdbwd") / ms_fb / 1e9
    res["pct_peak_fwd"] = 100.0 * res["tflops_fwd"] / PEAK_TFLOPS
    res["pct_peak_fwd_bwd"] = 100.0 * res["tflops_fwd_bwd"] / PEAK_TFLOPS
    print(f"[bench] {name}: fwd {ms_fwd:.3f} ms ({res['tflops_fwd']:.1f} TF), fwd+bwd {ms_fb:.3f} ms "
          f"({res['tflops_fwd_bwd']:.1f} TF)", file=sys.stderr, flush=True)
    if kernels:
        o, lse = _forward(q, k, v, w["causal"], w["window"], scale, store_lse=True)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        delta = torch.empty(lse.shape, dtype=torch.float32, device=device)
        bufs = (dq, dk, dv, delta)
        per = {
            "fwd": time_loop(lambda: _forward(q, k, v, w["causal"], w["window"], scale, store_lse=True), steps, 1),
            "dq": time_loop(lambda: _backward(q, k, v, o, lse, do, w["causal"], w["window"], scale,
                                              stages=_lib.GFA_BWD_DQ, out=bufs), steps, 1),
            "dkv": time_loop(lambda: _backward(q, k, v, o, lse, do, w["causal"], w["window"], scale,
                                               stages=_lib.GFA_BWD_DKV, out=bufs), steps, 1),
        }
        kf = kernel_flops(w)
        res["kernels"] = {kname: {"ms": ms, "tflops": kf[kname] / ms / 1e9,
                                  "pct_peak": 100.0 * kf[kname] / ms / 1e9 / PEAK_TFLOPS}
                          for kname, ms in per.items()}
        print(f"[bench] {name}: kernels " + ", ".join(f"{k_} {v_['ms']:.3f} ms {v_['tflops']:.1f} TF"
                                                     for k_, v_ in res["kernels"].items()), file=sys.stderr, flush=True)
    del q, k, v, do, qg, kg, vg
    torch.cuda.empty_cache()
    return res


def cpu_baseline(budget_s=12.0):
    """Reference CPU path (SDPA math, fp32) on config 1: B1 N1024 Hq32 Hkv4 D512 causal."""
    from oracle.cpu_baseline import time_forward

    w = dict(B=1, Hq=32, Hkv=4, N=1024, D=512, causal=True, window=0)
    first = time_forward(1, 32, 4, 1024, 512, causal=True, warmup=1, reps=1)
    reps = max(3, min(50, int(budget_s * 1e3 / max(first["ms"], 1e-3))))
    r = time_forward(1, 32, 4, 1024, 512, causal=True, warmup=0, reps=reps)
    tflops = charged_flops(w, "fwd") / r["ms"] / 1e9
    return {"value": tflops, "unit": "TFLOPS", "cores": r["threads"], "kind": "port",
            "ms": r["ms"], "cpu_count": r["cpu_count"], "cpu_model": r["cpu_model"],
            "sample": f"config 1 forward (B1 N1024 Hq32 Hkv4 D512 causal fp32, torch SDPA math via "
                      f"oracle/cpu_baseline.py restating attention_gqa_ref), median of {reps} reps"}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--all", action="store_true", help="also time BASELINE configs 2 and 4")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-kernels", action="store_true", help="skip per-kernel timing")
    ap.add_argument("--workloads", default="d512_causal_gqa8_n16k,d256_swa1024_gqa2_n16k",
                    help="comma list of workloads to time (the first one must be the headline)")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="also run a plain device copy of this many MiB (rocprof FETCH/WRITE_SIZE calibration)")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py: this engine is a single-GPU build; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is design-only, see DESIGN.md)", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    device = torch.device("cuda:0")
    head = "d512_causal_gqa8_n16k"
    names = [n for n in args.workloads.split(",") if n]
    for n in names:
        if n not in WORKLOADS:
            print(f"bench.py: unknown workload {n}; choose from {sorted(WORKLOADS)}", file=sys.stderr)
            return 2
    results = {}
    for n in names:
        steps = args.steps if n != "d256_swa1024_gqa2_n16k" else max(args.steps, 10)
        results[n] = bench_workload(n, WORKLOADS[n], steps, args.warmup, device, kernels=not args.no_kernels)
    if args.copy_calib_mib:
        nbytes = args.copy_calib_mib << 20
        src = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=device).normal_()
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"[bench] copy calibration: 3 x {args.copy_calib_mib} MiB device copies", file=sys.stderr, flush=True)
        del src, dst
    if head not in results:
        print(json.dumps({"metric": METRIC, "workloads": results}), flush=True)
        return 0
    if args.all:
        for name in ("c2_d512_causal_gqa8_n8k", "c4_d512_causal_gqa8_n32k"):
            results[name] = bench_workload(name, WORKLOADS[name], args.steps, args.warmup, device, kernels=False)

    h = results[head]
    roofline = None
    if "kernels" in h:
        dom = max(h["kernels"], key=lambda kname: h["kernels"][kname]["ms"])
        kd = h["kernels"][dom]
        roofline = {"bound": "mfma", "kernel": dom, "achieved": round(kd["tflops"], 2), "peak": PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(kd["tflops"] / PEAK_TFLOPS, 4), "traffic": None,
                    "ms_per_launch": round(kd["ms"], 4),
                    "flops_per_launch": kernel_flops(WORKLOADS[head])[dom]}
    cpu = None
    if not args.no_cpu:
        print("[bench] cpu baseline ...", file=sys.stderr, flush=True)
        cpu = cpu_baseline()
    w = WORKLOADS[head]
    line = {
        "metric": METRIC,
        "value": round(h["tflops_fwd_bwd"], 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["ms_fwd_bwd"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(h["tflops_fwd_bwd"] / H100_FWDBWD_TFLOPS, 3),
        "baseline_note": "vs reference H100 fp16 fwd+bwd 117.1 TFLOPS at this shape (BASELINE.md)",
        "dtype": "bf16",
        "data": "synthetic N(0,1), seed 0",
        "config": {"workload": head + "_fwd_bwd", "B": w["B"], "Hq": w["Hq"], "Hkv": w["Hkv"], "N": w["N"],
                   "D": w["D"], "causal": w["causal"], "window": w["window"]},
        "fwd_tflops": round(h["tflops_fwd"], 2),
        "pct_peak_fwd": round(h["pct_peak_fwd"], 2),
        "pct_peak_fwd_bwd": round(h["pct_peak_fwd_bwd"], 2),
        "workloads": {k_: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in r.items()}
                      for k_, r in results.items()},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
