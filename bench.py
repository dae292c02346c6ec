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
import csv
import glob
import os
import shutil
import signal
import subprocess
import sys
import tempfile
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
    # the headline and config-3 shapes in fp16, the dtype of the reference's published figures
    "d512_causal_gqa8_n16k_fp16": dict(B=1, Hq=32, Hkv=4, N=16384, D=512, causal=True, window=0, dtype="fp16",
                                       amp=1.0),
    "d256_swa1024_gqa2_n16k_fp16": dict(B=1, Hq=16, Hkv=8, N=16384, D=256, causal=True, window=1024, dtype="fp16",
                                        amp=1.0),
    # the rest of the reference's documented head-dim range (64-512): not Gemma-4 layers
    "d128_causal_gqa4_n16k": dict(B=1, Hq=32, Hkv=8, N=16384, D=128, causal=True, window=0, dtype="bf16", amp=1.0),
    "d64_causal_mha_n16k": dict(B=1, Hq=32, Hkv=32, N=16384, D=64, causal=True, window=0, dtype="bf16", amp=1.0),
}


# The reference's published H100 fp16 times of the same shapes (ms): D=512 causal 32:4 N=16384
# (/root/reference/benchmarks/attn_only_all_n.json:200-210) and D=256 W=1024 16:8 N=16384
# (/root/reference/benchmarks/moe_attn_sweep.json:47-57). Reported beside the fp16 rows only.
REFERENCE_H100_FP16_MS = {
    "d512_causal_gqa8_n16k_fp16": {"ms_fwd": 47.58, "ms_fwd_bwd": 262.98,
                                   "source": "benchmarks/attn_only_all_n.json:200-210"},
    "d256_swa1024_gqa2_n16k_fp16": {"ms_fwd": 0.854, "ms_fwd_bwd": 4.003,
                                    "source": "benchmarks/moe_attn_sweep.json:47-57"},
}


def charged_flops(w, passes):
    B, Hq, N, D, W = w["B"], w["Hq"], w["N"], w["D"], w["window"]
    if w["causal"] and 0 < W < N:
        P = W * (W + 1) / 2 + W * (N - W)
        return (4 if passes == "fwd" else 14) * B * Hq * D * P
    if w["causal"]:
        return (2 if passes == "fwd" else 7) * B * Hq * N * N * D
    return (4 if passes == "fwd" else 14) * B * Hq * N * N * D


def kernel_flops(w, materialised=False):
    """Algorithmic flops per launch of each kernel: 2*D per pair-product per attended
    (query, key) pair; forward 2 products, dKV 4 (S, dP, dV, dK), dQ 3 (S, dP, dQ) in the
    recomputing backward and 1 (dS K) in the materialised one, which reads dS from its store."""
    unit = charged_flops(w, "fwd") / 2.0  # = 2*D*pairs (causal convention)
    return {"fwd": 2 * unit, "dq": (1 if materialised else 3) * unit, "dkv": 4 * unit}


def kernel_bytes(w, ds_bytes=0):
    """Algorithmic HBM bytes per launch of each kernel: every tensor the kernel must touch,
    read or written once (16-bit Q/K/V/O/dO/dQ/dK/dV, fp32 LSE and delta). ``ds_bytes`` > 0:
    the materialised backward, whose "dkv" stage is the delta kernel (O, dO in; delta out) and
    dK/dV writing the dS store, and whose "dq" stage reads the store and K and writes dQ."""
    B, Hq, Hkv, N, D = w["B"], w["Hq"], w["Hkv"], w["N"], w["D"]
    qsz, kvsz, rows = 2 * B * Hq * N * D, 2 * B * Hkv * N * D, 4 * B * Hq * N
    if ds_bytes:
        return {"fwd": 2 * qsz + 2 * kvsz + rows,
                "dq": kvsz + ds_bytes + qsz,
                "dkv": (2 * qsz + rows) + (2 * qsz + 4 * kvsz + 2 * rows + ds_bytes)}
    return {"fwd": 2 * qsz + 2 * kvsz + rows,             # Q, K, V in; O, LSE out
            "dq": 4 * qsz + 2 * kvsz + 2 * rows,          # Q, O, dO, K, V, LSE in; dQ, delta out
            "dkv": 2 * qsz + 4 * kvsz + 2 * rows}         # Q, dO, K, V, LSE, delta in; dK, dV out


def make_inputs(w, device, layout="bhnd"):
    """q, k, v, dO of the workload. ``layout='bnhd'`` gives (B, H, N, D) views of
    (B, N, H, D) storage: the strides transformers hands to an attention function."""
    import torch

    dt = {"bf16": torch.bfloat16, "fp16": torch.float16}[w["dtype"]]
    g = torch.Generator().manual_seed(0)
    shapes = [(w["B"], w["Hq"], w["N"], w["D"]), (w["B"], w["Hkv"], w["N"], w["D"]),
              (w["B"], w["Hkv"], w["N"], w["D"]), (w["B"], w["Hq"], w["N"], w["D"])]
    ts = [(torch.randn(*s, generator=g) * w["amp"]).to(device=device, dtype=dt) for s in shapes]
    if layout == "bnhd":
        ts = [t.transpose(1, 2).contiguous().transpose(1, 2) for t in ts]
    return ts


def time_loop(fn, iters, warmup, min_warm_ms=0.0, min_time_ms=0.0):
    """Average ms per call of ``fn`` over ``iters`` timed calls after ``warmup`` untimed ones,
    HIP events on the current stream. With ``min_warm_ms`` / ``min_time_ms`` the warmup and
    the timed window are extended to at least that much GPU time (sub-millisecond layers:
    MI355X's clock settles over tens of milliseconds of work, and a few calls would time the
    ramp rather than the steady state)."""
    import torch

    for _ in range(warmup):
        fn()
    if min_warm_ms or min_time_ms:
        torch.cuda.synchronize()
        s0, e0 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        for _ in range(3):
            fn()
        e0.record()
        torch.cuda.synchronize()
        per = max(s0.elapsed_time(e0) / 3, 1e-3)
        for _ in range(int(min_warm_ms / per)):
            fn()
        iters = max(iters, int(math.ceil(min_time_ms / per)))
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters


def bench_workload(name, w, steps, warmup, device, kernels=True, layout="bhnd", exact=False):
    """Time one workload. ``exact``: the fwd and fwd+bwd loops run exactly ``warmup`` untimed
    and ``steps`` timed steps (the headline ``value``); otherwise, and for the per-kernel
    loops, warmup and timed window are extended to at least 100 and 200 ms of GPU time."""
    import torch

    import gemma_triton_flash_attn_amd as gfa
    from gemma_triton_flash_attn_amd import _lib
    from gemma_triton_flash_attn_amd.attention import _backward, _forward, backward_workspace

    print(f"[bench] {name}: {w}", file=sys.stderr, flush=True)
    q, k, v, do = make_inputs(w, device, layout)
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))  # clone keeps the strides
    scale = w["D"] ** -0.5

    def fwd():
        return gfa.flash_attn_gqa_train(qg, kg, vg, causal=w["causal"], slide_size=w["window"])

    def fwd_bwd():
        qg.grad = kg.grad = vg.grad = None
        o = fwd()
        o.backward(do)

    res = {}
    dt = {"bf16": torch.bfloat16, "fp16": torch.float16}[w["dtype"]]
    ws_bytes, materialised = backward_workspace(w["B"], w["Hq"], w["Hkv"], w["N"], w["D"], w["causal"], w["window"], dt)
    res["bwd_form"] = "materialised" if materialised else "recomputing"
    res["bwd_workspace_bytes"] = ws_bytes
    if materialised:  # the workspace beyond the (256-byte aligned) Q-split partials is the dS store
        base = _lib.bwd_workspace_size(w["B"], w["Hq"], w["Hkv"], w["N"], w["D"], w["causal"], w["window"])
        res["ds_store_bytes"] = ws_bytes - ((base + 255) // 256 * 256)
    ext = {} if exact else {"min_warm_ms": 100.0, "min_time_ms": 200.0}
    kext = {"min_warm_ms": 100.0, "min_time_ms": 200.0}
    with torch.no_grad():
        ms_fwd = time_loop(lambda: fwd(), steps, warmup, **ext)
    ms_fb = time_loop(fwd_bwd, steps, warmup, **ext)
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
        # The workspace persists over the stage loops: in the materialised form the GFA_BWD_DQ
        # stage reads the dS store the full backward below (and each GFA_BWD_DKV stage) leaves.
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes else None
        bufs = (dq, dk, dv, delta) + ((ws,) if ws is not None else ())
        _backward(q, k, v, o, lse, do, w["causal"], w["window"], scale, out=bufs)
        per = {
            "fwd": time_loop(lambda: _forward(q, k, v, w["causal"], w["window"], scale, store_lse=True), steps, 1,
                             **kext),
            "dq": time_loop(lambda: _backward(q, k, v, o, lse, do, w["causal"], w["window"], scale,
                                              stages=_lib.GFA_BWD_DQ, out=bufs), steps, 1, **kext),
            "dkv": time_loop(lambda: _backward(q, k, v, o, lse, do, w["causal"], w["window"], scale,
                                               stages=_lib.GFA_BWD_DKV, out=bufs), steps, 1, **kext),
        }
        kf = kernel_flops(w, materialised)
        res["kernels"] = {kname: {"ms": ms, "tflops": kf[kname] / ms / 1e9,
                                  "pct_peak": 100.0 * kf[kname] / ms / 1e9 / PEAK_TFLOPS}
                          for kname, ms in per.items()}
        print(f"[bench] {name}: kernels " + ", ".join(f"{k_} {v_['ms']:.3f} ms {v_['tflops']:.1f} TF"
                                                     for k_, v_ in res["kernels"].items()), file=sys.stderr, flush=True)
    ref = REFERENCE_H100_FP16_MS.get(name)
    if ref is not None:
        res["reference_h100_fp16"] = dict(ref, speedup_fwd=ref["ms_fwd"] / ms_fwd, speedup_fwd_bwd=ref["ms_fwd_bwd"] / ms_fb)
    del q, k, v, do, qg, kg, vg
    torch.cuda.empty_cache()
    return res


# Kernel-name tags per timed stage: the dQ stage is bwd_dq_kernel in the recomputing backward and
# bwd_dq_ds_kernel in the materialised one, whose dK/dV stage runs delta_kernel, then bwd_dkv_kernel
# (bwd_dkv_ds_kernel for the one-wave D=256 form); a stage's traffic is the sum over its kernels,
# as its time is.
KERNEL_TAGS = {"fwd": ("fwd_kernel",), "dq": ("bwd_dq_kernel", "bwd_dq_ds_kernel"),
               "dkv": ("bwd_dkv_kernel", "bwd_dkv_ds_kernel", "delta_kernel")}
PMC_COUNTERS = ("FETCH_SIZE", "WRITE_SIZE")  # KiB per dispatch, one counter per rocprofv3 pass


def pmc_child(name, calib_mib):
    """Body run under ``rocprofv3 --pmc``: one launch of each kernel at ``name``'s shape,
    then one plain elementwise copy (torch.neg, fp32) of ``calib_mib`` MiB whose counter
    reading calibrates the counter (known bytes: calib_mib MiB read + calib_mib MiB written)."""
    import torch

    from gemma_triton_flash_attn_amd import _lib
    from gemma_triton_flash_attn_amd.attention import _backward, _forward

    w = WORKLOADS[name]
    dev = torch.device("cuda:0")
    dt = {"bf16": torch.bfloat16, "fp16": torch.float16}[w["dtype"]]
    gen = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(w["B"], w["Hq"], w["N"], w["D"], device=dev, dtype=dt, generator=gen)
    k = torch.randn(w["B"], w["Hkv"], w["N"], w["D"], device=dev, dtype=dt, generator=gen)
    v = torch.randn(w["B"], w["Hkv"], w["N"], w["D"], device=dev, dtype=dt, generator=gen)
    do = torch.randn(w["B"], w["Hq"], w["N"], w["D"], device=dev, dtype=dt, generator=gen)
    scale = w["D"] ** -0.5
    o, lse = _forward(q, k, v, w["causal"], w["window"], scale, store_lse=True)
    bufs = (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
            torch.empty(lse.shape, dtype=torch.float32, device=dev))
    _backward(q, k, v, o, lse, do, w["causal"], w["window"], scale, out=bufs)  # every backward kernel once
    torch.cuda.synchronize()
    del q, k, v, do, o, lse, bufs
    src = torch.empty((calib_mib << 20) // 4, dtype=torch.float32, device=dev).normal_()
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(f"[pmc-child] {name}: fwd, dq, dkv and a {calib_mib} MiB copy done", file=sys.stderr, flush=True)
    return 0


def _read_pmc_csv(outdir, counter):
    """{kernel name: [per-dispatch value]} and the name of the last dispatch, from the
    rocprofv3 counter-collection CSV under ``outdir``."""
    files = glob.glob(os.path.join(outdir, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise RuntimeError(f"no counter_collection.csv under {outdir}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows += [r for r in csv.DictReader(fh) if r.get("Counter_Name") == counter]
    if not rows:
        raise RuntimeError(f"counter {counter} missing in {files}")
    rows.sort(key=lambda r: int(r.get("Dispatch_Id", 0)))
    vals = {}
    for r in rows:
        vals.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
    return vals, rows[-1]["Kernel_Name"]


def measure_traffic(name, calib_mib=1024, timeout_s=180, keep_dir=None):
    """HBM traffic per launch of each kernel, from two rocprofv3 --pmc passes (FETCH_SIZE,
    then WRITE_SIZE) over ``pmc_child``, each scaled by what the same counter reads for a
    copy of known size. Runs before this process touches the GPU; returns None (with a
    message) when rocprofv3 is missing or a pass fails."""
    exe = shutil.which("rocprofv3")
    if exe is None:
        print("[bench] traffic: rocprofv3 not found", file=sys.stderr, flush=True)
        return None
    copy_known_kib = calib_mib * 1024.0  # the copy reads this much and writes this much
    out = {"calib_mib": calib_mib, "kernels": {}}
    env = dict(os.environ, TMPDIR="/tmp")
    for counter in PMC_COUNTERS:
        d = keep_dir and os.path.join(keep_dir, counter.lower())
        d = d or tempfile.mkdtemp(prefix="gfa_pmc_", dir="/tmp")
        cmd = [exe, "--pmc", counter, "-d", d, "-o", "pmc", "--output-format", "csv", "--",
               sys.executable, os.path.abspath(__file__), "--pmc-child", name, "--copy-calib-mib", str(calib_mib)]
        print(f"[bench] traffic pass {counter}: {' '.join(cmd[:-6])} -- python bench.py --pmc-child {name}",
              file=sys.stderr, flush=True)
        proc = subprocess.Popen(cmd, cwd="/tmp", env=env, start_new_session=True,
                                stdout=subprocess.DEVNULL, stderr=subprocess.PIPE, text=True)
        try:
            _, err = proc.communicate(timeout=timeout_s)
        except subprocess.TimeoutExpired:
            os.killpg(proc.pid, signal.SIGKILL)
            proc.wait()
            print(f"[bench] traffic: {counter} pass timed out", file=sys.stderr, flush=True)
            return None
        try:
            vals, last = _read_pmc_csv(d, counter)
        except RuntimeError as e:
            print(f"[bench] traffic: {counter} pass rc={proc.returncode}: {e}\n{(err or '')[-1500:]}",
                  file=sys.stderr, flush=True)
            return None
        finally:
            if not keep_dir:
                shutil.rmtree(d, ignore_errors=True)
        copy_kib = vals[last][-1]
        factor = copy_known_kib / copy_kib if copy_kib > 0 else float("nan")
        out[f"{counter.lower()}_factor"] = factor
        out["copy_kernel"] = last
        for kname, tags in KERNEL_TAGS.items():
            hits = [v for kn, v in vals.items() if any(t in kn for t in tags) and "reduce" not in kn]
            if not hits:
                continue
            kib = sum(sum(h) / len(h) for h in hits)
            ent = out["kernels"].setdefault(kname, {})
            ent[f"{counter.lower()}_kib_raw"] = kib
            ent[f"{counter.lower()}_bytes"] = kib * 1024.0 * factor
    for ent in out["kernels"].values():
        if "fetch_size_bytes" in ent and "write_size_bytes" in ent:
            ent["traffic_bytes"] = ent["fetch_size_bytes"] + ent["write_size_bytes"]
    return out


# Config 5: a random-init model of the Gemma-4-E2B architecture (35 decoder layers: 28
# sliding-window layers with head dim 256, window 512, and 7 full-causal layers with head
# dim 512, the pattern four sliding then one full; GQA 8:1; per-layer input embeddings).
# Built locally from transformers' Gemma4TextConfig with random weights (no checkpoint).
def _e2e_config() -> dict:
    """Config 5's model configuration, committed beside this script."""
    with open(os.path.join(ROOT, "bench_e2e_config.json")) as f:
        return json.load(f)["gemma4_text_config"]


def bench_e2e(device, seq_len=16384, steps=3, warmup=1):
    """Config 5: forward latency and peak HBM of the E2B-architecture model at N=seq_len,
    every attention layer swapped to this engine by the one-call HF registration.

    Measured the reference's way (/root/reference/benchmarks/run_final_benchmark.py:122-135,
    tests/gemma4_integration/test_memory.py:44-70): a plain ``model(ids)`` forward under
    no_grad, which runs the lm_head over every position and materialises all N x vocab
    logits; peak HBM is the peak allocation of one such forward above what was allocated
    before it (weights and ids), after a 128-token warmup. A second, labelled figure times
    the same forward with ``logits_to_keep=1`` (last position's logits only, no cache)."""
    import gc

    import torch
    from transformers import Gemma4ForCausalLM, Gemma4TextConfig

    import gemma_triton_flash_attn_amd as gfa

    print(f"[bench] e2e: Gemma-4-E2B architecture, random init, N={seq_len}", file=sys.stderr, flush=True)
    gfa.register_triton_attention()
    cfg = Gemma4TextConfig(**_e2e_config())
    torch.manual_seed(0)
    with torch.device(device):
        model = Gemma4ForCausalLM(cfg)
    model = model.to(torch.bfloat16).eval()
    for m in model.modules():
        c = getattr(m, "config", None)
        if c is not None and hasattr(c, "_attn_implementation"):
            c._attn_implementation = "triton_gqa"
    n_params = sum(p.numel() for p in model.parameters())
    gen = torch.Generator().manual_seed(0)
    ids = torch.randint(0, cfg.vocab_size, (1, seq_len), generator=gen).to(device)
    warm_ids = torch.randint(0, cfg.vocab_size, (1, 128), generator=gen).to(device)

    def fwd_full():
        with torch.no_grad():
            return model(ids)

    def fwd_last():
        with torch.no_grad():
            return model(input_ids=ids, logits_to_keep=1, use_cache=False)

    with torch.no_grad():
        model(warm_ids)
    torch.cuda.synchronize()
    gc.collect()
    torch.cuda.empty_cache()
    weights = sum(p.numel() * p.element_size() for p in model.parameters())
    base = torch.cuda.memory_allocated(device)
    torch.cuda.reset_peak_memory_stats(device)
    out = fwd_full()
    torch.cuda.synchronize()
    peak_above = torch.cuda.max_memory_allocated(device) - base
    logits_shape = list(out.logits.shape)
    ok = bool(torch.isfinite(out.logits[0, -1]).all()) and bool(torch.isfinite(out.logits[0, :: 4096]).all())
    del out
    gc.collect()
    torch.cuda.empty_cache()
    ms_full = time_loop(fwd_full, steps, warmup)
    ms_last = time_loop(fwd_last, steps, warmup)
    res = {"workload": "gemma4_e2b_arch_random_init_fwd", "seq_len": seq_len, "batch": 1, "dtype": "bf16",
           "ms": round(ms_full, 2), "tokens_per_s": round(seq_len / ms_full * 1e3, 1),
           "method": "model(ids) under no_grad: all N x vocab logits, default cache "
                     "(reference run_final_benchmark.py:122-135)",
           "peak_above_weights_mib": round(peak_above / 2 ** 20, 1),
           "peak_method": "max_memory_allocated - memory_allocated before one model(ids), after a 128-token "
                          "warmup (reference test_memory.py:44-70)",
           "weights_gib": round(weights / 2 ** 30, 3), "logits_shape": logits_shape,
           "ms_logits_to_keep_1": round(ms_last, 2),
           "logits_to_keep_1_note": "same forward with logits_to_keep=1, use_cache=False: lm_head on the last "
                                    "position only; not the reference's measurement",
           "params": n_params, "finite": ok, "layers": cfg.num_hidden_layers,
           "attention": "triton_gqa (this engine via register_triton_attention)",
           "config_file": "bench_e2e_config.json",
           "config": {k: v for k, v in _e2e_config().items() if k != "layer_types"},
           "layer_pattern": "4 x sliding_attention (D=256, W=512) then 1 x full_attention (D=512), x7"}
    print(f"[bench] e2e: model(ids) {res['ms']} ms ({res['tokens_per_s']} tok/s), peak above weights "
          f"{res['peak_above_weights_mib']} MiB; logits_to_keep=1 {res['ms_logits_to_keep_1']} ms",
          file=sys.stderr, flush=True)
    del model
    gc.collect()
    torch.cuda.empty_cache()
    return res


def cpu_baseline(budget_s=12.0, shapes=True):
    """Reference CPU path (SDPA math, fp32) on config 1: B1 N1024 Hq32 Hkv4 D512 causal.

    With ``shapes``, the GPU workloads' shapes are also timed forward-only where the math
    path fits the host (one rep: it materialises the full N x N score matrix per head);
    the others are recorded as skipped with the reason."""
    from oracle.cpu_baseline import time_forward

    w = dict(B=1, Hq=32, Hkv=4, N=1024, D=512, causal=True, window=0)
    first = time_forward(1, 32, 4, 1024, 512, causal=True, warmup=1, reps=1)
    reps = max(3, min(50, int(budget_s * 1e3 / max(first["ms"], 1e-3))))
    r = time_forward(1, 32, 4, 1024, 512, causal=True, warmup=0, reps=reps)
    tflops = charged_flops(w, "fwd") / r["ms"] / 1e9
    out = {"value": tflops, "unit": "TFLOPS", "cores": r["threads"], "kind": "port",
           "ms": r["ms"], "cpu_count": r["cpu_count"], "cpu_model": r["cpu_model"],
           "sample": f"config 1 forward (B1 N1024 Hq32 Hkv4 D512 causal fp32, torch SDPA math via "
                     f"oracle/cpu_baseline.py restating attention_gqa_ref), median of {reps} reps"}
    if not shapes:
        return out
    per = {}
    # score-matrix bytes of the math path (fp32, B * Hq * N^2), about 3 live copies at peak
    for name in ("c2_d512_causal_gqa8_n8k", "d512_causal_gqa8_n16k", "d256_swa1024_gqa2_n16k",
                 "c4_d512_causal_gqa8_n32k"):
        wl = WORKLOADS[name]
        score_gib = 4.0 * wl["B"] * wl["Hq"] * wl["N"] ** 2 / 2 ** 30
        dense_fwd = 4.0 * wl["B"] * wl["Hq"] * wl["N"] ** 2 * wl["D"]  # the math path computes every pair
        est_s = dense_fwd / (tflops * 1e12) if tflops > 0 else float("inf")
        if 3 * score_gib > 48 or est_s > 20:
            per[name] = {"skipped": True,
                         "reason": f"SDPA math materialises {score_gib:.0f} GiB of fp32 scores per forward "
                                   f"(~{3 * score_gib:.0f} GiB at peak) and would take ~{est_s:.0f} s at the "
                                   f"config-1 rate; beyond this leg's bounded sample"}
            continue
        print(f"[bench] cpu baseline {name} (forward, 1 rep) ...", file=sys.stderr, flush=True)
        rr = time_forward(wl["B"], wl["Hq"], wl["Hkv"], wl["N"], wl["D"], causal=wl["causal"],
                          window=wl["window"], warmup=0, reps=1)
        per[name] = {"ms_fwd": rr["ms"], "tflops_fwd": charged_flops(wl, "fwd") / rr["ms"] / 1e9,
                     "reps": 1, "threads": rr["threads"]}
    out["workloads_fwd"] = per
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--all", action="store_true",
                    help="also time the D=128 / D=64 workloads")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-kernels", action="store_true", help="skip per-kernel timing")
    ap.add_argument("--workloads",
                    default="d512_causal_gqa8_n16k,d256_swa1024_gqa2_n16k,c2_d512_causal_gqa8_n8k,"
                            "c4_d512_causal_gqa8_n32k,d512_causal_gqa8_n16k_fp16,d256_swa1024_gqa2_n16k_fp16",
                    help="comma list of workloads to time (the first one must be the headline)")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 --pmc passes that measure HBM traffic per kernel")
    ap.add_argument("--copy-calib-mib", type=int, default=1024,
                    help="size of the plain copy that calibrates FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--no-e2e", action="store_true", help="skip the config-5 model forward (Gemma-4-E2B arch)")
    ap.add_argument("--no-strided", action="store_true",
                    help="skip the headline run on transformers-style (B, N, H, D)-strided inputs")
    ap.add_argument("--pmc-dir", default=None, help="keep the rocprofv3 counter CSVs in this directory")
    ap.add_argument("--pmc-child", default=None, metavar="WORKLOAD",
                    help="internal: the program profiled by the traffic passes")
    args = ap.parse_args(argv)
    if args.pmc_child:
        return pmc_child(args.pmc_child, args.copy_calib_mib)
    if args.gpus != 1:
        print(f"bench.py: this engine is a single-GPU build; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is design only in this build)", file=sys.stderr)
        return 2

    head = "d512_causal_gqa8_n16k"
    # The counter passes are child processes started before this process touches the GPU.
    traffic = None if args.no_traffic else measure_traffic(head, args.copy_calib_mib, keep_dir=args.pmc_dir)

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    device = torch.device("cuda:0")
    names = [n for n in args.workloads.split(",") if n]
    for n in names:
        if n not in WORKLOADS:
            print(f"bench.py: unknown workload {n}; choose from {sorted(WORKLOADS)}", file=sys.stderr)
            return 2
    results = {}
    for n in names:
        results[n] = bench_workload(n, WORKLOADS[n], args.steps, args.warmup, device, kernels=not args.no_kernels,
                                    exact=(n == head))
    if head not in results:
        print(json.dumps({"metric": METRIC, "workloads": results}), flush=True)
        return 0
    if not args.no_strided:
        # Same step on (B, H, N, D) views of (B, N, H, D) storage, read in place (no copy).
        results[head + "_hf_strided"] = bench_workload(head + " (B,N,H,D) strides", WORKLOADS[head], args.steps,
                                                       args.warmup, device, kernels=False, layout="bnhd", exact=True)
    if args.all:
        for name in ("d128_causal_gqa4_n16k", "d64_causal_mha_n16k"):
            if name not in results:
                results[name] = bench_workload(name, WORKLOADS[name], args.steps, args.warmup, device,
                                               kernels=not args.no_kernels)

    e2e = None
    if not args.no_e2e:
        try:
            e2e = bench_e2e(device)
        except Exception as exc:  # reported, never fatal for the headline line
            print(f"[bench] e2e failed: {type(exc).__name__}: {exc}", file=sys.stderr, flush=True)
            e2e = {"error": f"{type(exc).__name__}: {exc}"}
    h = results[head]
    roofline = None
    if "kernels" in h:
        dom = max(h["kernels"], key=lambda kname: h["kernels"][kname]["ms"])
        kd = h["kernels"][dom]
        kb = kernel_bytes(WORKLOADS[head], h.get("ds_store_bytes", 0))
        tk = (traffic or {}).get("kernels", {})
        for kname, ent in h["kernels"].items():
            ent["algorithmic_bytes"] = kb[kname]
            if "traffic_bytes" in tk.get(kname, {}):
                ent["traffic_bytes"] = round(tk[kname]["traffic_bytes"])
                ent["traffic_over_algorithmic"] = round(tk[kname]["traffic_bytes"] / kb[kname], 3)
        roofline = {"bound": "mfma", "kernel": dom, "achieved": round(kd["tflops"], 2), "peak": PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(kd["tflops"] / PEAK_TFLOPS, 4),
                    "traffic": kd.get("traffic_bytes"),
                    "algorithmic_bytes": kb[dom],
                    "ms_per_launch": round(kd["ms"], 4),
                    "flops_per_launch": kernel_flops(WORKLOADS[head], h.get("bwd_form") == "materialised")[dom]}
        if traffic:
            roofline["traffic_calibration"] = {k_: round(traffic[k_], 4) for k_ in ("fetch_size_factor",
                                                                                     "write_size_factor")
                                               if k_ in traffic}
            roofline["traffic_calibration"]["copy_mib"] = traffic["calib_mib"]
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
        "baseline_note": "vs the reference's published H100 fp16 fwd+bwd 117.1 TFLOPS at this shape",
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
        "e2e": e2e,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
