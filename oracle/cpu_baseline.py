"""The reference's CPU path, timed as a reported baseline (never a pass/fail gate).

TEST / BENCH INFRASTRUCTURE ONLY (imported by bench.py's cpu_baseline leg and tests).

Restates /root/reference/flash_attn/attention.py:611-619 (``attention_gqa_ref``): repeat
each KV head over its query group, then torch's scaled_dot_product_attention with
is_causal, scale 1/sqrt(D). The math backend is forced, as "SDPA math attention" in the
benchmark definition; for a sliding window an explicit (N, N) mask is built as in
attention.py:622-642. Runs in float32 on the host CPU.
"""
from __future__ import annotations

import os
import platform
import time

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel


def sdpa_math_gqa(q, k, v, causal=True, window=0):
    hq, hkv = q.shape[1], k.shape[1]
    if hq != hkv:
        r = hq // hkv
        k = k.repeat_interleave(r, dim=1)
        v = v.repeat_interleave(r, dim=1)
    with sdpa_kernel(SDPBackend.MATH):
        if causal and window and 0 < window < q.shape[2]:
            n = q.shape[2]
            idx = torch.arange(n)
            attend = (idx[None, :] <= idx[:, None]) & ((idx[:, None] - idx[None, :]) < window)
            mask = torch.where(attend, 0.0, float("-inf")).to(q.dtype)[None, None]
            return F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
        return F.scaled_dot_product_attention(q, k, v, is_causal=causal)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def time_forward(batch=1, heads_q=32, heads_kv=4, seq_len=1024, head_dim=512, causal=True, window=0, seed=0,
                 warmup=1, reps=3, threads=None):
    """Median wall time (ms) of the fp32 CPU SDPA-math forward on seeded N(0,1) inputs."""
    if threads:
        torch.set_num_threads(int(threads))
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, heads_q, seq_len, head_dim, generator=g)
    k = torch.randn(batch, heads_kv, seq_len, head_dim, generator=g)
    v = torch.randn(batch, heads_kv, seq_len, head_dim, generator=g)
    for _ in range(warmup):
        sdpa_math_gqa(q, k, v, causal, window)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        sdpa_math_gqa(q, k, v, causal, window)
        times.append((time.perf_counter() - t0) * 1e3)
    times.sort()
    return {
        "ms": times[len(times) // 2],
        "threads": torch.get_num_threads(),
        "cpu_count": os.cpu_count(),
        "cpu_model": cpu_model(),
    }
