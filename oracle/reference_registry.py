"""CPU restatement of the reference's HEAD_DIM-keyed tile selection (hot-path row R5).

TEST INFRASTRUCTURE ONLY. Only tests/ may import this module, as the checker of what the
engine's registry replaces. The engine's own registry (gemma-triton-flash-attn_amd/
registry.py and kRegistry in csrc/gfa_api.hip) picks gfx950 tiles; the reference's Triton
tiles below do not apply to those kernels.

Restated from /root/reference/flash_attn/attention.py:
  * training forward, 1444-1451: (BLOCK_Q, BLOCK_KV) = (64, 32) if D >= 512 else
    (128, 64); num_warps 8 if D >= 256 else 4; num_stages 2; both blocks clamped to
    next_pow2(N); grid (cdiv(N, BLOCK_Q), B * Hq). The inference forward (561-579) uses the
    same defaults;
  * dQ, 1498-1504: (BLOCK_Q, BLOCK_KV, warps) = (32, 64, 8) if D >= 512 else (64, 64, 4);
    clamped to next_pow2(N);
  * dK/dV, 1536-1564: D >= 512 -> (BKV, BQ, warps, stages) = (16, 64, 4, 2); otherwise
    (64, 128, 8, 1) when cdiv(N, 64) * B * Hkv >= 128 or <= 16, else (32, 64, 4, 2);
    clamped to next_pow2(N);
  * Q_SPLITS, 1576-1587: raw = cdiv(N, BKV) * B * Hkv, target 128 if BKV == 64 else 256,
    QS = the smallest of {1, 2, 4, 8} with raw * QS >= target (8 otherwise).

Pinned by tests/test_registry_cpu.py against the reference's own known-answer table for
this selection (context/baseline.md:1582-1592).
"""
from __future__ import annotations


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def _next_pow2(n: int) -> int:
    p = 1
    while p < n:
        p *= 2
    return p


def forward_tiles(N: int, D: int) -> dict:
    bq, bkv = (64, 32) if D >= 512 else (128, 64)
    return {"BLOCK_Q": min(bq, _next_pow2(N)), "BLOCK_KV": min(bkv, _next_pow2(N)),
            "num_warps": 8 if D >= 256 else 4, "num_stages": 2}


def dq_tiles(N: int, D: int) -> dict:
    bq, bkv, w = (32, 64, 8) if D >= 512 else (64, 64, 4)
    return {"BLOCK_Q": min(bq, _next_pow2(N)), "BLOCK_KV": min(bkv, _next_pow2(N)), "num_warps": w}


def dkv_tiles(B: int, Hkv: int, N: int, D: int) -> dict:
    if D >= 512:
        bkv, bq, w, st = 16, 64, 4, 2
    else:
        g64 = _cdiv(N, 64) * B * Hkv
        bkv, bq, w, st = (64, 128, 8, 1) if (g64 >= 128 or g64 <= 16) else (32, 64, 4, 2)
    bkv, bq = min(bkv, _next_pow2(N)), min(bq, _next_pow2(N))
    raw = _cdiv(N, bkv) * B * Hkv
    target = 128 if bkv == 64 else 256
    qs = next((s for s in (1, 2, 4) if raw * s >= target), 8)
    return {"BLOCK_KV": bkv, "BLOCK_Q": bq, "num_warps": w, "num_stages": st, "Q_SPLITS": qs,
            "raw_grid": raw, "grid": raw * qs}
