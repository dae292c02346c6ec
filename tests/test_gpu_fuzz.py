"""Seeded random sweep of the whole path against the oracle (float64 numpy).

Each case draws (B, Hq, Hkv, N, D, causal, window, dtype, layout, scale) from a fixed seed, so
the sweep is the same on every run: head dims 64-512, GQA groups 1-16, ragged N up to 300,
windows from 1 past N, non-causal cases, HF-style strided inputs and a non-default softmax
scale. A second sweep runs longer sequences (N 300-4096) against the oracle's query-chunked
torch fp32 path on the GPU. The bar is the one in tests/test_gpu_parity.py: O max-abs <= 1e-2 (fp16) / 2e-2
(bf16), dQ/dK/dV relative Frobenius error <= 5e-2 with an absolute floor for near-zero
gradients.
"""
from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from conftest import make_inputs
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

O_TOL = {torch.float16: 1e-2, torch.bfloat16: 2e-2}
GRAD_TOL = 5e-2
GRAD_ABS_RMS = 1e-3


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _rel(a, b):
    floor = GRAD_ABS_RMS * np.sqrt(b.size) / GRAD_TOL
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), floor))


def _cases(n=120, seed=2024):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        D = rng.choice([64, 128, 256, 512])
        Hkv = rng.choice([1, 2, 3, 4])
        R = rng.choice([1, 2, 3, 4, 8, 16])
        if Hkv * R > 32:
            R = 32 // Hkv
        B = rng.choice([1, 1, 2])
        N = rng.randint(1, 300 if D <= 256 else 200)
        causal = rng.random() < 0.75
        window = rng.choice([0, 0, 1, rng.randint(2, 64), rng.randint(1, N + 40)]) if causal else 0
        dtype = rng.choice([torch.float16, torch.bfloat16])
        layout = rng.choice(["bhnd", "bhnd", "bnhd"])
        scale = rng.choice([None, None, 0.5 * D ** -0.5, 1.5 * D ** -0.5])
        out.append((i, B, Hkv * R, Hkv, N, D, causal, window, dtype, layout, scale))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"c{c[0]}")
def test_random_case_vs_oracle(case, device):
    import gemma_triton_flash_attn_amd as gfa

    i, B, Hq, Hkv, N, D, causal, window, dtype, layout, scale = case
    print(f"case {i}: B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal} window={window} {dtype} "
          f"{layout} scale={scale}", flush=True)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, dtype, device, seed=1000 + i, layout=layout)
    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = gfa.flash_attn_gqa_train(qq, kk, vv, causal=causal, slide_size=window, scale=scale)
    o.backward(do)
    torch.cuda.synchronize()
    o_ref, _ = orc.forward(_np(q), _np(k), _np(v), causal, window, scale)
    dq_ref, dk_ref, dv_ref, _ = orc.backward(_np(q), _np(k), _np(v), _np(do), causal, window, scale)
    err_o = float(np.abs(_np(o) - o_ref).max())
    errs = [_rel(_np(g), r) for g, r in ((qq.grad, dq_ref), (kk.grad, dk_ref), (vv.grad, dv_ref))]
    print(f"  O max-abs {err_o:.3e}  dQ/dK/dV rel {errs[0]:.3e} {errs[1]:.3e} {errs[2]:.3e}", flush=True)
    assert err_o <= O_TOL[dtype]
    assert max(errs) <= GRAD_TOL


def _mid_cases(n=24, seed=77):
    """Longer sequences (300-4096): several key/query tiles per window, query splits chosen by
    the registry for small and mid-size grids, multi-workgroup causal imbalance."""
    rng = random.Random(seed)
    out = []
    for i in range(n):
        D = rng.choice([64, 128, 256, 512])
        Hkv = rng.choice([1, 2, 4])
        R = rng.choice([1, 2, 4, 8])
        B = rng.choice([1, 1, 2])
        N = rng.randint(300, 4096 if D <= 256 else 2048)
        causal = rng.random() < 0.8
        window = rng.choice([0, rng.randint(2, 300), rng.randint(300, N + 100)]) if causal else 0
        dtype = rng.choice([torch.float16, torch.bfloat16])
        layout = rng.choice(["bhnd", "bnhd"])
        out.append((i, B, Hkv * R, Hkv, N, D, causal, window, dtype, layout))
    return out


@pytest.mark.parametrize("case", _mid_cases(), ids=lambda c: f"m{c[0]}")
def test_mid_size_case_vs_chunked_oracle(case, device):
    """Same bar, against the oracle's query-chunked torch fp32 path run on the GPU."""
    import gemma_triton_flash_attn_amd as gfa

    i, B, Hq, Hkv, N, D, causal, window, dtype, layout = case
    print(f"case m{i}: B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal} window={window} {dtype} {layout}",
          flush=True)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, dtype, device, seed=5000 + i, layout=layout)
    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = gfa.flash_attn_gqa_train(qq, kk, vv, causal=causal, slide_size=window)
    o.backward(do)
    torch.cuda.synchronize()
    o_ref, lse_ref = orc.forward_chunked(q, k, v, causal, window)
    dq_ref, dk_ref, dv_ref, _ = orc.backward_chunked(q, k, v, do, causal, window, o=o_ref, lse=lse_ref)
    err_o = float((o.detach().float() - o_ref).abs().max())

    def rel(a, b):
        floor = GRAD_ABS_RMS * b.numel() ** 0.5 / GRAD_TOL
        return float(torch.linalg.vector_norm(a.float() - b) / max(float(torch.linalg.vector_norm(b)), floor))

    errs = [rel(g, r) for g, r in ((qq.grad, dq_ref), (kk.grad, dk_ref), (vv.grad, dv_ref))]
    print(f"  O max-abs {err_o:.3e}  dQ/dK/dV rel {errs[0]:.3e} {errs[1]:.3e} {errs[2]:.3e}", flush=True)
    assert err_o <= O_TOL[dtype]
    assert max(errs) <= GRAD_TOL

