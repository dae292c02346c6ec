"""Closed-form known answers checked on the GPU kernels directly (no oracle in the loop).

The known-answer list of the hot-path survey (attention with Q = 0, W = 1, N = 1, GQA versus
MHA on repeated K/V, the Q = 0 backward) fixes outputs that follow from the mathematics
alone. Each case runs through the C ABI (the package's public functions) at every head dim.
"""
from __future__ import annotations

import pytest
import torch

from conftest import make_inputs

pytestmark = pytest.mark.gpu

HEAD_DIMS = [64, 128, 256, 512]


def _allowed_counts(N, causal, window, device):
    i = torch.arange(N, device=device)
    if not causal:
        return torch.full((N,), N, device=device, dtype=torch.float64)
    lo = torch.clamp(i - window + 1, min=0) if 0 < window < N else torch.zeros_like(i)
    return (i - lo + 1).double()


def _window_mean(v, causal, window):
    """Mean of v over each query's allowed keys, in float64: (B, H, N, D)."""
    N = v.shape[2]
    vd = v.double()
    if not causal:
        return vd.mean(dim=2, keepdim=True).expand_as(vd)
    c = torch.cumsum(vd, dim=2)
    i = torch.arange(N, device=v.device)
    lo = torch.clamp(i - window + 1, min=0) if 0 < window < N else torch.zeros_like(i)
    prev = torch.where((lo > 0)[:, None], c[:, :, (lo - 1).clamp(min=0)], torch.zeros_like(c[:, :, :1]))
    return (c - prev) / (i - lo + 1).double()[:, None]


@pytest.mark.parametrize("D", HEAD_DIMS)
@pytest.mark.parametrize("causal,window", [(True, 0), (True, 37), (False, 0)])
def test_zero_queries_give_window_means_and_log_counts(D, causal, window, device):
    from gemma_triton_flash_attn_amd.attention import _forward

    B, Hq, Hkv, N = 1, 4, 2, 150
    print(f"case Q=0 D={D} causal={causal} window={window}", flush=True)
    q, k, v, _ = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=D + window)
    q = torch.zeros_like(q)
    o, lse = _forward(q, k, v, causal, window, D ** -0.5, store_lse=True)
    torch.cuda.synchronize()
    want = _window_mean(v, causal, window).repeat_interleave(Hq // Hkv, dim=1)
    assert float((o.double() - want).abs().max()) <= 2e-2          # bf16 output rounding
    counts = _allowed_counts(N, causal, window, device)
    assert float((lse[..., :N].double() - torch.log(counts)).abs().max()) <= 1e-4


@pytest.mark.parametrize("D", HEAD_DIMS)
def test_window_one_returns_v_exactly(D, device):
    import gemma_triton_flash_attn_amd as gfa

    B, Hq, Hkv, N = 2, 6, 3, 77
    q, k, v, _ = make_inputs(B, Hq, Hkv, N, D, torch.float16, device, seed=3 * D)
    o = gfa.attention_flash_gqa(q, k, v, causal=True, slide_size=1)
    torch.cuda.synchronize()
    # P = 1 on the diagonal: O = V, exactly representable
    assert torch.equal(o, v.repeat_interleave(Hq // Hkv, dim=1))


@pytest.mark.parametrize("D", HEAD_DIMS)
@pytest.mark.parametrize("causal", [True, False])
def test_single_row_returns_v0(D, causal, device):
    import gemma_triton_flash_attn_amd as gfa

    q, k, v, _ = make_inputs(2, 8, 2, 1, D, torch.bfloat16, device, seed=D)
    o = gfa.attention_flash_gqa(q, k, v, causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(o, v.repeat_interleave(4, dim=1))


@pytest.mark.parametrize("D", HEAD_DIMS)
@pytest.mark.parametrize("window", [0, 50])
def test_gqa_equals_mha_on_repeated_kv(D, window, device):
    import gemma_triton_flash_attn_amd as gfa

    B, Hq, Hkv, N = 1, 8, 2, 180
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=D + 1)
    R = Hq // Hkv
    kr, vr = k.repeat_interleave(R, dim=1), v.repeat_interleave(R, dim=1)

    def run(kk, vv):
        qq, k2, v2 = (t.detach().clone().requires_grad_(True) for t in (q, kk, vv))
        o = gfa.flash_attn_gqa_train(qq, k2, v2, causal=True, slide_size=window)
        o.backward(do)
        return o.detach(), qq.grad, k2.grad, v2.grad

    o1, dq1, dk1, dv1 = run(k, v)
    o2, dq2, dk2, dv2 = run(kr, vr)
    torch.cuda.synchronize()
    assert float((o1.float() - o2.float()).abs().max()) <= 1e-2
    assert float((dq1.float() - dq2.float()).norm() / dq2.float().norm()) <= 1e-2
    # dK/dV of a KV head = the sum over its query heads of the MHA gradients
    for g, g2 in ((dk1, dk2), (dv1, dv2)):
        summed = g2.float().reshape(B, Hkv, R, N, D).sum(dim=2)
        assert float((g.float() - summed).norm() / summed.norm()) <= 1e-2


@pytest.mark.parametrize("D", HEAD_DIMS)
@pytest.mark.parametrize("causal,window", [(True, 0), (True, 29)])
def test_zero_queries_backward_closed_form(D, causal, window, device):
    """Q = 0: every allowed key has P = 1/|allowed(i)|, so dV_j = sum over the queries that
    see key j of dO_i / |allowed(i)| (summed over the KV group), and dK = s * dS^T Q = 0."""
    import gemma_triton_flash_attn_amd as gfa

    B, Hq, Hkv, N = 1, 4, 1, 130
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=7 + D)
    q = torch.zeros_like(q)
    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = gfa.flash_attn_gqa_train(qq, kk, vv, causal=causal, slide_size=window)
    o.backward(do)
    torch.cuda.synchronize()
    i = torch.arange(N, device=device)[:, None]
    j = torch.arange(N, device=device)[None, :]
    allowed = j <= i
    if window:
        allowed &= (i - j) < window
    p = allowed.double() / allowed.sum(dim=1, keepdim=True).double()      # (N queries, N keys)
    dv_want = torch.einsum("ij,bhid->bjd", p, do.double())[:, None]       # summed over query heads
    assert float((vv.grad.double() - dv_want).norm() / dv_want.norm()) <= 1e-2
    assert float(kk.grad.float().abs().max()) == 0.0
