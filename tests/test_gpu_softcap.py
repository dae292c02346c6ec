"""Logit soft-capping (``softcap``): GPU parity of every kernel's soft-capped instance against the
oracle (float64 numpy, tanh of the scaled scores before the mask and the softmax, dS times
1 - tanh^2), on the same 16-bit inputs. The reference has no soft-capping (its adapter raises);
transformers' Gemma-2 eager attention defines the operation, and tests/test_oracle.py pins the
oracle to it. Inputs are scaled up so that many scores reach the cap.

Bar (as tests/test_gpu_parity.py): O max-abs <= 1e-2 (fp16) / 2e-2 (bf16); dQ, dK, dV relative
Frobenius error <= 5e-2, with an absolute floor for near-zero gradients.
"""
from __future__ import annotations

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


def _inputs(B, Hq, Hkv, N, D, dtype, device, seed):
    # scores of a few units after scaling, so that a cap of 2-5 bends most of them
    return make_inputs(B, Hq, Hkv, N, D, dtype, device, seed=seed, scale=2.0)


CASES = [
    # B, Hq, Hkv, N, D, causal, window, dtype, softcap
    (1, 8, 1, 96, 512, True, 0, torch.bfloat16, 3.0),
    (2, 4, 2, 70, 512, False, 0, torch.float16, 5.0),
    (1, 8, 1, 130, 512, True, 40, torch.bfloat16, 2.0),
    (2, 4, 2, 100, 256, True, 0, torch.bfloat16, 3.0),
    (1, 4, 2, 160, 256, True, 48, torch.bfloat16, 2.0),   # windowed: the one-wave dK/dV form
    (1, 8, 8, 33, 256, False, 0, torch.float16, 4.0),
    (1, 8, 2, 200, 128, True, 0, torch.bfloat16, 3.0),
    (2, 4, 1, 131, 128, True, 37, torch.float16, 2.5),
    (1, 8, 1, 300, 64, True, 0, torch.float16, 3.0),
    (2, 6, 2, 77, 64, True, 16, torch.bfloat16, 2.0),
    (1, 2, 2, 45, 64, False, 0, torch.bfloat16, 50.0),    # a cap that barely bends
]


@pytest.mark.parametrize("B,Hq,Hkv,N,D,causal,window,dtype,softcap", CASES)
def test_softcap_fwd_bwd_vs_oracle(B, Hq, Hkv, N, D, causal, window, dtype, softcap, device):
    import gemma_triton_flash_attn_amd as gfa

    print(f"softcap case B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal} window={window} {dtype} "
          f"cap={softcap}", flush=True)
    q, k, v, do = _inputs(B, Hq, Hkv, N, D, dtype, device, seed=N + D)
    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = gfa.flash_attn_gqa_train(qq, kk, vv, causal=causal, slide_size=window, softcap=softcap)
    o.backward(do)
    torch.cuda.synchronize()
    o_ref, _ = orc.forward(_np(q), _np(k), _np(v), causal, window, softcap=softcap)
    dq_ref, dk_ref, dv_ref, _ = orc.backward(_np(q), _np(k), _np(v), _np(do), causal, window, softcap=softcap)
    err_o = float(np.abs(_np(o) - o_ref).max())
    errs = [_rel(_np(g), r) for g, r in ((qq.grad, dq_ref), (kk.grad, dk_ref), (vv.grad, dv_ref))]
    print(f"  O max-abs {err_o:.3e}  dQ/dK/dV rel {errs[0]:.3e} {errs[1]:.3e} {errs[2]:.3e}", flush=True)
    assert err_o <= O_TOL[dtype]
    assert max(errs) <= GRAD_TOL
    if softcap < 10:
        # the cap matters at these magnitudes: the uncapped result is far from the capped one
        o_nocap, _ = orc.forward(_np(q), _np(k), _np(v), causal, window)
        assert float(np.abs(o_nocap - o_ref).max()) > 5 * O_TOL[dtype]


@pytest.mark.parametrize("D", [512, 256, 128, 64])
def test_softcap_inference_and_splits(D, device):
    """The inference forward (no LSE) equals the training forward bit for bit, and the dK/dV
    Q-split partial path (q_splits 1 and 4) agrees with the oracle under soft-capping."""
    import gemma_triton_flash_attn_amd as gfa
    from gemma_triton_flash_attn_amd.attention import _backward, _forward

    q, k, v, do = _inputs(1, 8, 2, 150, D, torch.bfloat16, device, seed=D)
    sc = D ** -0.5
    o_inf = gfa.attention_flash_gqa(q, k, v, causal=True, slide_size=64, softcap=3.0)
    o, lse = _forward(q, k, v, True, 64, sc, store_lse=True, softcap=3.0)
    torch.cuda.synchronize()
    assert torch.equal(o_inf, o)
    dq_ref, dk_ref, dv_ref, _ = orc.backward(_np(q), _np(k), _np(v), _np(do), True, 64, softcap=3.0)
    for qs in (1, 4):
        dq, dk, dv, _ = _backward(q, k, v, o, lse, do, True, 64, sc, q_splits=qs, softcap=3.0)
        torch.cuda.synchronize()
        errs = [_rel(_np(g), r) for g, r in ((dq, dq_ref), (dk, dk_ref), (dv, dv_ref))]
        assert max(errs) <= GRAD_TOL, (qs, errs)


def test_softcap_with_segments(device):
    """Soft-capping with a segment table (a padded batch) against the oracle."""
    import gemma_triton_flash_attn_amd as gfa

    B, Hq, Hkv, N, D = 2, 4, 2, 120, 256
    q, k, v, do = _inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=7)
    segs = gfa.segments.from_lengths([N - 30, N], N, device=device)
    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = gfa.flash_attn_gqa_train(qq, kk, vv, causal=True, segments=segs, softcap=3.0)
    o.backward(do)
    torch.cuda.synchronize()
    seg_np = (segs[0].cpu().numpy(), segs[1].cpu().numpy())
    o_ref, _ = orc.forward(_np(q), _np(k), _np(v), True, 0, segments=seg_np, softcap=3.0)
    dq_ref, dk_ref, dv_ref, _ = orc.backward(_np(q), _np(k), _np(v), _np(do), True, 0, segments=seg_np, softcap=3.0)
    assert float(np.abs(_np(o) - o_ref).max()) <= O_TOL[torch.bfloat16]
    errs = [_rel(_np(g), r) for g, r in ((qq.grad, dq_ref), (kk.grad, dk_ref), (vv.grad, dv_ref))]
    assert max(errs) <= GRAD_TOL


def test_hf_adapter_softcap(device):
    """transformers' ``softcap`` through the adapter (as Gemma-2 attention passes it)."""
    from types import SimpleNamespace

    import gemma_triton_flash_attn_amd as gfa

    B, Hq, Hkv, N, D = 1, 8, 2, 96, 256
    q, k, v, _ = _inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=11)
    mod = SimpleNamespace(head_dim=D, is_causal=True)
    out, _ = gfa.triton_gqa_attention(mod, q, k, v, None, scaling=D ** -0.5, softcap=4.0, sliding_window=40)
    torch.cuda.synchronize()
    o_ref, _ = orc.forward(_np(q), _np(k), _np(v), True, 40, softcap=4.0)
    assert tuple(out.shape) == (B, N, Hq, D)
    assert float(np.abs(_np(out.transpose(1, 2)) - o_ref).max()) <= O_TOL[torch.bfloat16]
