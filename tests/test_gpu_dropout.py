"""Attention dropout (``dropout_p``): GPU parity of every kernel's DROP instance against the oracle,
which restates the engine's counter-based mask (oracle/attention_oracle.py, dropout_mask) and is
pinned to float64 torch autograd through the same mask (tests/test_oracle.py). The reference has
no dropout (its adapter raises). With the same seed the kernels and the oracle drop the same
entries, so the comparison is element for element.

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
SEED = 0x5EED_1234_ABCD


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _rel(a, b):
    floor = GRAD_ABS_RMS * np.sqrt(b.size) / GRAD_TOL
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), floor))


CASES = [
    # B, Hq, Hkv, N, D, causal, window, dtype, p
    (1, 8, 1, 96, 512, True, 0, torch.bfloat16, 0.2),
    (2, 4, 2, 70, 512, False, 0, torch.float16, 0.5),
    (1, 8, 1, 130, 512, True, 40, torch.bfloat16, 0.1),
    (2, 4, 2, 100, 256, True, 0, torch.bfloat16, 0.3),
    (1, 4, 2, 160, 256, True, 48, torch.bfloat16, 0.2),   # windowed: the one-wave dK/dV form
    (1, 8, 8, 33, 256, False, 0, torch.float16, 0.5),
    (1, 8, 2, 200, 128, True, 0, torch.bfloat16, 0.25),
    (2, 4, 1, 131, 128, True, 37, torch.float16, 0.1),
    (1, 8, 1, 300, 64, True, 0, torch.float16, 0.4),
    (2, 6, 2, 77, 64, True, 16, torch.bfloat16, 0.2),
]


@pytest.mark.parametrize("B,Hq,Hkv,N,D,causal,window,dtype,p", CASES)
def test_dropout_fwd_bwd_vs_oracle(B, Hq, Hkv, N, D, causal, window, dtype, p, device):
    from gemma_triton_flash_attn_amd.attention import _backward, _forward

    print(f"dropout case B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal} window={window} {dtype} p={p}",
          flush=True)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, dtype, device, seed=N + D + 1)
    sc = D ** -0.5
    o, lse = _forward(q, k, v, causal, window, sc, store_lse=True, dropout_p=p, dropout_seed=SEED)
    dq, dk, dv, _ = _backward(q, k, v, o, lse, do, causal, window, sc, dropout_p=p, dropout_seed=SEED)
    torch.cuda.synchronize()
    o_ref, lse_ref = orc.forward(_np(q), _np(k), _np(v), causal, window, dropout=(p, SEED))
    dq_ref, dk_ref, dv_ref, _ = orc.backward(_np(q), _np(k), _np(v), _np(do), causal, window, dropout=(p, SEED))
    err_o = float(np.abs(_np(o) - o_ref).max())
    errs = [_rel(_np(g), r) for g, r in ((dq, dq_ref), (dk, dk_ref), (dv, dv_ref))]
    print(f"  O max-abs {err_o:.3e}  dQ/dK/dV rel {errs[0]:.3e} {errs[1]:.3e} {errs[2]:.3e}", flush=True)
    assert err_o <= O_TOL[dtype]
    assert max(errs) <= GRAD_TOL
    # the LSE is the undropped one
    assert float(np.abs(_np(lse[:, :, :N]) - lse_ref).max()) <= 1e-2
    # the mask matters: the undropped output is far away
    o_keep, _ = orc.forward(_np(q), _np(k), _np(v), causal, window)
    assert float(np.abs(o_keep - o_ref).max()) > 5 * O_TOL[dtype]


def test_dropout_training_api_seeding(device):
    """flash_attn_gqa_train draws its mask seed from torch's generator: the same manual seed
    gives the same output and gradients, another seed another mask; Q-split partials and the
    one-call op path agree with the oracle under the drawn seed."""
    import gemma_triton_flash_attn_amd as gfa
    from gemma_triton_flash_attn_amd.attention import _dropout_seed

    q, k, v, do = make_inputs(1, 8, 2, 150, 256, torch.bfloat16, device, seed=3)

    def run(fn, s):
        torch.manual_seed(s)
        qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        o = fn(qq, kk, vv, causal=True, slide_size=64, dropout_p=0.3)
        o.backward(do)
        torch.cuda.synchronize()
        return o, qq.grad, kk.grad, vv.grad

    a = run(gfa.flash_attn_gqa_train, 11)
    b = run(gfa.flash_attn_gqa_train, 11)
    c = run(gfa.flash_attn_gqa_train, 12)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    assert not torch.equal(a[0], c[0])
    torch.manual_seed(11)
    seed = _dropout_seed()
    o_ref, _ = orc.forward(_np(q), _np(k), _np(v), True, 64, dropout=(0.3, seed))
    dq_ref, dk_ref, dv_ref, _ = orc.backward(_np(q), _np(k), _np(v), _np(do), True, 64, dropout=(0.3, seed))
    assert float(np.abs(_np(a[0]) - o_ref).max()) <= O_TOL[torch.bfloat16]
    assert max(_rel(_np(g), r) for g, r in zip(a[1:], (dq_ref, dk_ref, dv_ref))) <= GRAD_TOL
    op = run(gfa.flash_attn_gqa_op, 11)
    for x, y in zip(a, op):
        assert torch.equal(x, y)


@pytest.mark.parametrize("D", [512, 128])
def test_dropout_q_splits(D, device):
    from gemma_triton_flash_attn_amd.attention import _backward, _forward

    q, k, v, do = make_inputs(1, 8, 2, 150, D, torch.bfloat16, device, seed=D + 5)
    sc = D ** -0.5
    o, lse = _forward(q, k, v, True, 0, sc, store_lse=True, dropout_p=0.25, dropout_seed=SEED)
    dq_ref, dk_ref, dv_ref, _ = orc.backward(_np(q), _np(k), _np(v), _np(do), True, 0, dropout=(0.25, SEED))
    for qs in (1, 4):
        dq, dk, dv, _ = _backward(q, k, v, o, lse, do, True, 0, sc, q_splits=qs, dropout_p=0.25, dropout_seed=SEED)
        torch.cuda.synchronize()
        assert max(_rel(_np(g), r) for g, r in ((dq, dq_ref), (dk, dk_ref), (dv, dv_ref))) <= GRAD_TOL, qs


def test_hf_adapter_dropout(device):
    """transformers passes ``dropout`` (the attention dropout in training, 0 in eval)."""
    from types import SimpleNamespace

    import gemma_triton_flash_attn_amd as gfa
    from gemma_triton_flash_attn_amd.attention import _dropout_seed

    B, Hq, Hkv, N, D = 1, 8, 2, 96, 256
    q, k, v, _ = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=13)
    mod = SimpleNamespace(head_dim=D, is_causal=True)
    torch.manual_seed(5)
    out, _ = gfa.triton_gqa_attention(mod, q, k, v, None, dropout=0.2, scaling=D ** -0.5)
    torch.cuda.synchronize()
    torch.manual_seed(5)
    o_ref, _ = orc.forward(_np(q), _np(k), _np(v), True, 0, dropout=(0.2, _dropout_seed()))
    assert float(np.abs(_np(out.transpose(1, 2)) - o_ref).max()) <= O_TOL[torch.bfloat16]


@pytest.mark.parametrize("D,window,kind", [(512, 0, "left_padded"), (512, 0, "packed"), (256, 40, "left_padded"),
                                           (256, 40, "packed"), (128, 24, "packed")])
def test_dropout_with_segments(D, window, kind, device):
    """Dropout on a padded or packed batch: the SEG+DROP forward instances and the segment paths of
    both backward kernels, against the oracle with the same segments and mask."""
    import gemma_triton_flash_attn_amd as gfa
    from gemma_triton_flash_attn_amd.attention import _backward, _forward

    print(f"dropout+segments case D={D} window={window} {kind}", flush=True)
    if kind == "left_padded":
        B, N = 2, 130
        segs = gfa.segments.from_lengths([N - 37, N - 5], N, left_padding=True, device=device)
    else:
        B, N = 1, 150
        segs = gfa.segments.from_cu_seqlens([0, 40, 41, 97, 140], N, device=device)
    q, k, v, do = make_inputs(B, 4, 2, N, D, torch.bfloat16, device, seed=D + N)
    sc = D ** -0.5
    o, lse = _forward(q, k, v, True, window, sc, store_lse=True, segments=segs, dropout_p=0.2, dropout_seed=SEED)
    dq, dk, dv, _ = _backward(q, k, v, o, lse, do, True, window, sc, segments=segs, dropout_p=0.2,
                              dropout_seed=SEED)
    torch.cuda.synchronize()
    seg_np = (segs[0].cpu().numpy(), segs[1].cpu().numpy())
    o_ref, _ = orc.forward(_np(q), _np(k), _np(v), True, window, segments=seg_np, dropout=(0.2, SEED))
    dq_ref, dk_ref, dv_ref, _ = orc.backward(_np(q), _np(k), _np(v), _np(do), True, window, segments=seg_np,
                                             dropout=(0.2, SEED))
    err_o = float(np.abs(_np(o) - o_ref).max())
    errs = [_rel(_np(g), r) for g, r in ((dq, dq_ref), (dk, dk_ref), (dv, dv_ref))]
    print(f"  O max-abs {err_o:.3e}  dQ/dK/dV rel {errs[0]:.3e} {errs[1]:.3e} {errs[2]:.3e}", flush=True)
    assert err_o <= O_TOL[torch.bfloat16]
    assert max(errs) <= GRAD_TOL
