"""The torch.library ops (ops.py) on the GPU: torch.library.opcheck over the registration,
bitwise agreement with the autograd.Function path (same kernels), and torch.compile with
fullgraph=True through forward and backward (no graph break at the attention call)."""
from __future__ import annotations

import pytest
import torch

import gemma_triton_flash_attn_amd  # noqa: F401  (registers gfa::attn_fwd / gfa::attn_bwd)
from conftest import make_inputs

pytestmark = pytest.mark.gpu

CASES = [(1, 8, 1, 128, 512, True, 0), (1, 4, 2, 96, 256, True, 40), (1, 2, 2, 64, 256, False, 0),
         (1, 8, 2, 80, 128, True, 24), (2, 4, 4, 50, 64, False, 0)]


@pytest.mark.parametrize("B,Hq,Hkv,N,D,causal,window", CASES)
def test_opcheck(B, Hq, Hkv, N, D, causal, window, device):
    print(f"case opcheck B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal} window={window}", flush=True)
    q, k, v, _ = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=3)
    q, k, v = (t.requires_grad_(True) for t in (q, k, v))
    torch.library.opcheck(torch.ops.gfa.attn_fwd, (q, k, v, causal, window, D ** -0.5),
                          test_utils=("test_schema", "test_autograd_registration", "test_faketensor"))


@pytest.mark.parametrize("B,Hq,Hkv,N,D,causal,window", CASES)
def test_op_matches_function_bitwise(B, Hq, Hkv, N, D, causal, window, device):
    import gemma_triton_flash_attn_amd as gfa

    print(f"case op-vs-function B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal} window={window}", flush=True)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=4)
    outs = []
    for fn in (gfa.flash_attn_gqa_train, gfa.flash_attn_gqa_op):
        qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
        o = fn(qq, kk, vv, causal=causal, slide_size=window)
        o.backward(do)
        outs.append((o.detach(), qq.grad, kk.grad, vv.grad))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_compile_fullgraph_forward_backward(device):
    import gemma_triton_flash_attn_amd as gfa

    print("case torch.compile fullgraph aot_eager D=256 window=48", flush=True)
    q, k, v, do = make_inputs(1, 8, 2, 160, 256, torch.bfloat16, device, seed=5, layout="bnhd")

    def layer(q, k, v):
        o = gfa.flash_attn_gqa_op(q * 1.0, k, v, causal=True, slide_size=48, scale=0.05)
        return o.transpose(1, 2).contiguous()

    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    res = []
    for fn in (layer, compiled):
        qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        o = fn(qq, kk, vv)
        o.backward(do.transpose(1, 2))
        res.append((o.detach(), qq.grad, kk.grad, vv.grad))
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_compile_fullgraph_with_dropout_and_segments(device):
    """The dropout seed is drawn inside the op (returned as a CPU tensor for the backward) and
    segment tables are checked without host reads under compilation, so a layer with attention
    dropout on a packed batch traces with fullgraph=True; under the same torch.manual_seed the
    compiled and eager runs draw the same seeds and agree bitwise, forward and backward."""
    import gemma_triton_flash_attn_amd as gfa

    print("case torch.compile fullgraph aot_eager dropout + packed segments D=256 window=48", flush=True)
    N = 160
    q, k, v, do = make_inputs(1, 8, 2, N, 256, torch.bfloat16, device, seed=6)
    lo, hi = gfa.segments.from_cu_seqlens([0, 50, 51, 120], N, device=device)

    def layer(q, k, v, lo, hi):
        return gfa.flash_attn_gqa_op(q, k, v, causal=True, slide_size=48, segments=(lo, hi), dropout_p=0.2)

    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    res = []
    for fn in (layer, compiled, compiled):
        torch.manual_seed(21)
        qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        o = fn(qq, kk, vv, lo, hi)
        o.backward(do)
        res.append((o.detach(), qq.grad, kk.grad, vv.grad))
    for r in res[1:]:
        for a, b in zip(res[0], r):
            assert torch.equal(a, b)
    # the mask is live: another seed gives another output
    torch.manual_seed(22)
    assert not torch.equal(compiled(q, k, v, lo, hi), res[0][0])


def test_compile_fullgraph_adapter_with_padding_mask(device):
    """The HF adapter path on a left-padded batch (mask creator, padding mask to segment tables,
    the op) traces with fullgraph=True and agrees bitwise with eager; so does an unpadded batch,
    which under compilation runs with a one-segment table instead of none."""
    from types import SimpleNamespace

    import gemma_triton_flash_attn_amd as gfa
    from gemma_triton_flash_attn_amd.hf_integration import padding_mask_for_engine

    print("case torch.compile fullgraph aot_eager HF adapter + padding mask D=128", flush=True)
    B, Hq, Hkv, N, D = 2, 4, 2, 96, 128
    q, k, v = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=8, with_do=False, layout="bnhd")
    mod = SimpleNamespace(head_dim=D, is_causal=True)

    def attn(q, k, v, mask):
        m = padding_mask_for_engine(B, N, N, attention_mask=mask)
        out, _ = gfa.triton_gqa_attention(mod, q, k, v, m, scaling=0.09, sliding_window=40)
        return out

    compiled = torch.compile(attn, backend="aot_eager", fullgraph=True)
    padded = torch.ones(B, N, dtype=torch.bool, device=device)
    padded[0, :17] = False
    full = torch.ones(B, N, dtype=torch.bool, device=device)
    for mask in (padded, full):
        assert torch.equal(compiled(q, k, v, mask), attn(q, k, v, mask))
