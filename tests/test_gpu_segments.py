"""Ragged batches on the GPU (segment tables, include/gfa.h): padded, left-padded, packed and
all-padding rows, forward and backward, against the oracle's segment semantics (pinned in
test_segments_cpu.py), at the north-star bar: O max-abs <= 1e-2 (fp16) / 2e-2 (bf16),
dQ/dK/dV relative Frobenius error <= 5e-2; padding tokens' outputs and gradients exactly 0.

Also: every entry point takes the tables (inference forward bit-identical to the training
forward, the torch.library op, q_splits, gfa_bwd_noalloc), a padded batch gives each
sequence what it gets alone, and the HF adapter inside a Gemma-4 model turns a left-padding
mask into the attention each unpadded sequence gets alone.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import make_inputs, recomputing
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

O_TOL = {torch.float16: 1e-2, torch.bfloat16: 2e-2}
GRAD_TOL = 5e-2


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _rel(a, b):
    nb = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / nb) if nb > 0 else float(np.linalg.norm(a))


def _tables(kind, B, N, device):
    import gemma_triton_flash_attn_amd as gfa

    seg = gfa.segments
    g = np.random.default_rng(N + B)
    if kind == "right":
        return seg.from_lengths(g.integers(1, N + 1, B).tolist(), N, device=device)
    if kind == "left":
        return seg.from_lengths(g.integers(1, N + 1, B).tolist(), N, left_padding=True, device=device)
    if kind == "packed":
        rows = []
        for _ in range(B):
            cuts = np.sort(g.choice(np.arange(1, N), size=min(5, N - 1), replace=False))
            end = int(g.integers(cuts[-1], N + 1))
            lo, hi = seg.from_cu_seqlens([0, *cuts.tolist(), end], N, device=device)
            rows.append((lo, hi))
        return torch.cat([r[0] for r in rows]), torch.cat([r[1] for r in rows])
    if kind == "mixed":  # one full row, one empty row, one right-padded row
        lens = [N, 0, max(1, N // 3)][:B] + [N] * max(0, B - 3)
        return seg.from_lengths(lens, N, device=device)
    raise ValueError(kind)


def _run(q, k, v, do, causal, window, segments, **kw):
    import gemma_triton_flash_attn_amd as gfa

    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = gfa.flash_attn_gqa_train(qq, kk, vv, causal=causal, slide_size=window, segments=segments, **kw)
    o.backward(do)
    torch.cuda.synchronize()
    return o.detach(), qq.grad, kk.grad, vv.grad


def _check(q, k, v, do, causal, window, segments, got):
    o, dq, dk, dv = got
    tabs = tuple(t.cpu().numpy() for t in segments)
    o_ref, _ = orc.forward(_np(q), _np(k), _np(v), causal, window, segments=tabs)
    g_ref = orc.backward(_np(q), _np(k), _np(v), _np(do), causal, window, segments=tabs)
    err_o = float(np.abs(_np(o) - o_ref).max())
    errs = [_rel(_np(a), b) for a, b in zip((dq, dk, dv), g_ref[:3])]
    assert err_o <= O_TOL[q.dtype], err_o
    assert max(errs) <= GRAD_TOL, errs
    # padding tokens: exactly zero output rows and gradient rows
    pad = (segments[0] == segments[1]).cpu()
    for b in range(q.shape[0]):
        p = pad[b].nonzero().flatten().tolist()
        if p:
            assert torch.count_nonzero(o[b][:, p]) == 0
            for g_ in (dq[b], dk[b], dv[b]):
                assert torch.count_nonzero(g_[:, p]) == 0
    return err_o, errs


CASES = [
    # kind, B, Hq, Hkv, N, D, causal, window, dtype
    ("right", 3, 4, 2, 150, 256, True, 0, torch.bfloat16),
    ("left", 3, 4, 2, 150, 256, True, 48, torch.bfloat16),
    ("packed", 2, 8, 1, 200, 512, True, 0, torch.bfloat16),
    ("packed", 1, 4, 2, 300, 256, True, 64, torch.float16),
    ("mixed", 3, 4, 1, 97, 512, True, 0, torch.float16),
    ("right", 2, 4, 4, 130, 128, False, 0, torch.bfloat16),
    ("packed", 2, 4, 2, 180, 128, True, 32, torch.float16),
    ("left", 2, 8, 2, 100, 64, True, 0, torch.bfloat16),
    ("packed", 1, 4, 1, 260, 64, False, 0, torch.float16),
    ("mixed", 3, 2, 2, 64, 64, True, 8, torch.bfloat16),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-D{c[5]}-N{c[4]}-c{int(c[6])}w{c[7]}" for c in CASES])
def test_segments_against_oracle(case, device):
    kind, B, Hq, Hkv, N, D, causal, window, dtype = case
    print(f"case {case}", flush=True)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, dtype, device, seed=N + D)
    segs = _tables(kind, B, N, device)
    err_o, errs = _check(q, k, v, do, causal, window, segs, _run(q, k, v, do, causal, window, segs))
    print(f"  O max-abs {err_o:.2e}  grads {errs[0]:.2e} {errs[1]:.2e} {errs[2]:.2e}", flush=True)


def test_segments_every_entry_point(device):
    """Inference forward, the torch.library op, forced q_splits and gfa_bwd_noalloc all take
    the tables and agree with the training path."""
    import gemma_triton_flash_attn_amd as gfa
    from gemma_triton_flash_attn_amd.attention import _backward, _forward

    B, Hq, Hkv, N, D = 2, 8, 1, 700, 512
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=3)
    segs = _tables("packed", B, N, device)
    o, dq, dk, dv = _run(q, k, v, do, True, 0, segs)
    inf = gfa.attention_flash_gqa(q, k, v, causal=True, segments=segs)
    assert torch.equal(inf, o)
    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    oo = gfa.flash_attn_gqa_op(qq, kk, vv, causal=True, segments=segs)
    oo.backward(do)
    assert torch.equal(oo, o) and torch.equal(qq.grad, dq) and torch.equal(kk.grad, dk) and torch.equal(vv.grad, dv)
    sc = D ** -0.5
    o2, lse = _forward(q, k, v, True, 0, sc, store_lse=True, segments=segs)
    for qs in (1, 2, 8):
        g = _backward(q, k, v, o2, lse, do, True, 0, sc, q_splits=qs, segments=segs)
        assert torch.equal(g[0], dq)
        for a, b in zip(g[1:3], (dk, dv)):
            assert _rel(_np(a), _np(b)) < 1e-2
    # gfa_bwd_noalloc runs the recomputing form: bit for bit gfa_bwd's recomputing form, and
    # within the bar of its default (materialised, the dS store narrowed by the tables)
    gn = _backward(q, k, v, o2, lse, do, True, 0, sc, q_splits=1, segments=segs, noalloc=True)
    with recomputing():
        g1 = _backward(q, k, v, o2, lse, do, True, 0, sc, q_splits=1, segments=segs)
    for a, b in zip(gn[:3], g1[:3]):
        assert torch.equal(a, b)
    for a, b in zip(gn[:3], (dq, dk, dv)):
        assert _rel(_np(a), _np(b)) < 1e-2


@pytest.mark.parametrize("D,window", [(512, 0), (256, 512)])
def test_padded_batch_equals_each_sequence_alone(D, window, device):
    """Right-padded rows of different lengths give, on their real tokens, what each sequence
    gives alone (to the bar: tile boundaries differ, so not bit for bit)."""
    import gemma_triton_flash_attn_amd as gfa

    lens = [1000, 1777, 64]
    N, Hq, Hkv = max(lens), 8, 1
    q, k, v, do = make_inputs(len(lens), Hq, Hkv, N, D, torch.bfloat16, device, seed=11)
    segs = gfa.segments.from_lengths(lens, N, device=device)
    o, dq, dk, dv = _run(q, k, v, do, True, window, segs)
    for b, n in enumerate(lens):
        o1, dq1, dk1, dv1 = _run(q[b:b + 1, :, :n], k[b:b + 1, :, :n], v[b:b + 1, :, :n], do[b:b + 1, :, :n], True,
                                 window if window < n else 0, None)
        assert float((o[b:b + 1, :, :n].float() - o1.float()).abs().max()) <= O_TOL[torch.bfloat16]
        for a, r in ((dq, dq1), (dk, dk1), (dv, dv1)):
            assert _rel(_np(a[b:b + 1, :, :n]), _np(r)) <= GRAD_TOL
        assert torch.count_nonzero(o[b, :, n:]) == 0


def test_hf_left_padded_batch_matches_each_sequence(device):
    """A left-padded batch through a Gemma-4 model on the engine: the padding mask reaches the
    adapter through the registered mask creator and becomes a segment table. The first
    layer's attention output on each row's real tokens (whose inputs are identical in both
    runs) must match that sequence run alone, at the reference's adapter bar (cos > 0.999,
    rel < 0.05); ignoring the mask would let real tokens attend to the padding tokens before
    them. The logits get a looser sanity bound (a random-init model amplifies rounding
    differences layer by layer)."""
    pytest.importorskip("transformers")
    from transformers import AttentionInterface

    import gemma_triton_flash_attn_amd as gfa
    from hf_models import build_model, tiny_gemma4_config

    captured = []

    def capturing(module, query, key, value, attention_mask, **kwargs):
        out, w = gfa.triton_gqa_attention(module, query, key, value, attention_mask, **kwargs)
        if module.layer_idx == 0:
            captured.append(out.detach().float().clone())
        return out, w

    gfa.register_triton_attention("gfa_seg_capture")
    AttentionInterface.register("gfa_seg_capture", capturing)  # keeps the engine's mask creator
    cfg = tiny_gemma4_config(n_layers=2, sliding_window=64)
    model = build_model(cfg, device, torch.bfloat16)
    for m in model.modules():
        c = getattr(m, "config", None)
        if c is not None and hasattr(c, "_attn_implementation"):
            c._attn_implementation = "gfa_seg_capture"
    lens = [300, 177]
    N = max(lens)
    gen = torch.Generator().manual_seed(4)
    seqs = [torch.randint(0, cfg.vocab_size, (n,), generator=gen).to(device) for n in lens]
    ids = torch.zeros(2, N, dtype=torch.long, device=device)
    mask = torch.zeros(2, N, dtype=torch.long, device=device)
    pos = torch.zeros(2, N, dtype=torch.long, device=device)
    for b, n in enumerate(lens):
        ids[b, N - n:] = seqs[b]
        mask[b, N - n:] = 1
        pos[b, N - n:] = torch.arange(n, device=device)
    with torch.no_grad():
        padded = model(input_ids=ids, attention_mask=mask, position_ids=pos, use_cache=False).logits.float()
        att_padded = captured[-1]
        for b, n in enumerate(lens):
            alone = model(input_ids=seqs[b][None], use_cache=False).logits.float()
            att_alone = captured[-1]
            a, r = att_padded[b, N - n:].flatten(), att_alone[0].flatten()
            cos = float(torch.nn.functional.cosine_similarity(a, r, dim=0))
            rel = float(torch.linalg.vector_norm(a - r) / torch.linalg.vector_norm(r))
            la, lr = padded[b, N - n:].flatten(), alone[0].flatten()
            lcos = float(torch.nn.functional.cosine_similarity(la, lr, dim=0))
            print(f"  row {b} (len {n}): layer-0 attention cos {cos:.6f} rel {rel:.3e}; logits cos {lcos:.5f}",
                  flush=True)
            assert cos > 0.999 and rel < 0.05
            assert lcos > 0.99
            if N - n:
                assert torch.count_nonzero(att_padded[b, :N - n]) == 0  # padding rows
