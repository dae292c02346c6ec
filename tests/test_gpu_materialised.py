"""The materialised backward (include/gfa.h: a delta kernel, dK/dV storing every 32 x 32 block of
dS it computes, then dQ = scale * dS K from that store) against the recomputing one on the same
inputs, and its host-side contract: the stage split through a persistent workspace, the store
size limit, and soft-capping and dropout in the materialised form. Both forms compute the same
quantities with the same roundings of P and dS to the input dtype, so they agree to accumulation
order (a few 1e-4 relative); the oracle comparisons of the other GPU tests run the default form,
which is the materialised one wherever it applies.
"""
from __future__ import annotations

import pytest
import torch

from conftest import make_inputs, recomputing

pytestmark = pytest.mark.gpu

FORM_TOL = 2e-3  # relative, materialised against recomputing (measured: 1e-5 .. 2e-4)

CASES = {
    # name: B, Hq, Hkv, N, D, causal, window, dtype, q_splits
    "d512_causal_gqa8": (1, 16, 2, 2048, 512, True, 0, torch.bfloat16, 0),
    "d512_causal_ragged": (1, 8, 2, 3001, 512, True, 0, torch.bfloat16, 0),
    "d512_noncausal_b2": (2, 8, 2, 700, 512, False, 0, torch.bfloat16, 0),
    "d512_causal_fp16": (1, 8, 1, 1024, 512, True, 0, torch.float16, 0),
    "d512_qsplit4": (1, 8, 1, 2048, 512, True, 0, torch.bfloat16, 4),
    "d512_tiny": (1, 4, 1, 33, 512, True, 0, torch.bfloat16, 0),
    "d512_swa700_ragged": (1, 8, 2, 2500, 512, True, 700, torch.bfloat16, 0),
    "d512_swa100_fp16_b2": (2, 4, 1, 1100, 512, True, 100, torch.float16, 0),
    "d256_swa1024": (1, 16, 8, 4096, 256, True, 1024, torch.bfloat16, 0),
    "d256_swa700_ragged": (1, 16, 4, 3000, 256, True, 700, torch.bfloat16, 0),
    "d256_swa31": (2, 8, 2, 517, 256, True, 31, torch.bfloat16, 0),
    "d256_swa512_fp16": (1, 8, 1, 1500, 256, True, 512, torch.float16, 0),
    # D=256 without a window: the one-wave dK/dV form (128-key workgroups) stores
    "d256_causal_gqa2": (1, 16, 8, 2048, 256, True, 0, torch.bfloat16, 0),
    "d256_causal_ragged": (1, 8, 2, 3001, 256, True, 0, torch.bfloat16, 0),
    "d256_noncausal_b2": (2, 8, 2, 700, 256, False, 0, torch.bfloat16, 0),
    "d256_causal_fp16": (1, 8, 1, 1100, 256, True, 0, torch.float16, 0),
    "d256_qsplit4": (1, 8, 1, 2048, 256, True, 0, torch.bfloat16, 4),
    "d256_tiny": (1, 4, 1, 33, 256, True, 0, torch.bfloat16, 0),
    "d256_window_ge_n": (1, 8, 2, 1000, 256, True, 1000, torch.bfloat16, 0),
}


def _rel(a, b):
    return float(torch.linalg.vector_norm(a.float() - b.float()) / torch.linalg.vector_norm(b.float()))


def _run(q, k, v, do, causal, window, q_splits, out=None, stages=0):
    from gemma_triton_flash_attn_amd.attention import _backward, _forward

    sc = q.shape[-1] ** -0.5
    o, lse = _forward(q, k, v, causal, window, sc, store_lse=True)
    res = _backward(q, k, v, o, lse, do, causal, window, sc, q_splits=q_splits, out=out, stages=stages)
    torch.cuda.synchronize()
    return res


FEATURE_CASES = {
    # name: B, Hq, Hkv, N, D, causal, window, dtype, softcap, dropout_p
    "d512_softcap30": (1, 8, 1, 1500, 512, True, 0, torch.bfloat16, 30.0, 0.0),
    "d512_dropout": (1, 8, 2, 1024, 512, True, 0, torch.bfloat16, 0.0, 0.1),
    "d512_swa700_softcap50_fp16": (1, 8, 2, 3000, 512, True, 700, torch.float16, 50.0, 0.0),
    "d512_swa512_dropout_b2": (2, 4, 1, 1500, 512, True, 512, torch.bfloat16, 0.0, 0.15),
    "d256_softcap30": (1, 8, 2, 1500, 256, True, 0, torch.bfloat16, 30.0, 0.0),
    "d256_swa700_softcap50_fp16": (1, 8, 2, 3000, 256, True, 700, torch.float16, 50.0, 0.0),
    "d256_noncausal_dropout": (2, 4, 1, 900, 256, False, 0, torch.bfloat16, 0.0, 0.1),
    "d256_swa100_dropout": (1, 8, 4, 1300, 256, True, 100, torch.bfloat16, 0.0, 0.15),
}


@pytest.mark.parametrize("name", list(FEATURE_CASES))
def test_materialised_softcap_dropout(name, device):
    """Soft-capping and dropout take the materialised form too (the dK/dV kernel's stored dS
    carries the soft-cap factor 1 - t^2 and the dropped dP; at D=256 their dK/dV instances are
    the one-wave form, with or without a window); against the recomputing form."""
    from gemma_triton_flash_attn_amd.attention import _backward, _forward, backward_workspace

    B, Hq, Hkv, N, D, causal, window, dtype, cap, dp = FEATURE_CASES[name]
    print(f"case {name}: B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} window={window} {dtype} softcap={cap} "
          f"dropout={dp}", flush=True)
    assert backward_workspace(B, Hq, Hkv, N, D, causal, window, dtype, softcap=cap, dropout_p=dp)[1]
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, dtype, device, seed=N + 7)
    sc = D ** -0.5
    kw = dict(softcap=cap, dropout_p=dp, dropout_seed=1234)
    o, lse = _forward(q, k, v, causal, window, sc, store_lse=True, **kw)

    def bwd():
        r = _backward(q, k, v, o, lse, do, causal, window, sc, **kw)
        torch.cuda.synchronize()
        return r

    mat = bwd()
    with recomputing():
        rec = bwd()
    for nm, a, b in zip(("dQ", "dK", "dV"), mat[:3], rec[:3]):
        assert torch.isfinite(a).all(), nm
        assert _rel(a, b) <= FORM_TOL, f"{nm}: {_rel(a, b):.3e}"


@pytest.mark.parametrize("name", list(CASES))
def test_materialised_matches_recomputing(name, device):
    from gemma_triton_flash_attn_amd.attention import backward_workspace

    B, Hq, Hkv, N, D, causal, window, dtype, qs = CASES[name]
    print(f"case {name}: B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal} window={window} {dtype} "
          f"q_splits={qs}", flush=True)
    assert backward_workspace(B, Hq, Hkv, N, D, causal, window, dtype, q_splits=qs)[1], "expected the materialised form"
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, dtype, device, seed=N + Hq)
    mat = _run(q, k, v, do, causal, window, qs)
    with recomputing():
        assert not backward_workspace(B, Hq, Hkv, N, D, causal, window, dtype, q_splits=qs)[1]
        rec = _run(q, k, v, do, causal, window, qs)
    for nm, a, b in zip(("dQ", "dK", "dV"), mat[:3], rec[:3]):
        assert torch.isfinite(a).all(), nm
        assert _rel(a, b) <= FORM_TOL, f"{nm}: {_rel(a, b):.3e}"
    # delta: the same row sums in another order
    assert float((mat[3][..., :N] - rec[3][..., :N]).abs().max()) <= 1e-3


SEG_CASES = {
    # name: B, Hq, Hkv, N, D, causal, window, dtype, table ("cu": cu_seqlens of one row, "len": the
    # rows' lengths, "left": the same left-padded), extra features
    "d512_packed": (1, 8, 2, 2000, 512, True, 0, torch.bfloat16, ("cu", [0, 300, 301, 1200, 1900]), {}),
    "d512_noncausal_lengths_b2": (2, 8, 2, 1100, 512, False, 0, torch.bfloat16, ("len", [1063, 550]), {}),
    "d512_left_padding_b2_fp16": (2, 4, 1, 900, 512, True, 0, torch.float16, ("left", [860, 897]), {}),
    "d512_swa300_packed_softcap": (1, 8, 1, 1500, 512, True, 300, torch.bfloat16,
                                   ("cu", [0, 700, 705, 1400]), {"softcap": 30.0}),
    "d512_padding_row_alone": (1, 4, 1, 993, 512, True, 0, torch.bfloat16, ("cu", [0, 500, 992]), {}),
    "d256_swa512_packed": (1, 16, 8, 3000, 256, True, 512, torch.bfloat16, ("cu", [0, 1000, 1001, 2500, 2999]), {}),
    "d256_causal_packed_full": (1, 8, 2, 2048, 256, True, 0, torch.bfloat16, ("cu", [0, 64, 700, 1500, 2048]), {}),
    "d256_noncausal_lengths_b2": (2, 8, 4, 777, 256, False, 0, torch.bfloat16, ("len", [777, 400]), {}),
    "d256_padding_row_alone_dropout": (1, 4, 2, 993, 256, True, 0, torch.bfloat16, ("cu", [0, 500, 992]),
                                       {"dropout_p": 0.1}),
}


@pytest.mark.parametrize("name", list(SEG_CASES))
def test_materialised_with_segments(name, device):
    """Segment tables (packed sequences, padding) in the materialised form: the dQ kernel reads
    only the blocks the segment-trimmed dK/dV iteration writes (ds_seg_units). Against the
    recomputing form; padding rows get dQ exactly 0 (their dS rows are 0)."""
    import gemma_triton_flash_attn_amd as gfa
    from gemma_triton_flash_attn_amd.attention import _backward, _forward, backward_workspace

    B, Hq, Hkv, N, D, causal, window, dtype, (kind, spec), kw = SEG_CASES[name]
    print(f"case {name}: B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal} window={window} {dtype} "
          f"{kind}={spec} {kw}", flush=True)
    if kind == "cu":
        segs = gfa.segments.from_cu_seqlens(spec, N, device=device)
    else:
        segs = gfa.segments.from_lengths(spec, N, left_padding=kind == "left", device=device)
    assert backward_workspace(B, Hq, Hkv, N, D, causal, window, dtype, segments=True, **kw)[1]
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, dtype, device, seed=N + 11)
    sc = D ** -0.5
    kw = dict(kw, dropout_seed=77) if kw.get("dropout_p") else kw
    o, lse = _forward(q, k, v, causal, window, sc, store_lse=True, segments=segs, **kw)

    def bwd():
        r = _backward(q, k, v, o, lse, do, causal, window, sc, segments=segs, **kw)
        torch.cuda.synchronize()
        return r

    mat = bwd()
    with recomputing():
        rec = bwd()
    for nm, a, b in zip(("dQ", "dK", "dV"), mat[:3], rec[:3]):
        assert torch.isfinite(a).all(), nm
        assert _rel(a, b) <= FORM_TOL, f"{nm}: {_rel(a, b):.3e}"
    lo, hi = segs
    pad = (lo == hi).to(device)  # (B, N): padding tokens (none in a fully packed row)
    if bool(pad.any()):
        dq_pad = mat[0].float().permute(0, 2, 1, 3)[pad]  # (padding tokens, Hq, D)
        assert float(dq_pad.abs().max()) == 0.0


def test_stage_split_through_the_workspace_is_bitwise(device):
    """GFA_BWD_DKV (delta and dK/dV, storing dS), then GFA_BWD_DQ reading the store the first call
    left in the same workspace, equals the one-call backward bit for bit."""
    from gemma_triton_flash_attn_amd import _lib
    from gemma_triton_flash_attn_amd.attention import backward_workspace

    B, Hq, Hkv, N, D = 1, 8, 2, 1500, 512
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=3)
    full = _run(q, k, v, do, True, 0, 0)
    nbytes, mat = backward_workspace(B, Hq, Hkv, N, D, True, 0)
    assert mat
    bufs = (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), torch.empty_like(full[3]),
            torch.empty(nbytes, dtype=torch.uint8, device=device))
    _run(q, k, v, do, True, 0, 0, out=bufs, stages=_lib.GFA_BWD_DKV)
    _run(q, k, v, do, True, 0, 0, out=bufs, stages=_lib.GFA_BWD_DQ)
    for nm, a, b in zip(("dQ", "dK", "dV"), bufs[:3], full[:3]):
        assert torch.equal(a, b), nm
    assert torch.equal(bufs[3][..., :N], full[3][..., :N])


def test_stage_split_with_segments_is_bitwise(device):
    """The stage split with a segment table (both calls take it): GFA_BWD_DKV then GFA_BWD_DQ
    through one workspace equals the one-call backward bit for bit."""
    import gemma_triton_flash_attn_amd as gfa
    from gemma_triton_flash_attn_amd import _lib
    from gemma_triton_flash_attn_amd.attention import _backward, _forward, backward_workspace

    B, Hq, Hkv, N, D = 1, 8, 2, 1300, 512
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=9)
    segs = gfa.segments.from_cu_seqlens([0, 400, 401, 1250], N, device=device)
    sc = D ** -0.5
    o, lse = _forward(q, k, v, True, 0, sc, store_lse=True, segments=segs)
    full = _backward(q, k, v, o, lse, do, True, 0, sc, segments=segs)
    nbytes, mat = backward_workspace(B, Hq, Hkv, N, D, True, 0, segments=True)
    assert mat
    bufs = (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), torch.empty_like(full[3]),
            torch.empty(nbytes, dtype=torch.uint8, device=device))
    _backward(q, k, v, o, lse, do, True, 0, sc, out=bufs, stages=_lib.GFA_BWD_DKV, segments=segs)
    _backward(q, k, v, o, lse, do, True, 0, sc, out=bufs, stages=_lib.GFA_BWD_DQ, segments=segs)
    torch.cuda.synchronize()
    for nm, a, b in zip(("dQ", "dK", "dV"), bufs[:3], full[:3]):
        assert torch.equal(a, b), nm


def test_store_limit_selects_the_form(device):
    """A store above the limit runs the recomputing form (bit for bit the limit-0 results); the
    limit restored, the materialised one again."""
    from gemma_triton_flash_attn_amd import _lib
    from gemma_triton_flash_attn_amd.attention import backward_workspace

    B, Hq, Hkv, N, D = 1, 8, 1, 1024, 512
    nbytes, mat = backward_workspace(B, Hq, Hkv, N, D, True, 0)
    assert mat and nbytes > 0
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=5)
    with recomputing():
        rec = _run(q, k, v, do, True, 0, 0)
    store = nbytes - (_lib.bwd_workspace_size(B, Hq, Hkv, N, D, True, 0) + 255) // 256 * 256  # past the partials
    prev = _lib.set_bwd_ds_limit(store - 1)
    try:
        assert not backward_workspace(B, Hq, Hkv, N, D, True, 0)[1]
        small = _run(q, k, v, do, True, 0, 0)
    finally:
        _lib.set_bwd_ds_limit(prev)
    for a, b in zip(small[:3], rec[:3]):
        assert torch.equal(a, b)
    mat_out = _run(q, k, v, do, True, 0, 0)
    assert not torch.equal(mat_out[0], rec[0])  # the other form ran (dQ accumulates in another order)
    assert _rel(mat_out[0], rec[0]) <= FORM_TOL
