"""Ragged batches on the CPU: the segment-table builders (segments.py) and the oracle's
segment semantics, pinned two independent ways.

* torch scaled_dot_product_attention (math backend, float64) with the equivalent boolean
  mask, on every query row that sees at least one key; rows that see none must come out
  as O = 0 and LSE = -inf;
* the segment-free oracle (already pinned by test_oracle.py) run on every segment alone:
  a padded or packed batch must give, on each segment's tokens, exactly the outputs and
  gradients of that segment computed by itself, and zero gradients on padding tokens. A
  wrong segment bound, an off-by-one at a run edge, or a leak between packed sequences
  fails here.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

import gemma_triton_flash_attn_amd as gfa
from oracle import attention_oracle as orc

seg = gfa.segments


def _tables(runs, n):
    """Tables for one row from a list of (start, end, is_segment) runs covering [0, n)."""
    lo, hi = np.arange(n), np.arange(n)
    for a, b, real in runs:
        if real:
            lo[a:b], hi[a:b] = a, b
    return lo, hi


def test_from_padding_mask_left_right_and_none():
    m = torch.tensor([[1, 1, 1, 0, 0], [0, 0, 1, 1, 1], [1, 1, 1, 1, 1], [0, 0, 0, 0, 0]], dtype=torch.bool)
    lo, hi = seg.from_padding_mask(m)
    assert lo.dtype == torch.int32 and lo.is_contiguous()
    assert lo.tolist() == [[0, 0, 0, 3, 4], [0, 1, 2, 2, 2], [0, 0, 0, 0, 0], [0, 1, 2, 3, 4]]
    assert hi.tolist() == [[3, 3, 3, 3, 4], [0, 1, 5, 5, 5], [5, 5, 5, 5, 5], [0, 1, 2, 3, 4]]
    with pytest.raises(ValueError, match="contiguous"):
        seg.from_padding_mask(torch.tensor([[1, 0, 1]]))
    lo2, hi2 = seg.from_lengths([3, 5], 5)
    assert lo2.tolist()[0] == [0, 0, 0, 3, 4] and hi2.tolist()[1] == [5] * 5
    lo3, _ = seg.from_lengths([3], 5, left_padding=True)
    assert lo3.tolist() == [[0, 1, 2, 2, 2]]


def test_from_cu_seqlens_and_position_ids_agree():
    lo, hi = seg.from_cu_seqlens([0, 3, 7, 8], 10)
    assert lo.tolist() == [[0, 0, 0, 3, 3, 3, 3, 7, 8, 9]]
    assert hi.tolist() == [[3, 3, 3, 7, 7, 7, 7, 8, 8, 9]]
    pos = torch.tensor([[0, 1, 2, 0, 1, 2, 3, 0, 0, 0]])
    plo, phi = seg.from_position_ids(pos)
    # the trailing padding tokens of the cu_seqlens form are one-token sequences here
    assert plo.tolist()[0][:8] == lo.tolist()[0][:8] and phi.tolist()[0][:8] == hi.tolist()[0][:8]
    assert plo.tolist()[0][8:] == [8, 9] and phi.tolist()[0][8:] == [9, 10]
    assert seg.is_packed(pos) and not seg.is_packed(torch.arange(6)[None])
    with pytest.raises(ValueError):
        seg.from_cu_seqlens([0, 5, 3], 10)
    with pytest.raises(ValueError):
        seg.from_cu_seqlens([0, 11], 10)


def test_from_cu_seqlens_without_sequences_is_all_padding():
    """cu_seqlens = [0] (no sequence): every token is padding, with no indexing past the
    one-element tensor (torch.where evaluates both of its branches)."""
    lo, hi = seg.from_cu_seqlens([0], 8)
    assert lo.tolist() == [list(range(8))] and hi.tolist() == [list(range(8))]
    with pytest.raises(ValueError):
        seg.from_cu_seqlens([], 8)
    seg.validate(lo, hi)


def test_builders_return_tables_that_validate():
    """Every builder's output is a SegmentTables (taken as well-formed by the entry points) and
    passes the partition check that user-supplied tables get."""
    m = torch.tensor([[1, 1, 1, 0, 0], [0, 0, 1, 1, 1], [1, 1, 1, 1, 1], [0, 0, 0, 0, 0]], dtype=torch.bool)
    built = [seg.from_padding_mask(m), seg.from_lengths([3, 5], 5), seg.from_cu_seqlens([0, 3, 7, 8], 10),
             seg.from_position_ids(torch.tensor([[0, 1, 2, 0, 1, 2, 3, 0, 0, 0]]))]
    for t in built:
        assert isinstance(t, seg.SegmentTables)
        seg.validate(*t)
    for name in ROWS:
        _, _, (lo, hi) = _build(name)
        seg.validate(torch.as_tensor(lo), torch.as_tensor(hi))


@pytest.mark.parametrize("lo,hi,why", [
    ([[0, 0, 2, 2]], [[2, 1, 4, 4]], "hi below the token"),
    ([[0, 0, 0, 0]], [[4, 4, 4, 5]], "hi past N"),
    ([[0, 0, 2, 3]], [[2, 2, 4, 4]], "a member that neither continues nor starts a segment"),
    ([[0, 0, 1, 1]], [[2, 2, 4, 4]], "a segment starting inside the previous one"),
    ([[0, 0, 0, 0]], [[3, 3, 4, 4]], "hi changing inside a segment"),
    ([[1, 1, 1, 1]], [[4, 4, 4, 4]], "a segment that starts before its first token"),
    ([[0, 0, 2, 0]], [[2, 2, 3, 4]], "lo decreasing"),
    ([[0, 5, 2, 3]], [[1, 5, 3, 4]], "a padding token with lo = hi away from itself"),
])
def test_malformed_user_tables_raise(lo, hi, why):
    """Tables that do not partition the row would make the kernels' tile-range trimming (from a
    block's first and last token) wrong without an error; they are rejected before any launch."""
    lo, hi = torch.tensor(lo, dtype=torch.int32), torch.tensor(hi, dtype=torch.int32)
    with pytest.raises(ValueError, match="partition"):
        seg.validate(lo, hi)
    from gemma_triton_flash_attn_amd.attention import _check_segments

    q = torch.empty(1, 2, lo.shape[1], 64)
    with pytest.raises(ValueError, match="partition"):
        _check_segments((lo, hi), q)
    # the same tensors wrapped as builder output are trusted (no device read)
    assert _check_segments(seg.SegmentTables(lo, hi), q) is not None


ROWS = {
    # name: N, list of per-row runs (start, end, is_segment)
    "right_left_full_empty": (13, [[(0, 9, True), (9, 10, False), (10, 11, False), (11, 12, False), (12, 13, False)],
                                   [(0, 1, False), (1, 2, False), (2, 3, False), (3, 13, True)],
                                   [(0, 13, True)],
                                   [(t, t + 1, False) for t in range(13)]]),
    "packed": (16, [[(0, 5, True), (5, 6, True), (6, 13, True), (13, 14, False), (14, 15, False), (15, 16, False)]]),
}


def _build(name):
    n, rows = ROWS[name]
    lo, hi = zip(*(_tables(r, n) for r in rows))
    return n, rows, (np.stack(lo), np.stack(hi))


@pytest.mark.parametrize("name", list(ROWS))
@pytest.mark.parametrize("causal,window", [(True, 0), (True, 3), (False, 0)])
def test_oracle_segments_match_sdpa_with_mask(name, causal, window):
    n, rows, segs = _build(name)
    B, Hq, Hkv, D = len(rows), 4, 2, 8
    rng = np.random.default_rng(5)
    q, k, v = (rng.standard_normal(s) for s in [(B, Hq, n, D), (B, Hkv, n, D), (B, Hkv, n, D)])
    o, lse = orc.forward(q, k, v, causal, window, segments=segs)
    i, j = np.arange(n)[:, None], np.arange(n)[None, :]
    for b in range(B):
        m = np.ones((n, n), bool)
        if causal:
            m &= j <= i
            if window:
                m &= (i - j) < window
        m &= (j >= segs[0][b][:, None]) & (j < segs[1][b][:, None])
        seen = m.any(1)
        qt = torch.tensor(q[b][None])
        ke = torch.tensor(np.repeat(k[b], Hq // Hkv, 0)[None])
        ve = torch.tensor(np.repeat(v[b], Hq // Hkv, 0)[None])
        with sdpa_kernel(SDPBackend.MATH):
            ref = F.scaled_dot_product_attention(qt, ke, ve, attn_mask=torch.tensor(m))[0].numpy()
        if seen.any():
            assert np.abs(o[b][:, seen] - ref[:, seen]).max() < 1e-12
        assert (o[b][:, ~seen] == 0).all() and np.isneginf(lse[b][:, ~seen]).all()
        assert np.isfinite(lse[b][:, seen]).all()


@pytest.mark.parametrize("name", list(ROWS))
@pytest.mark.parametrize("causal,window", [(True, 0), (True, 4), (False, 0)])
def test_oracle_segments_equal_each_segment_alone(name, causal, window):
    n, rows, segs = _build(name)
    B, Hq, Hkv, D = len(rows), 4, 2, 8
    rng = np.random.default_rng(6)
    q, k, v, do = (rng.standard_normal(s) for s in [(B, Hq, n, D), (B, Hkv, n, D), (B, Hkv, n, D), (B, Hq, n, D)])
    o, lse = orc.forward(q, k, v, causal, window, segments=segs)
    dq, dk, dv, _ = orc.backward(q, k, v, do, causal, window, segments=segs)
    for b, runs in enumerate(rows):
        for a, e, real in runs:
            if not real:
                assert (dq[b][:, a:e] == 0).all() and (dk[b][:, a:e] == 0).all() and (dv[b][:, a:e] == 0).all()
                continue
            sl = slice(a, e)
            w = window if window < e - a else 0
            o1, l1 = orc.forward(q[b:b + 1, :, sl], k[b:b + 1, :, sl], v[b:b + 1, :, sl], causal, w)
            g1 = orc.backward(q[b:b + 1, :, sl], k[b:b + 1, :, sl], v[b:b + 1, :, sl], do[b:b + 1, :, sl], causal, w)
            assert np.abs(o[b:b + 1, :, sl] - o1).max() < 1e-12
            assert np.abs(lse[b:b + 1, :, sl] - l1).max() < 1e-12
            for got, ref in zip((dq, dk, dv), g1[:3]):
                assert np.abs(got[b:b + 1, :, sl] - ref).max() < 1e-11


def test_chunked_oracle_with_segments_matches_dense():
    n, rows, segs = _build("right_left_full_empty")
    B, Hq, Hkv, D = len(rows), 4, 1, 16
    g = torch.Generator().manual_seed(8)
    q, k, v, do = (torch.randn(s, generator=g) for s in [(B, Hq, n, D), (B, Hkv, n, D), (B, Hkv, n, D), (B, Hq, n, D)])
    tseg = tuple(torch.tensor(x) for x in segs)
    o, lse = orc.forward_chunked(q, k, v, True, 5, chunk=4, segments=tseg)
    dq, dk, dv, _ = orc.backward_chunked(q, k, v, do, True, 5, chunk=4, segments=tseg)
    o2, lse2 = orc.forward(q.numpy(), k.numpy(), v.numpy(), True, 5, segments=segs)
    g2 = orc.backward(q.numpy(), k.numpy(), v.numpy(), do.numpy(), True, 5, segments=segs)
    assert np.abs(o.numpy() - o2).max() < 1e-5
    fin = np.isfinite(lse2)
    assert np.abs(lse.numpy()[fin] - lse2[fin]).max() < 1e-5 and np.isneginf(lse.numpy()[~fin]).all()
    for a, b in zip((dq, dk, dv), g2[:3]):
        assert np.abs(a.numpy() - b).max() < 1e-4
