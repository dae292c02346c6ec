"""Segment tables for variable-length and padded batches.

The kernels take an optional pair of int32 (B, N) tables (include/gfa.h, ``seg_lo`` /
``seg_hi``): token t of row b attends, and is attended by, only the tokens of keys
[lo[b, t], hi[b, t]), on top of the causal / sliding-window rule. Each row partitions
[0, N) into consecutive runs: a segment (its tokens all carry lo = its first token and
hi = one past its last) or padding (token t carries lo = hi = t, an empty segment: it takes
part in nothing, its output row is 0 and its gradient rows are 0).

The reference lists variable-length sequences and padding masks as unsupported
(/root/reference/README.md:255-262) and its HF adapter ignores ``attention_mask``
(flash_attn/hf_integration.py:43-47). These builders turn the usual descriptions of ragged
batches into tables:

  * ``from_padding_mask``  a (B, N) mask of real tokens (left or right padding);
  * ``from_lengths``       per-row real lengths, right or left padded;
  * ``from_cu_seqlens``    packed sequences: cumulative lengths over one row of N tokens;
  * ``from_position_ids``  packed sequences marked by position ids that restart.

All run on the input's device with tensor operations; ``from_padding_mask`` and
``from_cu_seqlens`` check their input and raise ``ValueError`` for shapes a table cannot
express (a padding mask whose real tokens are not one contiguous run). Those checks read
device values on the host; under ``torch.compile`` (which cannot trace such reads) they are
skipped and the input is taken as valid.

The builders return ``SegmentTables``, a (lo, hi) pair that the attention entry points take
as well-formed. A plain (lo, hi) tuple from elsewhere is checked there first
(``validate``).
"""
from __future__ import annotations

import torch


class SegmentTables(tuple):
    """(lo, hi): two int32 (B, N) tensors built by this module, so known to partition each
    row into segments and padding."""

    def __new__(cls, lo: torch.Tensor, hi: torch.Tensor):
        return super().__new__(cls, (lo, hi))


Segments = SegmentTables


def _host_checks() -> bool:
    """Whether checks that read device values on the host may run (not while torch.compile
    traces: a data-dependent read would break its graph)."""
    return not torch.compiler.is_compiling()


def validate(lo: torch.Tensor, hi: torch.Tensor) -> None:
    """Raise ValueError unless (lo, hi) partition every row of [0, N) into consecutive runs:
    each token is padding (lo = hi = t) or a member of [lo, hi) with 0 <= lo and hi <= N; a
    member either continues the previous token's segment (same lo and hi, t < hi[t - 1]) or
    starts a new one (lo = t). The kernels trim their tile ranges from the bounds of a block's
    first and last token, which is exact only for such tables; anything else would give wrong
    results silently. One device-to-host read."""
    if lo.dim() != 2 or lo.shape != hi.shape:
        raise ValueError("segment tables must be two (B, N) tensors of one shape")
    lo = lo.to(torch.int64)
    hi = hi.to(torch.int64)
    B, N = lo.shape
    if N == 0:
        return
    t = torch.arange(N, device=lo.device)[None, :]
    pad = (lo == t) & (hi == t)
    mem = (lo <= t) & (t < hi) & (lo >= 0) & (hi <= N)
    prev_lo = torch.cat([torch.full_like(lo[:, :1], -1), lo[:, :-1]], dim=1)
    prev_hi = torch.cat([torch.zeros_like(hi[:, :1]), hi[:, :-1]], dim=1)
    prev_mem = torch.cat([torch.zeros_like(mem[:, :1]), mem[:, :-1]], dim=1)
    inside = prev_mem & (t < prev_hi)  # t lies in the previous token's segment
    ok = (pad | mem) & torch.where(inside, mem & (lo == prev_lo) & (hi == prev_hi), ~mem | (lo == t))
    if not bool(ok.all()):
        b, j = (int(x) for x in (~ok).nonzero()[0])
        raise ValueError(f"segment tables do not partition each row into segments and padding "
                         f"(row {b}, token {j}: lo={int(lo[b, j])}, hi={int(hi[b, j])})")


def from_padding_mask(mask: torch.Tensor) -> Segments:
    """(B, N) mask of real tokens (nonzero / True) -> segment tables. The real tokens of a
    row must be one contiguous run (left padding, right padding or none); padding tokens get
    empty segments."""
    if mask.dim() != 2:
        raise ValueError(f"padding mask must be (B, N), got {tuple(mask.shape)}")
    m = mask.to(torch.bool)
    B, N = m.shape
    idx = torch.arange(N, device=m.device)
    mi = m.to(torch.int32)
    has = m.any(dim=1)
    start = torch.where(has, torch.argmax(mi, dim=1), torch.zeros_like(has, dtype=torch.long))
    end = torch.where(has, N - torch.argmax(mi.flip(1), dim=1), torch.zeros_like(has, dtype=torch.long))
    if _host_checks() and not bool((mi.sum(dim=1) == (end - start)).all()):
        raise ValueError("padding mask rows must hold one contiguous run of real tokens (left or right padding)")
    lo = torch.where(m, start[:, None], idx[None, :]).to(torch.int32).contiguous()
    hi = torch.where(m, end[:, None], idx[None, :]).to(torch.int32).contiguous()
    return SegmentTables(lo, hi)


def from_lengths(lengths, seq_len: int, left_padding: bool = False, device=None) -> Segments:
    """Per-row real lengths (right padding by default) -> segment tables."""
    lengths = torch.as_tensor(lengths, device=device).to(torch.long)
    idx = torch.arange(seq_len, device=lengths.device)
    if left_padding:
        mask = idx[None, :] >= (seq_len - lengths)[:, None]
    else:
        mask = idx[None, :] < lengths[:, None]
    return from_padding_mask(mask)


def from_cu_seqlens(cu_seqlens, seq_len: int, device=None) -> Segments:
    """Packed sequences in one row of ``seq_len`` tokens: sequence s holds tokens
    [cu_seqlens[s], cu_seqlens[s + 1]); tokens from cu_seqlens[-1] on are padding.
    Returns (1, seq_len) tables. ``[0]`` (no sequence) makes every token padding."""
    cu = torch.as_tensor(cu_seqlens, device=device).to(torch.long).flatten()
    if cu.numel() < 1:
        raise ValueError("cu_seqlens must start at 0, be non-decreasing and end at or before seq_len")
    if _host_checks() and (int(cu[0]) != 0 or bool((cu[1:] < cu[:-1]).any()) or int(cu[-1]) > seq_len):
        raise ValueError("cu_seqlens must start at 0, be non-decreasing and end at or before seq_len")
    idx = torch.arange(seq_len, device=cu.device)
    if cu.numel() == 1:  # no sequence: all padding (indexing cu[seg + 1] below needs two entries)
        lo = hi = idx.to(torch.int32)[None].contiguous()
        return SegmentTables(lo, hi.clone())
    seg = torch.searchsorted(cu[1:], idx, right=True)  # sequence of each token (== S for padding)
    real = idx < cu[-1]
    segc = seg.clamp(max=cu.numel() - 2)
    lo = torch.where(real, cu[segc], idx)
    hi = torch.where(real, cu[segc + 1], idx)
    return SegmentTables(lo.to(torch.int32)[None].contiguous(), hi.to(torch.int32)[None].contiguous())


def from_position_ids(position_ids: torch.Tensor) -> Segments:
    """Packed sequences marked by position ids (B, N): a new sequence starts wherever the
    position id is not the previous one plus one (the rule transformers uses to detect
    packed batches, masking_utils.find_packed_sequence_indices)."""
    pos = position_ids.to(torch.long)
    if pos.dim() == 1:
        pos = pos[None]
    B, N = pos.shape
    idx = torch.arange(N, device=pos.device).expand(B, N)
    start = torch.ones_like(pos, dtype=torch.bool)
    start[:, 1:] = pos[:, 1:] != pos[:, :-1] + 1
    lo = torch.where(start, idx, torch.zeros_like(idx)).cummax(dim=1).values
    nxt = torch.where(start, idx, torch.full_like(idx, N))
    nxt = torch.cat([nxt[:, 1:], torch.full_like(nxt[:, :1], N)], dim=1)
    hi = nxt.flip(1).cummin(dim=1).values.flip(1)
    return SegmentTables(lo.to(torch.int32).contiguous(), hi.to(torch.int32).contiguous())


def is_packed(position_ids: torch.Tensor) -> bool:
    """True when position ids restart inside a row (several sequences packed per row)."""
    pos = position_ids.to(torch.long)
    if pos.dim() == 1:
        pos = pos[None]
    return bool((pos[:, 1:] != pos[:, :-1] + 1).any())
