"""torch.library registration of the engine: ``gfa::attn_fwd`` and ``gfa::attn_bwd``.

The reference's training entry point is an ``autograd.Function`` whose forward and backward
launch Triton kernels (/root/reference/flash_attn/attention.py:1433-1635). The same calls
here go through ctypes into libgfa.so, which ``torch.compile`` cannot trace, so a compiled
model would break its graph at every attention layer. Registered as custom ops (with
shape-only "fake" implementations and an autograd formula), the engine is one opaque node
in the graph: ``flash_attn_gqa_op`` under ``torch.compile(fullgraph=True)`` traces
without a break, and the captured graph can be replayed with HIP graphs. The kernels and
numerics are the ones ``flash_attn_gqa_train`` runs.

``attn_fwd(q, k, v, causal, window, scale, seg_lo=None, seg_hi=None, softcap=0.0,
dropout_p=0.0) -> (O, LSE, seed)``: ``window`` is already normalised (0 = none; only honoured
when causal), LSE is fp32 (B, Hq, lse_ld(N)) and not differentiable; ``seg_lo`` / ``seg_hi``
are the optional int32 (B, N) segment tables of a ragged batch. With ``dropout_p`` > 0 the op
draws the mask seed itself, from torch's default generator as the eager path does, and returns
it as a one-element int64 CPU tensor that the backward consumes (0 without dropout). Drawing it
inside the op keeps the host read of the seed out of traced code: a compiled model with
attention dropout keeps one graph, and eager and compiled runs draw the same seeds under the
same ``torch.manual_seed``.
``attn_bwd(q, k, v, O, LSE, dO, causal, window, scale, seg_lo=None, seg_hi=None, softcap=0.0,
dropout_p=0.0, seed=None) -> (dQ, dK, dV)``.
"""
from __future__ import annotations

from typing import Optional

import torch

from .attention import (_backward, _check_cap_and_dropout, _check_dropout, _check_inputs, _check_segments,
                        _check_softcap, _default_scale, _dropout_seed, _forward, _layout_ok, _norm_window, _prep,
                        lse_ld)


def _segs(seg_lo, seg_hi):
    return None if seg_lo is None else (seg_lo, seg_hi)


def _out_like(t: torch.Tensor) -> torch.Tensor:
    """Output buffer with t's layout, or contiguous when that layout breaks the ABI's rules
    (the same choice the eager path makes; fake tensors have no data pointer, and real
    allocations are always 16-byte aligned, so only the layout is checked)."""
    o = torch.empty_like(t)
    if not _layout_ok(o):
        o = torch.empty(t.shape, dtype=t.dtype, device=t.device)
    return o


def _seed_of(seed: Optional[torch.Tensor]) -> int:
    return 0 if seed is None else int(seed.reshape(-1)[0].item())  # a CPU tensor: no device sync


@torch.library.custom_op("gfa::attn_fwd", mutates_args=(), device_types="cuda")
def attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool, window: int,
             scale: float, seg_lo: Optional[torch.Tensor] = None,
             seg_hi: Optional[torch.Tensor] = None, softcap: float = 0.0,
             dropout_p: float = 0.0) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    seed = _dropout_seed() if dropout_p > 0.0 else 0
    o, lse = _forward(q, k, v, causal, window, scale, store_lse=True, segments=_segs(seg_lo, seg_hi),
                      softcap=softcap, dropout_p=dropout_p, dropout_seed=seed)
    return o, lse, torch.tensor([seed], dtype=torch.int64)


@attn_fwd.register_fake
def _attn_fwd_fake(q, k, v, causal, window, scale, seg_lo=None, seg_hi=None, softcap=0.0, dropout_p=0.0):
    B, Hq, N, _ = q.shape
    return (_out_like(q), q.new_empty((B, Hq, lse_ld(N)), dtype=torch.float32),
            torch.empty((1,), dtype=torch.int64, device="cpu"))


@torch.library.custom_op("gfa::attn_bwd", mutates_args=(), device_types="cuda")
def attn_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor, lse: torch.Tensor,
             do: torch.Tensor, causal: bool, window: int, scale: float, seg_lo: Optional[torch.Tensor] = None,
             seg_hi: Optional[torch.Tensor] = None, softcap: float = 0.0, dropout_p: float = 0.0,
             seed: Optional[torch.Tensor] = None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    dq, dk, dv, _ = _backward(_prep(q), _prep(k), _prep(v), o, lse, do, causal, window, scale,
                              segments=_segs(seg_lo, seg_hi), softcap=softcap, dropout_p=dropout_p,
                              dropout_seed=_seed_of(seed) if dropout_p > 0.0 else 0)
    return dq, dk, dv


@attn_bwd.register_fake
def _attn_bwd_fake(q, k, v, o, lse, do, causal, window, scale, seg_lo=None, seg_hi=None, softcap=0.0, dropout_p=0.0,
                   seed=None):
    return _out_like(q), _out_like(k), _out_like(v)


def _setup_context(ctx, inputs, output):
    q, k, v, causal, window, scale, seg_lo, seg_hi, softcap, dropout_p = inputs
    o, lse, seed = output
    ctx.save_for_backward(q, k, v, o, lse, seg_lo, seg_hi, seed)
    ctx.causal, ctx.window, ctx.scale, ctx.softcap, ctx.dropout_p = causal, window, scale, softcap, dropout_p
    ctx.mark_non_differentiable(lse, seed)


def _attn_fwd_backward(ctx, do, _dlse, _dseed):
    q, k, v, o, lse, seg_lo, seg_hi, seed = ctx.saved_tensors
    dq, dk, dv = attn_bwd(q, k, v, o, lse, do, ctx.causal, ctx.window, ctx.scale, seg_lo, seg_hi, ctx.softcap,
                          ctx.dropout_p, seed)
    return dq, dk, dv, None, None, None, None, None, None, None


attn_fwd.register_autograd(_attn_fwd_backward, setup_context=_setup_context)


def flash_attn_gqa_op(q, k, v, causal=False, slide_size=0, *, scale=None, segments=None, softcap=None, dropout_p=0.0):
    """``flash_attn_gqa_train`` through the registered op: same arguments, kernels and
    results, and traceable by ``torch.compile`` (no graph break at the attention call, with or
    without dropout or segment tables)."""
    _check_inputs(q, k, v)
    segments = _check_segments(segments, q)
    window = _norm_window(causal, slide_size, q.shape[2])
    seg_lo, seg_hi = segments if segments is not None else (None, None)
    cap = _check_softcap(softcap)
    dp = _check_dropout(dropout_p)
    _check_cap_and_dropout(cap, dp)
    o, _, _ = torch.ops.gfa.attn_fwd(q, k, v, bool(causal), int(window), _default_scale(q.shape[3], scale),
                                     seg_lo, seg_hi, cap, dp)
    return o
