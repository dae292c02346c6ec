"""Host orchestration of the gfx950 GQA flash-attention path (the reference's public API).

Mirrors /root/reference/flash_attn/attention.py:
  * ``attention_flash_gqa``   inference forward, no LSE (reference 540-604)
  * ``FlashAttnGQAFunction``  autograd function: forward stores LSE, backward runs the
                              dQ kernel (fused delta) then the pack-GQA dKV kernel (1433-1622)
  * ``flash_attn_gqa_train``  training entry point (1625-1635)

(The reference's torch helper ``attention`` (11-17) lives in reference.py with the other
PyTorch reference functions.)

Tensors are (B, H, N, D) with any (batch, head, row) strides and a unit-stride head dim;
query head h uses KV head h // (Hq // Hkv). ``slide_size`` > 0 with ``causal`` limits query
i to keys in [i - slide_size + 1, i]; a window is ignored when not causal and a window
covering the whole sequence is plain causal (reference 1441-1443).

``segments`` (keyword, optional) is a pair of int32 (B, N) tables for variable-length,
padded or packed batches (segments.py builds them from padding masks, lengths, cu_seqlens or
position ids): token t attends, and is attended by, only keys [lo[b, t], hi[b, t]) on top of
the causal / window rule; padding tokens (empty segments) get zero outputs and gradients.
The reference has no such input (README.md:255-262 lists varlen and padding as unsupported).

Every call goes through libgfa.so's C ABI on the caller's current HIP stream. There is no
CPU or PyTorch fallback: unsupported inputs raise before anything is launched.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from . import segments as _seglib
from .registry import lookup

_DTYPES = {torch.float16: _lib.GFA_DTYPE_FP16, torch.bfloat16: _lib.GFA_DTYPE_BF16}


# One (batch, head) slice, plus the rows a tile copy may address past its end, must span at
# most 4 GiB: the kernels address tiles through 32-bit buffer offsets (gfa_api.hip,
# check_span).
_SLICE_LIMIT = 0xFFFFFFFF
_TILE_OVERRUN = 128


def _layout_ok(t: torch.Tensor) -> bool:
    """Strides the ABI can use: unit head-dim stride, other strides non-negative multiples
    of 8 elements, and one (batch, head) slice within the 4 GiB buffer range."""
    s = t.stride()
    return (s[3] == 1 and all(x % 8 == 0 and x >= 0 for x in s[:3])
            and ((t.shape[2] - 1 + _TILE_OVERRUN) * s[2] + t.shape[3]) * t.element_size() <= _SLICE_LIMIT)


def _needs_copy(t: torch.Tensor) -> bool:
    return not _layout_ok(t) or t.data_ptr() % 16 != 0


def _prep(t: torch.Tensor) -> torch.Tensor:
    """Rows must be 16-byte aligned with a unit-stride head dim; copy otherwise."""
    return t.contiguous() if _needs_copy(t) else t


def _check_inputs(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be 4-D (B, H, N, D)")
    B, Hq, N, D = q.shape
    if k.shape != v.shape or k.shape[0] != B or k.shape[2] != N or k.shape[3] != D:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    Hkv = k.shape[1]
    if Hkv == 0 or Hq % Hkv != 0:
        raise ValueError(f"N_Q_HEADS={Hq} must be a multiple of N_KV_HEADS={Hkv}")
    if q.dtype not in _DTYPES:
        raise TypeError(f"dtype {q.dtype} not supported (fp16 / bf16)")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("q, k, v must share one dtype")
    lookup(D)
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("q, k, v must be GPU tensors (the engine has no CPU path)")
    if k.device != q.device or v.device != q.device:
        raise ValueError("q, k, v must be on the same device")
    if N == 0 or B == 0:
        raise ValueError("empty sequence or batch")


def _check_segments(segments, q: torch.Tensor):
    """(lo, hi) int32 tables of shape (B, N) on q's device, made contiguous; None passes.
    Tables that segments.py did not build are checked to partition each row into segments and
    padding (segments.validate; one device-to-host read, skipped under torch.compile): the
    kernels read a block's range from its first and last token's bounds, so a malformed table
    would give wrong results without an error."""
    if segments is None:
        return None
    if len(segments) != 2:
        raise ValueError("segments must be a pair (lo, hi) of (B, N) int32 tensors")
    B, _, N, _ = q.shape
    out = []
    for t in segments:
        if not isinstance(t, torch.Tensor) or tuple(t.shape) != (B, N):
            raise ValueError(f"segment tables must be (B, N) = {(B, N)} tensors")
        if t.device != q.device:
            raise ValueError("segment tables must be on q's device")
        out.append(t.to(torch.int32).contiguous())
    if not isinstance(segments, _seglib.SegmentTables) and _seglib._host_checks():
        _seglib.validate(out[0], out[1])
    return tuple(out)


def _norm_window(causal: bool, slide_size: int, n: int) -> int:
    """attention.py:1441-1443: a window covering the whole sequence is plain causal.
    The library ignores the window when not causal (reference kernel 289-293)."""
    if slide_size is None:
        slide_size = 0
    slide_size = int(slide_size)
    if slide_size < 0:
        raise ValueError("slide_size must be >= 0")
    if slide_size > 0 and slide_size >= n:
        slide_size = 0
    return slide_size


def lse_ld(n: int) -> int:
    """Row length of the LSE / delta buffers: the backward reads whole query tiles of up
    to 64 rows (GFA_LSE_LD in include/gfa.h)."""
    return (n + 63) // 64 * 64


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _check_softcap(softcap) -> float:
    """0.0 for no soft-capping; otherwise a finite positive float (transformers' ``softcap``)."""
    if softcap is None:
        return 0.0
    c = float(softcap)
    if not math.isfinite(c) or c < 0.0:
        raise ValueError(f"softcap={softcap} must be finite and positive (None or 0 = off)")
    return c


def _check_dropout(p) -> float:
    """Attention dropout probability in [0, 1) (0 = off)."""
    c = float(p or 0.0)
    if not math.isfinite(c) or c < 0.0 or c >= 1.0:
        raise ValueError(f"dropout_p={p} must be in [0, 1)")
    return c


def _check_cap_and_dropout(softcap: float, dropout_p: float) -> None:
    """Soft-capping and dropout each run natively, but no kernel instance combines them: raise
    NotImplementedError (the adapter contract's error for unsupported features, reference
    hf_integration.py:60-63) before anything is launched."""
    if softcap > 0.0 and dropout_p > 0.0:
        raise NotImplementedError("softcap together with dropout_p > 0 is not built (each is supported alone)")


def _dropout_seed() -> int:
    """A fresh 63-bit mask seed from torch's default (CPU) generator: reproducible under
    torch.manual_seed, and the same value is handed to the backward."""
    return int(torch.randint(0, 2 ** 63 - 1, (1,)).item())


def _forward(q, k, v, causal: bool, slide_size: int, scale: float, store_lse: bool, block_kv: int = 0,
             segments=None, softcap: float = 0.0, dropout_p: float = 0.0, dropout_seed: int = 0):
    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    q, k, v = _prep(q), _prep(k), _prep(v)
    o = torch.empty_like(q)
    if _needs_copy(o):
        o = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    ld = lse_ld(N)
    lse = torch.empty((B, Hq, ld), dtype=torch.float32, device=q.device) if store_lse else None
    a = _lib.FwdArgs()
    a.q, a.k, a.v, a.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
    a.lse = lse.data_ptr() if lse is not None else None
    a.q_strides, a.k_strides, a.v_strides, a.o_strides = (_lib.strides_of(t) for t in (q, k, v, o))
    a.batch, a.heads_q, a.heads_kv, a.seq_len, a.head_dim = B, Hq, Hkv, N, D
    a.causal = int(bool(causal))
    a.window = int(slide_size)
    a.scale = float(scale)
    a.dtype = _DTYPES[q.dtype]
    a.block_kv = int(block_kv)
    a.lse_ld = ld
    a.softcap = float(softcap)
    a.dropout_p, a.dropout_seed = float(dropout_p), int(dropout_seed)
    a.stream = _stream(q.device)
    if segments is not None:
        a.seg_lo, a.seg_hi = segments[0].data_ptr(), segments[1].data_ptr()
    with torch.cuda.device(q.device):
        _lib.check(_lib.load().gfa_fwd(ctypes.byref(a)))
    return o, lse  # lse is (B, Hq, lse_ld(N)); rows >= N are padding


def _backward(q, k, v, o, lse, do, causal: bool, slide_size: int, scale: float, q_splits: int = 0,
              stages: int = 0, out=None, noalloc: bool = False, segments=None, softcap: float = 0.0,
              dropout_p: float = 0.0, dropout_seed: int = 0):
    """Run gfa_bwd. ``stages`` selects kernels (0 = all; GFA_BWD_DQ / GFA_BWD_DKV bits);
    ``out`` = (dq, dk, dv, delta) reuses caller buffers (profiling a single stage), and a fifth
    entry, a uint8 tensor, is the workspace (for the materialised form a GFA_BWD_DQ call reads the
    dS store a GFA_BWD_DKV call left there; it must hold gfa_bwd_workspace_bytes).
    ``noalloc`` calls gfa_bwd_noalloc instead: delta and the workspace then live in the
    library's own scratch (the returned delta is None)."""
    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    do = _prep(do)
    if do.dtype != q.dtype:
        do = do.to(q.dtype)
    ws = None
    if out is not None:
        dq, dk, dv, delta = out[:4]
        if len(out) > 4:
            ws = out[4]
    else:
        dq = torch.empty_like(q)
        dk = torch.empty_like(k)
        dv = torch.empty_like(v)
        dq, dk, dv = (t if not _needs_copy(t) else torch.empty(t.shape, dtype=t.dtype, device=t.device)
                      for t in (dq, dk, dv))
        delta = None if noalloc else torch.empty((B, Hq, lse_ld(N)), dtype=torch.float32, device=q.device)
    lib = _lib.load()
    a = _lib.BwdArgs()
    a.q, a.k, a.v, a.o, a.dout = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr()
    a.lse, a.delta = lse.data_ptr(), (delta.data_ptr() if delta is not None else None)
    a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    (a.q_strides, a.k_strides, a.v_strides, a.o_strides, a.do_strides, a.dq_strides, a.dk_strides,
     a.dv_strides) = (_lib.strides_of(t) for t in (q, k, v, o, do, dq, dk, dv))
    a.batch, a.heads_q, a.heads_kv, a.seq_len, a.head_dim = B, Hq, Hkv, N, D
    a.causal = int(bool(causal))
    a.window = int(slide_size)
    a.scale = float(scale)
    a.dtype = _DTYPES[q.dtype]
    a.q_splits = int(q_splits)
    a.lse_ld = lse.shape[-1]
    a.stages = int(stages)
    a.softcap = float(softcap)
    a.dropout_p, a.dropout_seed = float(dropout_p), int(dropout_seed)
    a.stream = _stream(q.device)
    if segments is not None:
        a.seg_lo, a.seg_hi = segments[0].data_ptr(), segments[1].data_ptr()
    if not noalloc:
        need = int(lib.gfa_bwd_workspace_bytes(ctypes.byref(a)))
        if ws is None or ws.numel() < need:
            ws = torch.empty(need, dtype=torch.uint8, device=q.device) if need else None
        a.workspace = ws.data_ptr() if ws is not None else None
        a.workspace_bytes = ws.numel() if ws is not None else 0
    with torch.cuda.device(q.device):
        _lib.check((lib.gfa_bwd_noalloc if noalloc else lib.gfa_bwd)(ctypes.byref(a)))
    return dq, dk, dv, delta


def backward_workspace(B: int, Hq: int, Hkv: int, N: int, D: int, causal: bool, slide_size: int, dtype=None,
                       q_splits: int = 0, segments: bool = False, softcap: float = 0.0, dropout_p: float = 0.0):
    """(bytes, materialised): the workspace gfa_bwd takes for this problem (gfa_bwd_workspace_bytes)
    and whether it then runs the materialised backward (a delta kernel, dK/dV storing dS, dQ from
    the store) rather than the recomputing one."""
    lib = _lib.load()
    a = _lib.BwdArgs()
    a.batch, a.heads_q, a.heads_kv, a.seq_len, a.head_dim = B, Hq, Hkv, N, D
    a.causal, a.window, a.q_splits = int(bool(causal)), int(slide_size), int(q_splits)
    a.dtype = _DTYPES[dtype if dtype is not None else torch.bfloat16]
    if segments:  # only the presence of a table matters for the size
        a.seg_lo = a.seg_hi = 16
    a.softcap, a.dropout_p = float(softcap), float(dropout_p)
    need = int(lib.gfa_bwd_workspace_bytes(ctypes.byref(a)))
    base = int(lib.gfa_bwd_workspace_size(B, Hq, Hkv, N, D, int(bool(causal)), int(slide_size), int(q_splits)))
    return need, need > base


def _default_scale(d: int, scale: float | None) -> float:
    return 1.0 / math.sqrt(d) if scale is None else float(scale)


class FlashAttnGQAFunction(torch.autograd.Function):
    """Autograd function of the GQA flash attention (reference attention.py:1433-1622).

    forward(q, k, v, causal, slide_size, scale=None, segments=None, softcap=None, dropout_p=0.0)
    -> O; saves q, k, v, O, the fp32 LSE (of the undropped probabilities), the segment tables and
    the dropout seed drawn for this call. backward(dO) -> dQ, dK, dV via gfa_bwd (the materialised
    form where it applies: delta, pack-GQA dKV storing dS, dQ from the store; else the dQ kernel
    with fused delta, then pack-GQA dKV), regenerating the same dropout mask from that seed.
    """

    @staticmethod
    def forward(ctx, q, k, v, causal=False, slide_size=0, scale=None, segments=None, softcap=None, dropout_p=0.0):
        _check_inputs(q, k, v)
        segments = _check_segments(segments, q)
        slide_size = _norm_window(causal, slide_size, q.shape[2])
        sc = _default_scale(q.shape[3], scale)
        cap = _check_softcap(softcap)
        dp = _check_dropout(dropout_p)
        _check_cap_and_dropout(cap, dp)
        seed = _dropout_seed() if dp > 0.0 else 0
        o, lse = _forward(q, k, v, causal, slide_size, sc, store_lse=True, segments=segments, softcap=cap,
                          dropout_p=dp, dropout_seed=seed)
        if segments is None:
            ctx.save_for_backward(q, k, v, o, lse)
        else:
            ctx.save_for_backward(q, k, v, o, lse, *segments)
        ctx.causal = bool(causal)
        ctx.slide_size = slide_size
        ctx.scale = sc
        ctx.softcap = cap
        ctx.dropout = (dp, seed)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse, *seg = ctx.saved_tensors
        q, k, v = _prep(q), _prep(k), _prep(v)
        dq, dk, dv, _ = _backward(q, k, v, o, lse, do, ctx.causal, ctx.slide_size, ctx.scale,
                                  segments=tuple(seg) if seg else None, softcap=ctx.softcap,
                                  dropout_p=ctx.dropout[0], dropout_seed=ctx.dropout[1])
        return dq, dk, dv, None, None, None, None, None, None


def flash_attn_gqa_train(q, k, v, causal=False, slide_size=0, *, scale=None, segments=None, softcap=None,
                         dropout_p=0.0):
    """Flash attention with autograd support (reference attention.py:1625-1635).

    q: (B, N_Q_HEADS, N, D); k, v: (B, N_KV_HEADS, N, D); fp16 or bf16; D in {64, 128, 256, 512}.
    ``scale`` defaults to 1/sqrt(D) like the reference; other values are used natively.
    ``segments``: optional (lo, hi) int32 (B, N) tables for ragged batches (segments.py).
    ``softcap``: optional logit soft-cap (scaled scores x -> softcap * tanh(x / softcap), as
    transformers' ``softcap``); not in the reference, whose adapter rejects it.
    ``dropout_p``: attention dropout on the softmax probabilities (kept ones scaled by
    1 / (1 - p)), with a fresh mask seed from torch's generator per call; not in the reference.
    """
    return FlashAttnGQAFunction.apply(q, k, v, causal, slide_size, scale, segments, softcap, dropout_p)


def attention_flash_gqa(q, k, v, causal=False, slide_size=0, BLOCK_Q=None, BLOCK_KV=None, BLOCK_D=None,
                        num_warps=None, num_stages=None, *, scale=None, segments=None, softcap=None):
    """Inference forward without LSE (reference attention.py:540-604). Default causal=False.

    ``BLOCK_KV`` selects one of the built LDS tile widths for this head dim. ``BLOCK_Q``,
    ``BLOCK_D``, ``num_warps`` and ``num_stages`` are Triton launch knobs of the reference;
    they are accepted for call compatibility and have no effect here (the gfx950 kernels
    always run 32-row waves or wave pairs with the registry's tiles).
    """
    _check_inputs(q, k, v)
    D = q.shape[3]
    cfg = lookup(D)
    bkv = 0
    if BLOCK_KV is not None:
        if int(BLOCK_KV) not in cfg.fwd_block_kv_options:
            raise ValueError(f"BLOCK_KV={BLOCK_KV} not built for head_dim={D}; options {cfg.fwd_block_kv_options}")
        bkv = int(BLOCK_KV)
    if BLOCK_D is not None and int(BLOCK_D) != D:
        raise ValueError("BLOCK_D must equal HEAD_DIM (no head-dim tiling)")
    slide_size = _norm_window(causal, slide_size, q.shape[2])
    o, _ = _forward(q, k, v, causal, slide_size, _default_scale(D, scale), store_lse=False, block_kv=bkv,
                    segments=_check_segments(segments, q), softcap=_check_softcap(softcap))
    return o

