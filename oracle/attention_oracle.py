"""CPU restatement of the reference's attention math: the parity oracle.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker. No engine code path
calls it; the engine has no CPU path.

What it restates (all paths under /root/reference, zzhhjjj/gemma-triton-flash-attn):
  * op and masks: flash_attn/attention.py:611-619 (attention_gqa_ref: GQA by
    repeat_interleave, scale 1/sqrt(D)), 622-642 (attention_swa_ref: key j visible to
    query i iff j <= i and i - j < slide_size), 347-355 (kernel mask; the window only
    applies when causal), 1441-1443 (window >= N is plain causal), 272 (query head h
    reads KV head h * Hkv // Hq);
  * forward outputs: 377 (O = acc / l), 382-388 (LSE in natural log);
  * backward: 733-744 (delta = rowsum(dO * O) in fp32), 785-793 (P = exp(S - LSE),
    dS = P * (dP - delta), dQ = scale * dS K), 1192-1202 (dV = P^T dO, dK = scale * dS^T Q,
    summed over the query heads of a KV group).

Variable-length / padded batches (the build's segment tables, include/gfa.h; the reference
lists varlen and padding masks as unsupported, README.md:255-262, and its HF adapter ignores
the mask, hf_integration.py:43-47): ``segments = (lo, hi)``, two (B, N) integer arrays; key
j is visible to query i of row b only if lo[b, i] <= j < hi[b, i], on top of the causal /
window rule. A query row with no visible key has O = 0 and LSE = -inf, and contributes no
gradient. Pinned by tests/test_oracle.py against torch SDPA with the equivalent boolean
mask (rows with a visible key) and against the segment-free oracle run on every segment
alone (padded and packed batches).

Logit soft-capping (``softcap`` > 0; the reference lists it as unsupported, README.md:255-262,
and its HF adapter raises for it, hf_integration.py:60-63): the scaled score z = scale q.k is
replaced by softcap * tanh(z / softcap) before the mask and the softmax, as transformers'
eager attention does (models/gemma2/modeling_gemma2.py, eager_attention_forward). In the
backward, dS is multiplied by the derivative 1 - tanh^2(z / softcap) before dQ and dK.
Pinned by tests/test_oracle.py against that transformers function (forward) and torch
autograd through it in float64 (backward).

Attention dropout (``dropout`` = (p, seed), p in (0, 1); also unsupported by the reference,
README.md:255-262, hf_integration.py:60-63): P_ij is kept with probability 1 - p and scaled by
1 / (1 - p), else zeroed, after the softmax (transformers' eager attention applies
nn.functional.dropout to the probabilities). The LSE is that of the undropped P; the backward
uses dS = P (M dP / (1 - p) - delta) with delta = rowsum(dO O). The mask M is the engine's
counter-based one (``dropout_mask``: a 32-bit xor-shift / multiply mixer of (seed, query head,
query row, key), restated from csrc/gfa_common.h, drop_row / drop_keep), so that the kernels'
results can be compared element for element. Pinned by tests/test_oracle.py against float64
torch autograd through softmax(S) * M / (1 - p) @ V with the same mask, and by the mask's
keep rate.

Two implementations of the same equations:
  * ``forward`` / ``backward``: numpy float64, dense (N x N per head) - small cases and
    golden vectors;
  * ``forward_chunked`` / ``backward_chunked``: torch float32 on any device, query-chunked
    so N = 32K fits - the large-shape check on the GPU box (a torch fp32 reference of the
    same op, never the engine). They take segments, soft-capping and dropout as well (the
    mask rows of a chunk from ``dropout_mask_rows``), and are pinned to the dense path with
    each of them.

Pinned by tests/test_oracle.py against: torch's scaled_dot_product_attention (math
backend, float64) and its autograd for forward/backward, the committed golden vectors in
tests/golden (written by that independent library path), finite differences, and
closed forms (Q = 0 gives prefix / window means and LSE = ln |allowed|; window 1 gives
O = V; GQA equals MHA on repeated K/V; shift invariance in K; convexity of O).
"""
from __future__ import annotations

import math

import numpy as np


def allowed_mask(n: int, causal: bool, window: int = 0) -> np.ndarray:
    """Boolean (N, N) mask: entry [i, j] is True when query i may attend key j."""
    i = np.arange(n)[:, None]
    j = np.arange(n)[None, :]
    m = np.ones((n, n), dtype=bool)
    if causal:
        m &= j <= i
        if window and 0 < window < n:
            m &= (i - j) < window
    return m


def _row_mask(mask, segments, b):
    """Allowed-mask of batch row b: the causal / window mask restricted to segments."""
    if segments is None:
        return mask
    lo = np.asarray(segments[0])[b][:, None]
    hi = np.asarray(segments[1])[b][:, None]
    j = np.arange(mask.shape[1])[None, :]
    return mask & (j >= lo) & (j < hi)


_U32 = 0xFFFFFFFF


def _mix32(x):
    """The engine's 32-bit mixer (uint32 numpy arrays, wrapping arithmetic)."""
    x = np.atleast_1d(np.asarray(x, dtype=np.uint32))  # arrays wrap silently (scalars would warn)
    x = x ^ (x >> np.uint32(16))
    x = x * np.uint32(0x7FEB352D)
    x = x ^ (x >> np.uint32(15))
    x = x * np.uint32(0x846CA68B)
    x = x ^ (x >> np.uint32(16))
    return x


def dropout_mask(seed: int, bh: int, n: int, p: float) -> np.ndarray:
    """Boolean (N, N) keep-mask of query head bh (= b * Hq + h): entry [i, j] keeps P_ij."""
    lo, hi = seed & _U32, (seed >> 32) & _U32
    base = int(_mix32(np.uint32((hi + bh * 0x9E3779B9) & _U32))[0]) ^ lo
    rows = _mix32((np.arange(n, dtype=np.uint64) + base) & _U32)
    keys = ((np.arange(n, dtype=np.uint64) * 0x85EBCA6B) & _U32).astype(np.uint32)
    u = _mix32(rows.astype(np.uint32)[:, None] ^ keys[None, :])
    p32 = float(np.float32(p))  # the ABI carries p as a float
    thresh = int(min(p32 * 4294967296.0, 4294967295.0)) if p32 > 0 else 0
    return u >= np.uint32(thresh)


def _drop(dropout, b, h, Hq, n):
    """(keep-mask, 1 / (1 - p)) of query head h of batch row b, or (None, 1) without dropout."""
    if dropout is None or not dropout[0]:
        return None, 1.0
    p, seed = dropout
    return dropout_mask(seed, b * Hq + h, n, p), 1.0 / (1.0 - float(np.float32(p)))


def _default_scale(d: int, scale):
    return 1.0 / math.sqrt(d) if scale is None else float(scale)


def _capped(s, softcap):
    """Scores after soft-capping and the derivative factor 1 - tanh^2 (1 without a cap)."""
    if not softcap:
        return s, None
    t = np.tanh(s / softcap)
    return softcap * t, 1.0 - t * t


def forward(q, k, v, causal=False, window=0, scale=None, segments=None, softcap=0.0, dropout=None):
    """O (B, Hq, N, D) and natural-log LSE (B, Hq, N), float64."""
    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    sc = _default_scale(D, scale)
    base = allowed_mask(N, causal, window)
    o = np.empty_like(q)
    lse = np.empty((B, Hq, N))
    for b in range(B):
        mask = _row_mask(base, segments, b)
        seen = mask.any(axis=1)[:, None]
        for h in range(Hq):
            g = h * Hkv // Hq
            s, _ = _capped(sc * (q[b, h] @ k[b, g].T), softcap)
            s = np.where(mask, s, -np.inf)
            mx = np.where(seen, s.max(axis=1, keepdims=True), 0.0)
            p = np.where(mask, np.exp(s - mx), 0.0)
            l = p.sum(axis=1, keepdims=True)
            pn = np.where(seen, p / np.where(seen, l, 1.0), 0.0)
            m, ik = _drop(dropout, b, h, Hq, N)
            if m is not None:
                pn = np.where(m, pn * ik, 0.0)
            o[b, h] = pn @ v[b, g]
            lse[b, h] = np.where(seen, mx + np.log(np.where(seen, l, 1.0)), -np.inf)[:, 0]
    return o, lse


def backward(q, k, v, do, causal=False, window=0, scale=None, segments=None, softcap=0.0, dropout=None):
    """dQ, dK, dV (float64) and delta = rowsum(dO * O) for the loss sum(O * dO)."""
    q, k, v, do = (np.asarray(x, dtype=np.float64) for x in (q, k, v, do))
    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    sc = _default_scale(D, scale)
    o, lse = forward(q, k, v, causal, window, scale, segments, softcap, dropout)
    base = allowed_mask(N, causal, window)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    delta = (do * o).sum(axis=-1)
    for b in range(B):
        mask = _row_mask(base, segments, b)
        for h in range(Hq):
            g = h * Hkv // Hq
            s, dcap = _capped(sc * (q[b, h] @ k[b, g].T), softcap)
            p = np.where(mask, np.exp(np.where(mask, s - lse[b, h][:, None], 0.0)), 0.0)
            dp = do[b, h] @ v[b, g].T
            m, ik = _drop(dropout, b, h, Hq, N)
            pd = p
            if m is not None:
                dp = np.where(m, dp * ik, 0.0)
                pd = np.where(m, p * ik, 0.0)
            ds = p * (dp - delta[b, h][:, None])
            if dcap is not None:
                ds = ds * dcap
            dq[b, h] = sc * (ds @ k[b, g])
            dk[b, g] += sc * (ds.T @ q[b, h])
            dv[b, g] += pd.T @ do[b, h]
    return dq, dk, dv, delta


# ----------------------------------------------------------------------------------------
# torch float32, query-chunked: the same equations for shapes too large for dense N x N.
# ----------------------------------------------------------------------------------------

def _chunk_mask(torch, q_lo, q_hi, n, causal, window, device, segments=None, b=0):
    i = torch.arange(q_lo, q_hi, device=device)[:, None]
    j = torch.arange(n, device=device)[None, :]
    m = torch.ones((q_hi - q_lo, n), dtype=torch.bool, device=device)
    if causal:
        m &= j <= i
        if window and 0 < window < n:
            m &= (i - j) < window
    if segments is not None:
        lo = segments[0][b, q_lo:q_hi].to(device)[:, None]
        hi = segments[1][b, q_lo:q_hi].to(device)[:, None]
        m &= (j >= lo) & (j < hi)
    return m


def _mix32_t(x):
    """``_mix32`` on int64 torch tensors holding uint32 values, exact: each product keeps its
    low 32 bits from two partial products below 2^49, so nothing overflows int64."""
    m = 0xFFFFFFFF

    def mul(a, c):
        return (a * (c & 0xFFFF) + (((a * (c >> 16)) & 0xFFFF) << 16)) & m

    x = x ^ (x >> 16)
    x = mul(x, 0x7FEB352D)
    x = x ^ (x >> 15)
    x = mul(x, 0x846CA68B)
    x = x ^ (x >> 16)
    return x


def dropout_mask_rows(seed: int, bh: int, q_lo: int, q_hi: int, n: int, p: float, device=None):
    """Rows [q_lo, q_hi) of ``dropout_mask`` as a torch bool tensor on ``device`` (the chunked
    path's form of the same mask: identical entries, pinned by tests/test_oracle.py)."""
    import torch

    lo, hi = seed & _U32, (seed >> 32) & _U32
    base = int(_mix32(np.uint32((hi + bh * 0x9E3779B9) & _U32))[0]) ^ lo
    rows = _mix32_t((torch.arange(q_lo, q_hi, device=device, dtype=torch.int64) + base) & _U32)
    keys = (torch.arange(n, device=device, dtype=torch.int64) * 0x85EBCA6B) & _U32
    u = _mix32_t(rows[:, None] ^ keys[None, :])
    p32 = float(np.float32(p))
    thresh = int(min(p32 * 4294967296.0, 4294967295.0)) if p32 > 0 else 0
    return u >= thresh


def forward_chunked(q, k, v, causal=False, window=0, scale=None, chunk=1024, segments=None, softcap=0.0,
                    dropout=None):
    """torch fp32 O and LSE for (B, H, N, D) tensors of any float dtype / device.
    ``segments``: (lo, hi) integer tensors (B, N); ``dropout``: (p, seed); both as in ``forward``."""
    import torch

    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    sc = _default_scale(D, scale)
    o = torch.empty((B, Hq, N, D), dtype=torch.float32, device=q.device)
    lse = torch.empty((B, Hq, N), dtype=torch.float32, device=q.device)
    for b in range(B):
        for g in range(Hkv):
            kf = k[b, g].float().contiguous()
            vf = v[b, g].float().contiguous()
            kt = kf.t().contiguous()
            for h in range(g * Hq // Hkv, (g + 1) * Hq // Hkv):
                qf = q[b, h].float()
                for lo in range(0, N, chunk):
                    hi = min(N, lo + chunk)
                    s = (qf[lo:hi] @ kt) * sc
                    if softcap:
                        s = softcap * torch.tanh(s / softcap)
                    mask = _chunk_mask(torch, lo, hi, N, causal, window, q.device, segments, b)
                    seen = mask.any(dim=1, keepdim=True)
                    s = s.masked_fill(~mask, float("-inf"))
                    m = torch.where(seen, s.amax(dim=1, keepdim=True), torch.zeros_like(s[:, :1]))
                    p = torch.exp(s - m)
                    l = p.sum(dim=1, keepdim=True)
                    l1 = torch.where(seen, l, torch.ones_like(l))
                    if dropout is not None and dropout[0]:
                        keep = dropout_mask_rows(dropout[1], b * Hq + h, lo, hi, N, dropout[0], q.device)
                        p = torch.where(keep, p * (1.0 / (1.0 - float(np.float32(dropout[0])))), 0.0)
                    o[b, h, lo:hi] = torch.where(seen, (p @ vf) / l1, torch.zeros_like(qf[lo:hi]))
                    lse[b, h, lo:hi] = torch.where(seen, m + torch.log(l1), torch.full_like(l, float("-inf")))[:, 0]
    return o, lse


def backward_chunked(q, k, v, do, causal=False, window=0, scale=None, chunk=1024, o=None, lse=None,
                     segments=None, softcap=0.0, dropout=None):
    """torch fp32 dQ, dK, dV, delta. ``o``/``lse`` may be passed to skip the recomputation
    (with ``dropout`` they must be the dropped forward's)."""
    import torch

    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    sc = _default_scale(D, scale)
    if o is None or lse is None:
        o, lse = forward_chunked(q, k, v, causal, window, scale, chunk, segments, softcap, dropout)
    dq = torch.empty((B, Hq, N, D), dtype=torch.float32, device=q.device)
    dk = torch.zeros((B, Hkv, N, D), dtype=torch.float32, device=q.device)
    dv = torch.zeros((B, Hkv, N, D), dtype=torch.float32, device=q.device)
    delta = (do.float() * o.float()).sum(dim=-1)
    for b in range(B):
        for g in range(Hkv):
            kf = k[b, g].float().contiguous()
            vf = v[b, g].float().contiguous()
            kt = kf.t().contiguous()
            vt = vf.t().contiguous()
            for h in range(g * Hq // Hkv, (g + 1) * Hq // Hkv):
                qf = q[b, h].float()
                dof = do[b, h].float()
                for lo in range(0, N, chunk):
                    hi = min(N, lo + chunk)
                    mask = _chunk_mask(torch, lo, hi, N, causal, window, q.device, segments, b)
                    s = (qf[lo:hi] @ kt) * sc
                    t = torch.tanh(s / softcap) if softcap else None
                    if softcap:
                        s = softcap * t
                    p = torch.exp((s - lse[b, h, lo:hi, None].float()).masked_fill(~mask, 0.0)).masked_fill(~mask, 0.0)
                    dp = dof[lo:hi] @ vt
                    pd = p
                    if dropout is not None and dropout[0]:
                        keep = dropout_mask_rows(dropout[1], b * Hq + h, lo, hi, N, dropout[0], q.device)
                        ik = 1.0 / (1.0 - float(np.float32(dropout[0])))
                        dp = torch.where(keep, dp * ik, 0.0)
                        pd = torch.where(keep, p * ik, 0.0)
                    ds = p * (dp - delta[b, h, lo:hi, None])
                    if softcap:
                        ds = ds * (1.0 - t * t)
                    dq[b, h, lo:hi] = (ds @ kf) * sc
                    dk[b, g] += (ds.t().contiguous() @ qf[lo:hi]) * sc
                    dv[b, g] += pd.t().contiguous() @ dof[lo:hi]
    return dq, dk, dv, delta
