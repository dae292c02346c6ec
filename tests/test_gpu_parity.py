"""GPU parity of the HIP kernels against the oracle (float64 numpy on the exact same
16-bit inputs) at sizes the oracle finishes in seconds, and against the golden vectors.

Tolerances: O max-abs <= 1e-2 (fp16) / 2e-2 (bf16);
dQ, dK, dV relative Frobenius error <= 5e-2. LSE is checked to 1e-2 absolute.
"""
from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

from conftest import make_inputs
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
O_TOL = {torch.float16: 1e-2, torch.bfloat16: 2e-2}
GRAD_TOL = 5e-2
# Absolute floor (RMS per element) for gradients whose exact value is ~0 (e.g. window 1,
# where dS = P * (dP - delta) cancels exactly): relative error is meaningless there.
GRAD_ABS_RMS = 1e-3


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _rel(a, b):
    """||a - b||_F / ||b||_F, with the denominator floored at GRAD_ABS_RMS * sqrt(numel)
    so that an exactly-zero reference gradient is judged by absolute error."""
    floor = GRAD_ABS_RMS * np.sqrt(b.size) / GRAD_TOL
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), floor))


def _run(q, k, v, do, causal, window):
    import gemma_triton_flash_attn_amd as gfa

    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = gfa.flash_attn_gqa_train(qq, kk, vv, causal=causal, slide_size=window)
    o.backward(do)
    torch.cuda.synchronize()
    return o, qq.grad, kk.grad, vv.grad


SMALL = [
    # B, Hq, Hkv, N, D, causal, window, dtype
    (1, 4, 1, 128, 512, True, 0, torch.bfloat16),
    (1, 8, 1, 96, 512, True, 0, torch.float16),
    (1, 2, 2, 70, 512, False, 0, torch.bfloat16),
    (2, 4, 2, 100, 256, True, 0, torch.bfloat16),
    (1, 4, 2, 160, 256, True, 48, torch.bfloat16),
    (1, 2, 1, 200, 256, True, 33, torch.float16),
    (1, 16, 2, 64, 256, True, 1, torch.bfloat16),
    (1, 2, 1, 40, 256, True, 64, torch.bfloat16),   # window >= N -> causal
    (1, 8, 8, 33, 256, False, 0, torch.float16),
    (1, 4, 4, 1, 512, True, 0, torch.bfloat16),     # N = 1
    (1, 6, 3, 31, 256, True, 0, torch.bfloat16),    # odd group size
    (2, 8, 2, 160, 512, True, 0, torch.float16),    # batch > 1 at D=512
    (1, 8, 1, 130, 512, True, 40, torch.bfloat16),  # sliding window at D=512
    (1, 6, 2, 100, 512, True, 0, torch.bfloat16),   # group size 3: one head per workgroup group
    (1, 16, 1, 96, 256, True, 20, torch.float16),   # group size 16
    (1, 4, 1, 257, 256, True, 100, torch.bfloat16), # window over many tiles, ragged N
    (2, 8, 2, 65, 512, False, 0, torch.float16),    # non-causal, batch > 1, D=512
    (1, 2, 1, 64, 512, True, 63, torch.bfloat16),   # window = N - 1
    # D=128 and D=64 (the rest of the reference's documented 64-512 range)
    (1, 8, 2, 200, 128, True, 0, torch.bfloat16),
    (2, 4, 1, 131, 128, True, 37, torch.float16),
    (1, 4, 4, 97, 128, False, 0, torch.bfloat16),
    (1, 8, 1, 300, 64, True, 0, torch.float16),
    (2, 6, 2, 77, 64, True, 16, torch.bfloat16),
    (1, 2, 2, 45, 64, False, 0, torch.float16),
    (1, 4, 1, 1, 64, True, 0, torch.bfloat16),      # N = 1 at D=64
]


@pytest.mark.parametrize("B,Hq,Hkv,N,D,causal,window,dtype", SMALL)
def test_fwd_bwd_vs_oracle(B, Hq, Hkv, N, D, causal, window, dtype, device):
    print(f"case B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal} window={window} {dtype}", flush=True)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, dtype, device, seed=N + D)
    o, dq, dk, dv = _run(q, k, v, do, causal, window)
    o_ref, lse_ref = orc.forward(_np(q), _np(k), _np(v), causal, window)
    dq_ref, dk_ref, dv_ref, _ = orc.backward(_np(q), _np(k), _np(v), _np(do), causal, window)
    err_o = float(np.abs(_np(o) - o_ref).max())
    errs = [_rel(_np(g), r) for g, r in ((dq, dq_ref), (dk, dk_ref), (dv, dv_ref))]
    print(f"  O max-abs {err_o:.3e}  dQ/dK/dV rel {errs[0]:.3e} {errs[1]:.3e} {errs[2]:.3e}", flush=True)
    assert err_o <= O_TOL[dtype]
    assert max(errs) <= GRAD_TOL


@pytest.mark.parametrize("B,Hq,Hkv,N,D,causal,window,dtype", SMALL[:6] + [c for c in SMALL if c[4] < 256][:3])
def test_lse_and_inference_path(B, Hq, Hkv, N, D, causal, window, dtype, device):
    from gemma_triton_flash_attn_amd.attention import _forward

    q, k, v, _ = make_inputs(B, Hq, Hkv, N, D, dtype, device, seed=7 + N)
    scale = D ** -0.5
    o, lse = _forward(q, k, v, causal, window if window < N else 0, scale, store_lse=True)
    o_ref, lse_ref = orc.forward(_np(q), _np(k), _np(v), causal, window)
    assert lse.shape[-1] % 64 == 0 and lse.shape[-1] >= N
    assert float(np.abs(_np(lse[..., :N]) - lse_ref).max()) <= 1e-2
    import gemma_triton_flash_attn_amd as gfa

    o_inf = gfa.attention_flash_gqa(q, k, v, causal=causal, slide_size=window)
    torch.cuda.synchronize()
    assert torch.equal(o_inf, o), "inference and training forward must agree bitwise"


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "d*_*.npz"))))
def test_golden_vectors(path, device):
    z = np.load(path)
    B, Hq, Hkv, N, D, causal, window = (int(x) for x in z["meta"])
    from gemma_triton_flash_attn_amd import SUPPORTED_HEAD_DIMS

    if D not in SUPPORTED_HEAD_DIMS:
        pytest.skip("head dim outside the kernel set (oracle-only vector)")
    print(f"golden {os.path.basename(path)}", flush=True)
    q, k, v, do = (torch.from_numpy(z[n].view(np.int16)).view(torch.bfloat16).to(device) for n in ("q", "k", "v", "do"))
    o, dq, dk, dv = _run(q, k, v, do, bool(causal), window)
    assert float(np.abs(_np(o) - z["o"]).max()) <= O_TOL[torch.bfloat16]
    for g, n in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        assert _rel(_np(g), z[n].astype(np.float64)) <= GRAD_TOL, n


def test_hf_strided_layout_matches_contiguous(device):
    """(B, H, N, D) views of (B, N, H, D) storage (what transformers passes) give the same
    bits as contiguous inputs, and O keeps the caller's layout."""
    import gemma_triton_flash_attn_amd as gfa

    args = (1, 8, 2, 96, 256, torch.bfloat16, device)
    qs, ks, vs, dos = make_inputs(*args, seed=3, layout="bnhd")
    qc, kc, vc, doc = (t.contiguous() for t in (qs, ks, vs, dos))
    o1, g1 = _run(qs, ks, vs, dos, True, 40)[0], _run(qs, ks, vs, dos, True, 40)[1:]
    o2, g2 = _run(qc, kc, vc, doc, True, 40)[0], _run(qc, kc, vc, doc, True, 40)[1:]
    assert torch.equal(o1, o2)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)
    o3 = gfa.attention_flash_gqa(qs, ks, vs, causal=True, slide_size=40)
    assert o3.stride() == qs.stride()


def test_deterministic(device):
    q, k, v, do = make_inputs(1, 8, 2, 192, 512, torch.bfloat16, device, seed=11)
    r1 = _run(q, k, v, do, True, 0)
    r2 = _run(q, k, v, do, True, 0)
    for a, b in zip(r1, r2):
        assert torch.equal(a, b)


@pytest.mark.parametrize("qs,D,window", [(2, 256, 0), (4, 256, 0), (8, 256, 0), (2, 256, 64), (8, 256, 100),
                                          (2, 512, 0), (8, 512, 0), (4, 128, 0), (8, 64, 0)])
def test_q_splits_match(qs, D, window, device):
    """Q-split fp32 partials + reduction agree with the single-split kernel (every dK/dV
    kernel form: one wave per 32 keys at D=256 and D=64, role-split pairs at D=512 and D=128,
    and at D=256 with a window)."""
    from gemma_triton_flash_attn_amd.attention import _backward, _forward

    q, k, v, do = make_inputs(1, 8, 1, 256, D, torch.bfloat16, device, seed=5)
    o, lse = _forward(q, k, v, True, window, D ** -0.5, store_lse=True)
    ref = _backward(q, k, v, o, lse, do, True, window, D ** -0.5, q_splits=1)
    got = _backward(q, k, v, o, lse, do, True, window, D ** -0.5, q_splits=qs)
    torch.cuda.synchronize()
    assert torch.equal(ref[0], got[0])  # dQ does not depend on the split
    for a, b in zip(ref[1:3], got[1:3]):
        assert _rel(_np(b), _np(a)) < 1e-2


@pytest.mark.parametrize("dtype,jump,D,window", [(torch.float16, 16.0, 256, 0), (torch.bfloat16, 60.0, 256, 0),
                                                (torch.float16, 5.0, 256, 0), (torch.float16, 16.0, 128, 0),
                                                (torch.float16, 16.0, 64, 0), (torch.float16, 16.0, 512, 0),
                                                (torch.bfloat16, 60.0, 512, 0), (torch.float16, 16.0, 256, 150),
                                                (torch.float16, 16.0, 512, 150), (torch.bfloat16, 60.0, 128, 0),
                                                (torch.bfloat16, 60.0, 256, 150), (torch.bfloat16, 40.0, 256, 0)])
def test_late_large_scores(dtype, jump, D, window, device):
    """Scores that grow far above the first tile's maximum. The forward fixes each row's
    reference max at its first visible tile; rows whose later scores exceed it by more
    than the 16-bit-safe margin force the exact-max second pass. Both paths must agree
    with the oracle (``jump`` is the score gap in natural-log units).

    Gradients are compared for fp16 only: at a 60-nat gap in bf16 the softmax is nearly
    one-hot and dS = P * (dP - delta) cancels, with delta = rowsum(dO * O) taken from the
    stored bf16 O (as in the reference, attention.py:733-742); the 2^-9 rounding of O then
    dominates dQ. For that case only the forward and the finiteness of the gradients are
    checked. With a window the D=256 forward walks its key tiles cyclically, not in order. In
    bf16 at D <= 256 the forward judges overflow from the row sum and finds the exact row max
    for the redo in a pass of its own; a 40-nat gap (58 in log2) stays under the 2^64 margin and
    is computed without a redo, with P up to 2^58."""
    B, Hq, Hkv, N = 1, 4, 2, 192
    g = torch.Generator().manual_seed(9)
    q = torch.randn(B, Hq, N, D, generator=g) * 0.1
    k = torch.randn(B, Hkv, N, D, generator=g) * 0.1
    v = torch.randn(B, Hkv, N, D, generator=g)
    do = torch.randn(B, Hq, N, D, generator=g)
    # Keys from 100 on align with a shared direction carried by every query.
    u = torch.ones(D) / D ** 0.5
    q += u * 4.0
    k[:, :, 100:] += u * (jump * D ** 0.5 / 4.0)
    q, k, v, do = (t.to(device=device, dtype=dtype) for t in (q, k, v, do))
    from gemma_triton_flash_attn_amd.attention import _forward

    o, dq, dk, dv = _run(q, k, v, do, True, window)
    o_ref, lse_ref = orc.forward(_np(q), _np(k), _np(v), True, window)
    dq_ref, dk_ref, dv_ref, _ = orc.backward(_np(q), _np(k), _np(v), _np(do), True, window)
    assert torch.isfinite(o).all()
    assert float(np.abs(_np(o) - o_ref).max()) <= O_TOL[dtype]
    _, lse = _forward(q, k, v, True, window, D ** -0.5, store_lse=True)
    lse = _np(lse)[..., :N]
    assert float((np.abs(lse - lse_ref) / np.maximum(1.0, np.abs(lse_ref))).max()) <= 1e-3
    for got, ref in ((dq, dq_ref), (dk, dk_ref), (dv, dv_ref)):
        assert torch.isfinite(got).all()
        if dtype == torch.float16:
            assert _rel(_np(got), ref) <= GRAD_TOL


@pytest.mark.parametrize("D", [256, 128, 64])
@pytest.mark.parametrize("block_kv", [32, 64])
def test_block_kv_override(block_kv, D, device):
    """attention_flash_gqa's BLOCK_KV picks one of the built forward tiles of the head dim;
    every choice matches the oracle and they agree with each other closely."""
    import gemma_triton_flash_attn_amd as gfa

    q, k, v, _ = make_inputs(1, 4, 2, 150, D, torch.bfloat16, device, seed=21)
    o = gfa.attention_flash_gqa(q, k, v, causal=True, slide_size=50, BLOCK_KV=block_kv)
    o_def = gfa.attention_flash_gqa(q, k, v, causal=True, slide_size=50)
    o_ref, _ = orc.forward(_np(q), _np(k), _np(v), True, 50)
    assert float(np.abs(_np(o) - o_ref).max()) <= O_TOL[torch.bfloat16]
    assert float((o.float() - o_def.float()).abs().max()) <= 1e-2


@pytest.mark.parametrize("N,D,window,segs", [(100, 256, 0, False), (77, 64, 16, False), (130, 128, 0, False),
                                             (45, 512, 0, False), (150, 256, 48, True)])
def test_delta_scratch_garbage_does_not_leak(N, D, window, segs, device):
    """The dK/dV kernel reads whole 32-row tiles of delta and multiplies masked entries
    (P = 0) by (dP - delta) without a guard: the dQ kernel must write every delta row such
    a tile covers, also those past N. A delta buffer prefilled with NaN (and a DKV-only call
    reading it after a DQ call) must give the same gradients as a fresh buffer, bit for bit."""
    from gemma_triton_flash_attn_amd import _lib
    from gemma_triton_flash_attn_amd.attention import _backward, _forward, lse_ld

    B, Hq, Hkv = 2, 4, 2
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=N + D)
    segments = None
    if segs:
        import gemma_triton_flash_attn_amd as gfa
        segments = gfa.segments.from_lengths([N - 17, N // 2], N, device=device)
    sc = D ** -0.5
    o, lse = _forward(q, k, v, True, window, sc, store_lse=True, segments=segments)
    ref = _backward(q, k, v, o, lse, do, True, window, sc, segments=segments)
    bufs = (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
            torch.full((B, Hq, lse_ld(N)), float("nan"), dtype=torch.float32, device=device))
    _backward(q, k, v, o, lse, do, True, window, sc, stages=_lib.GFA_BWD_DQ, out=bufs, segments=segments)
    _backward(q, k, v, o, lse, do, True, window, sc, stages=_lib.GFA_BWD_DKV, out=bufs, segments=segments)
    torch.cuda.synchronize()
    for a, r in zip(bufs[:3], ref[:3]):
        assert torch.isfinite(a.float()).all()
        assert torch.equal(a, r)
    # every delta row a 32-row tile covers is finite
    n32 = (N + 31) // 32 * 32
    assert torch.isfinite(bufs[3][:, :, :n32]).all()


@pytest.mark.parametrize("N,D,causal,window", [(100, 512, True, 0), (77, 256, True, 0), (150, 256, True, 48),
                                               (70, 256, False, 0), (131, 128, True, 37), (45, 64, False, 0),
                                               (300, 64, True, 0)])
def test_nan_past_sequence_end_does_not_leak(N, D, causal, window, device):
    """Every kernel reads whole 32-row tiles, also past row N - 1 of a (batch, head) slice.
    With q, k, v and dO held as views of buffers whose rows past N are NaN, the output, LSE
    and gradients must equal those of contiguous copies bit for bit: rows past N must be
    zero-filled by the buffer range check or clamped, never read as data."""
    B, Hq, Hkv = 2, 4, 2
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=3 * N + D)

    def padded(t):
        buf = torch.full((t.shape[0], t.shape[1], N + 128, D), float("nan"), dtype=t.dtype, device=device)
        buf[:, :, :N] = t
        return buf[:, :, :N]

    ref = _run(q, k, v, do, causal, window)
    got = _run(padded(q), padded(k), padded(v), padded(do), causal, window)
    for a, r in zip(got, ref):
        assert torch.isfinite(a.float()).all()
        assert torch.equal(a, r)
    from gemma_triton_flash_attn_amd.attention import _forward
    sc = D ** -0.5
    o_r, lse_r = _forward(q, k, v, causal, window, sc, store_lse=True)
    o_g, lse_g = _forward(padded(q), padded(k), padded(v), causal, window, sc, store_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(o_g, o_r)
    assert torch.equal(lse_g[:, :, :N], lse_r[:, :, :N])
