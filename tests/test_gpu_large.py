"""GPU parity at the BASELINE sizes (configs 2-4 and the N=16384 headline layer) and at the
bench's N=16384 D=128 / D=64 workloads.

Two kinds of check:
  * against the oracle's query-chunked torch float32 path (``forward_chunked`` /
    ``backward_chunked``) run on the GPU on the same 16-bit inputs, every KV head with its
    query heads. The reference runs on a few KV heads at a time (the largest shapes one at a
    time, to bound its fp32 memory); the engine runs the whole problem once, and a group's
    outputs and dK/dV depend on nothing outside it;
  * size-independent identities that hold for the full problem and need no reference:
      - every output row is a convex combination of V rows: min V <= O <= max V;
      - sum over keys of dV equals the sum of dO over the KV group's query heads (rows of P
        sum to one);
      - sum over keys of dK is zero (rows of dS sum to zero, since
        sum_j P_ij dP_ij = dO_i . O_i = delta_i), up to the 16-bit rounding of dS.

Inputs follow the measurement convention: seed 0, drawn on a CPU generator in the order
q, k, v, dO, then cast and moved (config 4 scales them by 0.5 and runs in fp16).
Tolerances as in test_gpu_parity.py: O max-abs 1e-2 (fp16) / 2e-2 (bf16), gradients 5e-2
relative (Frobenius).
"""
from __future__ import annotations

import pytest
import torch

from conftest import make_inputs
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

O_TOL = {torch.float16: 1e-2, torch.bfloat16: 2e-2}
GRAD_TOL = 5e-2

LARGE = {
    # name: B, Hq, Hkv, N, D, causal, window, dtype, amplitude, KV heads per reference run
    "c2_d512_causal_32x4_n8k": (1, 32, 4, 8192, 512, True, 0, torch.bfloat16, 1.0, 4),
    "c3_d256_swa1024_16x8_n16k": (1, 16, 8, 16384, 256, True, 1024, torch.bfloat16, 1.0, 8),
    "headline_d512_causal_32x4_n16k": (1, 32, 4, 16384, 512, True, 0, torch.bfloat16, 1.0, 1),
    "c4_d512_causal_16x2_n32k_fp16": (1, 16, 2, 32768, 512, True, 0, torch.float16, 0.5, 1),
    # the bench's D=128 / D=64 workloads (the rest of the reference's head-dim range)
    "d128_causal_32x8_n16k": (1, 32, 8, 16384, 128, True, 0, torch.bfloat16, 1.0, 2),
    "d64_causal_32x32_n16k": (1, 32, 32, 16384, 64, True, 0, torch.bfloat16, 1.0, 4),
    "d128_swa2048_16x4_n16k_fp16": (1, 16, 4, 16384, 128, True, 2048, torch.float16, 1.0, 4),
}


def _rel(a, b):
    return float(torch.linalg.vector_norm(a.float() - b.float()) / torch.linalg.vector_norm(b.float()))


def _engine(q, k, v, do, causal, window):
    import gemma_triton_flash_attn_amd as gfa

    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = gfa.flash_attn_gqa_train(qq, kk, vv, causal=causal, slide_size=window)
    o.backward(do)
    torch.cuda.synchronize()
    return o.detach(), qq.grad, kk.grad, vv.grad


def _check_kv_heads(q, k, v, do, o, dq, dk, dv, causal, window, dtype, kv_lo, kv_hi):
    """Compare the engine's outputs of KV heads [kv_lo, kv_hi) and their query heads with
    the chunked fp32 oracle run on those heads alone."""
    R = q.shape[1] // k.shape[1]
    hq = slice(kv_lo * R, kv_hi * R)
    hk = slice(kv_lo, kv_hi)
    o_ref, lse_ref = orc.forward_chunked(q[:, hq], k[:, hk], v[:, hk], causal, window)
    err_o = float((o[:, hq].float() - o_ref).abs().max())
    dq_ref, dk_ref, dv_ref, _ = orc.backward_chunked(q[:, hq], k[:, hk], v[:, hk], do[:, hq], causal, window,
                                                     o=o_ref, lse=lse_ref)
    errs = (_rel(dq[:, hq], dq_ref), _rel(dk[:, hk], dk_ref), _rel(dv[:, hk], dv_ref))
    print(f"  KV heads [{kv_lo}, {kv_hi}): O max-abs {err_o:.3e}  dQ/dK/dV rel {errs[0]:.3e} {errs[1]:.3e} "
          f"{errs[2]:.3e}", flush=True)
    del o_ref, lse_ref, dq_ref, dk_ref, dv_ref
    assert err_o <= O_TOL[dtype]
    assert max(errs) <= GRAD_TOL


@pytest.mark.parametrize("name", list(LARGE))
def test_large_vs_chunked_fp32(name, device):
    """Every KV head with its query heads, ``ref_kv`` KV heads per reference run."""
    B, Hq, Hkv, N, D, causal, window, dtype, amp, ref_kv = LARGE[name]
    print(f"case {name}", flush=True)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, dtype, device, seed=0, scale=amp)
    o, dq, dk, dv = _engine(q, k, v, do, causal, window)
    for kv_lo in range(0, Hkv, ref_kv):
        _check_kv_heads(q, k, v, do, o, dq, dk, dv, causal, window, dtype, kv_lo, min(Hkv, kv_lo + ref_kv))
        torch.cuda.empty_cache()


@pytest.mark.parametrize("name", ["headline_d512_causal_32x4_n16k", "c3_d256_swa1024_16x8_n16k",
                                  "d128_causal_32x8_n16k", "d64_causal_32x32_n16k"])
def test_large_invariants(name, device):
    B, Hq, Hkv, N, D, causal, window, dtype, amp, _ = LARGE[name]
    print(f"case {name}", flush=True)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, dtype, device, seed=1, scale=amp)
    o, dq, dk, dv = _engine(q, k, v, do, causal, window)
    R = Hq // Hkv
    # convexity (with the output's own rounding: one 16-bit ulp of the largest |V|)
    vmin = v.float().amin(dim=2).repeat_interleave(R, dim=1)[:, :, None]
    vmax = v.float().amax(dim=2).repeat_interleave(R, dim=1)[:, :, None]
    ulp = float(v.float().abs().max()) * (2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10)
    assert bool(((o.float() >= vmin - ulp) & (o.float() <= vmax + ulp)).all())
    # sum_j dV_j = sum over the group's query heads and rows of dO
    sdv = dv.float().sum(dim=2)
    sdo = do.float().sum(dim=2).view(B, Hkv, R, D).sum(dim=2)
    e_v = _rel(sdv, sdo)
    # sum_j dK_j = 0, judged against |dK|_F (independent per-key gradients would give ~1)
    sdk = dk.float().sum(dim=2)
    e_k = float(torch.linalg.vector_norm(sdk) / torch.linalg.vector_norm(dk.float()))
    print(f"  sum dV vs sum dO rel {e_v:.3e}; |sum dK| / |dK| {e_k:.3e}", flush=True)
    assert e_v <= 1e-2
    assert e_k <= 5e-2
    assert torch.isfinite(dq).all()
