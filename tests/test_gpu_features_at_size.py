"""GPU parity of the soft-capping, dropout and segment-table kernel instances at the BASELINE
sizes: N=16384 under the config-3 window (D=256, W=1024, GQA 2:1) and at the headline's full
causal D=512 (GQA 8:1, one KV head), against the oracle's query-chunked float32 path run on the
GPU on the same 16-bit inputs.

At these sizes a segment table's per-workgroup tile-range trimming (from the bounds of a
block's first and last token), the per-row dropout keys of queries and keys far from the
origin, and the soft-cap's derivative in both backward kernels meet rows thousands of tiles
long, which the small-N tests (test_gpu_segments.py, test_gpu_dropout.py, test_gpu_softcap.py)
do not reach. The oracle's chunked path is pinned to its dense float64 path with each feature
on the CPU (tests/test_oracle.py, tests/test_segments_cpu.py).

Dropout masks are keyed on the global query head index (b * Hq + h), so the oracle always runs
every head of the problem here (no head slicing).

Bar (as tests/test_gpu_parity.py): O max-abs <= 1e-2 (fp16) / 2e-2 (bf16); dQ, dK, dV relative
Frobenius error <= 5e-2.
"""
from __future__ import annotations

import pytest
import torch

from conftest import make_inputs
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

O_TOL = {torch.float16: 1e-2, torch.bfloat16: 2e-2}
GRAD_TOL = 5e-2
SEED = 0x0BAD_5EED_1357_9BDF
N = 16384
# several packed sequences of uneven lengths (one of a single token), then padding to N
CU = [0, 1500, 1501, 6000, 9000, 16000]

SHAPES = {
    # name: Hq, Hkv, D, causal, window
    "c3_d256_swa1024": (4, 2, 256, True, 1024),
    "headline_d512_causal": (8, 1, 512, True, 0),
}
FEATURES = {
    # name: softcap, dropout p, packed segments, dtype
    "softcap": (5.0, 0.0, False, torch.bfloat16),
    "dropout": (0.0, 0.1, False, torch.bfloat16),
    "cu_seqlens": (0.0, 0.0, True, torch.bfloat16),
    "dropout_cu_seqlens": (0.0, 0.15, True, torch.bfloat16),
    "softcap_cu_seqlens_fp16": (5.0, 0.0, True, torch.float16),
}


def _rel(a, b):
    return float(torch.linalg.vector_norm(a.float() - b.float()) / torch.linalg.vector_norm(b.float()))


@pytest.mark.parametrize("feature", list(FEATURES))
@pytest.mark.parametrize("shape", list(SHAPES))
def test_feature_at_size_vs_chunked_fp32(shape, feature, device):
    import gemma_triton_flash_attn_amd as gfa
    from gemma_triton_flash_attn_amd.attention import _backward, _forward

    Hq, Hkv, D, causal, window = SHAPES[shape]
    cap, p, packed, dtype = FEATURES[feature]
    print(f"case {shape} {feature}: B=1 Hq={Hq} Hkv={Hkv} N={N} D={D} window={window} softcap={cap} dropout={p} "
          f"packed={packed} {dtype}", flush=True)
    q, k, v, do = make_inputs(1, Hq, Hkv, N, D, dtype, device, seed=D + Hq + int(10 * cap + 100 * p))
    segs = gfa.segments.from_cu_seqlens(CU, N, device=device) if packed else None
    sc = D ** -0.5
    o, lse = _forward(q, k, v, causal, window, sc, store_lse=True, segments=segs, softcap=cap, dropout_p=p,
                      dropout_seed=SEED)
    dq, dk, dv, _ = _backward(q, k, v, o, lse, do, causal, window, sc, segments=segs, softcap=cap, dropout_p=p,
                              dropout_seed=SEED)
    torch.cuda.synchronize()
    drop = (p, SEED) if p > 0 else None
    o_ref, lse_ref = orc.forward_chunked(q, k, v, causal, window, segments=segs, softcap=cap, dropout=drop)
    dq_ref, dk_ref, dv_ref, _ = orc.backward_chunked(q, k, v, do, causal, window, o=o_ref, lse=lse_ref,
                                                     segments=segs, softcap=cap, dropout=drop)
    err_o = float((o.float() - o_ref).abs().max())
    errs = (_rel(dq, dq_ref), _rel(dk, dk_ref), _rel(dv, dv_ref))
    seen = torch.isfinite(lse_ref)
    err_lse = float((lse[:, :, :N] - lse_ref).abs()[seen].max())
    print(f"  O max-abs {err_o:.3e}  LSE {err_lse:.3e}  dQ/dK/dV rel {errs[0]:.3e} {errs[1]:.3e} {errs[2]:.3e}",
          flush=True)
    assert err_o <= O_TOL[dtype]
    assert max(errs) <= GRAD_TOL
    assert err_lse <= 1e-2  # undropped LSE, natural log
    if packed:
        # padding tokens past the last sequence: zero output and gradient rows
        assert float(o[:, :, CU[-1]:].abs().max()) == 0.0
        assert float(dq[:, :, CU[-1]:].abs().max()) == 0.0
        assert float(dk[:, :, CU[-1]:].abs().max()) == 0.0 and float(dv[:, :, CU[-1]:].abs().max()) == 0.0
    if p > 0:
        # the mask is applied: the undropped output is far from the dropped one
        o_keep, _ = orc.forward_chunked(q[:, :1], k[:, :1], v[:, :1], causal, window, segments=segs, softcap=cap)
        assert float((o_keep - o_ref[:, :1]).abs().max()) > 5 * O_TOL[dtype]
