"""The dK/dV kernel over the reference's tier-0 test matrix
(/root/reference/tests/test_packed_dkv.py:165-199): fp16 inputs, and dK / dV of two
differently reduced paths must agree to max-abs < 1e-2. The reference compares its packed
kernel with its split-and-reduce kernel; here the one-pass kernel (q_splits = 1) is compared
with the query-split path (q_splits = 8: fp32 partials summed by the reduction kernel), and
both with the oracle's fp32 backward at the parity bar (relative Frobenius error <= 5e-2).
"""
from __future__ import annotations

import pytest
import torch

from conftest import make_inputs
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

CONFIGS = [  # (Hq, Hkv, N, D, causal, window), test_packed_dkv.py:168-177
    (8, 1, 512, 256, True, 0),
    (8, 1, 1024, 256, True, 0),
    (8, 1, 2048, 256, True, 512),
    (8, 1, 2048, 256, True, 0),
    (32, 4, 1024, 512, True, 0),
    (32, 4, 2048, 512, True, 0),
    (32, 16, 2048, 256, True, 1024),
]


@pytest.mark.parametrize("Hq,Hkv,N,D,causal,window", CONFIGS)
def test_dkv_split_paths_and_oracle(Hq, Hkv, N, D, causal, window, device):
    from gemma_triton_flash_attn_amd.attention import _backward, _forward

    print(f"case dkv Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal} window={window} fp16", flush=True)
    q, k, v, do = make_inputs(1, Hq, Hkv, N, D, torch.float16, device, seed=0)
    sc = D ** -0.5
    o, lse = _forward(q, k, v, causal, window, sc, True)
    res = {}
    for qs in (1, 8):
        _, dk, dv, _ = _backward(q, k, v, o, lse, do, causal, window, sc, q_splits=qs)
        res[qs] = (dk.float(), dv.float())
    for name, a, b in zip(("dK", "dV"), res[1], res[8]):
        diff = float((a - b).abs().max())
        print(f"  {name} q_splits 1 vs 8 max-abs {diff:.2e}", flush=True)
        assert diff < 1e-2
    _, dk_r, dv_r, _ = orc.backward_chunked(q, k, v, do, causal, window, sc)
    for name, a, b in zip(("dK", "dV"), res[1], (dk_r, dv_r)):
        rel = float(torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(b))
        print(f"  {name} vs oracle rel {rel:.2e}", flush=True)
        assert rel <= 5e-2
