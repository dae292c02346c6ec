"""The HF adapter over the reference's adapter test matrix
(/root/reference/tests/gemma4_integration/test_adapter.py:131-175), with its pass criterion
(cosine similarity > 0.999 and relative Frobenius error < 0.05 in fp32, line 188).

Differences from the reference test: inputs are drawn on a CPU generator (seeded, so the
same on every host) instead of ``torch.manual_seed`` on CUDA, and the reference is the
oracle's fp32 path (the same masked-softmax math as its ``sdpa_reference``, 48-80).
"""
from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from conftest import make_inputs
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu


def _matrix():
    n_short, n_long, slide = 512, 2048, 512
    cases = []
    for hq, hkv in [(8, 8), (8, 4), (8, 2), (8, 1), (16, 2)]:
        cases += [(1, hq, hkv, n_short, 256, 0), (1, hq, hkv, n_long, 256, 0),
                  (1, hq, hkv, n_short, 256, slide), (1, hq, hkv, n_long, 256, slide)]
    cases += [(1, 32, 4, n, 512, 0) for n in (n_short, n_long)]
    cases += [(2, 8, 1, 1024, 256, 0), (2, 8, 1, 2048, 256, 512)]
    cases += [(1, 16, 8, 1024, 256, 1024), (1, 16, 8, 2048, 256, 1024)]
    cases += [(1, 16, 2, n, 512, 0) for n in (n_short, n_long)]
    return cases


@pytest.mark.parametrize("B,Hq,Hkv,N,D,slide", _matrix())
def test_adapter_matrix(B, Hq, Hkv, N, D, slide, device):
    import gemma_triton_flash_attn_amd as gfa

    print(f"case adapter B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} slide={slide}", flush=True)
    q, k, v, _ = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=0, with_do=False) + [None]
    module = SimpleNamespace(head_dim=D, is_causal=True)
    out, _ = gfa.triton_gqa_attention(module, q, k, v, attention_mask=None, dropout=0.0, scaling=None,
                                      softcap=None, sliding_window=slide if slide > 0 else None)
    ref, _ = orc.forward_chunked(q, k, v, True, slide if slide < N else 0, D ** -0.5)
    a, b = out.float().flatten(), ref.transpose(1, 2).float().flatten()
    cos = float(torch.nn.functional.cosine_similarity(a, b, dim=0))
    rel = float(torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(b))
    print(f"  cos {cos:.6f} rel {rel:.3e}", flush=True)
    assert cos > 0.999 and rel < 0.05
