"""Write the golden vectors in this directory.

The expected values come from torch's own scaled_dot_product_attention (math backend,
float64) and its autograd - a library implementation independent of oracle/ - so the
oracle and the GPU kernels are both checked against them.

Inputs are N(0,1) from a fixed CPU generator, rounded to bfloat16 (so the GPU kernels
see exactly the stored inputs) and stored as uint16 bit patterns; outputs are float32.
Each case uses a sequence length that is not a multiple of 32 and a GQA group > 1.

Run from the repo root: python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import numpy as np
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

HERE = os.path.dirname(os.path.abspath(__file__))

CASES = [
    # name, B, Hq, Hkv, N, D, causal, window
    ("d512_causal_gqa2", 1, 2, 1, 33, 512, True, 0),
    ("d256_swa7_gqa2", 1, 4, 2, 40, 256, True, 7),
    ("d256_full_gqa4", 1, 4, 1, 37, 256, False, 0),
    ("d8_causal_gqa3", 2, 6, 2, 19, 8, True, 0),
    ("d8_swa4_mha", 1, 3, 3, 23, 8, True, 4),
    ("d128_swa9_gqa4", 1, 8, 2, 45, 128, True, 9),
    ("d64_causal_gqa2", 2, 4, 2, 50, 64, True, 0),
    ("d64_full_mha", 1, 2, 2, 29, 64, False, 0),
]


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _mask(n, causal, window):
    i = torch.arange(n)[:, None]
    j = torch.arange(n)[None, :]
    m = torch.ones(n, n, dtype=torch.bool)
    if causal:
        m &= j <= i
        if window:
            m &= (i - j) < window
    return m


def make(name, B, Hq, Hkv, N, D, causal, window, seed=1234):
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = (torch.randn(*s, generator=g).to(torch.bfloat16)
                   for s in [(B, Hq, N, D), (B, Hkv, N, D), (B, Hkv, N, D), (B, Hq, N, D)])
    q64, k64, v64, do64 = (t.double().requires_grad_(True) for t in (q, k, v, do))
    r = Hq // Hkv
    ke = k64.repeat_interleave(r, dim=1)
    ve = v64.repeat_interleave(r, dim=1)
    mask = _mask(N, causal, window)
    bias = torch.zeros(N, N, dtype=torch.float64).masked_fill(~mask, float("-inf"))
    with sdpa_kernel(SDPBackend.MATH):
        o = F.scaled_dot_product_attention(q64, ke, ve, attn_mask=bias[None, None])
    (o * do64.detach()).sum().backward()
    s = (q64.detach() @ ke.detach().transpose(-1, -2)) / D ** 0.5 + bias
    lse = torch.logsumexp(s, dim=-1)
    np.savez(
        os.path.join(HERE, f"{name}.npz"),
        meta=np.array([B, Hq, Hkv, N, D, int(causal), window], dtype=np.int64),
        q=_bf16_bits(q), k=_bf16_bits(k), v=_bf16_bits(v), do=_bf16_bits(do),
        o=o.detach().float().numpy(), lse=lse.float().numpy(),
        dq=q64.grad.float().numpy(), dk=k64.grad.float().numpy(), dv=v64.grad.float().numpy(),
    )


if __name__ == "__main__":
    for c in CASES:
        make(*c)
        print("wrote", c[0])
