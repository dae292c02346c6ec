"""Math reference helpers kept from the reference's public API.

``attention`` restates /root/reference/flash_attn/attention.py:11-17 (plain torch
scaled_dot_product_attention: non-causal, any device, dtype and head dim, differentiable).
``attention_gqa_ref`` and ``attention_swa_ref`` restate attention.py:611-619 and 622-642:
GQA by repeating each KV head over its query group, scale 1/sqrt(D), causal /
sliding-window masks, evaluated with torch's scaled_dot_product_attention. They are the
reference's PyTorch reference functions, kept under the same names so code that calls them
keeps working and so users can compare the engine against them; no engine entry point
calls them, and they are not the engine (which is ``attention_flash_gqa`` /
``flash_attn_gqa_train``).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _expand_kv(q, k, v):
    hq, hkv = q.shape[1], k.shape[1]
    if hq != hkv:
        r = hq // hkv
        k = k.repeat_interleave(r, dim=1)
        v = v.repeat_interleave(r, dim=1)
    return k, v


def attention(q, k, v):
    """Standard scaled dot-product attention (reference attention.py:11-17):
    q, k, v (batch, n_heads, seq_len, head_dim) -> (batch, n_heads, seq_len, head_dim).
    torch SDPA, as in the reference: works on any device, dtype and head dim, with autograd."""
    return F.scaled_dot_product_attention(q, k, v)


def attention_gqa_ref(q, k, v, causal=False):
    """SDPA reference for GQA (reference attention.py:611-619)."""
    k, v = _expand_kv(q, k, v)
    return F.scaled_dot_product_attention(q, k, v, is_causal=causal)


def attention_swa_ref(q, k, v, slide_size):
    """Causal sliding-window reference (reference attention.py:622-642): query i attends to
    key j iff j <= i and i - j < slide_size. Builds an (N, N) mask: small N only."""
    k, v = _expand_kv(q, k, v)
    n = q.shape[2]
    idx = torch.arange(n, device=q.device)
    attend = (idx[None, :] <= idx[:, None]) & ((idx[:, None] - idx[None, :]) < slide_size)
    mask = torch.where(attend, 0.0, float("-inf")).to(q.dtype)[None, None]
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
