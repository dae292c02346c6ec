"""Math reference helpers kept from the reference's public API.

``attention_gqa_ref`` and ``attention_swa_ref`` restate
/root/reference/flash_attn/attention.py:611-619 and 622-642: GQA by repeating each KV head
over its query group, scale 1/sqrt(D), causal / sliding-window masks, evaluated with
torch's scaled_dot_product_attention. They are what a user compares the engine against;
no engine entry point calls them.
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
