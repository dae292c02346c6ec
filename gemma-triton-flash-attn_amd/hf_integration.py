"""HuggingFace transformers integration: one call swaps every attention layer.

Mirrors /root/reference/flash_attn/hf_integration.py:30-99. ``register_triton_attention``
adds ``triton_gqa_attention`` to transformers' attention registry under ``name``
(default ``"triton_gqa"``, the reference's name, kept so existing configs keep working);
then ``model.config._attn_implementation = name`` routes every layer through the gfx950
kernels.

Differences from the reference adapter:
  * ``scaling`` is passed to the kernels natively instead of pre-multiplying q
    (reference 55-58), which removes a full-size copy per call;
  * the output is allocated with q's strides, so for transformers' transposed
    (B, H, N, D) views of (B, N, H, D) projections the final ``transpose(1, 2)`` is
    already contiguous and ``.contiguous()`` does not copy (reference 75);
  * the call goes through the registered ``gfa::attn_fwd`` op (``ops.py``), so a model
    under ``torch.compile`` keeps one graph across its attention layers. The op launches on
    its tensors' device itself, which replaces the reference's ``torch.cuda.device`` guard
    (68-74).
"""
from __future__ import annotations

import torch

from .ops import flash_attn_gqa_op


def triton_gqa_attention(module, query, key, value, attention_mask, dropout: float = 0.0,
                         scaling: float | None = None, softcap: float | None = None,
                         sliding_window: int | None = None, **kwargs):
    """transformers attention-interface adapter: returns ``(out[B, N, Hq, D], None)``.

    ``attention_mask`` is ignored: the kernels build the causal / sliding-window mask from
    ``module.is_causal`` and ``sliding_window`` (reference 30-76). softcap and non-zero
    dropout raise NotImplementedError rather than return wrong numerics.
    """
    if softcap is not None:
        raise NotImplementedError("triton_gqa_attention does not support softcap")
    if dropout != 0.0:
        raise NotImplementedError("triton_gqa_attention does not support dropout")
    scale = scaling if scaling is not None else module.head_dim ** -0.5
    slide = int(sliding_window) if sliding_window else 0
    is_causal = getattr(module, "is_causal", True)
    out = flash_attn_gqa_op(query, key, value, causal=is_causal, slide_size=slide, scale=scale)
    return out.transpose(1, 2).contiguous(), None


def register_triton_attention(name: str = "triton_gqa") -> None:
    """Register ``triton_gqa_attention`` under ``name`` in transformers' global attention
    registry (reference 79-88)."""
    from transformers import AttentionInterface

    AttentionInterface.register(name, triton_gqa_attention)


def patch_transformers_5_5_4_flash_attn_key() -> None:
    """Work around transformers 5.5.4's ``KeyError: 'flash_attn'`` on config load
    (reference 91-99). Idempotent; harmless on other versions."""
    try:
        from transformers.utils.import_utils import PACKAGE_DISTRIBUTION_MAPPING
    except ImportError:
        return
    PACKAGE_DISTRIBUTION_MAPPING.setdefault("flash_attn", ["flash-attn"])


def patch_gemma4_shared_kv_states_for_fsdp2() -> bool:
    """The reference re-implements Gemma4TextModel.forward for FSDP2 on transformers 5.5.4
    (reference 102-229). Newer transformers already keep shared KV states in a mapping
    FSDP2 can traverse, and multi-GPU training is outside this single-GPU engine.

    Returns False (nothing patched) when the installed transformers does not need it;
    raises NotImplementedError on 5.5.x.
    """
    import transformers

    if transformers.__version__.startswith("5.5."):
        raise NotImplementedError("FSDP2 shared-KV patch for transformers 5.5.x is not provided")
    return False
