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
    (68-74);
  * padded and packed batches are computed, not ignored (the reference adapter drops
    ``attention_mask``, 43-47): a padding mask, ``cu_seq_lens_*`` or restarting
    ``position_ids`` become segment tables (segments.py) for the kernels.
"""
from __future__ import annotations

import torch

from . import segments as seglib
from .ops import flash_attn_gqa_op


def _segments_for(query, attention_mask, kwargs):
    """Segment tables for the batch described by the adapter's arguments, or None.

    * ``attention_mask``: the (B, N) padding mask handed over by ``padding_mask_for_engine``
      (None when nothing is padded); its real tokens must be one run per row;
    * ``cu_seq_lens_q`` / ``cu_seq_lens_k`` (transformers' packed-sequence keyword
      arguments): one row of packed sequences;
    * ``position_ids`` that restart inside a row (packing without a mask, which transformers
      detects the same way).
    Anything else the kernels cannot express raises NotImplementedError.

    Under torch.compile nothing here reads device values on the host (such a read would break
    the graph): the cu_seq_lens equality check is skipped, and position ids always become a
    table. For ids without a restart that table is one segment per row, so the results equal the
    eager path's, which passes no table then."""
    B, _, N, _ = query.shape
    host = seglib._host_checks()
    cu_q, cu_k = kwargs.get("cu_seq_lens_q"), kwargs.get("cu_seq_lens_k")
    if cu_q is not None or cu_k is not None:
        if cu_q is None or cu_k is None or (host and not torch.equal(cu_q.to(cu_k.device), cu_k)):
            raise NotImplementedError("packed sequences need equal cu_seq_lens_q and cu_seq_lens_k")
        if B != 1:
            raise NotImplementedError("packed sequences (cu_seq_lens) are one row of tokens")
        return seglib.from_cu_seqlens(cu_q.to(query.device), N)
    if attention_mask is not None:
        if attention_mask.dim() != 2:
            raise NotImplementedError("triton_gqa_attention takes padding masks, not prepared 4-D attention masks")
        if tuple(attention_mask.shape) != (B, N):
            raise NotImplementedError(f"padding mask {tuple(attention_mask.shape)} does not match (B, N) = {(B, N)}")
        try:
            return seglib.from_padding_mask(attention_mask.to(query.device))
        except ValueError as e:
            raise NotImplementedError(str(e)) from None
    pos = kwargs.get("position_ids")
    if pos is not None and pos.dim() == 2 and pos.shape[-1] == N and (not host or seglib.is_packed(pos)):
        return seglib.from_position_ids(pos.to(query.device).expand(B, N))
    return None


def triton_gqa_attention(module, query, key, value, attention_mask, dropout: float = 0.0,
                         scaling: float | None = None, softcap: float | None = None,
                         sliding_window: int | None = None, **kwargs):
    """transformers attention-interface adapter: returns ``(out[B, N, Hq, D], None)``.

    The kernels build the causal / sliding-window mask from ``module.is_causal`` and
    ``sliding_window`` (reference 30-76). ``attention_mask`` is what the mask creator
    registered beside this function hands over: None when no token is padded, else the
    (B, N) padding mask, which becomes a segment table, as do packed sequences
    (``cu_seq_lens_*`` or restarting ``position_ids``). Padding tokens' output rows are zero
    (as with transformers' flash-attention path, which drops them). ``softcap`` (Gemma-2's
    attention logit soft-capping) and ``dropout`` (the probability the model passes in
    training, 0 in eval) run natively; the reference adapter raises for both. A prepared 4-D
    mask raises NotImplementedError: never wrong numerics.
    """
    segments = _segments_for(query, attention_mask, kwargs)
    scale = scaling if scaling is not None else module.head_dim ** -0.5
    slide = int(sliding_window) if sliding_window else 0
    is_causal = getattr(module, "is_causal", True)
    out = flash_attn_gqa_op(query, key, value, causal=is_causal, slide_size=slide, scale=scale, segments=segments,
                            softcap=softcap, dropout_p=float(dropout or 0.0))
    return out.transpose(1, 2).contiguous(), None


def padding_mask_for_engine(batch_size, q_length, kv_length, q_offset=0, kv_offset=0, mask_function=None,
                            attention_mask=None, **kwargs):
    """Mask creator registered under the same name as the attention function.

    transformers drops a 2-D padding mask for attention functions that have no mask creator
    of their own (masking_utils._preprocess_mask_arguments), which would make padded
    batches silently wrong. This one hands the adapter the (B, kv_length) boolean padding
    mask when any key is padded, and None otherwise (the kernels build the causal and
    window masks themselves). Under torch.compile the mask is handed over as it is (testing
    it would read a device value on the host); an unpadded mask becomes one segment per row,
    with the same results."""
    if attention_mask is None:
        return None
    m = attention_mask[:, -kv_length:]
    if m.shape[1] == kv_length and seglib._host_checks() and bool(m.all()):
        return None
    return m


def register_triton_attention(name: str = "triton_gqa") -> None:
    """Register ``triton_gqa_attention`` under ``name`` in transformers' global attention
    registry (reference 79-88), with ``padding_mask_for_engine`` as its mask creator."""
    from transformers import AttentionInterface

    AttentionInterface.register(name, triton_gqa_attention)
    try:
        from transformers.masking_utils import AttentionMaskInterface
    except ImportError:  # transformers without mask interfaces: masks reach the adapter as given
        return
    AttentionMaskInterface.register(name, padding_mask_for_engine)


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
