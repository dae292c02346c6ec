"""gemma-triton-flash-attn_amd: MI355X (gfx950) GQA flash attention for Gemma4-style models.

Drop-in for zzhhjjj/gemma-triton-flash-attn's public API (reference flash_attn/__init__.py),
computed by hand-written HIP kernels behind a C ABI (include/gfa.h, libgfa.so):

    attention_flash_gqa(q, k, v, causal=False, slide_size=0) -> out      inference forward
    flash_attn_gqa_train(q, k, v, causal=False, slide_size=0) -> out     autograd forward
    FlashAttnGQAFunction                                                 the autograd function
    flash_attn_gqa_op(q, k, v, causal=False, slide_size=0) -> out        same, as torch.library
                                                                         ops gfa::attn_fwd/bwd
                                                                         (torch.compile-able)
    attention(q, k, v)                                                   torch SDPA (reference helper)
    attention_gqa_ref / attention_swa_ref                                torch math references
    register_triton_attention(name="triton_gqa"), triton_gqa_attention   HF integration
    REGISTRY / get_config                                                HEAD_DIM-keyed configs
    segments.from_padding_mask / from_lengths / from_cu_seqlens / from_position_ids
                                                                         ragged-batch tables
                                                                         (``segments=`` keyword)

q: (B, N_Q_HEADS, N, D), k/v: (B, N_KV_HEADS, N, D), fp16/bf16, D in {64, 128, 256, 512}.
"""
from .attention import FlashAttnGQAFunction, attention_flash_gqa, flash_attn_gqa_train
from . import segments
from .ops import flash_attn_gqa_op
from .hf_integration import (
    patch_gemma4_shared_kv_states_for_fsdp2,
    patch_transformers_5_5_4_flash_attn_key,
    register_triton_attention,
    triton_gqa_attention,
)
from .reference import attention, attention_gqa_ref, attention_swa_ref
from .registry import REGISTRY, SUPPORTED_HEAD_DIMS, KernelConfig, get_config

__version__ = "1.0.1"

__all__ = [
    "attention_flash_gqa",
    "flash_attn_gqa_train",
    "FlashAttnGQAFunction",
    "flash_attn_gqa_op",
    "attention_gqa_ref",
    "attention_swa_ref",
    "attention",
    "register_triton_attention",
    "triton_gqa_attention",
    "patch_transformers_5_5_4_flash_attn_key",
    "patch_gemma4_shared_kv_states_for_fsdp2",
    "REGISTRY",
    "SUPPORTED_HEAD_DIMS",
    "KernelConfig",
    "get_config",
    "segments",
    "__version__",
]
