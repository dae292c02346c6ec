"""Small random-init Gemma-4 text models for the HuggingFace integration tests, and an
attention function for transformers' registry that computes the same op with the oracle's
float32 torch path (the reference the engine is compared against inside a model)."""
from __future__ import annotations

import torch

from oracle import attention_oracle as orc


def tiny_gemma4_config(n_layers: int = 4, sliding_window: int = 64):
    """Gemma-4 text architecture at toy width: GQA 8:1, sliding layers with head dim 256,
    full-attention layers with head dim 512 (the layer pattern of the E2B family)."""
    from transformers import Gemma4TextConfig

    types = ["full_attention" if (i + 1) % 4 == 0 else "sliding_attention" for i in range(n_layers)]
    types[-1] = "full_attention"
    return Gemma4TextConfig(vocab_size=1024, hidden_size=256, intermediate_size=512, num_hidden_layers=n_layers,
                            num_attention_heads=8, num_key_value_heads=1, head_dim=256, global_head_dim=512,
                            sliding_window=sliding_window, vocab_size_per_layer_input=1024,
                            hidden_size_per_layer_input=64, layer_types=types, max_position_embeddings=8192)


class CallLog:
    def __init__(self):
        self.calls = []


def make_oracle_attention(log: CallLog | None = None):
    """transformers attention interface computing attention with the oracle's chunked
    float32 path; same argument contract as ``triton_gqa_attention``."""

    def oracle_attention(module, query, key, value, attention_mask, dropout=0.0, scaling=None, softcap=None,
                         sliding_window=None, **kwargs):
        scale = scaling if scaling is not None else module.head_dim ** -0.5
        window = int(sliding_window) if sliding_window else 0
        causal = getattr(module, "is_causal", True)
        if log is not None:
            log.calls.append((query.shape[-1], window, float(scale)))
        o, _ = orc.forward_chunked(query, key, value, causal, window, scale)
        return o.to(query.dtype).transpose(1, 2).contiguous(), None

    return oracle_attention


def build_model(config, device, dtype, seed: int = 0):
    from transformers import Gemma4ForCausalLM

    torch.manual_seed(seed)
    with torch.device(device):
        model = Gemma4ForCausalLM(config)
    return model.to(dtype).eval()


def logits_with(model, name: str, ids):
    model.config._attn_implementation = name
    for m in model.modules():
        cfg = getattr(m, "config", None)
        if cfg is not None and hasattr(cfg, "_attn_implementation"):
            cfg._attn_implementation = name
    with torch.no_grad():
        return model(input_ids=ids).logits.float()
