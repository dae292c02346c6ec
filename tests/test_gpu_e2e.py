"""Config 5 at its full size: the random-init Gemma-4-E2B-architecture model of
bench_e2e_config.json (35 layers, bf16) at N=16384, every attention layer on this engine
through the one-call HF registration.

During the engine forward, the q/k/v that transformers hands to the attention function of
the first and last sliding-window layers (head dim 256, window 512) and of the first and
last full-causal layers (head dim 512) are captured together with the engine's output for
them. Each captured call is then recomputed by the oracle's query-chunked float32 path at
the full N and compared in the reference's terms (tests/gemma4_integration/
test_adapter.py:131-175 and 188: cosine similarity > 0.999, relative error < 0.05) and at
the north-star bar for bf16 outputs, 2e-2, applied element by element as
|O - O_ref| <= 2e-2 * max(1, |O_ref|): absolute for outputs of unit size and relative above.
The bar is defined on N(0,1) synthetic inputs, whose outputs stay near unit size. This
model's attention is nearly one-hot (Gemma-4 passes scaling = 1 on unit-RMS q and k, so
the scores have a standard deviation near sqrt(D) = 16-23), so an output row is close to a
single V row and reaches |O| ~ 5, where one bf16 rounding step of the output alone is
0.016-0.03. The model's logits must be finite.
"""
from __future__ import annotations

import json
import os

import pytest
import torch

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")

from hf_models import build_model  # noqa: E402
from oracle import attention_oracle as orc  # noqa: E402

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
N = 16384
O_TOL_BF16 = 2e-2


def _cos_rel(a, b):
    a, b = a.float().flatten(), b.float().flatten()
    cos = float(torch.nn.functional.cosine_similarity(a, b, dim=0))
    rel = float(torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(b))
    return cos, rel


def test_config5_model_at_full_size(device):
    import gemma_triton_flash_attn_amd as gfa
    from transformers import AttentionInterface, Gemma4TextConfig

    with open(os.path.join(ROOT, "bench_e2e_config.json")) as f:
        cfg = Gemma4TextConfig(**json.load(f)["gemma4_text_config"])
    types = list(cfg.layer_types)
    sliding = [i for i, t in enumerate(types) if t == "sliding_attention"]
    full = [i for i, t in enumerate(types) if t == "full_attention"]
    want = {sliding[0], sliding[-1], full[0], full[-1]}
    print(f"case config-5 model, {len(types)} layers, N={N}, capturing layers {sorted(want)}", flush=True)

    gfa.register_triton_attention()
    captured = {}

    def capturing(module, query, key, value, attention_mask, **kwargs):
        out, w = gfa.triton_gqa_attention(module, query, key, value, attention_mask, **kwargs)
        if module.layer_idx in want:
            captured[module.layer_idx] = (query.detach().clone(), key.detach().clone(), value.detach().clone(),
                                          kwargs.get("scaling"), kwargs.get("sliding_window"),
                                          getattr(module, "is_causal", True), out.detach().clone())
        return out, w

    AttentionInterface.register("gfa_e2e_capture", capturing)
    model = build_model(cfg, device, torch.bfloat16)
    for m in model.modules():
        c = getattr(m, "config", None)
        if c is not None and hasattr(c, "_attn_implementation"):
            c._attn_implementation = "gfa_e2e_capture"
    ids = torch.randint(0, cfg.vocab_size, (1, N), generator=torch.Generator().manual_seed(0)).to(device)
    with torch.no_grad():
        logits = model(input_ids=ids, use_cache=False).logits
    torch.cuda.synchronize()
    assert logits.shape == (1, N, cfg.vocab_size)
    finite = all(bool(torch.isfinite(logits[0, lo:lo + 1024]).all()) for lo in range(0, N, 1024))
    print(f"  logits {tuple(logits.shape)} finite={finite}", flush=True)
    assert finite
    del logits, model
    torch.cuda.empty_cache()

    assert set(captured) == want
    for idx in sorted(want):
        q, k, v, scale, window, causal, out = captured[idx]
        D = q.shape[-1]
        exp_d = 512 if types[idx] == "full_attention" else 256
        assert D == exp_d and q.shape[2] == N
        assert (window or 0) == (cfg.sliding_window if types[idx] == "sliding_attention" else 0)
        ref, _ = orc.forward_chunked(q, k, v, causal, int(window or 0), scale)
        ref = ref.transpose(1, 2)  # the adapter returns (B, N, H, D)
        diff = (out.float() - ref).abs()
        err = float(diff.max())
        worst = float((diff / ref.abs().clamp(min=1.0)).max())
        cos, rel = _cos_rel(out, ref)
        print(f"  layer {idx} ({types[idx]}, D={D}, window={window}, scale={scale}): O max-abs {err:.3e} "
              f"(max |O_ref| {float(ref.abs().max()):.2f}), max |dO| / max(1, |O_ref|) {worst:.3e}, "
              f"cos {cos:.6f} rel {rel:.3e}", flush=True)
        assert worst <= O_TOL_BF16
        assert cos > 0.999 and rel < 0.05
        del ref
