"""Training through the engine, in the terms of the reference's training test
(/root/reference/tests/gemma4_integration/test_training.py:180-205): the same model, from
the same weights and batches, trained with the engine's attention and with a reference
attention, must give a step-0 loss within 0.05 nats and a loss trajectory within 0.5 nats
per step.

Offline differences: a random-init Gemma-4 text model (GQA 8:1, sliding D=256 and full
D=512 layers) replaces ``from_pretrained("google/gemma-4-E2B")``, synthetic token batches
replace wikitext, and the reference attention is the oracle's fp32 path (autograd through
torch) instead of SDPA."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")

from hf_models import build_model, make_oracle_attention, tiny_gemma4_config  # noqa: E402


def _train(attn_name, cfg, device, batches, steps):
    model = build_model(cfg, device, torch.bfloat16, seed=0).train()
    model.config._attn_implementation = attn_name
    for m in model.modules():
        c = getattr(m, "config", None)
        if c is not None and hasattr(c, "_attn_implementation"):
            c._attn_implementation = attn_name
    opt = torch.optim.AdamW(model.parameters(), lr=3e-4)
    losses = []
    for step in range(steps):
        ids = batches[step]
        out = model(input_ids=ids, labels=ids)
        losses.append(float(out.loss.detach()))
        out.loss.backward()
        opt.step()
        opt.zero_grad(set_to_none=True)
    return losses


def test_training_trajectory_matches_reference_attention(device):
    import gemma_triton_flash_attn_amd as gfa
    from transformers import AttentionInterface

    print("case training: tiny gemma4, 4 layers, B=2, N=256, 8 AdamW steps", flush=True)
    gfa.register_triton_attention()
    AttentionInterface.register("gfa_oracle_train", make_oracle_attention())
    cfg = tiny_gemma4_config(n_layers=4, sliding_window=64)
    g = torch.Generator().manual_seed(7)
    steps = 8
    batches = [torch.randint(0, cfg.vocab_size, (2, 256), generator=g).to(device) for _ in range(steps)]
    ref = _train("gfa_oracle_train", cfg, device, batches, steps)
    got = _train("triton_gqa", cfg, device, batches, steps)
    diffs = [abs(a - b) for a, b in zip(ref, got)]
    print(f"  reference losses {[round(x, 4) for x in ref]}", flush=True)
    print(f"  engine    losses {[round(x, 4) for x in got]}", flush=True)
    print(f"  step-0 diff {diffs[0]:.4f}, max diff {max(diffs):.4f}", flush=True)
    assert all(torch.isfinite(torch.tensor(got)))
    assert diffs[0] < 0.05
    assert max(diffs) < 0.5
