"""HuggingFace plumbing on the CPU (no kernel launch): a Gemma-4 text model routes every
decoder layer's attention through the name registered in transformers' attention registry,
with the head dims, sliding windows and scaling the engine's adapter relies on.

The registered function here is the oracle-backed reference from hf_models.py; the
engine's own adapter is exercised on the GPU (test_gpu_hf.py).
"""
from __future__ import annotations

import pytest
import torch

transformers = pytest.importorskip("transformers")

from hf_models import CallLog, build_model, logits_with, make_oracle_attention, tiny_gemma4_config  # noqa: E402


def test_every_layer_dispatches_through_the_registered_name():
    from transformers import AttentionInterface

    log = CallLog()
    AttentionInterface.register("gfa_oracle_cpu", make_oracle_attention(log))
    cfg = tiny_gemma4_config(n_layers=4, sliding_window=16)
    model = build_model(cfg, "cpu", torch.float32)
    ids = torch.randint(0, cfg.vocab_size, (1, 40), generator=torch.Generator().manual_seed(0))
    out = logits_with(model, "gfa_oracle_cpu", ids)
    assert out.shape == (1, 40, cfg.vocab_size) and torch.isfinite(out).all()
    assert len(log.calls) == cfg.num_hidden_layers
    dims = [c[0] for c in log.calls]
    windows = [c[1] for c in log.calls]
    assert dims == [256, 256, 256, 512]          # sliding layers D=256, full layer D=512
    assert windows == [16, 16, 16, 0]
    assert all(c[2] == 1.0 for c in log.calls)   # Gemma-4 normalises q/k; scaling = 1


def test_oracle_attention_matches_sdpa_inside_the_model():
    """The oracle-backed interface and transformers' own SDPA give the same logits (fp32,
    CPU), so it is a valid in-model reference for the GPU comparison."""
    from transformers import AttentionInterface

    AttentionInterface.register("gfa_oracle_cpu2", make_oracle_attention())
    cfg = tiny_gemma4_config(n_layers=4, sliding_window=16)
    model = build_model(cfg, "cpu", torch.float32)
    ids = torch.randint(0, cfg.vocab_size, (1, 48), generator=torch.Generator().manual_seed(1))
    a = logits_with(model, "gfa_oracle_cpu2", ids)
    b = logits_with(model, "sdpa", ids)
    assert float((a - b).abs().max()) < 1e-3
