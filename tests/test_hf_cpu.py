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


def test_padding_mask_reaches_the_adapter_and_becomes_segments():
    """transformers drops a 2-D padding mask for attention functions without a mask creator.
    register_triton_attention installs one, so a padded batch hands the adapter its padding
    mask (and an unpadded one hands over None); the adapter turns it, packed cu_seq_lens and
    restarting position ids into segment tables, and refuses what a table cannot express."""
    from types import SimpleNamespace

    from transformers import AttentionInterface

    import gemma_triton_flash_attn_amd as gfa
    from gemma_triton_flash_attn_amd.hf_integration import _segments_for

    seen = []

    def probe(module, query, key, value, attention_mask, **kwargs):
        seen.append(None if attention_mask is None else attention_mask.clone())
        o = torch.zeros(query.shape[0], query.shape[2], query.shape[1], query.shape[3], dtype=query.dtype)
        return o, None

    gfa.register_triton_attention("gfa_mask_probe")
    AttentionInterface.register("gfa_mask_probe", probe)  # same name: keeps the engine's mask creator
    cfg = tiny_gemma4_config(n_layers=2, sliding_window=8)
    model = build_model(cfg, "cpu", torch.float32)
    ids = torch.randint(0, cfg.vocab_size, (2, 24), generator=torch.Generator().manual_seed(2))
    pad = torch.ones(2, 24, dtype=torch.long)
    pad[1, 18:] = 0
    model.config._attn_implementation = "gfa_mask_probe"
    for m in model.modules():
        c = getattr(m, "config", None)
        if c is not None and hasattr(c, "_attn_implementation"):
            c._attn_implementation = "gfa_mask_probe"
    with torch.no_grad():
        model(input_ids=ids, attention_mask=pad, use_cache=False)
    assert len(seen) == 2 and all(s is not None and s.shape == (2, 24) for s in seen)
    assert torch.equal(seen[0].to(torch.long), pad)
    seen.clear()
    with torch.no_grad():
        model(input_ids=ids, attention_mask=torch.ones(2, 24, dtype=torch.long), use_cache=False)
    assert seen == [None, None]

    q = torch.zeros(2, 2, 24, 256)
    lo, hi = _segments_for(q, pad.bool(), {})
    assert lo[1].tolist() == [0] * 18 + list(range(18, 24)) and hi[1].tolist() == [18] * 18 + list(range(18, 24))
    assert lo[0].tolist() == [0] * 24 and hi[0].tolist() == [24] * 24
    assert _segments_for(q, None, {"position_ids": torch.arange(24)[None]}) is None
    q1 = q[:1]
    lo, hi = _segments_for(q1, None, {"cu_seq_lens_q": torch.tensor([0, 10, 24]), "cu_seq_lens_k": torch.tensor([0, 10, 24])})
    assert lo.tolist() == [[0] * 10 + [10] * 14] and hi.tolist() == [[10] * 10 + [24] * 14]
    pos = torch.cat([torch.arange(10), torch.arange(14)])[None]
    plo, phi = _segments_for(q1, None, {"position_ids": pos})
    assert torch.equal(plo, lo) and torch.equal(phi, hi)
    mod = SimpleNamespace(head_dim=256, is_causal=True)
    with pytest.raises(NotImplementedError, match="4-D"):
        gfa.triton_gqa_attention(mod, q, q, q, torch.ones(2, 1, 24, 24, dtype=torch.bool))
    holes = torch.ones(2, 24, dtype=torch.bool)
    holes[0, 5] = False
    with pytest.raises(NotImplementedError, match="contiguous"):
        gfa.triton_gqa_attention(mod, q, q, q, holes)
    with pytest.raises(NotImplementedError, match="cu_seq_lens"):
        gfa.triton_gqa_attention(mod, q1, q1, q1, None, cu_seq_lens_q=torch.tensor([0, 10, 24]))
