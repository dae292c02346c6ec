"""Run-time work distribution (gfa_set_runtime_scheduling): at head_dim 512 a forward or dQ grid
larger than one workgroup per CU runs as a persistent grid that takes its blocks from per-XCD
queues. Every block computes what it computes in the static grid, so the two launches must agree
bit for bit, and repeated persistent launches must agree with each other (the hand-out order
changes from run to run); dK/dV, which consume the dQ kernel's delta, check that hand-off too. The
shapes here are sized so that both static grids exceed the 256 CUs (one block per 32 or 64 query
rows of each head group), and cover the paths a block's body takes:
causal and not, a sliding window, GQA groups of 8 and 1, query splits, segment tables, dropout
and soft-capping. One case is also checked against the oracle's chunked float32 path.
"""
from __future__ import annotations

import pytest
import torch

from conftest import make_inputs, recomputing
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

CASES = {
    # name: B, Hq, Hkv, N, D, causal, window, extra (forward / dQ static grid sizes)
    "causal_gqa8": (2, 16, 2, 2048, 512, True, 0, {}),  # 512 / 1024
    "noncausal_mha_ragged": (1, 8, 8, 6000, 512, False, 0, {}),  # 376 / 752
    "window_gqa4": (1, 16, 4, 3000, 512, True, 700, {}),  # 376 / 752
    "causal_qsplit4": (1, 8, 1, 6144, 512, True, 0, {"q_splits": 4}),  # 384 / 768
    "segments": (2, 16, 2, 2048, 512, True, 0, {"segments": True}),  # 512 / 1024
    "dropout": (1, 16, 2, 4096, 512, True, 0, {"dropout_p": 0.2}),  # 512 / 1024
    "softcap_fp16": (1, 16, 2, 4096, 512, True, 0, {"softcap": 20.0, "dtype": torch.float16}),
}
SEED = 0x5C4ED


def _run(q, k, v, do, causal, window, extra):
    import gemma_triton_flash_attn_amd as gfa
    from gemma_triton_flash_attn_amd.attention import _backward, _forward

    segs = None
    if extra.get("segments"):
        B, _, N, _ = q.shape
        segs = gfa.segments.from_lengths([N - 300, N - 17][:B], N, left_padding=True, device=q.device)
    sc = q.shape[-1] ** -0.5
    kw = dict(segments=segs, softcap=extra.get("softcap", 0.0), dropout_p=extra.get("dropout_p", 0.0),
              dropout_seed=SEED)
    o, lse = _forward(q, k, v, causal, window, sc, store_lse=True, **kw)
    # the recomputing backward: its dQ kernel is the one with the run-time hand-out
    with recomputing():
        dq, dk, dv, delta = _backward(q, k, v, o, lse, do, causal, window, sc, q_splits=extra.get("q_splits", 0), **kw)
    torch.cuda.synchronize()
    return o, lse, dq, dk, dv, delta


@pytest.mark.parametrize("name", list(CASES))
def test_persistent_grid_matches_static_grid_bitwise(name, device):
    from gemma_triton_flash_attn_amd import _lib

    B, Hq, Hkv, N, D, causal, window, extra = CASES[name]
    dtype = extra.get("dtype", torch.bfloat16)
    print(f"case {name}: B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal} window={window} {extra}", flush=True)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, dtype, device, seed=N + Hq)
    prev = _lib.set_runtime_scheduling(False)
    try:
        static = _run(q, k, v, do, causal, window, extra)
        _lib.set_runtime_scheduling(True)
        dyn1 = _run(q, k, v, do, causal, window, extra)
        dyn2 = _run(q, k, v, do, causal, window, extra)
    finally:
        _lib.set_runtime_scheduling(prev)
    names = ("O", "LSE", "dQ", "dK", "dV", "delta")
    for nm, a, b, c in zip(names, static, dyn1, dyn2):
        if nm in ("LSE", "delta"):
            a, b, c = (x[..., :N] for x in (a, b, c))
        assert torch.equal(a, b), f"{nm}: persistent grid differs from the static grid"
        assert torch.equal(b, c), f"{nm}: two persistent launches differ"


def test_persistent_grid_vs_chunked_oracle(device):
    """The persistent path against the float32 reference (a D=512 GQA 8:1 causal case whose grids
    all run persistent)."""
    from gemma_triton_flash_attn_amd import _lib

    B, Hq, Hkv, N, D = 1, 16, 2, 4096, 512
    print(f"case persistent vs oracle: B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal", flush=True)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=41)
    prev = _lib.set_runtime_scheduling(True)
    try:
        o, lse, dq, dk, dv, _ = _run(q, k, v, do, True, 0, {})
    finally:
        _lib.set_runtime_scheduling(prev)
    o_ref, lse_ref = orc.forward_chunked(q, k, v, True, 0)
    dq_ref, dk_ref, dv_ref, _ = orc.backward_chunked(q, k, v, do, True, 0, o=o_ref, lse=lse_ref)
    rel = lambda a, b: float(torch.linalg.vector_norm(a.float() - b) / torch.linalg.vector_norm(b))  # noqa: E731
    err_o = float((o.float() - o_ref).abs().max())
    errs = (rel(dq, dq_ref), rel(dk, dk_ref), rel(dv, dv_ref))
    print(f"  O max-abs {err_o:.3e}  dQ/dK/dV rel {errs[0]:.3e} {errs[1]:.3e} {errs[2]:.3e}", flush=True)
    assert err_o <= 2e-2
    assert max(errs) <= 5e-2
    assert float((lse[..., :N] - lse_ref).abs().max()) <= 1e-2
