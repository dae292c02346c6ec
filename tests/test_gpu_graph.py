"""HIP-graph capture of the engine (torch.cuda.CUDAGraph on ROCm): the library never
allocates, frees, synchronises or memsets, and launches on the caller's stream, so a
forward, and a forward+backward, can be captured once and replayed. Every replay (with
the program's own eager work and synchronisations in between, and new input values copied
into the static buffers) must equal the eager result bitwise."""
from __future__ import annotations

import pytest
import torch

from conftest import make_inputs

pytestmark = pytest.mark.gpu


def _capture(fn, warmup_stream):
    with torch.cuda.stream(warmup_stream):  # warm up (allocator pools, lazy init) off the capture
        fn()
    torch.cuda.current_stream().wait_stream(warmup_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


# The last case's D=512 forward and dQ grids (512 and 1024 blocks) exceed the CU count, so they
# run persistent: each captured launch records the kernel that zeroes its work-queue counters.
@pytest.mark.parametrize("D,window,q_splits,shape", [(512, 0, 0, (1, 8, 2, 192)), (256, 40, 0, (1, 8, 2, 192)),
                                                     (256, 0, 4, (1, 8, 2, 192)), (128, 0, 2, (1, 8, 2, 192)),
                                                     (64, 17, 0, (1, 8, 2, 192)), (512, 0, 0, (1, 16, 2, 4096))])
def test_graph_replay_matches_eager(D, window, q_splits, shape, device):
    import gemma_triton_flash_attn_amd as gfa
    from gemma_triton_flash_attn_amd.attention import _backward, _forward

    B, Hq, Hkv, N = shape
    print(f"case graph D={D} window={window} q_splits={q_splits} B={B} Hq={Hq} Hkv={Hkv} N={N}", flush=True)
    sc = D ** -0.5
    static = [t.clone() for t in make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=11)]
    sq, sk, sv, sdo = static

    def infer():
        return gfa.attention_flash_gqa(sq, sk, sv, causal=True, slide_size=window)

    def train():
        o, lse = _forward(sq, sk, sv, True, window, sc, True)
        dq, dk, dv, _ = _backward(sq, sk, sv, o, lse, sdo, True, window, sc, q_splits=q_splits)
        return o, dq, dk, dv

    side = torch.cuda.Stream()
    g_inf, out_inf = _capture(infer, side)
    g_trn, out_trn = _capture(train, side)
    for rep in range(3):
        fresh = make_inputs(B, Hq, Hkv, N, D, torch.bfloat16, device, seed=100 + rep)
        for dst, src in zip(static, fresh):
            dst.copy_(src)
        g_inf.replay()
        g_trn.replay()
        torch.cuda.synchronize()
        ref_inf = gfa.attention_flash_gqa(*fresh[:3], causal=True, slide_size=window)
        o, lse = _forward(*fresh[:3], True, window, sc, True)
        ref_trn = (o,) + _backward(*fresh[:3], o, lse, fresh[3], True, window, sc, q_splits=q_splits)[:3]
        torch.cuda.synchronize()
        assert torch.equal(out_inf, ref_inf), f"inference replay {rep}"
        for name, a, b in zip(("O", "dQ", "dK", "dV"), out_trn, ref_trn):
            assert torch.equal(a, b), f"{name} replay {rep}"
