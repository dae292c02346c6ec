"""Row R5 (the HEAD_DIM-keyed registry) on the CPU.

1. The oracle's restatement of the reference's Triton tile selection reproduces the
   reference's own known-answer table (context/baseline.md:1582-1592) and its forward /
   dQ defaults (attention.py:1444-1451, 1498-1504).
2. The engine's registry, which replaces those tables with gfx950 tiles, gives fixed
   known answers on the BASELINE shapes: a change of the rule shows up here.
"""
from __future__ import annotations

import pytest

import gemma_triton_flash_attn_amd as gfa
from oracle import reference_registry as rr

# context/baseline.md:1582-1592: (config, Hkv, N) -> (BKV, QS, grid), D=256 (the D<512
# branch), B=1. Config A has H_KV=16, config B H_KV=1.
KNOWN = [
    (16, 1024, 64, 1, 256),
    (16, 2048, 64, 1, 512),
    (16, 4096, 64, 1, 1024),
    (1, 1024, 64, 8, 128),    # "rescue": tiny grid takes the big tile and QS=8
    (1, 2048, 32, 4, 256),
    (1, 4096, 32, 2, 256),
    (1, 8192, 64, 1, 128),
]


@pytest.mark.parametrize("Hkv,N,bkv,qs,grid", KNOWN)
def test_reference_dkv_selection_known_answers(Hkv, N, bkv, qs, grid):
    t = rr.dkv_tiles(1, Hkv, N, 256)
    assert (t["BLOCK_KV"], t["Q_SPLITS"], t["grid"]) == (bkv, qs, grid)


@pytest.mark.parametrize("Hkv,N", [(4, 1024), (4, 8192), (2, 32768), (1, 4096)])
def test_reference_dkv_d512_row(Hkv, N):
    """'D=512 any | 16 | 1': BKV = 16 and no Q split at the reference's D=512 shapes."""
    t = rr.dkv_tiles(1, Hkv, N, 512)
    assert (t["BLOCK_KV"], t["BLOCK_Q"], t["num_warps"], t["Q_SPLITS"]) == (16, 64, 4, 1)


def test_reference_forward_and_dq_defaults():
    assert rr.forward_tiles(16384, 512) == {"BLOCK_Q": 64, "BLOCK_KV": 32, "num_warps": 8, "num_stages": 2}
    assert rr.forward_tiles(16384, 256) == {"BLOCK_Q": 128, "BLOCK_KV": 64, "num_warps": 8, "num_stages": 2}
    assert rr.forward_tiles(40, 256)["BLOCK_Q"] == 64 and rr.forward_tiles(40, 256)["BLOCK_KV"] == 64
    assert rr.dq_tiles(16384, 512) == {"BLOCK_Q": 32, "BLOCK_KV": 64, "num_warps": 8}
    assert rr.dq_tiles(16384, 256) == {"BLOCK_Q": 64, "BLOCK_KV": 64, "num_warps": 4}
    # below D=256 the reference forward drops to 4 warps (attention.py:1448)
    assert rr.forward_tiles(4096, 128) == {"BLOCK_Q": 128, "BLOCK_KV": 64, "num_warps": 4, "num_stages": 2}
    assert rr.forward_tiles(4096, 64)["num_warps"] == 4
    assert rr.dq_tiles(4096, 128) == {"BLOCK_Q": 64, "BLOCK_KV": 64, "num_warps": 4}


# The engine's registry on the BASELINE shapes (B, Hq, Hkv, N, D) -> chosen tiles.
ENGINE_KNOWN = {
    (1, 32, 4, 16384, 512): dict(fwd_block_q=32, fwd_block_kv=32, dq_block_q=32, dkv_block_kv=64, dkv_block_q=32,
                                 q_splits=1),
    (1, 32, 4, 8192, 512): dict(fwd_block_q=32, fwd_block_kv=32, dq_block_q=32, dkv_block_kv=64, dkv_block_q=32,
                                q_splits=1),   # 512-workgroup key grid: two rounds of one per CU
    (1, 16, 2, 32768, 512): dict(fwd_block_q=32, fwd_block_kv=32, dq_block_q=32, dkv_block_kv=64, dkv_block_q=32,
                                 q_splits=1),
    (1, 16, 8, 16384, 256): dict(fwd_block_q=64, fwd_block_kv=32, dq_block_q=64, dkv_block_kv=128, dkv_block_q=32,
                                 q_splits=1),
    (1, 32, 4, 1024, 512): dict(fwd_block_q=32, fwd_block_kv=32, dq_block_q=32, dkv_block_kv=64, dkv_block_q=32,
                                q_splits=8),
    # group size 8 packs 4 heads x 1 query block per forward / dQ workgroup; the 16-workgroup
    # key grid needs the largest query split
    (1, 8, 1, 2048, 256): dict(fwd_block_q=32, fwd_block_kv=32, dq_block_q=32, dkv_block_kv=128, dkv_block_q=32,
                               q_splits=8),
    # D=128 / D=64 (the rest of the reference's documented head-dim range): 64-key forward
    # tiles; dK/dV on role-split pairs (64 keys per workgroup) at D=128, one wave per 32 keys
    # at D=64
    (1, 32, 8, 16384, 128): dict(fwd_block_q=32, fwd_block_kv=64, dq_block_q=32, dkv_block_kv=64, dkv_block_q=32,
                                 q_splits=1),
    (1, 8, 1, 4096, 128): dict(fwd_block_q=32, fwd_block_kv=64, dq_block_q=32, dkv_block_kv=64, dkv_block_q=32,
                               q_splits=8),
    (1, 32, 32, 4096, 64): dict(fwd_block_q=128, fwd_block_kv=64, dq_block_q=128, dkv_block_kv=128, dkv_block_q=32,
                                q_splits=1),
}


@pytest.mark.parametrize("shape", list(ENGINE_KNOWN))
def test_engine_registry_known_answers(shape):
    cfg = gfa.get_config(*shape)
    for key, want in ENGINE_KNOWN[shape].items():
        assert cfg[key] == want, (key, cfg[key], want)


def test_query_split_rule_by_mask_kind():
    """Full-causal key grids ask for two rounds of workgroups (unequal work per key block),
    windowed and non-causal ones for one; D=128 / D=64 keep two dK/dV workgroups per CU."""
    from gemma_triton_flash_attn_amd.registry import q_splits_for_problem as qs

    # D=256 16:8 N=4096: a 256-workgroup key grid
    assert qs(1, 8, 4096, 256, causal=True, window=0) == 2
    assert qs(1, 8, 4096, 256, causal=True, window=1024) == 1
    assert qs(1, 8, 4096, 256, causal=False) == 1
    assert qs(1, 8, 4096, 256, causal=True, window=4096) == 2  # a window covering N is plain causal
    # D=128 8:1 N=16384 W=1024: 256 workgroups, two per CU -> one round needs 512
    assert qs(1, 1, 16384, 128, causal=True, window=1024) == 2
    # D=64 16:2 N=8192: 128 workgroups of 128 keys; full causal asks for 2 x 256 x 2
    assert qs(1, 2, 8192, 64, causal=True) == 8
    assert qs(1, 4, 8192, 64, causal=True, window=1024) == 2


def test_windowed_forward_tile():
    """With a sliding window the D=128 forward runs 32-key tiles (less waste at the window
    edge); the other head dims keep their default."""
    from gemma_triton_flash_attn_amd.registry import REGISTRY

    assert REGISTRY[128].fwd_block_kv_window == 32
    assert all(REGISTRY[d].fwd_block_kv_window in (0, REGISTRY[d].fwd_block_kv) for d in (64, 256, 512))
    assert all(c.fwd_block_kv_window in (0,) + tuple(c.fwd_block_kv_options) for c in REGISTRY.values())

