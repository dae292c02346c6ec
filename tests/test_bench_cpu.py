"""bench.py's measurement arithmetic, on the CPU.

The FLOP charge follows the reference's convention (benchmarks/run_final_benchmark.py:217-224:
causal fwd 2*B*Hq*N^2*D, fwd+bwd 7*B*Hq*N^2*D; the window-adjusted pair count
P = W(W+1)/2 + W(N-W) of benchmarks/profile_swa.py:51-55 for sliding windows). The expected
values are worked out independently here (closed forms and brute-force pair counts), so a
dropped factor or a wrong pair count in bench.py fails.
"""
from __future__ import annotations

import numpy as np
import pytest

import bench


def _pairs_brute(N, W):
    i = np.arange(N)[:, None]
    j = np.arange(N)[None, :]
    m = j <= i
    if W:
        m &= (i - j) < W
    return int(m.sum())


@pytest.mark.parametrize("name,fwd_tf,fb_tf", [
    ("d512_causal_gqa8_n16k", 8.796, 30.786),     # headline: 2*32*16384^2*512
    ("c2_d512_causal_gqa8_n8k", 2.199, 7.697),
    ("c4_d512_causal_gqa8_n32k", 17.592, 61.573),
    ("d256_swa1024_gqa2_n16k", 0.2663, 0.9320),   # P = 16,253,440 attended pairs per head
])
def test_charged_flops_match_the_reference_convention(name, fwd_tf, fb_tf):
    w = bench.WORKLOADS[name]
    assert bench.charged_flops(w, "fwd") / 1e12 == pytest.approx(fwd_tf, rel=2e-4)
    assert bench.charged_flops(w, "fwdbwd") / 1e12 == pytest.approx(fb_tf, rel=2e-4)
    assert bench.charged_flops(w, "fwdbwd") / bench.charged_flops(w, "fwd") == pytest.approx(3.5)


@pytest.mark.parametrize("N,W", [(64, 7), (300, 32), (1000, 999), (513, 1)])
def test_window_pair_count_is_the_brute_force_count(N, W):
    w = dict(B=1, Hq=1, Hkv=1, N=N, D=1, causal=True, window=W)
    # 4 * D * P for the forward: the brute-force number of (query, key) pairs times 4
    assert bench.charged_flops(w, "fwd") == 4 * _pairs_brute(N, W)


def test_causal_convention_counts_half_the_square():
    w = dict(B=2, Hq=3, Hkv=1, N=40, D=8, causal=True, window=0)
    assert bench.charged_flops(w, "fwd") == 2 * 2 * 3 * 40 * 40 * 8   # N^2/2 pairs x 4D
    w_nc = dict(w, causal=False)
    assert bench.charged_flops(w_nc, "fwd") == 2 * bench.charged_flops(w, "fwd")


def test_kernel_flops_split_by_products():
    w = bench.WORKLOADS["d512_causal_gqa8_n16k"]
    kf = bench.kernel_flops(w)
    fwd = bench.charged_flops(w, "fwd")
    assert kf["fwd"] == fwd                   # S and PV
    assert kf["dq"] == 1.5 * fwd              # S, dP, dQ
    assert kf["dkv"] == 2 * fwd               # S, dP, dV, dK
    # The fwd+bwd charge counts 7 products (forward 2, backward S, dP, dV, dK, dQ). The two
    # backward kernels both compute S and dP, so the kernels do 2 products (one forward's
    # worth) more than the charge.
    assert kf["fwd"] + kf["dq"] + kf["dkv"] == pytest.approx(bench.charged_flops(w, "fwdbwd") + fwd)


def test_kernel_bytes_at_the_headline():
    w = bench.WORKLOADS["d512_causal_gqa8_n16k"]
    kb = bench.kernel_bytes(w)
    q = 32 * 16384 * 512 * 2          # Q, O, dO, dQ
    kv = 4 * 16384 * 512 * 2          # K, V, dK, dV
    rows = 32 * 16384 * 4             # LSE, delta
    assert kb == {"fwd": 2 * q + 2 * kv + rows, "dq": 4 * q + 2 * kv + 2 * rows, "dkv": 2 * q + 4 * kv + 2 * rows}
    assert kb["fwd"] == 1_210_056_704


def test_more_than_one_gpu_is_refused_before_touching_a_gpu(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "single-GPU" in capsys.readouterr().err
