"""Pins the oracle (oracle/attention_oracle.py) before anything is compared against it.

Checks, chosen so that a dropped term, a wrong sign/index or a transposed operand fails:
  * torch scaled_dot_product_attention (math backend, float64) and its autograd - an
    independent library implementation - on causal / sliding-window / full GQA cases;
  * the committed golden vectors (written by that library path);
  * finite differences of sum(O * dO) on tiny inputs;
  * closed forms: Q = 0 -> prefix / window means with LSE = ln |allowed|, window 1 ->
    O = V, N = 1, GQA == MHA on repeated K/V, shift invariance in K, convex rows,
    Q = 0 -> dV_j = sum_{i sees j} dO_i / |allowed(i)|;
  * the chunked torch fp32 variant against the float64 one.
"""
from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from oracle import attention_oracle as orc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")

CASES = [
    # B, Hq, Hkv, N, D, causal, window
    (1, 2, 2, 9, 4, False, 0),
    (2, 4, 2, 13, 8, True, 0),
    (1, 6, 2, 17, 8, True, 5),
    (1, 8, 1, 11, 16, True, 1),
    (1, 4, 4, 7, 4, True, 0),
    (1, 2, 1, 12, 8, True, 64),  # window >= N -> plain causal
]


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def _sdpa64(q, k, v, do, causal, window):
    q, k, v, do = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v, do))
    r = q.shape[1] // k.shape[1]
    ke, ve = k.repeat_interleave(r, 1), v.repeat_interleave(r, 1)
    n = q.shape[2]
    i = torch.arange(n)[:, None]
    j = torch.arange(n)[None, :]
    m = torch.ones(n, n, dtype=torch.bool)
    if causal:
        m &= j <= i
        if window and window < n:
            m &= (i - j) < window
    with sdpa_kernel(SDPBackend.MATH):
        o = F.scaled_dot_product_attention(q, ke, ve, attn_mask=torch.zeros(n, n, dtype=torch.float64)
                                           .masked_fill(~m, float("-inf"))[None, None])
    (o * do.detach()).sum().backward()
    return o.detach().numpy(), q.grad.numpy(), k.grad.numpy(), v.grad.numpy()


@pytest.mark.parametrize("B,Hq,Hkv,N,D,causal,window", CASES)
def test_oracle_matches_torch_sdpa_fwd_bwd(B, Hq, Hkv, N, D, causal, window):
    q, k, v, do = (_rand(s, i) for i, s in enumerate([(B, Hq, N, D), (B, Hkv, N, D), (B, Hkv, N, D), (B, Hq, N, D)]))
    o_ref, dq_ref, dk_ref, dv_ref = _sdpa64(q, k, v, do, causal, window)
    o, _ = orc.forward(q, k, v, causal, window)
    dq, dk, dv, delta = orc.backward(q, k, v, do, causal, window)
    np.testing.assert_allclose(o, o_ref, atol=1e-12, rtol=1e-10)
    np.testing.assert_allclose(dq, dq_ref, atol=1e-11, rtol=1e-9)
    np.testing.assert_allclose(dk, dk_ref, atol=1e-11, rtol=1e-9)
    np.testing.assert_allclose(dv, dv_ref, atol=1e-11, rtol=1e-9)
    np.testing.assert_allclose(delta, (do * o_ref).sum(-1), atol=1e-12)


def _bits_to_f32(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))))
def test_oracle_matches_golden(path):
    z = np.load(path)
    B, Hq, Hkv, N, D, causal, window = (int(x) for x in z["meta"])
    q, k, v, do = (_bits_to_f32(z[n]) for n in ("q", "k", "v", "do"))
    o, lse = orc.forward(q, k, v, bool(causal), window)
    dq, dk, dv, _ = orc.backward(q, k, v, do, bool(causal), window)
    np.testing.assert_allclose(o, z["o"], atol=2e-6, rtol=1e-5)
    np.testing.assert_allclose(lse, z["lse"], atol=2e-5, rtol=1e-5)
    for got, name in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        np.testing.assert_allclose(got, z[name], atol=2e-5, rtol=1e-4)


def test_finite_differences():
    B, Hq, Hkv, N, D = 1, 4, 2, 6, 3
    q, k, v, do = (_rand(s, 10 + i) for i, s in enumerate([(B, Hq, N, D), (B, Hkv, N, D), (B, Hkv, N, D), (B, Hq, N, D)]))
    for causal, window in ((True, 0), (True, 2), (False, 0)):
        dq, dk, dv, _ = orc.backward(q, k, v, do, causal, window)

        def loss(qq, kk, vv):
            return float((orc.forward(qq, kk, vv, causal, window)[0] * do).sum())

        eps = 1e-6
        for arr, grad, which in ((q, dq, 0), (k, dk, 1), (v, dv, 2)):
            for idx in [(0, 0, 0, 0), (0, 1, 3, 2), (0, arr.shape[1] - 1, N - 1, 1)]:
                xp = [q.copy(), k.copy(), v.copy()]
                xm = [q.copy(), k.copy(), v.copy()]
                xp[which][idx] += eps
                xm[which][idx] -= eps
                fd = (loss(*xp) - loss(*xm)) / (2 * eps)
                assert abs(fd - grad[idx]) < 1e-6, (causal, window, which, idx, fd, grad[idx])


@pytest.mark.parametrize("causal,window", [(True, 0), (True, 3), (False, 0)])
def test_zero_query_gives_means(causal, window):
    B, Hq, Hkv, N, D = 1, 4, 2, 10, 5
    q = np.zeros((B, Hq, N, D))
    k = _rand((B, Hkv, N, D), 1)
    v = _rand((B, Hkv, N, D), 2)
    o, lse = orc.forward(q, k, v, causal, window)
    for h in range(Hq):
        g = h // 2
        for i in range(N):
            if causal:
                lo = max(0, i - window + 1) if window else 0
                js = range(lo, i + 1)
            else:
                js = range(N)
            js = list(js)
            np.testing.assert_allclose(o[0, h, i], v[0, g, js].mean(0), atol=1e-12)
            assert abs(lse[0, h, i] - np.log(len(js))) < 1e-12
    # Backward closed form at Q = 0: P is uniform over the allowed set.
    do = _rand((B, Hq, N, D), 3)
    _, _, dv, _ = orc.backward(q, k, v, do, causal, window)
    mask = orc.allowed_mask(N, causal, window)
    cnt = mask.sum(1)
    expect = np.zeros((B, Hkv, N, D))
    for h in range(Hq):
        expect[0, h // 2] += (mask / cnt[:, None]).T @ do[0, h]
    np.testing.assert_allclose(dv, expect, atol=1e-12)


def test_window_one_and_single_row():
    k = _rand((1, 2, 8, 4), 4)
    v = _rand((1, 2, 8, 4), 5)
    q = _rand((1, 2, 8, 4), 6)
    o, _ = orc.forward(q, k, v, True, 1)
    np.testing.assert_allclose(o, v, atol=1e-12)
    o1, lse1 = orc.forward(q[:, :, :1], k[:, :, :1], v[:, :, :1], True, 0)
    np.testing.assert_allclose(o1, v[:, :, :1], atol=1e-12)


def test_gqa_equals_mha_on_repeated_kv_and_shift_invariance():
    q = _rand((1, 8, 12, 6), 7)
    k = _rand((1, 2, 12, 6), 8)
    v = _rand((1, 2, 12, 6), 9)
    o, lse = orc.forward(q, k, v, True, 5)
    o2, lse2 = orc.forward(q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1), True, 5)
    np.testing.assert_allclose(o, o2, atol=1e-13)
    np.testing.assert_allclose(lse, lse2, atol=1e-13)
    # Adding the same vector c to every key shifts each row's scores by q.c: O unchanged.
    c = _rand((1, 1, 1, 6), 10)
    o3, _ = orc.forward(q, k + c, v, True, 5)
    np.testing.assert_allclose(o, o3, atol=1e-12)
    # Rows are convex combinations of visible values.
    assert (o <= v.max(axis=2, keepdims=True).repeat(4, axis=1) + 1e-12).all()
    assert (o >= v.min(axis=2, keepdims=True).repeat(4, axis=1) - 1e-12).all()


def test_one_hot_selects_value():
    n = 6
    k = np.zeros((1, 1, n, n))
    k[0, 0] = np.eye(n) * 200.0  # key j is e_j scaled
    q = np.zeros((1, 1, n, n))
    q[0, 0, :, 2] = 1.0  # every query points at key 2 (visible from query 2 on)
    v = _rand((1, 1, n, n), 11)
    o, _ = orc.forward(q, k, v, False, 0)
    np.testing.assert_allclose(o[0, 0], np.repeat(v[0, 0, 2:3], n, axis=0), atol=1e-12)


@pytest.mark.parametrize("causal,window", [(True, 0), (True, 6), (False, 0)])
def test_chunked_matches_dense(causal, window):
    B, Hq, Hkv, N, D = 1, 4, 2, 37, 8
    q, k, v, do = (_rand(s, 20 + i) for i, s in enumerate([(B, Hq, N, D), (B, Hkv, N, D), (B, Hkv, N, D), (B, Hq, N, D)]))
    o, lse = orc.forward(q, k, v, causal, window)
    dq, dk, dv, delta = orc.backward(q, k, v, do, causal, window)
    tq, tk, tv, tdo = (torch.tensor(x, dtype=torch.float32) for x in (q, k, v, do))
    o2, lse2 = orc.forward_chunked(tq, tk, tv, causal, window, chunk=8)
    dq2, dk2, dv2, delta2 = orc.backward_chunked(tq, tk, tv, tdo, causal, window, chunk=8)
    for a, b in ((o, o2), (lse, lse2), (dq, dq2), (dk, dk2), (dv, dv2), (delta, delta2)):
        np.testing.assert_allclose(b.numpy(), a, atol=2e-5, rtol=1e-4)


@pytest.mark.parametrize("causal,window,segmented", [(True, 0, False), (True, 6, True), (False, 0, False),
                                                     (False, 0, True)])
def test_chunked_dropout_matches_dense(causal, window, segmented):
    """The chunked torch path with dropout (the large-size check on the GPU box) equals the dense
    float64 path, which test_dropout_matches_torch_autograd pins to torch autograd: same mask
    rows per chunk (a wrong row offset or head index in the chunked mask fails), same scaling,
    undropped LSE; also together with a packed segment table."""
    B, Hq, Hkv, N, D = 2, 4, 2, 37, 8
    q, k, v, do = (_rand(s, 40 + i) for i, s in enumerate([(B, Hq, N, D), (B, Hkv, N, D), (B, Hkv, N, D), (B, Hq, N, D)]))
    drop = (0.3, 0x0123_4567_89AB_CDEF)
    segs = None
    if segmented:
        lo = np.array([[0] * 10 + [10] * 20 + list(range(30, 37)), [0] * 37])
        hi = np.array([[10] * 10 + [30] * 20 + list(range(30, 37)), [37] * 37])
        segs = (lo, hi)
    o, lse = orc.forward(q, k, v, causal, window, segments=segs, dropout=drop)
    dq, dk, dv, delta = orc.backward(q, k, v, do, causal, window, segments=segs, dropout=drop)
    tq, tk, tv, tdo = (torch.tensor(x, dtype=torch.float32) for x in (q, k, v, do))
    tsegs = None if segs is None else tuple(torch.tensor(x) for x in segs)
    o2, lse2 = orc.forward_chunked(tq, tk, tv, causal, window, chunk=8, segments=tsegs, dropout=drop)
    dq2, dk2, dv2, delta2 = orc.backward_chunked(tq, tk, tv, tdo, causal, window, chunk=8, segments=tsegs,
                                                 dropout=drop)
    for a, b in ((o, o2), (lse, lse2), (dq, dq2), (dk, dk2), (dv, dv2), (delta, delta2)):
        np.testing.assert_allclose(b.numpy(), a, atol=2e-5, rtol=1e-4)
    # the undropped result is far away (the mask is applied)
    o0, _ = orc.forward(q, k, v, causal, window, segments=segs)
    assert np.abs(o0 - o).max() > 0.1


def test_chunked_dropout_mask_equals_dense_mask():
    """``dropout_mask_rows`` (int64 torch arithmetic) equals the numpy uint32 mask entry for entry,
    for every row slice, including seeds and heads that exercise the high mixer bits."""
    for seed, bh, n, p in ((7, 3, 300, 0.1), (0xFFFF_FFFF_FFFF_FFFF, 1000, 129, 0.5), (1 << 40, 0, 64, 0.9)):
        dense = orc.dropout_mask(seed, bh, n, p)
        for lo, hi in ((0, n), (5, 37), (n - 1, n)):
            np.testing.assert_array_equal(orc.dropout_mask_rows(seed, bh, lo, hi, n, p).numpy(), dense[lo:hi])


@pytest.mark.parametrize("causal,window", [(True, 0), (True, 7), (True, 1), (False, 0), (True, 64)])
def test_cpu_baseline_restatement_matches_oracle(causal, window):
    """The function the reported CPU baseline times (oracle/cpu_baseline.py sdpa_math_gqa,
    the reference's attention_gqa_ref / attention_swa_ref path) computes the same attention
    as the float64 oracle: GQA expansion, causal and sliding-window masks. A wrong head
    mapping, a window off by one or a dropped causal flag fails here."""
    from oracle.cpu_baseline import sdpa_math_gqa

    B, Hq, Hkv, N, D = 2, 8, 2, 29, 16
    q, k, v = (_rand(s, 40 + i) for i, s in enumerate([(B, Hq, N, D), (B, Hkv, N, D), (B, Hkv, N, D)]))
    got = sdpa_math_gqa(*(torch.tensor(x, dtype=torch.float32) for x in (q, k, v)), causal=causal, window=window)
    ref, _ = orc.forward(q, k, v, causal, window)
    assert got.shape == ref.shape
    assert float(np.abs(got.double().numpy() - ref).max()) < 2e-5


def _hf_eager64(q, k, v, do, causal, window, softcap):
    """transformers' eager attention (the Gemma-2 implementation, which soft-caps the scaled
    scores before the mask) in float64, with torch autograd for the gradients."""
    from types import SimpleNamespace

    from transformers.models.gemma2.modeling_gemma2 import eager_attention_forward

    q, k, v = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    n, d = q.shape[2], q.shape[3]
    mask = torch.tensor(orc.allowed_mask(n, causal, window))
    add = torch.zeros(n, n, dtype=torch.float64).masked_fill(~mask, float("-inf"))[None, None]
    module = SimpleNamespace(num_key_value_groups=q.shape[1] // k.shape[1], training=False, head_dim=d)
    o, _ = eager_attention_forward(module, q, k, v, add, dropout=0.0, scaling=d ** -0.5, softcap=softcap)
    o = o.transpose(1, 2)  # the function returns (B, N, H, D)
    (o * torch.tensor(do)).sum().backward()
    return o.detach().numpy(), q.grad.numpy(), k.grad.numpy(), v.grad.numpy()


@pytest.mark.parametrize("B,Hq,Hkv,N,D,causal,window,cap", [
    (1, 4, 2, 13, 8, True, 0, 5.0), (2, 6, 2, 17, 8, True, 5, 2.0), (1, 2, 2, 9, 4, False, 0, 0.7),
    (1, 8, 1, 11, 16, True, 64, 30.0)])
def test_softcap_matches_transformers_eager(B, Hq, Hkv, N, D, causal, window, cap):
    """Soft-capped scores (not in the reference; transformers' Gemma-2 eager attention is the
    independent implementation): forward and float64 autograd gradients. Scores are scaled up
    so that the cap bends them (a dropped tanh or a missing 1 - tanh^2 factor fails)."""
    q, k, v, do = (_rand(s, 60 + i) * (3.0 if i < 2 else 1.0)
                   for i, s in enumerate([(B, Hq, N, D), (B, Hkv, N, D), (B, Hkv, N, D), (B, Hq, N, D)]))
    o_ref, dq_ref, dk_ref, dv_ref = _hf_eager64(q, k, v, do, causal, window, cap)
    o, _ = orc.forward(q, k, v, causal, window, softcap=cap)
    dq, dk, dv, _ = orc.backward(q, k, v, do, causal, window, softcap=cap)
    # transformers runs its softmax in float32 whatever the input dtype: float32-level agreement
    for a, r in ((o, o_ref), (dq, dq_ref), (dk, dk_ref), (dv, dv_ref)):
        np.testing.assert_allclose(a, r, atol=2e-6, rtol=1e-4)
    # the cap changes the result at these score magnitudes (the check above is not vacuous)
    o_nocap, _ = orc.forward(q, k, v, causal, window)
    assert float(np.abs(o_nocap - o).max()) > 1e-3


def test_softcap_chunked_matches_dense_and_large_cap_is_no_cap():
    B, Hq, Hkv, N, D = 1, 4, 2, 37, 8
    q, k, v, do = (_rand(s, 80 + i) * (3.0 if i < 2 else 1.0)
                   for i, s in enumerate([(B, Hq, N, D), (B, Hkv, N, D), (B, Hkv, N, D), (B, Hq, N, D)]))
    for causal, window in ((True, 0), (True, 6), (False, 0)):
        o, lse = orc.forward(q, k, v, causal, window, softcap=4.0)
        dq, dk, dv, delta = orc.backward(q, k, v, do, causal, window, softcap=4.0)
        tq, tk, tv, tdo = (torch.tensor(x, dtype=torch.float32) for x in (q, k, v, do))
        o2, lse2 = orc.forward_chunked(tq, tk, tv, causal, window, chunk=8, softcap=4.0)
        dq2, dk2, dv2, delta2 = orc.backward_chunked(tq, tk, tv, tdo, causal, window, chunk=8, softcap=4.0)
        for a, b in ((o, o2), (lse, lse2), (dq, dq2), (dk, dk2), (dv, dv2), (delta, delta2)):
            np.testing.assert_allclose(b.numpy(), a, atol=5e-5, rtol=1e-4)
    # tanh(z / c) * c -> z as c grows
    o_big, _ = orc.forward(q, k, v, True, 0, softcap=1e7)
    o_none, _ = orc.forward(q, k, v, True, 0)
    np.testing.assert_allclose(o_big, o_none, atol=1e-9)


def _drop_torch64(q, k, v, do, causal, window, p, seed):
    """float64 torch autograd through softmax(S) * M / (1 - p) @ V with the oracle's mask."""
    q, k, v = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    B, Hq, n, d = q.shape
    r = Hq // k.shape[1]
    ke, ve = k.repeat_interleave(r, 1), v.repeat_interleave(r, 1)
    allowed = torch.tensor(orc.allowed_mask(n, causal, window))
    s = (q @ ke.transpose(-1, -2)) * d ** -0.5
    pr = torch.softmax(s.masked_fill(~allowed, float("-inf")), dim=-1)
    keep = torch.tensor(np.stack([np.stack([orc.dropout_mask(seed, b * Hq + h, n, p) for h in range(Hq)])
                                  for b in range(B)]))
    o = (pr * keep / (1.0 - float(np.float32(p)))) @ ve
    (o * torch.tensor(do)).sum().backward()
    return o.detach().numpy(), q.grad.numpy(), k.grad.numpy(), v.grad.numpy()


@pytest.mark.parametrize("B,Hq,Hkv,N,D,causal,window,p", [
    (1, 4, 2, 13, 8, True, 0, 0.25), (2, 6, 2, 17, 8, True, 5, 0.5), (1, 2, 2, 9, 4, False, 0, 0.1)])
def test_dropout_matches_torch_autograd(B, Hq, Hkv, N, D, causal, window, p):
    """Dropout (not in the reference): the oracle's forward and gradients equal float64 torch
    autograd through the same mask, the LSE is the undropped one, and p = 0 is no dropout."""
    q, k, v, do = (_rand(s, 90 + i) for i, s in enumerate([(B, Hq, N, D), (B, Hkv, N, D), (B, Hkv, N, D),
                                                           (B, Hq, N, D)]))
    seed = 0x1234_5678_9ABC_DEF0
    o_ref, dq_ref, dk_ref, dv_ref = _drop_torch64(q, k, v, do, causal, window, p, seed)
    o, lse = orc.forward(q, k, v, causal, window, dropout=(p, seed))
    dq, dk, dv, _ = orc.backward(q, k, v, do, causal, window, dropout=(p, seed))
    for a, r in ((o, o_ref), (dq, dq_ref), (dk, dk_ref), (dv, dv_ref)):
        np.testing.assert_allclose(a, r, atol=1e-10, rtol=1e-9)
    _, lse0 = orc.forward(q, k, v, causal, window)
    np.testing.assert_allclose(lse, lse0, atol=1e-12)
    o0, _ = orc.forward(q, k, v, causal, window, dropout=(0.0, seed))
    np.testing.assert_allclose(o0, orc.forward(q, k, v, causal, window)[0], atol=0)


def test_dropout_mask_rate_and_independence():
    """Keep rate 1 - p (to a few standard errors), per row and per column alike; different
    heads and seeds give different masks."""
    n = 512
    for p in (0.1, 0.5):
        m = orc.dropout_mask(7, 3, n, p)
        rate = m.mean()
        assert abs(rate - (1 - p)) < 4 * np.sqrt(p * (1 - p) / m.size)
        rows, cols = m.mean(axis=1), m.mean(axis=0)
        tol = 6 * np.sqrt(p * (1 - p) / n)
        assert np.abs(rows - (1 - p)).max() < tol and np.abs(cols - (1 - p)).max() < tol
    a = orc.dropout_mask(7, 3, 256, 0.5)
    assert (a != orc.dropout_mask(7, 4, 256, 0.5)).mean() > 0.4
    assert (a != orc.dropout_mask(8, 3, 256, 0.5)).mean() > 0.4
    assert (a != orc.dropout_mask(7 + (1 << 32), 3, 256, 0.5)).mean() > 0.4
