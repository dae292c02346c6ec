"""The torch.library registration (ops.py) on the CPU, with fake tensors: the ops exist, their
fake implementations give the shapes, dtypes and layouts the kernels write, and autograd
through ``flash_attn_gqa_op`` reaches ``gfa::attn_bwd`` with the saved tensors. No kernel
is launched (the GPU side is tests/test_gpu_ops.py)."""
from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import gemma_triton_flash_attn_amd as gfa
from gemma_triton_flash_attn_amd.attention import lse_ld


def test_ops_registered():
    assert hasattr(torch.ops.gfa, "attn_fwd") and hasattr(torch.ops.gfa, "attn_bwd")
    s = str(torch.ops.gfa.attn_fwd.default._schema)
    assert "bool causal, SymInt window, float scale" in s or "bool causal, int window, float scale" in s


@pytest.mark.parametrize("layout", ["bhnd", "bnhd"])
def test_fake_shapes_and_layouts(layout):
    with FakeTensorMode():
        if layout == "bhnd":
            q = torch.empty(2, 8, 100, 256, device="cuda", dtype=torch.bfloat16)
        else:  # transformers' (B, H, N, D) view of (B, N, H, D) storage
            q = torch.empty(2, 100, 8, 256, device="cuda", dtype=torch.bfloat16).transpose(1, 2)
        k = torch.empty(2, 2, 100, 256, device="cuda", dtype=torch.bfloat16)
        o, lse, seed = torch.ops.gfa.attn_fwd(q, k, k, True, 0, 0.0625)
        assert o.shape == q.shape and o.dtype == q.dtype and o.stride() == q.stride()
        assert lse.shape == (2, 8, lse_ld(100)) and lse.dtype == torch.float32
        # the dropout seed travels as a one-element int64 CPU tensor (no device sync to read it)
        assert seed.shape == (1,) and seed.dtype == torch.int64 and seed.device.type == "cpu"
        dq, dk, dv = torch.ops.gfa.attn_bwd(q, k, k, o, lse, o, True, 0, 0.0625)
        assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == k.shape
        assert dq.stride() == q.stride()


def test_fake_out_of_rule_layout_is_contiguous():
    """An input layout the ABI cannot write (row stride not a multiple of 8 elements) gets a
    contiguous output, as in the eager path."""
    with FakeTensorMode():
        base = torch.empty(1, 4, 64, 260, device="cuda", dtype=torch.float16)
        q = base[..., :256]
        k = torch.empty(1, 1, 64, 256, device="cuda", dtype=torch.float16)
        o, _, _ = torch.ops.gfa.attn_fwd(q, k, k, False, 0, 0.0625)
        assert o.is_contiguous()


def test_autograd_registration_and_formula():
    """The op has an Autograd kernel, and its backward formula turns the saved tensors into
    gfa::attn_bwd outputs of the input shapes (called directly: the autograd engine itself
    needs a device to run fake CUDA tensors)."""
    from types import SimpleNamespace

    from gemma_triton_flash_attn_amd.ops import _attn_fwd_backward

    assert torch._C._dispatch_has_kernel_for_dispatch_key("gfa::attn_fwd", "Autograd")

    def ctx_of(o, lse, seg, seed, softcap=0.0, dropout_p=0.0):
        return SimpleNamespace(saved_tensors=(q, k, k, o, lse, seg, seg, seed), causal=True, window=16, scale=0.04,
                               softcap=softcap, dropout_p=dropout_p)

    with FakeTensorMode():
        q = torch.empty(1, 8, 64, 512, device="cuda", dtype=torch.bfloat16)
        k = torch.empty(1, 1, 64, 512, device="cuda", dtype=torch.bfloat16)
        o, lse, seed = torch.ops.gfa.attn_fwd(q, k, k, True, 16, 0.04)
        grads = _attn_fwd_backward(ctx_of(o, lse, None, seed), torch.empty_like(o), None, None)
        assert len(grads) == 10 and grads[3:] == (None,) * 7
        assert grads[0].shape == q.shape and grads[1].shape == k.shape and grads[2].shape == k.shape
        # with a segment table (ragged batch): the same formula, the tables passed through
        lo = torch.empty(1, 64, device="cuda", dtype=torch.int32)
        o2, lse2, seed2 = torch.ops.gfa.attn_fwd(q, k, k, True, 16, 0.04, lo, lo)
        grads = _attn_fwd_backward(ctx_of(o2, lse2, lo, seed2), torch.empty_like(o2), None, None)
        assert len(grads) == 10 and grads[0].shape == q.shape
        # soft-capped: the cap reaches the backward op
        o3, lse3, seed3 = torch.ops.gfa.attn_fwd(q, k, k, True, 16, 0.04, None, None, 30.0)
        grads = _attn_fwd_backward(ctx_of(o3, lse3, None, seed3, softcap=30.0), torch.empty_like(o3), None, None)
        assert len(grads) == 10 and grads[0].shape == q.shape
        # dropout: the probability and the seed the forward drew reach the backward op
        o4, lse4, seed4 = torch.ops.gfa.attn_fwd(q, k, k, True, 16, 0.04, None, None, 0.0, 0.1)
        grads = _attn_fwd_backward(ctx_of(o4, lse4, None, seed4, dropout_p=0.1), torch.empty_like(o4), None, None)
        assert len(grads) == 10 and grads[0].shape == q.shape


def test_softcap_with_dropout_raises_not_implemented():
    """No kernel instance combines soft-capping with dropout: every entry point raises the
    adapter contract's NotImplementedError before anything is launched (the inputs here are CPU
    tensors, so reaching the device checks would raise ValueError instead)."""
    from types import SimpleNamespace

    from gemma_triton_flash_attn_amd.attention import _check_cap_and_dropout

    with pytest.raises(NotImplementedError, match="softcap"):
        _check_cap_and_dropout(30.0, 0.1)
    _check_cap_and_dropout(30.0, 0.0)
    _check_cap_and_dropout(0.0, 0.1)
    with FakeTensorMode():
        q = torch.empty(1, 8, 64, 256, device="cuda", dtype=torch.bfloat16)
        k = torch.empty(1, 2, 64, 256, device="cuda", dtype=torch.bfloat16)
        with pytest.raises(NotImplementedError, match="softcap"):
            gfa.flash_attn_gqa_op(q, k, k, causal=True, softcap=30.0, dropout_p=0.1)
        with pytest.raises(NotImplementedError, match="softcap"):
            gfa.flash_attn_gqa_train(q, k, k, causal=True, softcap=30.0, dropout_p=0.1)
        mod = SimpleNamespace(head_dim=256, is_causal=True)
        with pytest.raises(NotImplementedError, match="softcap"):
            gfa.triton_gqa_attention(mod, q, k, k, None, dropout=0.1, scaling=0.0625, softcap=30.0)


def test_op_entry_validates_like_the_eager_api():
    q = torch.zeros(1, 8, 16, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensors"):
        gfa.flash_attn_gqa_op(q, q[:, :1], q[:, :1], causal=True)
    with pytest.raises(ValueError, match="multiple"):
        gfa.flash_attn_gqa_op(q, q[:, :3], q[:, :3])
    with pytest.raises(Exception, match="head_dim|HEAD_DIM|registry|supported"):
        z = torch.zeros(1, 8, 16, 96, dtype=torch.bfloat16)
        gfa.flash_attn_gqa_op(z, z[:, :1], z[:, :1])
