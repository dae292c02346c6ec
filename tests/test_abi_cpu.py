"""CPU checks of the C ABI boundary and the host-side API (no kernel is launched).

* libgfa.so loads and exports every entry point declared in include/gfa.h;
* the ctypes structs match the C layout (sizeof / offsetof from a gcc-compiled probe);
* gfa_config agrees with the Python registry;
* invalid arguments are rejected before any launch, with the documented status codes;
* the Python API raises on inputs the engine cannot take (no silent fallback).
"""
from __future__ import annotations

import ctypes
import os
import re
import shutil
import subprocess

import pytest
import torch

import gemma_triton_flash_attn_amd as gfa
from gemma_triton_flash_attn_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gfa.h")

# Tests that hand the library fake device addresses rely on host-side validation rejecting
# every case before a launch. They run only where no GPU is visible, so that a future
# validation regression cannot launch a kernel on those addresses.
fake_pointers = pytest.mark.skipif(torch.cuda.is_available(),
                                   reason="passes fake device pointers; runs only without a visible GPU")


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    text = open(HEADER).read()
    declared = sorted(set(re.findall(r"^\s*(?:int|int64_t|size_t|const char\*)\s+(gfa_\w+)\s*\(", text, re.M)))
    assert declared, "no declarations parsed"
    assert set(declared) == set(_lib.EXPORTED)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.gfa_version() == int(re.search(r"#define GFA_VERSION (\d+)", text).group(1))
    assert _lib.ABI_VERSION == lib.gfa_version()


def test_runtime_scheduling_switch():
    """gfa_set_runtime_scheduling returns the previous setting, a negative argument only queries,
    and the binding restores it (no kernel is launched)."""
    lib = _lib.load()
    before = lib.gfa_set_runtime_scheduling(-1)
    assert before in (0, 1)
    assert _lib.set_runtime_scheduling(False) == bool(before)
    assert lib.gfa_set_runtime_scheduling(-1) == 0
    assert _lib.set_runtime_scheduling(True) is False
    assert lib.gfa_set_runtime_scheduling(-1) == 1
    _lib.set_runtime_scheduling(bool(before))


def test_loader_refuses_a_library_of_another_abi_version(monkeypatch):
    """A libgfa.so whose GFA_VERSION differs from the layout the ctypes structs mirror would read
    another prefix of the argument structs; load() raises instead."""
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "ABI_VERSION", _lib.ABI_VERSION - 1)
    with pytest.raises(RuntimeError, match="GFA_VERSION"):
        _lib.load()
    monkeypatch.undo()
    assert _lib.load().gfa_version() == _lib.ABI_VERSION


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_struct_layout_matches_c(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(f'''
#include <stdio.h>
#include <stddef.h>
#include "{HEADER}"
int main(void) {{
  printf("%zu %zu %zu\\n", sizeof(gfa_fwd_args), sizeof(gfa_bwd_args), sizeof(gfa_config_info));
  printf("%zu %zu %zu %zu %zu %zu\\n", offsetof(gfa_fwd_args, lse_ld), offsetof(gfa_fwd_args, stream),
         offsetof(gfa_bwd_args, stages), offsetof(gfa_bwd_args, workspace_bytes),
         offsetof(gfa_fwd_args, softcap), offsetof(gfa_bwd_args, softcap));
  printf("%zu %zu\\n", offsetof(gfa_fwd_args, dropout_seed), offsetof(gfa_bwd_args, dropout_seed));
  return 0;
}}
''')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    sizes = [int(x) for x in out]
    assert sizes[:3] == [ctypes.sizeof(_lib.FwdArgs), ctypes.sizeof(_lib.BwdArgs), ctypes.sizeof(_lib.ConfigInfo)]
    assert sizes[3:] == [_lib.FwdArgs.lse_ld.offset, _lib.FwdArgs.stream.offset, _lib.BwdArgs.stages.offset,
                         _lib.BwdArgs.workspace_bytes.offset, _lib.FwdArgs.softcap.offset, _lib.BwdArgs.softcap.offset,
                         _lib.FwdArgs.dropout_seed.offset, _lib.BwdArgs.dropout_seed.offset]


@pytest.mark.parametrize("shape", [(1, 32, 4, 16384, 512), (1, 16, 8, 16384, 256), (2, 6, 3, 33, 256),
                                   (1, 4, 4, 1, 512), (1, 8, 1, 1024, 512), (3, 16, 2, 32768, 512),
                                   (1, 32, 8, 16384, 128), (2, 8, 1, 300, 128), (1, 32, 32, 4096, 64),
                                   (4, 12, 12, 77, 64)])
def test_config_matches_python_registry(shape):
    assert _lib.config(*shape) == gfa.get_config(*shape)


@pytest.mark.parametrize("D", [64, 128, 256, 512])
@pytest.mark.parametrize("B,Hkv,N", [(1, 8, 16384), (1, 1, 16384), (1, 8, 4096), (2, 2, 8192), (1, 1, 1024)])
@pytest.mark.parametrize("causal,window", [(True, 0), (True, 512), (True, 1024), (True, 1 << 20), (False, 0),
                                           (False, 512)])
def test_query_split_choice_matches_python_registry(D, B, Hkv, N, causal, window):
    """The library's split count (seen through the workspace it asks for) is the Python
    registry's, windowed dK/dV form included."""
    from gemma_triton_flash_attn_amd.registry import q_splits_for_problem

    qs = q_splits_for_problem(B, Hkv, N, D, causal, window)
    want = 0 if qs == 1 else qs * 2 * B * Hkv * N * D * 4
    assert _lib.bwd_workspace_size(B, 2 * Hkv, Hkv, N, D, causal, window) == want


def _fwd_args(**over):
    a = _lib.FwdArgs()
    a.q = a.k = a.v = a.o = 256  # fake, 16-byte aligned: validation happens before any launch
    a.lse = 512
    a.batch, a.heads_q, a.heads_kv, a.seq_len, a.head_dim = 1, 8, 2, 64, 512
    for s in ("q_strides", "k_strides", "v_strides", "o_strides"):
        setattr(a, s, _lib.Strides(8 * 64 * 512, 64 * 512, 512))
    a.causal, a.window, a.scale, a.dtype, a.lse_ld = 1, 0, 512 ** -0.5, _lib.GFA_DTYPE_BF16, 64
    for k, v in over.items():
        setattr(a, k, v)
    return a


@fake_pointers
@pytest.mark.parametrize("over,status", [
    (dict(head_dim=96), 2),               # not a power of two
    (dict(head_dim=32), 2),               # below the reference's documented 64-512
    (dict(head_dim=1024), 2),
    (dict(heads_q=6, heads_kv=4), 1),
    (dict(seq_len=0), 1),
    (dict(dtype=7), 1),
    (dict(window=-1), 1),
    (dict(q=260), 1),                     # misaligned pointer
    (dict(lse_ld=16), 1),                 # lse rows shorter than GFA_LSE_LD(N)
    (dict(scale=float("nan")), 1),
    (dict(scale=0.0), 1),                 # the kernels mask with -inf before scaling: scale > 0
    (dict(scale=-0.125), 1),
    (dict(block_kv=48), 2),               # no such forward tile
    (dict(softcap=float("nan")), 1),
    (dict(softcap=-1.0), 1),
    (dict(head_dim=256, block_kv=64, softcap=5.0), 2),  # soft-capping runs the default tiles only
    (dict(dropout_p=1.0), 1),
    (dict(dropout_p=-0.1), 1),
    (dict(dropout_p=0.1, softcap=5.0), 2),  # not built together
    (dict(k_strides=_lib.Strides(8, 8, 4)), 1),  # row stride not a multiple of 8 elements
])
def test_fwd_rejects_bad_arguments(over, status):
    lib = _lib.load()
    a = _fwd_args(**over)
    assert lib.gfa_fwd(ctypes.byref(a)) == status
    assert lib.gfa_last_error()
    assert lib.gfa_fwd(None) == 1


@fake_pointers
def test_bwd_rejects_bad_arguments():
    lib = _lib.load()
    a = _lib.BwdArgs()
    for name in ("q", "k", "v", "o", "dout", "dq", "dk", "dv"):
        setattr(a, name, 256)
    for s in ("q_strides", "k_strides", "v_strides", "o_strides", "do_strides", "dq_strides", "dk_strides",
              "dv_strides"):
        setattr(a, s, _lib.Strides(8 * 64 * 512, 64 * 512, 512))
    a.batch, a.heads_q, a.heads_kv, a.seq_len, a.head_dim = 1, 8, 1, 64, 512
    a.causal, a.scale, a.dtype = 1, 512 ** -0.5, _lib.GFA_DTYPE_BF16
    a.lse_ld = 64
    # lse / delta missing
    assert lib.gfa_bwd(ctypes.byref(a)) == 1
    a.lse, a.delta = 512, 1024
    a.stages = 4
    assert lib.gfa_bwd(ctypes.byref(a)) == 1
    a.stages = 0
    a.q_splits = 3
    assert lib.gfa_bwd(ctypes.byref(a)) == 1
    a.q_splits = 4  # needs a workspace
    assert lib.gfa_bwd(ctypes.byref(a)) == 3
    need = lib.gfa_bwd_workspace_size(1, 8, 1, 64, 512, 1, 0, 4)
    assert need == 4 * 2 * 1 * 1 * 64 * 512 * 4
    a.workspace, a.workspace_bytes = 4096, need - 1
    assert lib.gfa_bwd(ctypes.byref(a)) == 3
    a.workspace, a.workspace_bytes = 4096, need
    for bad in (0.0, -0.5, float("inf")):
        a.scale = bad
        assert lib.gfa_bwd(ctypes.byref(a)) == 1


def test_python_api_validation_needs_no_gpu():
    q = torch.randn(1, 4, 16, 256, dtype=torch.bfloat16)
    k = torch.randn(1, 2, 16, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensors"):
        gfa.flash_attn_gqa_train(q, k, k, causal=True)
    with pytest.raises(TypeError):
        gfa.attention_flash_gqa(q, k.float(), k, causal=True)
    for d in (96, 32):
        with pytest.raises(ValueError, match="head_dim"):
            gfa.attention_flash_gqa(q[..., :d], k[..., :d], k[..., :d])
    with pytest.raises(ValueError, match="multiple"):
        gfa.attention_flash_gqa(q[:, :3], k, k)


def test_attention_helper_is_reference_sdpa():
    """attention() is the reference's torch SDPA helper (reference attention.py:11-17):
    non-causal, any device / dtype / head dim, and differentiable."""
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(2, 3, 7, 24, generator=g, dtype=torch.float64, requires_grad=True) for _ in range(3))
    o = gfa.attention(q, k, v)
    s = (q @ k.transpose(-1, -2)) / 24 ** 0.5
    ref = torch.softmax(s, dim=-1) @ v
    assert torch.allclose(o, ref, atol=1e-12)
    o.sum().backward()
    assert q.grad is not None and k.grad is not None and v.grad is not None
    assert torch.isfinite(q.grad).all()


def test_hf_adapter_rejects_unsupported_features():
    from types import SimpleNamespace

    mod = SimpleNamespace(head_dim=256, is_causal=True)
    q = torch.zeros(1, 2, 4, 256)
    with pytest.raises(NotImplementedError):  # a prepared 4-D mask
        gfa.triton_gqa_attention(mod, q, q, q, torch.zeros(1, 1, 4, 4))
    from gemma_triton_flash_attn_amd.attention import _check_dropout, _check_softcap

    for bad in (1.0, -0.1, float("nan")):
        with pytest.raises(ValueError, match="dropout_p"):
            _check_dropout(bad)
    assert _check_dropout(None) == 0.0 and _check_dropout(0.25) == 0.25
    with pytest.raises(ValueError, match="softcap"):
        _check_softcap(-1.0)
    assert _check_softcap(None) == 0.0


def test_register_into_transformers():
    pytest.importorskip("transformers")
    from transformers import AttentionInterface
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    gfa.register_triton_attention()
    assert ALL_ATTENTION_FUNCTIONS.get_interface("triton_gqa", None) is gfa.triton_gqa_attention
    assert "triton_gqa" in AttentionInterface._global_mapping
    gfa.register_triton_attention("gfa_custom")
    assert ALL_ATTENTION_FUNCTIONS.get_interface("gfa_custom", None) is gfa.triton_gqa_attention


@fake_pointers
def test_slice_span_over_4gib_is_rejected():
    """One (batch, head) slice at the row stride must fit the kernels' 32-bit buffer range:
    HF's (B, N, H, D) layout with 32 heads of 512 at N = 2^17 + 1 spans over 4 GiB."""
    lib = _lib.load()
    n, row = 131073, 32 * 512
    a = _fwd_args(seq_len=n, lse_ld=(n + 63) // 64 * 64, q_strides=_lib.Strides(n * row, 512, row))
    assert lib.gfa_fwd(ctypes.byref(a)) == 2
    assert b"4 GiB" in lib.gfa_last_error()
    # the Python layer copies such a view to the contiguous layout, which fits
    import torch

    from gemma_triton_flash_attn_amd.attention import _layout_ok

    def view(strides):
        return torch.empty_strided((1, 32, n, 512), strides, dtype=torch.bfloat16, device="meta")

    assert not _layout_ok(view((n * row, 512, row, 1)))
    assert _layout_ok(view((32 * n * 512, n * 512, 512, 1)))


@fake_pointers
def test_grid_larger_than_one_launch_is_rejected():
    lib = _lib.load()
    a = _fwd_args(batch=1100000, heads_q=1024, heads_kv=1024)  # 2 x 1.1e6 x 1024 > 2^31 workgroups
    for s in ("q_strides", "k_strides", "v_strides", "o_strides"):
        setattr(a, s, _lib.Strides(1024 * 64 * 512, 64 * 512, 512))
    assert lib.gfa_fwd(ctypes.byref(a)) == 2
    assert b"launch grid" in lib.gfa_last_error()


@fake_pointers
def test_bwd_noalloc_rejects_caller_scratch_and_oversize():
    """gfa_bwd_noalloc takes inputs and outputs only, and refuses requests whose delta (or
    explicit Q-split partials) exceed its fixed scratch, before touching any device."""
    lib = _lib.load()
    a = _lib.BwdArgs()
    for name in ("q", "k", "v", "o", "dout", "dq", "dk", "dv"):
        setattr(a, name, 256)
    a.lse = 512
    for s in ("q_strides", "k_strides", "v_strides", "o_strides", "do_strides", "dq_strides", "dk_strides",
              "dv_strides"):
        setattr(a, s, _lib.Strides(8 * 64 * 512, 64 * 512, 512))
    a.batch, a.heads_q, a.heads_kv, a.seq_len, a.head_dim = 1, 8, 1, 64, 512
    a.causal, a.scale, a.dtype, a.lse_ld = 1, 512 ** -0.5, _lib.GFA_DTYPE_BF16, 64
    a.delta = 1024  # caller scratch is not accepted
    assert lib.gfa_bwd_noalloc(ctypes.byref(a)) == 1
    assert b"NULL" in lib.gfa_last_error()
    a.delta = None
    a.workspace, a.workspace_bytes = 4096, 1 << 20
    assert lib.gfa_bwd_noalloc(ctypes.byref(a)) == 1
    a.workspace, a.workspace_bytes = None, 0
    # delta of 2^25 rows x 4 bytes = 128 MiB > 64 MiB scratch
    a.batch, a.heads_q, a.heads_kv, a.seq_len = 512, 64, 64, 1024
    a.lse_ld = 1024
    assert lib.gfa_bwd_noalloc(ctypes.byref(a)) == 3
    assert b"scratch" in lib.gfa_last_error()
    # explicit q_splits whose partials do not fit: 8 x 2 x 4 x 8192 x 512 x 4 B = 512 MiB
    a.batch, a.heads_q, a.heads_kv, a.seq_len, a.lse_ld = 1, 32, 4, 8192, 8192
    a.q_splits = 8
    assert lib.gfa_bwd_noalloc(ctypes.byref(a)) == 3
    assert lib.gfa_bwd_noalloc(None) == 1
