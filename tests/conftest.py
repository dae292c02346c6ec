"""Shared test setup: repo root on sys.path, the ``gpu`` marker, seeded input helpers."""
from __future__ import annotations

import contextlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def make_inputs(B, Hq, Hkv, N, D, dtype, device, seed=0, scale=1.0, with_do=True, layout="bhnd"):
    """Seeded N(0,1) * scale inputs drawn on a CPU generator in the order q, k, v, dO
    (reproducible across hosts), then cast and moved. ``layout='bnhd'`` returns
    (B, H, N, D) views of (B, N, H, D) storage, as transformers hands them over."""
    import torch

    g = torch.Generator().manual_seed(seed)
    shapes = [(B, Hq, N, D), (B, Hkv, N, D), (B, Hkv, N, D)] + ([(B, Hq, N, D)] if with_do else [])
    out = []
    for s in shapes:
        t = torch.randn(*s, generator=g) * scale
        if layout == "bnhd":
            t = t.transpose(1, 2).contiguous().to(device=device, dtype=dtype).transpose(1, 2)
        else:
            t = t.to(device=device, dtype=dtype)
        out.append(t)
    return out


@contextlib.contextmanager
def recomputing():
    """gfa_bwd in its recomputing form for the duration (the dS store limit at 0): the form of the
    reference and of gfa_bwd_noalloc, whose kernels a bitwise comparison needs on both sides."""
    from gemma_triton_flash_attn_amd import _lib

    prev = _lib.set_bwd_ds_limit(0)
    try:
        yield
    finally:
        _lib.set_bwd_ds_limit(prev)
