"""The dS store layout of the materialised backward (csrc/gfa_ds.h), compiled for the host with
g++ and checked against the dK/dV kernel's iteration (csrc/gfa_bwd_dkv.hip: workgroups of 64 keys,
query tiles [k0 / 32, nq) under causal masking, ending at (last key + window - 1) / 32 + 1 with a
window): every block the dK/dV kernel writes has a distinct index inside its (batch, head) slab,
and every block the dQ kernel reads (units jmin(i) .. jmax(i) of query tile i) is one the dK/dV
kernel writes, so no read sees memory no kernel wrote."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "gemma-triton-flash-attn_amd", "csrc")

PROG = r"""
#include <cstdio>
#include <cstdlib>
#include "gfa_ds.h"
int main(int argc, char** argv) {
  const int N = atoi(argv[1]), causal = atoi(argv[2]), window = atoi(argv[3]);
  const gfa::DsLayout l = gfa::ds_layout(N, causal, window);
  printf("%d %d %d %lld\n", l.nq, l.nk, l.lmax, (long long)l.slab);
  for (int i = 0; i < l.nq; ++i) {
    printf("%d %d", gfa::ds_jmin(l, i), gfa::ds_jmax(l, i));
    for (int j = gfa::ds_jmin(l, i); j <= gfa::ds_jmax(l, i); ++j) printf(" %lld", (long long)gfa::ds_index(l, i, j));
    printf("\n");
  }
  for (int j = 0; j < l.nk; ++j) {
    int lo, hi;
    gfa::ds_unit_rows(l, j, &lo, &hi);
    printf("%d %d\n", lo, hi);
  }
  return 0;
}
"""

CASES = ([(n, 1, 0) for n in (1, 31, 32, 33, 64, 65, 96, 127, 128, 129, 300, 1000, 1500, 4101)]
         + [(n, 0, 0) for n in (1, 33, 100, 257)]
         + [(n, 1, w) for n in (40, 300, 1000, 3000) for w in (1, 5, 31, 32, 33, 63, 64, 65, 100, 512, 700)]
         + [(16384, 1, 1024), (16384, 1, 512), (4096, 1, 1024)])


@pytest.fixture(scope="module")
def layout_prog(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    d = tmp_path_factory.mktemp("dslayout")
    src = d / "ds_layout.cpp"
    src.write_text(PROG)
    exe = d / "ds_layout"
    subprocess.run([gxx, "-std=c++17", "-O1", "-D__host__=", "-D__device__=", f"-I{CSRC}", str(src), "-o", str(exe)],
                   check=True)
    return str(exe)


def dkv_visits(N, causal, window, units=2):
    """(query tile, key unit) pairs the dK/dV kernel computes, per its workgroup loop: workgroups
    of `units` 32-key units (2: the role-pair forms, 4: the one-wave form)."""
    nq = (N + 31) // 32
    swa = causal and 0 < window < N
    span = 32 * units
    out = set()
    for kb in range((N + span - 1) // span):
        k0 = span * kb
        k_last = min(N, k0 + span) - 1
        lo = k0 // 32 if causal else 0
        hi = min(nq, (k_last + window - 1) // 32 + 1) if swa else nq
        for u in range(units):
            j = units * kb + u
            if 32 * j >= N:
                continue
            out.update((i, j) for i in range(lo, hi))
    return out


@pytest.mark.parametrize("N,causal,window", CASES)
def test_store_matches_the_dkv_iteration(layout_prog, N, causal, window):
    w = window if (causal and 0 < window < N) else 0
    lines = subprocess.run([layout_prog, str(N), str(causal), str(w)], check=True, capture_output=True,
                           text=True).stdout.splitlines()
    nq, nk, lmax, slab = (int(x) for x in lines[0].split())
    assert nq == nk == (N + 31) // 32
    stored = {}
    unit_rows = [tuple(int(x) for x in line.split()) for line in lines[1 + nq:]]
    for i, line in enumerate(lines[1:1 + nq]):
        vals = [int(x) for x in line.split()]
        jmin, jmax, idx = vals[0], vals[1], vals[2:]
        assert 0 <= jmin <= jmax < nk, (i, jmin, jmax)
        assert len(idx) == jmax - jmin + 1
        for j, x in zip(range(jmin, jmax + 1), idx):
            assert 0 <= x < slab
            stored[(i, j)] = x
    assert len(set(stored.values())) == len(stored), "two blocks share an index"
    visits = dkv_visits(N, causal, w)
    # dQ reads exactly the stored blocks; each must be written, and every write must land in one.
    assert set(stored) == visits
    # The one-wave form (128-key workgroups) visits every stored block and stores the visited
    # blocks inside jmin(i) .. jmax(i): exactly the layout again.
    one_wave = dkv_visits(N, causal, w, units=4)
    assert set(stored) <= one_wave
    assert {(i, j) for (i, j) in one_wave if i < nq and stored.get((i, j)) is not None} == set(stored)
    # ds_unit_rows (the one-wave form's test of which visited blocks to store): the query tiles
    # holding unit j form the interval it returns
    assert len(unit_rows) == nk
    for j, (lo, hi) in enumerate(unit_rows):
        assert {i for (i, jj) in stored if jj == j} == set(range(lo, hi)), (j, lo, hi)
    if w:
        assert lmax == max(jmax - jmin + 1 for jmin, jmax in
                           ((int(l.split()[0]), int(l.split()[1])) for l in lines[1:1 + nq]))


def test_workspace_sizes_and_forms():
    """gfa_bwd_workspace_bytes: which problems take the materialised form, and the exact size of its
    store at the headline shape (B1 32:4 N=16384 D=512 causal: query tile i of 512 stores units
    0 .. 2 (i >> 1) + 1, 131,584 blocks of 2 KiB per head)."""
    import torch

    from gemma_triton_flash_attn_amd import _lib
    from gemma_triton_flash_attn_amd.attention import backward_workspace

    base = _lib.bwd_workspace_size(1, 32, 4, 16384, 512, True, 0)
    nbytes, mat = backward_workspace(1, 32, 4, 16384, 512, True, 0)
    assert mat and nbytes == (base + 255) // 256 * 256 + 32 * 131584 * 2048
    assert backward_workspace(1, 16, 8, 16384, 256, True, 1024)[1]          # windowed D=256 (role pairs)
    assert backward_workspace(2, 8, 2, 700, 512, False, 0, torch.float16)[1]  # non-causal D=512
    for args in ((1, 16, 8, 16384, 256, True, 0), (1, 16, 8, 4096, 256, False, 0),  # D=256 one-wave form
                 (1, 16, 8, 4096, 256, True, 4096)):  # window >= N: full causal
        assert backward_workspace(*args)[1], args
    nb, m = backward_workspace(1, 16, 8, 4096, 256, True, 0)  # full causal: 8320 blocks per head (tiles i < 128: 2 (i >> 1) + 2)
    assert m and nb == (_lib.bwd_workspace_size(1, 16, 8, 4096, 256, True, 0) + 255) // 256 * 256 + 16 * 8320 * 2048
    for args in ((1, 16, 2, 4096, 128, True, 1024), (1, 8, 8, 1024, 64, True, 0)):  # D=128, D=64
        assert not backward_workspace(*args)[1], args
    nb, m = backward_workspace(1, 8, 1, 2048, 512, True, 0, segments=True)  # segment tables: the same store
    assert m and nb == backward_workspace(1, 8, 1, 2048, 512, True, 0)[0]
    for kw in ({"softcap": 30.0}, {"dropout_p": 0.1}):
        assert backward_workspace(1, 8, 1, 2048, 512, True, 0, **kw)[1], kw  # in the stored dS
        assert backward_workspace(1, 8, 1, 2048, 512, True, 500, **kw)[1], kw
        # D=256: their instances are the one-wave dK/dV form, which stores too
        assert backward_workspace(1, 16, 8, 4096, 256, True, 1024, **kw)[1], kw
        assert backward_workspace(1, 16, 8, 4096, 256, False, 0, **kw)[1], kw
        assert not backward_workspace(1, 16, 8, 4096, 128, True, 0, **kw)[1], kw
    prev = _lib.set_bwd_ds_limit(0)
    try:
        assert _lib.bwd_ds_limit() == 0
        assert not backward_workspace(1, 32, 4, 16384, 512, True, 0)[1]
        _lib.set_bwd_ds_limit(nbytes - (base + 255) // 256 * 256 - 1)  # one byte below this store
        assert not backward_workspace(1, 32, 4, 16384, 512, True, 0)[1]
    finally:
        _lib.set_bwd_ds_limit(prev)
    assert _lib.bwd_ds_limit() == prev == 32 << 30
