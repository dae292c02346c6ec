"""The materialised backward with segment tables: which blocks of the dS store the dQ kernel reads
(csrc/gfa_ds.h: the layout's units jmin(i) .. jmax(i) narrowed by ds_seg_units), compiled for the
host with g++ and checked against the dK/dV kernel's segment-trimmed iteration (csrc/
gfa_bwd_dkv_kernel.inc: workgroup query tiles [lo[first key] / 32, ceil(hi[last key] / 32)),
64 keys per workgroup in the role-pair forms, 128 in the one-wave form). On every table: the dQ
kernel reads exactly the blocks the role-pair forms write, only blocks the one-wave form writes,
and every block holding an attended (query, key) pair, so no read sees memory no kernel wrote
and no term of dQ is dropped. Tables follow the C-ABI's contract (include/gfa.h): each row a
partition into segments and single padding tokens."""
import os
import random
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "gemma-triton-flash-attn_amd", "csrc")

PROG = r"""
#include <cstdio>
#include <vector>
#include "gfa_ds.h"
int main() {
  int N, causal, window;
  while (scanf("%d %d %d", &N, &causal, &window) == 3) {
    std::vector<int> lo(N), hi(N);
    for (int t = 0; t < N; ++t) scanf("%d", &lo[t]);
    for (int t = 0; t < N; ++t) scanf("%d", &hi[t]);
    const gfa::DsLayout l = gfa::ds_layout(N, causal, window);
    for (int i = 0; i < l.nq; ++i) {
      int a, b;
      gfa::ds_seg_units(lo.data(), hi.data(), N, i, &a, &b);
      printf("%d %d %d %d\n", gfa::ds_jmin(l, i), gfa::ds_jmax(l, i), a, b);
    }
    printf("end\n");
  }
  return 0;
}
"""


@pytest.fixture(scope="module")
def seg_prog(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    d = tmp_path_factory.mktemp("dsseg")
    src = d / "ds_seg.cpp"
    src.write_text(PROG)
    exe = d / "ds_seg"
    subprocess.run([gxx, "-std=c++17", "-O1", "-D__host__=", "-D__device__=", f"-I{CSRC}", str(src), "-o", str(exe)],
                   check=True)
    return str(exe)


def table(runs):
    """(lo, hi) of a row from runs [(length, is_segment)]; a padding run is single tokens."""
    lo, hi, t = [], [], 0
    for n, seg in runs:
        for k in range(n):
            lo.append(t if seg else t + k)
            hi.append(t + n if seg else t + k)
        t += n
    return lo, hi


def dkv_writes(N, causal, window, lo, hi, units):
    """(query tile, key unit) pairs the dK/dV kernel computes with a segment table."""
    nq = (N + 31) // 32
    swa = causal and 0 < window < N
    cl = lambda x: min(max(x, 0), N)
    span = 32 * units
    out = set()
    for kb in range((N + span - 1) // span):
        k0 = span * kb
        k_last = min(N, k0 + span) - 1
        a = k0 // 32 if causal else 0
        b = min(nq, (k_last + window - 1) // 32 + 1) if swa else nq
        a = max(a, cl(lo[k0]) // 32)
        b = min(b, (cl(hi[k_last]) + 31) // 32)
        for u in range(units):
            j = units * kb + u
            if 32 * j < N:
                out.update((i, j) for i in range(a, b))
    return out


def attended_blocks(N, causal, window, lo, hi):
    swa = causal and 0 < window < N
    out = set()
    for q in range(N):
        for k in range(lo[q], hi[q]):
            if causal and k > q:
                continue
            if swa and q - k >= window:
                continue
            out.add((q // 32, k // 32))
    return out


def random_runs(rng, N):
    runs, t = [], 0
    while t < N:
        if rng.random() < 0.25:
            n = min(N - t, rng.choice((1, 1, 2, 5, 31, 33)))
            runs.append((n, False))
        else:
            n = min(N - t, rng.choice((1, 2, 17, 31, 32, 33, 63, 64, 65, 100, 200, 500)))
            runs.append((n, True))
        t += n
    return runs


def cases():
    rng = random.Random(20261202)
    out = []
    fixed = [
        (1000, [(1000, True)]),                                   # one segment
        (1000, [(300, True), (450, True), (250, True)]),          # packed
        (993, [(500, True), (492, True), (1, False)]),            # padding row alone in the last tile
        (1025, [(1024, True), (1, False)]),
        (700, [(200, False), (500, True)]),                       # left padding
        (700, [(500, True), (200, False)]),                       # right padding
        (129, [(129, False)]),                                    # all padding
        (96, [(1, True)] * 96),                                   # single-token segments
    ]
    for N, runs in fixed:
        for causal, window in ((1, 0), (0, 0), (1, 100), (1, 31)):
            out.append((N, causal, window, runs))
    for _ in range(60):
        N = rng.choice((33, 64, 65, 127, 300, 777, 1024, 1500))
        causal = rng.random() < 0.75
        window = rng.choice((0, 0, 1, 33, 64, 200, 512)) if causal else 0
        out.append((N, int(causal), window, random_runs(rng, N)))
    return out


def test_dq_reads_exactly_the_written_blocks(seg_prog):
    cs = cases()
    inp = []
    tables = []
    for N, causal, window, runs in cs:
        lo, hi = table(runs)
        assert len(lo) == N
        w = window if (causal and 0 < window < N) else 0
        tables.append((N, causal, w, lo, hi))
        inp.append(f"{N} {causal} {w}\n{' '.join(map(str, lo))}\n{' '.join(map(str, hi))}\n")
    res = subprocess.run([seg_prog], input="".join(inp), check=True, capture_output=True, text=True).stdout
    blocks = res.split("end\n")[:-1]
    assert len(blocks) == len(tables)
    for (N, causal, w, lo, hi), text in zip(tables, blocks):
        rows = [tuple(int(x) for x in line.split()) for line in text.splitlines()]
        assert len(rows) == (N + 31) // 32
        reads = {(i, j) for i, (jmin, jmax, a, b) in enumerate(rows) for j in range(max(jmin, a), min(jmax, b) + 1)}
        layout = {(i, j) for i, (jmin, jmax, _, _) in enumerate(rows) for j in range(jmin, jmax + 1)}
        pair = dkv_writes(N, causal, w, lo, hi, 2)
        one_wave = dkv_writes(N, causal, w, lo, hi, 4) & layout
        case = (N, causal, w)
        assert pair <= layout, case
        assert reads == pair, (case, sorted(reads ^ pair)[:5])
        assert reads <= one_wave, (case, sorted(reads - one_wave)[:5])
        missing = attended_blocks(N, causal, w, lo, hi) - reads
        assert not missing, (case, sorted(missing)[:5])


def test_padding_edge_case_is_in_the_cases():
    """The padding-row case of ds_seg_units: N = 993, the last token (row 992, alone in tile 31)
    padding. The last workgroup (keys 960 .. 992) ends at that row, whose hi is 992, so no
    workgroup writes tile 31, although unit 30's last key reaches lo[992]; the exact-read check
    above covers this table, with and without causal masking."""
    lo, hi = table([(500, True), (492, True), (1, False)])
    N, i = 993, 31
    assert lo[992] == hi[992] == 992
    for causal in (0, 1):
        assert not {b for b in dkv_writes(N, causal, 0, lo, hi, 2) if b[0] == i}
    assert any(N == 993 for N, _, _, _ in cases())
