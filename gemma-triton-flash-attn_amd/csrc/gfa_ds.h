// The dS store of the backward's materialised form: the dK/dV kernel writes every 32 x 32 block of
// dS it computes (16-bit, the input dtype, as the reference rounds dS before dS K), and the dQ
// kernel then only accumulates dQ = scale * dS K, without recomputing S, P and dP.
//
// Blocks. Query tile i (rows 32 i .. 32 i + 31) and key unit j (keys 32 j .. 32 j + 31) of one
// (batch, query head). A block is 1024 elements in four parts c = 0..3 of 512 bytes; part c holds,
// for each key 32 j + r (r = 0..31, 16 bytes at 16 r), the queries
//   sigma(8 c + e) = 32 i + 16 (c >> 1) + 8 (e >> 2) + 4 (c & 1) + (e & 3),   e = 0..7,
// the order in which one lane of the dK/dV kernel holds them (lane = key, half h = c & 1, score
// registers of half RO = c >> 1 of the 32 queries): the 64 lanes of one wave (h, r) store parts
// 2 RO and 2 RO + 1 as 1 KB contiguous. Seen as a 32 x 32 matrix (row = key, column n = query
// sigma(n)), column n is element n & 7 of part n >> 3; the dQ kernel reads it with transposing
// LDS reads, so that lane n of an MFMA B operand gets column n.
//
// Which blocks exist is the dK/dV kernel's iteration: its workgroup w (keys 64 w .. 64 w + 63,
// units 2 w and 2 w + 1) visits query tiles [2 w, nq) under causal masking, ending at
// (64 w + 63 + window - 1) / 32 + 1 with a sliding window, and all tiles without causal masking.
// The one-wave form's 128-key workgroups visit a superset of these (the tiles of their 64-key
// halves) and store only the blocks inside jmin(i) .. jmax(i).
// Per (batch, head) the blocks are stored query tile by query tile, each row of blocks holding
// units jmin(i) .. jmax(i):
// - no causal masking: all nk units, row stride nk;
// - causal, full: units 0 .. min(nk - 1, 2 (i >> 1) + 1), rows packed (a triangle);
// - causal with a window: units 2 wmin(i) .. min(nk - 1, 2 (i >> 1) + 1), row stride lmax.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace gfa {

struct DsLayout {
  uint16_t* ds;    // null: no dS store (the recomputing form)
  int mode;        // 0 no causal masking, 1 causal, 2 causal with a window
  int window;      // mode 2
  int nq, nk;      // query tiles, key units (both ceil(N / 32))
  int lmax;        // mode 2: units per row of blocks
  int64_t slab;    // blocks per (batch, head)
};

__host__ __device__ inline int ds_jmin(const DsLayout& l, int i) {
  if (l.mode != 2) return 0;
  const int num = 32 * i - l.window - 62;  // first workgroup whose last query tile reaches tile i
  return num <= 0 ? 0 : 2 * ((num + 63) / 64);
}
__host__ __device__ inline int ds_jmax(const DsLayout& l, int i) {
  if (l.mode == 0) return l.nk - 1;
  const int j = 2 * (i >> 1) + 1;
  return j < l.nk - 1 ? j : l.nk - 1;
}
// Block index of (i, j) inside the (batch, head) slab; (i, j) must be stored (jmin <= j <= jmax).
__host__ __device__ inline int64_t ds_index(const DsLayout& l, int i, int j) {
  if (l.mode == 0) return (int64_t)i * l.nk + j;
  if (l.mode == 2) return (int64_t)i * l.lmax + (j - ds_jmin(l, i));
  const int64_t m = i >> 1;
  return 2 * m * m + 2 * m + (i & 1) * (2 * m + 2) + j;
}

// Query tiles [*lo, *hi) whose rows of blocks hold key unit j (jmin(i) <= j <= jmax(i)): those the
// 64-key workgroup of unit j visits (from its first tile 2 (j >> 1) under causal masking, to the
// end of its window).
__host__ __device__ inline void ds_unit_rows(const DsLayout& l, int j, int* lo, int* hi) {
  if (l.mode == 0) {
    *lo = 0;
    *hi = l.nq;
    return;
  }
  const int m = j >> 1;
  *lo = 2 * m;
  *hi = l.nq;
  if (l.mode == 2) {
    const int e = (64 * m + 62 + l.window) / 32 + 1;
    if (e < *hi) *hi = e;
  }
}

// Segment tables (each row a partition of [0, N) into runs: a segment's tokens carry lo = its
// first token and hi = one past its last, a padding token t carries lo = hi = t): the key units
// [*jlo, *jhi] whose blocks of query tile i the dK/dV kernel computes, before the layout's own
// bounds. Its 64-key workgroup of keys g0 .. glast visits the tiles [lo[g0] / 32,
// ceil(hi[glast] / 32)), so unit j is in for tile i (rows r0 = 32 i .. r1) when
// - lo[g0] <= r0 + 31, i.e. g0 < max(r0 + 32, hi[r1]) (a key past the tile shares its segment
//   with row r1 exactly when it lies before hi[r1]);
// - hi[glast] > r0, i.e. glast >= lo[r0] (keys before r0 reach past it exactly when they share
//   row r0's segment), except for glast = r0 itself when that row is padding.
// Table values are clamped to [0, N], as the kernels clamp them. The one-wave form's 128-key
// workgroups visit a superset (their first key is no later, their last no earlier).
__host__ __device__ inline void ds_seg_units(const int* lo, const int* hi, int N, int i, int* jlo, int* jhi) {
  auto cl = [N](int x) { return x < 0 ? 0 : (x > N ? N : x); };
  const int r0 = 32 * i;
  const int r1 = r0 + 31 < N - 1 ? r0 + 31 : N - 1;
  int j0 = 2 * (cl(lo[r0]) / 64);  // the first unit whose workgroup's last key reaches lo[r0]
  const int g_end = 64 * (j0 >> 1) + 64;
  if (cl(hi[(g_end < N ? g_end : N) - 1]) <= r0) j0 += 2;
  const int h1 = cl(hi[r1]);
  const int e = h1 > r0 + 32 ? h1 : r0 + 32;
  *jlo = j0;
  *jhi = 2 * ((e - 1) / 64) + 1;
}

// Host: the layout of an N-row problem (without the pointer) and its size in blocks per slab.
inline DsLayout ds_layout(int N, int causal, int window) {
  DsLayout l;
  l.ds = nullptr;
  l.nq = l.nk = (N + 31) / 32;
  l.mode = causal ? (window > 0 ? 2 : 1) : 0;
  l.window = l.mode == 2 ? window : 0;
  l.lmax = 0;
  if (l.mode == 0) {
    l.slab = (int64_t)l.nq * l.nk;
  } else if (l.mode == 1) {
    const int last = l.nq - 1;
    l.slab = ds_index(l, last, 0) + ds_jmax(l, last) + 1;
  } else {
    for (int i = 0; i < l.nq; ++i) {
      const int len = ds_jmax(l, i) - ds_jmin(l, i) + 1;
      if (len > l.lmax) l.lmax = len;
    }
    l.slab = (int64_t)l.nq * l.lmax;
  }
  return l;
}

}  // namespace gfa
