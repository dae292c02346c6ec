// Kernel parameter blocks shared by the launchers and the device kernels.
// All strides are in elements; the head dimension is always unit-stride.
#pragma once
#include <stdint.h>

#include "gfa_ds.h"

namespace gfa {

// Row addressing of one (B, H, N, D) tensor: element (b, h, n, d) lives at
// base + b * sb + h * sh + n * sn + d.
struct RowView {
  int64_t sb, sh, sn;
};

// Logit soft-capping (the kernels' CAP instances): a raw score s = q.k becomes
// (softcap / scale) * tanh(s * cap_a), i.e. the scaled score scale * s becomes
// softcap * tanh(scale * s / softcap); the softmax exponent of the capped score is
// tanh(...) * cap_log2 in the log2 domain, and dS carries the factor 1 - tanh^2.
struct SoftCap {
  float cap_a;     // scale / softcap
  float cap_log2;  // softcap * log2(e)
};

// Attention dropout (the kernels' DROP instances): P_ij of query row i (query head bh = b Hq + h)
// and key j is kept, scaled by 1 / (1 - p), when drop_hash(drop_row(bh, i), j) >= thresh, and
// zeroed otherwise; the row sums and the LSE use the undropped P.
struct Dropout {
  unsigned seed_lo, seed_hi;
  unsigned thresh;  // round(p * 2^32): keep probability 1 - thresh / 2^32
  float inv_keep;   // 1 / (1 - p)
};

// Work decomposition shared by the forward and dQ kernels: a workgroup owns
// NWAVES (head, 32-query block) pairs of one KV head: `hpw` heads x `qbw` query blocks.
struct QGrid {
  int hpw;    // query heads per workgroup (divides R)
  int qbw;    // 32-row query blocks per workgroup (hpw * qbw == NWAVES)
  int n_hg;   // R / hpw head groups per KV head
  int n_qsb;  // ceil(N / (32 * qbw)) query super-blocks
  int nblocks;
};

// Run-time work hand-out (optional): with `wq` set, a kernel runs as a persistent grid of `grid`
// workgroups that take the blocks of its static grid (nblocks of them, in the static grid's order)
// from per-XCD queues: wq[x] counts the blocks taken from queue x, which holds the blocks b with
// b % 8 == x (the XCD the hardware would have dispatched b to). A workgroup empties its own XCD's
// queue first, then the others. The counters are zeroed before the launch. Null: the static grid
// (one workgroup per block, dispatched by the hardware).
struct WorkQueue {
  unsigned* wq;
  int grid;  // launch grid size (the static grid's block count when wq is null)
};

// Optional segment table, (B, N) int32 each, row b at seg_lo + b * N: token t attends and is
// attended only within keys [seg_lo[t], seg_hi[t]) (intersected with the causal / window
// rule). Null when the problem has none (one segment per sequence).
struct FwdParams {
  const int* seg_lo;
  const int* seg_hi;
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;  // (B, Hq, lse_ld), natural log; may be null when store_lse == 0
  RowView qv, kv, vv, ov;
  int B, Hq, Hkv, N, R;
  int causal;
  int window;        // 0 = no sliding window; only honoured when causal
  float scale_log2;  // softmax scale * log2(e)
  SoftCap cap;       // read by the CAP instances only
  Dropout drop;      // read by the DROP instances only
  int store_lse;
  int lse_ld;
  QGrid g;
  WorkQueue sched;
};

struct BwdDqParams {
  const int* seg_lo;  // optional segment table (as FwdParams)
  const int* seg_hi;
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  const float* lse;  // (B, Hq, lse_ld)
  float* delta;      // (B, Hq, lse_ld), written: rowsum(dO * O)
  uint16_t* dq;
  RowView qv, kv, vv, ov, dov, dqv;
  int B, Hq, Hkv, N, R;
  int causal, window;
  float scale;       // softmax scale (applied to dQ at the end)
  float scale_log2;  // scale * log2(e)
  SoftCap cap;       // read by the CAP instances only
  Dropout drop;      // read by the DROP instances only
  int lse_ld;
  QGrid g;
  WorkQueue sched;
};

struct BwdDkvParams {
  const int* seg_lo;  // optional segment table (as FwdParams)
  const int* seg_hi;
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* dout;
  const float* lse;    // (B, Hq, lse_ld), rows padded to a multiple of 64
  const float* delta;  // same layout
  uint16_t* dk;      // written directly when q_splits == 1
  uint16_t* dv;
  float* part;       // fp32 partials [q_splits][2][B][Hkv][N][D] when q_splits > 1
  RowView qv, kv, vv, dov, dkv, dvv;
  int B, Hq, Hkv, N, R;
  int causal, window;
  float scale, scale_log2;
  float inv_scale;   // 1 / scale
  SoftCap cap;       // read by the CAP instances only
  Dropout drop;      // read by the DROP instances only
  int q_splits;
  int lse_ld;
  int n_kb;          // number of key blocks (each WKV keys wide)
  int nblocks;       // q_splits * B * Hkv * n_kb rounded up to whole groups of four key blocks
  DsLayout dsl;      // dS store (dsl.ds null: none)
};

// delta = rowsum(dO * O) of every row of the 32-row tiles that cover N (rows past N repeat row
// N - 1), for the materialised backward, whose dQ kernel no longer computes it.
struct DeltaParams {
  const uint16_t* o;
  const uint16_t* dout;
  float* delta;  // (B, Hq, lse_ld)
  RowView ov, dov;
  int B, Hq, N, D;
  int lse_ld;
};

// dQ = scale * dS K from the dS store (the materialised backward).
struct BwdDqDsParams {
  const int* seg_lo;  // optional (B, N) segment table (with seg_hi), or null
  const int* seg_hi;
  const uint16_t* k;
  uint16_t* dq;
  RowView kv, dqv;
  int B, Hq, Hkv, N, R;
  float scale;
  DsLayout dsl;
  QGrid g;
};

}  // namespace gfa
