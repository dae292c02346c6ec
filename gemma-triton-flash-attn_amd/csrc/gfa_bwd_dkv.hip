// GQA flash-attention backward, pack-GQA Q-split dK/dV kernel (hot-path row R3) and the
// fp32 partial-sum reduction used when the query range is split.
//
// Semantics follow /root/reference/flash_attn/attention.py:1080-1213 (launch 1602-1620):
// for a block of keys j of KV head g,
//   dV_j = sum_{h in group g} sum_i P_ij dO_i
//   dK_j = s * sum_{h in group g} sum_i dS_ij q_i
// with P and dS recomputed from LSE and delta exactly as in the dQ kernel, P and dS cast
// to the input dtype before the products. The query range of a key block starts at the
// key block (causal) and ends at the last key + window - 1 (sliding window).
// With q_splits > 1 the (head, query tile) iteration space of every key block is cut into
// q_splits contiguous chunks; each chunk writes an fp32 partial (scaled) and
// dkv_reduce_kernel sums them in a fixed order (deterministic, no atomics; the reference
// uses atomic_add into 16-bit dK/dV, attention.py:1206-1209).
//
// MI355X design: a wave pair owns 32 keys and splits the work by role, not by head dim.
// Both waves keep a full-head-dim stationary B operand in VGPRs (lane = key): role 0 the
// K rows, role 1 the V rows. Per LDS tile of BQ queries
//   role 0: S = Q K^T (A = Q tile rows), P = exp2(S*scale*log2e - LSE*log2e) masked,
//           P handed to the partner through LDS (fp32), then dV^T += dO^T P;
//   role 1: dP = dO V^T (A = dO tile rows), dS = P (dP - delta), then dK^T += Q^T dS;
// the dV^T / dK^T accumulators (32 keys x D, fp32) fill the AGPRs at D=512, and the A operands of
// the two accumulations are read with ds_read_b64_tr_b16 from the same row-major tiles
// that fed the score products. The only cross-wave traffic is the one-way P hand-off, and
// no softmax work is duplicated. All R query heads of the KV head stream through the
// same workgroup (pack-GQA), so K/V are read once and dK/dV need no cross-head reduction.
#include "gfa_common.h"
#include "gfa_params.h"
#include "gfa_launch.h"

namespace gfa {

// ROLES = 2: a wave pair per 32 keys, split by role (see above). ROLES = 1: one wave per
// 32 keys does all four products (K and V rows resident, dV^T and dK^T both in AGPRs);
// used at D=64, and at D=256 without a window, where that is faster than the pair. Role-split
// pairs run D=512 (one wave per SIMD), D=128 (two) and D=256 with a window (two, everything
// in VGPRs: 64 keys per workgroup, two workgroups per CU). WPE: waves per SIMD the register
// budget is bounded for.
// One wave per 32 keys at D >= 128 stages its K / V rows (and its dK / dV rows) through LDS in
// whole-row copies; per-lane loads in the MFMA operand layout touch 32 rows per instruction.
constexpr bool dkv_stages_rows(int D, int roles) { return roles == 1 && D >= 128; }

template <int D, int BQ, bool IS_BF16, int NW, int ROLES, int WPE, bool CAP, bool DROP>
__global__ __launch_bounds__(NW * 64, WPE) void bwd_dkv_kernel(const BwdDkvParams p) {
  constexpr int KT = D / 16;   // MFMA k-steps of the score products (full head dim)
  constexpr int DB = D / 32;   // 32-row blocks of the dV^T / dK^T accumulator
  constexpr int SB = BQ / 32;  // 32-query score blocks per tile
  constexpr int TILE = BQ * D * 2;
  // Pair at D=512: the two roles share the softmax work (see the tile step); at D=128, with
  // three waves per SIMD filling each other's idle time, role 0 computes P alone and hands
  // it over (the shared form measured 9% slower there, 3% faster at D=512).
  constexpr bool SHARED = ROLES == 2 && D == 512;
  // Pair exchange area per 32-query score block: shared, four 2 KB slots (S and dP halves,
  // then P and dS halves); otherwise one fp32 P block. One f32x4 per lane per 1 KB plane.
  constexpr int PX = ROLES == 2 ? SB * (SHARED ? 4 * 2048 : 4096) : 0;
  constexpr int NU = NW / ROLES;                     // 32-key units per workgroup
  constexpr int NS = 3 - ROLES;                      // stationary operands / accumulators per wave
  static_assert(ROLES == 1 || ROLES == 2, "one wave or a role-split pair per 32 keys");
  static_assert(BQ % 32 == 0, "BQ must be a multiple of 32");
  static_assert(D == 64 || D == 128 || D == 256 || D == 512, "head dim must be 64, 128, 256 or 512");

  constexpr bool STAGE = dkv_stages_rows(D, ROLES);
  // Role pairs at two waves per SIMD (D=256): each wave stages its one stationary operand (K or
  // V rows) and its one accumulator's output rows through its own tile buffer.
  constexpr bool STAGE_PAIR = ROLES == 2 && D == 256 && WPE == 2;
  constexpr bool PRIO = WPE >= 2;
  static_assert(!STAGE_PAIR || NW == 4, "one tile buffer per wave");

  // Shared form: the row statistics of a tile (LSE then delta of its BQ rows) travel into LDS with
  // the tile, double buffered, so no VGPRs hold them across the score chain.
  constexpr int STB = SHARED ? 512 : 0;
  static_assert(!SHARED || BQ <= 64, "a statistics block holds 64 rows of LSE and of delta");
  __shared__ __attribute__((aligned(1024))) char smem_raw[4 * TILE + NU * PX + 2 * STB];
  char GFA_LDS* smem = (char GFA_LDS*)smem_raw;
  char GFA_LDS* const stat_lds = smem + 4 * TILE + NU * PX;
  // STAGE: each wave's TILE-byte block of this launch-sized array takes its V rows before the
  // loop and its dV, then dK rows after it (its K rows go to one of the tile buffers). Dynamic,
  // so the compiler's occupancy estimate (static LDS only) stays that of the tile buffers.
  extern __shared__ __attribute__((aligned(1024))) char stage_raw[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int unit = wave / ROLES;
  const int role = ROLES == 2 ? (wave & 1) : 0;  // pair: 0 = S, P and dV;  1 = dP, dS and dK
  const int h = lane >> 5;
  const int l32 = lane & 31;
  char GFA_LDS* px = smem + 4 * TILE + unit * PX + lane * 16;  // 1 KB planes of one f32x4 per lane

  // ---- workgroup -> (key block, split, b, kv head) ----
  // Heaviest first: under causal masking the early key blocks own the longest query
  // ranges, so groups of four adjacent key blocks are the slowest-varying index (a
  // key-block-fastest order mixes heavy and light blocks in every round: 1.5x the balanced
  // makespan on a 512-workgroup grid). Each group of four key blocks of one (split, b, kv
  // head) is four consecutive logical ids, which xcd_remap places on one XCD: they read the
  // same query tiles and share them in L2. Ids past the last key block have no work.
  int lid = xcd_remap(blockIdx.x, p.nblocks, 4);
  const int kb_lo = lid & 3;
  lid >>= 2;
  const int kvh = lid % p.Hkv;
  lid /= p.Hkv;
  const int b = lid % p.B;
  lid /= p.B;
  const int split = lid % p.q_splits;
  int kb = (lid / p.q_splits) * 4 + kb_lo;
  // Sliding window: nearly every key block has the same query range, so the short last blocks
  // (keys within a window of the end) go first; they end at staggered times and spread the
  // later blocks' prologues instead of every CU loading its rows at once.
  if (p.causal && p.window > 0) kb = (p.n_kb + 3) / 4 * 4 - 1 - kb;
  if (kb >= p.n_kb) return;  // whole workgroup, before any barrier

  const int wg_k0 = kb * NU * 32;
  const int wg_k_last = min(p.N, wg_k0 + NU * 32) - 1;
  const int k0 = wg_k0 + unit * 32;  // this pair's keys [k0, k0 + 32)
  const bool active = k0 < p.N;
  const int k_last = k0 + 31;
  const int key = k0 + l32;
  const int krow = min(key, p.N - 1);
  VisRange vis = queries_of_key(key, p.N, p.causal, p.window);

  const bool swa = p.causal && p.window > 0;
  // Query tiles the workgroup visits.
  int qt_lo = 0, qt_hi = (p.N + BQ - 1) / BQ;
  if (p.causal) {
    qt_lo = wg_k0 / BQ;
    if (swa) qt_hi = min(qt_hi, (wg_k_last + p.window - 1) / BQ + 1);
  }
  // Segment table (optional): a key serves the queries of its own segment only.
  const int* slo = p.seg_lo ? p.seg_lo + (int64_t)b * p.N : nullptr;
  const int* shi = p.seg_lo ? p.seg_hi + (int64_t)b * p.N : nullptr;
  if (slo) {
    qt_lo = max(qt_lo, clamp_n(slo[wg_k0], p.N) / BQ);
    qt_hi = min(qt_hi, (clamp_n(shi[wg_k_last], p.N) + BQ - 1) / BQ);
    vis = intersect(vis, clamp_n(slo[krow], p.N), clamp_n(shi[krow], p.N));
  }
  const int nqt = max(0, qt_hi - qt_lo);
  const int total = p.R * nqt;
  const int chunk = (total + p.q_splits - 1) / p.q_splits;
  const int it_lo = min(total, split * chunk);
  const int it_hi = min(total, it_lo + chunk);

  // Queries every key of this pair serves: [all_lo, all_hi).
  int all_lo = 0, all_hi = p.N;
  if (p.causal) {
    all_lo = k_last;
    if (swa) all_hi = min(p.N, k0 + p.window);  // q - key < window for the first key
  }
  if (slo && active) {
    all_lo = max(all_lo, clamp_n(slo[min(k_last, p.N - 1)], p.N));
    all_hi = min(all_hi, clamp_n(shi[k0], p.N));
  }
  const bool pair_full = k_last < p.N;

  // ---- stationary B operands (lane = key, full head dim) ----
  // pair: sf[0] = K rows (role 0) or V rows (role 1);  single wave: sf[0] = K, sf[1] = V.
  i16x8 sf[NS][KT];
  int roff[8];  // tile rows (A operand of S / dP): row l32, chunk 2*kk + h  (+256 * (kk >> 3))
#pragma unroll
  for (int kl = 0; kl < 8; ++kl) roff[kl] = l32 * (2 * D) + (((2 * kl + h) ^ swz<D>(l32)) << 4);
  if constexpr (STAGE_PAIR) {
    // This role's rows (K or V) into tile buffer `wave` (idle before the loop) in whole-row
    // copies, read back in the operand layout.
    char GFA_LDS* blk = smem + wave * TILE;
    const uint16_t* src = role == 0 ? p.k + (int64_t)b * p.kv.sb + (int64_t)kvh * p.kv.sh
                                    : p.v + (int64_t)b * p.vv.sb + (int64_t)kvh * p.vv.sh;
    const int64_t sn = role == 0 ? p.kv.sn : p.vv.sn;
    if (p.q_splits == 1) {  // no other workgroup reads these rows: non-temporal (C3 dK/dV 1.4%)
      copy_rows_lds<D, true>(src, sn, p.N, k0, lane, blk);
    } else {
      copy_rows_lds<D, false>(src, sn, p.N, k0, lane, blk);
    }
    drain_tile_copies();
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) sf[0][kk] = lds_read16(blk, roff[kk & 7] + 256 * (kk >> 3));
    barrier_lds();  // every wave has read its rows out of the tile buffers
  } else if constexpr (STAGE) {
    // K rows into tile buffer `wave` (idle before the loop), V rows into the stage block, in
    // whole-row copies; read back in the operand layout.
    static_assert(NS == 2 && NU == 4, "one wave per 32 keys, four per workgroup");
    char GFA_LDS* kblk = smem + wave * TILE;
    char GFA_LDS* vblk = (char GFA_LDS*)stage_raw + wave * TILE;
    if (p.q_splits == 1) {  // no other workgroup reads these rows: non-temporal
      copy_rows_lds<D, true>(p.k + (int64_t)b * p.kv.sb + (int64_t)kvh * p.kv.sh, p.kv.sn, p.N, k0, lane, kblk);
      copy_rows_lds<D, true>(p.v + (int64_t)b * p.vv.sb + (int64_t)kvh * p.vv.sh, p.vv.sn, p.N, k0, lane, vblk);
    } else {
      copy_rows_lds<D, false>(p.k + (int64_t)b * p.kv.sb + (int64_t)kvh * p.kv.sh, p.kv.sn, p.N, k0, lane, kblk);
      copy_rows_lds<D, false>(p.v + (int64_t)b * p.vv.sb + (int64_t)kvh * p.vv.sh, p.vv.sn, p.N, k0, lane, vblk);
    }
    drain_tile_copies();
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      sf[0][kk] = lds_read16(kblk, roff[kk & 7] + 256 * (kk >> 3));
      sf[1][kk] = lds_read16(vblk, roff[kk & 7] + 256 * (kk >> 3));
    }
    barrier_lds();  // every wave has read its K rows out of the tile buffers
  } else {
    const uint16_t* krp = p.k + (int64_t)b * p.kv.sb + (int64_t)kvh * p.kv.sh + (int64_t)krow * p.kv.sn + 8 * h;
    const uint16_t* vrp = p.v + (int64_t)b * p.vv.sb + (int64_t)kvh * p.vv.sh + (int64_t)krow * p.vv.sn + 8 * h;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const uint16_t* r = (i == 0 && role == 0) ? krp : vrp;
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) sf[i][kk] = *reinterpret_cast<const i16x8*>(r + 16 * kk);
    }
  }

  // 32 keys x D fp32 accumulators in AGPRs. pair: acc[0] = dV^T (role 0) or dK^T (role 1);
  // single wave: acc[0] = dV^T, acc[1] = dK^T.
  f32x16 acc[NS][DB];
#pragma unroll
  for (int i = 0; i < NS; ++i)
#pragma unroll
    for (int j = 0; j < DB; ++j) acc[i][j] = f32x16{};

  // Per-lane LDS offsets of the tile reads. At D=128 (two waves per SIMD, register-bound)
  // one base each: kstep_off and mma_tr_accumulate_b derive the others with an XOR next to
  // each read, where eight-entry offset tables would cost 14 registers (5% faster measured).
  // The other head dims keep the tables (measured 2-4% faster there).
  constexpr bool ONE_BASE = D == 128 || (D == 256 && WPE == 2);
  // One wave per 32 keys at D >= 256 (both accumulators fill the AGPRs): the two score chains
  // accumulate in VGPRs (mma32_vgpr), so no accumulator block is moved out and back around them.
  constexpr bool VCHAIN1 = ROLES == 1 && SB == 1 && D >= 256 && !ONE_BASE;
  static_assert(!VCHAIN1 || KT == 16, "the dP chain computes one exponential of the S block per product");
  // Role pairs at two waves per SIMD and D=256 (register-bound): the score chains start from
  // the row statistic instead of zero, so neither LSE nor delta stays live past the chain:
  // role 0 from -LSE / scale (P = exp2(scale * log2e * acc)), role 1 from -delta (dS = P acc).
  constexpr bool INIT = ROLES == 2 && D == 256;
  // CAP (soft-capped scores) needs the raw score, which a chain started from -LSE / scale no
  // longer holds; the host runs soft-capped problems on the other forms.
  static_assert(!((CAP || DROP) && INIT), "soft-capping and dropout need the plain score chains");
  const int roff0 = l32 * (2 * D) + ((h ^ swz<D>(l32)) << 4);  // tile row l32, chunk h (k-step 0)
  int toff0;  // tiles read transposed (A operands of dV^T, dK^T): rows 4h + t/4, column block 0
  int toffA[4], toffB[4];
  {
    const int t16 = lane & 15;
    const int half16 = (lane >> 4) & 1;
    const int rA = 4 * h + (t16 >> 2);
    const int rB = rA + 8;
    const int c0 = 2 * half16 + ((t16 >> 1) & 1);
    toff0 = rA * (2 * D) + ((c0 ^ swz<D>(rA)) << 4) + (t16 & 1) * 8;
#pragma unroll
    for (int dl = 0; dl < 4; ++dl) {
      const int c = 4 * dl + c0;
      toffA[dl] = rA * (2 * D) + ((c ^ swz<D>(rA)) << 4) + (t16 & 1) * 8;
      toffB[dl] = rB * (2 * D) + ((c ^ swz<D>(rB)) << 4) + (t16 & 1) * 8;
    }
  }
  // Score chains (the first one of a step with NL tile-copy instructions spread over it) and
  // accumulations from tiles read transposed, in the offset form chosen above.
  auto chain = [&](const char GFA_LDS* tile, int extra, const i16x8 (&bf)[KT], const f32x16& c0 = f32x16{})
                   __attribute__((always_inline)) {
    if constexpr (ONE_BASE) {
      return mma_chain1_lds_b<IS_BF16, KT, 4, 1>(tile, roff0, extra, bf, c0);
    } else {
      return mma_chain1_lds<IS_BF16, KT, 4, 1>(tile, roff, extra, bf, c0);
    }
  };
  auto chain_ld = [&](auto nl, const char GFA_LDS* tile, const i16x8 (&bf)[KT], auto&& ld,
                      const f32x16& c0 = f32x16{}) __attribute__((always_inline)) {
    constexpr int NL = decltype(nl)::value;
    if constexpr (ONE_BASE) {
      return mma_chain1_lds_ld_b<IS_BF16, KT, 4, NL>(tile, roff0, 0, bf, ld, c0);
    } else {
      return mma_chain1_lds_ld<IS_BF16, KT, 4, NL>(tile, roff, 0, bf, ld, c0);
    }
  };
  auto accumulate = [&](f32x16 (&acc_)[DB], const char GFA_LDS* tile, const i16x8 (&bop)[BQ / 16])
                        __attribute__((always_inline)) {
    if constexpr (ONE_BASE) {
      mma_tr_accumulate_b<IS_BF16, D, DB, BQ / 16, 4, 1>(acc_, tile, toff0, bop);
    } else {
      mma_tr_accumulate<IS_BF16, D, DB, BQ / 16, 4, 1>(acc_, tile, toffA, toffB, bop);
    }
  };

  TileLoader<D, BQ, NW> qload, dload;
  qload.init(p.q, p.qv.sn, p.N, wave, lane);
  dload.init(p.dout, p.dov.sn, p.N, wave, lane);
  const uint16_t* q_kv = p.q + (int64_t)b * p.qv.sb + (int64_t)kvh * p.R * p.qv.sh;
  const uint16_t* d_kv = p.dout + (int64_t)b * p.dov.sb + (int64_t)kvh * p.R * p.dov.sh;
  // Row statistics this wave needs. Single wave: st[0][sb][g] = LSE, st[1][sb][g] = delta of
  // rows 8g + 4h + 0..3. Pair, shared form: each role turns half of the rows (g = 2 role,
  // 2 role + 1) into P and dS: st[0][sb][0..1] = their LSE, st[0][sb][2..3] = their delta.
  // Pair, hand-off form: st[0] = LSE (role 0) or delta (role 1) of all rows.
  const int64_t stat_off = ((int64_t)b * p.Hq + (int64_t)kvh * p.R) * p.lse_ld;
  const float* stat_kv0 = p.lse + stat_off;
  const float* stat_kv1 = p.delta + stat_off;

  // Iteration `it` covers head kvh*R + r of query tile qt, the R heads of a tile back to back;
  // (r_c, qt_c) walk it incrementally. Neighbouring key blocks of one KV head run together on
  // one XCD, and the walk makes them read the same Q / dO tiles at the same time, so that the
  // tiles come from L2:
  // - causal: query tiles from the last one down, it = (qt_hi - 1 - qt) * R + r (every key
  //   block's range ends at the same last tile);
  // - sliding window: upward and cyclically inside [qt_lo, qt_hi), starting at the tile whose
  //   index is a multiple of nqt, so that step j of every workgroup reads a tile with index
  //   = j (mod nqt). Started at its own first (or last) tile, each key block ran a few tiles behind
  //   its neighbour, and three quarters of the dK/dV kernel's tile reads missed L2 (HBM reads
  //   3.7x this walk's; 3-5% slower).
  const bool rotate = swa;
  const int phase = rotate && nqt > 0 ? (nqt - qt_lo % nqt) % nqt : 0;
  int r_c = it_lo % p.R;
  int r_cur = r_c;  // head (within the group) of the tile being processed (the walk runs ahead)
  int qt_c = rotate ? qt_lo + (it_lo / p.R + phase) % max(nqt, 1) : qt_hi - 1 - it_lo / p.R;
  // Shared form: wave 0 copies the LSE rows, wave 1 the delta rows of head r, query tile qt into a
  // statistics block, 64 rows from the tile's first (one dword per lane; the tile uses BQ of them,
  // rows past the buffer's end read as zeros). Whole-wave copies keep the buffer resource
  // wave-uniform: under a lane-dependent branch the compiler rebuilt it from VGPRs every step.
  auto copy_stats = [&](int r, int qt, char GFA_LDS* dst) __attribute__((always_inline)) {
    if (wave < 2) {
      const float* base = (wave == 0 ? stat_kv0 : stat_kv1) + (int64_t)r * p.lse_ld;
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, p.lse_ld * 4, 0x00020000);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (void GFA_LDS*)(dst + wave * 256), 4, lane * 4, qt * BQ * 4, 0, 0);
    }
  };
  if (it_lo < it_hi) {
    qload.rebase(q_kv + (int64_t)r_c * p.qv.sh, p.qv.sn, p.N);
    dload.rebase(d_kv + (int64_t)r_c * p.dov.sh, p.dov.sn, p.N);
    qload.load(qt_c * BQ, smem);
    dload.load(qt_c * BQ, smem + 2 * TILE);
    if constexpr (SHARED) copy_stats(r_c, qt_c, stat_lds);
  }

  // P on the key lanes (rows = queries per register): exp2 against the row LSE, masked.

  // The dS store (p.dsl.ds set): the lane's 16 bytes of part c (= 2 * half-of-the-queries + h;
  // the lane's key l32, 8 queries) of the 32 x 32 block of query tile q0 / 32 and this pair's key
  // unit, head r_cur of the group, so that one wave's store is 1 KB contiguous; see gfa_ds.h.
  // The block's address is kept incrementally by the tile loop (ds_now: the block of the tile being
  // processed; one head further is one slab further), so the block-index formula runs only when
  // the walk moves to another query tile. The store form has 32-row query tiles (BQ = 32).
  const int64_t ds_slab_bytes = p.dsl.slab * 2048;
  char* const ds_group = reinterpret_cast<char*>(p.dsl.ds) + ((int64_t)b * p.Hq + kvh * p.R) * ds_slab_bytes;
  auto ds_block = [&](int r, int qt) __attribute__((always_inline)) {
    return ds_group + r * ds_slab_bytes + ds_index(p.dsl, qt, k0 / 32) * 2048;
  };
  char* ds_now = nullptr;
  auto store_ds = [&](int q0, int c, const i16x8& v) __attribute__((always_inline)) {
    (void)q0;
    if (p.dsl.ds != nullptr && active) {
      // Non-temporal: the block is read once, by the dQ kernel, so it should not push the query
      // tiles the key blocks share out of L2.
      __builtin_nontemporal_store(v, reinterpret_cast<i16x8*>(ds_now + c * 512 + l32 * 16));
    }
  };
  // exps_done: sc already holds the exponentials (computed under the dP chain), only the mask is left.
  auto p_elem = [&](float sv, float lse) __attribute__((always_inline)) {
    return fast_exp2(sv * p.scale_log2 - lse * kLog2e);
  };
  auto make_p = [&](f32x16 (&sc)[SB], const f32x4 (&lse)[SB][4], int q0, bool exps_done = false)
                    __attribute__((always_inline)) {
    const bool need_mask = !(active && pair_full && q0 >= all_lo && q0 + BQ <= all_hi && q0 + BQ <= p.N);
    if (!exps_done) {
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[sb][r] = p_elem(sc[sb][r], lse[sb][r >> 2][r & 3]);
      }
    }
    if (need_mask) {
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qi = q0 + sb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          sc[sb][r] = vis.has(qi) ? sc[sb][r] : 0.f;
        }
      }
    }
  };
  // P from a chain that started at -LSE / scale: exp2(scale * log2e * acc), masked.
  auto make_p_init = [&](f32x16 (&sc)[SB], int q0) __attribute__((always_inline)) {
    const bool need_mask = !(active && pair_full && q0 >= all_lo && q0 + BQ <= all_hi && q0 + BQ <= p.N);
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[sb][r] = fast_exp2(sc[sb][r] * p.scale_log2);
    }
    if (need_mask) {
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qi = q0 + sb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          sc[sb][r] = vis.has(qi) ? sc[sb][r] : 0.f;
        }
      }
    }
  };
  // CAP, hand-off form (role 0): P of the capped scores into sc, and P (1 - tanh^2), the factor
  // role 1 multiplies dP - delta by, into the exchange planes; both masked.
  auto make_p_cap = [&](f32x16 (&sc)[SB], const f32x4 (&lse)[SB][4], int q0, char GFA_LDS* pxr)
                        __attribute__((always_inline)) {
    const bool need_mask = !(active && pair_full && q0 >= all_lo && q0 + BQ <= all_hi && q0 + BQ <= p.N);
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * j + e;
          const float t = cap_tanh(sc[sb][r] * p.cap.cap_a);
          float pv = fast_exp2(t * p.cap.cap_log2 - lse[sb][j][e] * kLog2e);
          if (need_mask) pv = vis.has(q0 + sb * 32 + 8 * j + 4 * h + e) ? pv : 0.f;
          sc[sb][r] = pv;
          w[e] = pv * (1.f - t * t);
        }
        *reinterpret_cast<f32x4 GFA_LDS*>(pxr + (sb * 4 + j) * 1024) = w;
      }
    }
  };
  // DROP: is P of query qi (of the tile's head) and this lane's key kept? A dropped entry adds
  // nothing to dV and its dP counts 0 in dS; a kept one is scaled by 1 / (1 - p).
  auto kept = [&](int qi) __attribute__((always_inline)) {
    const int bh = b * p.Hq + kvh * p.R + r_cur;
    return drop_keep(drop_row(p.drop.seed_lo, p.drop.seed_hi, bh, qi), key, p.drop.thresh);
  };
  // dS = P * (dP - delta) in place of dP. Masked entries have P = 0 and give 0: delta is
  // finite on every row a tile covers (the dQ kernel writes the rows past N of the last
  // 32-row block too), so no guard is needed.
  auto make_ds = [&](f32x16& dp, const f32x4 pv4[4], const f32x4 (&del)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * j + e;
        dp[r] = pv4[j][e] * (dp[r] - del[j][e]);
      }
    }
  };
  auto pack = [&](const f32x16 (&v)[SB], i16x8 (&out)[BQ / 16]) __attribute__((always_inline)) {
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) out[sb * 2 + (r >> 3)][r & 7] = to16<IS_BF16>(v[sb][r]);
    }
  };

  // One query tile: prefetch the next tile into (qn, dn), score chains, P / dS,
  // accumulations reading the tiles transposed. The views are restrict-qualified: the
  // compiler then knows that no read of qt / dt / pxr touches the prefetch targets and
  // does not wait for the prefetch before reading the current tile.
  auto tile_step = [&](const char GFA_LDS* __restrict__ qt, const char GFA_LDS* __restrict__ dt,
                       char GFA_LDS* __restrict__ qn, char GFA_LDS* __restrict__ dn, char GFA_LDS* __restrict__ pxr,
                       const char GFA_LDS* __restrict__ stc, char GFA_LDS* __restrict__ stn, int r_n, int row_n, int q0,
                       const f32x4 (&st)[NS][SB][4]) __attribute__((always_inline)) {
    // The copies of the next tile are spread over the score chains, one every few MFMAs (a
    // run of copy issues would hold up the in-order MFMA stream).
    constexpr int NI = TileLoader<D, BQ, NW>::NI;  // copy instructions per tile and wave
    if constexpr (SHARED) copy_stats(r_n, row_n / BQ, stn);
    if constexpr (ROLES == 2) {
      // role 0: S = Q K^T from the Q tile, then dV^T += dO^T P reads the dO tile transposed.
      // role 1: dP = dO V^T from the dO tile, then dK^T += Q^T dS reads the Q tile transposed.
      const char GFA_LDS* ct = role == 0 ? qt : dt;
      const char GFA_LDS* tt = role == 0 ? dt : qt;
      f32x16 s[SB];
      f32x16 c0[SB];
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
        c0[sb] = f32x16{};
        if constexpr (INIT) {
          const float f = role == 0 ? -p.inv_scale : -1.f;
#pragma unroll
          for (int r = 0; r < 16; ++r) c0[sb][r] = st[0][sb][r >> 2][r & 3] * f;
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // the MFMA pipelines are scheduled on their own
      if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
        if (sb == 0) {
          auto ld = [&](int i) {
            if (i < NI) {
              qload.load_part(i, row_n, qn);
            } else {
              dload.load_part(i - NI, row_n, dn);
            }
          };
          if constexpr (SHARED) {
            // the chain in VGPRs (the AGPRs hold dV^T / dK^T; see mma32_vgpr)
            s[sb] = mma_chain1_lds_ld_vgpr<IS_BF16, KT, 4, 2 * NI>(ct, roff, sf[0], ld);
          } else {
            s[sb] = chain_ld(std::integral_constant<int, 2 * NI>{}, ct, sf[0], ld, c0[sb]);
          }
        } else {
          s[sb] = chain(ct, sb * 32 * (2 * D), sf[0], c0[sb]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
      i16x8 pb_sh[BQ / 16];  // shared form: P (role 0) or dS (role 1), packed, both halves
      if constexpr (SHARED) {
        // Shared softmax: role RO turns the rows of registers 8 RO .. 8 RO + 7 (g = 2 RO,
        // 2 RO + 1) into P and dS. Each role first hands its partner the half of its own chain
        // result the partner needs (role 0: S of registers 8..15; role 1: dP of 0..7), then
        // each hands back, packed to 16 bits, the half the partner accumulates (role 1: P of
        // 8..15 for dV; role 0: dS of 0..7 for dK). Exchange slots of one score block: 0 S half,
        // 1 dP half (two 1 KB planes of f32x4 each), 2 P half, 3 dS half (one 1 KB plane of
        // i16x8 each). Split this way neither wave waits for the other's exponentials or dS;
        // with P computed by role 0 alone, role 1 sat out about 20% of each step.
        const bool need_mask = !(active && pair_full && q0 >= all_lo && q0 + BQ <= all_hi && q0 + BQ <= p.N);
        auto slot = [&](int sb, int k, int j) __attribute__((always_inline)) { return pxr + (sb * 4 + k) * 2048 + j * 1024; };
        // this role's rows of the statistics block: LSE of rows 16 role + 8 j + 4 h + 0..3, then delta
        f32x4 stl[SB][4];
#pragma unroll
        for (int sb = 0; sb < SB; ++sb)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int off = (sb * 32 + 16 * role + 8 * j + 4 * h) * 4;
            stl[sb][j] = *reinterpret_cast<const f32x4 GFA_LDS*>(stc + off);
            stl[sb][2 + j] = *reinterpret_cast<const f32x4 GFA_LDS*>(stc + 256 + off);
          }
        auto shared = [&](auto ro) __attribute__((always_inline)) {
          constexpr int RO = decltype(ro)::value;
          constexpr int MH = 8 * RO, OH = 8 * (1 - RO);
  #pragma unroll
          for (int sb = 0; sb < SB; ++sb) {
  #pragma unroll
            for (int j = 0; j < 2; ++j) {
              const f32x4 v = {s[sb][OH + 4 * j], s[sb][OH + 4 * j + 1], s[sb][OH + 4 * j + 2], s[sb][OH + 4 * j + 3]};
              *reinterpret_cast<f32x4 GFA_LDS*>(slot(sb, RO, j)) = v;
            }
          }
          barrier_lds();  // both halves of both chains are in the slots
  #pragma unroll
          for (int sb = 0; sb < SB; ++sb) {
            f32x4 w[2];
  #pragma unroll
            for (int j = 0; j < 2; ++j) w[j] = *reinterpret_cast<const f32x4 GFA_LDS*>(slot(sb, 1 - RO, j));
            float pv[8], dsv[8], gcap[8];
  #pragma unroll
            for (int i = 0; i < 8; ++i) {
              const float sv = RO == 0 ? s[sb][MH + i] : w[i >> 2][i & 3];
              if constexpr (CAP) {
                const float t = cap_tanh(sv * p.cap.cap_a);
                pv[i] = fast_exp2(t * p.cap.cap_log2 - stl[sb][i >> 2][i & 3] * kLog2e);
                gcap[i] = 1.f - t * t;
                continue;
              }
              pv[i] = fast_exp2(sv * p.scale_log2 - stl[sb][i >> 2][i & 3] * kLog2e);
            }
            if (need_mask) {
  #pragma unroll
              for (int i = 0; i < 8; ++i) {
                const int qi = q0 + sb * 32 + 8 * (2 * RO + (i >> 2)) + 4 * h + (i & 3);
                pv[i] = vis.has(qi) ? pv[i] : 0.f;
              }
            }
  #pragma unroll
            for (int i = 0; i < 8; ++i) {
              const float dpv = RO == 1 ? s[sb][MH + i] : w[i >> 2][i & 3];
              dsv[i] = pv[i] * (dpv - stl[sb][2 + (i >> 2)][i & 3]);
              if constexpr (CAP) dsv[i] *= gcap[i];
              if constexpr (DROP) {
                // dS from the dropped dP; the P this role hands to dV (or keeps) dropped too
                const bool kp = kept(q0 + sb * 32 + 8 * (2 * RO + (i >> 2)) + 4 * h + (i & 3));
                dsv[i] = pv[i] * ((kp ? dpv * p.drop.inv_keep : 0.f) - stl[sb][2 + (i >> 2)][i & 3]);
                pv[i] = kp ? pv[i] * p.drop.inv_keep : 0.f;
              }
            }
            // Packed to 16 bits (the accumulations' B operand): the half this role accumulates
            // stays, the half the partner accumulates goes to its slot (role 0: dS, role 1: P).
            i16x8 keep, give;
  #pragma unroll
            for (int i = 0; i < 8; ++i) {
              keep[i] = to16<IS_BF16>(RO == 0 ? pv[i] : dsv[i]);
              give[i] = to16<IS_BF16>(RO == 0 ? dsv[i] : pv[i]);
            }
            *reinterpret_cast<i16x8 GFA_LDS*>(slot(sb, RO == 0 ? 3 : 2, 0)) = give;
            pb_sh[sb * 2 + RO] = keep;
            store_ds(q0 + sb * 32, 2 * RO + h, RO == 0 ? give : keep);
          }
          barrier_lds();  // the halves handed back are in the slots
  #pragma unroll
          for (int sb = 0; sb < SB; ++sb)
            pb_sh[sb * 2 + 1 - RO] = *reinterpret_cast<const i16x8 GFA_LDS*>(slot(sb, RO == 0 ? 2 : 3, 0));
        };
        if (role == 0) {
          shared(std::integral_constant<int, 0>{});
        } else {
          shared(std::integral_constant<int, 1>{});
        }
      } else {
        // Hand-off form: role 0 computes P of all rows and hands it to role 1 (fp32).
        if (role == 0) {
          if constexpr (CAP) {
            make_p_cap(s, st[0], q0, pxr);
          } else {
            if constexpr (INIT) {
              make_p_init(s, q0);
            } else {
              make_p(s, st[0], q0);
            }
  #pragma unroll
            for (int sb = 0; sb < SB; ++sb) {
  #pragma unroll
              for (int j = 0; j < 4; ++j) {
                const f32x4 v = {s[sb][4 * j], s[sb][4 * j + 1], s[sb][4 * j + 2], s[sb][4 * j + 3]};
                *reinterpret_cast<f32x4 GFA_LDS*>(pxr + (sb * 4 + j) * 1024) = v;
              }
            }
          }
        }
        if constexpr (DROP) {
          if (role == 0) {
  #pragma unroll
            for (int sb = 0; sb < SB; ++sb)
  #pragma unroll
              for (int r = 0; r < 16; ++r)
                s[sb][r] = kept(q0 + sb * 32 + 8 * (r >> 2) + 4 * h + (r & 3)) ? s[sb][r] * p.drop.inv_keep : 0.f;
          }
        }
        barrier_lds();  // P of this tile is in px
        if (role == 1) {
  #pragma unroll
          for (int sb = 0; sb < SB; ++sb) {
            f32x4 pv4[4];
  #pragma unroll
            for (int j = 0; j < 4; ++j) pv4[j] = *reinterpret_cast<const f32x4 GFA_LDS*>(pxr + (sb * 4 + j) * 1024);
            if constexpr (DROP) {
  #pragma unroll
              for (int r = 0; r < 16; ++r)
                s[sb][r] = kept(q0 + sb * 32 + 8 * (r >> 2) + 4 * h + (r & 3)) ? s[sb][r] * p.drop.inv_keep : 0.f;
            }
            if constexpr (INIT) {
#pragma unroll
              for (int r = 0; r < 16; ++r) s[sb][r] *= pv4[r >> 2][r & 3];  // dS = P (dP - delta)
            } else {
              make_ds(s[sb], pv4, st[0][sb]);
            }
          }
        }
      }
      // s now holds P (role 0) or dS (role 1) for all 32 queries (shared form: pb_sh, packed).
      i16x8 pb[BQ / 16];
      if constexpr (SHARED) {
#pragma unroll
        for (int i = 0; i < BQ / 16; ++i) pb[i] = pb_sh[i];
      } else {
        pack(s, pb);
        if (role == 1) {
#pragma unroll
          for (int i = 0; i < BQ / 16; ++i) store_ds(q0 + (i >> 1) * 32, 2 * (i & 1) + h, pb[i]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
      accumulate(acc[0], tt, pb);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    } else {
      // S = Q K^T, dP = dO V^T, then dV^T += dO^T P and dK^T += Q^T dS.
      f32x16 s[SB], dp[SB];
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
        if (sb == 0) {
          auto ldq = [&](int i) { qload.load_part(i, row_n, qn); };
          if constexpr (VCHAIN1) {
            s[sb] = mma_chain1_lds_ld_vgpr<IS_BF16, KT, 4, NI>(qt, roff, sf[0], ldq);
          } else {
            s[sb] = chain_ld(std::integral_constant<int, NI>{}, qt, sf[0], ldq);
          }
        } else {
          s[sb] = chain(qt, sb * 32 * (2 * D), sf[0]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
        if (sb == 0) {
          auto ldd = [&](int i) { dload.load_part(i, row_n, dn); };
          if constexpr (VCHAIN1) {
            if constexpr (!CAP) {
              // P of the finished S block, one element per product of the dP chain (the
              // exponentials issue under the matrix unit): full-causal D=256 0.2%, non-causal 0.8%.
              dp[sb] = mma_chain1_lds_ld_vgpr_side<IS_BF16, KT, 4, NI>(dt, roff, sf[1], ldd, nullptr, [&](int kk) {
                float x = s[0][kk];
                asm volatile("" : "+v"(x));
                x = p_elem(x, st[0][0][kk >> 2][kk & 3]);
                asm volatile("" : "+v"(x));
                s[0][kk] = x;
              });
            } else {
              dp[sb] = mma_chain1_lds_ld_vgpr<IS_BF16, KT, 4, NI>(dt, roff, sf[1], ldd);
            }
          } else {
            dp[sb] = chain_ld(std::integral_constant<int, NI>{}, dt, sf[1], ldd);
          }
        } else {
          dp[sb] = chain(dt, sb * 32 * (2 * D), sf[1]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
      if constexpr (DROP) {
        // dS = P (kept dP / (1 - p) - delta); dV takes the kept P / (1 - p).
        make_p(s, st[0], q0, VCHAIN1);
#pragma unroll
        for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const bool kp = kept(q0 + sb * 32 + 8 * (r >> 2) + 4 * h + (r & 3));
            const float pv = s[sb][r];
            dp[sb][r] = pv * ((kp ? dp[sb][r] * p.drop.inv_keep : 0.f) - st[NS - 1][sb][r >> 2][r & 3]);
            s[sb][r] = kp ? pv * p.drop.inv_keep : 0.f;
          }
        }
      } else if constexpr (CAP) {
        // P of the capped scores, and dS = P (1 - tanh^2) (dP - delta), element by element.
        const bool need_mask = !(active && pair_full && q0 >= all_lo && q0 + BQ <= all_hi && q0 + BQ <= p.N);
#pragma unroll
        for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float t = cap_tanh(s[sb][r] * p.cap.cap_a);
            float pv = fast_exp2(t * p.cap.cap_log2 - st[0][sb][r >> 2][r & 3] * kLog2e);
            if (need_mask) pv = vis.has(q0 + sb * 32 + 8 * (r >> 2) + 4 * h + (r & 3)) ? pv : 0.f;
            s[sb][r] = pv;
            dp[sb][r] = pv * (1.f - t * t) * (dp[sb][r] - st[NS - 1][sb][r >> 2][r & 3]);
          }
        }
      } else {
        make_p(s, st[0], q0, VCHAIN1);
#pragma unroll
        for (int sb = 0; sb < SB; ++sb) {
          f32x4 pv4[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) pv4[j] = f32x4{s[sb][4 * j], s[sb][4 * j + 1], s[sb][4 * j + 2], s[sb][4 * j + 3]};
          make_ds(dp[sb], pv4, st[NS - 1][sb]);
        }
      }
      i16x8 pb[BQ / 16], dsb[BQ / 16];
      pack(s, pb);
      pack(dp, dsb);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
      accumulate(acc[0], dt, pb);
      __builtin_amdgcn_sched_barrier(0);
      accumulate(acc[NS - 1], qt, dsb);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    }
    // D >= 256: the accumulators fill the AGPRs and stay there. At D=64 everything fits the
    // VGPRs of two waves per SIMD; unpinned, the MFMAs write VGPRs directly (12% faster).
    if constexpr (D >= 256 && WPE == 1) {
#pragma unroll
      for (int i = 0; i < NS; ++i)
#pragma unroll
        for (int db = 0; db < DB; ++db) pin_agpr(acc[i][db]);
    }
  };

  // dS store: the stores this wave issues per tile, after that tile's copies of the next one.
  // The tile barrier leaves them in flight (they complete in issue order, behind the copies).
  const int nst_wave = (p.dsl.ds != nullptr && active) ? (SHARED ? 1 : (ROLES == 2 && role == 1 ? BQ / 16 : 0)) : 0;
  static_assert(BQ == 32, "the dS store addresses 32-row query tiles");
  char* ds_next = p.dsl.ds != nullptr ? ds_block(r_c, qt_c) : nullptr;  // block of tile (r_c, qt_c)
  for (int it = it_lo; it < it_hi; ++it) {
    const int cur = (it - it_lo) & 1;
    // tile `it` landed; every wave is done with the other buffers and px
    const int nst = it == it_lo ? 0 : nst_wave;
    if (nst == 0) {
      barrier_tile();
    } else if (nst == 1) {
      barrier_tile_n<1>();
    } else {
      barrier_tile_n<BQ / 16>();
    }
    const int q0 = qt_c * BQ;
    // Row statistics of this tile (rows q0 + sb*32 + 8g + 4h + 0..3; rows padded to a
    // multiple of 64), issued before the prefetch so they are not queued behind it.
    f32x4 st[NS][SB][4];
    if constexpr (SHARED) {
      // shared form: the statistics come from LDS (copied with the tile), read after the chain
    } else
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      // pair: LSE for role 0, delta for role 1 (the start of its chain)
      const float* sbase = (ROLES == 2 && role == 1) || i == 1 ? stat_kv1 : stat_kv0;
      const float* srow = sbase + (int64_t)r_c * p.lse_ld + q0 + 4 * h;
#pragma unroll
      for (int sb = 0; sb < SB; ++sb)
#pragma unroll
        for (int g = 0; g < 4; ++g) st[i][sb][g] = *reinterpret_cast<const f32x4*>(srow + sb * 32 + 8 * g);
    }
    // Next tile; the last iteration re-fetches its own tile into the idle buffer (never
    // read) so the loop body stays branch-free.
    int r_n = r_c + 1, qt_n = qt_c;
    if (r_n == p.R) {
      r_n = 0;
      qt_n = rotate ? (qt_c + 1 == qt_hi ? qt_lo : qt_c + 1) : qt_c - 1;
    }
    if (it + 1 >= it_hi) {
      r_n = r_c;
      qt_n = qt_c;
    }
    qload.rebase(q_kv + (int64_t)r_n * p.qv.sh, p.qv.sn, p.N);
    dload.rebase(d_kv + (int64_t)r_n * p.dov.sh, p.dov.sn, p.N);
    r_cur = r_c;
    ds_now = ds_next;
    if (p.dsl.ds != nullptr) ds_next = qt_n == qt_c && r_n == r_c + 1 ? ds_next + ds_slab_bytes : ds_block(r_n, qt_n);
    r_c = r_n;
    qt_c = qt_n;
    tile_step(smem + cur * TILE, smem + (2 + cur) * TILE, smem + (cur ^ 1) * TILE, smem + (2 + (cur ^ 1)) * TILE, px,
              stat_lds + cur * STB, stat_lds + (cur ^ 1) * STB, r_n, qt_n * BQ, q0, st);
  }
  drain_tile_copies();

  // ---- epilogue: lane = key, registers = head-dim rows 32*db + 8*g + 4*h + e ----
  if (STAGE_PAIR && p.q_splits == 1) {
    // This wave's dV or dK rows through its tile buffer (after every wave is done with the last
    // tiles), then whole rows to HBM. The lane index is made opaque so the addresses are
    // computed here, not kept live over the loop from the prologue.
    barrier_lds();
    char GFA_LDS* sblk = smem + wave * TILE;
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int r32 = ln & 31;
    const int hh = ln >> 5;
    const float osc = role == 0 ? 1.f : p.scale;  // dK carries the softmax scale
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        i16x4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = to16<IS_BF16>(acc[0][db][4 * g + e] * osc);
        const int c = 4 * db + g;  // 16-byte chunk of row r32 that holds these 4 + 4 elements
        *reinterpret_cast<i16x4 GFA_LDS*>(sblk + r32 * (2 * D) + ((c ^ swz<D>(r32)) << 4) + 8 * hh) = o4;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (role == 0) {
      store_rows_lds<D>(p.dv + (int64_t)b * p.dvv.sb + (int64_t)kvh * p.dvv.sh, p.dvv.sn, active ? p.N : 0, k0, ln, sblk);
    } else {
      store_rows_lds<D>(p.dk + (int64_t)b * p.dkv.sb + (int64_t)kvh * p.dkv.sh, p.dkv.sn, active ? p.N : 0, k0, ln, sblk);
    }
  } else if (STAGE && p.q_splits == 1) {
    // dV, then dK rows through this wave's stage block (idle since the prologue; laid out like
    // a tile), then whole rows to HBM. The lane index is made opaque here so the addresses are
    // computed here, not shared with the prologue's (which keeps them live over the loop).
    char GFA_LDS* sblk = (char GFA_LDS*)stage_raw + wave * TILE;
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int r32 = ln & 31;
    const int hh = ln >> 5;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const float osc = i == 0 ? 1.f : p.scale;  // dK carries the softmax scale
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          i16x4 o4;
#pragma unroll
          for (int e = 0; e < 4; ++e) o4[e] = to16<IS_BF16>(acc[i][db][4 * g + e] * osc);
          const int c = 4 * db + g;  // 16-byte chunk of row r32 that holds these 4 + 4 elements
          *reinterpret_cast<i16x4 GFA_LDS*>(sblk + r32 * (2 * D) + ((c ^ swz<D>(r32)) << 4) + 8 * hh) = o4;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (i == 0) {
        store_rows_lds<D>(p.dv + (int64_t)b * p.dvv.sb + (int64_t)kvh * p.dvv.sh, p.dvv.sn, active ? p.N : 0, k0, ln,
                          sblk);
      } else {
        store_rows_lds<D>(p.dk + (int64_t)b * p.dkv.sb + (int64_t)kvh * p.dkv.sh, p.dkv.sn, active ? p.N : 0, k0, ln,
                          sblk);
      }
    }
  } else if (active && key < p.N) {
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int which = ROLES == 2 ? role : i;       // 0: dV, 1: dK
      const float osc = which == 0 ? 1.f : p.scale;  // dK carries the softmax scale
      if (p.q_splits == 1) {
        uint16_t* orow = which == 0
                             ? p.dv + (int64_t)b * p.dvv.sb + (int64_t)kvh * p.dvv.sh + (int64_t)key * p.dvv.sn
                             : p.dk + (int64_t)b * p.dkv.sb + (int64_t)kvh * p.dkv.sh + (int64_t)key * p.dkv.sn;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            i16x4 o4;
#pragma unroll
            for (int e = 0; e < 4; ++e) o4[e] = to16<IS_BF16>(acc[i][db][4 * g + e] * osc);
            *reinterpret_cast<i16x4*>(orow + db * 32 + 8 * g + 4 * h) = o4;
          }
        }
      } else {
        // fp32 partials [split][dk|dv][b][kvh][key][d], dK already scaled.
        const int64_t plane = (int64_t)p.B * p.Hkv * p.N * D;
        const int64_t rowoff = (((int64_t)b * p.Hkv + kvh) * p.N + key) * D;
        float* dst = p.part + (int64_t)split * 2 * plane + (which == 0 ? plane : 0) + rowoff;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const f32x4 v4 = {acc[i][db][4 * g] * osc, acc[i][db][4 * g + 1] * osc, acc[i][db][4 * g + 2] * osc,
                              acc[i][db][4 * g + 3] * osc};
            *reinterpret_cast<f32x4*>(dst + db * 32 + 8 * g + 4 * h) = v4;
          }
        }
      }
    }
  }
}

// dK/dV = sum over q_splits of the fp32 partials, in split order, cast to the input dtype.
// One thread converts 8 consecutive head-dim elements of one (tensor, b, kvh, key) row.
template <bool IS_BF16>
__global__ __launch_bounds__(256) void dkv_reduce_kernel(const BwdDkvParams p, int D) {
  const int64_t plane = (int64_t)p.B * p.Hkv * p.N * D;
  const int64_t n8 = 2 * plane / 8;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n8) return;
  const int64_t e0 = i * 8;
  const int which = e0 >= plane ? 1 : 0;
  const int64_t off = e0 - which * plane;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int s = 0; s < p.q_splits; ++s) {
    const float* src = p.part + (int64_t)s * 2 * plane + which * plane + off;
    const f32x4 a = *reinterpret_cast<const f32x4*>(src);
    const f32x4 c = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[e] += a[e];
      acc[4 + e] += c[e];
    }
  }
  const int d = (int)(off % D);
  int64_t rest = off / D;
  const int key = (int)(rest % p.N);
  rest /= p.N;
  const int kvh = (int)(rest % p.Hkv);
  const int b = (int)(rest / p.Hkv);
  const RowView& v = which ? p.dvv : p.dkv;
  uint16_t* dst = (which ? p.dv : p.dk) + (int64_t)b * v.sb + (int64_t)kvh * v.sh + (int64_t)key * v.sn + d;
  i16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = to16<IS_BF16>(acc[e]);
  *reinterpret_cast<i16x8*>(dst) = o;
}

// Explicit instantiations of every built variant (device code and host launch stubs).
#define GFA_DKV_INST(DD, BB, WW, RR, EE, CC, XX)                                                  \
  template __global__ void bwd_dkv_kernel<DD, BB, true, WW, RR, EE, CC, XX>(const BwdDkvParams);  \
  template __global__ void bwd_dkv_kernel<DD, BB, false, WW, RR, EE, CC, XX>(const BwdDkvParams);
GFA_DKV_INST(512, 32, 4, 2, 1, false, false)
GFA_DKV_INST(256, 32, 4, 1, 1, false, false)
GFA_DKV_INST(256, 32, 4, 2, 2, false, false)
GFA_DKV_INST(64, 32, 4, 1, 2, false, false)
GFA_DKV_INST(128, 32, 4, 2, 2, false, false)
// Soft-capped and dropout instances (D=256 runs the one-wave form; the windowed pair starts its
// chains from the row statistics).
#define GFA_DKV_EXT(CC, XX)                   \
  GFA_DKV_INST(512, 32, 4, 2, 1, CC, XX)      \
  GFA_DKV_INST(256, 32, 4, 1, 1, CC, XX)      \
  GFA_DKV_INST(64, 32, 4, 1, 2, CC, XX)       \
  GFA_DKV_INST(128, 32, 4, 2, 2, CC, XX)
GFA_DKV_EXT(true, false)
GFA_DKV_EXT(false, true)
#undef GFA_DKV_EXT
#undef GFA_DKV_INST
template __global__ void dkv_reduce_kernel<true>(const BwdDkvParams, int);
template __global__ void dkv_reduce_kernel<false>(const BwdDkvParams, int);

template <int D, int BQ, bool IS_BF16, int NW, int ROLES, int WPE, bool CAP, bool DROP>
static hipError_t launch_dkv_t(const BwdDkvParams& p, hipStream_t stream) {
  const unsigned stage_bytes = dkv_stages_rows(D, ROLES) ? NW * BQ * D * 2 : 0;  // the kernel's stage_raw
  hipLaunchKernelGGL((bwd_dkv_kernel<D, BQ, IS_BF16, NW, ROLES, WPE, CAP, DROP>), dim3(p.nblocks), dim3(NW * 64),
                     stage_bytes, stream, p);
  return hipGetLastError();
}

// Built dK/dV variants: (head dim, queries per tile, waves per workgroup, waves per 32 keys,
// waves per SIMD).
hipError_t launch_bwd_dkv(const BwdDkvParams& p, int D, int bq, int nw, int roles, bool bf16, bool cap, bool drop,
                          hipStream_t stream) {
#define GFA_DKV_CASE(DD, BB, WW, RR, EE, CC, XX)                                           \
  if (D == DD && bq == BB && nw == WW && roles == RR && cap == CC && drop == XX) {         \
    return bf16 ? launch_dkv_t<DD, BB, true, WW, RR, EE, CC, XX>(p, stream)                \
                : launch_dkv_t<DD, BB, false, WW, RR, EE, CC, XX>(p, stream);              \
  }
  GFA_DKV_CASE(512, 32, 4, 2, 1, false, false)
  GFA_DKV_CASE(256, 32, 4, 1, 1, false, false)
  GFA_DKV_CASE(256, 32, 4, 2, 2, false, false)
  GFA_DKV_CASE(64, 32, 4, 1, 2, false, false)
  GFA_DKV_CASE(128, 32, 4, 2, 2, false, false)
#define GFA_DKV_EXT(CC, XX)                   \
  GFA_DKV_CASE(512, 32, 4, 2, 1, CC, XX)      \
  GFA_DKV_CASE(256, 32, 4, 1, 1, CC, XX)      \
  GFA_DKV_CASE(64, 32, 4, 1, 2, CC, XX)       \
  GFA_DKV_CASE(128, 32, 4, 2, 2, CC, XX)
  GFA_DKV_EXT(true, false)
  GFA_DKV_EXT(false, true)
#undef GFA_DKV_EXT
#undef GFA_DKV_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_dkv_reduce(const BwdDkvParams& p, int D, bool bf16, hipStream_t stream) {
  const int64_t n8 = 2 * (int64_t)p.B * p.Hkv * p.N * D / 8;
  const int blocks = (int)((n8 + 255) / 256);
  if (bf16) {
    hipLaunchKernelGGL(dkv_reduce_kernel<true>, dim3(blocks), dim3(256), 0, stream, p, D);
  } else {
    hipLaunchKernelGGL(dkv_reduce_kernel<false>, dim3(blocks), dim3(256), 0, stream, p, D);
  }
  return hipGetLastError();
}

}  // namespace gfa
