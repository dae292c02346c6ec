// GQA flash-attention backward, dQ kernel with the fused delta prologue (hot-path row R2).
//
// Semantics follow /root/reference/flash_attn/attention.py:687-797 run with
// STORE_DELTA=True (launch at 1506-1523):
//   delta_i = sum_d dO_id * O_id                        (fp32, stored for the dKV kernel)
//   P_ij    = exp2(s*log2e * q_i.k_j - LSE_i*log2e)      (masked -> 0)
//   dS_ij   = P_ij * (dO_i.v_j - delta_i)                 (masked -> 0, cast to input dtype)
//   dQ_i    = s * sum_j dS_ij k_j
//
// MI355X design: D <= 256, one wave owns 32 query rows of one head and keeps its Q and dO
// rows in VGPRs (B operands of S^T = K Q^T and dP^T = V dO^T, lane = query). D = 512, a wave
// pair owns them and splits the work by role: role 0 keeps the Q rows and runs S^T, role 1
// keeps the dO rows, computes delta and runs dP^T, both over the full head dim; each turns half
// of the score block into dS (swapping the chain-result halves it needs through LDS, then the
// packed dS halves) and accumulates its head-dim half of dQ^T. P^T and dS^T then live on the
// query lanes with per-lane LSE, and dQ^T += K^T dS^T reads its A operand with ds_read_b64_tr_b16 from the
// same row-major K tile that fed S^T. K and V tiles are double-buffered in LDS via buffer
// loads that write LDS directly; the copies of the next tile are spread over the chains.
#include "gfa_common.h"
#include "gfa_params.h"
#include "gfa_launch.h"

namespace gfa {

// One wave per 32 rows at D >= 128 stages its rows (and its dQ rows) through LDS in whole-row
// copies. At D = 64 three workgroups share a CU and hide the per-lane loads' latency; staging
// there only adds a barrier and a round trip (measured 0.7% slower).
constexpr bool dq_stages_rows(int D, int split) { return split == 1 && D >= 128; }

template <int D, int BKV, bool IS_BF16, int NW, int SPLIT, bool CAP, bool DROP>
__global__ __launch_bounds__(NW * 64, 1) void bwd_dq_kernel(const BwdDqParams p_arg) {
  constexpr int DH = D / SPLIT;  // head-dim slice of dQ^T one wave accumulates
  constexpr int KT = D / 16;     // k-steps of a score chain (always the full head dim)
  constexpr int DBH = DH / 32;
  constexpr int SB = BKV / 32;
  constexpr int TILE = BKV * D * 2;
  // Pair: the roles share the dS work, each turning half of the registers into dS (see the
  // tile step; 3% faster than both computing all of it). Exchange area per score block: S half
  // and dP^T - delta half (2 KB each, fp32), then the two dS halves (1 KB each, packed 16-bit).
  constexpr bool SHARED = SPLIT == 2;
  constexpr int XSB = 2 * 2048 + 2 * 1024;
  constexpr int XCH = SHARED ? SB * XSB : 0;  // per pair
  static_assert(BKV == 32, "32-key tiles: one 32 x 32 score block per tile and wave");
  static_assert(SPLIT == 1 || SPLIT == 2, "one wave or a wave pair per 32 query rows");
  static_assert(D == 64 || D == 128 || D == 256 || D == 512, "head dim must be 64, 128, 256 or 512");
  // The swizzle permutes 16-chunk groups, so a head-dim half must be whole groups.
  static_assert(SPLIT == 1 || DH % 128 == 0, "a head-dim split needs halves of 128 or more elements");
  constexpr bool STAGE = dq_stages_rows(D, SPLIT);
  constexpr bool PRIO = D <= 128;  // several waves per SIMD
  static_assert(!STAGE || NW == 4, "each wave stages its Q rows in one of four tile buffers");

  // Four distinct LDS tile objects (not one array indexed by a buffer id): with the loop
  // unrolled by two every access names its buffer statically, so the compiler's wait
  // insertion can tell the in-flight copies (into the other buffers) from the tile being
  // read and does not stall on them.
  __shared__ __attribute__((aligned(1024))) char k_lds0[TILE];
  __shared__ __attribute__((aligned(1024))) char k_lds1[TILE];
  __shared__ __attribute__((aligned(1024))) char v_lds0[TILE];
  __shared__ __attribute__((aligned(1024))) char v_lds1[TILE];
  __shared__ __attribute__((aligned(1024))) char xch_raw[XCH > 0 ? (NW / 2) * XCH : 16];
  __shared__ int work_slot[3];  // the block the run-time work hand-out gave the workgroup (two slots), its state
  // STAGE: each wave stages its dO rows, then its O rows, and at the end its dQ rows in its
  // TILE-byte block of this launch-sized array (its Q rows go to one of the tile buffers, idle
  // before the loop). Dynamic, so the compiler's occupancy estimate (static LDS only) is that of
  // the tile buffers: declared static, the 4 * TILE more bytes lower it, and the loop is then
  // scheduled into a larger register set with extra AGPR copies per step.
  extern __shared__ __attribute__((aligned(1024))) char stage_raw[];
  char GFA_LDS* const K0 = (char GFA_LDS*)k_lds0;
  char GFA_LDS* const K1 = (char GFA_LDS*)k_lds1;
  char GFA_LDS* const V0 = (char GFA_LDS*)v_lds0;
  char GFA_LDS* const V1 = (char GFA_LDS*)v_lds1;
  char GFA_LDS* xch = (char GFA_LDS*)xch_raw;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int unit = wave / SPLIT;
  // Pair (SPLIT == 2): role 0 runs S^T = K Q^T, role 1 dP^T = V dO^T, each over the full head
  // dim; they swap the results and each accumulates its head-dim half dh = role of dQ^T.
  const int dh = SPLIT == 2 ? (wave & 1) : 0;
  const int h = lane >> 5;
  const int l32 = lane & 31;

  // One block of the static grid (vblock = its workgroup id there): the body below, run once per
  // block the workgroup is given.
  // D=512 (DYN): the host may run the kernel as a persistent grid, several blocks per workgroup.
  constexpr bool DYN = D == 512;
  auto body = [&](const int vblock) __attribute__((always_inline)) {
  const BwdDqParams& p = DYN ? *kernel_args<BwdDqParams>() : p_arg;
  int lid = xcd_remap(vblock, p.g.nblocks, p.g.n_hg);
  const int hg = lid % p.g.n_hg;
  lid /= p.g.n_hg;
  const int kvh = lid % p.Hkv;
  lid /= p.Hkv;
  const int b = lid % p.B;
  lid /= p.B;
  // Full causal: longest rows first. Sliding window: nearly every block has the same key
  // range, so the short first blocks (queries below the window) go first; they end at
  // staggered times and spread the later blocks' prologues (row copies) over time instead of
  // every CU loading its rows at once.
  const int qsb = (p.causal && p.window <= 0) ? (p.g.n_qsb - 1 - lid) : lid;

  const int head = kvh * p.R + hg * p.g.hpw + (unit % p.g.hpw);
  const int q0 = (qsb * p.g.qbw + unit / p.g.hpw) * 32;
  const int wg_q_lo = qsb * p.g.qbw * 32;
  const int wg_q_hi = min(p.N, wg_q_lo + p.g.qbw * 32);

  const bool swa = p.causal && p.window > 0;
  int k_lo = 0, k_hi = p.N;
  if (p.causal) {
    k_hi = wg_q_hi;
    if (swa) k_lo = max(0, wg_q_lo - p.window + 1);
  }
  // Segment table (optional): the workgroup's queries see keys from the first query's
  // segment start to the last query's segment end (both rows are non-decreasing).
  const int* slo = p.seg_lo ? p.seg_lo + (int64_t)b * p.N : nullptr;
  const int* shi = p.seg_lo ? p.seg_hi + (int64_t)b * p.N : nullptr;
  if (slo) {
    k_lo = max(k_lo, clamp_n(slo[wg_q_lo], p.N));
    k_hi = min(k_hi, clamp_n(shi[wg_q_hi - 1], p.N));
  }
  const int t_lo = k_lo / BKV;
  // Even tile count (the loop is unrolled by two): an odd range gets one extra tile past
  // the workgroup's keys, which is fully masked (dS = 0; zero-filled past the sequence end).
  const int t_hi = t_lo + ((((k_hi + BKV - 1) / BKV) - t_lo + 1) & ~1);

  const bool active = q0 < p.N;
  const int q_last = q0 + 31;
  int all_lo = 0, all_hi = p.N;
  if (p.causal) {
    all_hi = min(p.N, q0 + 1);
    if (swa) all_lo = q_last - p.window + 1;
  }

  const int q = q0 + l32;
  const int qrow = min(q, p.N - 1);
  VisRange vis = keys_of_query(q, p.N, p.causal, p.window);
  if (slo) {
    if (active) {
      all_lo = max(all_lo, clamp_n(slo[min(q_last, p.N - 1)], p.N));
      all_hi = min(all_hi, clamp_n(shi[q0], p.N));
    }
    vis = intersect(vis, clamp_n(slo[qrow], p.N), clamp_n(shi[qrow], p.N));
  }
  int koff[8];
#pragma unroll
  for (int kl = 0; kl < 8; ++kl) koff[kl] = l32 * (2 * D) + (((2 * kl + h) ^ swz<D>(l32)) << 4);

  const uint16_t* kbase = p.k + (int64_t)b * p.kv.sb + (int64_t)kvh * p.kv.sh;
  const uint16_t* vbase = p.v + (int64_t)b * p.vv.sb + (int64_t)kvh * p.vv.sh;
  TileLoader<D, BKV, NW> kload, vload;
  kload.init(kbase, p.kv.sn, p.N, wave, lane);
  vload.init(vbase, p.vv.sn, p.N, wave, lane);

  // ---- B operands of the score chains, resident; delta ----
  // One wave: Q and dO rows (full head dim); STAGE: staged through LDS by whole-row copies and
  // read back in the operand layout, the first key tile's copies issued before the O rows are
  // read for delta. Pair: role 0 the Q rows, role 1 the dO rows (loaded per lane; the D = 512
  // pair's prologue is a small part of its blocks); role 1 also computes delta and hands it to
  // role 0 below.
  // The row's LSE first: its load then overlaps the row copies.
  const float lse_log2 = p.lse[((int64_t)b * p.Hq + head) * p.lse_ld + qrow] * kLog2e;
  i16x8 qf[KT];                      // Q rows (one wave / role 0) or dO rows (role 1)
  i16x8 df[SPLIT == 1 ? KT : 1];     // dO rows (one wave)
  float dpart = 0.f;
  {
    const uint16_t* qb = p.q + (int64_t)b * p.qv.sb + (int64_t)head * p.qv.sh;
    const uint16_t* db = p.dout + (int64_t)b * p.dov.sb + (int64_t)head * p.dov.sh;
    const uint16_t* ob = p.o + (int64_t)b * p.ov.sb + (int64_t)head * p.ov.sh;
    if constexpr (STAGE) {
      // Each wave's own blocks: Q in tile buffer `wave`, dO and then O in its stage block.
      char GFA_LDS* qblk = wave == 0 ? K0 : wave == 1 ? K1 : wave == 2 ? V0 : V1;
      char GFA_LDS* sblk = (char GFA_LDS*)stage_raw + wave * TILE;
      copy_rows_lds<D>(qb, p.qv.sn, p.N, q0, lane, qblk);
      copy_rows_lds<D>(db, p.dov.sn, p.N, q0, lane, sblk);
      drain_tile_copies();
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
        qf[kk] = lds_read16(qblk, koff[kk & 7] + 256 * (kk >> 3));
        df[kk] = lds_read16(sblk, koff[kk & 7] + 256 * (kk >> 3));
      }
      barrier_lds();  // every wave has read its Q block out of the tile buffers
      copy_rows_lds<D>(ob, p.ov.sn, p.N, q0, lane, sblk);
      if (t_lo < t_hi) {
        kload.load(t_lo * BKV, K0);
        vload.load(t_lo * BKV, V0);
      }
      drain_tile_copies();
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
        const i16x8 of = lds_read16(sblk, koff[kk & 7] + 256 * (kk >> 3));
#pragma unroll
        for (int e = 0; e < 8; ++e) dpart += from16<IS_BF16>(df[kk][e]) * from16<IS_BF16>(of[e]);
      }
    } else {
      const uint16_t* qr = qb + (int64_t)qrow * p.qv.sn + 8 * h;
      const uint16_t* dr = db + (int64_t)qrow * p.dov.sn + 8 * h;
      const uint16_t* orow = ob + (int64_t)qrow * p.ov.sn + 8 * h;
      if constexpr (SPLIT == 1) {
#pragma unroll
        for (int kk = 0; kk < KT; ++kk) {
          qf[kk] = *reinterpret_cast<const i16x8*>(qr + 16 * kk);
          df[kk] = *reinterpret_cast<const i16x8*>(dr + 16 * kk);
          const i16x8 of = *reinterpret_cast<const i16x8*>(orow + 16 * kk);
#pragma unroll
          for (int e = 0; e < 8; ++e) dpart += from16<IS_BF16>(df[kk][e]) * from16<IS_BF16>(of[e]);
        }
      } else {
        const uint16_t* br = dh == 0 ? qr : dr;
#pragma unroll
        for (int kk = 0; kk < KT; ++kk) qf[kk] = *reinterpret_cast<const i16x8*>(br + 16 * kk);
        if (dh == 1) {
#pragma unroll
          for (int kk = 0; kk < KT; ++kk) {
            const i16x8 of = *reinterpret_cast<const i16x8*>(orow + 16 * kk);
#pragma unroll
            for (int e = 0; e < 8; ++e) dpart += from16<IS_BF16>(qf[kk][e]) * from16<IS_BF16>(of[e]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int kk = 0; kk < KT; ++kk) pin_vgpr(qf[kk]);
  if constexpr (SPLIT == 1) {
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) pin_vgpr(df[kk]);
  }
  const float delta = halves_sum(dpart);  // stored after the loop
  // The S^T and dP^T chains accumulate in VGPRs through inline-asm MFMAs (mma32_vgpr), so the dS
  // work and the pair's exchange read them without AGPR moves (16-32 per tile). The dP^T chain
  // starts from -delta (the lane's query; a block of 16 VGPRs the chain reads as its C operand),
  // so it yields dP - delta and dS costs one multiply per element; in a pair role 1 runs that
  // chain and role 0 receives its half already shifted. DROP scales dP by the mask before delta
  // is subtracted, so there the chain starts from zero and dS subtracts delta: in a pair both
  // roles then subtract it from their dP half, but only role 1 holds the dO rows it comes from,
  // and it hands delta over through the pair's exchange area (idle until the first tile step,
  // which starts behind a barrier).
  constexpr bool DP_FROM_DELTA = !DROP;
  // One wave at D = 256: P^T is computed during the dP^T chain (one of the block's 16 elements
  // per product), so the tile step below only multiplies it by dP^T - delta.
  constexpr bool EARLY_P = SPLIT == 1 && D > 128;
  static_assert(!EARLY_P || KT == 16, "one exponential per product of the dP^T chain");
  f32x16 neg_delta;
#pragma unroll
  for (int r = 0; r < 16; ++r) neg_delta[r] = -delta;
  float delta_row = delta;
  if constexpr (SPLIT == 2 && !DP_FROM_DELTA) {
    float GFA_LDS* const slot = reinterpret_cast<float GFA_LDS*>(xch + (wave >> 1) * XCH) + lane;
    if (dh == 1) *slot = delta;
    barrier_lds();
    delta_row = *slot;
  }

  f32x16 acc[DBH];
#pragma unroll
  for (int i = 0; i < DBH; ++i) acc[i] = f32x16{};

  // DROP: the row key of this lane's query; dP of a dropped entry is 0, a kept one / (1 - p).
  const unsigned drow = DROP ? drop_row(p.drop.seed_lo, p.drop.seed_hi, b * p.Hq + head, q) : 0u;
  auto dp_kept = [&](float dpv, int key) __attribute__((always_inline)) {
    if constexpr (DROP) {
      return drop_keep(drow, key, p.drop.thresh) ? dpv * p.drop.inv_keep : 0.f;
    } else {
      return dpv;
    }
  };
  // P of a raw score, times dS's soft-cap factor 1 - tanh^2 with CAP (so dS = this * (dP - delta)).
  auto p_of = [&](float sv) __attribute__((always_inline)) {
    if constexpr (CAP) {
      const float t = cap_tanh(sv * p.cap.cap_a);
      return fast_exp2(t * p.cap.cap_log2 - lse_log2) * (1.f - t * t);
    } else {
      return fast_exp2(sv * p.scale_log2 - lse_log2);
    }
  };

  int toffA[4], toffB[4];  // K tile read transposed (A operand of dQ^T = K^T dS^T)
  {
    const int t16 = lane & 15;
    const int half16 = (lane >> 4) & 1;
    const int rA = 4 * h + (t16 >> 2);
    const int rB = rA + 8;
#pragma unroll
    for (int dl = 0; dl < 4; ++dl) {
      const int c = 4 * dl + 2 * half16 + ((t16 >> 1) & 1);
      toffA[dl] = rA * (2 * D) + ((c ^ swz<D>(rA)) << 4) + (t16 & 1) * 8 + dh * DH * 2;
      toffB[dl] = rB * (2 * D) + ((c ^ swz<D>(rB)) << 4) + (t16 & 1) * 8 + dh * DH * 2;
    }
  }

  // Shared dS (pair). Role RO turns the registers 8 RO .. 8 RO + 7 of a score block (keys
  // 8 g + 4 h + 0..3, g = 2 RO, 2 RO + 1) into dS: it first hands its partner the half of its
  // own chain result the partner needs (role 0: S^T of registers 8..15; role 1: dP^T - delta of
  // 0..7), computes its dS half, packs it to 16 bits and hands that over, so that each wave ends
  // with the full dS^T and no exponential is computed twice.
  auto shared_ds = [&](auto ro, const f32x16 (&own)[SB], i16x8 (&dsb)[BKV / 16], int k0)
                       __attribute__((always_inline)) {
    constexpr int RO = decltype(ro)::value;
    constexpr int MH = 8 * RO, OH = 8 * (1 - RO);
    char GFA_LDS* xp = xch + (wave >> 1) * XCH + lane * 16;
    // slots of score block sb: 0 S half, 1 dP half (two 1 KB f32x4 planes each), 2 / 3 the dS
    // halves of role 0 / 1 (one 1 KB plane of i16x8 each)
    auto slot = [&](int sb, int k) __attribute__((always_inline)) {
      return xp + sb * XSB + (k < 2 ? k * 2048 : 4096 + (k - 2) * 1024);
    };
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const f32x4 v = {own[sb][OH + 4 * j], own[sb][OH + 4 * j + 1], own[sb][OH + 4 * j + 2], own[sb][OH + 4 * j + 3]};
        *reinterpret_cast<f32x4 GFA_LDS*>(slot(sb, RO) + j * 1024) = v;
      }
    }
    barrier_lds();  // both halves of both chain results are in the slots
    const bool need_mask = !(active && k0 + BKV <= all_hi && k0 >= all_lo);
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) {
      f32x4 w[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) w[j] = *reinterpret_cast<const f32x4 GFA_LDS*>(slot(sb, 1 - RO) + j * 1024);
      float ds[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float sv = RO == 0 ? own[sb][MH + i] : w[i >> 2][i & 3];
        const float dpv = RO == 1 ? own[sb][MH + i] : w[i >> 2][i & 3];
        const int key = k0 + sb * 32 + 8 * ((MH + i) >> 2) + 4 * h + (i & 3);
        ds[i] = p_of(sv) * (DP_FROM_DELTA ? dpv : dp_kept(dpv, key) - delta_row);
      }
      if (need_mask) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int key = k0 + sb * 32 + 8 * ((MH + i) >> 2) + 4 * h + (i & 3);
          ds[i] = vis.has(key) ? ds[i] : 0.f;
        }
      }
      i16x8 mine;
#pragma unroll
      for (int i = 0; i < 8; ++i) mine[i] = to16<IS_BF16>(ds[i]);
      *reinterpret_cast<i16x8 GFA_LDS*>(slot(sb, 2 + RO)) = mine;
      dsb[sb * 2 + RO] = mine;
    }
    barrier_lds();  // both dS halves are in the slots
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) dsb[sb * 2 + 1 - RO] = *reinterpret_cast<const i16x8 GFA_LDS*>(slot(sb, 3 - RO));
  };

  // One key tile: wait for it, then S^T = K Q^T and dP^T = V dO^T with the copies of tile
  // t+1 into the other buffers spread over the two chains (a run of copy issues would hold
  // up the in-order MFMA stream), dS^T, and dQ^T += K^T dS^T.
  constexpr int NI = TileLoader<D, BKV, NW>::NI;  // copy instructions per tile and wave
  auto step = [&](int t, const char GFA_LDS* kt, const char GFA_LDS* vt, char GFA_LDS* kn,
                  char GFA_LDS* vn) __attribute__((always_inline)) {
    barrier_tile();  // tile t landed; every wave is done reading the other buffers
    // The last step re-fetches its own tile into the idle buffers (never read) so the
    // body stays branch-free.
    const int rn = min(t + 1, t_hi - 1) * BKV;
    const int k0 = t * BKV;

    // No per-pair skip: a tile this pair cannot see is fully masked below, and the
    // straight-line body keeps the accumulators resident in registers.
    f32x16 s[SB], dp[SB];
    i16x8 dsb[BKV / 16];  // dS^T, packed 16-bit: the B operand of dQ^T += K^T dS^T
    if constexpr (SPLIT == 1 && D <= 128) {
      // D <= 128: the two chains interleaved product by product (two fragments ahead each), so
      // no MFMA waits on the one before it: 1.2% (D=128) and 1.5% (D=64) faster; at D=256 1% slower.
      mma_chain2_lds_ld_vgpr<IS_BF16, KT, 2, 2 * NI>(s[0], dp[0], kt, vt, koff, qf, df, [&](int i) {
        if (i < NI) {
          kload.load_part(i, rn, kn);
        } else {
          vload.load_part(i - NI, rn, vn);
        }
      }, DP_FROM_DELTA ? &neg_delta : nullptr);
      __builtin_amdgcn_sched_barrier(0);
    } else if constexpr (SPLIT == 1) {
      s[0] = mma_chain1_lds_ld_vgpr<IS_BF16, KT, 4, NI>(kt, koff, qf, [&](int i) { kload.load_part(i, rn, kn); });
      __builtin_amdgcn_sched_barrier(0);
      // P^T of the finished S^T block, one element per product of the dP^T chain: the
      // exponentials then issue under the matrix unit instead of after the chain (0.2-0.9%).
      dp[0] = mma_chain1_lds_ld_vgpr_side<IS_BF16, KT, 4, NI>(
          vt, koff, df, [&](int i) { vload.load_part(i, rn, vn); }, DP_FROM_DELTA ? &neg_delta : nullptr,
          [&](int kk) {
            float x = s[0][kk];
            asm volatile("" : "+v"(x));
            x = p_of(x);
            asm volatile("" : "+v"(x));
            s[0][kk] = x;
          });
      __builtin_amdgcn_sched_barrier(0);
    } else {
      // This role's chain over the full head dim, with both tiles' copies spread over it;
      // then the swap: each wave reads S^T and dP^T - delta from the exchange slots.
      // The tile is picked by a (wave-uniform) branch, not a pointer select: each path then
      // reads a statically named LDS object, which lets the compiler's wait insertion tell the
      // reads from the in-flight copies (with a select it waits for the copies every product:
      // 2.5x slower).
      f32x16 own[SB];
      auto run = [&](const char GFA_LDS* ct, const f32x16* c0) __attribute__((always_inline)) {
        auto ld = [&](int i) {
          if (i < NI) {
            kload.load_part(i, rn, kn);
          } else {
            vload.load_part(i - NI, rn, vn);
          }
        };
        own[0] = mma_chain1_lds_ld_vgpr<IS_BF16, KT, 4, 2 * NI>(ct, koff, qf, ld, c0);
        __builtin_amdgcn_sched_barrier(0);
      };
      if (dh == 0) {
        run(kt, nullptr);
      } else {
        run(vt, DP_FROM_DELTA ? &neg_delta : nullptr);
      }
      if (dh == 0) {
        shared_ds(std::integral_constant<int, 0>{}, own, dsb, k0);
      } else {
        shared_ds(std::integral_constant<int, 1>{}, own, dsb, k0);
      }
    }

    if constexpr (!SHARED) {
    const bool need_mask = !(active && k0 + BKV <= all_hi && k0 >= all_lo);
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float dpd = DP_FROM_DELTA ? dp[sb][r]
                                        : dp_kept(dp[sb][r], k0 + sb * 32 + 8 * (r >> 2) + 4 * h + (r & 3)) - delta_row;
        s[sb][r] = (EARLY_P ? s[sb][r] : p_of(s[sb][r])) * dpd;
      }
    }
    if (need_mask) {
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + sb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          s[sb][r] = vis.has(key) ? s[sb][r] : 0.f;
        }
      }
    }
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) dsb[sb * 2 + (r >> 3)][r & 7] = to16<IS_BF16>(s[sb][r]);
    }
    }
    // dQ^T[half] += K^T[half] dS^T, A operand read transposed from the K tile.
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
    mma_tr_accumulate<IS_BF16, D, DBH, BKV / 16, 2, 1>(acc, kt, toffA, toffB, dsb);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int db = 0; db < DBH; ++db) pin_agpr(acc[db]);
  };

  if (!STAGE && t_lo < t_hi) {  // STAGE: issued in the prologue
    kload.load(t_lo * BKV, K0);
    vload.load(t_lo * BKV, V0);
  }
  for (int t = t_lo; t < t_hi; t += 2) {
    step(t, K0, V0, K1, V1);
    __builtin_amdgcn_sched_barrier(0);
    step(t + 1, K1, V1, K0, V0);
    __builtin_amdgcn_sched_barrier(0);
  }
  drain_tile_copies();

  // Delta is stored here, not after the prologue: a store there would hold up the first tile
  // barrier (its vmcnt wait covers stores too). Written for every row of an active block, also
  // the rows past N in the last one (they repeat row N-1's value): the dK/dV kernel reads whole
  // 32-row tiles of delta and relies on them being finite (its dS = P (dP - delta) with P = 0
  // on those rows).
  if (active && dh == SPLIT - 1 && h == 0) p.delta[((int64_t)b * p.Hq + head) * p.lse_ld + q] = delta;
  if constexpr (STAGE) {
    // dQ rows through this wave's stage block (idle since the prologue; laid out like a tile),
    // then whole rows to HBM: per-lane stores of 4 elements straight from the accumulator
    // layout touch 32 rows per instruction and hold the block's end up.
    char GFA_LDS* sblk = (char GFA_LDS*)stage_raw + wave * TILE;
    // The lane index, opaque from here: the epilogue's addresses are then computed here, not
    // shared with the prologue's (which would keep them live, in AGPR copies, over the loop).
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int r32 = ln & 31;
    const int hh = ln >> 5;
#pragma unroll
    for (int db = 0; db < DBH; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        i16x4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = to16<IS_BF16>(acc[db][4 * g + e] * p.scale);
        const int c = 4 * db + g;  // 16-byte chunk of row l32 that holds these 4 + 4 elements
        *reinterpret_cast<i16x4 GFA_LDS*>(sblk + r32 * (2 * D) + ((c ^ swz<D>(r32)) << 4) + 8 * hh) = o4;
      }
      __builtin_amdgcn_sched_barrier(0);  // one block at a time (else every accumulator is read out first)
    }
    store_rows_lds<D>(p.dq + (int64_t)b * p.dqv.sb + (int64_t)head * p.dqv.sh, p.dqv.sn, active ? p.N : 0, q0, ln,
                      sblk);
  } else if (active && q < p.N) {
    uint16_t* dqrow = p.dq + (int64_t)b * p.dqv.sb + (int64_t)head * p.dqv.sh + (int64_t)q * p.dqv.sn + dh * DH;
#pragma unroll
    for (int db = 0; db < DBH; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        i16x4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = to16<IS_BF16>(acc[db][4 * g + e] * p.scale);
        *reinterpret_cast<i16x4*>(dqrow + db * 32 + 8 * g + 4 * h) = o4;
      }
    }
  }
  };

  // Static grid: the workgroup's own block. Run-time hand-out (p.sched.wq): blocks from the
  // per-XCD queues until all are empty; the barrier that publishes a block also keeps every wave's
  // LDS use of the previous block ahead of the next one's copies.
  if constexpr (!DYN) {
    body((int)blockIdx.x);
    return;
  }
  if (threadIdx.x == 0) work_slot[2] = 0;  // queues found empty (work_next)
  int slot = 0;
  auto fetch = [&]() __attribute__((always_inline)) {
    const BwdDqParams& pa = *kernel_args<BwdDqParams>();
    if (pa.sched.wq == nullptr) return -1;
    if (threadIdx.x == 0) work_slot[slot] = work_next(pa.sched.wq, pa.g.nblocks, &work_slot[2]);
    barrier_lds();
    const int v = __builtin_amdgcn_readfirstlane(work_slot[slot]);
    slot ^= 1;  // the next hand-out writes the other slot, so no wave reads a slot being rewritten
    return v;
  };
  for (int vb = p_arg.sched.wq ? fetch() : (int)blockIdx.x; vb >= 0; vb = fetch()) body(vb);
}

// Explicit instantiations of every built variant (device code and host launch stubs), plain and
// soft-capped.
#define GFA_DQ_INST(DD, SS)                                                                 \
  template __global__ void bwd_dq_kernel<DD, 32, true, 4, SS, false, false>(const BwdDqParams);  \
  template __global__ void bwd_dq_kernel<DD, 32, false, 4, SS, false, false>(const BwdDqParams); \
  template __global__ void bwd_dq_kernel<DD, 32, true, 4, SS, true, false>(const BwdDqParams);   \
  template __global__ void bwd_dq_kernel<DD, 32, false, 4, SS, true, false>(const BwdDqParams);  \
  template __global__ void bwd_dq_kernel<DD, 32, true, 4, SS, false, true>(const BwdDqParams);   \
  template __global__ void bwd_dq_kernel<DD, 32, false, 4, SS, false, true>(const BwdDqParams);
GFA_DQ_INST(512, 2)
GFA_DQ_INST(256, 1)
GFA_DQ_INST(128, 1)
GFA_DQ_INST(64, 1)
#undef GFA_DQ_INST

template <int D, int BKV, bool IS_BF16, int NW, int SPLIT>
static hipError_t launch_dq_t(const BwdDqParams& p, bool cap, bool drop, hipStream_t stream) {
  const unsigned stage_bytes = dq_stages_rows(D, SPLIT) ? NW * BKV * D * 2 : 0;  // the kernel's stage_raw
  if (cap) {
    hipLaunchKernelGGL((bwd_dq_kernel<D, BKV, IS_BF16, NW, SPLIT, true, false>), dim3(p.sched.grid), dim3(NW * 64),
                       stage_bytes, stream, p);
  } else if (drop) {
    hipLaunchKernelGGL((bwd_dq_kernel<D, BKV, IS_BF16, NW, SPLIT, false, true>), dim3(p.sched.grid), dim3(NW * 64),
                       stage_bytes, stream, p);
  } else {
    hipLaunchKernelGGL((bwd_dq_kernel<D, BKV, IS_BF16, NW, SPLIT, false, false>), dim3(p.sched.grid), dim3(NW * 64),
                       stage_bytes, stream, p);
  }
  return hipGetLastError();
}

// Built dQ variants: D=512 on wave pairs (head-dim halves), D=256/128/64 one wave per 32 rows.
hipError_t launch_bwd_dq(const BwdDqParams& p, int D, int bkv, int split, bool bf16, bool cap, bool drop,
                         hipStream_t stream) {
  if (cap && drop) return hipErrorInvalidValue;  // not built together
#define GFA_DQ_CASE(DD, SS)                                                                       \
  if (D == DD && bkv == 32 && split == SS)                                                        \
    return bf16 ? launch_dq_t<DD, 32, true, 4, SS>(p, cap, drop, stream)                          \
                : launch_dq_t<DD, 32, false, 4, SS>(p, cap, drop, stream);
  GFA_DQ_CASE(512, 2)
  GFA_DQ_CASE(256, 1)
  GFA_DQ_CASE(128, 1)
  GFA_DQ_CASE(64, 1)
#undef GFA_DQ_CASE
  return hipErrorInvalidValue;
}

}  // namespace gfa
