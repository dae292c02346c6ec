// GQA flash-attention forward for gfx950 (hot-path row R1).
//
// Semantics follow the reference forward kernel
// (/root/reference/flash_attn/attention.py:245-388): O = softmax(s * Q K^T) V over the
// allowed keys (key <= query when causal; additionally query - key < window when causal
// and window > 0; the window is ignored when not causal), LSE stored in natural log.
//
// MI355X design (not a port of the Triton kernel):
//  * A workgroup holds NW waves; each wave owns 32 query rows of one query head over the
//    whole head dim. The waves of a workgroup are different query heads of the SAME KV
//    head (pack-GQA) and/or neighbouring query blocks, so each K/V tile is fetched
//    HBM -> LDS once per workgroup and consumed by NW * 32 query rows.
//  * The wave computes S^T = K Q^T with v_mfma_f32_32x32x16 (A = K rows from LDS, B = the
//    wave's Q fragments, resident in VGPRs for the whole kernel). Queries sit on lanes, so
//    softmax statistics are per-lane values and P^T stays in registers in exactly the
//    B-operand layout of O^T += V^T P^T, whose A operand is read with the transposing
//    ds_read_b64_tr_b16 from the row-major V tile. O^T (32 x D fp32) lives in AGPRs.
//  * K/V tiles move HBM -> LDS with buffer loads that write LDS directly (no VGPR
//    staging; the buffer range check turns rows past the sequence end into zeros), double
//    buffered, XOR-swizzled so both LDS read patterns are bank-conflict free. The copy of
//    the next tile is spread over the S^T chain, one copy instruction every two MFMAs: the
//    copies of all waves share the CU's texture path, and a run of them would hold up the
//    in-order MFMA stream. The tile loop body is straight-line code (no per-wave skips,
//    branch-free prefetch) so the accumulators never leave the AGPRs.
//  * Softmax uses a fixed per-row reference max instead of a running rescale: the first
//    tile in which a row sees a key sets m_ref, later tiles use p = exp2(s - m_ref), so the
//    loop never rescales O. If any row later meets a score above m_ref + kMargin (P could
//    leave the 16-bit range) the workgroup redoes its rows once with m_ref = the exact row
//    max (observed in the first pass; for bf16 at D <= 256, where the first pass takes the
//    tile max only until m_ref is set and judges overflow from the row sum, found by a pass
//    that runs the score chains alone). Exact either way (LSE = m_ref + log2 l); the redo
//    is never taken for ordinary inputs.
//  * Scores are scaled by scale*log2(e) once and exponentiated with v_exp_f32. Causal and
//    window masks are evaluated only on tiles that straddle a boundary.
#include "gfa_common.h"
#include "gfa_params.h"
#include "gfa_launch.h"

namespace gfa {

template <int D, int BKV, bool IS_BF16, int NW, int WPE, bool SEG, bool CAP, bool DROP>
__global__ __launch_bounds__(NW * 64, WPE) void fwd_kernel(const FwdParams p_arg) {
  constexpr int KT = D / 16;   // MFMA k-steps over the head dim
  constexpr int DB = D / 32;   // 32-row blocks of the O^T accumulator
  constexpr int SB = BKV / 32; // 32-key score blocks per tile
  constexpr int TILE = BKV * D * 2;
  // Largest allowed exp2 argument: P stays below 2^15 in fp16 (max 65504); bf16 P and the
  // fp32 accumulators have range to spare.
  constexpr float kMargin = IS_BF16 ? 64.0f : 15.0f;
  constexpr float kMaxRowSum = 18446744073709551616.0f;  // 2^64 = 2^kMargin for bf16
  static_assert(BKV % 32 == 0, "BKV must be a multiple of 32");
  static_assert(D == 64 || D == 128 || D == 256 || D == 512, "head dim must be 64, 128, 256 or 512");
  // LDS read-ahead of the score chain: shallower when several waves share a SIMD's registers.
  constexpr int PF = WPE == 1 ? 4 : 2;

  // Four distinct LDS objects (not one array indexed by a buffer id): with the loop
  // unrolled by two every access names its buffer statically, so the compiler's wait
  // insertion can tell the in-flight prefetch (into the other buffer) from the tile being
  // read and does not stall on it.
  __shared__ __attribute__((aligned(1024))) char k_lds0[TILE];
  __shared__ __attribute__((aligned(1024))) char k_lds1[TILE];
  __shared__ __attribute__((aligned(1024))) char v_lds0[TILE];
  __shared__ __attribute__((aligned(1024))) char v_lds1[TILE];
  __shared__ int redo_flag;
  __shared__ int work_slot[3];  // the block the run-time work hand-out gave the workgroup (two slots), its state
  char GFA_LDS* const K0 = (char GFA_LDS*)k_lds0;
  char GFA_LDS* const K1 = (char GFA_LDS*)k_lds1;
  char GFA_LDS* const V0 = (char GFA_LDS*)v_lds0;
  char GFA_LDS* const V1 = (char GFA_LDS*)v_lds1;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5;
  const int l32 = lane & 31;

  // One block of the static grid (vblock = its workgroup id there): the body below, run once per
  // block the workgroup is given.
  // D=512 (DYN): the host may run the kernel as a persistent grid, several blocks per workgroup.
  constexpr bool DYN = D == 512;
  auto body = [&](const int vblock) __attribute__((always_inline)) {
  const FwdParams& p = DYN ? *kernel_args<FwdParams>() : p_arg;
  // ---- workgroup -> (b, kv head, head group, query super-block) ----
  int lid = xcd_remap(vblock, p.g.nblocks, p.g.n_hg);
  const int hg = lid % p.g.n_hg;
  lid /= p.g.n_hg;
  const int kvh = lid % p.Hkv;
  lid /= p.Hkv;
  const int b = lid % p.B;
  lid /= p.B;
  const int qsb = p.causal ? (p.g.n_qsb - 1 - lid) : lid;  // causal: longest rows first

  const int head = kvh * p.R + hg * p.g.hpw + (wave % p.g.hpw);
  const int q0 = (qsb * p.g.qbw + wave / p.g.hpw) * 32;
  const int wg_q_lo = qsb * p.g.qbw * 32;
  const int wg_q_hi = min(p.N, wg_q_lo + p.g.qbw * 32);

  const bool swa = p.causal && p.window > 0;
  int k_lo = 0, k_hi = p.N;
  if (p.causal) {
    k_hi = wg_q_hi;
    if (swa) k_lo = max(0, wg_q_lo - p.window + 1);
  }
  // Segment table (SEG): the workgroup's queries see keys from the first query's segment
  // start to the last query's segment end (both rows are non-decreasing).
  const int* slo = SEG ? p.seg_lo + (int64_t)b * p.N : nullptr;
  const int* shi = SEG ? p.seg_hi + (int64_t)b * p.N : nullptr;
  if constexpr (SEG) {
    k_lo = max(k_lo, clamp_n(slo[wg_q_lo], p.N));
    k_hi = min(k_hi, clamp_n(shi[wg_q_hi - 1], p.N));
  }
  const int t_lo = k_lo / BKV;
  // Even tile count (the loop is unrolled by two): an odd range gets one extra tile past
  // the workgroup's keys, which is fully masked (and zero-filled past the sequence end).
  // An empty range (k_hi <= k_lo, only with segments) gives no tiles at all.
  const int t_hi = t_lo + ((((k_hi + BKV - 1) / BKV) - t_lo + 1) & ~1);
  // Sliding window at D=256: the loop's tile t reads tile rot(t), a cyclic walk of [t_lo, t_hi)
  // that starts at the tile whose index is a multiple of the tile count, so that step j of
  // every workgroup reads a tile with index = j (mod count). The neighbouring query blocks that
  // run together on one XCD then read the same K / V tiles at the same time and share them in
  // L2 (each started at its own first tile, they run a few tiles apart): 1-3.5% faster on
  // windows of 512 and 1024. Other head dims walk in order: at D=512 the extra scalar state
  // spills (1-2% slower), at D=128 it is even.
  constexpr bool ROT = D == 256;
  const int nt = t_hi - t_lo;
  const int t_shift = (ROT && swa && nt > 0) ? (nt - t_lo % nt) % nt : 0;
  auto rot = [&](int t) __attribute__((always_inline)) {
    if constexpr (!ROT) return t;
    return t + t_shift < t_hi ? t + t_shift : t + t_shift - nt;
  };

  // Keys every query of this wave sees: [all_lo, all_hi).
  const bool active = q0 < p.N;
  int all_lo = 0, all_hi = p.N;
  if (p.causal) {
    all_hi = min(p.N, q0 + 1);
    if (swa) all_lo = q0 + 31 - p.window + 1;
  }
  const int q = q0 + l32;
  VisRange vis_seg{};  // per-lane visible keys, held only with segments
  if constexpr (SEG) {
    if (active) {
      all_lo = max(all_lo, clamp_n(slo[min(q0 + 31, p.N - 1)], p.N));
      all_hi = min(all_hi, clamp_n(shi[q0], p.N));
    }
    const int qr = min(q, p.N - 1);
    vis_seg = intersect(keys_of_query(q, p.N, p.causal, p.window), clamp_n(slo[qr], p.N), clamp_n(shi[qr], p.N));
  }

  // ---- Q fragments (B operand of S^T = K Q^T), resident for the whole kernel ----
  i16x8 qf[KT];
  {
    const int qrow = min(q, p.N - 1);
    const uint16_t* qr = p.q + (int64_t)b * p.qv.sb + (int64_t)head * p.qv.sh + (int64_t)qrow * p.qv.sn + 8 * h;
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) qf[kk] = *reinterpret_cast<const i16x8*>(qr + 16 * kk);
  }

  // Per-lane LDS byte offsets inside a tile, one base each (kstep_off and
  // mma_tr_accumulate_b derive the others with an XOR next to each read).
  const int koff0 = l32 * (2 * D) + ((h ^ swz<D>(l32)) << 4);  // K row l32, chunk h (k-step 0)
  int voff0;  // V read transposed: rows 4h + t/4, column block 0
  {
    const int t16 = lane & 15;
    const int half16 = (lane >> 4) & 1;
    const int rA = 4 * h + (t16 >> 2);
    const int c = 2 * half16 + ((t16 >> 1) & 1);
    voff0 = rA * (2 * D) + ((c ^ swz<D>(rA)) << 4) + (t16 & 1) * 8;
  }

  const uint16_t* kbase = p.k + (int64_t)b * p.kv.sb + (int64_t)kvh * p.kv.sh;
  const uint16_t* vbase = p.v + (int64_t)b * p.vv.sb + (int64_t)kvh * p.vv.sh;
  TileLoader<D, BKV, NW> kload, vload;
  kload.init(kbase, p.kv.sn, p.N, wave, lane);
  vload.init(vbase, p.vv.sn, p.N, wave, lane);

  if (threadIdx.x == 0) redo_flag = 0;  // read only after a later barrier

  f32x16 acc[DB];
  float m_ref = kNegBig;   // per-row reference max (log2 domain); same in both lane halves
  float m_seen = kNegBig;  // exact running max (only consulted for the redo pass)
  float l_run = 0.f;       // partial row sum over this lane half's keys
  bool ovf = false;
  // One key tile: wait for it, then S^T = K Q^T with the copy of tile t+1 into the other
  // buffers spread over the chain, softmax against the fixed reference max, O^T += V^T P^T.
  constexpr int NI = TileLoader<D, BKV, NW>::NI;  // copy instructions per tile and wave
  // bf16 (LAZY): the tile's row max is taken only while some row of the wave has no reference
  // max yet (a wave-uniform test), and overflow is judged once per pass from the row sum: a P
  // above 2^kMargin makes l above it too. The rare redo then first finds the exact row max in a
  // pass that runs the S^T chains alone (MODE 1). 6% faster at D=64, 3% at D=128, 1% at D=256 and
  // D=512 (at D=512 1% slower while the score chain ran in AGPRs). fp16's margin (2^15) is within
  // reach of a long row's sum, so fp16 keeps the per-tile max and check.
  constexpr bool LAZY = IS_BF16;
  // One wave per SIMD with O^T pinned in AGPRs: the S^T chain accumulates in VGPRs through
  // inline-asm MFMAs (mma32_vgpr); built from the builtin it runs in AGPRs, and the softmax then
  // reads its scores back with AGPR moves.
  constexpr bool VCHAIN = WPE == 1 && SB == 1;
  auto step = [&](auto mode, int t, const char GFA_LDS* kt, const char GFA_LDS* vt, char GFA_LDS* kn,
                  char GFA_LDS* vn) __attribute__((always_inline)) {
    constexpr int MODE = decltype(mode)::value;  // 0: accumulate; 1: row max only
    barrier_tile();  // tile t landed; every wave is done reading the other buffers
    // Issue priority: raised while the wave runs MFMA chains, normal during the softmax, so
    // that with several waves on a SIMD the matrix unit is fed first and the waves drift
    // out of phase (one's softmax overlapping another's products): 2-4% at D=256.
    __builtin_amdgcn_s_setprio(1);
    // The last step re-fetches its own tile into the idle buffers (never read) so the
    // body stays branch-free.
    const int rn = rot(min(t + 1, t_hi - 1)) * BKV;
    const int k0 = rot(t) * BKV;
    f32x16 s[SB];
    auto ld = [&](int i) {
      if (i < NI) {
        kload.load_part(i, rn, kn);
      } else {
        vload.load_part(i - NI, rn, vn);
      }
    };
    if constexpr (VCHAIN) {
      s[0] = mma_chain1_lds_ld_b_vgpr<IS_BF16, KT, PF, 2 * NI>(kt, koff0, qf, ld);
    } else {
      s[0] = mma_chain1_lds_ld_b<IS_BF16, KT, PF, 2 * NI>(kt, koff0, 0, qf, ld);
    }
#pragma unroll
    for (int sb = 1; sb < SB; ++sb) s[sb] = mma_chain1_lds_b<IS_BF16, KT, 4>(kt, koff0, sb * 32 * (2 * D), qf);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    // CAP: soft-capped scores. The tile now holds tanh(scale s / softcap); the exponent
    // multiplier below is softcap log2(e) instead of scale log2(e).
    if constexpr (CAP) {
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[sb][r] = cap_tanh(s[sb][r] * p.cap.cap_a);
      }
    }
    const float xs = CAP ? p.cap.cap_log2 : p.scale_log2;

    const bool need_mask = !(active && k0 + BKV <= all_hi && k0 >= all_lo);
    if (need_mask) {
      // Rebuilt from the lane id on the (few) boundary tiles rather than held in two
      // registers for the whole kernel.
      const VisRange vis = SEG ? vis_seg : keys_of_query(q0 + opaque(l32), p.N, p.causal, p.window);
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + sb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          const bool ok = vis.has(key);
          s[sb][r] = ok ? s[sb][r] : -INFINITY;
        }
      }
    }
    // Row max of the scaled scores as scale * (max of the raw ones): the scale is positive
    // (checked at the boundary; masking to -inf before scaling needs that too), so one
    // multiply replaces sixteen. The exponent argument scales each score in its FMA.
    auto row_max = [&]() __attribute__((always_inline)) {
      float m = -INFINITY;
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) m = fmaxf(m, s[sb][r]);
      }
      return halves_max(m) * xs;
    };
    if constexpr (MODE == 1) {
      m_seen = fmaxf(m_seen, row_max());
      return;
    }
    if (!LAZY || __builtin_amdgcn_ballot_w64(m_ref == kNegBig) != 0) {
      const float mt = row_max();
      // First tile with a visible key fixes m_ref; acc and l are still zero for this row.
      m_ref = (m_ref == kNegBig && mt > kNegBig) ? mt : m_ref;
      if constexpr (!LAZY) {
        ovf = ovf || (mt > m_ref + kMargin);
        m_seen = fmaxf(m_seen, mt);
      }
    }
    i16x8 pb[BKV / 16];
    // DROP: the row sum takes every P, the PV product only the kept ones (1 / (1 - p) is
    // applied with the normalisation).
    const unsigned drow = DROP ? drop_row(p.drop.seed_lo, p.drop.seed_hi, b * p.Hq + head, q0 + l32) : 0u;
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = fast_exp2(s[sb][r] * xs - m_ref);
        l_run += pv;
        float pk = pv;
        if constexpr (DROP) pk = drop_keep(drow, k0 + sb * 32 + 8 * (r >> 2) + 4 * h + (r & 3), p.drop.thresh) ? pv : 0.f;
        pb[sb * 2 + (r >> 3)][r & 7] = to16<IS_BF16>(pk);
      }
    }
    // O^T += V^T P^T with a fixed read-ahead pipeline.
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);
    mma_tr_accumulate_b<IS_BF16, D, DB, BKV / 16, 2, 1>(acc, vt, voff0, pb);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    // One wave per SIMD (D >= 256): keep O^T in AGPRs across iterations (the VGPRs hold Q
    // and the working set). With several waves per SIMD (D <= 128) everything fits the
    // VGPRs; left unpinned, the MFMAs then write VGPRs directly and the softmax needs no
    // AGPR reads (5-10% faster there).
    if constexpr (WPE == 1) {
#pragma unroll
      for (int db = 0; db < DB; ++db) pin_agpr(acc[db]);
    }
  };

  // One pass over the workgroup's key tiles. Written once, expanded twice below: the
  // rare redo pass is a second straight-line copy rather than an outer loop, which keeps
  // the accumulators' live ranges simple enough to stay in AGPRs.
  auto run_pass = [&](auto mode) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < DB; ++i) acc[i] = f32x16{};
    l_run = 0.f;
    if (t_lo < t_hi) {
      kload.load(rot(t_lo) * BKV, K0);
      vload.load(rot(t_lo) * BKV, V0);
    }
    for (int t = t_lo; t < t_hi; t += 2) {
      // Scheduling fences keep the two tile steps from being interleaved, which would
      // raise register pressure past the VGPR budget.
      step(mode, t, K0, V0, K1, V1);
      __builtin_amdgcn_sched_barrier(0);
      step(mode, t + 1, K1, V1, K0, V0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  constexpr std::integral_constant<int, 0> kAccumulate{};
  run_pass(kAccumulate);
  if constexpr (LAZY) ovf = halves_sum(l_run) > kMaxRowSum;
  // Workgroup vote: does any row need the exact-max redo?
  if (__any(ovf) && lane == 0) redo_flag = 1;
  barrier_tile();  // also drains the last (redundant) prefetch before LDS is reused
  if (redo_flag != 0) {
    if constexpr (LAZY) {
      run_pass(std::integral_constant<int, 1>{});  // exact row max into m_seen
      barrier_tile();
    }
    m_ref = m_seen;
    run_pass(kAccumulate);
    barrier_tile();  // the redo pass's last (redundant) prefetch landed; every wave is done with LDS
  }

  // ---- epilogue: normalise, store O and LSE ----
  // O goes out through LDS (each wave's 32 rows in one of the four idle tile buffers) so that
  // every store instruction writes whole rows: 16 bytes per lane, RPI rows per instruction,
  // instead of 8 bytes into each of 32 rows. The wave reads back only what it wrote itself.
  // The lane index is made opaque so that these addresses are computed here, not shared with
  // the loop's (which would keep them live from the prologue).
  char GFA_LDS* const sblk = wave == 0 ? K0 : wave == 1 ? K1 : wave == 2 ? V0 : V1;
  static_assert(TILE >= 32 * D * 2, "a tile buffer holds a wave's 32 output rows");
  const int ln = opaque(lane);
  const int r32 = ln & 31;
  const float l_tot = halves_sum(l_run);
  if (active && q < p.N) {
    // a row that sees no key (empty segment): O = 0; DROP: kept P scaled by 1 / (1 - p)
    const float inv = l_tot > 0.f ? (DROP ? p.drop.inv_keep : 1.0f) / l_tot : 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        i16x4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = to16<IS_BF16>(acc[db][4 * g + e] * inv);
        const int c = 4 * db + g;  // 16-byte chunk of row l32 that holds these 4 + 4 elements
        *reinterpret_cast<i16x4 GFA_LDS*>(sblk + r32 * (2 * D) + ((c ^ swz<D>(r32)) << 4) + 8 * (ln >> 5)) = o4;
      }
    }
    if (p.store_lse && h == 0) {
      p.lse[((int64_t)b * p.Hq + head) * p.lse_ld + q] = (m_ref + __log2f(l_tot)) * kLn2;
    }
  }
  if (active) store_rows_lds<D>(p.o + (int64_t)b * p.ov.sb + (int64_t)head * p.ov.sh, p.ov.sn, p.N, q0, ln, sblk);
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
    const FwdParams& pa = *kernel_args<FwdParams>();
    if (pa.sched.wq == nullptr) return -1;
    if (threadIdx.x == 0) work_slot[slot] = work_next(pa.sched.wq, pa.g.nblocks, &work_slot[2]);
    barrier_lds();
    const int v = __builtin_amdgcn_readfirstlane(work_slot[slot]);
    slot ^= 1;  // the next hand-out writes the other slot, so no wave reads a slot being rewritten
    return v;
  };
  for (int vb = p_arg.sched.wq ? fetch() : (int)blockIdx.x; vb >= 0; vb = fetch()) body(vb);
}

// Explicit instantiations of every built variant (both the device code and the host
// launch stubs must exist for each one).
#define GFA_FWD_INST(DD, BB, WW, EE, CC, XX)                                                  \
  template __global__ void fwd_kernel<DD, BB, true, WW, EE, false, CC, XX>(const FwdParams);  \
  template __global__ void fwd_kernel<DD, BB, false, WW, EE, false, CC, XX>(const FwdParams); \
  template __global__ void fwd_kernel<DD, BB, true, WW, EE, true, CC, XX>(const FwdParams);   \
  template __global__ void fwd_kernel<DD, BB, false, WW, EE, true, CC, XX>(const FwdParams);
GFA_FWD_INST(512, 32, 4, 1, false, false)
GFA_FWD_INST(256, 64, 4, 1, false, false)
GFA_FWD_INST(256, 32, 4, 2, false, false)
GFA_FWD_INST(128, 64, 4, 2, false, false)
GFA_FWD_INST(128, 32, 4, 2, false, false)
GFA_FWD_INST(64, 64, 4, 3, false, false)
GFA_FWD_INST(64, 32, 4, 3, false, false)
// Soft-capped and dropout instances: the registry's default tiles only.
#define GFA_FWD_EXT(CC, XX)                  \
  GFA_FWD_INST(512, 32, 4, 1, CC, XX)        \
  GFA_FWD_INST(256, 32, 4, 2, CC, XX)        \
  GFA_FWD_INST(128, 64, 4, 2, CC, XX)        \
  GFA_FWD_INST(128, 32, 4, 2, CC, XX)        \
  GFA_FWD_INST(64, 64, 4, 3, CC, XX)
GFA_FWD_EXT(true, false)
GFA_FWD_EXT(false, true)
#undef GFA_FWD_EXT
#undef GFA_FWD_INST

template <int D, int BKV, bool IS_BF16, int NW, int WPE, bool CAP, bool DROP>
static hipError_t launch_fwd_t(const FwdParams& p, hipStream_t stream) {
  if (p.seg_lo != nullptr) {
    hipLaunchKernelGGL((fwd_kernel<D, BKV, IS_BF16, NW, WPE, true, CAP, DROP>), dim3(p.sched.grid), dim3(NW * 64), 0,
                       stream, p);
  } else {
    hipLaunchKernelGGL((fwd_kernel<D, BKV, IS_BF16, NW, WPE, false, CAP, DROP>), dim3(p.sched.grid), dim3(NW * 64), 0,
                       stream, p);
  }
  return hipGetLastError();
}

// Built forward variants: (head dim, keys per tile, waves per workgroup, waves per SIMD).
hipError_t launch_fwd(const FwdParams& p, int D, int bkv, int nw, bool bf16, bool cap, bool drop, hipStream_t stream) {
#define GFA_FWD_CASE(DD, BB, WW, EE, CC, XX)                                              \
  if (D == DD && bkv == BB && nw == WW && cap == CC && drop == XX) {                      \
    return bf16 ? launch_fwd_t<DD, BB, true, WW, EE, CC, XX>(p, stream)                   \
                : launch_fwd_t<DD, BB, false, WW, EE, CC, XX>(p, stream);                 \
  }
  GFA_FWD_CASE(512, 32, 4, 1, false, false)
  GFA_FWD_CASE(256, 64, 4, 1, false, false)
  GFA_FWD_CASE(256, 32, 4, 2, false, false)
  GFA_FWD_CASE(128, 64, 4, 2, false, false)
  GFA_FWD_CASE(128, 32, 4, 2, false, false)
  GFA_FWD_CASE(64, 64, 4, 3, false, false)
  GFA_FWD_CASE(64, 32, 4, 3, false, false)
#define GFA_FWD_EXT(CC, XX)                   \
  GFA_FWD_CASE(512, 32, 4, 1, CC, XX)         \
  GFA_FWD_CASE(256, 32, 4, 2, CC, XX)         \
  GFA_FWD_CASE(128, 64, 4, 2, CC, XX)         \
  GFA_FWD_CASE(128, 32, 4, 2, CC, XX)         \
  GFA_FWD_CASE(64, 64, 4, 3, CC, XX)
  GFA_FWD_EXT(true, false)
  GFA_FWD_EXT(false, true)
#undef GFA_FWD_EXT
#undef GFA_FWD_CASE
  return hipErrorInvalidValue;
}

}  // namespace gfa
