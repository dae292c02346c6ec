// GQA flash-attention backward, materialised form: the delta kernel and dQ from the dS store.
//
// Same results as /root/reference/flash_attn/attention.py:687-797 (dQ kernel, STORE_DELTA=True),
// by another decomposition. The dK/dV kernel (gfa_bwd_dkv.hip) computes dS = P (dP - delta) for
// every 32 x 32 block it visits anyway; in this form it also stores that block, rounded to the
// input dtype (the reference rounds dS there too, attention.py:791, before dS K). dQ is then one
// product per block, dQ = scale * dS K (attention.py:791-797), instead of the three of the
// recomputing kernel (S, dP and dS K): a third of its matrix work, for 2 KB of dS per block read
// from HBM. Delta = rowsum(dO O) (attention.py:733-744), which the recomputing dQ kernel
// produces in its prologue, comes from its own small kernel ahead of dK/dV.
#include "gfa_common.h"
#include "gfa_params.h"
#include "gfa_launch.h"

namespace gfa {

// One workgroup per 32 rows of one (batch, head): each row's 16-byte chunks spread over the
// lanes of one wave (whole rows per instruction, coalesced), partial products summed across
// those lanes. Rows past N repeat row N - 1, as the recomputing dQ kernel writes them. O and dO
// are read non-temporally (once each): 0.155 ms at the headline, 6.96 TB/s (0.183 ms before), and
// kept out of L2 they leave it to the dK/dV kernel's tiles.
template <int D, bool IS_BF16>
__global__ __launch_bounds__(256) void delta_kernel(const DeltaParams p) {
  constexpr int CPR = D / 8;     // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;  // rows per wave and instruction
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int bh = blockIdx.y;  // b * Hq + head
  const int b = bh / p.Hq, head = bh % p.Hq;
  const uint16_t* ob = p.o + (int64_t)b * p.ov.sb + (int64_t)head * p.ov.sh;
  const uint16_t* db = p.dout + (int64_t)b * p.dov.sb + (int64_t)head * p.dov.sh;
  const int lc = lane % CPR;
#pragma unroll
  for (int it = 0; it < 32 / (4 * RPI); ++it) {
    const int row = blockIdx.x * 32 + (it * 4 + wave) * RPI + lane / CPR;
    const int r = min(row, p.N - 1);
    const i16x8 o = __builtin_nontemporal_load(reinterpret_cast<const i16x8*>(ob + (int64_t)r * p.ov.sn + 8 * lc));
    const i16x8 d = __builtin_nontemporal_load(reinterpret_cast<const i16x8*>(db + (int64_t)r * p.dov.sn + 8 * lc));
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += from16<IS_BF16>(d[e]) * from16<IS_BF16>(o[e]);
#pragma unroll
    for (int m = CPR / 2; m >= 1; m >>= 1) s += __shfl_xor(s, m, CPR);
    if (lc == 0) p.delta[(int64_t)bh * p.lse_ld + row] = s;
  }
}

// dQ from the dS store. A workgroup is four waves and owns four (head, 32-row query tile) units of
// one KV head (the QGrid split of the forward). Wave w accumulates units 2 (w >> 1) and
// 2 (w >> 1) + 1 over head-dim half w & 1: every K^T fragment it reads from LDS feeds the
// products of both units, half the LDS reads per product of one unit per wave. The waves share
// the K tiles, in a ring of LDS buffers filled by direct global->LDS copies two tiles ahead (four
// buffers and one barrier per two tiles with one workgroup per CU, three and one per tile with
// two); wave w copies the 2 KB dS block of unit w next to them (the blocks come from HBM,
// further away than a tile step). Per tile and wave:
// dQ^T[half] += K^T[half] dS^T for both units, two k-steps of 16 keys, A operands read transposed
// from the K tile (as in the recomputing kernel), B operands read transposed from the dS blocks:
// lane n gets the query sigma(n) of the block layout (gfa_ds.h), the query of its accumulator
// column. A unit's B operand is zero on tiles outside its own row of blocks (the workgroup's
// range is the union of its units'; the block's LDS slot then holds the zeros of an empty copy).
template <int D, bool IS_BF16, int WPE>
__global__ __launch_bounds__(256, WPE) void bwd_dq_ds_kernel(const BwdDqDsParams p) {
  constexpr int NW = 4;
  constexpr int BKV = 32;
  constexpr int TILE = BKV * D * 2;
  constexpr int DH = D / 2;     // head-dim half of one wave
  constexpr int DBH = DH / 32;  // its 32-wide accumulator blocks
  constexpr int DSB = 2048;     // one dS block
  // PAIRED (one workgroup per CU): a ring of four tile buffers and one barrier per two tiles;
  // otherwise (two workgroups per CU) a ring of three and a barrier per tile.
  constexpr bool PAIRED = WPE == 1;
  // Distinct LDS objects (the loop is unrolled over the ring, so every access names its buffer
  // and the compiler's wait insertion can tell the reads from the copies in flight).
  __shared__ __attribute__((aligned(1024))) char k_lds0[TILE];
  __shared__ __attribute__((aligned(1024))) char k_lds1[TILE];
  __shared__ __attribute__((aligned(1024))) char k_lds2[TILE];
  __shared__ __attribute__((aligned(1024))) char k_lds3[PAIRED ? TILE : 16];
  __shared__ __attribute__((aligned(1024))) char s_lds0[NW * DSB];
  __shared__ __attribute__((aligned(1024))) char s_lds1[NW * DSB];
  __shared__ __attribute__((aligned(1024))) char s_lds2[NW * DSB];
  __shared__ __attribute__((aligned(1024))) char s_lds3[PAIRED ? NW * DSB : 16];
  char GFA_LDS* const K0 = (char GFA_LDS*)k_lds0;
  char GFA_LDS* const K1 = (char GFA_LDS*)k_lds1;
  char GFA_LDS* const K2 = (char GFA_LDS*)k_lds2;
  char GFA_LDS* const K3 = (char GFA_LDS*)k_lds3;
  char GFA_LDS* const S0 = (char GFA_LDS*)s_lds0;
  char GFA_LDS* const S1 = (char GFA_LDS*)s_lds1;
  char GFA_LDS* const S2 = (char GFA_LDS*)s_lds2;
  char GFA_LDS* const S3 = (char GFA_LDS*)s_lds3;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5;
  const int l32 = lane & 31;
  const int dh = wave & 1;        // head-dim half
  const int u0 = 2 * (wave >> 1);  // this wave's units u0, u0 + 1

  int lid = xcd_remap((int)blockIdx.x, p.g.nblocks, p.g.n_hg);
  const int hg = lid % p.g.n_hg;
  lid /= p.g.n_hg;
  const int kvh = lid % p.Hkv;
  lid /= p.Hkv;
  const int b = lid % p.B;
  lid /= p.B;
  // Full causal: longest rows first. Sliding window: the short first blocks first.
  const int qsb = p.dsl.mode == 1 ? (p.g.n_qsb - 1 - lid) : lid;
  auto head_of = [&](int u) __attribute__((always_inline)) { return kvh * p.R + hg * p.g.hpw + u % p.g.hpw; };
  auto qt_of = [&](int u) __attribute__((always_inline)) { return qsb * p.g.qbw + u / p.g.hpw; };
  // Query tile qt's stored blocks [jlo, jhi]: the layout's row, narrowed by the segment table to
  // the blocks the dK/dV kernel computes there (empty past the last query tile).
  const int* slo = p.seg_lo ? p.seg_lo + (int64_t)b * p.N : nullptr;
  const int* shi = p.seg_lo ? p.seg_hi + (int64_t)b * p.N : nullptr;
  auto jlo_at = [&](int qt) __attribute__((always_inline)) {
    if (qt >= p.dsl.nq) return 1;
    int lo = ds_jmin(p.dsl, qt);
    if (slo) {
      int a, c;
      ds_seg_units(slo, shi, p.N, qt, &a, &c);
      lo = max(lo, a);
    }
    return lo;
  };
  auto jhi_at = [&](int qt) __attribute__((always_inline)) {
    if (qt >= p.dsl.nq) return 0;
    int hi = ds_jmax(p.dsl, qt);
    if (slo) {
      int a, c;
      ds_seg_units(slo, shi, p.N, qt, &a, &c);
      hi = min(hi, c);
    }
    return hi;
  };
  auto jlo_of = [&](int u) __attribute__((always_inline)) { return jlo_at(qt_of(u)); };
  auto jhi_of = [&](int u) __attribute__((always_inline)) { return jhi_at(qt_of(u)); };

  // Tile range: the union of the workgroup's rows of blocks (both bounds do not decrease with
  // the query tile), made a multiple of the loop's unroll (four or three tiles); empty when a
  // segment table leaves the workgroup's tiles no block.
  constexpr int UNROLL = PAIRED ? 4 : 3;
  const int wg_qt_lo = qsb * p.g.qbw;
  const int wg_qt_last = min(p.dsl.nq, wg_qt_lo + p.g.qbw) - 1;
  const int t_lo = jlo_at(wg_qt_lo);
  const int t_last = jhi_at(wg_qt_last);
  const int t_hi = t_last >= t_lo ? t_lo + (t_last + 1 - t_lo + UNROLL - 1) / UNROLL * UNROLL : t_lo;
  const int jlo0 = jlo_of(u0), jhi0 = jhi_of(u0), jlo1 = jlo_of(u0 + 1), jhi1 = jhi_of(u0 + 1);

  TileLoader<D, BKV, NW> kload;
  kload.init(p.k + (int64_t)b * p.kv.sb + (int64_t)kvh * p.kv.sh, p.kv.sn, p.N, wave, lane);
  // The dS block of unit `wave` and unit j into its slot of sbuf: two 1 KB whole-wave copies,
  // always issued (a block outside the unit's row reads through an empty buffer resource, which
  // returns zeros and touches no memory), so every step issues the same number of copies and
  // the tile barrier can count them.
  constexpr int NI = TileLoader<D, BKV, NW>::NI;  // K tile copy instructions per wave
  // Inside a row the block index grows by one per key unit: block j of the row is srow + j.
  const int cjlo = jlo_of(wave), cjhi = jhi_of(wave), cqt = qt_of(wave);
  const uint16_t* slab = p.dsl.ds + ((int64_t)b * p.Hq + head_of(wave)) * p.dsl.slab * 1024;
  const int64_t srow = cjlo <= cjhi ? ds_index(p.dsl, cqt, cjlo) - cjlo : 0;
  // In LDS the 16-byte key rows of part c sit at row r ^ 4c (part c of a block at 512 c): the
  // transposing B reads of one 32-lane half, which span the four parts at the same rows, then fall
  // in distinct banks (unswizzled, the parts 512 bytes apart share banks: 4-way conflicts). Lane L
  // of copy instruction i writes row L & 31 of part 2 i + (L >> 5), so it fetches that part's row
  // (L & 31) ^ 4 (2 i + (L >> 5)).
  unsigned svoff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = 2 * i + (lane >> 5);
    svoff[i] = (unsigned)(c * 512 + 16 * ((lane & 31) ^ (4 * c)));
  }
  auto copy_ds = [&](int j, char GFA_LDS* sbuf) __attribute__((always_inline)) {
    const bool have = cjlo <= j && j <= cjhi;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(slab + (have ? (srow + j) * 1024 : 0)), 0, have ? DSB : 0, 0x00020000);
#pragma unroll
    for (int c = 0; c < 2; ++c)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (void GFA_LDS*)(sbuf + wave * DSB + c * 1024), 16, svoff[c], 0, 0,
                                               2 /* nt: read once */);
  };

  // Transposed-read offsets: K tile (A operands, rows = keys 4h + t/4 and 8 further, swizzled
  // chunks, this wave's head-dim half) and dS block (B operands, rows = keys at 16 bytes inside
  // each 512-byte part).
  int toffA[4], toffB[4];
  int soffA, soffB;
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
    // part c = 2 half16 + ((t16 >> 1) & 1) (columns 8 c ..), 16-byte rows inside a part, row r at
    // r ^ 4c (the copy's swizzle; the second k-step's rows, 16 further, keep it: 4c < 16)
    const int c = 2 * half16 + ((t16 >> 1) & 1);
    soffA = c * 512 + 16 * (rA ^ (4 * c)) + (t16 & 1) * 8;
    soffB = c * 512 + 16 * (rB ^ (4 * c)) + (t16 & 1) * 8;
  }

  f32x16 acc0[DBH], acc1[DBH];
#pragma unroll
  for (int i = 0; i < DBH; ++i) acc0[i] = acc1[i] = f32x16{};

  // Copies of tile t into kn, sn. Past the end: the last tile's K again (never read) and empty
  // dS copies.
  auto issue = [&](int t, char GFA_LDS* kn, char GFA_LDS* sn) __attribute__((always_inline)) {
    kload.load(min(t, t_hi - 1) * BKV, kn);
    copy_ds(t, sn);
  };
  // The products of tile t (landed, in kt and st).
  auto compute = [&](int t, const char GFA_LDS* kt, const char GFA_LDS* st) __attribute__((always_inline)) {
    const bool in0 = jlo0 <= t && t <= jhi0, in1 = jlo1 <= t && t <= jhi1;
    if (in0 || in1) {
      i16x8 b0[2], b1[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {  // (a block outside a unit's row is zeros in LDS)
        b0[ks] = tr_frag(st + u0 * DSB, soffA, soffB, ks * 256);
        b1[ks] = tr_frag(st + (u0 + 1) * DSB, soffA, soffB, ks * 256);
      }
      // Own scheduling region for the products: a fixed read-ahead of PF A fragments, two
      // transposing reads after each pair of products.
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (WPE > 1) __builtin_amdgcn_s_setprio(1);
      constexpr int N = 2 * DBH, PF = 2;
      auto frag = [&](int i) __attribute__((always_inline)) {
        const int ks = i / DBH, db = i % DBH;
        return tr_frag(kt, toffA[db & 3], toffB[db & 3], ks * 16 * (2 * D) + 256 * (db >> 2));
      };
      i16x8 a[PF];
#pragma unroll
      for (int i = 0; i < PF; ++i) a[i] = frag(i);
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int ks = i / DBH, db = i % DBH;
        const i16x8 cur = a[i % PF];
        if (i + PF < N) a[i % PF] = frag(i + PF);
        acc0[db] = mma32<IS_BF16>(cur, b0[ks], acc0[db]);
        acc1[db] = mma32<IS_BF16>(cur, b1[ks], acc1[db]);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * PF, 0);
#pragma unroll
      for (int i = 0; i < N - PF; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * PF, 0);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (WPE > 1) __builtin_amdgcn_s_setprio(0);
    }
    if constexpr (WPE == 1) {
#pragma unroll
      for (int db = 0; db < DBH; ++db) {
        pin_agpr(acc0[db]);
        pin_agpr(acc1[db]);
      }
    }
  };

  // The products of tiles t and t + 1 (both landed, in ka, sa and kb, sb) as one stream: the B
  // operands of both tiles are read up front (a unit's block outside its row is zeros in LDS, its
  // copy having read through an empty buffer resource), and the A read-ahead runs across the
  // tile boundary. mid() (the next copies) is issued between the two tiles' products.
  auto compute_pair = [&](int t, const char GFA_LDS* ka, const char GFA_LDS* sa, const char GFA_LDS* kb,
                          const char GFA_LDS* sb, auto&& mid) __attribute__((always_inline)) {
    const bool on = (jlo0 <= t + 1 && t <= jhi0) || (jlo1 <= t + 1 && t <= jhi1);
    constexpr int N = 2 * DBH, PF = 2;
    auto frag = [&](const char GFA_LDS* kt, int i) __attribute__((always_inline)) {
      const int ks = i / DBH, db = i % DBH;
      return tr_frag(kt, toffA[db & 3], toffB[db & 3], ks * 16 * (2 * D) + 256 * (db >> 2));
    };
    i16x8 b0[2][2], b1[2][2], a[PF];
    if (on) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        b0[0][ks] = tr_frag(sa + u0 * DSB, soffA, soffB, ks * 256);
        b1[0][ks] = tr_frag(sa + (u0 + 1) * DSB, soffA, soffB, ks * 256);
      }
#pragma unroll
      for (int i = 0; i < PF; ++i) a[i] = frag(ka, i);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        b0[1][ks] = tr_frag(sb + u0 * DSB, soffA, soffB, ks * 256);
        b1[1][ks] = tr_frag(sb + (u0 + 1) * DSB, soffA, soffB, ks * 256);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int ks = i / DBH, db = i % DBH;
        const i16x8 cur = a[i % PF];
        a[i % PF] = i + PF < N ? frag(ka, i + PF) : frag(kb, i + PF - N);
        acc0[db] = mma32<IS_BF16>(cur, b0[0][ks], acc0[db]);
        acc1[db] = mma32<IS_BF16>(cur, b1[0][ks], acc1[db]);
      }
#pragma unroll
      for (int i = 0; i < N; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    mid();
    if (on) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int ks = i / DBH, db = i % DBH;
        const i16x8 cur = a[i % PF];
        if (i + PF < N) a[i % PF] = frag(kb, i + PF);
        acc0[db] = mma32<IS_BF16>(cur, b0[1][ks], acc0[db]);
        acc1[db] = mma32<IS_BF16>(cur, b1[1][ks], acc1[db]);
      }
#pragma unroll
      for (int i = 0; i < N - PF; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * PF, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int db = 0; db < DBH; ++db) {
      pin_agpr(acc0[db]);
      pin_agpr(acc1[db]);
    }
  };

  // A step of the three-buffer ring: tile t landed (the wave's NI + 2 most recent copies, of
  // tile t + 1, may still be in flight) and every wave is done reading tile t - 1, whose buffers
  // kn, sn take tile t + 2.
  auto step = [&](int t, const char GFA_LDS* kt, const char GFA_LDS* st, char GFA_LDS* kn, char GFA_LDS* sn)
                  __attribute__((always_inline)) {
    barrier_tile_n<NI + 2>();
    issue(t + 2, kn, sn);
    compute(t, kt, st);
  };

  if (t_lo < t_hi) {
    issue(t_lo, K0, S0);
    issue(t_lo + 1, K1, S1);
  }
  if constexpr (PAIRED) {
    // Tiles two at a time: past the barrier tiles t, t + 1 have landed and every wave is done
    // with t - 2, t - 1, whose buffers take t + 2, t + 3 (each copy issued before the products
    // of the tile two ahead of it).
    for (int t = t_lo; t < t_hi; t += 4) {
      barrier_tile();
      issue(t + 2, K2, S2);
      compute_pair(t, K0, S0, K1, S1, [&]() __attribute__((always_inline)) { issue(t + 3, K3, S3); });
      __builtin_amdgcn_sched_barrier(0);
      barrier_tile();
      issue(t + 4, K0, S0);
      compute_pair(t + 2, K2, S2, K3, S3, [&]() __attribute__((always_inline)) { issue(t + 5, K1, S1); });
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    for (int t = t_lo; t < t_hi; t += 3) {
      step(t, K0, S0, K2, S2);
      __builtin_amdgcn_sched_barrier(0);
      step(t + 1, K1, S1, K0, S0);
      __builtin_amdgcn_sched_barrier(0);
      step(t + 2, K2, S2, K1, S1);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  drain_tile_copies();

  // Epilogue. Column l32 of the accumulators is query sigma(l32) of the unit's tile, at row
  // qoff of it; rows are head-dim elements DH dh + 32 db + 8 g + 4 h + 0..3. Each wave stages its
  // half-rows (its two units x 32 queries x DH, scaled and rounded) through its own LDS block and
  // stores them as whole half-rows, 16 bytes per lane and non-temporally (written once; 8-byte
  // stores straight from the accumulators leave partial lines, which cannot go non-temporal).
  // The staging blocks are the tile buffers: every wave must be past the loop first.
  barrier_lds();
  constexpr int HB = 32 * DH * 2;  // one unit's staged half-rows
  constexpr int NCH = DH / 8;      // 16-byte chunks per half-row
  static_assert(2 * HB <= TILE, "a tile buffer holds a wave's two staged units");
  char GFA_LDS* stg0;
  char GFA_LDS* stg1;
  if constexpr (PAIRED) {
    stg0 = wave == 0 ? K0 : wave == 1 ? K1 : wave == 2 ? K2 : K3;
    stg1 = stg0 + HB;
  } else {  // three tile buffers; the fourth wave's units go to two dS buffers (NW * DSB >= HB)
    static_assert(NW * DSB >= HB, "a dS buffer holds one staged unit");
    stg0 = wave == 0 ? K0 : wave == 1 ? K1 : wave == 2 ? K2 : S0;
    stg1 = wave == 3 ? S1 : stg0 + HB;
  }
  const int ln = opaque(lane);
  const int c8 = (ln & 31) >> 3, e8 = ln & 7;
  const int qoff = 16 * (c8 >> 1) + 8 * (e8 >> 2) + 4 * (c8 & 1) + (e8 & 3);
  auto stage = [&](const f32x16 (&acc)[DBH], char GFA_LDS* blk) __attribute__((always_inline)) {
#pragma unroll
    for (int db = 0; db < DBH; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        i16x4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = to16<IS_BF16>(acc[db][4 * g + e] * p.scale);
        const int c = 4 * db + g;  // chunk of the half-row: elements 32 db + 8 g .. + 7
        *reinterpret_cast<i16x4 GFA_LDS*>(blk + qoff * (DH * 2) + ((c ^ (qoff % NCH)) << 4) + 8 * (ln >> 5)) = o4;
      }
    }
  };
  stage(acc0, stg0);
  stage(acc1, stg1);
  constexpr int RPI = 64 / NCH;  // half-rows per store instruction
  auto put = [&](int u, const char GFA_LDS* blk) __attribute__((always_inline)) {
    const int q0 = qt_of(u) * 32;
    uint16_t* base = p.dq + (int64_t)b * p.dqv.sb + (int64_t)head_of(u) * p.dqv.sh + dh * DH;
    const int c = ln % NCH;
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
      const int r = i * RPI + ln / NCH;
      const i16x8 v = lds_read16(blk, r * (DH * 2) + ((c ^ (r % NCH)) << 4));
      if (q0 + r < p.N) __builtin_nontemporal_store(v, reinterpret_cast<i16x8*>(base + (int64_t)(q0 + r) * p.dqv.sn + 8 * c));
    }
  };
  put(u0, stg0);
  put(u0 + 1, stg1);
}

#define GFA_DS_INST(DD, WW)                                                                   \
  template __global__ void bwd_dq_ds_kernel<DD, true, WW>(const BwdDqDsParams);               \
  template __global__ void bwd_dq_ds_kernel<DD, false, WW>(const BwdDqDsParams);              \
  template __global__ void delta_kernel<DD, true>(const DeltaParams);                         \
  template __global__ void delta_kernel<DD, false>(const DeltaParams);
GFA_DS_INST(512, 1)
GFA_DS_INST(256, 2)
#undef GFA_DS_INST

hipError_t launch_delta(const DeltaParams& p, bool bf16, hipStream_t stream) {
  const dim3 grid((p.N + 31) / 32, p.B * p.Hq);
#define GFA_DELTA_CASE(DD)                                                                              \
  if (p.D == DD) {                                                                                      \
    if (bf16) {                                                                                         \
      hipLaunchKernelGGL((delta_kernel<DD, true>), grid, dim3(256), 0, stream, p);                    \
    } else {                                                                                            \
      hipLaunchKernelGGL((delta_kernel<DD, false>), grid, dim3(256), 0, stream, p);                   \
    }                                                                                                   \
    return hipGetLastError();                                                                           \
  }
  GFA_DELTA_CASE(512)
  GFA_DELTA_CASE(256)
#undef GFA_DELTA_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_dq_ds(const BwdDqDsParams& p, int head_dim, bool bf16, hipStream_t stream) {
  const dim3 grid(p.g.nblocks);
  if (head_dim == 512) {
    if (bf16) {
      hipLaunchKernelGGL((bwd_dq_ds_kernel<512, true, 1>), grid, dim3(256), 0, stream, p);
    } else {
      hipLaunchKernelGGL((bwd_dq_ds_kernel<512, false, 1>), grid, dim3(256), 0, stream, p);
    }
    return hipGetLastError();
  }
  if (head_dim == 256) {
    if (bf16) {
      hipLaunchKernelGGL((bwd_dq_ds_kernel<256, true, 2>), grid, dim3(256), 0, stream, p);
    } else {
      hipLaunchKernelGGL((bwd_dq_ds_kernel<256, false, 2>), grid, dim3(256), 0, stream, p);
    }
    return hipGetLastError();
  }
  return hipErrorInvalidValue;
}

}  // namespace gfa
