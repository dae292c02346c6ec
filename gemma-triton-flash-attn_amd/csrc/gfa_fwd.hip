// GQA flash-attention forward for gfx950 (hot-path row R1).
//
// Semantics follow the reference forward kernel
// (/root/reference/flash_attn/attention.py:245-388): O = softmax(s * Q K^T) V over the
// allowed keys (key <= query when causal; additionally query - key < window when causal
// and window > 0; the window is ignored when not causal), LSE stored in natural log.
//
// MI355X design (not a port of the Triton kernel):
//  * A workgroup holds NW waves = NW/2 wave PAIRS. A pair owns 32 query rows of one
//    query head; each wave of the pair owns one half of the head dim. The pairs of a
//    workgroup are different query heads of the SAME KV head (pack-GQA) and/or
//    neighbouring query blocks, so each K/V tile is fetched HBM -> LDS once per
//    workgroup and consumed by every wave.
//  * Each wave computes a partial S^T = K[:, half] Q[:, half]^T with
//    v_mfma_f32_32x32x16 (A = K rows from LDS, B = its Q half held in VGPRs for the
//    whole kernel); the pair swaps partials through LDS so both hold the full scores.
//    Queries sit on lanes, so softmax statistics are per-lane values and P^T stays in
//    registers in exactly the B-operand layout of O^T[half] += V^T[half] P^T, whose
//    A operand is read with the transposing ds_read_b64_tr_b16 from the row-major V tile.
//    Per wave: 32 x D/2 fp32 accumulator + D/2 Q columns - no spills at D = 512.
//  * K/V tiles move HBM -> LDS with global_load_lds (no VGPR staging), double
//    buffered, XOR-swizzled so both LDS read patterns are bank-conflict free.
//  * Scores are scaled by scale*log2(e) once and exponentiated with v_exp_f32. The
//    running max is only raised when a tile exceeds it by more than 8 (2^8 headroom), so
//    the O/l rescale is rare; results are identical up to rounding.
//  * Causal/window masks are evaluated only on tiles straddling a boundary; fully
//    hidden tiles are skipped per pair, interior tiles run mask-free.
#include "gfa_common.h"
#include "gfa_params.h"
#include "gfa_launch.h"

namespace gfa {

template <int D, int BKV, bool IS_BF16, int NW>
__global__ __launch_bounds__(NW * 64, 1) void fwd_kernel(const FwdParams p) {
  constexpr int DH = D / 2;      // head-dim columns owned by one wave of a pair
  constexpr int KTH = DH / 16;   // MFMA k-steps over the half
  constexpr int DBH = DH / 32;   // 32-row blocks of the O^T half accumulator
  constexpr int SB = BKV / 32;   // 32-key score blocks per tile
  constexpr int TILE = BKV * D * 2;
  constexpr int XCH = SB * 16 * 64 * 4;  // bytes of partial scores one wave publishes
  static_assert(BKV % 32 == 0, "BKV must be a multiple of 32");
  static_assert(DH % 128 == 0, "head dim must be 256 or 512");

  __shared__ __attribute__((aligned(1024))) char smem_raw[4 * TILE + NW * XCH];
  char GFA_LDS* smem = (char GFA_LDS*)smem_raw;
  char GFA_LDS* xch = smem + 4 * TILE;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int unit = wave >> 1;  // wave pair
  const int dh = wave & 1;     // head-dim half
  const int h = lane >> 5;
  const int l32 = lane & 31;

  // ---- workgroup -> (b, kv head, head group, query super-block) ----
  int lid = xcd_remap(blockIdx.x, p.g.nblocks, p.g.n_hg);
  const int hg = lid % p.g.n_hg;
  lid /= p.g.n_hg;
  const int kvh = lid % p.Hkv;
  lid /= p.Hkv;
  const int b = lid % p.B;
  lid /= p.B;
  const int qsb = p.causal ? (p.g.n_qsb - 1 - lid) : lid;  // causal: longest rows first

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
  const int t_lo = k_lo / BKV;
  const int t_hi = (k_hi + BKV - 1) / BKV;

  // Keys every query of this pair sees: [all_lo, all_hi).
  const bool active = q0 < p.N;
  const int q_last = q0 + 31;
  int all_lo = 0, all_hi = p.N;
  if (p.causal) {
    all_hi = min(p.N, q0 + 1);
    if (swa) all_lo = q_last - p.window + 1;
  }

  // ---- Q half fragments (B operand of S^T = K Q^T), resident for the whole kernel ----
  i16x8 qf[KTH];
  {
    const int qrow = min(q0 + l32, p.N - 1);
    const uint16_t* qr = p.q + (int64_t)b * p.qv.sb + (int64_t)head * p.qv.sh + (int64_t)qrow * p.qv.sn + dh * DH + 8 * h;
#pragma unroll
    for (int kk = 0; kk < KTH; ++kk) qf[kk] = *reinterpret_cast<const i16x8*>(qr + 16 * kk);
  }

  f32x16 acc[DBH];
#pragma unroll
  for (int i = 0; i < DBH; ++i) acc[i] = f32x16{};
  float m_run = kNegBig;  // running max (log2 domain); identical across the pair and lane halves
  float l_run = 0.f;      // partial row sum over this lane half's keys

  // Per-lane LDS byte offsets inside a tile. The swizzle only touches the low 4 bits of
  // the 16-byte chunk index, so chunk groups of 16 differ by a constant 256 bytes.
  int koff[8];  // K row l32, chunk dh*DH/8 + 2*kk + h  (+256 * (kk >> 3))
#pragma unroll
  for (int kl = 0; kl < 8; ++kl) koff[kl] = l32 * (2 * D) + (((2 * kl + h) ^ swz(l32)) << 4) + dh * DH * 2;
  int voffA[4], voffB[4];  // V read transposed: rows 4h + t/4 (+8), columns dh*DH + 32*db + ...
  {
    const int t16 = lane & 15;
    const int half16 = (lane >> 4) & 1;
    const int rA = 4 * h + (t16 >> 2);
    const int rB = rA + 8;
#pragma unroll
    for (int dl = 0; dl < 4; ++dl) {
      const int c = 4 * dl + 2 * half16 + ((t16 >> 1) & 1);
      voffA[dl] = rA * (2 * D) + ((c ^ swz(rA)) << 4) + (t16 & 1) * 8 + dh * DH * 2;
      voffB[dl] = rB * (2 * D) + ((c ^ swz(rB)) << 4) + (t16 & 1) * 8 + dh * DH * 2;
    }
  }
  char GFA_LDS* xmine = xch + wave * XCH + lane * 16;
  const char GFA_LDS* xpart = xch + (wave ^ 1) * XCH + lane * 16;

  const uint16_t* kbase = p.k + (int64_t)b * p.kv.sb + (int64_t)kvh * p.kv.sh;
  const uint16_t* vbase = p.v + (int64_t)b * p.vv.sb + (int64_t)kvh * p.vv.sh;

  if (t_lo < t_hi) {
    load_tile_async<D, BKV, NW>(kbase, p.kv.sn, t_lo * BKV, p.N, smem, wave, lane);
    load_tile_async<D, BKV, NW>(vbase, p.vv.sn, t_lo * BKV, p.N, smem + 2 * TILE, wave, lane);
  }

  for (int t = t_lo; t < t_hi; ++t) {
    const int cur = (t - t_lo) & 1;
    barrier_tile();  // tile t landed; every wave is done with tile t-1 and its exchange slot
    {
      // Prefetch the next tile; the last iteration re-fetches its own tile into the idle
      // buffer (never read) so the loop body stays branch-free.
      const int tn = min(t + 1, t_hi - 1);
      load_tile_async<D, BKV, NW>(kbase, p.kv.sn, tn * BKV, p.N, smem + (cur ^ 1) * TILE, wave, lane);
      load_tile_async<D, BKV, NW>(vbase, p.vv.sn, tn * BKV, p.N, smem + (2 + (cur ^ 1)) * TILE, wave, lane);
    }
    const int k0 = t * BKV;
    const char GFA_LDS* kt = smem + cur * TILE;
    const char GFA_LDS* vt = smem + (2 + cur) * TILE;

    // ---- partial S^T = K[:, half] Q[:, half]^T, published to the partner ----
    f32x16 s[SB];
    {
      // No per-pair skip: a tile this pair cannot see is fully masked below, and the
      // straight-line body keeps the accumulators resident in registers.
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
        s[sb] = mma_chain_lds<IS_BF16, KTH, 4>(kt, koff, sb * 32 * (2 * D), qf);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4 v = {s[sb][4 * j], s[sb][4 * j + 1], s[sb][4 * j + 2], s[sb][4 * j + 3]};
          *reinterpret_cast<f32x4 GFA_LDS*>(xmine + (sb * 4 + j) * 1024) = v;
        }
      }
    }
    barrier_lds();  // partials visible
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 v = *reinterpret_cast<const f32x4 GFA_LDS*>(xpart + (sb * 4 + j) * 1024);
        // Same summation order in both waves (a + b == b + a) keeps the pair bit-identical.
#pragma unroll
        for (int e = 0; e < 4; ++e) s[sb][4 * j + e] = s[sb][4 * j + e] + v[e];
      }
    }

    // ---- online softmax (lane = query column) ----
    const bool need_mask = !(active && k0 + BKV <= all_hi && k0 >= all_lo);
    if (need_mask) {
      const int q = q0 + l32;
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + sb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          bool ok = key < p.N;
          if (p.causal) ok = ok && key <= q;
          if (swa) ok = ok && (q - key) < p.window;
          s[sb][r] = ok ? s[sb][r] : -INFINITY;
        }
      }
    }
    float mt = -INFINITY;
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[sb][r] *= p.scale_log2;
        mt = fmaxf(mt, s[sb][r]);
      }
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    if (__any(mt > m_run + 8.0f)) {
      const float m_new = fmaxf(m_run, mt);
      const float alpha = fast_exp2(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < DBH; ++i) acc[i] *= alpha;
      m_run = m_new;
    }
    i16x8 pb[BKV / 16];
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = fast_exp2(s[sb][r] - m_run);
        l_run += pv;
        pb[sb * 2 + (r >> 3)][r & 7] = to16<IS_BF16>(pv);
      }
    }

    // ---- O^T[half] += V^T[half] P^T ----
#pragma unroll
    for (int ks = 0; ks < BKV / 16; ++ks) {
#pragma unroll
      for (int db = 0; db < DBH; ++db) {
        const int imm = ks * 16 * (2 * D) + 256 * (db >> 2);
        const i16x4 lo = lds_read_tr(vt, voffA[db & 3] + imm);
        const i16x4 hi = lds_read_tr(vt, voffB[db & 3] + imm);
        const i16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        acc[db] = mma32<IS_BF16>(a, pb[ks], acc[db]);
      }
    }
  }

  // ---- epilogue: normalise, store this wave's O half and (dh == 0) the LSE ----
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const int q = q0 + l32;
  if (active && q < p.N) {
    const float inv = 1.0f / l_tot;
    uint16_t* orow = p.o + (int64_t)b * p.ov.sb + (int64_t)head * p.ov.sh + (int64_t)q * p.ov.sn + dh * DH;
#pragma unroll
    for (int db = 0; db < DBH; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        i16x4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = to16<IS_BF16>(acc[db][4 * g + e] * inv);
        *reinterpret_cast<i16x4*>(orow + db * 32 + 8 * g + 4 * h) = o4;
      }
    }
    if (p.store_lse && h == 0 && dh == 0) {
      p.lse[((int64_t)b * p.Hq + head) * p.lse_ld + q] = (m_run + __log2f(l_tot)) * kLn2;
    }
  }
}

template <int D, int BKV, bool IS_BF16, int NW>
static hipError_t launch_fwd_t(const FwdParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((fwd_kernel<D, BKV, IS_BF16, NW>), dim3(p.g.nblocks), dim3(NW * 64), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_fwd(const FwdParams& p, int D, int bkv, int nw, bool bf16, hipStream_t stream) {
#define GFA_FWD_CASE(DD, BB, WW)                                                                       \
  if (D == DD && bkv == BB && nw == WW) {                                                              \
    return bf16 ? launch_fwd_t<DD, BB, true, WW>(p, stream) : launch_fwd_t<DD, BB, false, WW>(p, stream); \
  }
  GFA_FWD_CASE(512, 32, 4)
  GFA_FWD_CASE(512, 32, 8)
  GFA_FWD_CASE(256, 32, 4)
  GFA_FWD_CASE(256, 64, 4)
#undef GFA_FWD_CASE
  return hipErrorInvalidValue;
}

}  // namespace gfa
