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

// Two kernels from one body (gfa_bwd_dkv_kernel.inc). bwd_dkv_kernel: every form; the role
// pairs store dS where p.dsl.ds is set. bwd_dkv_ds_kernel: one wave per 32 keys storing dS (the
// materialised backward at D=256), in instances of its own since the store's address arithmetic,
// present, costs the one-wave recomputing form 1-2%.
#define GFA_DKV_KERNEL bwd_dkv_kernel
#define GFA_DKV_STORE (ROLES == 2)
#include "gfa_bwd_dkv_kernel.inc"
#undef GFA_DKV_KERNEL
#undef GFA_DKV_STORE
#define GFA_DKV_KERNEL bwd_dkv_ds_kernel
#define GFA_DKV_STORE true
#include "gfa_bwd_dkv_kernel.inc"
#undef GFA_DKV_KERNEL
#undef GFA_DKV_STORE

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
#define GFA_DKV_DS_INST(CC, XX)                                                                     \
  template __global__ void bwd_dkv_ds_kernel<256, 32, true, 4, 1, 1, CC, XX>(const BwdDkvParams);  \
  template __global__ void bwd_dkv_ds_kernel<256, 32, false, 4, 1, 1, CC, XX>(const BwdDkvParams);
GFA_DKV_DS_INST(false, false)
GFA_DKV_DS_INST(true, false)
GFA_DKV_DS_INST(false, true)
#undef GFA_DKV_DS_INST
template __global__ void dkv_reduce_kernel<true>(const BwdDkvParams, int);
template __global__ void dkv_reduce_kernel<false>(const BwdDkvParams, int);

template <int D, int BQ, bool IS_BF16, int NW, int ROLES, int WPE, bool CAP, bool DROP>
static hipError_t launch_dkv_t(const BwdDkvParams& p, hipStream_t stream) {
  const unsigned stage_bytes = dkv_stages_rows(D, ROLES) ? NW * BQ * D * 2 : 0;  // the kernel's stage_raw
  if constexpr (ROLES == 1 && D == 256) {
    if (p.dsl.ds != nullptr) {
      hipLaunchKernelGGL((bwd_dkv_ds_kernel<D, BQ, IS_BF16, NW, ROLES, WPE, CAP, DROP>), dim3(p.nblocks),
                         dim3(NW * 64), stage_bytes, stream, p);
      return hipGetLastError();
    }
  }
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
