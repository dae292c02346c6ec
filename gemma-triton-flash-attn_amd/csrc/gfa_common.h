// Shared device helpers for the gfx950 (CDNA4) GQA flash-attention kernels.
//
// Everything here is written for wave64 and the gfx950 MFMA shapes
// v_mfma_f32_32x32x16_{f16,bf16}. Operand/result lane layouts (verified on
// MI355X with an in-bounds probe):
//   A (32 x 16): lane L holds A[L % 32][8 * (L / 32) + e], e = 0..7
//   B (16 x 32): lane L holds B[8 * (L / 32) + e][L % 32], e = 0..7
//   C (32 x 32): lane L, register r holds C[8 * (r / 4) + 4 * (L / 32) + r % 4][L % 32]
// ds_read_b64_tr_b16 (transposing LDS read): inside each 16-lane group, lane t
// supplies the address of 4 consecutive 16-bit elements M[row0 + t / 4][col0 + 4 * (t % 4) + 0..3];
// lane i of the group receives M[row0 + e][col0 + i] for e = 0..3.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gfa {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

#define GFA_LDS __attribute__((address_space(3)))

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Finite stand-in for -inf as the initial running max: exp2(-inf - kNegBig) == 0 and
// exp2(kNegBig - kNegBig) == 1, so fully-masked rows never produce NaN.
constexpr float kNegBig = -1.0e30f;

// 32x32x16 MFMA on raw 16-bit operands; IS_BF16 selects the bf16 or fp16 form.
template <bool IS_BF16>
__device__ __forceinline__ f32x16 mma32(i16x8 a, i16x8 b, f32x16 c) {
  if constexpr (IS_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// fp32 -> 16-bit storage (round to nearest even), returned as raw bits.
template <bool IS_BF16>
__device__ __forceinline__ short to16(float x) {
  if constexpr (IS_BF16) {
    return __builtin_bit_cast(short, (__bf16)x);
  } else {
    return __builtin_bit_cast(short, (_Float16)x);
  }
}

template <bool IS_BF16>
__device__ __forceinline__ float from16(short x) {
  if constexpr (IS_BF16) {
    return (float)__builtin_bit_cast(__bf16, x);
  } else {
    return (float)__builtin_bit_cast(_Float16, x);
  }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Keep a kernel-lifetime MFMA operand fragment in AGPRs. MFMA reads A/B operands from
// AGPRs directly; left alone, the allocator keeps such fragments in the 256 arch VGPRs
// and spills once the fp32 accumulators fill the AGPR file.
__device__ __forceinline__ void pin_agpr(i16x8& x) { asm volatile("" : "+a"(x)); }

// XOR swizzle of the 16-byte chunk index inside one LDS tile row. It makes
//  * ds_read_b128 of one chunk column across 16 consecutive rows hit 16 distinct
//    4-bank groups, and
//  * ds_read_b64_tr_b16 of 2 adjacent chunks across 4 consecutive rows
//    (rows aligned to 4) hit 8 distinct chunk slots.
// Row bits (0,1) -> chunk bits (1,2); row bit 2 -> chunk bit 3; row bit 3 -> chunk bit 0.
__device__ __forceinline__ int swz(int row) {
  return ((row & 3) << 1) | (((row >> 2) & 1) << 3) | ((row >> 3) & 1);
}

// Byte offset of (row, 16B-chunk c) inside a tile whose rows hold D 16-bit elements.
template <int D>
__device__ __forceinline__ int tile_off(int row, int c) {
  return row * (D * 2) + ((c ^ swz(row)) << 4);
}

__device__ __forceinline__ i16x8 lds_read16(const char GFA_LDS* base, int off) {
  return *reinterpret_cast<const i16x8 GFA_LDS*>(base + off);
}

__device__ __forceinline__ i16x4 lds_read_tr(const char GFA_LDS* base, int off) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((i16x4 GFA_LDS*)(base + off));
}

// Asynchronous 16-byte global -> LDS copy. The LDS destination of lane L is
// lds_wave_base + 16 * L (lds_wave_base must be wave-uniform).
__device__ __forceinline__ void dma16(const void* gsrc, char GFA_LDS* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(gsrc, (void GFA_LDS*)lds_wave_base, 16, 0, 0);
}

// Workgroup barrier for LDS producer/consumer hand-offs. It waits only for this
// wave's outstanding LDS operations (lgkmcnt), unlike __syncthreads(), whose release
// fence also drains every outstanding global load (including in-flight tile prefetches).
// The "memory" clobber keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Barrier after this wave's global->LDS tile copies have landed (vmcnt) and its own
// LDS traffic has drained (lgkmcnt): afterwards the whole tile is visible to every wave.
__device__ __forceinline__ void barrier_tile() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Copy one BKV x D tile (rows row0.., clamped to n_rows-1) from global memory into
// a swizzled LDS tile. The tile holds BKV * D / 8 chunks of 16 bytes; one wave-level
// global_load_lds fills 64 consecutive LDS chunks (64 / (D / 8) whole rows), so wave w
// of NW issues chunk groups w, w + NW, ... The row part of the global address is
// wave-uniform (scalar); each lane adds only its row-in-group and swizzled chunk.
template <int D, int BKV, int NW>
__device__ __forceinline__ void load_tile_async(const uint16_t* gbase, int64_t row_stride, int row0, int n_rows,
                                                char GFA_LDS* tile, int wave, int lane) {
  constexpr int CPR = D / 8;      // chunks per row
  constexpr int RPI = 64 / CPR;   // rows per wave instruction
  constexpr int NI = BKV * CPR / (64 * NW);
  static_assert(CPR >= 16 && CPR <= 64, "head dim must be 128..512");
  static_assert(BKV * CPR % (64 * NW) == 0, "tile must split evenly over the waves");
  const int lrow = lane / CPR;
  const int lc = lane % CPR;
  const int stride_b = (int)row_stride * 2;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int grp = i * NW + wave;
    // Rows past the end re-read the last row (their scores are masked); the clamp is
    // branch-free: scalar group base, per-lane row offset min(lrow, last - base).
    const int srow = min(row0 + grp * RPI, n_rows - 1);
    const int lr = min(lrow, n_rows - 1 - srow);
    const char* rbase = reinterpret_cast<const char*>(gbase + (int64_t)srow * row_stride);
    const unsigned voff = (unsigned)(lr * stride_b + ((lc ^ swz(grp * RPI + lrow)) << 4));
    dma16(rbase + voff, tile + grp * 1024);
  }
}

// Partial score block C(32 x 32) = sum_kk A_kk * B_kk over KT k-steps, where A_kk are rows
// of a swizzled LDS tile (per-lane offsets koff[kk % 8] + 256 * (kk / 8) + extra) and B_kk
// are register-resident fragments. LDS reads run PF steps ahead of the MFMAs; two
// independent accumulation chains are summed at the end.
template <bool IS_BF16, int KT, int PF>
__device__ __forceinline__ f32x16 mma_chain_lds(const char GFA_LDS* tile, const int (&koff)[8], int extra,
                                                const i16x8 (&bf)[KT]) {
  static_assert(KT % 2 == 0 && PF <= KT, "bad chain shape");
  f32x16 c0 = f32x16{}, c1 = f32x16{};
  i16x8 a[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) a[i] = lds_read16(tile, koff[i & 7] + 256 * (i >> 3) + extra);
#pragma unroll
  for (int kk = 0; kk < KT; ++kk) {
    const i16x8 cur = a[kk % PF];
    if (kk + PF < KT) a[kk % PF] = lds_read16(tile, koff[(kk + PF) & 7] + 256 * ((kk + PF) >> 3) + extra);
    if (kk & 1) {
      c1 = mma32<IS_BF16>(cur, bf[kk], c1);
    } else {
      c0 = mma32<IS_BF16>(cur, bf[kk], c0);
    }
  }
  return c0 + c1;
}

// Map the hardware workgroup id to a logical id so that GROUP consecutive logical
// ids (which share K/V tiles) land on the same XCD. Workgroups are dispatched to
// the 8 XCDs round-robin by blockIdx.x; the tail that does not fill 8*GROUP maps 1:1.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks, int group) {
  const int span = 8 * group;
  const int full = (nblocks / span) * span;
  if (bid >= full) return bid;
  const int xcd = bid & 7;
  const int j = bid >> 3;
  return (j / group) * span + xcd * group + (j % group);
}

}  // namespace gfa
