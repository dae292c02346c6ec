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

// Dropout mask: a 32-bit integer mixer (xor-shift / multiply, the "lowbias32" constants) applied
// twice, first to the row (seed, query head, query row), then to that and the key index. Pure
// function of the position, so the forward and both backward kernels draw the same mask in
// their different lane layouts; oracle/attention_oracle.py restates it.
__device__ __forceinline__ unsigned drop_mix(unsigned x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}
// Row key of query row i of query head bh (= b * Hq + h).
__device__ __forceinline__ unsigned drop_row(unsigned seed_lo, unsigned seed_hi, int bh, int i) {
  return drop_mix((seed_lo ^ drop_mix(seed_hi + (unsigned)bh * 0x9e3779b9u)) + (unsigned)i);
}
__device__ __forceinline__ bool drop_keep(unsigned row, int j, unsigned thresh) {
  return drop_mix(row ^ ((unsigned)j * 0x85ebca6bu)) >= thresh;
}

// tanh(x) = 1 - 2 / (exp(2x) + 1): one exp2 and one reciprocal (v_exp_f32, v_rcp_f32),
// exactly +-1 once exp(2x) overflows or underflows; absolute error about 1e-7.
__device__ __forceinline__ float cap_tanh(float x) {
  const float e = fast_exp2(x * 2.8853900817779268f);  // exp(2x) = exp2(2x log2(e))
  return 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
}

// Combine a value with the one held by the lane 32 apart (the other half of a 32-row
// fragment): v_permlane32_swap exchanges the wave halves in registers, without an LDS
// round trip. Both lanes of a pair get the same result.
__device__ __forceinline__ float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The visible set of one query (keys) or one key (queries) is a contiguous index range
// (reference attention.py:347-355: key < N; key <= q when causal; q - key < window when
// causal with a window). Built once per lane; a membership test is then one subtract and
// one unsigned compare.
struct VisRange {
  int base;        // first visible index
  unsigned width;  // last - first; an empty range has base far below any index
  __device__ __forceinline__ bool has(int x) const { return (unsigned)(x - base) <= width; }
};

__device__ __forceinline__ VisRange make_range(int lo, int hi) {
  const bool empty = hi < lo;
  return VisRange{empty ? -(1 << 30) : lo, empty ? 0u : (unsigned)(hi - lo)};
}

// Keys visible to query q.
__device__ __forceinline__ VisRange keys_of_query(int q, int n, int causal, int window) {
  const int hi = q < n ? (causal ? q : n - 1) : -1;
  const int lo = (causal && window > 0) ? q - window + 1 : 0;
  return make_range(lo < 0 ? 0 : lo, hi);
}

// Queries that see key k.
__device__ __forceinline__ VisRange queries_of_key(int k, int n, int causal, int window) {
  const int lo = causal ? k : 0;
  int hi = k < n ? n - 1 : -1;
  if (causal && window > 0) hi = min(hi, k + window - 1);
  return make_range(lo, hi);
}

// Segment tables (optional): token t of a batch row attends and is attended only within
// keys [lo[t], hi[t]); an empty segment (lo == hi) marks a token that takes part in nothing
// (padding). Both rows are non-decreasing in t. Table values are clamped to [0, n], so any
// table content keeps every tile range inside the sequence.
__device__ __forceinline__ int clamp_n(int x, int n) { return min(max(x, 0), n); }

// [v] intersected with keys (or queries) [lo, hi).
__device__ __forceinline__ VisRange intersect(VisRange v, int lo, int hi) {
  const int b0 = max(v.base, lo);
  const int e0 = min(v.base + (int)v.width, hi - 1);
  return make_range(b0, e0);
}

// Keep a kernel-lifetime MFMA operand fragment in AGPRs. MFMA reads A/B operands from
// AGPRs directly; left alone, the allocator keeps such fragments in the 256 arch VGPRs
// and spills once the fp32 accumulators fill the AGPR file.
__device__ __forceinline__ void pin_agpr(i16x8& x) { asm volatile("" : "+a"(x)); }
__device__ __forceinline__ void pin_agpr(f32x16& x) { asm volatile("" : "+a"(x)); }
__device__ __forceinline__ void pin_vgpr(i16x8& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin_vgpr(f32x16& x) { asm volatile("" : "+v"(x)); }

// XOR swizzle of the 16-byte chunk index inside one LDS tile row. Two read patterns must be
// bank-conflict free (64 banks of 4 bytes):
//  * ds_read_b128, 16 lanes per cycle: one chunk column across 16 consecutive rows;
//  * ds_read_b64_tr_b16, 32 lanes per cycle: 4 consecutive rows (aligned to 4) x an
//    aligned group of 4 chunks.
// D >= 128 (16 or more chunks per row; only the low 4 bits of the chunk index change): the
// first pattern needs swz to be a bijection on row bits 0..3, the second needs swz bits 2..3
// to be a bijection on row bits 0..1. swz swaps the two bit pairs of the row index: chunk
// bits (2,3) <- row bits (0,1), chunk bits (0,1) <- row bits (2,3).
// D = 64 (8 chunks per row, so rows r and r+1 share one 256-byte bank line): the first
// pattern needs swz to be a bijection from row bits 1..3 onto the 3-bit chunk index, the
// second needs swz bit 2 to follow row bit 1. swz = chunk bit 2 <- row bit 1, chunk bits
// (0,1) <- row bits (2,3).
template <int D>
__device__ __forceinline__ int swz(int row) {
  static_assert(D == 64 || D == 128 || D == 256 || D == 512, "head dim must be 64, 128, 256 or 512");
  if constexpr (D >= 128) {
    return ((row & 3) << 2) | ((row >> 2) & 3);
  } else {
    return (((row >> 1) & 1) << 2) | ((row >> 2) & 3);
  }
}

__device__ __forceinline__ i16x8 lds_read16(const char GFA_LDS* base, int off) {
  return *reinterpret_cast<const i16x8 GFA_LDS*>(base + off);
}

__device__ __forceinline__ i16x4 lds_read_tr(const char GFA_LDS* base, int off) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((i16x4 GFA_LDS*)(base + off));
}

// Workgroup barrier for LDS producer/consumer hand-offs. It waits only for this
// wave's outstanding LDS operations (lgkmcnt), unlike __syncthreads(), whose release
// fence also drains every outstanding global load (including in-flight tile prefetches).
// The "memory" clobber keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Barrier after this wave's global->LDS tile copies have landed (vmcnt) and its own
// LDS traffic has drained (lgkmcnt): afterwards the whole tile is visible to every wave.
__device__ __forceinline__ void barrier_tile() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// barrier_tile leaving this wave's N most recent vector-memory operations outstanding (vmcnt
// counts loads and stores and completes them in issue order): the tile is there when the N
// operations the wave issued after its copies are stores (or prefetches of later tiles) that the
// barrier need not wait for.
template <int N>
__device__ __forceinline__ void barrier_tile_n() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Wait for this wave's outstanding global->LDS copies (the last, redundant prefetch of a
// tile loop) so none lands after the workgroup's LDS has been handed to another one.
__device__ __forceinline__ void drain_tile_copies() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Buffer resource (V#) over one (batch, head) slice of a (B, H, N, D) tensor: raw
// addressing (stride 0), num_records = bytes up to the end of row n_rows - 1. Buffer loads
// whose total offset (soffset + voffset) falls past num_records return zeros, so reads of
// rows >= n_rows need no clamping (their scores are masked anyway).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t slice_rsrc(const uint16_t* base, int64_t row_stride, int n_rows,
                                                            int row_elems) {
  const unsigned bytes = (unsigned)(((int64_t)(n_rows - 1) * row_stride + row_elems) * 2);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), 0, (int)bytes, 0x00020000);
}

// Copies BKV x D tiles (rows row0.. of a row-major 16-bit slice) from global memory into
// swizzled LDS tiles, asynchronously (buffer_load ... lds: no VGPR staging; completion is
// tracked by vmcnt).
//
// A tile holds BKV * D / 8 chunks of 16 bytes. One wave-level instruction fills 64
// consecutive LDS chunks (RPI = 64 / (D / 8) whole rows); wave w of NW issues chunk groups
// w, w + NW, ... The row offset of an instruction is a scalar (soffset); each lane adds a
// per-lane offset (row-in-group, swizzled chunk) computed once per kernel.
template <int D, int BKV, int NW>
struct TileLoader {
  static constexpr int CPR = D / 8;     // chunks per row
  static constexpr int RPI = 64 / CPR;  // rows per wave instruction
  static constexpr int NI = BKV * CPR / (64 * NW);
  // The swizzle repeats every 16 rows, so the lane offsets repeat every PERIOD instructions.
  static constexpr int STEP_ROWS = NW * RPI;
  static constexpr int PERIOD = STEP_ROWS >= 16 ? 1 : 16 / STEP_ROWS;
  static constexpr int NV = NI < PERIOD ? NI : PERIOD;  // distinct lane offsets
  static_assert(CPR >= 8 && CPR <= 64, "head dim must be 64..512");
  static_assert(BKV * CPR % (64 * NW) == 0, "tile must split evenly over the waves");
  static_assert(STEP_ROWS >= 16 ? STEP_ROWS % 16 == 0 : 16 % STEP_ROWS == 0, "swizzle period");

  __amdgpu_buffer_rsrc_t rsrc;
  unsigned voff[NV];
  unsigned stride_b;  // bytes between rows
  int wave;

  __device__ __forceinline__ void init(const uint16_t* base, int64_t row_stride, int n_rows, int wave_, int lane) {
    wave = wave_;
    stride_b = (unsigned)(row_stride * 2);
    rsrc = slice_rsrc(base, row_stride, n_rows, D);
    const int lrow = lane / CPR;
    const int lc = lane % CPR;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int row = (i * NW + wave) * RPI + lrow;
      voff[i] = lrow * stride_b + (unsigned)((lc ^ swz<D>(row)) << 4);
    }
  }

  // Re-point at another slice with the same row stride (dKV streams several heads).
  __device__ __forceinline__ void rebase(const uint16_t* base, int64_t row_stride, int n_rows) {
    rsrc = slice_rsrc(base, row_stride, n_rows, D);
  }

  // Instruction i (< NI) of load(): lets a caller spread a tile copy over other work.
  __device__ __forceinline__ void load_part(int i, int row0, char GFA_LDS* tile) const {
    const int grp = i * NW + wave;
    const unsigned soff = (unsigned)(row0 + grp * RPI) * stride_b;
    // sc0: each CU reads a tile once, into LDS, so the copy gains nothing from the CU's L1 (the
    // workgroups that share a tile share it in L2); headline dK/dV 0.6% faster, the rest even.
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (void GFA_LDS*)(tile + grp * 1024), 16, voff[i % NV], soff, 0, 1);
  }

  __device__ __forceinline__ void load(int row0, char GFA_LDS* tile) const {
#pragma unroll
    for (int i = 0; i < NI; ++i) load_part(i, row0, tile);
  }
};

// One wave copies rows [row0, row0 + 32) of a (batch, head) slice into an LDS block laid out
// like a TileLoader tile (row-major, chunk c of row r at position c ^ swz(r)), rows past
// n_rows repeating row n_rows - 1. Each of the D/16 direct global->LDS copies covers whole
// rows (1 KB, coalesced); loading the same rows straight into the MFMA operand layout (lane =
// row) touches 32 rows per instruction and is several times slower. The caller waits for
// vmcnt before reading the block. NT: non-temporal reads, for rows no other workgroup reads
// (kept out of L2 they leave it to the shared tiles).
template <int D, bool NT = false>
__device__ __forceinline__ void copy_rows_lds(const uint16_t* base, int64_t row_stride, int n_rows, int row0, int lane,
                                              char GFA_LDS* blk) {
  constexpr int CPR = D / 8;
  constexpr int RPI = 64 / CPR;
  const __amdgpu_buffer_rsrc_t rs = slice_rsrc(base, row_stride, n_rows, D);
  const unsigned sb = (unsigned)(row_stride * 2);
  const int lrow = lane / CPR;
  const int lc = lane % CPR;
#pragma unroll
  for (int i = 0; i < 32 / RPI; ++i) {
    const int r = i * RPI + lrow;
    const unsigned vo = (unsigned)min(row0 + r, n_rows - 1) * sb + (unsigned)((lc ^ swz<D>(r)) << 4);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (void GFA_LDS*)(blk + i * 1024), 16, vo, 0, 0, NT ? 2 : 0);
  }
}

// The reverse of copy_rows_lds: one wave writes rows [row0, row0 + 32) of a (batch, head)
// slice from an LDS block in the same layout, skipping rows at or past n_rows; each store
// instruction covers whole rows (16 bytes per lane). The stores are non-temporal: an output row
// is written once and not read by this kernel, and kept out of L2 it does not evict the tiles
// that neighbouring workgroups are still reading (sliding-window forward 5% faster at C3, the
// windowed dK/dV 1.5%; even elsewhere).
template <int D>
__device__ __forceinline__ void store_rows_lds(uint16_t* base, int64_t row_stride, int n_rows, int row0, int lane,
                                               const char GFA_LDS* blk) {
  constexpr int CPR = D / 8;
  constexpr int RPI = 64 / CPR;
  const int lrow = lane / CPR;
  const int lc = lane % CPR;
#pragma unroll
  for (int i = 0; i < 32 / RPI; ++i) {
    const int r = i * RPI + lrow;
    const i16x8 v = lds_read16(blk, i * 1024 + lrow * (2 * D) + ((lc ^ swz<D>(r)) << 4));
    if (row0 + r < n_rows)
      __builtin_nontemporal_store(v, reinterpret_cast<i16x8*>(base + (int64_t)(row0 + r) * row_stride + 8 * lc));
  }
}

// Score block C(32 x 32) = sum_kk A_kk * B_kk over KT k-steps, where A_kk are rows of a
// swizzled LDS tile (per-lane offsets koff[kk % 8] + 256 * (kk / 8) + extra) and B_kk are
// register-resident fragments, as one chain of back-to-back dependent MFMAs (a second,
// independent chain measured slower and costs 16 live registers). LDS reads run PF steps
// ahead of the MFMAs. With SG != 0 the scheduler is told to keep PF LDS reads in flight: PF
// reads first, then one read after every MFMA (call it inside its own scheduling region,
// between two sched_barrier(0)).
template <bool IS_BF16, int KT, int PF, int SG = 0>
__device__ __forceinline__ f32x16 mma_chain1_lds(const char GFA_LDS* tile, const int (&koff)[8], int extra,
                                                 const i16x8 (&bf)[KT], const f32x16& c_init = f32x16{}) {
  static_assert(PF <= KT, "bad chain shape");
  f32x16 c = c_init;
  i16x8 a[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) a[i] = lds_read16(tile, koff[i & 7] + 256 * (i >> 3) + extra);
#pragma unroll
  for (int kk = 0; kk < KT; ++kk) {
    const i16x8 cur = a[kk % PF];
    if (kk + PF < KT) a[kk % PF] = lds_read16(tile, koff[(kk + PF) & 7] + 256 * ((kk + PF) >> 3) + extra);
    c = mma32<IS_BF16>(cur, bf[kk], c);
  }
  if constexpr (SG) {
    __builtin_amdgcn_sched_group_barrier(0x100, PF, 0);
#pragma unroll
    for (int kk = 0; kk < KT - PF; ++kk) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, PF, 0);
  }
  return c;
}

// Per-lane LDS offsets of the k-steps of a score chain, from one base register. The row read
// by k-step kk sits at chunk (2 * kk + h) ^ swz(row); the swizzle XORs the low chunk bits with a
// per-row constant, and the k-step only moves chunk bits 1..3 (kk & 7) and whole 256-byte groups
// (kk >> 3), so offset(kk) = offset(0) ^ ((kk & 7) << 5) + 256 * (kk >> 3): the row term is a
// multiple of 2 * D >= 128 bytes and never overlaps bits 5..6 (D = 64) or 5..7 (D >= 128).
// `opaque` hides the base from loop-invariant code motion, so the XORs are recomputed next to
// their reads (one VALU op each) instead of being hoisted into eight live registers.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}
__device__ __forceinline__ int kstep_off(int base, int kk) { return (base ^ ((kk & 7) << 5)) + 256 * (kk >> 3); }

// mma_chain1_lds with the k-step offsets derived from one base (kstep_off).
template <bool IS_BF16, int KT, int PF, int SG = 0>
__device__ __forceinline__ f32x16 mma_chain1_lds_b(const char GFA_LDS* tile, int koff0, int extra,
                                                   const i16x8 (&bf)[KT], const f32x16& c_init = f32x16{}) {
  static_assert(PF <= KT, "bad chain shape");
  const int kb = opaque(koff0) + extra;
  f32x16 c = c_init;
  i16x8 a[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) a[i] = lds_read16(tile, kstep_off(kb, i));
#pragma unroll
  for (int kk = 0; kk < KT; ++kk) {
    const i16x8 cur = a[kk % PF];
    if (kk + PF < KT) a[kk % PF] = lds_read16(tile, kstep_off(kb, kk + PF));
    c = mma32<IS_BF16>(cur, bf[kk], c);
  }
  if constexpr (SG) {
    __builtin_amdgcn_sched_group_barrier(0x100, PF, 0);
#pragma unroll
    for (int kk = 0; kk < KT - PF; ++kk) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, PF, 0);
  }
  return c;
}

// mma_chain1_lds_b with NL tile-copy instructions spread over the chain (as mma_chain1_lds_ld).
template <bool IS_BF16, int KT, int PF, int NL, typename LD>
__device__ __forceinline__ f32x16 mma_chain1_lds_ld_b(const char GFA_LDS* tile, int koff0, int extra,
                                                      const i16x8 (&bf)[KT], LD&& ld, const f32x16& c_init = f32x16{}) {
  static_assert(PF <= KT && NL >= 1 && KT % NL == 0, "bad chain shape");
  constexpr int EV = KT / NL;
  const int kb = opaque(koff0) + extra;
  f32x16 c = c_init;
  i16x8 a[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) a[i] = lds_read16(tile, kstep_off(kb, i));
#pragma unroll
  for (int kk = 0; kk < KT; ++kk) {
    const i16x8 cur = a[kk % PF];
    if (kk + PF < KT) a[kk % PF] = lds_read16(tile, kstep_off(kb, kk + PF));
    c = mma32<IS_BF16>(cur, bf[kk], c);
    if (kk % EV == 0) ld(kk / EV);
  }
  __builtin_amdgcn_sched_group_barrier(0x100, PF, 0);
#pragma unroll
  for (int kk = 0; kk < KT; ++kk) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (kk + PF < KT) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    if (kk % EV == 0) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
  }
  return c;
}

// One 32x32x16 MFMA into a VGPR accumulator, as inline assembly: in a kernel whose fp32
// accumulators are pinned to AGPRs (asm "a" constraints) the compiler selects the AGPR form for
// every MFMA, so a score chain built from the builtin runs in AGPRs, and with the AGPR file full
// it moves an accumulator block out to VGPRs and back around every chain. FIRST: the chain's
// first product (C = 0). The destination is early-clobber so that it never overlaps an input.
// Dependent products back to back on one accumulator need no wait states; the caller pads the
// chain's end before the result is read (mfma_result_fence).
template <bool IS_BF16, bool FIRST>
__device__ __forceinline__ void mma32_vgpr(f32x16& c, const i16x8& a, const i16x8& b) {
  if constexpr (FIRST) {
    if constexpr (IS_BF16) {
      asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(c) : "v"(a), "v"(b));
    } else {
      asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(c) : "v"(a), "v"(b));
    }
  } else {
    if constexpr (IS_BF16) {
      asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
    } else {
      asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
    }
  }
}
// First product of a VGPR chain started from c0 (C = c0, a VGPR block the chain does not write).
// The leading s_nop covers the two wait states a VALU write of c0 needs before an MFMA reads it
// as its C operand, in case the compiler materializes c0 right before the chain.
template <bool IS_BF16>
__device__ __forceinline__ void mma32_vgpr_from(f32x16& d, const i16x8& a, const i16x8& b, const f32x16& c0) {
  if constexpr (IS_BF16) {
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %3" : "=&v"(d) : "v"(a), "v"(b), "v"(c0));
  } else {
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %3" : "=&v"(d) : "v"(a), "v"(b), "v"(c0));
  }
}
// The compiler cannot see the pass count of an MFMA written in inline assembly, so it inserts no
// wait states before the first read of its result. An 8-pass XDL op on gfx950 needs 12 before a
// VALU, LDS or memory instruction reads its VGPR result; 16 are inserted here.
__device__ __forceinline__ void mfma_result_fence(f32x16& c) { asm volatile("s_nop 7\n\ts_nop 7" : "+v"(c)); }

// mma_chain1_lds_ld with the chain accumulating in VGPRs (mma32_vgpr), started from zero or, with
// c0, from that VGPR block (mma32_vgpr_from).
// side(kk) runs after product kk: vector work on registers the chain does not touch issues
// between the dependent products, which leave the vector unit idle (one product every ~38
// cycles, 32 of them matrix work). side fences its values with empty asm statements (the
// products are volatile asm, which the scheduler keeps in order) so that they stay there.
template <bool IS_BF16, int KT, int PF, int NL, typename LD, typename SIDE>
__device__ __forceinline__ f32x16 mma_chain1_lds_ld_vgpr_side(const char GFA_LDS* tile, const int (&koff)[8],
                                                              const i16x8 (&bf)[KT], LD&& ld, const f32x16* c0,
                                                              SIDE&& side) {
  static_assert(PF <= KT && NL >= 1 && KT % NL == 0, "bad chain shape");
  constexpr int EV = KT / NL;
  f32x16 c;
  i16x8 a[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) a[i] = lds_read16(tile, koff[i & 7] + 256 * (i >> 3));
#pragma unroll
  for (int kk = 0; kk < KT; ++kk) {
    const i16x8 cur = a[kk % PF];
    if (kk + PF < KT) a[kk % PF] = lds_read16(tile, koff[(kk + PF) & 7] + 256 * ((kk + PF) >> 3));
    if (kk == 0 && c0 != nullptr) {
      mma32_vgpr_from<IS_BF16>(c, cur, bf[kk], *c0);
    } else if (kk == 0) {
      mma32_vgpr<IS_BF16, true>(c, cur, bf[kk]);
    } else {
      mma32_vgpr<IS_BF16, false>(c, cur, bf[kk]);
    }
    if (kk % EV == 0) ld(kk / EV);
    side(kk);
  }
  mfma_result_fence(c);
  return c;
}

template <bool IS_BF16, int KT, int PF, int NL, typename LD>
__device__ __forceinline__ f32x16 mma_chain1_lds_ld_vgpr(const char GFA_LDS* tile, const int (&koff)[8],
                                                         const i16x8 (&bf)[KT], LD&& ld,
                                                         const f32x16* c0 = nullptr) {
  return mma_chain1_lds_ld_vgpr_side<IS_BF16, KT, PF, NL>(tile, koff, bf, ld, c0, [](int) {});
}

// Two independent VGPR chains interleaved product by product: cA over the rows of tile tA with
// fragments bfA (from zero), cB over tile tB with bfB (from zero, or from c0B). Back-to-back
// MFMAs then never depend on each other (a dependent chain on one accumulator issues a product
// every ~38-40 cycles instead of 32). NL copy instructions (ld(i)) are spread over the 2 KT
// products.
template <bool IS_BF16, int KT, int PF, int NL, typename LD>
__device__ __forceinline__ void mma_chain2_lds_ld_vgpr(f32x16& cA, f32x16& cB, const char GFA_LDS* tA,
                                                       const char GFA_LDS* tB, const int (&koff)[8],
                                                       const i16x8 (&bfA)[KT], const i16x8 (&bfB)[KT], LD&& ld,
                                                       const f32x16* c0B = nullptr) {
  static_assert(PF <= KT && NL >= 1 && (2 * KT) % NL == 0, "bad chain shape");
  constexpr int EV = 2 * KT / NL;
  i16x8 aA[PF], aB[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) {
    aA[i] = lds_read16(tA, koff[i & 7] + 256 * (i >> 3));
    aB[i] = lds_read16(tB, koff[i & 7] + 256 * (i >> 3));
  }
#pragma unroll
  for (int kk = 0; kk < KT; ++kk) {
    const i16x8 curA = aA[kk % PF];
    const i16x8 curB = aB[kk % PF];
    if (kk + PF < KT) {
      aA[kk % PF] = lds_read16(tA, koff[(kk + PF) & 7] + 256 * ((kk + PF) >> 3));
      aB[kk % PF] = lds_read16(tB, koff[(kk + PF) & 7] + 256 * ((kk + PF) >> 3));
    }
    if (kk == 0) {
      mma32_vgpr<IS_BF16, true>(cA, curA, bfA[kk]);
    } else {
      mma32_vgpr<IS_BF16, false>(cA, curA, bfA[kk]);
    }
    if ((2 * kk) % EV == 0) ld((2 * kk) / EV);
    if (kk == 0 && c0B != nullptr) {
      mma32_vgpr_from<IS_BF16>(cB, curB, bfB[kk], *c0B);
    } else if (kk == 0) {
      mma32_vgpr<IS_BF16, true>(cB, curB, bfB[kk]);
    } else {
      mma32_vgpr<IS_BF16, false>(cB, curB, bfB[kk]);
    }
    if ((2 * kk + 1) % EV == 0) ld((2 * kk + 1) / EV);
  }
  mfma_result_fence(cA);
  mfma_result_fence(cB);
}

// mma_chain1_lds_ld_b with the chain accumulating in VGPRs (mma32_vgpr), started from zero.
template <bool IS_BF16, int KT, int PF, int NL, typename LD>
__device__ __forceinline__ f32x16 mma_chain1_lds_ld_b_vgpr(const char GFA_LDS* tile, int koff0, const i16x8 (&bf)[KT],
                                                           LD&& ld) {
  static_assert(PF <= KT && NL >= 1 && KT % NL == 0, "bad chain shape");
  constexpr int EV = KT / NL;
  const int kb = opaque(koff0);
  f32x16 c;
  i16x8 a[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) a[i] = lds_read16(tile, kstep_off(kb, i));
#pragma unroll
  for (int kk = 0; kk < KT; ++kk) {
    const i16x8 cur = a[kk % PF];
    if (kk + PF < KT) a[kk % PF] = lds_read16(tile, kstep_off(kb, kk + PF));
    if (kk == 0) {
      mma32_vgpr<IS_BF16, true>(c, cur, bf[kk]);
    } else {
      mma32_vgpr<IS_BF16, false>(c, cur, bf[kk]);
    }
    if (kk % EV == 0) ld(kk / EV);
  }
  mfma_result_fence(c);
  return c;
}

// mma_chain1_lds with NL tile-copy instructions ld(0..NL-1) spread over the chain, one after
// every KT / NL MFMAs. A wave issues in order and the copies of all its workgroup's waves
// share the CU's texture path (each copy instruction moves 1 KB), so a run of copy issues
// holds up the MFMAs behind it; one copy every few MFMAs keeps the MFMA stream moving.
// c_init: the accumulator the chain starts from (zero by default).
template <bool IS_BF16, int KT, int PF, int NL, typename LD>
__device__ __forceinline__ f32x16 mma_chain1_lds_ld(const char GFA_LDS* tile, const int (&koff)[8], int extra,
                                                    const i16x8 (&bf)[KT], LD&& ld, const f32x16& c_init = f32x16{}) {
  static_assert(PF <= KT && NL >= 1 && KT % NL == 0, "bad chain shape");
  constexpr int EV = KT / NL;
  f32x16 c = c_init;
  i16x8 a[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) a[i] = lds_read16(tile, koff[i & 7] + 256 * (i >> 3) + extra);
#pragma unroll
  for (int kk = 0; kk < KT; ++kk) {
    const i16x8 cur = a[kk % PF];
    if (kk + PF < KT) a[kk % PF] = lds_read16(tile, koff[(kk + PF) & 7] + 256 * ((kk + PF) >> 3) + extra);
    c = mma32<IS_BF16>(cur, bf[kk], c);
    if (kk % EV == 0) ld(kk / EV);
  }
  __builtin_amdgcn_sched_group_barrier(0x100, PF, 0);
#pragma unroll
  for (int kk = 0; kk < KT; ++kk) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (kk + PF < KT) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    if (kk % EV == 0) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
  }
  return c;
}

// A operand of O^T += V^T P^T (or any product whose A operand is a row-major LDS tile read
// transposed): two ds_read_b64_tr_b16 at the per-lane offsets offA / offB (+ imm).
__device__ __forceinline__ i16x8 tr_frag(const char GFA_LDS* tile, int offA, int offB, int imm) {
  const i16x4 lo = lds_read_tr(tile, offA + imm);
  const i16x4 hi = lds_read_tr(tile, offB + imm);
  return i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// acc[db] += A(ks, db) * B[ks] over ks < NKS, db < DB, where A(ks, db) is read transposed
// from `tile` (row block ks * 16, column block db * 32 of a D-wide row-major tile). The
// reads run PF products ahead of the MFMAs; SG != 0 pins that pipeline in the schedule
// (2*PF transposing reads first, then two after every MFMA).
template <bool IS_BF16, int D, int DB, int NKS, int PF, int SG = 0>
__device__ __forceinline__ void mma_tr_accumulate(f32x16 (&acc)[DB], const char GFA_LDS* tile, const int (&offA)[4],
                                                  const int (&offB)[4], const i16x8 (&bop)[NKS]) {
  constexpr int N = NKS * DB;
  static_assert(PF <= N, "prefetch deeper than the product count");
  i16x8 a[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) {
    const int ks = i / DB, db = i % DB;
    a[i] = tr_frag(tile, offA[db & 3], offB[db & 3], ks * 16 * (2 * D) + 256 * (db >> 2));
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int ks = i / DB, db = i % DB;
    const i16x8 cur = a[i % PF];
    if (i + PF < N) {
      const int ks2 = (i + PF) / DB, db2 = (i + PF) % DB;
      a[i % PF] = tr_frag(tile, offA[db2 & 3], offB[db2 & 3], ks2 * 16 * (2 * D) + 256 * (db2 >> 2));
    }
    acc[db] = mma32<IS_BF16>(cur, bop[ks], acc[db]);
  }
  if constexpr (SG) {
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * PF, 0);
#pragma unroll
    for (int i = 0; i < N - PF; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, PF, 0);
  }
}

// Transposed-read offsets from one base: the A fragment of column block db (< 4) is read at
// base_a ^ (db << 6) (rows 4h + t/4) and base_b ^ (db << 6) (8 rows further down), where
// base_b = (base_a ^ 32) + 16 * D: the swizzle of a row 8 further differs in chunk bit 1 only.
// Same reasoning as kstep_off: the column block moves chunk bits 2..3, the swizzle XORs them
// with a per-row constant, and the row and half-chunk terms never overlap bits 5..7.
template <bool IS_BF16, int D, int DB, int NKS, int PF, int SG = 0>
__device__ __forceinline__ void mma_tr_accumulate_b(f32x16 (&acc)[DB], const char GFA_LDS* tile, int offA0,
                                                    const i16x8 (&bop)[NKS]) {
  constexpr int N = NKS * DB;
  static_assert(PF <= N, "prefetch deeper than the product count");
  const int a0 = opaque(offA0);
  const int b0 = (a0 ^ 32) + 16 * D;
  auto frag = [&](int i) __attribute__((always_inline)) {
    const int ks = i / DB, db = i % DB;
    const int x = (db & 3) << 6;
    return tr_frag(tile, a0 ^ x, b0 ^ x, ks * 16 * (2 * D) + 256 * (db >> 2));
  };
  i16x8 a[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) a[i] = frag(i);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int db = i % DB;
    const i16x8 cur = a[i % PF];
    if (i + PF < N) a[i % PF] = frag(i + PF);
    acc[db] = mma32<IS_BF16>(cur, bop[i / DB], acc[db]);
  }
  if constexpr (SG) {
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * PF, 0);
#pragma unroll
    for (int i = 0; i < N - PF; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, PF, 0);
  }
}

// The kernel's argument block (the kernels take one struct, at offset 0 of the kernarg segment),
// through a pointer the compiler cannot see through: a kernel that runs several blocks reads its
// arguments per block from the kernarg segment (scalar loads) instead of keeping every field live
// in SGPRs across the block loop, which spilled them.
template <typename P>
__device__ __forceinline__ const P* kernel_args() {
  const P __attribute__((address_space(4)))* a =
      (const P __attribute__((address_space(4)))*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(a));
  return (const P*)a;
}

// Run-time hand-out of a static grid's blocks to a persistent grid (WorkQueue in gfa_params.h),
// called by one lane of the workgroup: takes the next block of its XCD's queue (the blocks b with
// b % 8 == the XCD, in order), then, once that is empty, of the other XCDs' queues in turn; -1
// when all are empty. Faster XCDs thereby take more blocks, and no CU waits behind the hardware's
// in-order dispatch. `tried` (the workgroup's count of queues found empty, zero before its first
// call) lives in LDS, so no register holds the hand-out's state across a block; an emptied queue
// is never asked again by the same workgroup, so every workgroup ends after at most eight failed
// takes.
__device__ __forceinline__ int work_next(unsigned* ctr, int nblocks, int* tried) {
  const int xcd = (int)(__builtin_amdgcn_s_getreg(0xF814) & 7);  // HW_REG_XCC_ID: this workgroup's XCD
  int t = *tried;
  int b = -1;
  while (t < 8) {
    const int x = (xcd + t) & 7;
    const unsigned j = atomicAdd(ctr + x, 1u);
    const long long cand = 8ll * j + x;
    if (cand < nblocks) {
      b = (int)cand;
      break;
    }
    ++t;
  }
  *tried = t;
  return b;
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
