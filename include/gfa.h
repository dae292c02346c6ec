/*
 * gfa.h - C ABI of the MI355X (gfx950) GQA flash-attention engine.
 *
 * Plain C: raw device pointers, element strides and sizes, a hipStream_t passed as
 * void*. No framework types cross this boundary. The library never allocates, frees
 * or synchronises; every call is stream-ordered on the caller's stream and device.
 *
 * Tensor layout: q/o/do/dq are (B, Hq, N, D); k/v/dk/dv are (B, Hkv, N, D); every
 * tensor is addressed through its own (batch, head, row) element strides and must have
 * a unit-stride head dimension and 16-byte aligned rows. lse/delta are float32
 * (B, Hq, lse_ld) with lse_ld >= GFA_LSE_LD(N): the backward kernels read whole query
 * tiles of up to 64 rows, so rows N..lse_ld-1 must exist (their values are never used).
 * Query head h reads KV head h / (Hq / Hkv) (contiguous groups). head_dim is 64, 128, 256
 * or 512 (the reference documents 64-512, powers of two); anything else returns
 * GFA_ERR_UNSUPPORTED, as does a (batch, head) slice that, with 127 rows of margin past its
 * end, spans more than 4 GiB.
 *
 * Variable-length and padded batches: seg_lo / seg_hi (optional, both or neither) are
 * int32 (B, N) tables, row b at seg_lo + b * N. Token t of row b attends, and is attended
 * by, only the tokens of keys [seg_lo[t], seg_hi[t]), intersected with the causal / window
 * rule. Each row must partition [0, N) into consecutive runs: a segment, whose tokens all
 * carry lo = first token and hi = one past its last, or padding, where token t carries
 * lo = hi = t (an empty segment: its O row is 0, its LSE -inf, and its dQ/dK/dV rows 0).
 * So both columns are non-decreasing. Left and right padding and packed sequences (the
 * reference's unsupported varlen case, README.md:255-262) are all such tables. The kernels
 * clamp table values to [0, N], so no content makes them address outside the tensors.
 *
 * The entry points replace the reference's Triton launch sites (file:line in
 * /root/reference, zzhhjjj/gemma-triton-flash-attn):
 *   gfa_fwd          flash_attn/attention.py:1454-1468 (_flash_attn_gqa_kernel launch,
 *                    STORE_LSE=True, training forward) and attention.py:589-601
 *                    (inference forward, STORE_LSE=False -> lse == NULL)
 *   gfa_bwd          flash_attn/attention.py:1506-1620 (dQ kernel with fused delta,
 *                    then the pack-GQA dKV kernel with its Q_SPLITS partial sums)
 *   gfa_config       the HEAD_DIM-keyed tile tables at attention.py:561-579, 1445-1451,
 *                    1498-1504, 1536-1564 and the Q_SPLITS choice at 1576-1587
 *   gfa_bwd_workspace_size
 *                    sizing of the (2,)+k.shape pre-zeroed buffer of attention.py:1594-1600
 *                    (here: fp32 partials, owned by the caller)
 */
#ifndef GFA_H_
#define GFA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GFA_VERSION 106 /* 1.0.6: materialised backward (1.0.5: run-time work distribution, 1.0.4: attention dropout, 1.0.3: soft-capping) */

typedef enum {
  GFA_DTYPE_FP16 = 0,
  GFA_DTYPE_BF16 = 1
} gfa_dtype;

typedef enum {
  GFA_OK = 0,
  GFA_ERR_INVALID_ARGUMENT = 1, /* shape / stride / dtype / alignment / head-dim problem */
  GFA_ERR_UNSUPPORTED = 2,      /* valid request outside the built kernel set          */
  GFA_ERR_WORKSPACE = 3,        /* workspace missing or too small                      */
  GFA_ERR_LAUNCH = 4            /* the HIP runtime rejected a kernel launch            */
} gfa_status;

/* Smallest legal lse_ld for a sequence length. */
#define GFA_LSE_LD(seq_len) ((((seq_len) + 63) / 64) * 64)

/* gfa_bwd_args.stages bits */
#define GFA_BWD_DQ 1  /* recomputing form: delta + dQ kernel; materialised: dQ from the dS store */
#define GFA_BWD_DKV 2 /* dK/dV kernel (+ Q-split reduction); materialised: delta kernel, then dK/dV */

/* Element strides (batch, head, row) of one 4-D tensor; the head-dim stride is 1. */
typedef struct {
  int64_t batch, head, row;
} gfa_strides;

typedef struct {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse; /* (B, Hq, lse_ld) natural-log logsumexp; NULL = inference (not stored) */
  gfa_strides q_strides, k_strides, v_strides, o_strides;
  int32_t batch, heads_q, heads_kv, seq_len, head_dim;
  int32_t causal;      /* 0 / 1 */
  int32_t window;      /* sliding window; 0 = off; honoured only when causal; >= seq_len -> off */
  float scale;         /* softmax scale, finite and > 0; the reference uses 1/sqrt(head_dim) */
  int32_t dtype;       /* gfa_dtype, shared by q/k/v/o */
  int32_t block_kv;    /* 0 = registry default, else a built tile width */
  int32_t lse_ld;      /* row length of lse (>= GFA_LSE_LD(seq_len)); ignored when lse == NULL */
  void* stream;        /* hipStream_t */
  const int32_t* seg_lo; /* optional (B, N) segment table (see above); NULL = one segment per row */
  const int32_t* seg_hi;
  float softcap;       /* 0 = off; > 0: every scaled score x = scale q.k becomes softcap tanh(x / softcap)
                          before the mask and softmax (transformers' logit soft-capping; the reference
                          has none). Runs the registry's default tiles (block_kv must be 0 or it). */
  float dropout_p;     /* 0 = off; in (0, 1): each P_ij is kept with probability 1 - dropout_p and scaled by
                          1 / (1 - dropout_p), else zeroed (the LSE is that of the undropped P). The mask
                          is a pure function of (dropout_seed, b, query head, i, j); the backward must get
                          the same seed. Not combined with softcap. Default tiles only, as softcap. */
  uint64_t dropout_seed;
} gfa_fwd_args;

typedef struct {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  const float* lse; /* from gfa_fwd, (B, Hq, lse_ld) */
  float* delta;     /* (B, Hq, lse_ld) scratch written by the dQ kernel: rowsum(dO * O), for
                       every row below seq_len rounded up to 32 (rows past seq_len repeat
                       row seq_len-1) */
  void* dq;
  void* dk;
  void* dv;
  gfa_strides q_strides, k_strides, v_strides, o_strides, do_strides, dq_strides, dk_strides, dv_strides;
  int32_t batch, heads_q, heads_kv, seq_len, head_dim;
  int32_t causal, window;
  float scale;
  int32_t dtype;
  int32_t q_splits;       /* 0 = registry choice, else 1, 2, 4 or 8 */
  int32_t lse_ld;         /* row length of lse and delta (>= GFA_LSE_LD(seq_len)) */
  int32_t stages;         /* 0 = all; else bitwise OR of GFA_BWD_DQ and GFA_BWD_DKV (profiling:
                             recomputing form: GFA_BWD_DKV alone reads the delta a previous
                             GFA_BWD_DQ wrote; materialised form: GFA_BWD_DKV runs delta and dK/dV,
                             GFA_BWD_DQ alone reads the dS store a previous GFA_BWD_DKV call left in
                             the same workspace) */
  void* workspace;        /* >= gfa_bwd_workspace_size(...) bytes when q_splits > 1; with
                             gfa_bwd_workspace_bytes(args) bytes the call runs the materialised
                             backward where that form exists */
  size_t workspace_bytes;
  void* stream;
  const int32_t* seg_lo;  /* the forward's segment table, or NULL */
  const int32_t* seg_hi;
  float softcap;          /* the forward's soft-cap (0 = off) */
  float dropout_p;        /* the forward's dropout probability and seed (0 = off) */
  uint64_t dropout_seed;
} gfa_bwd_args;

/* Tile configuration the library uses for one problem (mirrors the Python registry). */
typedef struct {
  int32_t head_dim;
  int32_t fwd_block_q;      /* query rows per forward workgroup */
  int32_t fwd_block_kv;     /* keys per LDS tile */
  int32_t fwd_waves;
  int32_t dq_block_q;
  int32_t dq_block_kv;
  int32_t dq_waves;
  int32_t dkv_block_kv;     /* keys per dKV workgroup */
  int32_t dkv_block_q;      /* queries per LDS tile */
  int32_t dkv_waves;
  int32_t q_splits;
} gfa_config_info;

/* Forward: O (and LSE unless lse == NULL). Returns a gfa_status. */
int gfa_fwd(const gfa_fwd_args* args);

/* Backward: delta, dQ, then dK/dV (summing Q-split fp32 partials when q_splits > 1).
 * Two forms, the same results to rounding:
 * - recomputing (the reference's, attention.py:1506-1620): the dQ kernel recomputes S, P and dP
 *   and computes delta in its prologue, then the dK/dV kernel;
 * - materialised: a delta kernel, the dK/dV kernel, which also stores every 32 x 32 block of dS
 *   it computes (16-bit, in the workspace), then dQ = scale * dS K from that store. It replaces
 *   two thirds of the dQ kernel's matrix work with 2 KiB of dS per block, written once and read
 *   once. Runs when the workspace holds the store (gfa_bwd_workspace_bytes), the store is within
 *   gfa_bwd_ds_limit and head_dim is 256 or 512 (soft-capping, dropout and segment tables
 *   included: the first two are in the stored dS, and the dQ kernel reads only the blocks the
 *   segment-trimmed dK/dV kernel writes); otherwise the recomputing form runs. */
int gfa_bwd(const gfa_bwd_args* args);

/* Bytes of the library-owned device scratch of gfa_bwd_noalloc, per GPU. */
#define GFA_NOALLOC_SCRATCH_BYTES (64u << 20)

/* gfa_bwd without caller-provided scratch. No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving or training
 * loops, harnesses that forbid hipMalloc). The caller passes inputs and outputs only: delta
 * and workspace must be NULL and workspace_bytes 0. delta and the Q-split partials live in a
 * file-scope device array of GFA_NOALLOC_SCRATCH_BYTES that each GPU the library runs on holds
 * until the process ends; the call itself allocates nothing. delta takes
 * batch * heads_q * lse_ld * 4 bytes (rounded up to 256) and the partials
 * gfa_bwd_workspace_size(...) bytes: a request beyond the scratch returns GFA_ERR_WORKSPACE.
 * q_splits = 0 takes the registry's split count, halved until its partials fit (1 needs none).
 * Every call on one GPU shares that GPU's scratch and leaves its contents there (a later
 * stages = GFA_BWD_DKV call reads the delta of the last GFA_BWD_DQ call): calls that overlap
 * on one GPU (concurrent streams or threads) race. It always runs the recomputing form (a dS
 * store does not fit a fixed scratch). Otherwise as gfa_bwd. */
int gfa_bwd_noalloc(const gfa_bwd_args* args);

/* Workspace bytes gfa_bwd needs for the given problem and q_splits (0 = registry choice) in the
 * recomputing form. */
size_t gfa_bwd_workspace_size(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t seq_len, int32_t head_dim,
                              int32_t causal, int32_t window, int32_t q_splits);

/* Workspace bytes of gfa_bwd(args) (the workspace fields are not read): the Q-split partials,
 * plus, where the materialised form applies, the dS store (batch * heads_q blocks of 2 KiB per
 * stored 32 x 32 (query tile, key tile) pair: per batch entry about heads_q * seq_len^2 bytes
 * under full causal masking, twice that without causal masking, 2 * heads_q * seq_len *
 * (window + 96) bytes with a sliding window). No counterpart in the reference. */
size_t gfa_bwd_workspace_bytes(const gfa_bwd_args* args);

/* Largest dS store the materialised backward uses, in bytes (default 32 GiB); a larger problem
 * runs the recomputing form, and 0 switches the materialised form off. A negative value only
 * queries. Process-wide; returns the limit before the call. No counterpart in the reference. */
int64_t gfa_bwd_ds_limit(int64_t bytes);

/* Fill *out with the configuration used for this problem without a sliding window (with a
 * window shorter than the sequence, the forward at head_dim 128 runs 32-key tiles, and the
 * dK/dV kernel at head_dim 256 runs role-split wave pairs, 64 keys per workgroup, two
 * workgroups per CU; gfa_bwd_workspace_size reports the split count for either). Returns a
 * gfa_status. */
int gfa_config(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t seq_len, int32_t head_dim,
               gfa_config_info* out);

/* Run-time work distribution of the long grids (no counterpart in the reference, whose grids the
 * Triton runtime launches as they are). With it on (the default), the forward and dQ kernels at
 * head_dim 512, when their grid exceeds one workgroup per CU, run as a persistent grid of one
 * workgroup per CU that takes the static grid's blocks, in their static order, from per-XCD
 * queues at run time (a faster XCD takes more blocks, no CU idles behind the hardware's in-order
 * dispatch). The queue counters live in a library-owned device array, one slot per launch out of
 * 256 used round-robin, zeroed by a one-workgroup kernel on the caller's stream before the
 * launch; the call still allocates nothing. Launches that overlap in time on different streams
 * must not share a slot: they must be fewer than 256 persistent launches apart. A launch captured
 * into a HIP graph keeps its slot for every replay, so graphs whose replays overlap on different
 * streams must not have been captured a multiple of 256 persistent launches apart (or must run
 * with this switched off). Every block computes exactly what it computes in the static grid, so
 * results are bit for bit the same either way. enable = 0 launches the static grids; a negative
 * value only queries. Process-wide; returns the setting before the call. */
int gfa_set_runtime_scheduling(int32_t enable);

/* Message of the last failing call on this thread ("" if none). */
const char* gfa_last_error(void);

/* GFA_VERSION of the built library. */
int gfa_version(void);

#ifdef __cplusplus
}
#endif

#endif /* GFA_H_ */
