// C ABI of the engine: argument validation, the HEAD_DIM-keyed tile registry, work
// decomposition and kernel dispatch. Nothing here allocates, frees or synchronises.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "gfa.h"
#include "gfa_launch.h"
#include "gfa_params.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return GFA_OK;
}

// ---------------------------------------------------------------------------------
// HEAD_DIM-keyed registry (mirrors registry.py). Replaces the reference's if/else tile
// tables (/root/reference/flash_attn/attention.py:561-579, 1445-1451, 1498-1504,
// 1536-1564) with MI355X tiles. Forward: one wave per 32 query rows over the full head
// dim; dQ: dq_split waves per 32 query rows (2 = a pair splitting the work by role, 1 = one
// wave over the full head dim). fwd_bkv_window is the forward tile used with a sliding window
// (narrower tiles waste less at the window edge: 8-11% faster at D=128 for windows up to 1024).
// dK/dV: see DkvForm; dkv_window is the form used with a sliding window.
// ---------------------------------------------------------------------------------
// dK/dV kernel form: queries per LDS tile, waves per workgroup, waves per 32 keys (2 = a
// pair splitting the work by role, P/dV and dS/dK; 1 = one wave doing all four products) and
// workgroups resident per CU.
struct DkvForm {
  int bq, waves, roles, wgs_per_cu;
};

struct Entry {
  int head_dim;
  int fwd_bkv, fwd_waves, fwd_bkv_window;
  int dq_bkv, dq_waves, dq_split;
  DkvForm dkv, dkv_window;
};

// D=256 with a window: role-split pairs at two waves per SIMD (64 keys per workgroup, two
// workgroups per CU), 5-10% faster on windows of 512 and 1024 than one wave per 32 keys,
// which stays for full causal and non-causal grids (2-5% faster there).
constexpr Entry kRegistry[] = {
    {512, 32, 4, 32, 32, 4, 2, {32, 4, 2, 1}, {32, 4, 2, 1}},
    {256, 32, 4, 32, 32, 4, 1, {32, 4, 1, 1}, {32, 4, 2, 2}},
    {128, 64, 4, 32, 32, 4, 1, {32, 4, 2, 2}, {32, 4, 2, 2}},
    {64, 64, 4, 64, 32, 4, 1, {32, 4, 1, 2}, {32, 4, 1, 2}},
};

// The window is in effect only with causal masking and when shorter than the sequence.
bool is_windowed(int causal, int window, int N) { return causal && window > 0 && window < N; }

const DkvForm& dkv_form(const Entry* e, int causal, int window, int N) {
  return is_windowed(causal, window, N) ? e->dkv_window : e->dkv;
}
// The form gfa_bwd launches: soft-capped and dropout instances exist for the default form only.
const DkvForm& bwd_dkv_form(const Entry* e, const gfa_bwd_args* a) {
  return (a->softcap > 0.f || a->dropout_p > 0.f) ? e->dkv : dkv_form(e, a->causal, a->window, a->seq_len);
}

const Entry* lookup(int d) {
  for (const Entry& e : kRegistry)
    if (e.head_dim == d) return &e;
  return nullptr;
}

bool fwd_built(int d, int bkv, int nw, bool cap) {
  if (cap)  // soft-capped instances: the registry's default tiles
    return nw == 4 && ((d == 512 && bkv == 32) || (d == 256 && bkv == 32) || (d == 128 && (bkv == 32 || bkv == 64)) ||
                       (d == 64 && bkv == 64));
  return nw == 4 && ((d == 512 && bkv == 32) || (d <= 256 && (bkv == 32 || bkv == 64)));
}

// Soft-capping: finite and >= 0 (0 = off); the kernels' multipliers.
int check_softcap(float softcap) {
  if (!std::isfinite(softcap) || softcap < 0.f)
    return fail(GFA_ERR_INVALID_ARGUMENT, "softcap=%g must be finite and >= 0 (0 = off)", (double)softcap);
  return GFA_OK;
}
// Dropout probability in [0, 1) (0 = off), not together with soft-capping.
int check_dropout(float p, float softcap) {
  if (!std::isfinite(p) || p < 0.f || p >= 1.f)
    return fail(GFA_ERR_INVALID_ARGUMENT, "dropout_p=%g must be in [0, 1)", (double)p);
  if (p > 0.f && softcap > 0.f) return fail(GFA_ERR_UNSUPPORTED, "dropout together with softcap is not built");
  return GFA_OK;
}
gfa::Dropout dropout_of(float p, uint64_t seed) {
  gfa::Dropout d;
  d.seed_lo = (unsigned)(seed & 0xffffffffu);
  d.seed_hi = (unsigned)(seed >> 32);
  const double t = (double)p * 4294967296.0;
  d.thresh = p > 0.f ? (unsigned)std::min(t, 4294967295.0) : 0u;
  d.inv_keep = 1.0f / (1.0f - p);
  return d;
}
gfa::SoftCap soft_cap(float scale, float softcap) {
  gfa::SoftCap c;
  c.cap_a = softcap > 0.f ? scale / softcap : 0.f;
  c.cap_log2 = softcap * 1.4426950408889634f;
  return c;
}

int largest_pow2_divisor_le(int r, int cap) {
  int x = 1;
  while (x * 2 <= cap && r % (x * 2) == 0) x *= 2;
  return x;
}

// units = 32-row query blocks per workgroup: one per wave in the forward kernel, one per
// wave pair in the dQ kernel.
gfa::QGrid make_qgrid(int B, int Hkv, int R, int N, int nu) {
  gfa::QGrid g;
  g.hpw = largest_pow2_divisor_le(R, nu);
  g.qbw = nu / g.hpw;
  g.n_hg = R / g.hpw;
  g.n_qsb = (N + 32 * g.qbw - 1) / (32 * g.qbw);
  g.nblocks = g.n_qsb * B * Hkv * g.n_hg;
  return g;
}

// Smallest of {1, 2, 4, 8} that fills the GPU with dK/dV workgroups: `rounds` rounds of
// 256 CUs x wgs_per_cu resident workgroups. A full-causal grid needs two rounds: its key
// blocks carry unequal work, which the heaviest-first grid order balances once there are
// two rounds or more; windowed and non-causal grids have near-uniform work and need one.
// Beyond that a split only adds fp32 partial traffic (measured on grids of 32 to 1024
// workgroups at D = 64..512, causal, windowed and full). units = 32-key units per workgroup.
int pick_q_splits(int B, int Hkv, int N, int units, int wgs_per_cu, bool full_causal) {
  const int keys_per_wg = 32 * units;
  const long long grid = (long long)((N + keys_per_wg - 1) / keys_per_wg) * B * Hkv;
  const long long want = (full_causal ? 2 : 1) * 256LL * wgs_per_cu;
  int qs = 1;
  while (qs < 8 && grid * qs < want) qs *= 2;
  return qs;
}

int pick_q_splits(const Entry* e, int B, int Hkv, int N, int causal, int window) {
  const DkvForm& f = dkv_form(e, causal, window, N);
  return pick_q_splits(B, Hkv, N, f.waves / f.roles, f.wgs_per_cu, causal && !is_windowed(causal, window, N));
}

gfa::RowView rv(const gfa_strides& s) { return gfa::RowView{s.batch, s.head, s.row}; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Rows past the end of a slice that a tile copy may address (largest tile 64 rows, and a
// loop's last prefetch starts at most one tile past the last row).
constexpr int kTileOverrun = 128;

int check_view(const char* name, const void* ptr, const gfa_strides& s, bool need_ptr) {
  if (need_ptr && ptr == nullptr) return fail(GFA_ERR_INVALID_ARGUMENT, "%s is NULL", name);
  if (ptr != nullptr && !aligned16(ptr)) return fail(GFA_ERR_INVALID_ARGUMENT, "%s is not 16-byte aligned", name);
  if ((s.row & 7) != 0 || (s.head & 7) != 0 || (s.batch & 7) != 0)
    return fail(GFA_ERR_INVALID_ARGUMENT, "%s strides (%lld, %lld, %lld) must be multiples of 8 elements", name,
                (long long)s.batch, (long long)s.head, (long long)s.row);
  if (s.row < 0 || s.head < 0 || s.batch < 0) return fail(GFA_ERR_INVALID_ARGUMENT, "%s has negative strides", name);
  return GFA_OK;
}

// The kernels move tiles with buffer instructions whose record count and offsets are 32-bit,
// one buffer resource per (batch, head) slice, so one slice (N rows at the row stride) must
// fit in 4 GiB. The last tile of a loop also addresses up to 127 rows past the sequence end
// (the range check turns them into zeros), and those offsets must not wrap either.
// Contiguous (B, H, N, D) tensors reach the limit only at (N + 127) * D > 2^31.
int check_span(const char* name, const gfa_strides& s, int N, int D) {
  const long long span = ((long long)(N - 1 + kTileOverrun) * s.row + D) * 2;
  if (span > 0xFFFFFFFFll)
    return fail(GFA_ERR_UNSUPPORTED,
                "%s: one (batch, head) slice spans %lld bytes; the tile copies address at most 4 GiB per slice "
                "(a contiguous (B, H, N, D) layout spans N * D * 2 bytes)",
                name, span);
  return GFA_OK;
}

int check_segments(const int32_t* lo, const int32_t* hi) {
  if ((lo == nullptr) != (hi == nullptr)) return fail(GFA_ERR_INVALID_ARGUMENT, "seg_lo and seg_hi go together");
  if (lo && ((reinterpret_cast<uintptr_t>(lo) & 3u) || (reinterpret_cast<uintptr_t>(hi) & 3u)))
    return fail(GFA_ERR_INVALID_ARGUMENT, "segment tables must be 4-byte aligned");
  return GFA_OK;
}

int check_dims(int B, int Hq, int Hkv, int N, int D, int dtype, int window) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || N <= 0)
    return fail(GFA_ERR_INVALID_ARGUMENT, "empty problem: B=%d Hq=%d Hkv=%d N=%d", B, Hq, Hkv, N);
  if (Hq % Hkv != 0) return fail(GFA_ERR_INVALID_ARGUMENT, "heads_q=%d is not a multiple of heads_kv=%d", Hq, Hkv);
  if (lookup(D) == nullptr) return fail(GFA_ERR_UNSUPPORTED, "head_dim=%d is not in the registry (64, 128, 256, 512)", D);
  if (dtype != GFA_DTYPE_FP16 && dtype != GFA_DTYPE_BF16) return fail(GFA_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
  if (window < 0) return fail(GFA_ERR_INVALID_ARGUMENT, "window=%d must be >= 0", window);
  // Every grid is at most one workgroup per 32-row block of every query head (forward, dQ)
  // or per 32 keys of every KV head and query split (dK/dV, up to 8 splits); grid sizes are
  // 32-bit.
  const long long blocks = ((long long)N + 31) / 32;
  if (blocks * B * Hq > 0x7fffffffll || blocks * B * Hkv * 8 > 0x7fffffffll)
    return fail(GFA_ERR_UNSUPPORTED, "B=%d Hq=%d N=%d needs more workgroups than one launch grid holds", B, Hq, N);
  return GFA_OK;
}

// ---------------------------------------------------------------------------------
// Run-time work hand-out (gfa::WorkQueue) for the D=512 forward and dQ grids. Their blocks carry
// unequal work (causal rows) and last 0.1-7 ms, and with one workgroup per CU the hardware's
// in-order dispatch leaves CUs idle while the next block waits for a CU on a busy shader engine;
// the eight XCDs also run at clocks up to 10% apart, and a static grid gives each the same share.
// A persistent grid of one workgroup per CU takes the blocks from per-XCD queues instead
// (gfa::WorkFetch): 1-2% off the forward and 2-3% off dQ at 8k-32k tokens. The dK/dV grid keeps
// the hardware's dispatch: the same hand-out made it 3-4% slower, with or without taking blocks
// from other XCDs' queues.
// The queue counters live in a library-owned device array of slots, handed out round-robin, one
// per launch; each launch first zeroes its slot with a one-workgroup kernel on the same stream (a
// kernel, not a memset, so that graph capture records an ordinary kernel node). A slot is reused
// after kWqSlots further launches on the device, which only a caller keeping that many launches
// in flight on other streams at once could overlap. Every GPU holds its own copy of the array;
// in host code `wq_pool` only names the symbol, whose address hipGetSymbolAddress gives per device.
// ---------------------------------------------------------------------------------
constexpr int kWqSlots = 256;
constexpr int kWqStride = 16;  // counters per slot (8 used), 64 bytes
static __device__ __align__(256) unsigned wq_pool[kWqSlots * kWqStride];

__global__ void wq_reset_kernel(unsigned* c) {
  if (threadIdx.x < kWqStride) c[threadIdx.x] = 0u;
}

struct WqDevice {
  std::atomic<unsigned*> base{nullptr};  // published after cus (release / acquire)
  int cus = 0;
  std::atomic<unsigned> next{0};
};
constexpr int kMaxWqDevices = 64;
std::mutex g_wq_mu;
WqDevice g_wq[kMaxWqDevices];

// The grids that take their blocks at run time: the forward and dQ kernels at D=512 (one
// workgroup per CU), unless switched off (gfa_set_runtime_scheduling).
std::atomic<int> g_runtime_scheduling{1};
bool dynamic_grid(int head_dim) { return head_dim == 512 && g_runtime_scheduling.load(std::memory_order_relaxed) != 0; }

// Fills `q` for a launch of `nblocks` static blocks on `stream`: the static grid, or a persistent
// grid of one workgroup per CU with a freshly zeroed counter slot.
int setup_queue(hipStream_t stream, int head_dim, int nblocks, gfa::WorkQueue* q) {
  q->wq = nullptr;
  q->grid = nblocks;
  if (!dynamic_grid(head_dim)) return GFA_OK;
  int dev = -1;
  hipError_t err = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (err != hipSuccess) return fail(GFA_ERR_LAUNCH, "cannot resolve the stream's device: %s", hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxWqDevices) return GFA_OK;  // untracked device: the static grid
  WqDevice& d = g_wq[dev];
  unsigned* base = d.base.load(std::memory_order_acquire);
  if (base == nullptr) {
    std::lock_guard<std::mutex> lock(g_wq_mu);
    base = d.base.load(std::memory_order_relaxed);
    if (base == nullptr) {
      int cur = -1;
      if ((err = hipGetDevice(&cur)) != hipSuccess)
        return fail(GFA_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(err));
      if (cur != dev && (err = hipSetDevice(dev)) != hipSuccess)
        return fail(GFA_ERR_LAUNCH, "hipSetDevice(%d) failed: %s", dev, hipGetErrorString(err));
      void* p = nullptr;
      int cus = 0;
      err = hipGetSymbolAddress(&p, HIP_SYMBOL(wq_pool));
      hipError_t err2 = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
      const hipError_t restore = cur != dev ? hipSetDevice(cur) : hipSuccess;  // the caller's device again
      if (err != hipSuccess || p == nullptr)
        return fail(GFA_ERR_LAUNCH, "hipGetSymbolAddress(wq_pool) failed on device %d: %s", dev, hipGetErrorString(err));
      if (err2 != hipSuccess || cus <= 0)
        return fail(GFA_ERR_LAUNCH, "cannot read the CU count of device %d: %s", dev, hipGetErrorString(err2));
      if (restore != hipSuccess)
        return fail(GFA_ERR_LAUNCH, "hipSetDevice(%d) restoring the caller's device failed: %s", cur,
                    hipGetErrorString(restore));
      d.cus = cus;
      base = static_cast<unsigned*>(p);
      d.base.store(base, std::memory_order_release);
    }
  }
  if (nblocks <= d.cus) return GFA_OK;  // one round: nothing to balance
  unsigned* c = base + (size_t)(d.next.fetch_add(1, std::memory_order_relaxed) % kWqSlots) * kWqStride;
  hipLaunchKernelGGL(wq_reset_kernel, dim3(1), dim3(64), 0, stream, c);
  if ((err = hipGetLastError()) != hipSuccess)
    return fail(GFA_ERR_LAUNCH, "work-queue reset launch failed: %s", hipGetErrorString(err));
  q->wq = c;
  q->grid = d.cus;
  return GFA_OK;
}

}  // namespace

extern "C" {

const char* gfa_last_error(void) { return g_err; }

int gfa_set_runtime_scheduling(int32_t enable) {
  if (enable < 0) return g_runtime_scheduling.load();
  return g_runtime_scheduling.exchange(enable ? 1 : 0);
}

int gfa_version(void) { return GFA_VERSION; }

int gfa_config(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t seq_len, int32_t head_dim,
               gfa_config_info* out) {
  if (out == nullptr) return fail(GFA_ERR_INVALID_ARGUMENT, "out is NULL");
  const Entry* e = lookup(head_dim);
  if (e == nullptr) return fail(GFA_ERR_UNSUPPORTED, "head_dim=%d is not in the registry (64, 128, 256, 512)", head_dim);
  if (heads_kv <= 0 || heads_q % heads_kv != 0 || batch <= 0 || seq_len <= 0)
    return fail(GFA_ERR_INVALID_ARGUMENT, "bad problem size");
  const gfa::QGrid g = make_qgrid(batch, heads_kv, heads_q / heads_kv, seq_len, e->fwd_waves);
  out->head_dim = head_dim;
  out->fwd_block_q = 32 * g.qbw;
  out->fwd_block_kv = e->fwd_bkv;
  out->fwd_waves = e->fwd_waves;
  const gfa::QGrid gq = make_qgrid(batch, heads_kv, heads_q / heads_kv, seq_len, e->dq_waves / e->dq_split);
  out->dq_block_q = 32 * gq.qbw;
  out->dq_block_kv = e->dq_bkv;
  out->dq_waves = e->dq_waves;
  out->dkv_block_kv = 32 * (e->dkv.waves / e->dkv.roles);
  out->dkv_block_q = e->dkv.bq;
  out->dkv_waves = e->dkv.waves;
  out->q_splits = pick_q_splits(e, batch, heads_kv, seq_len, 1, 0);
  return ok();
}

int gfa_fwd(const gfa_fwd_args* a) {
  if (a == nullptr) return fail(GFA_ERR_INVALID_ARGUMENT, "args is NULL");
  int rc = check_dims(a->batch, a->heads_q, a->heads_kv, a->seq_len, a->head_dim, a->dtype, a->window);
  if (rc) return rc;
  if ((rc = check_view("q", a->q, a->q_strides, true))) return rc;
  if ((rc = check_view("k", a->k, a->k_strides, true))) return rc;
  if ((rc = check_view("v", a->v, a->v_strides, true))) return rc;
  if ((rc = check_view("o", a->o, a->o_strides, true))) return rc;
  {
    const char* names[] = {"q", "k", "v", "o"};
    const gfa_strides* views[] = {&a->q_strides, &a->k_strides, &a->v_strides, &a->o_strides};
    for (int i = 0; i < 4; ++i)
      if ((rc = check_span(names[i], *views[i], a->seq_len, a->head_dim))) return rc;
  }
  if (!std::isfinite(a->scale) || !(a->scale > 0.f))
    return fail(GFA_ERR_INVALID_ARGUMENT, "scale=%g must be finite and positive", (double)a->scale);
  if ((rc = check_segments(a->seg_lo, a->seg_hi))) return rc;
  if ((rc = check_softcap(a->softcap))) return rc;
  if ((rc = check_dropout(a->dropout_p, a->softcap))) return rc;
  const bool cap = a->softcap > 0.f;
  const bool drop = a->dropout_p > 0.f;
  const Entry* e = lookup(a->head_dim);
  const bool windowed = is_windowed(a->causal, a->window, a->seq_len);
  const int bkv = a->block_kv ? a->block_kv : (windowed ? e->fwd_bkv_window : e->fwd_bkv);
  const int nw = e->fwd_waves;
  if (!fwd_built(a->head_dim, bkv, nw, cap || drop))
    return fail(GFA_ERR_UNSUPPORTED, "no forward kernel built for head_dim=%d block_kv=%d%s", a->head_dim, bkv,
                cap ? " with softcap" : drop ? " with dropout" : "");

  gfa::FwdParams p;
  p.seg_lo = a->seg_lo;
  p.seg_hi = a->seg_hi;
  p.q = static_cast<const uint16_t*>(a->q);
  p.k = static_cast<const uint16_t*>(a->k);
  p.v = static_cast<const uint16_t*>(a->v);
  p.o = static_cast<uint16_t*>(a->o);
  p.lse = a->lse;
  p.qv = rv(a->q_strides);
  p.kv = rv(a->k_strides);
  p.vv = rv(a->v_strides);
  p.ov = rv(a->o_strides);
  p.B = a->batch;
  p.Hq = a->heads_q;
  p.Hkv = a->heads_kv;
  p.N = a->seq_len;
  p.R = a->heads_q / a->heads_kv;
  p.causal = a->causal ? 1 : 0;
  // attention.py:1441-1443: a window covering the whole sequence is plain causal.
  p.window = is_windowed(a->causal, a->window, a->seq_len) ? a->window : 0;
  p.scale_log2 = a->scale * 1.4426950408889634f;
  p.cap = soft_cap(a->scale, a->softcap);
  p.drop = dropout_of(a->dropout_p, a->dropout_seed);
  p.store_lse = a->lse != nullptr;
  p.lse_ld = a->lse_ld;
  if (p.store_lse && (a->lse_ld < GFA_LSE_LD(a->seq_len) || !aligned16(a->lse) || (a->lse_ld & 3)))
    return fail(GFA_ERR_INVALID_ARGUMENT, "lse_ld=%d must be >= %d (multiple of 4, 16-byte aligned lse)", a->lse_ld,
                GFA_LSE_LD(a->seq_len));
  p.g = make_qgrid(p.B, p.Hkv, p.R, p.N, nw);
  if (p.g.nblocks <= 0) return fail(GFA_ERR_INVALID_ARGUMENT, "empty grid");
  if ((rc = setup_queue(static_cast<hipStream_t>(a->stream), a->head_dim, p.g.nblocks, &p.sched))) return rc;
  const hipError_t err = gfa::launch_fwd(p, a->head_dim, bkv, nw, a->dtype == GFA_DTYPE_BF16, cap, drop,
                                         static_cast<hipStream_t>(a->stream));
  if (err != hipSuccess) return fail(GFA_ERR_LAUNCH, "forward launch failed: %s", hipGetErrorString(err));
  return ok();
}

size_t gfa_bwd_workspace_size(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t seq_len, int32_t head_dim,
                              int32_t causal, int32_t window, int32_t q_splits) {
  (void)heads_q;
  const Entry* e = lookup(head_dim);
  if (e == nullptr || batch <= 0 || heads_kv <= 0 || seq_len <= 0) return 0;
  const int qs = q_splits > 0 ? q_splits : pick_q_splits(e, batch, heads_kv, seq_len, causal, window);
  if (qs <= 1) return 0;
  return (size_t)qs * 2 * batch * heads_kv * (size_t)seq_len * head_dim * sizeof(float);
}

}  // extern "C"

namespace {

// Validation and launches of the backward. `delta` and `ws` are the caller's buffers
// (gfa_bwd) or slices of the library's scratch array (gfa_bwd_noalloc); `qs_in` is the
// q_splits to use (0 = registry choice).
// Materialised backward (gfa_ds.h): the byte size of the dS store of `a`, 0 when the problem
// runs the recomputing form (store disabled or above the limit, segment tables, soft-capping,
// dropout, or a dK/dV form without 64-key workgroups and a dQ-from-dS kernel).
std::atomic<int64_t> g_ds_limit{int64_t(32) << 30};
size_t ds_store_bytes(const gfa_bwd_args* a) {
  const int64_t limit = g_ds_limit.load();
  // Segment tables trim the dK/dV kernel's query-tile ranges per key block and the dQ kernel
  // reads the same blocks (ds_seg_units); soft-capping and dropout are in the stored dS already.
  if (limit <= 0) return 0;
  const bool win = is_windowed(a->causal, a->window, a->seq_len);
  // D=128: the store's cost about equals the dQ work it saves (a timing variant measured the whole
  // backward 3% faster to 6% slower), so D <= 128 keeps the recomputing form.
  if (a->head_dim != 512 && a->head_dim != 256) return 0;
  const Entry* e = lookup(a->head_dim);
  // The storing forms: 4 waves, 32-row query tiles (role pairs, or one wave per 32 keys at D=256).
  const DkvForm& f = bwd_dkv_form(e, a);
  if (f.waves != 4 || f.bq != 32 || (f.roles != 1 && f.roles != 2)) return 0;
  const gfa::DsLayout l = gfa::ds_layout(a->seq_len, a->causal, win ? a->window : 0);
  const size_t bytes = (size_t)a->batch * a->heads_q * (size_t)l.slab * 2048;
  return bytes <= (size_t)limit ? bytes : 0;
}
size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

int bwd_impl(const gfa_bwd_args* a, float* delta_buf, void* ws_buf, size_t ws_bytes, int qs_in, bool allow_ds) {
  int rc = check_dims(a->batch, a->heads_q, a->heads_kv, a->seq_len, a->head_dim, a->dtype, a->window);
  if (rc) return rc;
  if ((rc = check_view("q", a->q, a->q_strides, true))) return rc;
  if ((rc = check_view("k", a->k, a->k_strides, true))) return rc;
  if ((rc = check_view("v", a->v, a->v_strides, true))) return rc;
  if ((rc = check_view("o", a->o, a->o_strides, true))) return rc;
  if ((rc = check_view("dout", a->dout, a->do_strides, true))) return rc;
  if ((rc = check_view("dq", a->dq, a->dq_strides, true))) return rc;
  if ((rc = check_view("dk", a->dk, a->dk_strides, true))) return rc;
  if ((rc = check_view("dv", a->dv, a->dv_strides, true))) return rc;
  {
    const char* names[] = {"q", "k", "v", "o", "dout", "dq", "dk", "dv"};
    const gfa_strides* views[] = {&a->q_strides, &a->k_strides, &a->v_strides, &a->o_strides,
                                  &a->do_strides, &a->dq_strides, &a->dk_strides, &a->dv_strides};
    for (int i = 0; i < 8; ++i)
      if ((rc = check_span(names[i], *views[i], a->seq_len, a->head_dim))) return rc;
  }
  if (a->lse == nullptr || delta_buf == nullptr) return fail(GFA_ERR_INVALID_ARGUMENT, "lse and delta are required");
  if (a->lse_ld < GFA_LSE_LD(a->seq_len) || (a->lse_ld & 3) || !aligned16(a->lse) || !aligned16(delta_buf))
    return fail(GFA_ERR_INVALID_ARGUMENT, "lse_ld=%d must be >= %d (multiple of 4, 16-byte aligned lse/delta)",
                a->lse_ld, GFA_LSE_LD(a->seq_len));
  if (!std::isfinite(a->scale) || !(a->scale > 0.f))
    return fail(GFA_ERR_INVALID_ARGUMENT, "scale=%g must be finite and positive", (double)a->scale);
  if ((rc = check_segments(a->seg_lo, a->seg_hi))) return rc;
  if ((rc = check_softcap(a->softcap))) return rc;
  if ((rc = check_dropout(a->dropout_p, a->softcap))) return rc;
  const bool cap = a->softcap > 0.f;
  const bool drop = a->dropout_p > 0.f;
  const int stages = a->stages ? a->stages : (GFA_BWD_DQ | GFA_BWD_DKV);
  if (stages & ~(GFA_BWD_DQ | GFA_BWD_DKV)) return fail(GFA_ERR_INVALID_ARGUMENT, "unknown stages bits 0x%x", stages);
  const Entry* e = lookup(a->head_dim);
  const int qs = qs_in > 0 ? qs_in : pick_q_splits(e, a->batch, a->heads_kv, a->seq_len, a->causal, a->window);
  if (qs != 1 && qs != 2 && qs != 4 && qs != 8) return fail(GFA_ERR_INVALID_ARGUMENT, "q_splits=%d not in {1,2,4,8}", qs);
  const size_t need = gfa_bwd_workspace_size(a->batch, a->heads_q, a->heads_kv, a->seq_len, a->head_dim, a->causal,
                                             a->window, qs);
  if (need > 0 && (ws_buf == nullptr || ws_bytes < need))
    return fail(GFA_ERR_WORKSPACE, "workspace of %zu bytes required (got %zu)", need, ws_bytes);
  if (need > 0 && !aligned16(ws_buf)) return fail(GFA_ERR_INVALID_ARGUMENT, "workspace is not 16-byte aligned");
  // The materialised form when the caller's workspace also holds the dS store.
  const size_t ds_bytes = allow_ds ? ds_store_bytes(a) : 0;
  const size_t ds_off = align256(need);
  const bool use_ds = ds_bytes > 0 && ws_buf != nullptr && aligned16(ws_buf) && ws_bytes >= ds_off + ds_bytes;

  const bool bf16 = a->dtype == GFA_DTYPE_BF16;
  const int R = a->heads_q / a->heads_kv;
  const int window = is_windowed(a->causal, a->window, a->seq_len) ? a->window : 0;
  const float scale_log2 = a->scale * 1.4426950408889634f;
  hipStream_t stream = static_cast<hipStream_t>(a->stream);

  gfa::BwdDqParams pq;
  pq.seg_lo = a->seg_lo;
  pq.seg_hi = a->seg_hi;
  pq.q = static_cast<const uint16_t*>(a->q);
  pq.k = static_cast<const uint16_t*>(a->k);
  pq.v = static_cast<const uint16_t*>(a->v);
  pq.o = static_cast<const uint16_t*>(a->o);
  pq.dout = static_cast<const uint16_t*>(a->dout);
  pq.lse = a->lse;
  pq.delta = delta_buf;
  pq.dq = static_cast<uint16_t*>(a->dq);
  pq.qv = rv(a->q_strides);
  pq.kv = rv(a->k_strides);
  pq.vv = rv(a->v_strides);
  pq.ov = rv(a->o_strides);
  pq.dov = rv(a->do_strides);
  pq.dqv = rv(a->dq_strides);
  pq.B = a->batch;
  pq.Hq = a->heads_q;
  pq.Hkv = a->heads_kv;
  pq.N = a->seq_len;
  pq.R = R;
  pq.causal = a->causal ? 1 : 0;
  pq.window = window;
  pq.scale = a->scale;
  pq.scale_log2 = scale_log2;
  pq.cap = soft_cap(a->scale, a->softcap);
  pq.drop = dropout_of(a->dropout_p, a->dropout_seed);
  pq.lse_ld = a->lse_ld;
  pq.g = make_qgrid(pq.B, pq.Hkv, R, pq.N, e->dq_waves / e->dq_split);
  hipError_t err = hipSuccess;
  if (stages & GFA_BWD_DQ && !use_ds) {
    if ((rc = setup_queue(stream, a->head_dim, pq.g.nblocks, &pq.sched))) return rc;
    err = gfa::launch_bwd_dq(pq, a->head_dim, e->dq_bkv, e->dq_split, bf16, cap, drop, stream);
    if (err != hipSuccess) return fail(GFA_ERR_LAUNCH, "dQ launch failed: %s", hipGetErrorString(err));
  }
  if (!(stages & GFA_BWD_DKV) && !use_ds) return ok();

  gfa::BwdDkvParams pk;
  pk.seg_lo = a->seg_lo;
  pk.seg_hi = a->seg_hi;
  pk.q = pq.q;
  pk.k = pq.k;
  pk.v = pq.v;
  pk.dout = pq.dout;
  pk.lse = a->lse;
  pk.delta = delta_buf;
  pk.dk = static_cast<uint16_t*>(a->dk);
  pk.dv = static_cast<uint16_t*>(a->dv);
  pk.part = static_cast<float*>(ws_buf);
  pk.qv = pq.qv;
  pk.kv = pq.kv;
  pk.vv = pq.vv;
  pk.dov = pq.dov;
  pk.dkv = rv(a->dk_strides);
  pk.dvv = rv(a->dv_strides);
  pk.B = a->batch;
  pk.Hq = a->heads_q;
  pk.Hkv = a->heads_kv;
  pk.N = a->seq_len;
  pk.R = R;
  pk.causal = pq.causal;
  pk.window = window;
  pk.scale = a->scale;
  pk.scale_log2 = scale_log2;
  pk.inv_scale = 1.0f / a->scale;
  pk.cap = pq.cap;
  pk.drop = pq.drop;
  pk.q_splits = qs;
  pk.lse_ld = a->lse_ld;
  // Soft-capped problems run the plain-chain form: the windowed D=256 pair starts its chains
  // from the row statistics and keeps no raw score. The split count stays the shared rule's
  // (any split is exact), so the workspace size does not depend on the cap.
  const DkvForm& f = bwd_dkv_form(e, a);
  const int keys_per_wg = 32 * (f.waves / f.roles);
  pk.n_kb = (pk.N + keys_per_wg - 1) / keys_per_wg;
  pk.nblocks = (pk.n_kb + 3) / 4 * 4 * pk.B * pk.Hkv * qs;  // key blocks in groups of four (bwd_dkv_kernel)
  pk.dsl = gfa::ds_layout(a->seq_len, a->causal, window);
  pk.dsl.ds = use_ds ? reinterpret_cast<uint16_t*>(static_cast<char*>(ws_buf) + ds_off) : nullptr;
  if (use_ds) {
    // delta, dK/dV (storing dS), then dQ from the store; GFA_BWD_DKV runs the first two,
    // GFA_BWD_DQ the last (reading the store a GFA_BWD_DKV call left in the same workspace).
    if (stages & GFA_BWD_DKV) {
      gfa::DeltaParams pd;
      pd.o = pq.o;
      pd.dout = pq.dout;
      pd.delta = delta_buf;
      pd.ov = pq.ov;
      pd.dov = pq.dov;
      pd.B = a->batch;
      pd.Hq = a->heads_q;
      pd.N = a->seq_len;
      pd.D = a->head_dim;
      pd.lse_ld = a->lse_ld;
      err = gfa::launch_delta(pd, bf16, stream);
      if (err != hipSuccess) return fail(GFA_ERR_LAUNCH, "delta launch failed: %s", hipGetErrorString(err));
      err = gfa::launch_bwd_dkv(pk, a->head_dim, f.bq, f.waves, f.roles, bf16, cap, drop, stream);
      if (err != hipSuccess) return fail(GFA_ERR_LAUNCH, "dKV launch failed: %s", hipGetErrorString(err));
      if (qs > 1) {
        err = gfa::launch_dkv_reduce(pk, a->head_dim, bf16, stream);
        if (err != hipSuccess) return fail(GFA_ERR_LAUNCH, "dKV reduce launch failed: %s", hipGetErrorString(err));
      }
    }
    if (stages & GFA_BWD_DQ) {
      gfa::BwdDqDsParams pz;
      pz.seg_lo = a->seg_lo;
      pz.seg_hi = a->seg_hi;
      pz.k = pq.k;
      pz.dq = pq.dq;
      pz.kv = pq.kv;
      pz.dqv = pq.dqv;
      pz.B = a->batch;
      pz.Hq = a->heads_q;
      pz.Hkv = a->heads_kv;
      pz.N = a->seq_len;
      pz.R = R;
      pz.scale = a->scale;
      pz.dsl = pk.dsl;
      pz.g = make_qgrid(pz.B, pz.Hkv, R, pz.N, 4);
      err = gfa::launch_bwd_dq_ds(pz, a->head_dim, bf16, stream);
      if (err != hipSuccess) return fail(GFA_ERR_LAUNCH, "dQ (from dS) launch failed: %s", hipGetErrorString(err));
    }
    return ok();
  }
  err = gfa::launch_bwd_dkv(pk, a->head_dim, f.bq, f.waves, f.roles, bf16, cap, drop, stream);
  if (err != hipSuccess) return fail(GFA_ERR_LAUNCH, "dKV launch failed: %s", hipGetErrorString(err));
  if (qs > 1) {
    err = gfa::launch_dkv_reduce(pk, a->head_dim, bf16, stream);
    if (err != hipSuccess) return fail(GFA_ERR_LAUNCH, "dKV reduce launch failed: %s", hipGetErrorString(err));
  }
  return ok();
}

// ---------------------------------------------------------------------------------
// Library-owned scratch of gfa_bwd_noalloc: the delta rows, then the Q-split fp32 partials.
// Every GPU the library runs on holds its own copy at its own address until the process
// ends. In host code `scratch` is only a stand-in for the symbol: its device address comes
// from hipGetSymbolAddress, taken once per device with that device current.
// ---------------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[GFA_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device `stream` belongs to (the current device for the
// null stream).
int scratch_on(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t err = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (err != hipSuccess) return fail(GFA_ERR_LAUNCH, "cannot resolve the stream's device: %s", hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxDevices) return fail(GFA_ERR_UNSUPPORTED, "device %d beyond the %d the library tracks", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    if ((err = hipGetDevice(&cur)) != hipSuccess)
      return fail(GFA_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(err));
    if (cur != dev && (err = hipSetDevice(dev)) != hipSuccess)
      return fail(GFA_ERR_LAUNCH, "hipSetDevice(%d) failed: %s", dev, hipGetErrorString(err));
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t restore = cur != dev ? hipSetDevice(cur) : hipSuccess;  // the caller's device again
    if (err != hipSuccess || p == nullptr)
      return fail(GFA_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(err));
    if (restore != hipSuccess)
      return fail(GFA_ERR_LAUNCH, "hipSetDevice(%d) restoring the caller's device failed: %s", cur,
                  hipGetErrorString(restore));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return GFA_OK;
}

}  // namespace

extern "C" {

size_t gfa_bwd_workspace_bytes(const gfa_bwd_args* a) {
  if (a == nullptr) return 0;
  const Entry* e = lookup(a->head_dim);
  if (e == nullptr || a->batch <= 0 || a->heads_kv <= 0 || a->seq_len <= 0) return 0;
  const int qs = a->q_splits > 0 ? a->q_splits : pick_q_splits(e, a->batch, a->heads_kv, a->seq_len, a->causal, a->window);
  const size_t need = gfa_bwd_workspace_size(a->batch, a->heads_q, a->heads_kv, a->seq_len, a->head_dim, a->causal,
                                             a->window, qs);
  const size_t ds = ds_store_bytes(a);
  return ds > 0 ? align256(need) + ds : need;
}

int64_t gfa_bwd_ds_limit(int64_t bytes) {
  if (bytes < 0) return g_ds_limit.load();
  return g_ds_limit.exchange(bytes);
}

int gfa_bwd(const gfa_bwd_args* a) {
  if (a == nullptr) return fail(GFA_ERR_INVALID_ARGUMENT, "args is NULL");
  return bwd_impl(a, a->delta, a->workspace, a->workspace_bytes, a->q_splits, true);
}

int gfa_bwd_noalloc(const gfa_bwd_args* a) {
  if (a == nullptr) return fail(GFA_ERR_INVALID_ARGUMENT, "args is NULL");
  if (a->delta != nullptr || a->workspace != nullptr || a->workspace_bytes != 0)
    return fail(GFA_ERR_INVALID_ARGUMENT,
                "gfa_bwd_noalloc keeps delta and the workspace in its own scratch: pass delta = NULL, "
                "workspace = NULL, workspace_bytes = 0");
  int rc = check_dims(a->batch, a->heads_q, a->heads_kv, a->seq_len, a->head_dim, a->dtype, a->window);
  if (rc) return rc;
  if (a->lse_ld < GFA_LSE_LD(a->seq_len) || (a->lse_ld & 3))
    return fail(GFA_ERR_INVALID_ARGUMENT, "lse_ld=%d must be >= %d (multiple of 4)", a->lse_ld, GFA_LSE_LD(a->seq_len));
  const size_t cap = GFA_NOALLOC_SCRATCH_BYTES;
  const size_t delta_bytes = ((size_t)a->batch * a->heads_q * a->lse_ld * sizeof(float) + 255) & ~(size_t)255;
  if (delta_bytes > cap)
    return fail(GFA_ERR_WORKSPACE, "delta needs %zu bytes; gfa_bwd_noalloc's scratch holds %zu (use gfa_bwd)",
                delta_bytes, cap);
  int qs = a->q_splits;
  if (qs == 0) {
    // The registry's split count, halved until its partials fit beside delta (1 needs none).
    const Entry* e = lookup(a->head_dim);
    qs = pick_q_splits(e, a->batch, a->heads_kv, a->seq_len, a->causal, a->window);
    while (qs > 1 && delta_bytes + gfa_bwd_workspace_size(a->batch, a->heads_q, a->heads_kv, a->seq_len, a->head_dim,
                                                          a->causal, a->window, qs) > cap)
      qs /= 2;
  }
  if (qs != 1 && qs != 2 && qs != 4 && qs != 8) return fail(GFA_ERR_INVALID_ARGUMENT, "q_splits=%d not in {1,2,4,8}", qs);
  const size_t ws = gfa_bwd_workspace_size(a->batch, a->heads_q, a->heads_kv, a->seq_len, a->head_dim, a->causal,
                                           a->window, qs);
  if (delta_bytes + ws > cap)
    return fail(GFA_ERR_WORKSPACE,
                "q_splits=%d needs %zu scratch bytes (delta %zu + partials %zu); gfa_bwd_noalloc holds %zu "
                "(use q_splits=0 or gfa_bwd)", qs, delta_bytes + ws, delta_bytes, ws, cap);
  void* base = nullptr;
  if ((rc = scratch_on(static_cast<hipStream_t>(a->stream), &base))) return rc;
  char* p = static_cast<char*>(base);
  return bwd_impl(a, reinterpret_cast<float*>(p), ws ? p + delta_bytes : nullptr, ws, qs, false);
}

}  // extern "C"
