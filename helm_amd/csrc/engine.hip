// C-ABI of libhelm_amd.so: launch planning, the per-device engine (copy
// stream, workspace, staging ring, descriptor uploads), page append and the
// evict / prefetch copies.  Declarations and contracts: include/helm_amd.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "attn_kernel.h"
#include "attn_mfma.h"
#include "front.h"
#include "helm_amd.h"

extern char** environ;

namespace helm {
namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  g_err = std::string(what) + ": " + hipGetErrorString(e);
  return static_cast<int>(e);
}

#define HELM_HIP(call)                                 \
  do {                                                 \
    hipError_t e_ = (call);                            \
    if (e_ != hipSuccess) return hip_fail(e_, #call);  \
  } while (0)

int elem_bytes(int dt) {
  switch (dt) {
    case HELM_F16:
    case HELM_BF16: return 2;
    case HELM_F32: return 4;
    default: return 0;
  }
}

// A mask's element type: HELM_F32, HELM_BF16 or HELM_F16 (read when mask != NULL).
bool mask_dtype_ok(const void* mask, int mask_dtype) {
  return !mask || mask_dtype == HELM_F32 || mask_dtype == HELM_BF16 || mask_dtype == HELM_F16;
}

int device_cus() {
  static int cus = 0;
  static std::once_flag once;
  std::call_once(once, [] {
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess) {
      int n = 0;
      if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount,
                                dev) == hipSuccess)
        cus = n;
    }
    if (cus <= 0) cus = 256;
  });
  return cus;
}

// The HELM_AMD_* switches, read per call.  getenv scans the whole
// environment for each name, and one call plans with about ten of them, so
// every public entry point that plans a launch opens an EnvScope: one pass
// over the environment keeps this thread's HELM_AMD_* entries, and env_get
// looks names up among those until the scope closes.  Outside a scope (or
// with more entries than the table holds) env_get is getenv.
struct EnvSnap {
  static constexpr int kMax = 32;
  bool active = false;
  int n = 0;
  const char* entry[kMax];  // "NAME=value" strings of the environment
};
thread_local EnvSnap g_env;

class EnvScope {
 public:
  EnvScope() : outer_(!g_env.active) {
    if (!outer_) return;
    int n = 0;
    bool fits = true;
    for (char** e = environ; e && *e; ++e) {
      if (std::strncmp(*e, "HELM_AMD_", 9) != 0) continue;
      if (n == EnvSnap::kMax) {
        fits = false;
        break;
      }
      g_env.entry[n++] = *e;
    }
    g_env.n = n;
    g_env.active = fits;
  }
  ~EnvScope() {
    if (outer_) g_env.active = false;
  }
  EnvScope(const EnvScope&) = delete;
  EnvScope& operator=(const EnvScope&) = delete;

 private:
  bool outer_;
};

const char* env_get(const char* name) {
  if (!g_env.active) return std::getenv(name);
  const size_t len = std::strlen(name);
  for (int i = 0; i < g_env.n; ++i) {
    const char* e = g_env.entry[i];
    if (std::strncmp(e, name, len) == 0 && e[len] == '=') return e + len + 1;
  }
  return nullptr;
}

int env_int(const char* name, int dflt) {
  const char* v = env_get(name);
  if (!v || !*v) return dflt;
  return std::atoi(v);
}

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// ---- kernel choice and split planning -----------------------------------
// Three kernels, chosen per call:
//   mfma    — matrix-core kernel (attn_mfma.h): 16-bit q == KV type, D = 128,
//             16-byte aligned operands; up to 16 query rows per tile;
//   fast    — vector-ALU dot2 kernel: same types, G <= 8 rows per tile;
//   generic — any D <= 256, fp32 or mixed q, 4 rows per tile.
// HELM_AMD_KERNEL = mfma | valu | generic restricts the choice (valu: no
// matrix cores; generic: the element-wise kernel only).
struct Plan {
  int mfma, fast, nw, fused, gm, rows, epl, n_qtiles, bpp, pps, max_splits;
  int row_waves;  // query chunks: 16-row tiles per wave (1: chunk_mfma_kernel, 2: chunk32)
  int direct;     // row-wave plan with one split: output written by the split kernel
  // workgroups per (sequence, KV head) along the query rows
  int qblocks() const {
    return row_waves ? (n_qtiles + nw * row_waves - 1) / (nw * row_waves) : n_qtiles;
  }
  size_t ticket_bytes, count_bytes, ml_bytes, o_bytes;
  size_t total() const { return ticket_bytes + count_bytes + ml_bytes + o_bytes; }
};

int pick_epl(int D) {
  for (int e : {1, 2, 4, 8, 16})
    if (16 * e >= D) return e;
  return 0;
}

// Smallest pages-per-split the automatic choice uses: every one of the nw
// waves gets at least two 16-token blocks.
int min_pps(int bpp, int nw) { return std::max(1, (2 * nw + bpp - 1) / bpp); }

// Waves per workgroup of the matrix-core kernel (HELM_AMD_WAVES = 4 | 8).
int mfma_waves() { return env_int("HELM_AMD_WAVES", 4) == 8 ? 8 : 4; }

// Split merge.  merge_splits_kernel spreads the merge of every tile over
// many workgroups; merging in-kernel (the last split of a tile to arrive
// reads every partial) saves that launch but is bound by one CU's load
// latency, so it is used only for tiles of at most kFusedMaxSplits splits.
// Measured per call (bf16, B = 1, D = 128, merge kernel vs in-kernel merge):
// Qwen3-8B shape 1k 8.6 vs 7.9 us, 2k (16 splits) 9.7 vs 8.7, Qwen3-0.6B 2k
// 9.7 vs 8.7; at 32 splits of 8-32 pages (4k-16k) the kernel wins, 10.5 vs
// 11.3, 12.7 vs 13.4, 17.4 vs 17.8.  HELM_AMD_MERGE = fused | kernel forces one.
constexpr int kFusedMaxSplits = 16;
int fused_merge(int max_splits) {
  const char* v = env_get("HELM_AMD_MERGE");
  if (v && !std::strcmp(v, "kernel")) return 0;
  if (v && !std::strcmp(v, "fused")) return 1;
  return max_splits <= kFusedMaxSplits ? 1 : 0;
}

int kernel_choice() {
  const char* v = env_get("HELM_AMD_KERNEL");
  if (!v || !*v || !std::strcmp(v, "auto") || !std::strcmp(v, "mfma")) return 2;
  if (!std::strcmp(v, "valu")) return 1;
  return 0;
}

// The in-kernel merge's tickets live in a fixed region at the start of every
// workspace that nothing else uses: zero since the workspace was zeroed and
// left zero by every call, whatever shapes earlier calls had (a region sized
// per call would grow into bytes an earlier call used for split counts or
// partials).  A call with more tiles than it holds merges in the second kernel.
constexpr size_t kTicketRegionBytes = 64 << 10;
// its second half holds the dynamic block claims' counters (256 tiles)
constexpr size_t kClaimRegionBytes = 32 << 10;

void size_plan(Plan& pl, int B, int Hkv, int D) {
  const size_t tiles = (size_t)B * Hkv * pl.n_qtiles;
  pl.ticket_bytes = kTicketRegionBytes;
  pl.count_bytes = align_up(tiles * 4, 256);
  pl.ml_bytes = align_up(tiles * pl.max_splits * pl.rows * 2 * 4, 256);
  pl.o_bytes = align_up(tiles * pl.max_splits * pl.rows * (size_t)D * 4, 256);
}

// Fused merge only where its tickets fit the ticket region and its 31-bit
// partial offsets reach every partial.
void settle_fused(Plan& pl, int B, int Hkv) {
  const size_t tiles = (size_t)B * Hkv * pl.n_qtiles;
  if (pl.o_bytes >= 0x7ffffff0u || tiles * 4 > kTicketRegionBytes - kClaimRegionBytes ||
      pl.row_waves)
    pl.fused = 0;
  pl.direct = (pl.row_waves && pl.max_splits == 1) ? 1 : 0;
}

// Rows, tiles and the split limits of a kernel choice.
void plan_shape(Plan& pl, int G, int q_len, int D, int max_tok_per_page) {
  pl.nw = pl.mfma ? mfma_waves() : kWaves;
  if (pl.mfma) {
    pl.gm = kMfmaRows;
    pl.rows = std::min(kMfmaRows, G * q_len);
    pl.epl = 8;
  } else {
    pl.gm = pl.fast ? G : 4;
    pl.rows = pl.gm;
    pl.epl = pl.fast ? 8 : pick_epl(D);
  }
  pl.n_qtiles = (G * q_len + pl.gm - 1) / pl.gm;
  pl.bpp = std::max(1, (max_tok_per_page + kBlockTok - 1) / kBlockTok);
  // query chunks of several 16-row tiles: the waves of a workgroup take one
  // tile each over the same pages (K/V read once per workgroup from L2, not
  // once per tile); HELM_AMD_ROW_WAVES=0 keeps one tile per workgroup
  // (HELM_AMD_CHUNK=16 keeps 16-row waves: chunk_mfma_kernel)
  pl.row_waves = (pl.mfma && pl.n_qtiles >= 2 && env_int("HELM_AMD_ROW_WAVES", 1))
                     ? (env_int("HELM_AMD_CHUNK", 32) == 16 ? 1 : 2)
                     : 0;
  if (pl.row_waves) pl.nw = kChunkStage;  // four waves per workgroup (see make_plan)
}

// chunk_mfma_kernel reads its page records in windows: a split may be long
constexpr int kChunkMaxPps = 1 << 20;
int max_pps_of(const Plan& pl) {
  return pl.row_waves ? kChunkMaxPps : pl.mfma ? kMfmaMaxPps : kMaxPps;
}
constexpr int kRaggedPps = 48;
int max_splits_of(const Plan& pl) { return pl.mfma ? kMfmaMaxSplits : kMaxSplits; }

// Pages per split for a batch whose page counts are known (helm_paged_attn_seqs
// with the compact grid): the split length in [lo_pps, max_pps] that
// minimises the busiest CU's share, ceil(units x sum_b ceil(pages_b / pps) /
// target) x (pps + kSplitCostPages), the longer split on a tie; a split's own
// cost (records, first loads, partial and merge) counts as kSplitCostPages
// pages.
constexpr int kSplitCostPages = 8;
int batch_pps(const int32_t* pages, int B, int units, int target, int lo_pps, int max_pps) {
  int best_pps = max_pps;
  int64_t best = -1;
  for (int pps = max_pps; pps >= std::max(1, lo_pps); --pps) {
    int64_t splits = 0;
    for (int b = 0; b < B; ++b) splits += (pages[b] + pps - 1) / pps;
    const int64_t cost =
        ((int64_t)units * splits + target - 1) / target * (pps + kSplitCostPages);
    if (best < 0 || cost < best) {
      best = cost;
      best_pps = pps;
    }
  }
  return best_pps;
}

// Pages per split when the split length cap (max_pps) leaves more splits
// than one round of `target` workgroups holds: every split is the same work,
// so the call lasts about as long as the busiest CU's share, ceil(workgroups
// / target) splits of pps pages.  The split count is chosen to minimise that
// (fewer splits on a tie): a sequence of 2,049 pages on 8 KV heads takes 63
// splits of 33 pages (two per CU) instead of 33 of 64 pages, where one CU of
// each XCD would walk two 64-page splits while the others walk one
// (Qwen3-8B shape, 32k + a few tokens through _decode_batched: 40.9 -> 34.0
// us per call; the Qwen3-14B B4 x 64k 40-layer step: 140.2 -> 141-142 steps/s,
// 138.4 -> 142-143 under the decode mask).
int balanced_pps(double pages, double units, int target, int lo_pps, int max_pps) {
  const double P = std::max(1.0, pages);
  const int s_min = (int)std::ceil(P / max_pps);
  int best_pps = max_pps;
  double best = -1.0;
  for (int s = s_min; s <= 4 * s_min; ++s) {
    const int pps = (int)std::ceil(P / s);
    if (pps < lo_pps) break;
    const double s_eff = std::ceil(P / pps);
    const double cost = std::ceil(units * s_eff / target) * pps;
    if (best < 0.0 || cost < best) {
      best = cost;
      best_pps = pps;
    }
  }
  return best_pps;
}

// work_pages: pages one (sequence, head, tile) walks on average; max_pages:
// the longest sequence (bounds the split count).
int make_plan(Plan& pl, int kv_dtype, int q_dtype, int B, int Hq, int Hkv,
              int q_len, int D, int max_tok_per_page, int max_pages,
              double avg_pages, int pps_req, bool aligned16) {
  if (Hkv <= 0 || Hq <= 0 || Hq % Hkv != 0)
    return fail(HELM_E_INVALID, "Hq must be a positive multiple of Hkv");
  if (D <= 0 || D > 256)
    return fail(HELM_E_UNSUPPORTED, "head_dim must be in [1, 256]");
  if (q_len <= 0 || B <= 0) return fail(HELM_E_INVALID, "empty query");
  if (elem_bytes(kv_dtype) == 0 || elem_bytes(q_dtype) == 0)
    return fail(HELM_E_INVALID, "unknown dtype");
  if (q_dtype != kv_dtype && q_dtype != HELM_F32)
    return fail(HELM_E_UNSUPPORTED,
                "query dtype must equal the KV dtype or be float32");
  const int G = Hq / Hkv;
  const int choice = kernel_choice();
  const bool same16 = kv_dtype == q_dtype && kv_dtype != HELM_F32 && D == 128 && aligned16;
  pl.mfma = (choice >= 2 && same16) ? 1 : 0;
  pl.fast = (!pl.mfma && choice >= 1 && same16 && G <= 8) ? 1 : 0;
  plan_shape(pl, G, q_len, D, max_tok_per_page);
  // chunk32 with eight waves (one workgroup of 256 query rows per CU) where a
  // KV head has at least 256 rows and the chunk attends over at least twice
  // its own length: each stage's K/V then crosses into LDS once per 256 rows
  // instead of once per 128 (512-token chunk over 32k: 0.43 -> 0.41 ms); a
  // first prompt chunk keeps four (its causal walks end earlier per
  // workgroup).  HELM_AMD_CHUNK_WAVES = 4 | 8 forces one.
  if (pl.row_waves == 2) {
    const int forced = env_int("HELM_AMD_CHUNK_WAVES", 0);
    const bool eight = forced ? forced == 8
                              : pl.n_qtiles >= 16 &&
                                    avg_pages * max_tok_per_page >= 2.0 * q_len;
    if (eight) pl.nw = 8;
  }
  int pps = pps_req > 0 ? pps_req : env_int("HELM_AMD_PPS", 0);
  if (pps <= 0) {
    const double units = (double)B * Hkv * pl.qblocks();
    // one workgroup per CU (two for the four-wave chunk kernels, whose 64 KiB
    // of LDS and 2 waves per SIMD let two share a CU): longer splits mean
    // fewer partials
    const int target =
        env_int("HELM_AMD_WG_PER_CU", pl.row_waves && pl.nw == 4 ? 2 : 1) * device_cus();
    const double splits = std::max(1.0, target / units);
    pps = (int)std::ceil(std::max(1.0, avg_pages) / splits);
    pps = std::max(pps, min_pps(pl.bpp, pl.nw));
    const bool capped = pps > max_pps_of(pl);
    pps = std::min(pps, max_pps_of(pl));
    const bool ragged = B > 1 && max_pages > 1.5 * avg_pages;
    // ragged batches that need several rounds of workgroups end with a long
    // tail of the longest sequences' splits; shorter splits shorten it
    // (Qwen3-14B B8, 4k-32k: 146.6 us at 64 pages per split, 123.6 at 48;
    // equal-length batches are best at 64)
    if (pl.mfma && !pl.row_waves && ragged && pps > kRaggedPps &&
        units * std::ceil(avg_pages / pps) > 2.0 * device_cus())
      pps = kRaggedPps;
    else if (capped && !ragged)
      pps = balanced_pps(avg_pages, units, target, min_pps(pl.bpp, pl.nw), pps);
  }
  pps = std::min(pps, max_pps_of(pl));
  pps = std::max(pps, (max_pages + max_splits_of(pl) - 1) / max_splits_of(pl));
  if (pps > max_pps_of(pl))
    return fail(HELM_E_UNSUPPORTED,
                "context longer than the split limit of the chosen kernel");
  pl.pps = std::max(pps, 1);
  pl.max_splits = std::max(1, (max_pages + pl.pps - 1) / pl.pps);
  pl.fused = fused_merge(pl.max_splits);
  size_plan(pl, B, Hkv, D);
  settle_fused(pl, B, Hkv);
  return HELM_OK;
}

// Splits of a chained (mixed residency) call: one run of splits per launch.
int chained_splits(const std::vector<std::pair<int, int>>& ranges, int pps) {
  int total = 0;
  for (const auto& r : ranges) total += (r.second - r.first + pps - 1) / pps;
  return total;
}

// Bytes from a page's head-0 token-0 element to the end of its last used
// token of the last head: what a host page's K (or V) copy must cover.
size_t page_extent(const helm_page& p, int Hkv, int D, int eb) {
  return ((size_t)(Hkv - 1) * p.head_stride + (size_t)p.used * D) * eb;
}

bool aligned(const void* p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

void fill_params(AttnParams& a, const Plan& pl, const void* q, void* out,
                 int B, int Hq, int Hkv, int q_len, int D, float scale,
                 float softcap, const void* mask, int64_t mbs, int64_t mhs,
                 int64_t mqs, int mask_dt, int causal, char* ws) {
  a.q = q;
  a.out = out;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.G = Hq / Hkv;
  a.S = q_len;
  a.D = D;
  a.rows_per_tile = pl.rows;
  a.n_qtiles = pl.n_qtiles;
  a.row_waves = pl.row_waves;
  a.direct_out = pl.direct;
  a.scale = scale;
  a.softcap = softcap;
  a.mask = mask;
  a.mask_bstride = mbs;
  a.mask_hstride = mhs;
  a.mask_qstride = mqs;
  a.mask_dt = mask_dt;
  a.causal = causal;
  a.pps = pl.pps;
  a.bpp = pl.bpp;
  a.bpp_log2 = -1;
  for (int k = 0; k < 31; ++k)
    if (pl.bpp == (1 << k)) a.bpp_log2 = k;
  a.lo = 0;
  a.hi = 0x7fffffff;
  a.split_base = 0;
  a.total_splits = 0;
  a.max_splits = pl.max_splits;
  a.full_d = 0;
  a.tickets = reinterpret_cast<uint32_t*>(ws);
  a.counts = reinterpret_cast<int*>(ws + pl.ticket_bytes);
  a.fused = pl.fused;
  a.ws_ml = reinterpret_cast<float*>(ws + pl.ticket_bytes + pl.count_bytes);
  a.ws_o = reinterpret_cast<float*>(ws + pl.ticket_bytes + pl.count_bytes + pl.ml_bytes);
  a.stamps = nullptr;
  a.dyn = 0;
  a.claims = nullptr;
}

// Dynamic block claiming for a one-launch matrix-core decode call
// (HELM_AMD_CLAIM=1): its counters sit in the second half of the ticket
// region (zero between calls), one 128-byte line per tile.  Which wave sums
// which block then depends on timing, so the fp32 sums' order (and the last
// bits of a result) can change from call to call; the static split (the
// default) gives the same bits for the same inputs.
void enable_claims(AttnParams& a, const Plan& pl, int B, int Hkv, char* ws) {
  const size_t tiles = (size_t)B * Hkv * pl.n_qtiles;
  if (!pl.mfma || pl.row_waves || tiles * kClaimStride * 4 > kClaimRegionBytes ||
      !env_int("HELM_AMD_CLAIM", 0))
    return;
  a.dyn = 1;
  a.claims = reinterpret_cast<uint32_t*>(ws + kTicketRegionBytes - kClaimRegionBytes);
}

hipError_t dispatch(const LaunchSpec& s, hipStream_t st) {
  switch (s.kv_dtype) {
    case HELM_F16: return launch_attn_f16(s, st);
    case HELM_BF16: return launch_attn_bf16(s, st);
    case HELM_F32: return launch_attn_f32(s, st);
    default: return hipErrorInvalidValue;
  }
}

// ---- split-kernel timing (helm_profile_split_kernels) ---------------------------
// Start / stop events of the split kernel launch of the next armed calls:
// pair i belongs to the i-th timed call.  g_prof_left > 0 only while armed,
// so an unarmed launch reads one atomic.
std::mutex g_prof_mu;
std::vector<hipEvent_t> g_prof_ev;
int g_prof_used = 0;
std::atomic<int> g_prof_left{0};

void prof_free_locked() {
  for (hipEvent_t ev : g_prof_ev)
    if (ev) (void)hipEventDestroy(ev);
  g_prof_ev.clear();
  g_prof_used = 0;
  g_prof_left.store(0);
}

// ---- workgroup stamps (helm_profile_workgroup_stamps) ----------------------------
// A caller's device buffer that the next decode-kernel launch writes its
// workgroups' stamps into; taken (and disarmed) by that launch.
std::atomic<uint64_t*> g_stamp_buf{nullptr};
std::atomic<int> g_stamp_cap{0};

// dispatch() with the armed timing events attached to the launch itself
// (hipExtLaunchKernelGGL's start / stop events: the kernel's own start and
// end, no queue gap before it)
hipError_t dispatch_timed(const LaunchSpec& s, hipStream_t st) {
  if (s.mfma && !s.p.row_waves && g_stamp_buf.load(std::memory_order_relaxed)) {
    const uint64_t wgs = (uint64_t)s.grid.x * s.grid.y * s.grid.z;
    if (wgs <= (uint64_t)g_stamp_cap.load()) {
      uint64_t* buf = g_stamp_buf.exchange(nullptr);
      if (buf) {
        LaunchSpec t = s;
        t.p.stamps = buf;
        return dispatch(t, st);
      }
    }
  }
  if (g_prof_left.load(std::memory_order_relaxed) > 0) {
    LaunchSpec t = s;
    {
      std::lock_guard<std::mutex> lock(g_prof_mu);
      if (g_prof_left.load() > 0) {
        t.ev_start = g_prof_ev[2 * g_prof_used];
        t.ev_stop = g_prof_ev[2 * g_prof_used + 1];
        ++g_prof_used;
        g_prof_left.fetch_sub(1);
      }
    }
    return dispatch(t, st);
  }
  return dispatch(s, st);
}

// Combines the split partials of every tile into the output (after the
// split kernels, on the same stream).
hipError_t launch_merge(const LaunchSpec& s, int B, int Hkv, hipStream_t st) {
  if (s.p.fused || s.p.direct_out) return hipSuccess;
  // column groups: spread each row's partial reads over several CUs
  const int chunks = (s.p.D % 4 == 0) ? s.p.D / 4 : s.p.D;
  const int groups = std::max(1, std::min(env_int("HELM_AMD_MERGE_GROUPS", 1), chunks));
  const dim3 grid(B * Hkv * s.p.n_qtiles, s.p.rows_per_tile, groups);
  // few splits per tile (query chunks): one thread per (row, column chunk)
  // walking the splits, eight rows per workgroup
  if (s.p.D == 128 && groups == 1 && s.p.max_splits <= kMergeBatch &&
      env_int("HELM_AMD_MERGE_ROWS", 1)) {
    const dim3 rgrid(B * Hkv * s.p.n_qtiles, (s.p.rows_per_tile + 7) / 8);
    switch (s.q_dtype) {
      case HELM_F16:
        hipLaunchKernelGGL(merge_rows_d128_kernel<f16_t>, rgrid, dim3(kThreads), 0, st, s.p);
        return hipGetLastError();
      case HELM_BF16:
        hipLaunchKernelGGL(merge_rows_d128_kernel<bf16_t>, rgrid, dim3(kThreads), 0, st, s.p);
        return hipGetLastError();
      case HELM_F32:
        hipLaunchKernelGGL(merge_rows_d128_kernel<float>, rgrid, dim3(kThreads), 0, st, s.p);
        return hipGetLastError();
      default: return hipErrorInvalidValue;
    }
  }
  if (s.p.D == 128 && groups == 1) {
    switch (s.q_dtype) {
      case HELM_F16:
        hipLaunchKernelGGL(merge_splits_d128_kernel<f16_t>, grid, dim3(kThreads), 0, st, s.p);
        return hipGetLastError();
      case HELM_BF16:
        hipLaunchKernelGGL(merge_splits_d128_kernel<bf16_t>, grid, dim3(kThreads), 0, st, s.p);
        return hipGetLastError();
      case HELM_F32:
        hipLaunchKernelGGL(merge_splits_d128_kernel<float>, grid, dim3(kThreads), 0, st, s.p);
        return hipGetLastError();
      default: return hipErrorInvalidValue;
    }
  }
  switch (s.q_dtype) {
    case HELM_F16:
      hipLaunchKernelGGL(merge_splits_kernel<f16_t>, grid, dim3(kThreads), 0, st, s.p);
      break;
    case HELM_BF16:
      hipLaunchKernelGGL(merge_splits_kernel<bf16_t>, grid, dim3(kThreads), 0, st, s.p);
      break;
    case HELM_F32:
      hipLaunchKernelGGL(merge_splits_kernel<float>, grid, dim3(kThreads), 0, st, s.p);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ---- page append kernel -----------------------------------------------------
constexpr int kAppendSegsPerLaunch = 24;
struct AppendArgs {
  helm_append_seg seg[kAppendSegsPerLaunch];
  int n_seg;
  int D;
  int eb;  // element bytes
};

// grid = (segment, kv head); copies n_tok x D elements of one head, 16 bytes
// per thread-step when every address and row is 16-byte aligned.
__global__ __launch_bounds__(256) void page_append_kernel(AppendArgs a) {
  const helm_append_seg& sg = a.seg[blockIdx.x];
  const int h = blockIdx.y;
  const int eb = a.eb;
  const int64_t row_b = (int64_t)a.D * eb;
  const char* sk = reinterpret_cast<const char*>(sg.src_k) +
                   (int64_t)h * sg.src_head_stride * eb;
  const char* sv = reinterpret_cast<const char*>(sg.src_v) +
                   (int64_t)h * sg.src_head_stride * eb;
  char* dk = reinterpret_cast<char*>(sg.dst_k) +
             ((int64_t)h * sg.dst_head_stride + (int64_t)sg.dst_tok * a.D) * eb;
  char* dv = reinterpret_cast<char*>(sg.dst_v) +
             ((int64_t)h * sg.dst_head_stride + (int64_t)sg.dst_tok * a.D) * eb;
  const int64_t sstride_b = sg.src_tok_stride * eb;
  const bool vec = (row_b % 16 == 0) && (sstride_b % 16 == 0) &&
                   ((reinterpret_cast<uintptr_t>(sk) |
                     reinterpret_cast<uintptr_t>(sv) |
                     reinterpret_cast<uintptr_t>(dk) |
                     reinterpret_cast<uintptr_t>(dv)) % 16 == 0);
  if (vec) {
    const int per_row = (int)(row_b / 16);
    const int n = sg.n_tok * per_row;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      const int s = i / per_row;
      const int c = i - s * per_row;
      const uint4 kx =
          *reinterpret_cast<const uint4*>(sk + s * sstride_b + c * 16);
      const uint4 vx =
          *reinterpret_cast<const uint4*>(sv + s * sstride_b + c * 16);
      *reinterpret_cast<uint4*>(dk + s * row_b + c * 16) = kx;
      *reinterpret_cast<uint4*>(dv + s * row_b + c * 16) = vx;
    }
  } else {
    const int n = sg.n_tok * a.D;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      const int s = i / a.D;
      const int d = i - s * a.D;
      if (eb == 4) {
        *reinterpret_cast<uint32_t*>(dk + s * row_b + d * 4) =
            *reinterpret_cast<const uint32_t*>(sk + s * sstride_b + d * 4);
        *reinterpret_cast<uint32_t*>(dv + s * row_b + d * 4) =
            *reinterpret_cast<const uint32_t*>(sv + s * sstride_b + d * 4);
      } else {
        *reinterpret_cast<uint16_t*>(dk + s * row_b + d * 2) =
            *reinterpret_cast<const uint16_t*>(sk + s * sstride_b + d * 2);
        *reinterpret_cast<uint16_t*>(dv + s * row_b + d * 2) =
            *reinterpret_cast<const uint16_t*>(sv + s * sstride_b + d * 2);
      }
    }
  }
}

}  // namespace

// Sets this thread's message (helm_last_error_string) for the library's
// other translation units; returns code.
int report_error(int code, const std::string& msg) { return fail(code, msg); }

}  // namespace helm

using namespace helm;

// ---- engine -------------------------------------------------------------------
struct helm_engine {
  int device = 0;
  hipStream_t copy = nullptr;
  // workspace: tickets (zeroed at allocation, left zero by every call),
  // split counts and partials
  char* ws = nullptr;
  size_t ws_bytes = 0;
  // staging ring for host pages
  char* ring = nullptr;
  size_t chunk_bytes = 0;
  int ring_slots = 0;
  int next_slot = 0;
  // per ring slot: its copies are complete (recorded on `copy`) / the launch
  // that reads it is complete (recorded on the caller's stream)
  std::vector<hipEvent_t> slot_ready, slot_free;
  // per ring slot, how its last reader was ordered: 0 none since the ring was
  // allocated, 1 slot_free recorded after it, 2 on the caller's stream only
  std::vector<uint8_t> slot_reader;
  // the last helm_evict_pages call's copies are complete (each eviction on a
  // new stream first waits for the previous one, so it covers them all)
  hipEvent_t evict_done = nullptr;
  hipStream_t evict_stream = nullptr;
  bool evict_recorded = false;
  // the ends of the last side-stream calls (recorded on the caller's stream),
  // by call count modulo kSideRing: the next such call waits on the host for
  // the one HELM_AMD_SIDE_AHEAD calls back
  static constexpr int kSideRing = 4;
  hipEvent_t side_done[kSideRing] = {};
  long long side_calls = 0;
  // descriptor uploads (pinned host -> device), a ring so the host can run ahead
  static constexpr int kUp = 8;
  char* up_host[kUp] = {};
  char* up_dev[kUp] = {};
  size_t up_bytes[kUp] = {};
  hipEvent_t up_done[kUp] = {};
  int up_used[kUp] = {};
  int up_next = 0;
  hipEvent_t ev_a = nullptr, ev_b = nullptr;
  // pinned host allocations [base, end) the device reads at the same address
  std::vector<std::pair<uint64_t, uint64_t>> host_ranges;
};

// ---- the no-allocation entry point's scratch ---------------------------------
// One array per GPU, in the code object's device memory: it exists from the
// module's load on that GPU to the end of the process.  Host code reaches it
// only through the address hipGetSymbolAddress returns for the current
// device (its name on the host is a stand-in, not a device address).
static __device__ __align__(256) unsigned char scratch[HELM_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};
bool g_scratch_dirty[kMaxScratchDevices] = {};

__global__ void zero_words_kernel(uint32_t* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    p[i] = 0u;
}

// The current device's scratch address (looked up once per device), with
// its ticket region cleared on `st` the first time, and again after a call
// that may not have completed (the split-merge tickets must start at zero;
// every completed call leaves them zero).  Allocates nothing.
int static_scratch(hipStream_t st, int* dev_out, void** out) {
  int dev = -1;
  HELM_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(HELM_E_UNSUPPORTED, "device index beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    HELM_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_scratch_ptr[dev] = p;
    g_scratch_dirty[dev] = true;
  }
  if (g_scratch_dirty[dev]) {
    const int words = static_cast<int>(kTicketRegionBytes / 4);
    hipLaunchKernelGGL(zero_words_kernel, dim3((words + 255) / 256), dim3(256), 0, st,
                       static_cast<uint32_t*>(g_scratch_ptr[dev]), words);
    HELM_HIP(hipGetLastError());
    g_scratch_dirty[dev] = false;
  }
  *dev_out = dev;
  *out = g_scratch_ptr[dev];
  return HELM_OK;
}

int engine_ensure_ws(helm_engine* e, size_t need, hipStream_t st) {
  if (need <= e->ws_bytes) return HELM_OK;
  HELM_HIP(hipStreamSynchronize(st));
  HELM_HIP(hipDeviceSynchronize());
  if (e->ws) HELM_HIP(hipFree(e->ws));
  e->ws = nullptr;
  e->ws_bytes = 0;
  const size_t sz = align_up(std::max(need, (size_t)(1 << 20)) * 3 / 2, 1 << 20);
  HELM_HIP(hipMalloc(&e->ws, sz));
  HELM_HIP(hipMemset(e->ws, 0, sz));
  e->ws_bytes = sz;
  return HELM_OK;
}

int engine_ensure_ring(helm_engine* e, size_t min_chunk) {
  if (min_chunk <= e->chunk_bytes && e->ring) return HELM_OK;
  HELM_HIP(hipDeviceSynchronize());
  if (e->ring) HELM_HIP(hipFree(e->ring));
  e->ring = nullptr;
  e->chunk_bytes = align_up(std::max(min_chunk, e->chunk_bytes), 1 << 20);
  HELM_HIP(hipMalloc(&e->ring, e->chunk_bytes * e->ring_slots));
  e->slot_reader.assign(e->ring_slots, 0);
  return HELM_OK;
}

// ---- host pages read in place --------------------------------------------------
// A host page is read by the kernel directly over the host link (no staging
// copy) when its K and V regions each lie inside one pinned host allocation
// that the device maps at the host address.  The kernels bound every load by
// the page's used tokens (buffer-resource limits), so they never touch bytes
// past page_extent().

// HELM_AMD_HOST_READ: "copy" stages every host page, "direct" reads every
// readable one in place, default "auto" decides per call (host_runs_favor_copy).
int host_read_mode() {
  const char* e = env_get("HELM_AMD_HOST_READ");
  if (e && std::strcmp(e, "copy") == 0) return 0;
  if (e && std::strcmp(e, "direct") == 0) return 2;
  return 1;
}

bool host_read_in_place() { return host_read_mode() != 0; }

// Where a call's staging copies go: on the engine's side stream
// (HELM_AMD_STAGE_STREAM=side) they run while the device pages' launch runs
// on the caller's stream, or (the default) on the caller's stream.
bool stage_on_side_stream() {
  const char* e = env_get("HELM_AMD_STAGE_STREAM");
  return e && std::strcmp(e, "side") == 0;
}

// How many side-stream calls may be queued ahead of the host: a call first
// waits until the one this many calls back has completed on its stream
// (HELM_AMD_SIDE_AHEAD, 0..4, 0 = no bound).  Unbounded, the host ran 3-6
// calls ahead and hipMemcpyAsync itself then held the calling thread for
// 5-16 ms at a time (the copies queued behind the earlier calls' kernels),
// after which the link and the kernels both waited for the host; two calls
// keep the side stream's copies one call ahead of the kernels without that.
int side_calls_ahead() {
  return std::min(helm_engine::kSideRing, std::max(0, env_int("HELM_AMD_SIDE_AHEAD", 2)));
}

// The staging copies reach the link's rate only in large runs: hipMemcpyAsync
// costs ~9 us per call here, so host pages that coalesce (adjacent in host
// memory, e.g. evicted in address order) into runs averaging >= 2 MiB are
// copied; scattered pages are read in place by the kernel.
constexpr uint64_t kStageMinRun = 2u << 20;

bool host_runs_favor_copy(const helm_page* pages, const std::vector<char>& sel,
                          int Hkv, int D, int eb) {
  std::vector<std::pair<uint64_t, uint64_t>> regions;
  for (size_t i = 0; i < sel.size(); ++i) {
    if (!sel[i]) continue;
    const uint64_t rb = page_extent(pages[i], Hkv, D, eb);
    regions.push_back({pages[i].k, rb});
    regions.push_back({pages[i].v, rb});
  }
  if (regions.empty()) return false;
  std::sort(regions.begin(), regions.end());
  uint64_t runs = 1, total = regions[0].second, end = regions[0].first + regions[0].second;
  for (size_t i = 1; i < regions.size(); ++i) {
    if (regions[i].first != end) ++runs;
    end = regions[i].first + regions[i].second;
    total += regions[i].second;
  }
  return total / runs >= kStageMinRun;
}

// [base, end) of the pinned host allocation holding `p`, if the device reads
// it at the same address.
bool query_host_range(uint64_t p, uint64_t* base, uint64_t* end) {
  hipPointerAttribute_t a{};
  if (hipPointerGetAttributes(&a, reinterpret_cast<void*>(p)) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  if (a.type != hipMemoryTypeHost ||
      reinterpret_cast<uint64_t>(a.devicePointer) != p ||
      reinterpret_cast<uint64_t>(a.hostPointer) != p)
    return false;
  hipDeviceptr_t b = nullptr;
  size_t sz = 0;
  if (hipMemGetAddressRange(&b, &sz, reinterpret_cast<hipDeviceptr_t>(p)) !=
      hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  *base = reinterpret_cast<uint64_t>(b);
  *end = *base + sz;
  return sz > 0 && p >= *base && p < *end;
}

// Index of the cached range holding [p, p + n), or -1.
int find_host_range(const helm_engine* e, uint64_t p, uint64_t n) {
  const auto& v = e->host_ranges;
  auto it = std::upper_bound(
      v.begin(), v.end(), p,
      [](uint64_t x, const std::pair<uint64_t, uint64_t>& r) { return x < r.first; });
  if (it == v.begin()) return -1;
  --it;
  if (p >= it->first && p + n <= it->second) return (int)(it - v.begin());
  return -1;
}

int add_host_range(helm_engine* e, uint64_t base, uint64_t end) {
  auto& v = e->host_ranges;
  if (v.size() >= 4096) v.clear();
  // drop stale entries overlapping the new allocation
  v.erase(std::remove_if(v.begin(), v.end(),
                         [&](const std::pair<uint64_t, uint64_t>& r) {
                           return r.first < end && base < r.second;
                         }),
          v.end());
  auto it = std::lower_bound(
      v.begin(), v.end(), std::make_pair(base, end));
  it = v.insert(it, {base, end});
  return (int)(it - v.begin());
}

// Marks direct[i] = 1 for the host pages the kernel can read in place.  Every
// allocation used is confirmed against the runtime on this call (a cached
// range whose allocation changed is dropped and its pages re-queried).
void resolve_host_pages(helm_engine* e, const helm_page* pages, int n, int Hkv,
                        int D, int eb, std::vector<char>& direct) {
  direct.assign(n, 0);
  if (!host_read_in_place()) return;
  for (int pass = 0; pass < 2; ++pass) {
    std::vector<int> used_idx;
    auto region_ok = [&](uint64_t p, uint64_t bytes) {
      int idx = find_host_range(e, p, bytes);
      if (idx < 0) {
        uint64_t b = 0, en = 0;
        if (!query_host_range(p, &b, &en) || p + bytes > en) return false;
        add_host_range(e, b, en);
      }
      return true;
    };
    for (int i = 0; i < n; ++i) {
      const helm_page& pg = pages[i];
      if (!(pg.flags & HELM_PAGE_HOST)) continue;
      const uint64_t bytes = page_extent(pg, Hkv, D, eb);
      direct[i] = region_ok(pg.k, bytes) && region_ok(pg.v, bytes);
    }
    // confirm every range this call relies on
    bool stale = false;
    std::vector<std::pair<uint64_t, uint64_t>> keep;
    for (int i = 0; i < n; ++i) {
      if (!direct[i]) continue;
      const uint64_t bytes = page_extent(pages[i], Hkv, D, eb);
      for (uint64_t p : {pages[i].k, pages[i].v}) {
        const int idx = find_host_range(e, p, bytes);
        if (idx < 0) { stale = true; break; }
        keep.push_back(e->host_ranges[idx]);
      }
    }
    std::sort(keep.begin(), keep.end());
    keep.erase(std::unique(keep.begin(), keep.end()), keep.end());
    for (const auto& r : keep) {
      uint64_t b = 0, en = 0;
      if (!query_host_range(r.first, &b, &en) || b != r.first || en != r.second) {
        stale = true;
        break;
      }
    }
    if (!stale) return;
    e->host_ranges.clear();
    direct.assign(n, 0);
  }
  direct.assign(n, 0);  // still inconsistent: stage every host page
}

// Two-phase upload through a ring of pinned staging buffers: reserve hands
// out the next slot's pinned host buffer (the caller writes `n` bytes there)
// and its device twin; commit queues the copy on `st`.  The slot is reused
// once the kernels that read it have run (engine_mark_upload_consumed).
int engine_upload_reserve(helm_engine* e, size_t n, char** host, char** dev) {
  const int i = e->up_next;
  if (e->up_used[i]) HELM_HIP(hipEventSynchronize(e->up_done[i]));
  e->up_used[i] = 0;
  if (n > e->up_bytes[i]) {
    if (e->up_host[i]) HELM_HIP(hipHostFree(e->up_host[i]));
    if (e->up_dev[i]) HELM_HIP(hipFree(e->up_dev[i]));
    e->up_host[i] = nullptr;
    e->up_dev[i] = nullptr;
    e->up_bytes[i] = 0;
    const size_t sz = align_up(std::max(n, (size_t)65536) * 2, 4096);
    HELM_HIP(hipHostMalloc(reinterpret_cast<void**>(&e->up_host[i]), sz,
                           hipHostMallocDefault));
    HELM_HIP(hipMalloc(&e->up_dev[i], sz));
    e->up_bytes[i] = sz;
  }
  *host = e->up_host[i];
  *dev = e->up_dev[i];
  return HELM_OK;
}

int engine_upload_commit(helm_engine* e, size_t n, hipStream_t st) {
  const int i = e->up_next;
  e->up_next = (e->up_next + 1) % helm_engine::kUp;
  HELM_HIP(hipMemcpyAsync(e->up_dev[i], e->up_host[i], n,
                          hipMemcpyHostToDevice, st));
  e->up_used[i] = 1;
  // the event is recorded by the caller after the consuming kernels
  return HELM_OK;
}

int engine_mark_upload_consumed(helm_engine* e, hipStream_t st) {
  const int i = (e->up_next + helm_engine::kUp - 1) % helm_engine::kUp;
  HELM_HIP(hipEventRecord(e->up_done[i], st));
  return HELM_OK;
}

// D2H / H2D copies on `st`, after everything already queued there; regions
// adjacent on both sides become one copy.  sync != 0 returns once they are
// done.
int engine_copies(helm_engine* e, int n, const uint64_t* src,
                  const uint64_t* dst, const uint64_t* bytes, hipMemcpyKind kind,
                  int sync, hipStream_t st) {
  if (n < 0) return fail(HELM_E_INVALID, "negative region count");
  if (n == 0) return HELM_OK;
  for (int i = 0; i < n; ++i)
    if (!src[i] || !dst[i]) return fail(HELM_E_INVALID, "null copy address");
  std::vector<int> idx(n);
  for (int i = 0; i < n; ++i) idx[i] = i;
  std::sort(idx.begin(), idx.end(),
            [&](int a, int b) { return src[a] < src[b]; });
  int i = 0;
  while (i < n) {
    uint64_t s0 = src[idx[i]], d0 = dst[idx[i]], len = bytes[idx[i]];
    int j = i + 1;
    while (j < n && src[idx[j]] == s0 + len && dst[idx[j]] == d0 + len) {
      len += bytes[idx[j]];
      ++j;
    }
    if (len)
      HELM_HIP(hipMemcpyAsync(reinterpret_cast<void*>(d0),
                              reinterpret_cast<const void*>(s0), len, kind, st));
    i = j;
  }
  if (sync) {
    HELM_HIP(hipEventRecord(e->ev_b, st));
    HELM_HIP(hipEventSynchronize(e->ev_b));
  }
  return HELM_OK;
}

}  // namespace

extern "C" {

const char* helm_last_error_string(void) { return g_err.c_str(); }

int helm_abi_version(void) { return HELM_AMD_ABI_VERSION; }

int helm_engine_create(int device, size_t chunk_bytes, int ring_slots,
                       helm_engine** out) {
  if (!out) return fail(HELM_E_INVALID, "null engine out pointer");
  *out = nullptr;
  HELM_HIP(hipSetDevice(device));
  helm_engine* e = new helm_engine();
  e->device = device;
  e->chunk_bytes = chunk_bytes ? chunk_bytes : (size_t)64 << 20;
  e->ring_slots = ring_slots > 0 ? ring_slots : 2;
  int rc = HELM_OK;
  auto chk = [&](hipError_t err, const char* what) {
    if (err != hipSuccess && rc == HELM_OK) rc = hip_fail(err, what);
  };
  chk(hipStreamCreateWithFlags(&e->copy, hipStreamNonBlocking),
      "hipStreamCreateWithFlags");
  for (int i = 0; i < helm_engine::kUp; ++i)
    chk(hipEventCreateWithFlags(&e->up_done[i], hipEventDisableTiming),
        "hipEventCreate");
  chk(hipEventCreateWithFlags(&e->ev_a, hipEventDisableTiming),
      "hipEventCreate");
  chk(hipEventCreateWithFlags(&e->ev_b, hipEventDisableTiming),
      "hipEventCreate");
  chk(hipEventCreateWithFlags(&e->evict_done, hipEventDisableTiming),
      "hipEventCreate");
  for (int i = 0; i < helm_engine::kSideRing; ++i)
    chk(hipEventCreateWithFlags(&e->side_done[i], hipEventDisableTiming), "hipEventCreate");
  e->slot_reader.assign(e->ring_slots, 0);
  e->slot_ready.assign(e->ring_slots, nullptr);
  e->slot_free.assign(e->ring_slots, nullptr);
  for (int i = 0; i < e->ring_slots; ++i) {
    chk(hipEventCreateWithFlags(&e->slot_ready[i], hipEventDisableTiming), "hipEventCreate");
    chk(hipEventCreateWithFlags(&e->slot_free[i], hipEventDisableTiming), "hipEventCreate");
  }
  if (rc != HELM_OK) {
    helm_engine_destroy(e);
    return rc;
  }
  *out = e;
  return HELM_OK;
}

int helm_profile_split_kernels(int n) {
  if (n < 0) return fail(HELM_E_INVALID, "negative call count");
  std::lock_guard<std::mutex> lock(g_prof_mu);
  prof_free_locked();
  if (n == 0) return HELM_OK;
  g_prof_ev.assign(2 * (size_t)n, nullptr);
  for (hipEvent_t& ev : g_prof_ev) {
    const hipError_t e = hipEventCreate(&ev);
    if (e != hipSuccess) {
      prof_free_locked();
      return hip_fail(e, "hipEventCreate");
    }
  }
  g_prof_left.store(n);
  return HELM_OK;
}

int helm_profile_workgroup_stamps(void* dev_buf, int max_workgroups) {
  if (max_workgroups < 0 || (max_workgroups > 0 && !dev_buf))
    return fail(HELM_E_INVALID, "bad stamp buffer");
  g_stamp_cap.store(max_workgroups);
  g_stamp_buf.store(max_workgroups > 0 ? reinterpret_cast<uint64_t*>(dev_buf) : nullptr);
  return HELM_OK;
}

int helm_profile_split_read(float* us_out, int max_n) {
  if (!us_out || max_n < 0) return fail(HELM_E_INVALID, "bad output array");
  std::lock_guard<std::mutex> lock(g_prof_mu);
  const int n = std::min(g_prof_used, max_n);
  for (int i = 0; i < n; ++i) {
    HELM_HIP(hipEventSynchronize(g_prof_ev[2 * i + 1]));
    float ms = 0.f;
    HELM_HIP(hipEventElapsedTime(&ms, g_prof_ev[2 * i], g_prof_ev[2 * i + 1]));
    us_out[i] = ms * 1e3f;
  }
  return n;
}

int helm_engine_destroy(helm_engine* e) {
  if (!e) return HELM_OK;
  // teardown: report nothing, release everything that was created
  (void)hipSetDevice(e->device);
  (void)hipDeviceSynchronize();
  if (e->ws) (void)hipFree(e->ws);
  if (e->ring) (void)hipFree(e->ring);
  for (int i = 0; i < helm_engine::kUp; ++i) {
    if (e->up_host[i]) (void)hipHostFree(e->up_host[i]);
    if (e->up_dev[i]) (void)hipFree(e->up_dev[i]);
    if (e->up_done[i]) (void)hipEventDestroy(e->up_done[i]);
  }
  if (e->ev_a) (void)hipEventDestroy(e->ev_a);
  if (e->ev_b) (void)hipEventDestroy(e->ev_b);
  if (e->evict_done) (void)hipEventDestroy(e->evict_done);
  for (hipEvent_t ev : e->side_done)
    if (ev) (void)hipEventDestroy(ev);
  for (hipEvent_t ev : e->slot_ready)
    if (ev) (void)hipEventDestroy(ev);
  for (hipEvent_t ev : e->slot_free)
    if (ev) (void)hipEventDestroy(ev);
  if (e->copy) (void)hipStreamDestroy(e->copy);
  delete e;
  return HELM_OK;
}

void* helm_engine_copy_stream(helm_engine* e) {
  return e ? reinterpret_cast<void*>(e->copy) : nullptr;
}

size_t helm_query_workspace_bytes(int B, int Hq, int Hkv, int q_len, int D,
                                  int max_pages, int page_size,
                                  int pages_per_split) {
  if (B <= 0 || Hkv <= 0 || Hq <= 0 || Hq % Hkv || q_len <= 0 || D <= 0 ||
      page_size <= 0 || max_pages < 0)
    return 0;
  const int G = Hq / Hkv;
  size_t best = 0;
  // the largest of the plans any kernel choice can make for this shape
  for (int kind = 0; kind < 3; ++kind) {
    Plan pl{};
    pl.mfma = kind == 2;
    pl.fast = kind == 1 && G <= 8;
    plan_shape(pl, G, q_len, D, page_size);
    int pps = pages_per_split > 0 ? std::min(pages_per_split, max_pps_of(pl))
                                  : min_pps(pl.bpp, 4);
    pps = std::min(pps, max_pps_of(pl));
    pps = std::max(pps, (max_pages + max_splits_of(pl) - 1) / max_splits_of(pl));
    pl.max_splits = std::max(1, (max_pages + pps - 1) / pps);
    size_plan(pl, B, Hkv, D);
    best = std::max(best, pl.total());
  }
  return best;
}

int helm_paged_decode_attn(const void* q, void* out, const void* k_pool,
                           const void* v_pool, int64_t slot_stride,
                           int64_t head_stride, const int32_t* page_table,
                           int table_stride, const int32_t* seq_lens, int B,
                           int Hq, int Hkv, int q_len, int D, int page_size,
                           int max_pages, int total_pages, const int32_t* seq_lens_host,
                           float scale, float softcap, const void* mask,
                           int64_t mask_bstride, int64_t mask_hstride,
                           int64_t mask_qstride, int mask_dtype, int kv_dtype, int q_dtype,
                           int pages_per_split, void* workspace,
                           size_t ws_bytes, void* stream) {
  EnvScope env_scope;
  if (!q || !out || !k_pool || !v_pool || !page_table || !seq_lens ||
      !workspace)
    return fail(HELM_E_INVALID, "null pointer argument");
  if (page_size <= 0 || max_pages < 0 || table_stride < max_pages)
    return fail(HELM_E_INVALID, "bad page_size / max_pages / table_stride");
  if (!mask_dtype_ok(mask, mask_dtype)) return fail(HELM_E_INVALID, "unknown mask dtype");
  const int eb = elem_bytes(kv_dtype);
  const int qb = elem_bytes(q_dtype);
  const bool al = aligned(q, 16) && aligned(out, 16) && aligned(k_pool, 16) &&
                  aligned(v_pool, 16) && (slot_stride * eb) % 16 == 0 &&
                  (head_stride * eb) % 16 == 0 && (D * qb) % 16 == 0;
  const double avg = total_pages > 0 ? (double)total_pages / B : max_pages;
  Plan pl{};
  int rc = make_plan(pl, kv_dtype, q_dtype, B, Hq, Hkv, q_len, D, page_size,
                     max_pages, avg, pages_per_split, al);
  if (rc != HELM_OK) return rc;
  // the sequences' lengths on the host (a batch on the decode kernel): the
  // split length from every sequence's page count and a grid of exactly
  // their splits, as helm_paged_attn_seqs numbers them; the partial buffers
  // keep the stride of the declared table width
  int32_t seq_np[kSeqArgs];
  bool compact = seq_lens_host && pl.mfma && !pl.row_waves && B > 1 && B <= kSeqArgs &&
                 env_int("HELM_AMD_COMPACT", 1);
  for (int b = 0; b < B && compact; ++b) {
    const int64_t np = ((int64_t)seq_lens_host[b] + page_size - 1) / page_size;
    seq_np[b] = (int32_t)std::min<int64_t>(np, max_pages);
    compact = seq_lens_host[b] > 0;
  }
  if (compact) {
    if (pages_per_split <= 0 && env_int("HELM_AMD_PPS", 0) <= 0) {
      const int cand = batch_pps(seq_np, B, Hkv * pl.qblocks(), device_cus(),
                                 min_pps(pl.bpp, pl.nw), max_pps_of(pl));
      if ((max_pages + cand - 1) / cand <= max_splits_of(pl)) pl.pps = cand;
    }
    pl.max_splits = std::max(1, (max_pages + pl.pps - 1) / pl.pps);
    pl.fused = fused_merge(pl.max_splits);
    size_plan(pl, B, Hkv, D);
    settle_fused(pl, B, Hkv);
  }
  if (ws_bytes < pl.total())
    return fail(HELM_E_WORKSPACE,
                "workspace too small: need " + std::to_string(pl.total()));
  LaunchSpec s{};
  fill_params(s.p, pl, q, out, B, Hq, Hkv, q_len, D, scale, softcap, mask,
              mask_bstride, mask_hstride, mask_qstride, mask_dtype, 0,
              reinterpret_cast<char*>(workspace));
  enable_claims(s.p, pl, B, Hkv, reinterpret_cast<char*>(workspace));
  s.p.full_d = (al && D == 16 * pl.epl) ? 1 : 0;
  s.mode = 0;
  s.pool.k_pool = reinterpret_cast<const char*>(k_pool);
  s.pool.v_pool = reinterpret_cast<const char*>(v_pool);
  s.pool.slot_stride_b = slot_stride * eb;
  s.pool.head_stride_b = head_stride * eb;
  s.pool.table = page_table;
  s.pool.table_stride = table_stride;
  s.pool.seq_lens = seq_lens;
  s.pool.page_size = page_size;
  s.pool.max_pages = max_pages;
  s.kv_dtype = kv_dtype;
  s.q_dtype = q_dtype;
  s.epl = pl.epl;
  s.gm = pl.gm;
  s.fast = pl.fast;
  s.mfma = pl.mfma;
  s.nw = pl.nw;
  s.feat = (mask ? kFeatMask : 0) | (mask && mask_dtype != HELM_F32 ? kFeatMask16 : 0) |
           (softcap > 0.f ? kFeatCap : 0);
  s.grid = dim3(std::max(1, pl.max_splits), Hkv * pl.qblocks(), B);
  if (compact) {
    int all_splits = 0;
    for (int b = 0; b < B; ++b) {
      s.pool.seq_split0[b] = all_splits;
      all_splits += (seq_np[b] + pl.pps - 1) / pl.pps;
    }
    s.pool.compact = 1;
    s.pool.n_seq = B;
    s.grid = dim3(all_splits, Hkv * pl.qblocks(), 1);
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipError_t e = dispatch_timed(s, st);
  if (e != hipSuccess) return hip_fail(e, "paged_attn launch");
  e = launch_merge(s, B, Hkv, st);
  if (e != hipSuccess) return hip_fail(e, "merge launch");
  return HELM_OK;
}

int helm_paged_decode_attn_static(const void* q, void* out, const void* k_pool,
                                  const void* v_pool, int64_t slot_stride,
                                  int64_t head_stride, const int32_t* page_table,
                                  int table_stride, const int32_t* seq_lens, int B,
                                  int Hq, int Hkv, int q_len, int D, int page_size,
                                  int max_pages, int total_pages,
                                  const int32_t* seq_lens_host, float scale,
                                  float softcap, const void* mask,
                                  int64_t mask_bstride, int64_t mask_hstride,
                                  int64_t mask_qstride, int mask_dtype, int kv_dtype, int q_dtype,
                                  int pages_per_split, void* stream) {
  EnvScope env_scope;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  int dev = -1;
  void* ws = nullptr;
  int rc = static_scratch(st, &dev, &ws);
  if (rc != HELM_OK) return rc;
  rc = helm_paged_decode_attn(q, out, k_pool, v_pool, slot_stride, head_stride, page_table,
                              table_stride, seq_lens, B, Hq, Hkv, q_len, D, page_size,
                              max_pages, total_pages, seq_lens_host, scale, softcap, mask,
                              mask_bstride, mask_hstride, mask_qstride, mask_dtype, kv_dtype,
                              q_dtype, pages_per_split, ws, HELM_STATIC_SCRATCH_BYTES, stream);
  if (rc > 0) {
    // a launch failed part-way: the tickets may not be back at zero
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    g_scratch_dirty[dev] = true;
  }
  if (rc == HELM_E_WORKSPACE)
    return fail(HELM_E_WORKSPACE,
                "this shape needs more than the static scratch's " +
                    std::to_string(HELM_STATIC_SCRATCH_BYTES >> 20) +
                    " MiB (use helm_paged_decode_attn with a workspace)");
  return rc;
}

int helm_stream_attn(helm_engine* eng, const void* q, void* out, int B,
                     int Hq, int Hkv, int q_len, int D, const helm_page* pages,
                     const int32_t* seq_off, float scale, float softcap,
                     const void* mask, int64_t mask_bstride,
                     int64_t mask_hstride, int64_t mask_qstride, int mask_dtype, int causal,
                     int kv_dtype, int q_dtype, void* stream) {
  EnvScope env_scope;
  if (!eng || !q || !out || !seq_off)
    return fail(HELM_E_INVALID, "null pointer argument");
  if (B <= 0) return fail(HELM_E_INVALID, "B must be positive");
  if (Hkv <= 0 || D <= 0) return fail(HELM_E_INVALID, "bad Hkv / D");
  if (causal < 0) return fail(HELM_E_INVALID, "causal must be >= 0");
  if (!mask_dtype_ok(mask, mask_dtype)) return fail(HELM_E_INVALID, "unknown mask dtype");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int eb = elem_bytes(kv_dtype);
  const int qb = elem_bytes(q_dtype);
  if (!eb || !qb) return fail(HELM_E_INVALID, "unknown dtype");
  const int n_all = seq_off[B];
  if (seq_off[0] != 0 || n_all < 0)
    return fail(HELM_E_INVALID, "seq_off must start at 0");
  if (n_all > 0 && !pages) return fail(HELM_E_INVALID, "null pages");

  // ---- validate -------------------------------------------------------------
  int max_pages = 0, max_tok = 1, n_hostflag = 0;
  for (int b = 0; b < B; ++b) {
    const int n = seq_off[b + 1] - seq_off[b];
    if (n < 0) return fail(HELM_E_INVALID, "seq_off not monotone");
    max_pages = std::max(max_pages, n);
  }
  for (int i = 0; i < n_all; ++i) {
    const helm_page& p = pages[i];
    if (p.used <= 0 || !p.k || !p.v || p.head_stride < p.used * D)
      return fail(HELM_E_INVALID, "bad page descriptor " + std::to_string(i));
    max_tok = std::max(max_tok, p.used);
    if (p.flags & HELM_PAGE_HOST) ++n_hostflag;
  }
  // host pages in mapped pinned memory are read in place; the rest are staged
  std::vector<char> direct;
  if (n_hostflag) resolve_host_pages(eng, pages, n_all, Hkv, D, eb, direct);
  else direct.assign(n_all, 0);
  if (n_hostflag && B == 1 && host_read_mode() == 1 &&
      host_runs_favor_copy(pages, direct, Hkv, D, eb))
    direct.assign(n_all, 0);
  int n_host = 0;
  size_t max_region = 0;
  for (int i = 0; i < n_all; ++i) {
    if ((pages[i].flags & HELM_PAGE_HOST) && !direct[i]) {
      ++n_host;
      max_region = std::max(max_region, 2 * page_extent(pages[i], Hkv, D, eb));
    }
  }
  if (n_host && B != 1)
    return fail(HELM_E_UNSUPPORTED,
                "host pages outside mapped pinned memory need B == 1");

  // ---- descriptor order: per sequence the host pages read in place (the
  // longest-running splits start first), then device pages; staged host
  // pages follow chunk by chunk -------------------------------------------
  std::vector<helm_page> desc;
  desc.reserve(n_all);
  std::vector<int32_t> off(B + 1, 0);
  struct Launch { int lo, hi, chunk; };
  struct Run { uint64_t src; size_t bytes; size_t dst_off; };
  std::vector<Launch> launches;
  std::vector<std::vector<Run>> chunk_runs;
  std::vector<int> chunk_slot;
  auto push_resident = [&](int lo, int hi) {
    for (int i = lo; i < hi; ++i)
      if (direct[i]) {
        desc.push_back(pages[i]);
        desc.back().flags = 0;
      }
    for (int i = lo; i < hi; ++i)
      if (!(pages[i].flags & HELM_PAGE_HOST)) desc.push_back(pages[i]);
  };

  // all pages on the device: the caller's records are uploaded as they are
  bool as_given = !n_hostflag;
  if (!n_host) {
    if (n_hostflag)
      for (int b = 0; b < B; ++b) push_resident(seq_off[b], seq_off[b + 1]);
    for (int b = 0; b <= B; ++b) off[b] = seq_off[b];
  } else {
    int rc = engine_ensure_ring(eng, max_region);
    if (rc != HELM_OK) return rc;
    push_resident(0, n_all);
    if (!desc.empty()) launches.push_back({0, (int)desc.size(), -1});
    std::vector<int> hidx;
    for (int i = 0; i < n_all; ++i)
      if ((pages[i].flags & HELM_PAGE_HOST) && !direct[i]) hidx.push_back(i);
    std::sort(hidx.begin(), hidx.end(),
              [&](int a, int b) { return pages[a].k < pages[b].k; });
    size_t used_b = 0;
    int chunk_lo = (int)desc.size();
    chunk_runs.emplace_back();
    // Staged position of a host region; regions adjacent in host memory stay
    // adjacent in the chunk and share one copy.
    auto add_region = [&](uint64_t src, size_t bytes) -> uint64_t {
      std::vector<Run>& runs = chunk_runs.back();
      const size_t dst = used_b;
      if (!runs.empty() && runs.back().src + runs.back().bytes == src &&
          runs.back().dst_off + runs.back().bytes == dst)
        runs.back().bytes += bytes;
      else
        runs.push_back({src, bytes, dst});
      used_b += bytes;
      return dst;
    };
    for (int i : hidx) {
      const helm_page& p = pages[i];
      const size_t rb = page_extent(p, Hkv, D, eb);
      if (used_b > 0 && used_b + 2 * rb > eng->chunk_bytes) {
        launches.push_back(
            {chunk_lo, (int)desc.size(), (int)chunk_runs.size() - 1});
        chunk_lo = (int)desc.size();
        chunk_runs.emplace_back();
        used_b = 0;
      }
      helm_page d = p;
      d.k = add_region(p.k, rb);  // chunk offsets, rebased below
      d.v = add_region(p.v, rb);
      desc.push_back(d);
    }
    launches.push_back(
        {chunk_lo, (int)desc.size(), (int)chunk_runs.size() - 1});
    off[1] = (int)desc.size();
    chunk_slot.resize(chunk_runs.size());
    for (size_t c = 0; c < chunk_runs.size(); ++c) {
      chunk_slot[c] = eng->next_slot;
      eng->next_slot = (eng->next_slot + 1) % eng->ring_slots;
    }
    for (const Launch& L : launches) {
      if (L.chunk < 0) continue;
      const uint64_t base = reinterpret_cast<uint64_t>(eng->ring) +
                            (uint64_t)chunk_slot[L.chunk] * eng->chunk_bytes;
      for (int i = L.lo; i < L.hi; ++i) {
        desc[i].k += base;
        desc[i].v += base;
        desc[i].flags = 0;
      }
    }
  }

  // ---- token order under causal masking -----------------------------------
  // The chunk kernel ends a workgroup's page walk at the first block past its
  // last query position, so a causal call must list each sequence's pages of
  // a launch in token order.  Staged pages follow host addresses and pages
  // read in place go first: each launch's range (each sequence's, without
  // staging) is sorted back by token offset.  The copy runs were planned from
  // the addresses and do not move.
  if (causal > 0) {
    auto by_tok = [](const helm_page& a, const helm_page& b) { return a.tok_off < b.tok_off; };
    if (as_given) {
      bool sorted = true;
      for (int b = 0; b < B && sorted; ++b)
        for (int i = seq_off[b] + 1; i < seq_off[b + 1] && sorted; ++i)
          sorted = pages[i - 1].tok_off <= pages[i].tok_off;
      if (!sorted) {
        desc.assign(pages, pages + n_all);
        as_given = false;
      }
    }
    if (!as_given && !n_host) {
      for (int b = 0; b < B; ++b)
        std::stable_sort(desc.begin() + off[b], desc.begin() + off[b + 1], by_tok);
    } else if (n_host) {
      for (const Launch& L : launches)
        std::stable_sort(desc.begin() + L.lo, desc.begin() + L.hi, by_tok);
    }
  }

  // ---- kernel choice on the final addresses ---------------------------------
  bool al = aligned(q, 16) && aligned(out, 16) && (D * qb) % 16 == 0;
  const helm_page* dsrc = as_given ? pages : desc.data();
  const size_t n_desc = as_given ? (size_t)n_all : desc.size();
  for (size_t i = 0; i < n_desc; ++i) {
    const helm_page& p = dsrc[i];
    al = al && (p.k % 16 == 0) && (p.v % 16 == 0) &&
         ((int64_t)p.head_stride * eb) % 16 == 0;
  }
  Plan pl{};
  int rc = make_plan(pl, kv_dtype, q_dtype, B, Hq, Hkv, q_len, D, max_tok,
                     std::max(max_pages, 1), (double)n_all / B, 0, al);
  if (rc != HELM_OK) return rc;
  if (n_host) {
    // every launch owns whole splits; keep the call within the split limit
    std::vector<std::pair<int, int>> ranges;
    for (const Launch& L : launches) ranges.push_back({L.lo, L.hi});
    while (chained_splits(ranges, pl.pps) > max_splits_of(pl)) {
      if (pl.pps >= max_pps_of(pl))
        return fail(HELM_E_UNSUPPORTED, "too many staged chunks for one call");
      pl.pps = std::min(max_pps_of(pl), pl.pps * 2);
    }
    if ((int)launches.size() > max_splits_of(pl))
      return fail(HELM_E_UNSUPPORTED, "too many staged chunks for one call");
  }
  int total_splits = 0;
  std::vector<int> split_base;
  for (const Launch& L : launches) {
    split_base.push_back(total_splits);
    total_splits += (L.hi - L.lo + pl.pps - 1) / pl.pps;
  }
  pl.max_splits = n_host ? std::max(1, total_splits)
                         : std::max(1, (max_pages + pl.pps - 1) / pl.pps);
  pl.fused = fused_merge(pl.max_splits);
  size_plan(pl, B, Hkv, D);
  settle_fused(pl, B, Hkv);
  rc = engine_ensure_ws(eng, pl.total(), st);
  if (rc != HELM_OK) return rc;

  // ---- bounded run-ahead of side-stream calls (before any HIP copy call) ----
  const bool side = n_host > 0 && stage_on_side_stream();
  if (side) {
    const int ahead = side_calls_ahead();
    if (ahead > 0 && eng->side_calls >= ahead)
      HELM_HIP(hipEventSynchronize(
          eng->side_done[(eng->side_calls - ahead) % helm_engine::kSideRing]));
  }

  // ---- upload descriptors + sequence offsets --------------------------------
  const size_t dbytes = n_desc * sizeof(helm_page);
  const size_t blob_bytes = align_up(dbytes, 16) + (B + 1) * sizeof(int32_t);
  char* host_blob = nullptr;
  char* dev_blob = nullptr;
  rc = engine_upload_reserve(eng, blob_bytes, &host_blob, &dev_blob);
  if (rc != HELM_OK) return rc;
  if (dbytes) std::memcpy(host_blob, dsrc, dbytes);
  std::memcpy(host_blob + align_up(dbytes, 16), off.data(),
              (B + 1) * sizeof(int32_t));
  rc = engine_upload_commit(eng, blob_bytes, st);
  if (rc != HELM_OK) return rc;

  LaunchSpec s{};
  fill_params(s.p, pl, q, out, B, Hq, Hkv, q_len, D, scale, softcap, mask,
              mask_bstride, mask_hstride, mask_qstride, mask_dtype, causal, eng->ws);
  s.p.full_d = (al && D == 16 * pl.epl) ? 1 : 0;
  s.mode = 1;
  s.desc.pages = reinterpret_cast<const helm_page*>(dev_blob);
  s.desc.seq_off =
      reinterpret_cast<const int32_t*>(dev_blob + align_up(dbytes, 16));
  s.desc.elem_bytes = eb;
  s.kv_dtype = kv_dtype;
  s.q_dtype = q_dtype;
  s.epl = pl.epl;
  s.gm = pl.gm;
  s.fast = pl.fast;
  s.mfma = pl.mfma;
  s.nw = pl.nw;
  s.feat = (mask ? kFeatMask : 0) | (mask && mask_dtype != HELM_F32 ? kFeatMask16 : 0) |
           (softcap > 0.f ? kFeatCap : 0) |
           (causal ? kFeatCausal : 0);

  if (!n_host) {
    s.grid = dim3(std::max(1, pl.max_splits), Hkv * pl.qblocks(), B);
    hipError_t e = dispatch(s, st);
    if (e != hipSuccess) return hip_fail(e, "stream_attn launch");
    e = launch_merge(s, B, Hkv, st);
    if (e != hipSuccess) return hip_fail(e, "merge launch");
    return engine_mark_upload_consumed(eng, st);
  }

  // ---- mixed residency (B == 1) ---------------------------------------------
  // With HELM_AMD_STAGE_STREAM=side, staged chunks are copied on the engine's
  // side stream while the caller's stream runs the device pages' launch and
  // then, chunk by chunk, the launch that reads each one: chunk c's launch
  // waits for chunk c's copies only, so the host link stays busy while the
  // kernels run.  Once this engine has evicted pages (helm_evict_pages), the
  // side stream waits only for what its copies depend on: the last eviction
  // (the copies that wrote host pages) and, per ring slot, the launch that
  // last read it (in this call or an earlier one), so a call's copies may
  // start while the earlier calls' kernels still run; host pages written by
  // other means must then be complete when the call is made.  Before the
  // first eviction, or when a slot was last read by a launch of the default
  // mode (which records no event), the side stream first waits for
  // everything queued on the caller's stream before this call.  Events carry
  // no timestamps.  Without the side stream (the default) every copy is
  // queued on the caller's stream in launch order.
  const int n_chunks = (int)chunk_runs.size();
  auto issue_copies = [&](int c) -> int {
    const int slot = chunk_slot[c];
    char* dst = eng->ring + (size_t)slot * eng->chunk_bytes;
    hipStream_t cs = side ? eng->copy : st;
    if (side && eng->slot_reader[slot] == 1)
      HELM_HIP(hipStreamWaitEvent(eng->copy, eng->slot_free[slot], 0));
    for (const Run& r : chunk_runs[c])
      HELM_HIP(hipMemcpyAsync(dst + r.dst_off, reinterpret_cast<const void*>(r.src), r.bytes,
                              hipMemcpyHostToDevice, cs));
    if (side) HELM_HIP(hipEventRecord(eng->slot_ready[slot], eng->copy));
    return HELM_OK;
  };
  int issued = 0;
  if (side) {
    bool join_all = !eng->evict_recorded;
    for (int c = 0; c < n_chunks && c < eng->ring_slots; ++c)
      join_all = join_all || eng->slot_reader[chunk_slot[c]] == 2;
    if (join_all) {
      HELM_HIP(hipEventRecord(eng->ev_a, st));
      HELM_HIP(hipStreamWaitEvent(eng->copy, eng->ev_a, 0));
      for (int c = 0; c < n_chunks && c < eng->ring_slots; ++c)
        eng->slot_reader[chunk_slot[c]] = 0;
    }
    if (eng->evict_recorded) HELM_HIP(hipStreamWaitEvent(eng->copy, eng->evict_done, 0));
    for (; issued < n_chunks && issued < eng->ring_slots; ++issued) {
      rc = issue_copies(issued);
      if (rc != HELM_OK) return rc;
    }
  }
  s.p.total_splits = total_splits;
  for (size_t li = 0; li < launches.size(); ++li) {
    const Launch& L = launches[li];
    s.p.lo = L.lo;
    s.p.hi = L.hi;
    s.p.split_base = split_base[li];
    const int nsp = (L.hi - L.lo + pl.pps - 1) / pl.pps;
    s.grid = dim3(std::max(1, nsp), Hkv * pl.qblocks(), 1);
    const int slot = L.chunk >= 0 ? chunk_slot[L.chunk] : -1;
    if (L.chunk >= 0) {
      if (side) {
        HELM_HIP(hipStreamWaitEvent(st, eng->slot_ready[slot], 0));
      } else {
        rc = issue_copies(L.chunk);
        if (rc != HELM_OK) return rc;
      }
    }
    hipError_t e = dispatch(s, st);
    if (e != hipSuccess) return hip_fail(e, "stream_attn chunk launch");
    if (L.chunk >= 0) {
      if (side) HELM_HIP(hipEventRecord(eng->slot_free[slot], st));
      eng->slot_reader[slot] = side ? 1 : 2;
    }
    if (side && L.chunk >= 0 && issued < n_chunks) {
      // the next chunk for this slot (chunks take the slots in turn)
      rc = issue_copies(issued++);
      if (rc != HELM_OK) return rc;
    }
  }
  hipError_t e = launch_merge(s, 1, Hkv, st);
  if (e != hipSuccess) return hip_fail(e, "merge launch");
  if (side) {
    HELM_HIP(hipEventRecord(eng->side_done[eng->side_calls % helm_engine::kSideRing], st));
    ++eng->side_calls;
  }
  return engine_mark_upload_consumed(eng, st);
}

// helm_paged_attn_seqs, and with `app` (one new token per sequence) the
// decode call that also writes those tokens (helm_paged_attn_seqs_append).
static int paged_attn_seqs(helm_engine* eng, const void* q, void* out, int B, int Hq, int Hkv,
                    int q_len, int D, const uint64_t* seq_pages, const int32_t* seq_npages,
                    const int32_t* seq_tokens, int page_tokens, int aligned16, float scale,
                    float softcap, const void* mask, int64_t mask_bstride,
                    int64_t mask_hstride, int64_t mask_qstride, int mask_dtype, int causal, int kv_dtype,
                    int q_dtype, const helm_append_seg* app, void* stream) {
  if (!eng || !q || !out || !seq_pages || !seq_npages || !seq_tokens)
    return fail(HELM_E_INVALID, "null pointer argument");
  if (B <= 0 || Hkv <= 0 || D <= 0 || page_tokens <= 0)
    return fail(HELM_E_INVALID, "bad shape");
  if (causal < 0) return fail(HELM_E_INVALID, "causal must be >= 0");
  if (!mask_dtype_ok(mask, mask_dtype)) return fail(HELM_E_INVALID, "unknown mask dtype");
  if (B > kSeqArgs)
    return fail(HELM_E_UNSUPPORTED,
                "more than " + std::to_string(kSeqArgs) + " sequences per call");
  const int eb = elem_bytes(kv_dtype);
  const int qb = elem_bytes(q_dtype);
  if (!eb || !qb) return fail(HELM_E_INVALID, "unknown dtype");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  int max_pages = 0;
  int64_t all_pages = 0;
  for (int b = 0; b < B; ++b) {
    if (seq_npages[b] < 0 || seq_tokens[b] < 0 ||
        (int64_t)seq_tokens[b] > (int64_t)seq_npages[b] * page_tokens ||
        (seq_npages[b] > 0 && !seq_pages[b]))
      return fail(HELM_E_INVALID, "bad sequence " + std::to_string(b));
    max_pages = std::max(max_pages, seq_npages[b]);
    all_pages += seq_npages[b];
  }
  const bool al = aligned16 && aligned(q, 16) && aligned(out, 16) &&
                  (D * qb) % 16 == 0;
  Plan pl{};
  int rc = make_plan(pl, kv_dtype, q_dtype, B, Hq, Hkv, q_len, D, page_tokens,
                     std::max(max_pages, 1), (double)all_pages / B, 0, al);
  if (rc != HELM_OK) return rc;
  if (app) {
    // the token writes run inside the matrix-core decode kernel only
    if (!(pl.mfma && !pl.row_waves && q_len == 1 && D == 128 && eb == 2))
      return fail(HELM_E_UNSUPPORTED, "token writes need the matrix-core decode kernel");
    for (int b = 0; b < B; ++b) {
      const helm_append_seg& a = app[b];
      if (a.n_tok != 1 || seq_npages[b] < 1 || seq_tokens[b] < 1 || !a.src_k || !a.src_v)
        return fail(HELM_E_INVALID, "bad token write for sequence " + std::to_string(b));
      if ((a.src_k | a.src_v) % 16 != 0 || (a.src_head_stride * eb) % 16 != 0)
        return fail(HELM_E_UNSUPPORTED, "token source of sequence " + std::to_string(b) +
                                            " is not 16-byte aligned");
    }
  }
  // a batch on the decode kernel whose sequences all hold pages: the grid
  // numbers exactly their splits (no workgroups of a short sequence that find
  // no split), with the split length chosen from every sequence's page count
  bool compact = pl.mfma && !pl.row_waves && B > 1 && env_int("HELM_AMD_COMPACT", 1);
  for (int b = 0; b < B && compact; ++b) compact = seq_npages[b] > 0;
  if (compact && env_int("HELM_AMD_PPS", 0) <= 0) {
    const int cand = batch_pps(seq_npages, B, Hkv * pl.qblocks(), device_cus(),
                               min_pps(pl.bpp, pl.nw), max_pps_of(pl));
    if ((max_pages + cand - 1) / cand <= max_splits_of(pl)) pl.pps = cand;
  }
  pl.max_splits = std::max(1, (max_pages + pl.pps - 1) / pl.pps);
  pl.fused = fused_merge(pl.max_splits);
  size_plan(pl, B, Hkv, D);
  settle_fused(pl, B, Hkv);
  rc = engine_ensure_ws(eng, pl.total(), st);
  if (rc != HELM_OK) return rc;

  LaunchSpec s{};
  fill_params(s.p, pl, q, out, B, Hq, Hkv, q_len, D, scale, softcap, mask,
              mask_bstride, mask_hstride, mask_qstride, mask_dtype, causal, eng->ws);
  enable_claims(s.p, pl, B, Hkv, eng->ws);
  s.p.full_d = (al && D == 16 * pl.epl) ? 1 : 0;
  s.mode = 1;
  s.desc.elem_bytes = eb;
  s.desc.by_value = 1;
  int all_splits = 0;
  for (int b = 0; b < B; ++b) {
    s.desc.seq_pages[b] = reinterpret_cast<const helm_page*>(seq_pages[b]);
    s.desc.seq_n[b] = seq_npages[b];
    s.desc.seq_tokens[b] = seq_tokens[b];
    s.desc.seq_split0[b] = all_splits;
    all_splits += (seq_npages[b] + pl.pps - 1) / pl.pps;
  }
  if (compact) {
    s.desc.compact = 1;
    s.desc.n_seq = B;
  }
  if (app) {
    s.desc.app_n = B;
    for (int b = 0; b < B; ++b) {
      s.desc.app_k[b] = reinterpret_cast<const char*>(app[b].src_k);
      s.desc.app_v[b] = reinterpret_cast<const char*>(app[b].src_v);
      s.desc.app_hs[b] = app[b].src_head_stride;
    }
  }
  s.kv_dtype = kv_dtype;
  s.q_dtype = q_dtype;
  s.epl = pl.epl;
  s.gm = pl.gm;
  s.fast = pl.fast;
  s.mfma = pl.mfma;
  s.nw = pl.nw;
  s.feat = (mask ? kFeatMask : 0) | (mask && mask_dtype != HELM_F32 ? kFeatMask16 : 0) |
           (softcap > 0.f ? kFeatCap : 0) |
           (causal ? kFeatCausal : 0);
  s.grid = compact ? dim3(all_splits, Hkv * pl.qblocks(), 1)
                  : dim3(std::max(1, pl.max_splits), Hkv * pl.qblocks(), B);
  hipError_t e = dispatch_timed(s, st);
  if (e != hipSuccess) return hip_fail(e, "paged_attn_seqs launch");
  e = launch_merge(s, B, Hkv, st);
  if (e != hipSuccess) return hip_fail(e, "merge launch");
  return HELM_OK;
}

int helm_paged_attn_seqs(helm_engine* eng, const void* q, void* out, int B,
                         int Hq, int Hkv, int q_len, int D,
                         const uint64_t* seq_pages, const int32_t* seq_npages,
                         const int32_t* seq_tokens, int page_tokens,
                         int aligned16, float scale, float softcap,
                         const void* mask, int64_t mask_bstride,
                         int64_t mask_hstride, int64_t mask_qstride, int mask_dtype, int causal,
                         int kv_dtype, int q_dtype, void* stream) {
  EnvScope env_scope;
  return paged_attn_seqs(eng, q, out, B, Hq, Hkv, q_len, D, seq_pages, seq_npages, seq_tokens,
                         page_tokens, aligned16, scale, softcap, mask, mask_bstride,
                         mask_hstride, mask_qstride, mask_dtype, causal, kv_dtype, q_dtype, nullptr,
                         stream);
}

int helm_paged_attn_seqs_append(helm_engine* eng, const void* q, void* out, int B,
                                int Hq, int Hkv, int D, const uint64_t* seq_pages,
                                const int32_t* seq_npages, const int32_t* seq_tokens,
                                int page_tokens, int aligned16, float scale, float softcap,
                                const void* mask, int64_t mask_bstride,
                                int64_t mask_hstride, int64_t mask_qstride, int mask_dtype, int kv_dtype,
                                const helm_append_seg* tokens, void* stream) {
  EnvScope env_scope;
  if (!tokens) return fail(HELM_E_INVALID, "null pointer argument");
  return paged_attn_seqs(eng, q, out, B, Hq, Hkv, 1, D, seq_pages, seq_npages, seq_tokens,
                         page_tokens, aligned16, scale, softcap, mask, mask_bstride,
                         mask_hstride, mask_qstride, mask_dtype, 0, kv_dtype, kv_dtype, tokens, stream);
}

static_assert(sizeof(helm_decode_args) == 744, "helm_decode_args layout (helm_amd/_native.py)");

int helm_decode_step(helm_engine* eng, const helm_decode_args* a) {
  EnvScope env_scope;
  if (!a) return fail(HELM_E_INVALID, "null pointer argument");
  if (a->B <= 0 || a->B > HELM_DECODE_MAX_SEQS)
    return fail(HELM_E_UNSUPPORTED, "B must be in [1, " +
                                        std::to_string(HELM_DECODE_MAX_SEQS) + "]");
  const void* mask = reinterpret_cast<const void*>(a->mask);
  void* st = reinterpret_cast<void*>(a->stream);
  if (!a->append)
    return paged_attn_seqs(eng, reinterpret_cast<const void*>(a->q),
                           reinterpret_cast<void*>(a->out), a->B, a->Hq, a->Hkv, 1, a->D,
                           a->seq_pages, a->seq_npages, a->seq_tokens, a->page_tokens,
                           a->aligned16, a->scale, a->softcap, mask, a->mask_bstride,
                           a->mask_hstride, a->mask_qstride, a->mask_dtype, 0, a->kv_dtype,
                           a->kv_dtype, nullptr, st);
  helm_append_seg app[HELM_DECODE_MAX_SEQS];
  for (int b = 0; b < a->B; ++b) {
    app[b] = helm_append_seg{};
    app[b].src_k = a->tok_k[b];
    app[b].src_v = a->tok_v[b];
    app[b].src_head_stride = a->tok_head_stride[b];
    app[b].n_tok = 1;
  }
  return helm_paged_attn_seqs_append(
      eng, reinterpret_cast<const void*>(a->q), reinterpret_cast<void*>(a->out), a->B, a->Hq,
      a->Hkv, a->D, a->seq_pages, a->seq_npages, a->seq_tokens, a->page_tokens, a->aligned16,
      a->scale, a->softcap, mask, a->mask_bstride, a->mask_hstride, a->mask_qstride,
      a->mask_dtype, a->kv_dtype, app, st);
}

int helm_upload(helm_engine* eng, void* dst, const void* src, size_t bytes,
                void* stream) {
  if (!eng || (bytes && (!dst || !src)))
    return fail(HELM_E_INVALID, "null pointer argument");
  if (!bytes) return HELM_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* host = nullptr;
  char* dev = nullptr;
  int rc = engine_upload_reserve(eng, bytes, &host, &dev);
  if (rc != HELM_OK) return rc;
  std::memcpy(host, src, bytes);
  const int i = eng->up_next;
  eng->up_next = (i + 1) % helm_engine::kUp;
  HELM_HIP(hipMemcpyAsync(dst, host, bytes, hipMemcpyHostToDevice, st));
  HELM_HIP(hipEventRecord(eng->up_done[i], st));
  eng->up_used[i] = 1;
  return HELM_OK;
}

int helm_host_pages_in_place(helm_engine* eng, const helm_page* pages, int n,
                             int Hkv, int D, int kv_dtype, uint8_t* in_place) {
  EnvScope env_scope;
  if (!eng || (n > 0 && (!pages || !in_place)))
    return fail(HELM_E_INVALID, "null pointer argument");
  if (n < 0 || Hkv <= 0 || D <= 0) return fail(HELM_E_INVALID, "bad shape");
  const int eb = elem_bytes(kv_dtype);
  if (!eb) return fail(HELM_E_INVALID, "unknown dtype");
  for (int i = 0; i < n; ++i)
    if (pages[i].used <= 0 || !pages[i].k || !pages[i].v ||
        pages[i].head_stride < pages[i].used * D)
      return fail(HELM_E_INVALID, "bad page descriptor " + std::to_string(i));
  std::vector<char> direct;
  resolve_host_pages(eng, pages, n, Hkv, D, eb, direct);
  for (int i = 0; i < n; ++i) in_place[i] = direct[i] ? 1 : 0;
  return HELM_OK;
}

int helm_page_append(const helm_append_seg* segs, int n_segs, int Hkv, int D,
                     int dtype, void* stream) {
  const int eb = elem_bytes(dtype);
  if (!eb) return fail(HELM_E_INVALID, "unknown dtype");
  if (n_segs < 0 || Hkv <= 0 || D <= 0)
    return fail(HELM_E_INVALID, "bad append shape");
  if (n_segs == 0) return HELM_OK;
  if (!segs) return fail(HELM_E_INVALID, "null segments");
  for (int i = 0; i < n_segs; ++i) {
    const helm_append_seg& s = segs[i];
    if (!s.dst_k || !s.dst_v || !s.src_k || !s.src_v || s.n_tok < 0 ||
        s.dst_tok < 0 || s.dst_head_stride < (s.dst_tok + s.n_tok) * D)
      return fail(HELM_E_INVALID, "bad append segment " + std::to_string(i));
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  for (int base = 0; base < n_segs; base += kAppendSegsPerLaunch) {
    AppendArgs a{};
    a.n_seg = std::min(kAppendSegsPerLaunch, n_segs - base);
    a.D = D;
    a.eb = eb;
    for (int i = 0; i < a.n_seg; ++i) a.seg[i] = segs[base + i];
    hipLaunchKernelGGL(page_append_kernel, dim3(a.n_seg, Hkv), dim3(256), 0,
                       st, a);
    HELM_HIP(hipGetLastError());
  }
  return HELM_OK;
}

int helm_decode_front(const void* q_proj, const void* k_proj, const void* v_proj,
                      int64_t q_stride, int64_t kv_stride, const void* q_norm_w,
                      const void* k_norm_w, int norm_mode, float eps, const void* cos,
                      const void* sin, int64_t cs_stride, int cs_dtype, void* q_out,
                      const helm_append_seg* dst, int B, int Hq, int Hkv, int D, int dtype,
                      void* stream) {
  const int eb = elem_bytes(dtype);
  if (!eb) return fail(HELM_E_INVALID, "unknown dtype");
  if (cs_dtype != dtype && cs_dtype != HELM_F32)
    return fail(HELM_E_UNSUPPORTED, "cos / sin must have the projection dtype or float32");
  if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || D < 2 || D % 2 != 0 || D > kFrontMaxD)
    return fail(HELM_E_INVALID, "bad decode front shape (D even, at most 256)");
  if (norm_mode < 0 || norm_mode > 2) return fail(HELM_E_INVALID, "norm_mode must be 0, 1 or 2");
  if (B == 0) return HELM_OK;
  if (!q_proj || !k_proj || !v_proj || !cos || !sin || !q_out || !dst ||
      (norm_mode && (!q_norm_w || !k_norm_w)))
    return fail(HELM_E_INVALID, "null pointer argument");
  if (q_stride < (int64_t)Hq * D || kv_stride < (int64_t)Hkv * D || cs_stride < 0)
    return fail(HELM_E_INVALID, "projection rows overlap");
  for (int b = 0; b < B; ++b)
    if (!dst[b].dst_k || !dst[b].dst_v || dst[b].dst_tok < 0 ||
        dst[b].dst_head_stride < (dst[b].dst_tok + 1) * D)
      return fail(HELM_E_INVALID, "bad destination " + std::to_string(b));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  for (int b0 = 0; b0 < B; b0 += kFrontMaxSeqs) {
    FrontArgs a{};
    const int nb = std::min(kFrontMaxSeqs, B - b0);
    a.q = static_cast<const char*>(q_proj);
    a.k = static_cast<const char*>(k_proj);
    a.v = static_cast<const char*>(v_proj);
    a.q_stride = q_stride;
    a.kv_stride = kv_stride;
    a.qw = static_cast<const char*>(q_norm_w);
    a.kw = static_cast<const char*>(k_norm_w);
    a.eps = eps;
    a.norm = norm_mode;
    a.cos = static_cast<const char*>(cos);
    a.sin = static_cast<const char*>(sin);
    a.cs_stride = cs_stride;
    a.q_out = static_cast<char*>(q_out);
    a.b0 = b0;
    a.Hq = Hq;
    a.Hkv = Hkv;
    a.D = D;
    for (int i = 0; i < nb; ++i) {
      a.dst_k[i] = dst[b0 + i].dst_k;
      a.dst_v[i] = dst[b0 + i].dst_v;
      a.dst_head_stride[i] = dst[b0 + i].dst_head_stride;
      a.dst_tok[i] = dst[b0 + i].dst_tok;
    }
    const dim3 grid(nb, Hq + Hkv);
    const bool c32 = cs_dtype == HELM_F32;
    switch (dtype) {
      case HELM_BF16:
        if (c32) hipLaunchKernelGGL((decode_front_kernel<bf16_t, float>), grid, dim3(64), 0, st, a);
        else hipLaunchKernelGGL((decode_front_kernel<bf16_t, bf16_t>), grid, dim3(64), 0, st, a);
        break;
      case HELM_F16:
        if (c32) hipLaunchKernelGGL((decode_front_kernel<f16_t, float>), grid, dim3(64), 0, st, a);
        else hipLaunchKernelGGL((decode_front_kernel<f16_t, f16_t>), grid, dim3(64), 0, st, a);
        break;
      default:
        hipLaunchKernelGGL((decode_front_kernel<float, float>), grid, dim3(64), 0, st, a);
        break;
    }
    HELM_HIP(hipGetLastError());
  }
  return HELM_OK;
}

int helm_evict_pages(helm_engine* eng, int n, const uint64_t* src_dev,
                     const uint64_t* dst_host, const uint64_t* bytes, int sync,
                     void* stream) {
  if (!eng) return fail(HELM_E_INVALID, "null engine");
  if (n > 0 && (!src_dev || !dst_host || !bytes))
    return fail(HELM_E_INVALID, "null region arrays");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (n > 0 && eng->evict_recorded && st != eng->evict_stream)
    HELM_HIP(hipStreamWaitEvent(st, eng->evict_done, 0));
  int rc = engine_copies(eng, n, src_dev, dst_host, bytes, hipMemcpyDeviceToHost, sync, st);
  if (rc != HELM_OK || n <= 0) return rc;
  // side-stream staging copies wait for this event, not for the whole stream
  HELM_HIP(hipEventRecord(eng->evict_done, st));
  eng->evict_stream = st;
  eng->evict_recorded = true;
  return HELM_OK;
}

int helm_prefetch_pages(helm_engine* eng, int n, const uint64_t* src_host,
                        const uint64_t* dst_dev, const uint64_t* bytes,
                        int sync, void* stream) {
  if (!eng) return fail(HELM_E_INVALID, "null engine");
  if (n > 0 && (!src_host || !dst_dev || !bytes))
    return fail(HELM_E_INVALID, "null region arrays");
  return engine_copies(eng, n, src_host, dst_dev, bytes,
                       hipMemcpyHostToDevice, sync,
                       reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
