// Host side of the attention kernels: launch geometry, workspace layout and
// dispatch.  Nothing here allocates device memory.
#include "attention_kernel.h"

#include <algorithm>
#include <mutex>
#include <utility>
#include <vector>

namespace slmt {

// ---------------------------------------------------------------------------
// Kernel timing hook (slmt_kernel_timing): a pool of event pairs created when
// recording is switched on, so a recording call itself creates nothing.
// ---------------------------------------------------------------------------
namespace {
constexpr int kTimingSlots = 4096;
struct KernelTiming {
  std::mutex mu;
  bool on = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pool;
  int used = 0;
  const char* last = "";   // kernel of the most recent timed call
};
KernelTiming& kernel_timing() {
  static KernelTiming t;
  return t;
}
}  // namespace

bool kernel_timing_events(hipEvent_t* start, hipEvent_t* stop, const char* kernel) {
  KernelTiming& t = kernel_timing();
  std::lock_guard<std::mutex> lock(t.mu);
  if (!t.on || t.used >= (int)t.pool.size()) return false;
  *start = t.pool[t.used].first;
  *stop = t.pool[t.used].second;
  ++t.used;
  t.last = kernel;
  return true;
}

const char* kernel_timing_kernel() {
  KernelTiming& t = kernel_timing();
  std::lock_guard<std::mutex> lock(t.mu);
  return t.last;
}

int set_kernel_timing(bool enable) {
  KernelTiming& t = kernel_timing();
  std::lock_guard<std::mutex> lock(t.mu);
  if (enable && t.pool.empty()) {
    t.pool.reserve(kTimingSlots);
    for (int i = 0; i < kTimingSlots; ++i) {
      hipEvent_t a, b;
      if (hipEventCreate(&a) != hipSuccess) return fail(SLMT_ERR_HIP, "timing: hipEventCreate failed");
      if (hipEventCreate(&b) != hipSuccess) {
        (void)hipEventDestroy(a);
        return fail(SLMT_ERR_HIP, "timing: hipEventCreate failed");
      }
      t.pool.emplace_back(a, b);
    }
  }
  t.on = enable;
  return SLMT_OK;
}

int read_kernel_timing(float* us, int max_n) {
  KernelTiming& t = kernel_timing();
  std::lock_guard<std::mutex> lock(t.mu);
  const int n = std::min(t.used, std::max(max_n, 0));
  for (int i = 0; i < n; ++i) {
    float ms = 0.f;
    if (hipEventSynchronize(t.pool[i].second) != hipSuccess ||
        hipEventElapsedTime(&ms, t.pool[i].first, t.pool[i].second) != hipSuccess) {
      t.used = 0;
      fail(SLMT_ERR_HIP, "timing: reading the decode kernel events failed");
      return -1;
    }
    us[i] = ms * 1000.f;
  }
  t.used = 0;
  return n;
}

namespace {

// KV heads a group of hpg query heads can touch, over all group alignments.
int worst_nkv(int hpg, int G) { return (hpg + G - 1) / G + 1; }

struct WsLayout {
  int64_t part_o, part_ml, counters, total;
};

constexpr int64_t kCounterCap = kWsCounterInts;

// Zero n ints with plain vector stores (a kernel node, not a memset node, so
// the call stays capturable in a HIP graph).
__global__ void __launch_bounds__(256) zero_ints(int* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0;
}

WsLayout ws_layout(const AttnPlan& pl, int B, int H, int D) {
  auto al = [](int64_t x) { return (x + 255) & ~255LL; };
  WsLayout w;
  w.counters = 0;
  w.part_o = kCounterCap * 4;
  w.part_ml = w.part_o + al((int64_t)pl.W_ws * 2 * H * D * 4);
  w.total = w.part_ml + al((int64_t)pl.W_ws * 2 * H * 2 * 4);
  (void)B;
  return w;
}

}  // namespace

// Query heads per workgroup of a plan: all of them, at most 8 waves of 4.
static int hpg_max(int H) {
  const int h = ((H + 3) / 4) * 4;
  return h < 4 * (attn::MAX_THREADS / 64) ? h : 4 * (attn::MAX_THREADS / 64);
}

int plan_attention(int B, int H, int G, int D, int dma_kv, AttnPlan* plan) {
  (void)B;
  const int cus = device_cu_count();
  if (cus <= 0) return fail(SLMT_ERR_HIP, "attention: could not query the device");
  // Register-staged plan: up to 32 heads (8 waves) per group, LDS kept small
  // enough for two workgroups per CU when the waves allow it.
  const size_t kBudget = 64 * 1024;
  int hpg = hpg_max(H);
  while (hpg > 4 && (size_t)attn::lds_geom(worst_nkv(hpg, G), D, hpg / 4).total > kBudget) hpg -= 4;
  int waves = hpg / 4;
  size_t lds = attn::lds_geom(worst_nkv(hpg, G), D, waves).total;
  if (lds > 160 * 1024) return fail(SLMT_ERR_UNSUPPORTED, "attention: KV row too wide for LDS");
  int groups = (H + hpg - 1) / hpg;
  // waves_cap: waves per CU the kernel's registers allow (the register-staged
  // kernel may use up to 256 VGPRs: 2 waves per SIMD; the direct-load kernel
  // stays within 168: 3 per SIMD).  The launch lowers W to the occupancy the
  // runtime reports, so this is an upper bound for the workspace.
  auto workgroups = [&](size_t lds_b, int wv, int grp, int waves_cap) {
    int per_cu = waves_cap / wv;
    const int by_lds = (int)((160 * 1024) / lds_b);
    per_cu = per_cu < by_lds ? per_cu : by_lds;
    if (per_cu < 1) per_cu = 1;
    const int W = cus * per_cu / grp;
    return W < 1 ? 1 : W;
  };
  plan->heads_per_group = hpg;
  plan->groups = groups;
  plan->waves = waves;
  plan->W = workgroups(lds, waves, groups, 8);
  plan->W_ws = plan->W;
  plan->dma = false;
  plan->lds_bytes = lds;
  plan->rows = false;
  plan->rows_nkv = plan->rows_wpk = plan->rows_groups = 0;
  if (dma_kv <= 0) return SLMT_OK;

  // Whole-row kernel first: it covers head_dim 64 and 128 with 4 or 8 query
  // heads per KV head.  The workspace is sized for the larger of its grid and the
  // other plans' (W_ws).
  int nkv, wpk, rgroups;
  if (rows_shape(H, G, D, dma_kv, &nkv, &wpk, &rgroups)) {
    plan->rows = true;
    plan->rows_nkv = nkv;
    plan->rows_wpk = wpk;
    plan->rows_groups = rgroups;
    plan->W_ws = std::max(plan->W_ws, rows_max_workgroups(D, nkv, wpk, rgroups, cus));
  }

  // Direct-load plan: every wave's 4 heads share one KV head (G % 4 == 0) and
  // cache rows are a multiple of 16 bytes (an even number of KV heads), so a
  // wave's widened KV slot stays in its row.
  if (G % 4 != 0 || ((int64_t)dma_kv * (D + 8)) % 16 != 0) return SLMT_OK;
  const int dh = hpg_max(H) < attn::DHEADS ? hpg_max(H) : attn::DHEADS;
  const int dwaves = dh / 4;
  const attn::DmaGeom geo = attn::dma_geom(D, dwaves);
  if (geo.total > 160 * 1024) return SLMT_OK;
  plan->heads_per_group = dh;
  plan->groups = (H + dh - 1) / dh;
  plan->waves = dwaves;
  plan->W = workgroups((size_t)geo.total, dwaves, plan->groups, 12);
  plan->dma = true;
  plan->lds_bytes = (size_t)geo.total;
  if (plan->W > plan->W_ws) plan->W_ws = plan->W;
  if (plan->rows) plan->W_ws = std::max(plan->W_ws, rows_max_workgroups(D, nkv, wpk, rgroups, cus));
  return SLMT_OK;
}

int64_t attention_workspace_bytes(int B, int H, int KV, int D) {
  if (B < 0 || H <= 0 || KV <= 0 || H % KV != 0) {
    fail(SLMT_ERR_INVALID, "workspace: invalid sizes");
    return -1;
  }
  AttnPlan pl;
  if (plan_attention(B, H, H / KV, D, KV, &pl) != SLMT_OK) return -1;
  if ((int64_t)std::max(pl.groups, pl.rows_groups) * B > kCounterCap) {
    fail(SLMT_ERR_UNSUPPORTED, "attention: more than 2^20 (sequence, head group) pairs in one call");
    return -1;
  }
  return ws_layout(pl, B, H, D).total;
}

int launch_attention(int mode, int D, AttnParams& p, void* workspace, int64_t ws_bytes, hipStream_t stream,
                     bool clear_counters) {
  // Direct loads need a power-of-two block of at least 16 tokens (a tile is
  // then one run of consecutive slots) and a 16-byte aligned cache.
  const bool dma_ok = mode == SRC_PAGED && p.block_shift >= 4 && p.num_blocks < (int64_t(1) << 31) &&
                      (reinterpret_cast<uintptr_t>(p.cache) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(p.q) & 15) == 0 && p.q_seq_stride % 8 == 0 &&
                      p.q_head_stride % 8 == 0 && ((int64_t)p.H * p.q_head_stride + D) * 2 < (int64_t(1) << 31);
  AttnPlan pl;
  int rc = plan_attention(p.B, p.H, p.G, D, dma_ok ? p.cache_kv : 0, &pl);
  if (rc != SLMT_OK) return rc;
  const int groups = pl.rows ? std::max(pl.groups, pl.rows_groups) : pl.groups;
  if ((int64_t)groups * p.B > kCounterCap)
    return fail(SLMT_ERR_UNSUPPORTED, "attention: more than 2^20 (sequence, head group) pairs in one call");
  const WsLayout lay = ws_layout(pl, p.B, p.H, D);
  if (workspace == nullptr || ws_bytes < lay.total)
    return fail(SLMT_ERR_INVALID, "attention: workspace of " + std::to_string(lay.total) + " bytes required, got " +
                                      std::to_string(ws_bytes));
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  p.part_o = reinterpret_cast<float*>(ws + lay.part_o);
  p.part_ml = reinterpret_cast<float*>(ws + lay.part_ml);
  p.counters = reinterpret_cast<int*>(ws + lay.counters);
  p.heads_per_group = pl.heads_per_group;
  p.W = pl.W;
  p.nthreads = pl.waves * 64;
  if (p.min_tiles <= 0) p.min_tiles = 4;
  if (mode == SRC_PAGED && pl.rows) {
    p.W = pl.W_ws;   // the kernel lowers it to the workgroups the CUs hold (no counters used)
    if (mfma_rows_enabled(D, pl.rows_nkv, pl.rows_wpk))
      return launch_attention_mfma(D, pl.rows_nkv, pl.rows_wpk, pl.rows_groups, p, stream);
    return launch_attention_rows(D, pl.rows_nkv, pl.rows_wpk, pl.rows_groups, p, stream);
  }
  if (clear_counters) {
    // the last-arriver merges count pieces in counters[group * B + b]
    const int64_t n = (int64_t)pl.groups * p.B;
    const int blocks = (int)std::min<int64_t>((n + 255) / 256, 1024);
    hipLaunchKernelGGL(zero_ints, dim3(blocks), dim3(256), 0, stream, p.counters, n);
    if (int rc = check_launch("attention counters")) return rc;
  }
  const dim3 grid(pl.W, pl.groups), block(pl.waves * 64);
  if (mode == SRC_PAGED) {
    const bool shared = (p.G % 4) == 0;   // every wave's 4 heads share one KV head
    return launch_attention_paged(D, shared, pl.dma, p, grid, block, pl.lds_bytes, stream);
  }
  return launch_attention_contig(mode, D, p, grid, block, pl.lds_bytes, stream);
}

}  // namespace slmt
