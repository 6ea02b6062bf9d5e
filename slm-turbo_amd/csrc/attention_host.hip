// Host side of the attention kernels: launch geometry, workspace layout and
// dispatch.  Nothing here allocates device memory.
#include "attention_kernel.h"

namespace slmt {

namespace {

// KV heads a group of hpg query heads can touch, over all group alignments.
int worst_nkv(int hpg, int G) { return (hpg + G - 1) / G + 1; }

struct WsLayout {
  int64_t part_o, part_ml, counters, total;
};

// Arrival counters live in a fixed region at the start of every workspace, so
// calls of any shape that share a workspace never overwrite each other's
// counters with partial results (each call leaves its counters at zero).
constexpr int64_t kCounterCap = int64_t(1) << 20;

WsLayout ws_layout(const AttnPlan& pl, int B, int H, int D) {
  auto al = [](int64_t x) { return (x + 255) & ~255LL; };
  WsLayout w;
  w.counters = 0;
  w.part_o = kCounterCap * 4;
  w.part_ml = w.part_o + al((int64_t)pl.W * 2 * H * D * 4);
  w.total = w.part_ml + al((int64_t)pl.W * 2 * H * 2 * 4);
  (void)B;
  return w;
}

}  // namespace

int plan_attention(int B, int H, int G, int D, AttnPlan* plan) {
  (void)B;
  const size_t kBudget = 64 * 1024;   // leaves room for two workgroups per CU
  int hpg = ((H + 3) / 4) * 4;
  if (hpg > 4 * (attn::MAX_THREADS / 64)) hpg = 4 * (attn::MAX_THREADS / 64);
  while (hpg > 4 && attn::lds_bytes_for(worst_nkv(hpg, G), D, hpg / 4) > kBudget) hpg -= 4;
  const int waves = hpg / 4;
  const size_t lds = attn::lds_bytes_for(worst_nkv(hpg, G), D, waves);
  if (lds > 160 * 1024) return fail(SLMT_ERR_UNSUPPORTED, "attention: KV row too wide for LDS");
  const int groups = (H + hpg - 1) / hpg;
  const int cus = device_cu_count();
  if (cus <= 0) return fail(SLMT_ERR_HIP, "attention: could not query the device");
  int per_cu = 8 / waves;                           // up to 256 VGPRs per lane -> 8 waves per CU
  const int by_lds = (int)((160 * 1024) / lds);
  per_cu = per_cu < by_lds ? per_cu : by_lds;
  if (per_cu < 1) per_cu = 1;
  int W = cus * per_cu / groups;
  if (W < 1) W = 1;
  plan->heads_per_group = hpg;
  plan->groups = groups;
  plan->waves = waves;
  plan->W = W;
  plan->lds_bytes = lds;
  return SLMT_OK;
}

int64_t attention_workspace_bytes(int B, int H, int KV, int D) {
  if (B < 0 || H <= 0 || KV <= 0 || H % KV != 0) {
    fail(SLMT_ERR_INVALID, "workspace: invalid sizes");
    return -1;
  }
  AttnPlan pl;
  if (plan_attention(B, H, H / KV, D, &pl) != SLMT_OK) return -1;
  if ((int64_t)pl.groups * B > kCounterCap) {
    fail(SLMT_ERR_UNSUPPORTED, "attention: more than 2^20 (sequence, head group) pairs in one call");
    return -1;
  }
  return ws_layout(pl, B, H, D).total;
}

int launch_attention(int mode, int D, AttnParams& p, void* workspace, int64_t ws_bytes, hipStream_t stream) {
  AttnPlan pl;
  int rc = plan_attention(p.B, p.H, p.G, D, &pl);
  if (rc != SLMT_OK) return rc;
  if ((int64_t)pl.groups * p.B > kCounterCap)
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
  if (p.min_tiles <= 0) p.min_tiles = 4;
  const dim3 grid(pl.W, pl.groups), block(pl.waves * 64);
  if (mode == SRC_PAGED) {
    const bool shared = (p.G % 4) == 0;   // every wave's 4 heads share one KV head
    // contiguous tiles: 16 | block_size and one group covering the whole cache row
    const bool fast = p.block_shift >= 4 && pl.groups == 1 && ((int64_t)p.cache_kv * (D + 8)) % 8 == 0;
    return launch_attention_paged(D, shared, fast, p, grid, block, pl.lds_bytes, stream);
  }
  return launch_attention_contig(mode, D, p, grid, block, pl.lds_bytes, stream);
}

}  // namespace slmt
