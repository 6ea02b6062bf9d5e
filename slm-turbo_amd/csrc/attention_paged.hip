// Instantiations of the attention kernel for the paged per-token cache.
#include "attention_kernel.h"

#include <map>
#include <mutex>
#include <tuple>

namespace slmt {

// Workgroups of `kern` with `threads` threads and `lds` dynamic LDS bytes
// that one CU holds at once (cached per shape; 0 if the runtime cannot say).
static int blocks_per_cu(const void* kern, int threads, size_t lds) {
  static std::mutex mu;
  static std::map<std::tuple<const void*, int, size_t>, int> cache;
  const auto key = std::make_tuple(kern, threads, lds);
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  // the direct-load rings can exceed the default 64 KB dynamic LDS limit
  (void)hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, threads, lds) != hipSuccess) n = 0;
  (void)hipGetLastError();
  cache[key] = n;
  return n;
}

template <int D, bool SHARED, bool DMA>
static void launch_one(AttnParams p, dim3 grid, dim3 block, size_t lds, hipStream_t stream) {
  auto kern = attn::attention_kernel<D, SRC_PAGED, SHARED, DMA>;
  // Every workgroup must be resident at once for the stream-K split to
  // balance: cap W at what the CUs hold (the workspace is sized for more).
  const int per_cu = blocks_per_cu(reinterpret_cast<const void*>(kern), (int)block.x, lds);
  const int cus = device_cu_count();
  if (per_cu > 0 && cus > 0) {
    const int fit = cus * per_cu / (int)grid.y;
    if (fit >= 1 && fit < (int)grid.x) {
      grid.x = fit;
      p.W = fit;
    }
  }
  hipLaunchKernelGGL(kern, grid, block, lds, stream, p);
}

template <int D>
static void launch_d(bool shared, bool dma, const AttnParams& p, dim3 grid, dim3 block, size_t lds,
                     hipStream_t stream) {
  if (dma) {   // planned only when every wave's heads share a KV head
    launch_one<D, true, true>(p, grid, block, lds, stream);
  } else {
    if (shared) launch_one<D, true, false>(p, grid, block, lds, stream);
    else launch_one<D, false, false>(p, grid, block, lds, stream);
  }
}

int launch_attention_paged(int D, bool shared, bool dma, const AttnParams& p, dim3 grid, dim3 block,
                           size_t lds, hipStream_t stream) {
  switch (D) {
    case 64: launch_d<64>(shared, dma, p, grid, block, lds, stream); break;
    case 80: launch_d<80>(shared, dma, p, grid, block, lds, stream); break;
    case 128: launch_d<128>(shared, dma, p, grid, block, lds, stream); break;
    default: return fail(SLMT_ERR_INVALID, "paged decode: head_dim must be 64/80/128, got " + std::to_string(D));
  }
  return check_launch("paged decode");
}

}  // namespace slmt
