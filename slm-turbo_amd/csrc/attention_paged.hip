// Instantiations of the attention kernel for the paged per-token cache.
#include "attention_kernel.h"

namespace slmt {

template <int D, bool SHARED, bool DMA>
static void launch_one(const AttnParams& p, dim3 grid, dim3 block, size_t lds, hipStream_t stream) {
  auto kern = attn::attention_kernel<D, SRC_PAGED, SHARED, DMA>;
  if (lds > 64 * 1024) {
    // raise the dynamic LDS limit once per instantiation (the ring can exceed 64 KB)
    static const hipError_t once =
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024);
    (void)once;
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
