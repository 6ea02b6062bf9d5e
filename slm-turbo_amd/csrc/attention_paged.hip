// Instantiations of the attention kernel for the paged per-token cache.
#include "attention_kernel.h"

namespace slmt {

template <int D, bool SHARED, bool FAST>
static void launch_one(const AttnParams& p, dim3 grid, dim3 block, size_t lds, hipStream_t stream) {
  hipLaunchKernelGGL((attn::attention_kernel<D, SRC_PAGED, SHARED, FAST>), grid, block, lds, stream, p);
}

template <int D>
static void launch_d(bool shared, bool fast, const AttnParams& p, dim3 grid, dim3 block, size_t lds,
                     hipStream_t stream) {
  if (fast) {
    if (shared) launch_one<D, true, true>(p, grid, block, lds, stream);
    else launch_one<D, false, true>(p, grid, block, lds, stream);
  } else {
    if (shared) launch_one<D, true, false>(p, grid, block, lds, stream);
    else launch_one<D, false, false>(p, grid, block, lds, stream);
  }
}

int launch_attention_paged(int D, bool shared, bool fast, const AttnParams& p, dim3 grid, dim3 block,
                           size_t lds, hipStream_t stream) {
  switch (D) {
    case 64: launch_d<64>(shared, fast, p, grid, block, lds, stream); break;
    case 80: launch_d<80>(shared, fast, p, grid, block, lds, stream); break;
    case 128: launch_d<128>(shared, fast, p, grid, block, lds, stream); break;
    default: return fail(SLMT_ERR_INVALID, "paged decode: head_dim must be 64/80/128, got " + std::to_string(D));
  }
  return check_launch("paged decode");
}

}  // namespace slmt
