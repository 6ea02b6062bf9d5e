// Instantiations of the attention kernel for the contiguous per-token and
// per-channel layouts (standalone decode and prefill).  These are launched once
// per request, so only the general (any GQA grouping) variant is built.
#include "attention_kernel.h"

namespace slmt {

template <int D, int MODE>
static void launch_one(const AttnParams& p, dim3 grid, dim3 block, size_t lds, hipStream_t stream) {
  hipLaunchKernelGGL((attn::attention_kernel<D, MODE, false, false>), grid, block, lds, stream, p);
}

int launch_attention_contig(int mode, int D, const AttnParams& p, dim3 grid, dim3 block, size_t lds,
                            hipStream_t stream) {
  switch (mode * 1000 + D) {
    case SRC_TOKEN * 1000 + 64: launch_one<64, SRC_TOKEN>(p, grid, block, lds, stream); break;
    case SRC_TOKEN * 1000 + 80: launch_one<80, SRC_TOKEN>(p, grid, block, lds, stream); break;
    case SRC_TOKEN * 1000 + 128: launch_one<128, SRC_TOKEN>(p, grid, block, lds, stream); break;
    case SRC_CHANNEL * 1000 + 64: launch_one<64, SRC_CHANNEL>(p, grid, block, lds, stream); break;
    case SRC_CHANNEL * 1000 + 80: launch_one<80, SRC_CHANNEL>(p, grid, block, lds, stream); break;
    case SRC_CHANNEL * 1000 + 128: launch_one<128, SRC_CHANNEL>(p, grid, block, lds, stream); break;
    default: return fail(SLMT_ERR_INVALID, "attention: head_dim must be 64/80/128, got " + std::to_string(D));
  }
  return check_launch("attention");
}

}  // namespace slmt
