// slmt_decode_paged_batched_noalloc: the batched paged decode for callers that
// cannot allocate (code under HIP graph capture, tight serving loops).
//
// Its workspace (split-sequence partials and arrival counters) lives in a
// file-scope device array, `scratch`, of SLMT_NOALLOC_SCRATCH_BYTES.  Every GPU
// the library runs on holds its own copy for the life of the process.  The host
// never uses the array's name as an address: on a device's first call the
// entry point asks the runtime for that device's address of the array
// (hipGetSymbolAddress, with the device current) and keeps it per device.
// Nothing here calls hipMalloc, hipFree or an allocating library routine.
//
// All calls on one GPU share its array, which keeps the last call's contents:
// the arrival counters a call uses are cleared by a fill kernel on the call's
// stream before the decode, and calls that overlap on one GPU (unordered
// streams, or threads) race on the array.
#include "slmt_internal.h"

#include <mutex>
#include <string>

namespace slmt {
namespace {

constexpr int64_t kScratchBytes = SLMT_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};

// This device's address of `scratch`, looked up once per device.
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(SLMT_ERR_HIP, std::string("paged decode (no-alloc): hipGetDevice failed: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(SLMT_ERR_UNSUPPORTED, "paged decode (no-alloc): device index " + std::to_string(dev) + " out of range");
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(SLMT_ERR_HIP, std::string("paged decode (no-alloc): hipGetSymbolAddress(scratch) failed: ") +
                                    hipGetErrorString(e));
    g_scratch[dev] = ptr;
  }
  *out = g_scratch[dev];
  return SLMT_OK;
}

}  // namespace
}  // namespace slmt

using namespace slmt;

extern "C" int slmt_decode_paged_batched_noalloc(const void* q, int64_t q_seq_stride, int64_t q_head_stride,
                                                 const void* kv_cache, int64_t num_blocks, int block_size,
                                                 const void* block_tables, int block_table_bits,
                                                 int64_t block_table_stride, const int32_t* seq_lens,
                                                 int fixed_seq_len, int num_seqs, int num_heads, int num_kv_heads,
                                                 int head_dim, void* out, int out_dtype, int64_t out_seq_stride,
                                                 int64_t out_head_stride, slmt_stream_t stream) {
  clear_error();
  if (num_seqs < 0) return fail(SLMT_ERR_INVALID, "paged decode: num_seqs must be >= 0");
  if (num_seqs == 0) return SLMT_OK;
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return fail(SLMT_ERR_INVALID, "H not divisible by num_kv_heads");
  if (head_dim != 64 && head_dim != 80 && head_dim != 128)
    return fail(SLMT_ERR_INVALID, "paged decode: head_dim must be 64/80/128, got " + std::to_string(head_dim));
  const int64_t need = attention_workspace_bytes(num_seqs, num_heads, num_kv_heads, head_dim);
  if (need < 0) return last_status();   // the sizing's own status and message
  if (need > kScratchBytes)
    return fail(SLMT_ERR_UNSUPPORTED, "paged decode (no-alloc): this call needs " + std::to_string(need) +
                                          " bytes of workspace, above the " + std::to_string(kScratchBytes) +
                                          " bytes of the entry point's static scratch; use "
                                          "slmt_decode_paged_batched with a caller-owned workspace");
  void* ws = nullptr;
  if (int rc = scratch_address(&ws)) return rc;
  return decode_paged_batched(q, q_seq_stride, q_head_stride, kv_cache, num_blocks, block_size, block_tables,
                              block_table_bits, block_table_stride, seq_lens, fixed_seq_len, num_seqs, num_heads,
                              num_kv_heads, head_dim, out, out_dtype, out_seq_stride, out_head_stride, ws,
                              kScratchBytes, reinterpret_cast<hipStream_t>(stream), /*clear_counters=*/true);
}
