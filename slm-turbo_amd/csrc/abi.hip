// extern "C" entry points of libslmturbo_hip.so (declared in include/slmturbo.h).
//
// This layer replaces the reference's pybind11/ATen launchers
// (kernels/kv_dequant_cuda.cu:53-456): it validates sizes, strides and
// alignment with the same phase-prefixed wording as the reference's
// TORCH_CHECKs, then enqueues the kernels on the caller's stream (the
// reference used the legacy default stream).  Nothing here allocates.
#include "slmt_internal.h"

#include <mutex>
#include <string>

namespace slmt {

namespace {
thread_local std::string g_error;
thread_local int g_status = SLMT_OK;
}

void set_error(const std::string& msg) { g_error = msg; }
void clear_error() {
  g_error.clear();
  g_status = SLMT_OK;
}
int fail(int code, const std::string& msg) {
  g_error = msg;
  g_status = code;
  return code;
}
int last_status() { return g_status == SLMT_OK ? SLMT_ERR_INVALID : g_status; }
int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SLMT_ERR_HIP, std::string(what) + ": launch failed: " + hipGetErrorString(e));
  return SLMT_OK;
}

int device_cu_count() {
  static std::mutex mu;
  static int counts[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -1;
  std::lock_guard<std::mutex> lock(mu);
  if (counts[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
    counts[dev] = n;
  }
  return counts[dev];
}

namespace {

bool head_dim_ok(int D) { return D == 64 || D == 80 || D == 128; }
bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }
std::string s(int64_t v) { return std::to_string(v); }

int block_shift_of(int bs) {
  if (bs <= 0 || (bs & (bs - 1)) != 0) return -1;
  int k = 0;
  while ((1 << k) < bs) ++k;
  return k;
}

AttnParams blank_params() {
  AttnParams p{};
  p.block_shift = -1;
  p.min_tiles = 4;
  return p;
}

// Shared checks of the contiguous-source entry points.
int check_contig(const char* phase, const void* q, const void* kp, const void* vp, const void* r[4],
                 int H, int KVt, int KV, int S, int D, const float* out) {
  if (!head_dim_ok(D)) return fail(SLMT_ERR_INVALID, std::string(phase) + ": head_dim must be 64/80/128, got " + s(D));
  if (KV <= 0 || H <= 0 || H % KV != 0)
    return fail(SLMT_ERR_INVALID, std::string(phase) + ": num_kv_heads " + s(KV) + " must divide query heads " + s(H));
  if (KV > KVt)
    return fail(SLMT_ERR_INVALID, std::string(phase) + ": num_kv_heads " + s(KV) +
                                      " exceeds the packed KV heads " + s(KVt));
  if (S < 0) return fail(SLMT_ERR_INVALID, std::string(phase) + ": sequence length must be >= 0");
  if (!q || !kp || !vp || !out || !r[0] || !r[1] || !r[2] || !r[3])
    return fail(SLMT_ERR_INVALID, std::string(phase) + ": null pointer argument");
  if (!aligned(q, 16) || !aligned(kp, 8) || !aligned(vp, 8) || !aligned(out, 8))
    return fail(SLMT_ERR_INVALID, std::string(phase) + ": q must be 16-byte, packed KV and out 8-byte aligned");
  return SLMT_OK;
}

int check_workspace(const char* phase, int B, int H, int KV, int D, const void* ws, int64_t ws_bytes) {
  const int64_t need = attention_workspace_bytes(B, H, KV, D);
  if (need < 0) return last_status();
  if (!ws || ws_bytes < need)
    return fail(SLMT_ERR_INVALID, std::string(phase) + ": workspace of " + s(need) + " bytes required, got " + s(ws_bytes));
  return SLMT_OK;
}

}  // namespace

int decode_paged_batched(const void* q, int64_t q_seq_stride, int64_t q_head_stride, const void* kv_cache,
                         int64_t num_blocks, int block_size, const void* block_tables, int block_table_bits,
                         int64_t block_table_stride, const int32_t* seq_lens, int fixed_seq_len, int num_seqs,
                         int num_heads, int num_kv_heads, int head_dim, void* out, int out_dtype,
                         int64_t out_seq_stride, int64_t out_head_stride, void* workspace, int64_t workspace_bytes,
                         hipStream_t stream, bool clear_counters) {
  const char* ph = "paged decode";
  if (!head_dim_ok(head_dim)) return fail(SLMT_ERR_INVALID, "paged decode: head_dim must be 64/80/128, got " + s(head_dim));
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return fail(SLMT_ERR_INVALID, "H not divisible by num_kv_heads");
  if (block_size <= 0) return fail(SLMT_ERR_INVALID, "paged decode: block_size must be positive, got " + s(block_size));
  if (block_table_bits != 32 && block_table_bits != 64)
    return fail(SLMT_ERR_INVALID, "paged decode: block table must be int32 or int64");
  if (out_dtype != SLMT_OUT_F32 && out_dtype != SLMT_OUT_F16)
    return fail(SLMT_ERR_INVALID, "paged decode: out dtype must be fp32 or fp16");
  if (num_seqs < 0) return fail(SLMT_ERR_INVALID, "paged decode: num_seqs must be >= 0");
  if (!seq_lens && fixed_seq_len < 0) return fail(SLMT_ERR_INVALID, "paged decode: seq_len must be >= 0");
  if (num_seqs == 0) return SLMT_OK;
  if (!q || !kv_cache || !block_tables || !out) return fail(SLMT_ERR_INVALID, "paged decode: null pointer argument");
  if (!aligned(q, 16) || (q_seq_stride % 8) || (q_head_stride % 8))
    return fail(SLMT_ERR_INVALID, "paged decode: q must be 16-byte aligned with strides that are multiples of 8");
  if (!aligned(out, out_dtype == SLMT_OUT_F32 ? 8 : 4) || (out_seq_stride & 1) || (out_head_stride & 1))
    return fail(SLMT_ERR_INVALID, "paged decode: out must be aligned with even strides");
  if (!aligned(kv_cache, 8)) return fail(SLMT_ERR_INVALID, "paged decode: kv_cache must be 8-byte aligned");
  int rc = check_workspace(ph, num_seqs, num_heads, num_kv_heads, head_dim, workspace, workspace_bytes);
  if (rc != SLMT_OK) return rc;
  AttnParams p = blank_params();
  p.q = reinterpret_cast<const uint16_t*>(q);
  p.q_seq_stride = q_seq_stride;
  p.q_head_stride = q_head_stride;
  p.cache = reinterpret_cast<const uint8_t*>(kv_cache);
  p.block_tables = block_tables;
  p.bt_stride = block_table_stride;
  p.bt64 = block_table_bits == 64;
  p.block_size = block_size;
  p.block_shift = block_shift_of(block_size);
  p.cache_kv = num_kv_heads;
  p.num_blocks = num_blocks;
  p.seq_lens = seq_lens;
  p.fixed_len = fixed_seq_len;
  p.B = num_seqs;
  p.H = num_heads;
  p.G = num_heads / num_kv_heads;
  p.out = out;
  p.out_f16 = out_dtype == SLMT_OUT_F16;
  p.out_seq_stride = out_seq_stride;
  p.out_head_stride = out_head_stride;
  return launch_attention(SRC_PAGED, head_dim, p, workspace, workspace_bytes, stream, clear_counters);
}

}  // namespace slmt

using namespace slmt;

extern "C" {

const char* slmt_last_error(void) { return g_error.c_str(); }

int slmt_abi_version(void) { return SLMT_ABI_VERSION; }

int64_t slmt_attention_workspace_bytes(int num_seqs, int num_heads, int num_kv_heads, int head_dim) {
  clear_error();
  if (!head_dim_ok(head_dim)) return fail(SLMT_ERR_INVALID, "workspace: head_dim must be 64/80/128, got " + s(head_dim)), -1;
  return attention_workspace_bytes(num_seqs, num_heads, num_kv_heads, head_dim);
}

int slmt_quantize_store(const void* key, int64_t key_token_stride, const void* value,
                        int64_t value_token_stride, void* kv_cache, int64_t num_blocks,
                        int block_size, const int64_t* slot_mapping, int64_t num_tokens,
                        int num_kv_heads, int head_dim, slmt_stream_t stream) {
  clear_error();
  if (!head_dim_ok(head_dim)) return fail(SLMT_ERR_INVALID, "store: head_dim must be 64/80/128, got " + s(head_dim));
  if (num_tokens < 0 || num_kv_heads <= 0 || block_size <= 0 || num_blocks < 0)
    return fail(SLMT_ERR_INVALID, "store: invalid sizes (N=" + s(num_tokens) + ", KV=" + s(num_kv_heads) +
                                      ", block_size=" + s(block_size) + ")");
  if (num_tokens == 0) return SLMT_OK;
  if (!key || !value || !kv_cache || !slot_mapping) return fail(SLMT_ERR_INVALID, "store: null pointer argument");
  if (key_token_stride < (int64_t)num_kv_heads * head_dim || value_token_stride < (int64_t)num_kv_heads * head_dim)
    return fail(SLMT_ERR_INVALID, "store: token stride smaller than KV*D");
  if ((key_token_stride & 1) || (value_token_stride & 1) || !aligned(key, 4) || !aligned(value, 4) ||
      !aligned(kv_cache, 8))
    return fail(SLMT_ERR_INVALID, "store: key/value rows must be 4-byte aligned and the cache 8-byte aligned");
  return launch_quantize_store(key, key_token_stride, value, value_token_stride, kv_cache,
                               num_blocks * (int64_t)block_size, slot_mapping, num_tokens,
                               num_kv_heads, head_dim, reinterpret_cast<hipStream_t>(stream));
}

int slmt_quantize_per_channel(const void* x, int num_kv_heads, int seq_len, int head_dim, void* packed,
                              void* scale, void* zero, slmt_stream_t stream) {
  clear_error();
  if (!head_dim_ok(head_dim))
    return fail(SLMT_ERR_INVALID, "quantize: head_dim must be 64/80/128, got " + s(head_dim));
  if (num_kv_heads < 0 || seq_len <= 0)
    return fail(SLMT_ERR_INVALID, "quantize: need KV >= 0 and S >= 1 (got KV=" + s(num_kv_heads) + ", S=" + s(seq_len) + ")");
  if (num_kv_heads == 0) return SLMT_OK;
  if (!x || !packed || !scale || !zero) return fail(SLMT_ERR_INVALID, "quantize: null pointer argument");
  if (!aligned(x, 4) || !aligned(scale, 2) || !aligned(zero, 2))
    return fail(SLMT_ERR_INVALID, "quantize: x must be 4-byte aligned");
  return launch_quantize_per_channel(x, num_kv_heads, seq_len, head_dim, packed, scale, zero,
                                     reinterpret_cast<hipStream_t>(stream));
}

int slmt_quantize_with_rulers(const void* x, int64_t x_head_stride, int64_t x_seq_stride, int num_kv_heads,
                              int seq_len, int head_dim, const void* scale, const void* zero, void* packed,
                              int64_t out_head_stride, int64_t out_seq_stride, slmt_stream_t stream) {
  clear_error();
  if (!head_dim_ok(head_dim))
    return fail(SLMT_ERR_INVALID, "quantize_tensor: head_dim must be 64/80/128, got " + s(head_dim));
  if (num_kv_heads < 0 || seq_len < 0)
    return fail(SLMT_ERR_INVALID, "quantize_tensor: need KV >= 0 and S >= 0");
  if (num_kv_heads == 0 || seq_len == 0) return SLMT_OK;
  if (!x || !scale || !zero || !packed) return fail(SLMT_ERR_INVALID, "quantize_tensor: null pointer argument");
  if ((x_head_stride & 1) || (x_seq_stride & 1) || !aligned(x, 4) || !aligned(scale, 4) || !aligned(zero, 4))
    return fail(SLMT_ERR_INVALID, "quantize_tensor: x rows and the rulers must be 4-byte aligned (even strides)");
  if ((seq_len > 1 && (x_seq_stride < head_dim || out_seq_stride < head_dim / 2)) ||
      (num_kv_heads > 1 && (x_head_stride < head_dim || out_head_stride < head_dim / 2)))
    return fail(SLMT_ERR_INVALID, "quantize_tensor: strides smaller than a row");
  return launch_quantize_rulers(x, x_head_stride, x_seq_stride, num_kv_heads, seq_len, head_dim, scale, zero,
                                packed, out_head_stride, out_seq_stride, reinterpret_cast<hipStream_t>(stream));
}

int slmt_decode_paged_batched(const void* q, int64_t q_seq_stride, int64_t q_head_stride,
                              const void* kv_cache, int64_t num_blocks, int block_size,
                              const void* block_tables, int block_table_bits, int64_t block_table_stride,
                              const int32_t* seq_lens, int fixed_seq_len, int num_seqs, int num_heads,
                              int num_kv_heads, int head_dim, void* out, int out_dtype,
                              int64_t out_seq_stride, int64_t out_head_stride, void* workspace,
                              int64_t workspace_bytes, slmt_stream_t stream) {
  clear_error();
  return decode_paged_batched(q, q_seq_stride, q_head_stride, kv_cache, num_blocks, block_size, block_tables,
                              block_table_bits, block_table_stride, seq_lens, fixed_seq_len, num_seqs, num_heads,
                              num_kv_heads, head_dim, out, out_dtype, out_seq_stride, out_head_stride, workspace,
                              workspace_bytes, reinterpret_cast<hipStream_t>(stream), false);
}

int slmt_decode_paged(const void* q, const void* kv_cache, int64_t num_blocks, int block_size,
                      const int64_t* block_table, int seq_len, int num_heads, int num_kv_heads,
                      int head_dim, float* out, void* workspace, int64_t workspace_bytes,
                      slmt_stream_t stream) {
  // One request = a batch of one with a fixed length and an int64 block row.
  if (seq_len < 0) {
    clear_error();
    return fail(SLMT_ERR_INVALID, "paged decode: seq_len must be >= 0");
  }
  return slmt_decode_paged_batched(q, (int64_t)num_heads * head_dim, head_dim, kv_cache, num_blocks,
                                   block_size, block_table, 64, 0, nullptr, seq_len, 1, num_heads,
                                   num_kv_heads, head_dim, out, SLMT_OUT_F32,
                                   (int64_t)num_heads * head_dim, head_dim, workspace, workspace_bytes,
                                   stream);
}

int slmt_decode_per_token(const void* q, const void* k_packed, const void* k_min, const void* k_step,
                          const void* v_packed, const void* v_min, const void* v_step, int num_heads,
                          int kv_tensor_heads, int num_kv_heads, int seq_len, int head_dim, int block_n,
                          float* out, void* workspace, int64_t workspace_bytes, slmt_stream_t stream) {
  clear_error();
  const char* ph = "per-token decode";
  if (block_n != 32 && block_n != 64)
    return fail(SLMT_ERR_INVALID, "per-token decode: BLOCK_N must be 32 or 64, got " + s(block_n));
  const void* r[4] = {k_min, k_step, v_min, v_step};
  int rc = check_contig(ph, q, k_packed, v_packed, r, num_heads, kv_tensor_heads, num_kv_heads, seq_len, head_dim, out);
  if (rc != SLMT_OK) return rc;
  rc = check_workspace(ph, 1, num_heads, num_kv_heads, head_dim, workspace, workspace_bytes);
  if (rc != SLMT_OK) return rc;
  AttnParams p = blank_params();
  p.q = reinterpret_cast<const uint16_t*>(q);
  p.q_seq_stride = (int64_t)num_heads * head_dim;
  p.q_head_stride = head_dim;
  p.kp = reinterpret_cast<const uint8_t*>(k_packed);
  p.vp = reinterpret_cast<const uint8_t*>(v_packed);
  p.kr0 = reinterpret_cast<const uint16_t*>(k_min);
  p.kr1 = reinterpret_cast<const uint16_t*>(k_step);
  p.vr0 = reinterpret_cast<const uint16_t*>(v_min);
  p.vr1 = reinterpret_cast<const uint16_t*>(v_step);
  p.s_rows = seq_len;
  p.fixed_len = seq_len;
  p.B = 1;
  p.H = num_heads;
  p.G = num_heads / num_kv_heads;
  p.out = out;
  p.out_seq_stride = (int64_t)num_heads * head_dim;
  p.out_head_stride = head_dim;
  return launch_attention(SRC_TOKEN, head_dim, p, workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

int slmt_decode_per_channel(const void* q, const void* k_packed, const void* k_scale, const void* k_zero,
                            const void* v_packed, const void* v_scale, const void* v_zero, int num_heads,
                            int kv_tensor_heads, int num_kv_heads, int seq_len, int head_dim, int block_n,
                            int use_quant, float* out, void* workspace, int64_t workspace_bytes,
                            slmt_stream_t stream) {
  clear_error();
  const char* ph = "kv_dequant_decode";
  if (block_n != 32 && block_n != 64)
    return fail(SLMT_ERR_INVALID, "kv_dequant_decode: BLOCK_N must be 32 or 64, got " + s(block_n));
  const void* r[4] = {k_scale, k_zero, v_scale, v_zero};
  int rc = check_contig(ph, q, k_packed, v_packed, r, num_heads, kv_tensor_heads, num_kv_heads, seq_len, head_dim, out);
  if (rc != SLMT_OK) return rc;
  rc = check_workspace(ph, 1, num_heads, num_kv_heads, head_dim, workspace, workspace_bytes);
  if (rc != SLMT_OK) return rc;
  // one short sequence: split over (KV head, key chunk) when the shape allows it
  rc = launch_decode_channel_split(q, k_packed, k_scale, k_zero, v_packed, v_scale, v_zero, num_heads,
                                   num_heads / num_kv_heads, seq_len, head_dim, use_quant, out, workspace,
                                   workspace_bytes, reinterpret_cast<hipStream_t>(stream));
  if (rc != SLMT_ERR_UNSUPPORTED) return rc;
  AttnParams p = blank_params();
  p.q = reinterpret_cast<const uint16_t*>(q);
  p.q_seq_stride = (int64_t)num_heads * head_dim;
  p.q_head_stride = head_dim;
  p.kp = reinterpret_cast<const uint8_t*>(k_packed);
  p.vp = reinterpret_cast<const uint8_t*>(v_packed);
  p.kr0 = reinterpret_cast<const uint16_t*>(k_scale);
  p.kr1 = reinterpret_cast<const uint16_t*>(k_zero);
  p.vr0 = reinterpret_cast<const uint16_t*>(v_scale);
  p.vr1 = reinterpret_cast<const uint16_t*>(v_zero);
  p.use_quant = use_quant ? 1 : 0;
  p.s_rows = seq_len;
  p.fixed_len = seq_len;
  p.B = 1;
  p.H = num_heads;
  p.G = num_heads / num_kv_heads;
  p.out = out;
  p.out_seq_stride = (int64_t)num_heads * head_dim;
  p.out_head_stride = head_dim;
  return launch_attention(SRC_CHANNEL, head_dim, p, workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

int slmt_prefill_per_channel(const void* q, const void* k_packed, const void* k_scale, const void* k_zero,
                             const void* v_packed, const void* v_scale, const void* v_zero, int num_heads,
                             int kv_tensor_heads, int num_kv_heads, int num_queries, int seq_len, int head_dim,
                             int block_m, int block_n, int causal, int use_quant, float* out, void* workspace,
                             int64_t workspace_bytes, slmt_stream_t stream) {
  clear_error();
  const char* ph = "kv_dequant_prefill";
  if (block_m != 16 && block_m != 32)
    return fail(SLMT_ERR_INVALID, "kv_dequant_prefill: BLOCK_M must be 16 or 32, got " + s(block_m));
  if (block_n != 32 && block_n != 64)
    return fail(SLMT_ERR_INVALID, "kv_dequant_prefill: BLOCK_N must be 32 or 64, got " + s(block_n));
  const bool combo_ok = (block_m == 16 && block_n == 32) || head_dim == 64;
  if (!combo_ok)
    return fail(SLMT_ERR_INVALID, "kv_dequant_prefill: (BLOCK_M=" + s(block_m) + ", BLOCK_N=" + s(block_n) +
                                      ") does not fit the 48 KB shared budget for head_dim=" + s(head_dim) +
                                      ". Use BLOCK_M=16, BLOCK_N=32 for D>=80.");
  const void* r[4] = {k_scale, k_zero, v_scale, v_zero};
  int rc = check_contig(ph, q, k_packed, v_packed, r, num_heads, kv_tensor_heads, num_kv_heads, seq_len, head_dim, out);
  if (rc != SLMT_OK) return rc;
  if (num_queries < 0) return fail(SLMT_ERR_INVALID, "kv_dequant_prefill: M must be >= 0");
  if (num_queries == 0) return SLMT_OK;
  if (prefill_mfma_supported(head_dim))
    return launch_prefill_mfma(q, k_packed, k_scale, k_zero, v_packed, v_scale, v_zero, num_heads,
                               num_heads / num_kv_heads, num_queries, seq_len, head_dim, causal, use_quant, out,
                               reinterpret_cast<hipStream_t>(stream));
  rc = check_workspace(ph, num_queries, num_heads, num_kv_heads, head_dim, workspace, workspace_bytes);
  if (rc != SLMT_OK) return rc;
  AttnParams p = blank_params();
  p.q = reinterpret_cast<const uint16_t*>(q);
  p.q_seq_stride = head_dim;                          // query row m
  p.q_head_stride = (int64_t)num_queries * head_dim;  // [H, M, D]
  p.kp = reinterpret_cast<const uint8_t*>(k_packed);
  p.vp = reinterpret_cast<const uint8_t*>(v_packed);
  p.kr0 = reinterpret_cast<const uint16_t*>(k_scale);
  p.kr1 = reinterpret_cast<const uint16_t*>(k_zero);
  p.vr0 = reinterpret_cast<const uint16_t*>(v_scale);
  p.vr1 = reinterpret_cast<const uint16_t*>(v_zero);
  p.use_quant = use_quant ? 1 : 0;
  p.s_rows = seq_len;
  p.fixed_len = seq_len;
  p.causal_rows = causal ? 1 : 0;
  p.B = num_queries;
  p.H = num_heads;
  p.G = num_heads / num_kv_heads;
  p.out = out;
  p.out_seq_stride = head_dim;
  p.out_head_stride = (int64_t)num_queries * head_dim;
  return launch_attention(SRC_CHANNEL, head_dim, p, workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

int slmt_kernel_timing(int enable) {
  clear_error();
  return set_kernel_timing(enable != 0);
}

const char* slmt_kernel_timing_kernel(void) { return kernel_timing_kernel(); }

int slmt_kernel_timing_read(float* us, int max_n) {
  clear_error();
  if (us == nullptr && max_n > 0) return fail(SLMT_ERR_INVALID, "timing: output array is null"), -1;
  return read_kernel_timing(us, max_n);
}

}  // extern "C"
