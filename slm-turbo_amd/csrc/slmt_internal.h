// Internal declarations shared by the HIP translation units of libslmturbo_hip.so.
// gfx950 (CDNA4) only: wave64, DPP row operations, permlane16/32 swaps, dot8/dot2.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <string>

#include "../../include/slmturbo.h"

namespace slmt {

// ---------------------------------------------------------------------------
// Host-side error plumbing: a thread-local message returned by slmt_last_error.
// ---------------------------------------------------------------------------
void set_error(const std::string& msg);
void clear_error();
int fail(int code, const std::string& msg);
// Status of the calling thread's last fail() since clear_error() (for helpers
// that report failure through their return value, such as a negative size).
int last_status();
int check_launch(const char* what);

// Device properties cached per device (compute-unit count).
int device_cu_count();

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float h2f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t f2h(float f) {  // round to nearest even
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// DPP controls (GFX9 encoding).
enum : int {
  DPP_QUAD_XOR1 = 0xB1,   // quad_perm [1,0,3,2]
  DPP_QUAD_XOR2 = 0x4E,   // quad_perm [2,3,0,1]
  DPP_QUAD_ROT1 = 0x39,   // quad_perm [1,2,3,0]: lane i reads lane (i+1) & 3 of its quad
  DPP_QUAD_ROT3 = 0x93,   // quad_perm [3,0,1,2]: lane i reads lane (i+3) & 3
  DPP_ROW_ROR4 = 0x124,
  DPP_ROW_ROR8 = 0x128,
  DPP_ROW_SHL4 = 0x104,   // lane i reads lane i+4 of its row (0 past the row's end)
};

// Every control used here (quad permutations, rotations within a row) reads
// a lane of the same row, so no lane keeps its old value: the move has no
// "old" operand, which lets the backend fuse it into the consuming VALU op.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, CTRL, 0xf, 0xf, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}

// Exchange with the partner row (rows 0<->1, 2<->3) and the partner half-wave.
// Each swap returns both halves of the exchanged pair; combining them with a
// commutative op folds "self" and "partner" in every lane.  The two results
// are copied into scalars before any bit-cast: bit-casting a subscript of the
// returned vector directly reads element 0 twice with this compiler.
__device__ __forceinline__ void swap16(float x, float& a, float& b) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const unsigned r0 = r[0];
  const unsigned r1 = r[1];
  a = __builtin_bit_cast(float, r0);
  b = __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ void swap32(float x, float& a, float& b) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const unsigned r0 = r[0];
  const unsigned r1 = r[1];
  a = __builtin_bit_cast(float, r0);
  b = __builtin_bit_cast(float, r1);
}

// Two-register forms: permlane16 swaps the odd rows (16 lanes) of a with the
// even rows of b; permlane32 swaps the upper half-wave of a with the lower
// half-wave of b.  Afterwards a + b holds, per row, the sum of a pair of rows
// of one of the two inputs, so two values are folded at once.
__device__ __forceinline__ void permlane16_swap_pair(float& a, float& b) {
  auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, a), __builtin_bit_cast(unsigned, b),
                                            false, false);
  const unsigned r0 = r[0];
  const unsigned r1 = r[1];
  a = __builtin_bit_cast(float, r0);
  b = __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ void permlane32_swap_pair(float& a, float& b) {
  auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, a), __builtin_bit_cast(unsigned, b),
                                            false, false);
  const unsigned r0 = r[0];
  const unsigned r1 = r[1];
  a = __builtin_bit_cast(float, r0);
  b = __builtin_bit_cast(float, r1);
}

// Reductions over the 16 lanes that share (lane & 3): lanes 4p+g, p = 0..15.
__device__ __forceinline__ float red16_max(float x) {
  x = fmaxf(x, dpp_f<DPP_ROW_ROR4>(x));
  x = fmaxf(x, dpp_f<DPP_ROW_ROR8>(x));
  float a, b;
  swap16(x, a, b); x = fmaxf(a, b);
  swap32(x, a, b); x = fmaxf(a, b);
  return x;
}
__device__ __forceinline__ float red16_sum(float x) {
  x += dpp_f<DPP_ROW_ROR4>(x);
  x += dpp_f<DPP_ROW_ROR8>(x);
  float a, b;
  swap16(x, a, b); x = a + b;
  swap32(x, a, b); x = a + b;
  return x;
}

// Weight reference of the decode softmax (base-2 logits).  A token's P.V
// weight is fp16(exp2(s - R) * step) against a per-head reference R.  R
// follows the running max up; when a tile's max lies more than kRefDrop below
// R, R moves down to kRefDrop / 2 above that max, but never further than
// kRefFloor below the running max.  Every tile's largest weight then stays
// within 2^-kRefDrop of its step, so a long tail of tokens far below an early
// maximum (an attention sink) keeps fp16 precision instead of underflowing to
// zero, and the fp32 sums, rescaled by exp2(R_old - R_new) <= 2^kRefFloor,
// stay finite.  The half-threshold margin keeps R still while tile maxima
// wander within +-kRefDrop / 2 of where it moved (heavy-tailed scores would
// otherwise move it down and up again nearly every tile).
constexpr float kRefDrop = 10.0f;
constexpr float kRefFloor = 64.0f;

// Whether some 16-lane row of a wave ballot (lanes 16 g .. 16 g + 15) is
// empty: a 16-bit field f of m is zero exactly when (m - 1 per field) & ~m
// has f's top bit set (borrows only reach fields above a zero field).
__device__ __forceinline__ bool some_row_empty(uint64_t m) {
  return ((m - 0x0001000100010001ull) & ~m & 0x8000800080008000ull) != 0;
}
// Whether some lane class (lane & 3) == g of a wave ballot is empty.
__device__ __forceinline__ bool some_class4_empty(uint64_t m) {
  constexpr uint64_t c = 0x1111111111111111ull;
  return (m & c) == 0 || (m & (c << 1)) == 0 || (m & (c << 2)) == 0 || (m & (c << 3)) == 0;
}

// Full wave (64-lane) reductions with the hardware's fminf/fmaxf semantics:
// NaN operands are ignored and -0 orders below +0.
__device__ __forceinline__ float wave_min(float x) {
  x = fminf(x, dpp_f<DPP_QUAD_XOR1>(x));
  x = fminf(x, dpp_f<DPP_QUAD_XOR2>(x));
  x = fminf(x, dpp_f<DPP_ROW_ROR4>(x));
  x = fminf(x, dpp_f<DPP_ROW_ROR8>(x));
  float a, b;
  swap16(x, a, b); x = fminf(a, b);
  swap32(x, a, b); x = fminf(a, b);
  return x;
}
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp_f<DPP_QUAD_XOR1>(x));
  x = fmaxf(x, dpp_f<DPP_QUAD_XOR2>(x));
  x = fmaxf(x, dpp_f<DPP_ROW_ROR4>(x));
  x = fmaxf(x, dpp_f<DPP_ROW_ROR8>(x));
  float a, b;
  swap16(x, a, b); x = fmaxf(a, b);
  swap32(x, a, b); x = fmaxf(a, b);
  return x;
}

// ---------------------------------------------------------------------------
// Launchers (defined next to their kernels)
// ---------------------------------------------------------------------------
int launch_quantize_store(const void* key, int64_t key_stride, const void* value,
                          int64_t value_stride, void* cache, int64_t num_slots,
                          const int64_t* slot_mapping, int64_t N, int KV, int D,
                          hipStream_t stream);

int launch_quantize_rulers(const void* x, int64_t x_head_stride, int64_t x_seq_stride, int KV, int S, int D,
                           const void* scale, const void* zero, void* packed, int64_t out_head_stride,
                           int64_t out_seq_stride, hipStream_t stream);
int launch_quantize_per_channel(const void* x, int KV, int S, int D, void* packed,
                                void* scale, void* zero, hipStream_t stream);

// Attention source layouts.
enum SrcMode : int { SRC_PAGED = 0, SRC_TOKEN = 1, SRC_CHANNEL = 2 };

struct AttnParams {
  // queries: element (b, h, d) at q + b*q_seq_stride + h*q_head_stride + d
  const uint16_t* q;
  int64_t q_seq_stride, q_head_stride;
  // paged source
  const uint8_t* cache;
  const void* block_tables;
  int64_t bt_stride;
  int bt64;
  int block_size;
  int block_shift;   // log2(block_size) when a power of two, else -1
  int cache_kv;      // KV heads in the cache row
  int64_t num_blocks;
  // contiguous sources ([KV_t, S, D/2] codes; rulers [KV_t, S] or [KV_t, D])
  const uint8_t* kp;
  const uint8_t* vp;
  const uint16_t* kr0;  // k_min   | k_scale
  const uint16_t* kr1;  // k_step  | k_zero
  const uint16_t* vr0;  // v_min   | v_scale
  const uint16_t* vr1;  // v_step  | v_zero
  int s_rows;           // S of the contiguous tensors
  int use_quant;
  // sequences: L_b = seq_lens[b], or fixed_len, or min(fixed_len, b+1) (causal rows)
  const int32_t* seq_lens;
  int fixed_len;
  int causal_rows;
  int B, H, G;           // G = H / num_kv_heads
  int heads_per_group;   // query heads per workgroup (multiple of 4)
  // output: element (b, h, d) at out + b*out_seq_stride + h*out_head_stride + d
  void* out;
  int out_f16;
  int64_t out_seq_stride, out_head_stride;
  // workspace
  float* part_o;    // [W][2][H][D]
  float* part_ml;   // [W][2][H][2]
  int* counters;    // [groups][B]
  int W;            // workgroups per head group (grid.x)
  int min_tiles;    // minimum 16-token tiles per workgroup
  int nthreads;     // threads per workgroup (blockDim.x)
};

// Geometry chosen on the host for a launch.  W_ws is the workgroup count the
// workspace is sized for (the register-staged plan's, never below W).
struct AttnPlan {
  int heads_per_group, groups, waves, W, W_ws;
  bool dma;
  size_t lds_bytes;
  // whole-row kernel (head_dim 128, 4 or 8 query heads per KV head): KV heads
  // and waves per KV head of a workgroup, head groups
  bool rows;
  int rows_nkv, rows_wpk, rows_groups;
};

// dma_kv > 0 asks for the paged direct-load plan over a cache row of dma_kv
// KV heads; it is taken when every head group covers whole, 16-byte aligned
// KV heads and the LDS ring fits.
int plan_attention(int B, int H, int G, int D, int dma_kv, AttnPlan* plan);

// Whole-row kernel (attention_rows.hip): its shape for a request (false if it
// does not apply), the workgroups per head group it may use, and its launch.
bool rows_shape(int H, int G, int D, int cache_kv, int* nkv, int* wpk, int* groups);
int rows_max_workgroups(int D, int nkv, int wpk, int groups, int cus);
int launch_attention_rows(int D, int nkv, int wpk, int groups, const AttnParams& p, hipStream_t stream);
// Event pair for a whole-row decode kernel when slmt_kernel_timing is on: the
// next free pair of the pool (false when off or full).  The launch passes them
// to hipExtLaunchKernelGGL, which stamps them from the kernel's own dispatch.
// `kernel` (a string with static storage) names the timed kernel.
bool kernel_timing_events(hipEvent_t* start, hipEvent_t* stop, const char* kernel);
const char* kernel_timing_kernel();           // slmt_kernel_timing_kernel
int set_kernel_timing(bool enable);            // slmt_kernel_timing
int read_kernel_timing(float* us, int max_n);  // slmt_kernel_timing_read
// Matrix-core variant of the whole-row kernel (attention_mfma.hip): whether it
// serves a whole-row shape (SLMT_PAGED_DECODE=valu turns it off), and its launch.
bool mfma_rows_enabled(int D, int nkv, int wpk);
int launch_attention_mfma(int D, int nkv, int wpk, int groups, const AttnParams& p, hipStream_t stream);
int64_t attention_workspace_bytes(int B, int H, int KV, int D);

// Arrival counters live in a fixed region at the start of every workspace, so
// calls of any shape that share a workspace never overwrite each other's
// counters with partial results (each call leaves its counters at zero).
constexpr int64_t kWsCounterInts = int64_t(1) << 20;

// Single-sequence per-channel decode split over (KV head, key chunk)
// workgroups (decode_channel.hip), head_dim 64 and 128, up to 8 query heads per
// KV head and 16384 keys.  Returns SLMT_ERR_UNSUPPORTED (without an error
// message) when the request falls outside that, so the caller can take the
// general path.
int launch_decode_channel_split(const void* q, const void* kp, const void* ks, const void* kz, const void* vp,
                                const void* vs, const void* vz, int H, int G, int S, int D, int use_quant, float* out,
                                void* workspace, int64_t ws_bytes, hipStream_t stream);

// Per-channel prefill on the matrix cores (prefill_mfma.hip), head_dim 64 and 128;
// no workspace.  q [H, M, D] fp16, codes [KV_t, S, D/2], rulers [KV_t, D].
bool prefill_mfma_supported(int D);
int launch_prefill_mfma(const void* q, const void* kp, const void* ks, const void* kz, const void* vp, const void* vs,
                        const void* vz, int H, int G, int M, int S, int D, int causal, int use_quant, float* out,
                        hipStream_t stream);
// clear_counters: zero the arrival counters the launch uses (a fill kernel on
// the stream, before the decode) instead of relying on the previous call
// having left them at zero.
int launch_attention(int mode, int D, AttnParams& p, void* workspace, int64_t ws_bytes,
                     hipStream_t stream, bool clear_counters = false);

// Body of slmt_decode_paged_batched (abi.hip) over a given workspace.
int decode_paged_batched(const void* q, int64_t q_seq_stride, int64_t q_head_stride, const void* kv_cache,
                         int64_t num_blocks, int block_size, const void* block_tables, int block_table_bits,
                         int64_t block_table_stride, const int32_t* seq_lens, int fixed_seq_len, int num_seqs,
                         int num_heads, int num_kv_heads, int head_dim, void* out, int out_dtype,
                         int64_t out_seq_stride, int64_t out_head_stride, void* workspace, int64_t workspace_bytes,
                         hipStream_t stream, bool clear_counters);

}  // namespace slmt
