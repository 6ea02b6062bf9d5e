// Quantize-on-write store into the packed per-token 4-bit paged cache.
//
// Same arithmetic as the reference's kv_quantize_store_kernel
// (kernels/kv_dequant_kernels.cuh:816-919), laid out for CDNA4: one wave64 per
// (token, kv head) row, two adjacent dims per lane (one fp16x2 load), min/max
// by DPP + permlane swaps instead of a 128-thread LDS tree, and one lane-wide
// byte store per packed byte.  Every fp32 operation is rounded separately
// (contraction off) so codes and fp16 rulers are bit-exact with the reference.
#include "slmt_internal.h"

namespace slmt {

namespace {

constexpr int kRowsPerBlock = 4;  // 4 waves, one row each

template <int D>
__device__ __forceinline__ void quantize_pair(float x0, float x1, float mn, float step,
                                              uint8_t& byte) {
#pragma clang fp contract(off)
  int q0 = (int)((x0 - mn) / step + 0.5f);
  int q1 = (int)((x1 - mn) / step + 0.5f);
  q0 = q0 < 0 ? 0 : (q0 > 15 ? 15 : q0);
  q1 = q1 < 0 ? 0 : (q1 > 15 ? 15 : q1);
  byte = (uint8_t)(q0 | (q1 << 4));
}

template <int D>
__device__ __forceinline__ void row_stats(float x0, float x1, bool active, float& mn, float& step) {
#pragma clang fp contract(off)
  float lo = active ? fminf(x0, x1) : INFINITY;
  float hi = active ? fmaxf(x0, x1) : -INFINITY;
  mn = wave_min(lo);
  float mx = wave_max(hi);
  step = (mx - mn) / 15.0f;
  if (!(step > 0.0f)) step = 1.0f;  // constant (or all-NaN) row guard
}

template <int D>
__global__ void __launch_bounds__(64 * kRowsPerBlock)
quantize_store_kernel(const uint16_t* __restrict__ key, int64_t key_stride,
                      const uint16_t* __restrict__ value, int64_t value_stride,
                      uint8_t* __restrict__ cache, int64_t num_slots,
                      const int64_t* __restrict__ slot_mapping, int64_t N, int KV) {
  constexpr int SLOT = D + 8;
  constexpr int HALF = D / 2;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= N * KV) return;                       // wave-uniform
  const int64_t t = row / KV;
  const int h = (int)(row - t * KV);
  // The row is quantized whether or not its slot is valid and only the stores
  // test it: with an early exit on the slot the row's K/V loads were issued
  // after the slot's had returned, two dependent round trips per call.
  const int64_t slot = slot_mapping[t];
  const bool valid = slot >= 0 && slot < num_slots;   // padding token / out of range: no store
  const bool active = lane < HALF;
  const int li = active ? lane : 0;
  const uint32_t kw = *reinterpret_cast<const uint32_t*>(key + t * key_stride + (int64_t)h * D + 2 * li);
  const uint32_t vw = *reinterpret_cast<const uint32_t*>(value + t * value_stride + (int64_t)h * D + 2 * li);
  const float k0 = h2f((uint16_t)(kw & 0xffffu)), k1 = h2f((uint16_t)(kw >> 16));
  const float v0 = h2f((uint16_t)(vw & 0xffffu)), v1 = h2f((uint16_t)(vw >> 16));

  float kmin, kstep, vmin, vstep;
  row_stats<D>(k0, k1, active, kmin, kstep);
  row_stats<D>(v0, v1, active, vmin, vstep);

  uint8_t kb, vb;
  quantize_pair<D>(k0, k1, kmin, kstep, kb);
  quantize_pair<D>(v0, v1, vmin, vstep, vb);

  if (!valid) return;
  uint8_t* dst = cache + (slot * KV + h) * (int64_t)SLOT;
  if (active) {
    dst[lane] = kb;
    dst[HALF + lane] = vb;
  }
  if (lane == 0) {
    const uint32_t r0 = (uint32_t)f2h(kmin) | ((uint32_t)f2h(kstep) << 16);
    const uint32_t r1 = (uint32_t)f2h(vmin) | ((uint32_t)f2h(vstep) << 16);
    *reinterpret_cast<uint2*>(dst + D) = make_uint2(r0, r1);   // slot base is 8-byte aligned
  }
}

}  // namespace

int launch_quantize_store(const void* key, int64_t key_stride, const void* value,
                          int64_t value_stride, void* cache, int64_t num_slots,
                          const int64_t* slot_mapping, int64_t N, int KV, int D,
                          hipStream_t stream) {
  if (N == 0) return SLMT_OK;
  const int64_t rows = N * KV;
  const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  if (blocks > 0x7fffffffLL) return fail(SLMT_ERR_UNSUPPORTED, "store: too many tokens for one launch");
  const dim3 grid((unsigned)blocks), block(64 * kRowsPerBlock);
  auto k = reinterpret_cast<const uint16_t*>(key);
  auto v = reinterpret_cast<const uint16_t*>(value);
  auto c = reinterpret_cast<uint8_t*>(cache);
  switch (D) {
    case 64:
      hipLaunchKernelGGL(quantize_store_kernel<64>, grid, block, 0, stream, k, key_stride, v,
                         value_stride, c, num_slots, slot_mapping, N, KV);
      break;
    case 80:
      hipLaunchKernelGGL(quantize_store_kernel<80>, grid, block, 0, stream, k, key_stride, v,
                         value_stride, c, num_slots, slot_mapping, N, KV);
      break;
    case 128:
      hipLaunchKernelGGL(quantize_store_kernel<128>, grid, block, 0, stream, k, key_stride, v,
                         value_stride, c, num_slots, slot_mapping, N, KV);
      break;
    default:
      return fail(SLMT_ERR_INVALID, "store: head_dim must be 64/80/128, got " + std::to_string(D));
  }
  return check_launch("store");
}

}  // namespace slmt
