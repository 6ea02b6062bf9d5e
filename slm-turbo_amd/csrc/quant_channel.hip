// Per-channel asymmetric 4-bit quantizer of the standalone path, on the GPU.
//
// The reference runs this as host-side torch code on fp16 tensors
// (compute_scale_zero / quantize_tensor, kernels/benchmark/benchmark.py:26-56):
// every op produces an fp16 result, i.e. it is evaluated in fp32 and rounded
// to nearest-even fp16.  fp32 carries >= 2*11+2 significand bits, so
// fp16(fp32(a op b)) is the correctly rounded fp16 result and this kernel
// reproduces torch's bytes exactly.  Reductions follow torch.min/torch.max
// (a NaN anywhere in a channel makes the channel's min/max NaN).
//
// Layout: one workgroup per (kv head, 64-channel slice); 4 waves stride over
// the sequence so each wave reads 64 consecutive fp16 (128 B) per row.
#include "slmt_internal.h"

namespace slmt {

namespace {

constexpr int kCols = 64;     // channels per workgroup
constexpr int kPhases = 4;    // waves striding over S

__device__ __forceinline__ float r16(float x) { return h2f(f2h(x)); }  // round to fp16

__device__ __forceinline__ float nan_min(float a, float b) {  // torch.min semantics
  return (a != a || b != b) ? __builtin_nanf("") : fminf(a, b);
}
__device__ __forceinline__ float nan_max(float a, float b) {
  return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b);
}
__device__ __forceinline__ float clamp_keep_nan(float x, float lo, float hi) {  // torch.clamp
  return (x != x) ? x : fminf(fmaxf(x, lo), hi);
}

__global__ void __launch_bounds__(kCols * kPhases)
quantize_per_channel_kernel(const uint16_t* __restrict__ x, int S, int D,
                            uint8_t* __restrict__ packed, uint16_t* __restrict__ scale_out,
                            uint16_t* __restrict__ zero_out) {
#pragma clang fp contract(off)
  __shared__ float s_min[kPhases][kCols], s_max[kPhases][kCols];
  __shared__ float s_scale[kCols], s_zero[kCols];
  const int kv = blockIdx.x;
  const int c0 = blockIdx.y * kCols;
  const int col = threadIdx.x & (kCols - 1);
  const int ph = threadIdx.x / kCols;
  const int d = c0 + col;
  const bool dv = d < D;
  const uint16_t* base = x + (int64_t)kv * S * D;

  float mn = INFINITY, mx = -INFINITY;
  if (dv) {
    for (int s = ph; s < S; s += kPhases) {
      const float v = h2f(base[(int64_t)s * D + d]);
      mn = nan_min(mn, v);
      mx = nan_max(mx, v);
    }
  }
  s_min[ph][col] = mn;
  s_max[ph][col] = mx;
  __syncthreads();
  if (ph == 0) {
    for (int k = 1; k < kPhases; ++k) {
      mn = nan_min(mn, s_min[k][col]);
      mx = nan_max(mx, s_max[k][col]);
    }
    // scale = (max - min) / 15 ; zero = 0 - round(min / scale)   (fp16 after each op)
    const float scale_raw = r16(r16(mx - mn) / 15.0f);
    const float zero_raw = r16(0.0f - __builtin_rintf(r16(mn / scale_raw)));
    const bool is_const = (mx == mn);
    const float sc = is_const ? 1.0f : scale_raw;
    const float zp = clamp_keep_nan(is_const ? 0.0f : zero_raw, 0.0f, 15.0f);
    s_scale[col] = sc;
    s_zero[col] = zp;
    if (dv) {
      scale_out[(int64_t)kv * D + d] = f2h(sc);
      zero_out[(int64_t)kv * D + d] = f2h(zp);
    }
  }
  __syncthreads();

  // quantize: q = clamp(round(x / scale) + zero, 0, 15) -> uint8; pack pairs.
  const int pairs = kCols / 2;
  const int pj = threadIdx.x % pairs;           // pair within the slice
  const int rph = threadIdx.x / pairs;          // 8 row phases
  const int rphases = (kCols * kPhases) / pairs;
  const int d0 = c0 + 2 * pj;
  if (d0 < D) {
    const float sc0 = s_scale[2 * pj], sc1 = s_scale[2 * pj + 1];
    const float zp0 = s_zero[2 * pj], zp1 = s_zero[2 * pj + 1];
    uint8_t* prow = packed + (int64_t)kv * S * (D / 2) + d0 / 2;
    for (int s = rph; s < S; s += rphases) {
      const uint32_t w = *reinterpret_cast<const uint32_t*>(base + (int64_t)s * D + d0);
      const float x0 = h2f((uint16_t)(w & 0xffffu)), x1 = h2f((uint16_t)(w >> 16));
      float q0 = clamp_keep_nan(r16(__builtin_rintf(r16(x0 / sc0)) + zp0), 0.0f, 15.0f);
      float q1 = clamp_keep_nan(r16(__builtin_rintf(r16(x1 / sc1)) + zp1), 0.0f, 15.0f);
      const int i0 = (q0 != q0) ? 0 : (int)q0;   // NaN codes (scale underflow) -> 0
      const int i1 = (q1 != q1) ? 0 : (int)q1;
      prow[(int64_t)s * (D / 2)] = (uint8_t)(i0 | (i1 << 4));
    }
  }
}

// Append with fixed rulers (quantize_tensor of the reference,
// kernels/benchmark/benchmark.py:45-56): the same per-pair arithmetic as the
// second half of the kernel above, with the scale and zero point given.  One
// thread per pair of dims (one fp16x2 load, one byte store); the grid's y axis
// is the KV head.
__global__ void __launch_bounds__(256)
quantize_rulers_kernel(const uint16_t* __restrict__ x, int64_t x_head_stride, int64_t x_seq_stride,
                       int S, int D, const uint16_t* __restrict__ scale, const uint16_t* __restrict__ zero,
                       uint8_t* __restrict__ packed, int64_t out_head_stride, int64_t out_seq_stride) {
#pragma clang fp contract(off)
  const int kv = blockIdx.y;
  const int half = D / 2;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)S * half) return;
  const int s = (int)(t / half);
  const int j = (int)(t - (int64_t)s * half);
  const uint32_t w = *reinterpret_cast<const uint32_t*>(x + kv * x_head_stride + s * x_seq_stride + 2 * j);
  const uint32_t sw = *reinterpret_cast<const uint32_t*>(scale + (int64_t)kv * D + 2 * j);
  const uint32_t zw = *reinterpret_cast<const uint32_t*>(zero + (int64_t)kv * D + 2 * j);
  const float x0 = h2f((uint16_t)(w & 0xffffu)), x1 = h2f((uint16_t)(w >> 16));
  const float sc0 = h2f((uint16_t)(sw & 0xffffu)), sc1 = h2f((uint16_t)(sw >> 16));
  const float zp0 = h2f((uint16_t)(zw & 0xffffu)), zp1 = h2f((uint16_t)(zw >> 16));
  // q = clamp(round(x / scale) + zero, 0, 15), an fp16 result after each op
  const float q0 = clamp_keep_nan(r16(__builtin_rintf(r16(x0 / sc0)) + zp0), 0.0f, 15.0f);
  const float q1 = clamp_keep_nan(r16(__builtin_rintf(r16(x1 / sc1)) + zp1), 0.0f, 15.0f);
  const int i0 = (q0 != q0) ? 0 : (int)q0;   // NaN codes -> 0
  const int i1 = (q1 != q1) ? 0 : (int)q1;
  packed[kv * out_head_stride + s * out_seq_stride + j] = (uint8_t)(i0 | (i1 << 4));
}

}  // namespace

int launch_quantize_rulers(const void* x, int64_t x_head_stride, int64_t x_seq_stride, int KV, int S, int D,
                           const void* scale, const void* zero, void* packed, int64_t out_head_stride,
                           int64_t out_seq_stride, hipStream_t stream) {
  if (KV == 0 || S == 0) return SLMT_OK;
  const int64_t items = (int64_t)S * (D / 2);
  const int64_t blocks = (items + 255) / 256;
  if (blocks > 0x7fffffffLL || KV > 65535) return fail(SLMT_ERR_UNSUPPORTED, "quantize_tensor: too large for one launch");
  hipLaunchKernelGGL(quantize_rulers_kernel, dim3((unsigned)blocks, KV), dim3(256), 0, stream,
                     reinterpret_cast<const uint16_t*>(x), x_head_stride, x_seq_stride, S, D,
                     reinterpret_cast<const uint16_t*>(scale), reinterpret_cast<const uint16_t*>(zero),
                     reinterpret_cast<uint8_t*>(packed), out_head_stride, out_seq_stride);
  return check_launch("quantize_tensor");
}

int launch_quantize_per_channel(const void* x, int KV, int S, int D, void* packed,
                                void* scale, void* zero, hipStream_t stream) {
  if (KV == 0) return SLMT_OK;
  const dim3 grid(KV, (D + kCols - 1) / kCols), block(kCols * kPhases);
  hipLaunchKernelGGL(quantize_per_channel_kernel, grid, block, 0, stream,
                     reinterpret_cast<const uint16_t*>(x), S, D,
                     reinterpret_cast<uint8_t*>(packed), reinterpret_cast<uint16_t*>(scale),
                     reinterpret_cast<uint16_t*>(zero));
  return check_launch("quantize_per_channel");
}

}  // namespace slmt
