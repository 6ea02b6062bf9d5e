// Fused 4-bit KV dequant + decode attention for gfx950 (kernel template).
//
// One kernel template serves every attention entry point of the reference's
// kernels/kv_dequant.py:
//   SRC_PAGED   paged per-token min/step cache [nb, bs, KV, D+8]
//               (kernels/kv_dequant_kernels.cuh:671-801, batched here)
//   SRC_TOKEN   contiguous per-token buffers (kernels/kv_dequant_kernels.cuh:528-655)
//   SRC_CHANNEL contiguous per-channel buffers, decode and causal prefill
//               (kernels/kv_dequant_kernels.cuh:113-275, 293-502)
//
// Design (GEMV-shaped and bandwidth-bound; no MFMA):
// * Work split: the tokens of all sequences are cut into 16-token tiles; the
//   concatenated tile list is divided evenly over W workgroups ("stream-K").
//   A workgroup walks its tile range, which may cover the end of one
//   sequence, whole sequences and the start of another.  A sequence split
//   over several workgroups is merged by the last workgroup to finish its
//   piece (log-sum-exp merge of (m, l, o) partials; arrival counter per
//   sequence), so one launch produces the final output.
// * Staging: each tile (16 tokens x the workgroup's KV heads) is copied into
//   LDS with coalesced 8-byte loads, double-buffered; the next tile's loads
//   are in flight (in registers) while the current tile is computed.  Tile
//   barriers fence LDS only, so those loads stay in flight across them.
// * QK (lane = token p x query head g of the wave's 4 heads): the query is
//   quantized once per sequence to 16-bit fixed point and split into four
//   4-bit limbs; v_dot8_u32_u4 multiplies 8 packed key nibbles by 8 limb
//   nibbles directly, so keys are never unpacked.  q.n = sum_k 16^k dot_k,
//   offset-corrected with the nibble sum; the per-token affine dequant is
//   folded in algebraically: q.K = step * q.n + min * sum(q).
// * Softmax: online, base 2 (log2(e)/sqrt(D) folded into the score scale),
//   per-tile max via DPP row rotations and permlane16/32 swaps.
// * PV (lane = packed byte j, i.e. dims 2j and 2j+1, for all 4 heads):
//   v_dot2c_f32_f16 over token pairs.  The 16-bit halves of the operand are
//   the masked nibbles themselves read as fp16 subnormals (n * 2^-24), which
//   the instruction multiplies exactly, so unpacking a V byte pair costs one
//   AND per dim.  Weights are p * step in fp16; accumulation is fp32; the
//   per-token min enters once per token as sum(p * min).
#pragma once

#include "slmt_internal.h"

#include <type_traits>

namespace slmt {
namespace attn {

constexpr int TILE = 16;
constexpr int WSCR = 1024;        // per-wave LDS scratch bytes (query limbs / weights)
constexpr int MAX_THREADS = 512;   // 8 waves: up to 256 VGPRs per wave
constexpr int MAXP = 5;           // 8-byte chunks prefetched per thread

__device__ __forceinline__ float readlane_f(float x, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

__device__ __forceinline__ float fdot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
}

// Workgroup barrier that orders LDS only: global loads issued before it stay
// in flight (a full __syncthreads would wait for them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// Orders this wave's LDS writes before its later LDS reads by other lanes.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

__device__ __forceinline__ int seq_len_of(const AttnParams& p, int b) {
  if (b >= p.B) return 0;
  int L = p.seq_lens ? p.seq_lens[b] : (p.causal_rows ? min(p.fixed_len, b + 1) : p.fixed_len);
  return L < 0 ? 0 : L;
}
__device__ __forceinline__ int tiles_of(int L) { return (L + TILE - 1) / TILE; }

// First tile of workgroup w when T tiles are split over Weff workgroups.
__device__ __forceinline__ int range_start(int w, int T, int Weff) {
  return (int)(((long long)w * T) / Weff);
}
// Workgroup whose range holds tile t.
__device__ __forceinline__ int range_owner(int t, int T, int Weff) {
  return (int)((((long long)t + 1) * Weff - 1) / T);
}

struct Cursor {
  int b, tb, Tb, Lb, Pb;   // sequence, tile in sequence, tiles/length of b, first global tile of b
};

__device__ __forceinline__ void cursor_next(const AttnParams& p, Cursor& c) {
  c.tb++;
  if (c.tb >= c.Tb) {
    c.Pb += c.Tb;
    c.tb = 0;
    do {
      c.b++;
      c.Lb = seq_len_of(p, c.b);
      c.Tb = tiles_of(c.Lb);
    } while (c.Tb == 0 && c.b < p.B);
  }
}

__device__ __forceinline__ int64_t block_of(const AttnParams& p, int b, int idx) {
  if (p.bt64) return reinterpret_cast<const int64_t*>(p.block_tables)[(int64_t)b * p.bt_stride + idx];
  return reinterpret_cast<const int32_t*>(p.block_tables)[(int64_t)b * p.bt_stride + idx];
}

// Tile loader: chunk c of a tile is 8 bytes; a thread owns chunks tid + k*NT.
// The first MAXP chunks of a thread are prefetched into registers; further
// chunks (very wide rows) are copied at commit time.
template <int D, int MODE>
struct Loader {
  static constexpr int SLOT = D + 8;
  static constexpr int PP = D / 8 + (MODE == SRC_TOKEN ? 1 : 0);   // pieces per (token, kv) in contiguous modes
  uint2 reg[MAXP];
  int dst[MAXP];

  __device__ static int chunks_per_row(int nkv) {
    if constexpr (MODE == SRC_PAGED) return nkv * SLOT / 8;
    else return nkv * PP;
  }

  __device__ static uint2 fetch(const AttnParams& p, int c, int cpr, int row_lds, int kv_lo, int b,
                                int tok0, int Lb, int& dst_off, bool& ok) {
    const int r = c / cpr;
    const int ci = c - r * cpr;
    const int tok = tok0 + r;
    ok = tok < Lb;
    uint2 v = make_uint2(0u, 0u);
    if constexpr (MODE == SRC_PAGED) {
      dst_off = r * row_lds + ci * 8;
      if (ok) {
        int64_t blk, pos;
        if (p.block_shift >= 0) {
          blk = tok >> p.block_shift;
          pos = tok & (p.block_size - 1);
        } else {
          blk = tok / p.block_size;
          pos = tok - blk * p.block_size;
        }
        const int64_t phys = block_of(p, b, (int)blk);
        const uint8_t* src = p.cache + ((phys * p.block_size + pos) * p.cache_kv + kv_lo) * (int64_t)SLOT +
                             (int64_t)ci * 8;
        v = *reinterpret_cast<const uint2*>(src);
      }
    } else {
      const int kvl = ci / PP;
      const int i = ci - kvl * PP;
      const int64_t rowi = (int64_t)(kv_lo + kvl) * p.s_rows + tok;
      if (i < D / 16) {
        dst_off = r * row_lds + kvl * SLOT + i * 8;
        if (ok) v = *reinterpret_cast<const uint2*>(p.kp + rowi * (D / 2) + i * 8);
      } else if (i < D / 8) {
        dst_off = r * row_lds + kvl * SLOT + D / 2 + (i - D / 16) * 8;
        if (ok) v = *reinterpret_cast<const uint2*>(p.vp + rowi * (D / 2) + (i - D / 16) * 8);
      } else {
        dst_off = r * row_lds + kvl * SLOT + D;
        if (ok) {
          v.x = (uint32_t)p.kr0[rowi] | ((uint32_t)p.kr1[rowi] << 16);
          v.y = (uint32_t)p.vr0[rowi] | ((uint32_t)p.vr1[rowi] << 16);
        }
      }
    }
    return v;
  }

  __device__ void issue(const AttnParams& p, int total, int cpr, int row_lds, int kv_lo, int b, int tok0,
                        int Lb) {
#pragma unroll
    for (int k = 0; k < MAXP; ++k) {
      const int c = threadIdx.x + k * blockDim.x;
      dst[k] = -1;
      if (c < total) {
        bool ok;
        int off;
        reg[k] = fetch(p, c, cpr, row_lds, kv_lo, b, tok0, Lb, off, ok);
        dst[k] = ok ? off : -1;
      }
    }
  }

  __device__ void commit(const AttnParams& p, uint8_t* stage, int total, int cpr, int row_lds, int kv_lo,
                         int b, int tok0, int Lb) {
#pragma unroll
    for (int k = 0; k < MAXP; ++k)
      if (dst[k] >= 0) *reinterpret_cast<uint2*>(stage + dst[k]) = reg[k];
    for (int c = threadIdx.x + MAXP * blockDim.x; c < total; c += blockDim.x) {
      bool ok;
      int off;
      const uint2 v = fetch(p, c, cpr, row_lds, kv_lo, b, tok0, Lb, off, ok);
      if (ok) *reinterpret_cast<uint2*>(stage + off) = v;
    }
  }
};

// Paged fast path (block_size a multiple of 16 and the workgroup covering
// every KV head of the cache row): a tile is one contiguous byte range of the
// cache, so chunk k of a thread is at tile_base + (tid + k*NT) * 8.  Rows past
// the sequence end are still inside the tile's block and are loaded; the
// compute masks them.
template <int D>
struct FastLoader {
  uint2 reg[MAXP];
  int dst[MAXP];    // LDS offset, or -1 when the thread has no k-th chunk
  const uint2* base = nullptr;   // tile base of the last issue (uniform)
  int total = 0, cpr = 1, row_lds = 0;

  __device__ void init(int total_, int cpr_, int row_lds_) {
    total = total_;
    cpr = cpr_;
    row_lds = row_lds_;
#pragma unroll
    for (int k = 0; k < MAXP; ++k) {
      const int c = threadIdx.x + k * blockDim.x;
      const int r = c / cpr;
      dst[k] = c < total ? r * row_lds + (c - r * cpr) * 8 : -1;
    }
  }

  __device__ static const uint8_t* tile_base(const AttnParams& p, int b, int tok0) {
    const int64_t phys = block_of(p, b, tok0 >> p.block_shift);
    const int64_t slot0 = phys * p.block_size + (tok0 & (p.block_size - 1));
    return p.cache + slot0 * p.cache_kv * (int64_t)(D + 8);
  }

  __device__ void issue(const AttnParams& p, int b, int tok0) {
    base = reinterpret_cast<const uint2*>(tile_base(p, b, tok0));
    const uint2* src = base + threadIdx.x;
#pragma unroll
    for (int k = 0; k < MAXP; ++k)
      if (dst[k] >= 0) reg[k] = src[k * blockDim.x];
  }

  __device__ void commit(uint8_t* stage) {
#pragma unroll
    for (int k = 0; k < MAXP; ++k)
      if (dst[k] >= 0) *reinterpret_cast<uint2*>(stage + dst[k]) = reg[k];
    // chunks beyond MAXP per thread (small workgroups, wide rows): copy now
    for (int c = threadIdx.x + MAXP * blockDim.x; c < total; c += blockDim.x) {
      const int r = c / cpr;
      *reinterpret_cast<uint2*>(stage + r * row_lds + (c - r * cpr) * 8) = base[c];
    }
  }
};

// SHARED: the 4 query heads of every wave read one KV head (G % 4 == 0),
// so a V byte pair is unpacked once for all 4 heads.
// FAST: paged tiles are contiguous (FastLoader); otherwise the general Loader.
template <int D, int MODE, bool SHARED, bool FAST>
__global__ void __launch_bounds__(MAX_THREADS) attention_kernel(const AttnParams p) {
  constexpr int SLOT = D + 8;
  constexpr int KD = D / 8;              // key dwords per token (8 dims each)
  constexpr int VB = D / 2;              // value bytes per token
  constexpr int PH = (D == 64) ? 2 : 1;  // PV token phases (two half-waves for D = 64)
  constexpr int PAIRS = TILE / 2 / PH;   // token pairs per PV lane per tile
  constexpr float kC = 1.4426950408889634f /
                       (D == 64 ? 8.0f : (D == 128 ? 11.313708498984761f : 8.94427190999916f));  // log2(e)/sqrt(D)

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int NT = blockDim.x;
  const int nwaves = NT >> 6;
  const int group = blockIdx.y;
  const int G = p.G;
  const int h0 = group * p.heads_per_group;
  const int h1 = min(p.H, h0 + p.heads_per_group);
  const int kv_lo = h0 / G;
  const int nkv = (h1 - 1) / G - kv_lo + 1;
  const int row_bytes = nkv * SLOT;
  const int row_lds = row_bytes + ((row_bytes & 15) == 0 ? 8 : 0);   // odd multiple of 8: conflict-free K reads
  const int stage_bytes = (TILE * row_lds + 15) & ~15;
  uint8_t* wscr = smem + 2 * stage_bytes + wave * WSCR;
  // misc[0..16]: wave sums of the tile scan; misc[20..22]: broadcast slots
  int* misc = reinterpret_cast<int*>(smem + 2 * stage_bytes + nwaves * WSCR);

  // ---------------------------------------------------------------- schedule
  // Exclusive scan of the per-sequence tile counts (threads own contiguous chunks).
  int T, my_excl, mysum = 0;
  const int chunk = (p.B + NT - 1) / NT;
  const int cb0 = min(p.B, tid * chunk), cb1 = min(p.B, cb0 + chunk);
  for (int b = cb0; b < cb1; ++b) mysum += tiles_of(seq_len_of(p, b));
  {
    int v = mysum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int n = __shfl_up(v, o, 64);
      if (lane >= o) v += n;
    }
    if (lane == 63) misc[wave] = v;
    lds_barrier();
    if (tid == 0) {
      int run = 0;
      for (int w = 0; w < nwaves; ++w) {
        const int t = misc[w];
        misc[w] = run;
        run += t;
      }
      misc[nwaves] = run;
    }
    lds_barrier();
    my_excl = v - mysum + misc[wave];
    T = uniform(misc[nwaves]);
  }
  const int Weff = max(1, min(p.W, (T + p.min_tiles - 1) / p.min_tiles));
  const int wg = blockIdx.x;
  if (wg >= Weff) return;

  // Sequences of length 0 produce zeros (spread over the workgroups).
  for (int b = wg; b < p.B; b += Weff) {
    if (seq_len_of(p, b) == 0) {
      for (int e = tid; e < (h1 - h0) * D; e += NT) {
        const int h = h0 + e / D, d = e % D;
        const int64_t o = (int64_t)b * p.out_seq_stride + (int64_t)h * p.out_head_stride + d;
        if (p.out_f16) reinterpret_cast<uint16_t*>(p.out)[o] = 0;
        else reinterpret_cast<float*>(p.out)[o] = 0.0f;
      }
    }
  }
  if (T == 0) return;
  const int lo = range_start(wg, T, Weff);
  const int hi = range_start(wg + 1, T, Weff);

  // Locate the sequence holding tile lo.
  if (lo >= my_excl && lo < my_excl + mysum) {
    int run = my_excl;
    for (int b = cb0; b < cb1; ++b) {
      const int t = tiles_of(seq_len_of(p, b));
      if (lo < run + t) {
        misc[20] = b;
        misc[21] = run;
        break;
      }
      run += t;
    }
  }
  lds_barrier();
  Cursor cc;
  cc.b = uniform(misc[20]);
  cc.Pb = uniform(misc[21]);
  cc.Lb = seq_len_of(p, cc.b);
  cc.Tb = tiles_of(cc.Lb);
  cc.tb = lo - cc.Pb;
  Cursor lc = cc;                          // loader cursor runs one tile ahead

  const int cpr = Loader<D, MODE>::chunks_per_row(nkv);
  const int total_chunks = TILE * cpr;

  // ---------------------------------------------------------------- lane roles
  const int qp = lane >> 2;                // QK: token within the tile
  const int qg = lane & 3;                 // QK: head slot within the wave
  const int hq = h0 + wave * 4 + qg;
  const bool hvalid = hq < h1;
  const int kvl = hvalid ? hq / G - kv_lo : 0;
  int kvw[4];                              // local kv row of each head of the wave (uniform)
  bool hw[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int h = h0 + wave * 4 + g;
    hw[g] = h < h1;
    kvw[g] = hw[g] ? h / G - kv_lo : 0;
  }
  const int pj = (PH == 2) ? (lane & 31) : lane;        // PV: byte index
  const int pph = (PH == 2) ? (lane >> 5) : 0;          // PV: token phase
  const int jj = min(pj, VB - 1);

  // ---------------------------------------------------------------- prologue loads
  using LoaderT = typename std::conditional<FAST, FastLoader<D>, Loader<D, MODE>>::type;
  LoaderT ld;
  auto issue = [&](const Cursor& c) {
    if constexpr (FAST) ld.issue(p, c.b, c.tb * TILE);
    else ld.issue(p, total_chunks, cpr, row_lds, kv_lo, c.b, c.tb * TILE, c.Lb);
  };
  auto commit = [&](const Cursor& c, uint8_t* stage) {
    if constexpr (FAST) ld.commit(stage);
    else ld.commit(p, stage, total_chunks, cpr, row_lds, kv_lo, c.b, c.tb * TILE, c.Lb);
  };
  if constexpr (FAST) ld.init(total_chunks, cpr, row_lds);
  issue(lc);
  commit(lc, smem);
  if (lo + 1 < hi) {
    cursor_next(p, lc);
    issue(lc);
  }
  lds_barrier();

  // per-segment state
  uint32_t ql[KD][4];
  float qa = 0.f, qb = 0.f;
  float m_run = -INFINITY, l_run = 0.f, vmt = 0.f;
  float acc[4][2];
  int seg_first_tile = lo;                 // global index of the segment's first tile

  for (int t = lo; t < hi; ++t) {
    const int buf = (t - lo) & 1;
    const uint8_t* S = smem + buf * stage_bytes;
    const bool seg_start = (t == lo) || (cc.tb == 0);
    const bool seg_end = (t == hi - 1) || (cc.tb == cc.Tb - 1);

    // ------------------------------------------------------------ new sequence: query limbs
    if (seg_start) {
      seg_first_tile = t;
      m_run = -INFINITY;
      l_run = 0.f;
      vmt = 0.f;
#pragma unroll
      for (int g = 0; g < 4; ++g) acc[g][0] = acc[g][1] = 0.f;
      float qv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) qv[i] = 0.f;
      const bool dvalid = hvalid && (qp * 8 < D);
      float zsum = 0.f;
      float zv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) zv[i] = 0.f;
      if (dvalid) {
        const uint16_t* qrow = p.q + (int64_t)cc.b * p.q_seq_stride + (int64_t)hq * p.q_head_stride + qp * 8;
        const uint4 w = *reinterpret_cast<const uint4*>(qrow);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          qv[2 * i] = h2f((uint16_t)(ws[i] & 0xffffu));
          qv[2 * i + 1] = h2f((uint16_t)(ws[i] >> 16));
        }
        if constexpr (MODE == SRC_CHANNEL) {
          if (p.use_quant) {
            const int64_t kvg = kv_lo + kvl;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              qv[i] *= h2f(p.kr0[kvg * D + qp * 8 + i]);          // q' = q * k_scale
              zv[i] = h2f(p.kr1[kvg * D + qp * 8 + i]);           // k_zero
            }
          }
        }
      }
      float amax = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(qv[i]));
      amax = red16_max(amax);
      const float sq = amax > 0.f ? 32767.0f / amax : 1.0f;
      // The score is computed exactly for the quantized query qi/sq: both the
      // nibble dot and the ruler terms (sum q, sum q*zero) use qi, so the
      // quantization error enters as sum(dq * K) with K the dequantized key.
      uint32_t limb[4] = {0u, 0u, 0u, 0u};
      int isum = 0;
      float qzsum = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int qi = (int)__builtin_rintf(qv[i] * sq);
        qi = max(-32767, min(32767, qi));
        isum += qi;
        if constexpr (MODE == SRC_CHANNEL) qzsum += (float)qi * zv[i];
        const uint32_t qu = (uint32_t)(qi + 32768);
#pragma unroll
        for (int k = 0; k < 4; ++k) limb[k] |= ((qu >> (4 * k)) & 15u) << (4 * i);
      }
      const float qsum = red16_sum((float)isum) / sq;     // |sum qi| < 2^24: exact
      if constexpr (MODE == SRC_CHANNEL) zsum = red16_sum(qzsum) / sq;
      uint32_t* wl = reinterpret_cast<uint32_t*>(wscr);
      wave_lds_sync();                     // previous tile's weight reads are done
      if (qp < KD) {
#pragma unroll
        for (int k = 0; k < 4; ++k) wl[(qg * 4 + k) * 16 + qp] = limb[k];
      }
      wave_lds_sync();
#pragma unroll
      for (int kd = 0; kd < KD; ++kd)
#pragma unroll
        for (int k = 0; k < 4; ++k) ql[kd][k] = wl[(qg * 4 + k) * 16 + kd];
      qa = kC / sq;
      if constexpr (MODE == SRC_CHANNEL) qb = -kC * zsum;
      else qb = kC * qsum;
    }

    // ------------------------------------------------------------ QK
    const int tok0 = cc.tb * TILE;
    const uint8_t* kb = S + qp * row_lds + kvl * SLOT;
    uint32_t a0 = 0, a1 = 0, a2 = 0, a3 = 0, sn = 0;
#pragma unroll
    for (int j = 0; j < KD / 2; ++j) {
      const uint2 w = *reinterpret_cast<const uint2*>(kb + 8 * j);
      a0 = __builtin_amdgcn_udot8(w.x, ql[2 * j][0], a0, false);
      a1 = __builtin_amdgcn_udot8(w.x, ql[2 * j][1], a1, false);
      a2 = __builtin_amdgcn_udot8(w.x, ql[2 * j][2], a2, false);
      a3 = __builtin_amdgcn_udot8(w.x, ql[2 * j][3], a3, false);
      a0 = __builtin_amdgcn_udot8(w.y, ql[2 * j + 1][0], a0, false);
      a1 = __builtin_amdgcn_udot8(w.y, ql[2 * j + 1][1], a1, false);
      a2 = __builtin_amdgcn_udot8(w.y, ql[2 * j + 1][2], a2, false);
      a3 = __builtin_amdgcn_udot8(w.y, ql[2 * j + 1][3], a3, false);
      sn = __builtin_amdgcn_udot8(w.x, 0x11111111u, sn, false);
      sn = __builtin_amdgcn_udot8(w.y, 0x11111111u, sn, false);
    }
    const int iacc = (int)(a0 + (a1 << 4) + (a2 << 8) + (a3 << 12)) - (int)(sn << 15);
    const float x = (float)iacc;                 // = S_q * (q . n)
    const bool tvalid = hvalid && (tok0 + qp < cc.Lb);
    float s2, wv, vmin = 0.f, vstep = 0.f;
    if constexpr (MODE == SRC_CHANNEL) {
      s2 = x * qa + qb;
    } else {
      const uint2 rr = *reinterpret_cast<const uint2*>(kb + D);
      const float kmin = h2f((uint16_t)(rr.x & 0xffffu));
      const float kstep = h2f((uint16_t)(rr.x >> 16));
      vmin = h2f((uint16_t)(rr.y & 0xffffu));
      vstep = h2f((uint16_t)(rr.y >> 16));
      s2 = (x * qa) * kstep + kmin * qb;
    }
    s2 = tvalid ? s2 : -INFINITY;
    const float tmax = red16_max(s2);
    const float m_new = fmaxf(m_run, tmax);
    const float msafe = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - msafe);
    const float pr = __builtin_amdgcn_exp2f(s2 - msafe);
    l_run = l_run * alpha + pr;
    if constexpr (MODE == SRC_CHANNEL) {
      wv = pr;
    } else {
      wv = tvalid ? pr * vstep : 0.f;
      vmt = vmt * alpha + (tvalid ? pr * vmin : 0.f);
    }
    m_run = m_new;
    // weights as fp16 pairs: wscr[pair][head] = (w(2i), w(2i+1))
    wave_lds_sync();                     // limb reads of this wave are done
    reinterpret_cast<uint16_t*>(wscr)[((qp >> 1) * 4 + qg) * 2 + (qp & 1)] = f2h(wv);
    // rescale the PV accumulators by each head's alpha (uniform per head)
    float al[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) al[g] = readlane_f(alpha, g);
    if (al[0] != 1.f || al[1] != 1.f || al[2] != 1.f || al[3] != 1.f) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        acc[g][0] *= al[g];
        acc[g][1] *= al[g];
      }
    }
    wave_lds_sync();

    // ------------------------------------------------------------ PV
#pragma unroll
    for (int i = 0; i < PAIRS; ++i) {
      const int pr2 = pph * PAIRS + i;
      const uint4 wq = *reinterpret_cast<const uint4*>(wscr + pr2 * 16);
      if constexpr (SHARED) {
        const uint8_t* vb = S + kvw[0] * SLOT + VB + jj;
        const uint32_t tw = (uint32_t)vb[(2 * pr2) * row_lds] | ((uint32_t)vb[(2 * pr2 + 1) * row_lds] << 16);
        const uint32_t vlo = tw & 0x000F000Fu, vhi = tw & 0x00F000F0u;
        acc[0][0] = fdot2(wq.x, vlo, acc[0][0]);
        acc[0][1] = fdot2(wq.x, vhi, acc[0][1]);
        acc[1][0] = fdot2(wq.y, vlo, acc[1][0]);
        acc[1][1] = fdot2(wq.y, vhi, acc[1][1]);
        acc[2][0] = fdot2(wq.z, vlo, acc[2][0]);
        acc[2][1] = fdot2(wq.z, vhi, acc[2][1]);
        acc[3][0] = fdot2(wq.w, vlo, acc[3][0]);
        acc[3][1] = fdot2(wq.w, vhi, acc[3][1]);
      } else {
        const uint32_t wgs[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint8_t* vb = S + kvw[g] * SLOT + VB + jj;
          const uint32_t tw = (uint32_t)vb[(2 * pr2) * row_lds] | ((uint32_t)vb[(2 * pr2 + 1) * row_lds] << 16);
          acc[g][0] = fdot2(wgs[g], tw & 0x000F000Fu, acc[g][0]);
          acc[g][1] = fdot2(wgs[g], tw & 0x00F000F0u, acc[g][1]);
        }
      }
    }

    // ------------------------------------------------------------ end of a segment
    if (seg_end) {
      const float lt = red16_sum(l_run);
      const float vt = (MODE == SRC_CHANNEL) ? 0.f : red16_sum(vmt);
      float o[4][2];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        o[g][0] = acc[g][0];
        o[g][1] = acc[g][1];
        if constexpr (PH == 2) {
          float a, b2;
          swap32(o[g][0], a, b2);
          o[g][0] = a + b2;
          swap32(o[g][1], a, b2);
          o[g][1] = a + b2;
        }
      }
      const int Pb = cc.Pb, Tb = cc.Tb, b = cc.b;
      const bool complete = (seg_first_tile == Pb) && (t == Pb + Tb - 1);
      const bool writer = (PH == 1 || pph == 0) && pj < VB;
      const int d0 = 2 * pj;
      if (complete) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          if (!hw[g] || !writer) continue;
          const int h = h0 + wave * 4 + g;
          const float L = readlane_f(lt, g);
          const float vg = readlane_f(vt, g);
          const float n0 = o[g][0] * 16777216.0f + vg;   // 2^24: nibble-as-subnormal scale
          const float n1 = o[g][1] * 1048576.0f + vg;    // 2^20: high nibble carried x16
          float r0 = n0 / L, r1 = n1 / L;
          if constexpr (MODE == SRC_CHANNEL) {
            if (p.use_quant) {
              const int64_t kvg = h / G;
              r0 = h2f(p.vr0[kvg * D + d0]) * (r0 - h2f(p.vr1[kvg * D + d0]));
              r1 = h2f(p.vr0[kvg * D + d0 + 1]) * (r1 - h2f(p.vr1[kvg * D + d0 + 1]));
            }
          }
          const int64_t off = (int64_t)b * p.out_seq_stride + (int64_t)h * p.out_head_stride + d0;
          if (p.out_f16) {
            *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(p.out) + off) =
                (uint32_t)f2h(r0) | ((uint32_t)f2h(r1) << 16);
          } else {
            *reinterpret_cast<float2*>(reinterpret_cast<float*>(p.out) + off) = make_float2(r0, r1);
          }
        }
      } else {
        // partial piece: slot 0 when this segment is the workgroup's first, else 1
        const int slot = (seg_first_tile == lo) ? 0 : 1;
        const int64_t pbase = ((int64_t)wg * 2 + slot) * p.H;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          if (!hw[g] || !writer) continue;
          const int h = h0 + wave * 4 + g;
          const float vg = readlane_f(vt, g);
          const float n0 = o[g][0] * 16777216.0f + vg;
          const float n1 = o[g][1] * 1048576.0f + vg;
          *reinterpret_cast<float2*>(p.part_o + (pbase + h) * D + d0) = make_float2(n0, n1);
          if (pj == 0) {
            p.part_ml[(pbase + h) * 2] = readlane_f(m_run, g);
            p.part_ml[(pbase + h) * 2 + 1] = readlane_f(lt, g);
          }
        }
        // arrival: the last piece of sequence b merges all pieces
        const int w_first = range_owner(Pb, T, Weff);
        const int w_last = range_owner(Pb + Tb - 1, T, Weff);
        const int pieces = w_last - w_first + 1;
        // Every wave publishes its own partial stores at agent scope (waits
        // for them and writes back L2) before the arrival is counted: a
        // barrier alone does not wait for other waves' stores, and the merge
        // may run on another XCD.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        __syncthreads();
        if (tid == 0) {
          const int prev = __hip_atomic_fetch_add(p.counters + (int64_t)group * p.B + b, 1, __ATOMIC_ACQ_REL,
                                                  __HIP_MEMORY_SCOPE_AGENT);
          misc[22] = (prev == pieces - 1) ? 1 : 0;
        }
        __syncthreads();
        if (misc[22]) {
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
          const int first_slot = (range_start(w_first, T, Weff) == Pb) ? 0 : 1;
          for (int e = tid; e < (h1 - h0) * D; e += NT) {
            const int h = h0 + e / D, d = e - (e / D) * D;
            float M = -INFINITY;
            for (int w = w_first; w <= w_last; ++w) {
              const int s = (w == w_first) ? first_slot : 0;
              M = fmaxf(M, p.part_ml[(((int64_t)w * 2 + s) * p.H + h) * 2]);
            }
            float Lsum = 0.f, Osum = 0.f;
            for (int w = w_first; w <= w_last; ++w) {
              const int s = (w == w_first) ? first_slot : 0;
              const int64_t base = ((int64_t)w * 2 + s) * p.H + h;
              const float sc = __builtin_amdgcn_exp2f(p.part_ml[base * 2] - M);
              Lsum += sc * p.part_ml[base * 2 + 1];
              Osum += sc * p.part_o[base * D + d];
            }
            float r = Osum / Lsum;
            if constexpr (MODE == SRC_CHANNEL) {
              if (p.use_quant) {
                const int64_t kvg = h / G;
                r = h2f(p.vr0[kvg * D + d]) * (r - h2f(p.vr1[kvg * D + d]));
              }
            }
            const int64_t off = (int64_t)b * p.out_seq_stride + (int64_t)h * p.out_head_stride + d;
            if (p.out_f16) reinterpret_cast<uint16_t*>(p.out)[off] = f2h(r);
            else reinterpret_cast<float*>(p.out)[off] = r;
          }
          if (tid == 0)
            __hip_atomic_store(p.counters + (int64_t)group * p.B + b, 0, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }

    // ------------------------------------------------------------ advance the pipeline
    if (t + 1 < hi) {
      cursor_next(p, cc);
      // tile t+1 is in registers (issued by the loader cursor); commit it
      commit(lc, smem + (buf ^ 1) * stage_bytes);
      if (t + 2 < hi) {
        cursor_next(p, lc);
        issue(lc);
      }
      lds_barrier();
    }
  }
}

// Per-launch dynamic LDS bytes for nkv KV heads per workgroup.
inline size_t lds_bytes_for(int nkv, int D, int waves) {
  const int row = nkv * (D + 8);
  const int row_lds = row + ((row & 15) == 0 ? 8 : 0);
  const size_t stage = ((size_t)TILE * row_lds + 15) & ~(size_t)15;
  return 2 * stage + (size_t)waves * WSCR + 32 * sizeof(int);
}

}  // namespace attn

// Launch one instantiation (defined in the per-mode translation units).
int launch_attention_paged(int D, bool shared, bool fast, const AttnParams& p, dim3 grid, dim3 block,
                           size_t lds, hipStream_t stream);
int launch_attention_contig(int mode, int D, const AttnParams& p, dim3 grid, dim3 block, size_t lds,
                            hipStream_t stream);

}  // namespace slmt
