// Batched paged 4-bit decode attention for head_dim 64 or 128 with 4 or 8
// query heads per KV head: the "whole-row" kernel (reference kernel it replaces:
// kv_dequant_decode_per_token_paged_kernel, kernels/kv_dequant_kernels.cuh:671-801,
// batched over the whole decode step instead of launched per request).
//
// A workgroup owns NKV consecutive KV heads (a 16-byte aligned sub-row of every
// cache row, NKV * (D + 8) bytes) and their 4*WPK query heads each, one wave per 4
// query heads.  Tiles are TT tokens (64, or 32 where a wave's share of a
// 64-token tile would cross a paged block).  Work is split stream-K over the
// concatenated tile list of all sequences, exactly as in attention_kernel.h;
// split sequences leave (m, l, o) partials that merge_kernel, launched next on
// the same stream, combines.
//
// Staging: the workgroup copies each tile with 16-byte direct loads
// (global_load_lds_dwordx4, no VGPRs) into a 2-stage LDS ring, two tiles
// ahead of the one being computed; wave w copies the TT/WAVES consecutive rows
// starting at row w*TT/WAVES, which lie in one paged block.  Every lane chooses
// its source unit, so the staged rows get an odd number of 16-byte units (the
// pad unit re-reads the row's last unit): the 16 rows that the QK lanes read
// at once then fall in 16 different bank groups.  Two barriers per tile: one
// publishes the stage, one releases it for the tile after next.
//
// QK (lane = token p of 16 x key quarter c of 4; TT/16 rounds per tile): the
// fp16 query is used exactly as given (scaled by a power of two).  Each key
// dword becomes four fp16 pairs of subnormal integer codes with four masks,
// and v_dot2c_f32_f16 multiplies them exactly by the matching query pairs
// with fp32 accumulation (key_pairs / query_pairs in attention_kernel.h).
// Each lane dots its quarter of the key with all 4 heads; a reduce-scatter
// over the quad leaves head c's dot in lane c.  q.K = step * q.n + min * sum(q).
//
// Weights: P.V multiplies the codes by the fp16 weight w = fp16(p * step);
// the softmax sums use the probability that w stands for, w / step, so the
// output is an exact weighted mean of the dequantized rows whatever the
// rounding of w (rows past a sequence's end get weight 0 and rulers 0).
//
// PV (lane = V dword column c of 16 x token group g of 4): group g takes the
// tokens 16m + 4g .. 16m + 4g + 3 of each 16-token round m.  The groups' rows
// are 4 apart, and 4 rows of an odd number of units are 16 banks apart, so
// each half-wave's two groups read disjoint banks.  Two tokens' bytes k are
// packed into one dword (one v_perm_b32) and read as an fp16 pair of
// subnormals, (lo + 16 hi) * 2^-24, which v_dot2c_f32_f16 multiplies exactly
// with the fp16 weights p * step; a second product with the low nibbles alone
// (one AND) separates the two dims.  The per-token min enters once per token
// as sum(p * min).  The 4 groups' partial sums are added at the end of a
// segment.  PV of a tile runs one iteration after its QK, from V words read
// into registers with the tile's keys.
//
// Weights never go through LDS: the 16 QK lanes of a row hold the weights of
// exactly the tokens that the PV lanes of the same row need.  A DPP move packs
// the fp16 weights of tokens p and p+1 into one dword (lane of token p), and
// every PV product reads its weight pair from the source lane of its row with
// a row_newbcast DPP operand.
#include "attention_kernel.h"

#include <hip/hip_ext.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <type_traits>

namespace slmt {
namespace rows {

using namespace attn;

template <int D, int NKV, int WPK, int TT>
struct Shape {
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static_assert(NKV % 2 == 0, "sub-rows must be a whole number of 16-byte units");
  static_assert(TT % 16 == 0, "tiles of whole QK rounds");
  static constexpr int SLOT = D + 8;            // bytes of one KV head in a cache row
  static constexpr int DQ = D / 32;             // key dwords per QK quarter = V bytes per PV lane
  static constexpr int NS = 2;                  // LDS ring stages
  static constexpr int WAVES = NKV * WPK;
  static constexpr int THREADS = WAVES * 64;
  static constexpr int UPR = NKV * SLOT / 16;   // 16-byte units of a sub-row
  static constexpr int RP = UPR | 1;            // units of a staged row
  static constexpr int RSTRIDE = RP * 16;
  static constexpr int RW = TT / WAVES;         // rows copied per wave
  static_assert(TT % WAVES == 0 && RW <= 16 && 16 % RW == 0, "a wave's rows must lie in one block");
  static constexpr int WUNITS = RW * RP;
  static constexpr int NOPS = (WUNITS + 63) / 64;
  static constexpr int LAST = WUNITS - 64 * (NOPS - 1);   // lanes of the wave's last load
  static constexpr int ROUNDS = TT / 16;                  // QK rounds of 16 tokens
  static constexpr int NP = TT / 8;                       // PV token pairs per lane
  static constexpr int STAGE = TT * RSTRIDE;
  static constexpr int QOFF = NS * STAGE;                 // one 1 KB query slot per wave
  static constexpr int WOFF = QOFF + WAVES * 1024;        // per-wave query-pair table
  static constexpr int MOFF = WOFF + WAVES * 1024;        // misc ints
  static constexpr int STASH = 256;                       // sequence lengths kept in LDS
  static constexpr int SOFF = MOFF + 32 * 4;
  static constexpr int LDS = SOFF + STASH * 4;
  static_assert(LDS <= 160 * 1024, "LDS ring too large");
};

// log2(e) / sqrt(D)
template <int D>
constexpr float kC = D == 128 ? 1.4426950408889634f / 11.313708498984761f : 1.4426950408889634f / 8.0f;

// One token pair's PV products: al[k][h] += dot(w of lane 8*I + h of this
// row, lo[k]) and af[k][h] += dot(that w, fu[k]) for bytes k and heads h, 32
// independent products behind one wait for the DPP read of w (DPP reads of a
// register written by the previous VALU instruction need two wait states,
// which the compiler does not insert for inline asm).
template <int I>
__device__ __forceinline__ void pv_pair_bcast(float (&al)[4][4], float (&af)[4][4], uint32_t w, const uint32_t (&lo)[4],
                                              const uint32_t (&fu)[4]) {
  asm("s_nop 1\n\t"
      "v_dot2c_f32_f16_dpp %0, %32, %33 row_newbcast:%41 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %16, %32, %37 row_newbcast:%41 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %4, %32, %34 row_newbcast:%41 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %20, %32, %38 row_newbcast:%41 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %8, %32, %35 row_newbcast:%41 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %24, %32, %39 row_newbcast:%41 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %12, %32, %36 row_newbcast:%41 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %28, %32, %40 row_newbcast:%41 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %1, %32, %33 row_newbcast:%42 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %17, %32, %37 row_newbcast:%42 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %5, %32, %34 row_newbcast:%42 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %21, %32, %38 row_newbcast:%42 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %9, %32, %35 row_newbcast:%42 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %25, %32, %39 row_newbcast:%42 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %13, %32, %36 row_newbcast:%42 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %29, %32, %40 row_newbcast:%42 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %2, %32, %33 row_newbcast:%43 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %18, %32, %37 row_newbcast:%43 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %6, %32, %34 row_newbcast:%43 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %22, %32, %38 row_newbcast:%43 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %10, %32, %35 row_newbcast:%43 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %26, %32, %39 row_newbcast:%43 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %14, %32, %36 row_newbcast:%43 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %30, %32, %40 row_newbcast:%43 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %3, %32, %33 row_newbcast:%44 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %19, %32, %37 row_newbcast:%44 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %7, %32, %34 row_newbcast:%44 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %23, %32, %38 row_newbcast:%44 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %11, %32, %35 row_newbcast:%44 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %27, %32, %39 row_newbcast:%44 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %15, %32, %36 row_newbcast:%44 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %31, %32, %40 row_newbcast:%44 row_mask:0xf bank_mask:0xf"
      : "+v"(al[0][0]), "+v"(al[0][1]), "+v"(al[0][2]), "+v"(al[0][3]), "+v"(al[1][0]), "+v"(al[1][1]), "+v"(al[1][2]), "+v"(al[1][3]), "+v"(al[2][0]), "+v"(al[2][1]), "+v"(al[2][2]), "+v"(al[2][3]), "+v"(al[3][0]), "+v"(al[3][1]), "+v"(al[3][2]), "+v"(al[3][3]), "+v"(af[0][0]), "+v"(af[0][1]), "+v"(af[0][2]), "+v"(af[0][3]), "+v"(af[1][0]), "+v"(af[1][1]), "+v"(af[1][2]), "+v"(af[1][3]), "+v"(af[2][0]), "+v"(af[2][1]), "+v"(af[2][2]), "+v"(af[2][3]), "+v"(af[3][0]), "+v"(af[3][1]), "+v"(af[3][2]), "+v"(af[3][3])
      : "v"(w), "v"(lo[0]), "v"(lo[1]), "v"(lo[2]), "v"(lo[3]), "v"(fu[0]), "v"(fu[1]), "v"(fu[2]), "v"(fu[3]),
        "n"(8 * I), "n"(8 * I + 1), "n"(8 * I + 2), "n"(8 * I + 3));
}

// The same for head_dim 64, where a PV lane holds 2 V bytes per token: 16
// products.
template <int I>
__device__ __forceinline__ void pv_pair_bcast(float (&al)[2][4], float (&af)[2][4], uint32_t w, const uint32_t (&lo)[2],
                                              const uint32_t (&fu)[2]) {
  asm("s_nop 1\n\t"
      "v_dot2c_f32_f16_dpp %0, %16, %17 row_newbcast:%21 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %8, %16, %19 row_newbcast:%21 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %4, %16, %18 row_newbcast:%21 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %12, %16, %20 row_newbcast:%21 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %1, %16, %17 row_newbcast:%22 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %9, %16, %19 row_newbcast:%22 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %5, %16, %18 row_newbcast:%22 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %13, %16, %20 row_newbcast:%22 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %2, %16, %17 row_newbcast:%23 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %10, %16, %19 row_newbcast:%23 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %6, %16, %18 row_newbcast:%23 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %14, %16, %20 row_newbcast:%23 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %3, %16, %17 row_newbcast:%24 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %11, %16, %19 row_newbcast:%24 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %7, %16, %18 row_newbcast:%24 row_mask:0xf bank_mask:0xf\n\t"
      "v_dot2c_f32_f16_dpp %15, %16, %20 row_newbcast:%24 row_mask:0xf bank_mask:0xf"
      : "+v"(al[0][0]), "+v"(al[0][1]), "+v"(al[0][2]), "+v"(al[0][3]), "+v"(al[1][0]), "+v"(al[1][1]), "+v"(al[1][2]), "+v"(al[1][3]), "+v"(af[0][0]), "+v"(af[0][1]), "+v"(af[0][2]), "+v"(af[0][3]), "+v"(af[1][0]), "+v"(af[1][1]), "+v"(af[1][2]), "+v"(af[1][3])
      : "v"(w), "v"(lo[0]), "v"(lo[1]), "v"(fu[0]), "v"(fu[1]),
        "n"(8 * I), "n"(8 * I + 1), "n"(8 * I + 2), "n"(8 * I + 3));
}

// Sum of x over the 4 rows of 16 lanes (lanes l, l + 16, l + 32, l + 48).
__device__ __forceinline__ float rows_sum(float x) {
  float a, b;
  swap16(x, a, b);
  x = a + b;
  swap32(x, a, b);
  return a + b;
}

// x *= s in x's own register: a conditionally rescaled accumulator then stays
// in one register on both paths of the branch (no copies on the common path).
__device__ __forceinline__ void scale_in_place(float& x, float s) {
  asm volatile("v_mul_f32 %0, %1, %0" : "+v"(x) : "s"(s));
}

template <int D, int NKV, int WPK, int TT>
__global__ void __launch_bounds__(NKV * WPK * 64) rows_kernel(const AttnParams p) {
  using S = Shape<D, NKV, WPK, TT>;
  constexpr int SLOT = S::SLOT, DQ = S::DQ;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = uniform(tid >> 6);
  const int group = blockIdx.y;
  const int wg = blockIdx.x;
  const int h0 = group * 4 * S::WAVES, h1 = h0 + 4 * S::WAVES;   // the host checks H % (4 * WAVES) == 0
  const int kv_lo = group * NKV;
  const int kvw = wave / WPK;                                     // the wave's KV head within the group
  const int hw = h0 + 4 * wave;                                   // the wave's first query head
  int* misc = reinterpret_cast<int*>(smem + S::MOFF);
  uint8_t* const wscr = smem + S::WOFF + wave * 1024;

  TileRange rng;
  int* const stash = reinterpret_cast<int*>(smem + S::SOFF);
  if (!schedule_range<TT, D, false>(p, misc, h0, h1, rng, stash, S::STASH)) return;
  const int lo = rng.lo, hi = rng.hi;

  // ---------------------------------------------------------------- loads
  // The wave copies rows rw0 .. rw0+RW-1 of each tile, consecutive rows of one
  // paged block.  Load i moves LDS units 64i .. 64i+63 of its run; lane l unit
  // u = 64i + l = row rw0 + u / RP, column u % RP (the pad column re-reads
  // column UPR-1), at byte (u / RP) * cache_row + a0 + 16 * column from the
  // wave's first row.
  const int cache_row = p.cache_kv * SLOT;
  const int a0 = kv_lo * SLOT;
  const int rw0 = wave * S::RW;
  uint32_t goff[S::NOPS];
#pragma unroll
  for (int i = 0; i < S::NOPS; ++i) {
    const int u = 64 * i + lane;
    const int r = u / S::RP, c = min(u % S::RP, S::UPR - 1);
    goff[i] = u < S::WUNITS ? (uint32_t)(r * cache_row + a0 + c * 16) : 0u;
  }
  const uint32_t lds_smem = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  const uint32_t lds_run = lds_smem + rw0 * S::RSTRIDE;
  // query rows: lane (qp, qg) moves dims 8qp .. 8qp+7 of head hw + qg (head_dim
  // 64: lanes qp >= 8 re-read dims 8(qp - 8) .., which begin() ignores)
  const int qp = lane >> 2, qg = lane & 3;
  const int qd = D == 128 ? qp : (qp & 7);
  const uint32_t qoff = (uint32_t)(((hw + qg) * p.q_head_stride + qd * 8) * 2);

  // Tile descriptors, 64 tiles at a time, lane i for tile dchunk + i: the
  // address of this wave's first row and an info word
  //   sequence << 8 | first tile of the sequence << 7 | last tile << 6 | (valid tokens - 1).
  // Block-table entries are read as their low 32 bits (num_blocks < 2^31).
  const int esh = p.bt64 ? 3 : 2;
  const uint8_t* btab = reinterpret_cast<const uint8_t*>(p.block_tables);
  const int64_t blk_bytes = (int64_t)p.block_size * cache_row;

  uint32_t dlo = 0, dhi = 0;
  int dinfo = 0, dchunk = lo;
  int cb = rng.b, cP = rng.Pb;                  // a sequence at or before the next chunk's first tile
  auto build = [&](int first) {
    // Lane j takes sequence b0 + j: its length (one vector load for the 64
    // sequences) and, by a wave scan, its first tile; then every sequence
    // that overlaps tiles [first, first + 64) hands its tiles to their lanes.
    const int t = first + lane;
    int mb = -1, mtb = 0, mL = 0, mTb = 0;
    int b0 = cb, P0 = cP;
    for (;;) {
      const int bl = b0 + lane;
      const int Ll = bl < S::STASH && bl < p.B ? stash[bl] : seq_len_lane(p, bl);   // 0 past the last sequence
      const int Tl = tiles_of<TT>(Ll);
      int incl = Tl;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int n = __shfl_up(incl, o, 64);
        if (lane >= o) incl += n;
      }
      const int sl = P0 + incl - Tl;
      uint64_t ov = __builtin_amdgcn_ballot_w64(Tl > 0 && sl < first + 64 && sl + Tl > first);
      while (ov) {
        const int j = __builtin_ctzll(ov);
        ov &= ov - 1;
        const int s0 = __builtin_amdgcn_readlane(sl, j), n = __builtin_amdgcn_readlane(Tl, j);
        if (t >= s0 && t < s0 + n) {
          mb = b0 + j;
          mtb = t - s0;
          mL = __builtin_amdgcn_readlane(Ll, j);
          mTb = n;
        }
        cb = b0 + j;
        cP = s0;
      }
      const int total = __builtin_amdgcn_readlane(incl, 63);
      if (P0 + total >= min(first + 64, hi) || b0 + 64 >= p.B) break;
      b0 += 64;
      P0 += total;
    }
    uint64_t base = reinterpret_cast<uint64_t>(p.cache);
    dinfo = 0;
    if (mb >= 0 && t < hi) {
      const int tok0 = mtb * TT;
      const int tok = tok0 + rw0 < mL ? tok0 + rw0 : tok0;     // past the end: any valid block
      const int32_t e =
          *reinterpret_cast<const int32_t*>(btab + (((int64_t)mb * p.bt_stride + (tok >> p.block_shift)) << esh));
      base += (uint64_t)(uint32_t)e * (uint64_t)blk_bytes + (uint64_t)((tok & (p.block_size - 1)) * cache_row);
      dinfo = (mb << 8) | ((mtb == 0) << 7) | ((mtb == mTb - 1) << 6) | (min(TT, mL - tok0) - 1);
    }
    dlo = (uint32_t)base;
    dhi = (uint32_t)(base >> 32);
    dchunk = first;
  };
  // Tile t's rows into ring stage st, in parts: `fetch` reads the tile's
  // descriptor, `loads` issues this wave's loads [k0, k1).
  struct Pending {
    const uint8_t* base;
    uint32_t dst;
    int info;
  };
  auto fetch = [&](int t, int st) -> Pending {
    const int i = t - dchunk;
    Pending d;
    d.base = reinterpret_cast<const uint8_t*>((uint64_t)readlane_u32(dlo, i) | ((uint64_t)readlane_u32(dhi, i) << 32));
    d.info = __builtin_amdgcn_readlane(dinfo, i);
    d.dst = lds_run + st * S::STAGE;
    return d;
  };
  auto loads = [&](const Pending& d, auto k0c, auto k1c) {
    constexpr int k0 = decltype(k0c)::value, k1 = decltype(k1c)::value;
#pragma unroll
    for (int k = k0; k < k1; ++k) {
      if (k < S::NOPS - 1 || S::LAST == 64 || lane < S::LAST) lds_load16(d.base, goff[k], d.dst + k * 1024);
    }
  };
  auto issue = [&](int t, int st) -> int {
    const Pending d = fetch(t, st);
    loads(d, std::integral_constant<int, 0>{}, std::integral_constant<int, S::NOPS>{});
    return d.info;
  };
  // Issues the query rows of sequence b into this wave's query slot.
  const uint32_t qslot = lds_smem + S::QOFF + wave * 1024;
  auto issue_q = [&](int b) { lds_load16(p.q + (int64_t)b * p.q_seq_stride, qoff, qslot); };

  // ---------------------------------------------------------------- per-wave state
  // QK lane (token p, key quarter qc = lane & 3): query pairs of all 4 heads
  // for the lane's DQ key dwords, in the order the lane reads them (head_dim
  // 128: odd quarters read their two 8-byte halves swapped, so the quad
  // covers all 32 banks).  Heads are stored rotated: slot j holds head
  // (qc + j) & 3, so the quad's reduce-scatter needs no per-lane selects.
  uint32_t qpr[4][DQ][4];             // [head slot][dword][pair]
  // Scores are kept as u = step * dot + min * sum(q) * 2^-24 (q.K in units of
  // 2^(24 - e), e the query's scale exponent); qa converts them to base-2
  // logits, so a weight is exp2((u - m_run) * qa) and m_run is the weight
  // reference of the lane's head: the running max of u, or kRefDrop / 2 above
  // a later tile's max when that lies more than kRefDrop base-2 units below it
  // (m_lo = m_run - tu, tu = kRefDrop in units of u; m_top is the running max).
  float qa = 0.f, qb = 0.f, mq = 0.f, m_run = -INFINITY, l_run = 0.f, vmt = 0.f;
  float m_lo = -INFINITY, m_top = -INFINITY, tu = 0.f;
  float accl[DQ][4], accf[DQ][4];     // [byte k][head]: sum w * lo, sum w * (lo + 16 hi), units of 2^-24
  const int pc = lane & 15, pq = lane >> 4;   // PV: V column (DQ bytes), token group

  auto begin = [&](const uint4 w) {
    m_run = m_lo = m_top = -INFINITY;
    l_run = 0.f;
    vmt = 0.f;
#pragma unroll
    for (int k = 0; k < DQ; ++k)
#pragma unroll
      for (int h = 0; h < 4; ++h) accl[k][h] = accf[k][h] = 0.f;
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    const bool qlive = D == 128 || qp < 8;
    float qv[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qv[2 * i] = qlive ? h2f((uint16_t)(ws[i] & 0xffffu)) : 0.f;
      qv[2 * i + 1] = qlive ? h2f((uint16_t)(ws[i] >> 16)) : 0.f;
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(qv[i]));
    amax = red16_max(amax);
    const int ex = query_exponent(amax);
    float qs[8], qsum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      qs[i] = __builtin_amdgcn_ldexpf(qv[i], ex);   // exact
      qsum += qs[i];
    }
    uint32_t pr[4];
    query_pairs(qs, pr);
    qsum = red16_sum(qsum);
    // table of (head, key dword) pairs: word (h * KDW + i) * 4 + k
    constexpr int KDW = D / 8;
    uint32_t* wl = reinterpret_cast<uint32_t*>(wscr);
    wave_lds_sync();                     // earlier table reads of this wave are done
    if (qp < KDW) *reinterpret_cast<uint4*>(wl + (qg * KDW + qp) * 4) = make_uint4(pr[0], pr[1], pr[2], pr[3]);
    wave_lds_sync();
    // key dwords DQ*qc .. DQ*qc+DQ-1 of this lane's quarter, in read order
    const bool swp = qg & 1;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int h = (qg + j) & 3;
#pragma unroll
      for (int d = 0; d < DQ; ++d) {
        const int i = DQ * qg + ((D == 128 && swp) ? (d ^ 2) : d);
        const uint4 v = *reinterpret_cast<const uint4*>(wl + (h * KDW + i) * 4);
        qpr[j][d][0] = v.x;
        qpr[j][d][1] = v.y;
        qpr[j][d][2] = v.z;
        qpr[j][d][3] = v.w;
      }
    }
    qa = __builtin_amdgcn_ldexpf(kC<D>, 24 - ex);
    tu = __builtin_amdgcn_ldexpf(kRefDrop / kC<D>, ex - 24);
    qb = __builtin_amdgcn_ldexpf(qsum, -24);
  };

  // Score u of this lane's token for head qg: the lane's key quarter kq
  // against all 4 heads' query pairs (exact products, fp32 sums), then the
  // quad's partial dots for head qg gathered from the rotated slots with
  // three DPP adds; kr: the token's rulers.
  auto score = [&](const uint32_t (&kq)[DQ], uint2 kr) -> float {
    float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < DQ; ++d) {
      uint32_t P[4];
      key_pairs(kq[d], P);
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) part[j] = fdot2(P[k], qpr[j][d][k], part[j]);
    }
    // lane c: head c lives in slot 0 here, slot 3 of lane c+1, 2 of c+2, 1 of c+3
    // (the empty asm keeps each DPP move next to a two-operand add, which the
    // backend then fuses into one v_add_f32_dpp)
    float z = part[0] + dpp_f<DPP_QUAD_ROT1>(part[3]);
    asm volatile("" : "+v"(z));
    z += dpp_f<DPP_QUAD_XOR2>(part[2]);
    asm volatile("" : "+v"(z));
    z += dpp_f<DPP_QUAD_ROT3>(part[1]);
    const float kmin = h2f((uint16_t)(kr.x & 0xffffu));
    const float kstep = h2f((uint16_t)(kr.x >> 16));
    return __builtin_fmaf(z, kstep, kmin * qb);
  };

  // PV token pairs of this lane's group: pairs P = 8m + 2pq and 8m + 2pq + 1,
  // i.e. tokens 16m + 4pq .. 16m + 4pq + 3, for m = 0 .. TT/16 - 1.
  auto pair_of = [&](int j) { return 8 * (j >> 1) + 2 * pq + (j & 1); };

  // LDS reads of tile data for this lane: its key quarter and rulers of its
  // QK tokens, and its V words (PV, used one iteration later).
  auto read_tile = [&](const uint8_t* Sb, uint32_t (&kq)[S::ROUNDS][DQ], uint2 (&kr)[S::ROUNDS],
                       uint32_t (&xv)[2 * S::NP]) {
    const int sw = (qg & 1) * 8;
#pragma unroll
    for (int r = 0; r < S::ROUNDS; ++r) {
      const uint8_t* kb = Sb + (16 * r + qp) * S::RSTRIDE;
      if constexpr (D == 128) {
        const uint2 k01 = *reinterpret_cast<const uint2*>(kb + 16 * qg + sw);
        const uint2 k23 = *reinterpret_cast<const uint2*>(kb + 16 * qg + 8 - sw);
        kq[r][0] = k01.x;
        kq[r][1] = k01.y;
        kq[r][2] = k23.x;
        kq[r][3] = k23.y;
      } else {
        const uint2 k01 = *reinterpret_cast<const uint2*>(kb + 8 * qg);
        kq[r][0] = k01.x;
        kq[r][1] = k01.y;
      }
      kr[r] = *reinterpret_cast<const uint2*>(kb + D);
    }
    const uint8_t* vb = Sb + D / 2 + DQ * pc;
#pragma unroll
    for (int j = 0; j < S::NP; ++j) {
      const int P = pair_of(j);
      if constexpr (D == 128) {
        xv[2 * j] = *reinterpret_cast<const uint32_t*>(vb + (2 * P) * S::RSTRIDE);
        xv[2 * j + 1] = *reinterpret_cast<const uint32_t*>(vb + (2 * P + 1) * S::RSTRIDE);
      } else {
        xv[2 * j] = *reinterpret_cast<const uint16_t*>(vb + (2 * P) * S::RSTRIDE);
        xv[2 * j + 1] = *reinterpret_cast<const uint16_t*>(vb + (2 * P + 1) * S::RSTRIDE);
      }
    }
  };

  // QK and softmax of one tile.  Its weights w = p * step come back in W:
  // W[r] of the lane of (token 16r + qp, head qg) with qp even holds the fp16
  // pair (w(token), w(token + 1)) of head qg.  Tokens past the sequence end
  // get u = -inf, hence weight exp2(-inf) = 0.
  auto qk_softmax = [&](const uint32_t (&kq)[S::ROUNDS][DQ], const uint2 (&kr)[S::ROUNDS], int nvalid,
                        uint32_t (&W)[S::ROUNDS]) {
    float s2[S::ROUNDS];
#pragma unroll
    for (int r = 0; r < S::ROUNDS; ++r) {
      const float sc = score(kq[r], kr[r]);
      s2[r] = 16 * r + qp < nvalid ? sc : -INFINITY;
    }
    float tl = s2[0];
#pragma unroll
    for (int r = 1; r < S::ROUNDS; ++r) tl = fmaxf(tl, s2[r]);
    // online softmax: the reference per head is only recomputed (and the
    // sums rescaled) when some score of the tile exceeds it, or when some head
    // has no score of the tile within kRefDrop of it
    const uint64_t up = __builtin_amdgcn_ballot_w64(tl > m_run);
    const uint64_t near = __builtin_amdgcn_ballot_w64(tl >= m_lo);
    if (up || some_class4_empty(near)) {
      const float tmax = red16_max(tl);
      const bool grow = tmax > m_run;
      // down to half the threshold above the tile's max (finite: the head
      // has a valid token here), at most kRefFloor below the running max
      const bool drop = !grow && tmax > -INFINITY && tmax < m_lo;
      const float R = grow ? tmax : drop ? fmaxf(__builtin_fmaf(0.5f, tu, tmax), m_top - (kRefFloor / kRefDrop) * tu)
                                         : m_run;
      // 0 when growing from -inf
      const float alpha = grow || drop ? __builtin_amdgcn_exp2f((m_run - R) * qa) : 1.f;
      l_run *= alpha;
      vmt *= alpha;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const float ah = readlane_f(alpha, h);
#pragma unroll
        for (int k = 0; k < DQ; ++k) {
          scale_in_place(accl[k][h], ah);
          scale_in_place(accf[k][h], ah);
        }
      }
      m_top = fmaxf(m_top, tmax);
      m_run = R;
      m_lo = R - tu;
      mq = grow || drop ? R * qa : mq;
    }
#pragma unroll
    for (int r = 0; r < S::ROUNDS; ++r) {
      // m_run > -inf here: token 0 of every tile is valid
      const float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(s2[r], qa, -mq));
      float vmin = h2f((uint16_t)(kr[r].y & 0xffffu));
      float vstep = h2f((uint16_t)(kr[r].y >> 16));
      if (nvalid < TT) {
        // the sequence's last tile: slots past its end may hold anything
        // (a reused block), so their rulers must not reach the sums
        const bool ok = 16 * r + qp < nvalid;
        vmin = ok ? vmin : 0.f;
        vstep = ok ? vstep : 0.f;
      }
      const uint32_t wl = f2h(pr * vstep);
      // P.V applies wl; the sums take the probability it stands for, wl /
      // step.  Steps below 2^-10 keep pr: there the difference moves the
      // output by less than 2^-22 of the token's weight.
      const float pp = vstep >= 0x1p-10f ? h2f((uint16_t)wl) * __builtin_amdgcn_rcpf(vstep) : pr;
      l_run += pp;
      vmt = __builtin_fmaf(pp, vmin, vmt);
      W[r] = wl | (dpp_u<DPP_ROW_SHL4>(wl) << 16);   // token qp + 1 is 4 lanes up
    }
  };

  // PV of one tile from its V words and its weights W.  Pair j (tokens
  // 16m + 4pq + 2i and the next, m = j / 2, i = j % 2) has its weights for
  // head h in W[m] of lane 8i + h of this lane's row.
  auto pv = [&](const uint32_t (&xv)[2 * S::NP], const uint32_t (&W)[S::ROUNDS]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < S::NP; ++j) {
      const uint32_t x0 = xv[2 * j], x1 = xv[2 * j + 1];
      uint32_t lo[DQ], fu[DQ];
#pragma unroll
      for (int k = 0; k < DQ; ++k) {
        // byte k of both tokens at bits 0-7 and 16-23
        fu[k] = __builtin_amdgcn_perm(x1, x0, 0x0C000C00u | ((4u + k) << 16) | (uint32_t)k);
        lo[k] = fu[k] & 0x000F000Fu;
      }
      if (j & 1) pv_pair_bcast<1>(accl, accf, W[j >> 1], lo, fu);
      else pv_pair_bcast<0>(accl, accf, W[j >> 1], lo, fu);
    }
  };

  // End of a segment of sequence b whose first tile is seg_first (a whole
  // sequence when `whole`): add the token groups' sums and write the output
  // or a partial piece.
  auto finish = [&](int b, int seg_first, bool whole, bool last_of_seq) {
    const float lt = red16_sum(l_run);   // lane g: head g
    const float vt = red16_sum(vmt);
    if constexpr (D == 64) {
      // Every accumulator summed over the 4 token groups (rows) in every lane;
      // lane (pc, row pq) then writes byte pq & 1 of its column (dims 4pc +
      // 2(pq & 1), +1) for heads 2(pq >> 1) and 2(pq >> 1) + 1.
      const int kb = pq & 1, hp = pq >> 1;
      float o[2][2];                     // [head 2hp + i][dim]
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        float lo_t[2], fu_t[2], vh[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int h = 2 * hh + i;
          const float l0 = rows_sum(accl[0][h]), l1 = rows_sum(accl[1][h]);
          const float f0 = rows_sum(accf[0][h]), f1 = rows_sum(accf[1][h]);
          lo_t[hh] = kb ? l1 : l0;
          fu_t[hh] = kb ? f1 : f0;
          vh[hh] = readlane_f(vt, h);
        }
        const float lsel = hp ? lo_t[1] : lo_t[0], fsel = hp ? fu_t[1] : fu_t[0], vsel = hp ? vh[1] : vh[0];
        o[i][0] = lsel * 16777216.0f + vsel;             // 2^24: nibble-as-subnormal scale
        o[i][1] = (fsel - lsel) * 1048576.0f + vsel;     // (16 hi) * 2^-24 -> hi
      }
      const int dcol = 4 * pc + 2 * kb;
      if (whole && last_of_seq) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const float l0 = readlane_f(lt, i), l2 = readlane_f(lt, 2 + i);
          const float rL = __builtin_amdgcn_rcpf(hp ? l2 : l0);
          const int h = 2 * hp + i;
          const int64_t off = (int64_t)b * p.out_seq_stride + (int64_t)(hw + h) * p.out_head_stride + dcol;
          if (p.out_f16) {
            *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(p.out) + off) =
                (uint32_t)f2h(o[i][0] * rL) | ((uint32_t)f2h(o[i][1] * rL) << 16);
          } else {
            *reinterpret_cast<float2*>(reinterpret_cast<float*>(p.out) + off) = make_float2(o[i][0] * rL, o[i][1] * rL);
          }
        }
      } else {
        const int slot = (seg_first == lo) ? 0 : 1;
        const int64_t pbase = ((int64_t)wg * 2 + slot) * p.H;
#pragma unroll
        for (int i = 0; i < 2; ++i)
          store_pair_agent(p.part_o + (pbase + hw + 2 * hp + i) * D + dcol, o[i][0], o[i][1]);
        if (lane < 4) store_pair_agent(p.part_ml + (pbase + hw + lane) * 2, m_run * qa, lt);
      }
    } else {
    // Sum every accumulator over the 4 token groups (rows of 16 lanes).  The
    // four values (head h, lo|full, byte k = 0..3) are folded together: two
    // permlane16 swaps and one permlane32 swap leave the total of byte k in
    // row k.  Lane (pc, row pq) then owns dims 8pc + 2pq and 8pc + 2pq + 1.
    float o[4][2];                       // [head][dim 8pc + 2pq + i], un-normalized
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      float r[2];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        float v0 = x ? accf[0][h] : accl[0][h], v1 = x ? accf[1][h] : accl[1][h];
        float v2 = x ? accf[2][h] : accl[2][h], v3 = x ? accf[3][h] : accl[3][h];
        permlane16_swap_pair(v0, v1);    // v0 + v1: rows [b0 r01, b1 r01, b0 r23, b1 r23]
        permlane16_swap_pair(v2, v3);
        float s01 = v0 + v1, s23 = v2 + v3;
        permlane32_swap_pair(s01, s23);  // s01 + s23: row k holds byte k's total
        r[x] = s01 + s23;
      }
      const float vh = readlane_f(vt, h);
      o[h][0] = r[0] * 16777216.0f + vh;            // 2^24: nibble-as-subnormal scale
      o[h][1] = (r[1] - r[0]) * 1048576.0f + vh;    // (16 hi) * 2^-24 -> hi
    }
    const int dcol = 8 * pc + 2 * pq;
    if (whole && last_of_seq) {
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const float rL = __builtin_amdgcn_rcpf(readlane_f(lt, h));
        const int64_t off = (int64_t)b * p.out_seq_stride + (int64_t)(hw + h) * p.out_head_stride + dcol;
        if (p.out_f16) {
          *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(p.out) + off) =
              (uint32_t)f2h(o[h][0] * rL) | ((uint32_t)f2h(o[h][1] * rL) << 16);
        } else {
          *reinterpret_cast<float2*>(reinterpret_cast<float*>(p.out) + off) = make_float2(o[h][0] * rL, o[h][1] * rL);
        }
      }
    } else {
      // partial piece: slot 0 when this segment is the range's first, else 1
      const int slot = (seg_first == lo) ? 0 : 1;
      const int64_t pbase = ((int64_t)wg * 2 + slot) * p.H;
#pragma unroll
      for (int h = 0; h < 4; ++h) store_pair_agent(p.part_o + (pbase + hw + h) * D + dcol, o[h][0], o[h][1]);
      // lane g: head g; the running max in base-2 logits
      if (lane < 4) store_pair_agent(p.part_ml + (pbase + hw + lane) * 2, m_run * qa, lt);
    }
    }
  };

  // ---------------------------------------------------------------- pipeline
  // Two LDS stages; tile t lives in stage (t - lo) & 1 and is issued two
  // iterations ahead.  Iteration t:
  //   wait for this wave's loads of tile t (tile t+1's may still fly), then a
  //   barrier: tile t is complete in LDS;
  //   read all of tile t this lane needs into registers (and the segment's
  //   query rows), run PV of tile t-1 from registers while the reads land,
  //   finish a segment that ended at tile t-1;
  //   a second barrier: every wave is done reading the stage, which now takes
  //   tile t+2 (after the query rows of tile t+1 when that starts a segment);
  //   QK and softmax of tile t.
  // While tile t is computed, tiles t+1 and t+2 are in flight.  The loads of
  // one tile are followed by at most the next tile's query load and loads,
  // so waiting until NOPS operations remain covers tile t and its query.
  build(lo);
  int sinfo[2];
  issue_q(rng.b);               // the query rows first: begin runs while tile lo flies
  sinfo[0] = issue(lo, 0);
  sinfo[1] = lo + 1 < hi ? issue(lo + 1, 1) : 0;
  if (lo + 1 < hi) vm_wait_n<2 * S::NOPS>();
  else vm_wait_n<S::NOPS>();
  int seg_first = lo;
  bool seg_whole = (sinfo[0] >> 7) & 1;
  begin(*reinterpret_cast<const uint4*>(smem + S::QOFF + wave * 1024 + lane * 16));
  uint32_t xvs[2][2 * S::NP];   // V words of the tiles in the two stages
  uint32_t Ws[2][S::ROUNDS];    // their weights
  int pinfo = 0;                // info of the previous tile
#pragma unroll
  for (int i = 0; i < 2 * S::NP; ++i) xvs[0][i] = xvs[1][i] = 0;
#pragma unroll
  for (int i = 0; i < S::ROUNDS; ++i) Ws[0][i] = Ws[1][i] = 0;

  auto iteration = [&](int t, auto stage) {
    constexpr int st = decltype(stage)::value;
    constexpr int so = st ^ 1;
    if (t + 1 < hi) vm_wait_n<S::NOPS>();
    else vm_wait_n<0>();
    lds_barrier();
    const int info = sinfo[st];
    const bool first_of_seq = (info >> 7) & 1;
    const bool seg_start = t != lo && first_of_seq;   // the range's first segment began before the loop
    uint32_t kq[S::ROUNDS][DQ];
    uint2 kr[S::ROUNDS];
    read_tile(smem + st * S::STAGE + kvw * SLOT, kq, kr, xvs[st]);
    uint4 qw = make_uint4(0u, 0u, 0u, 0u);
    if (seg_start) qw = *reinterpret_cast<const uint4*>(smem + S::QOFF + wave * 1024 + lane * 16);
    if (t > lo) {
      pv(xvs[so], Ws[so]);
      if ((pinfo >> 6) & 1) finish(pinfo >> 8, seg_first, seg_whole, true);
    }
    lds_barrier();
    // tile t+2 into this stage, in three parts spread over the rest of the
    // iteration
    constexpr int K1 = (S::NOPS + 2) / 3, K2 = (2 * S::NOPS + 2) / 3;
    using IC0 = std::integral_constant<int, 0>;
    using IC1 = std::integral_constant<int, K1>;
    using IC2 = std::integral_constant<int, K2>;
    using IC3 = std::integral_constant<int, S::NOPS>;
    if (t + 1 < hi && ((sinfo[so] >> 7) & 1)) issue_q(sinfo[so] >> 8);
    const bool more = t + 2 < hi;
    Pending nx;
    if (more) {
      if (t + 2 - dchunk >= 64) build(t + 2);
      nx = fetch(t + 2, st);
      sinfo[st] = nx.info;
      loads(nx, IC0{}, IC1{});
    }
    if (seg_start) {
      seg_first = t;
      seg_whole = first_of_seq;
      begin(qw);
    }
    if (more) loads(nx, IC1{}, IC2{});
    qk_softmax(kq, kr, (info & 63) + 1, Ws[st]);
    if (more) loads(nx, IC2{}, IC3{});
    pinfo = info;
  };
  for (int t = lo; t < hi; t += 2) {
    iteration(t, std::integral_constant<int, 0>{});
    if (t + 1 < hi) iteration(t + 1, std::integral_constant<int, 1>{});
  }
  // the range's last tile
  if ((hi - 1 - lo) & 1) pv(xvs[1], Ws[1]);
  else pv(xvs[0], Ws[0]);
  finish(pinfo >> 8, seg_first, seg_whole, (pinfo >> 6) & 1);

  // Split sequences are merged, and empty sequences zeroed, by merge_kernel,
  // launched after this kernel on the same stream.
}

// Merge of the split sequences (and zeros for empty ones), launched after the
// decode kernel on the same stream: split_merge in attention_kernel.h.
template <int D, int TT>
__global__ void __launch_bounds__(128) merge_kernel(const AttnParams p) {
  split_merge<D, TT>(p);
}

// Workgroups one CU holds at once (cached per kernel; 0 if unknown).
static int blocks_per_cu(const void* kern, int threads, size_t lds) {
  static std::mutex mu;
  static std::map<std::tuple<const void*, int, size_t>, int> cache;
  const auto key = std::make_tuple(kern, threads, lds);
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  (void)hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, threads, lds) != hipSuccess) n = 0;
  (void)hipGetLastError();
  cache[key] = n;
  return n;
}

// Name of an instantiation, for the timing hook.
template <int D, int NKV, int WPK, int TT>
static const char* kernel_name() {
  static const std::string n = "rows_kernel<" + std::to_string(D) + "," + std::to_string(NKV) + "," +
                               std::to_string(WPK) + "," + std::to_string(TT) + "> (vector ALUs)";
  return n.c_str();
}

template <int D, int NKV, int WPK, int TT>
static int launch(AttnParams p, int groups, hipStream_t stream) {
  using S = Shape<D, NKV, WPK, TT>;
  auto kern = rows_kernel<D, NKV, WPK, TT>;
  const int per_cu = blocks_per_cu(reinterpret_cast<const void*>(kern), S::THREADS, S::LDS);
  const int cus = device_cu_count();
  int W = std::max(1, cus * std::max(1, per_cu) / groups);
  if (W > p.W) W = p.W;          // the workspace holds partials for p.W workgroups
  p.W = W;
  p.nthreads = S::THREADS;
  p.heads_per_group = 4 * S::WAVES;
  hipEvent_t ev0, ev1;
  if (kernel_timing_events(&ev0, &ev1, kernel_name<D, NKV, WPK, TT>()))
    hipExtLaunchKernelGGL(kern, dim3(W, groups), dim3(S::THREADS), S::LDS, stream, ev0, ev1, 0, p);
  else
    hipLaunchKernelGGL(kern, dim3(W, groups), dim3(S::THREADS), S::LDS, stream, p);
  if (int rc = check_launch("paged decode")) return rc;
  if (p.B > 0) {
    constexpr int MH = split_merge_heads<D>();
    hipLaunchKernelGGL((merge_kernel<D, TT>), dim3(p.B, (p.H + MH - 1) / MH), dim3(128), 0, stream, p);
    return check_launch("paged decode merge");
  }
  return 0;
}

}  // namespace rows

// Shape of the whole-row kernel for a request, or false if it does not apply.
bool rows_shape(int H, int G, int D, int cache_kv, int* nkv, int* wpk, int* groups) {
  if ((D != 64 && D != 128) || (G != 4 && G != 8) || H % G != 0) return false;
  const int KV = H / G;
  if (cache_kv != KV || cache_kv % 2 != 0) return false;
  const int w = G / 4;
  int n = 0;
  // Two waves per KV head: at head_dim 64 two KV heads per workgroup (4 waves,
  // three workgroups per CU) keep more independent waves on each SIMD than
  // four (8 waves, one workgroup per CU by registers); at 128 the reverse
  // measured faster.
  if (w == 1) n = KV % 8 == 0 ? 8 : KV % 4 == 0 ? 4 : KV % 2 == 0 ? 2 : 0;
  else if (D == 64) n = KV % 2 == 0 ? 2 : 0;
  else n = KV % 4 == 0 ? 4 : KV % 2 == 0 ? 2 : 0;
  if (n == 0) return false;
  *nkv = n;
  *wpk = w;
  *groups = KV / n;
  return true;
}

// Instantiations (head_dim, KV heads per workgroup, waves per KV head, tokens
// per tile): 64-token tiles where a wave's rows fit one 16-row block, 32-token
// tiles otherwise.
#define SLMT_ROWS_CONFIGS(X)                                                                 \
  X(128, 8, 1, 64) X(128, 4, 1, 64) X(128, 2, 1, 32) X(128, 4, 2, 64) X(128, 2, 2, 64)     \
  X(64, 8, 1, 64) X(64, 4, 1, 64) X(64, 2, 1, 32) X(64, 4, 2, 64) X(64, 2, 2, 64)
#define SLMT_ROWS_KEY(d, a, b) ((d) * 100 + (a) * 10 + (b))

// Workgroups per head group the whole-row kernel may use (its workspace bound).
int rows_max_workgroups(int D, int nkv, int wpk, int groups, int cus) {
  const int waves = nkv * wpk;
  // at most 8 waves per CU at head_dim 128 (up to 256 VGPRs each), 12 at 64
  // (up to 168), and the ring's LDS
  size_t lds = 0;
  switch (SLMT_ROWS_KEY(D, nkv, wpk)) {
#define SLMT_ROWS_LDS(d, a, b, c) case SLMT_ROWS_KEY(d, a, b): lds = rows::Shape<d, a, b, c>::LDS; break;
    SLMT_ROWS_CONFIGS(SLMT_ROWS_LDS)
#undef SLMT_ROWS_LDS
    default: return 1;
  }
  int per_cu = std::min((D == 64 ? 12 : 8) / waves, (int)((160 * 1024) / lds));
  per_cu = std::max(1, per_cu);
  return std::max(1, cus * per_cu / groups);
}

int launch_attention_rows(int D, int nkv, int wpk, int groups, const AttnParams& p, hipStream_t stream) {
  switch (SLMT_ROWS_KEY(D, nkv, wpk)) {
#define SLMT_ROWS_LAUNCH(d, a, b, c) case SLMT_ROWS_KEY(d, a, b): return rows::launch<d, a, b, c>(p, groups, stream);
    SLMT_ROWS_CONFIGS(SLMT_ROWS_LAUNCH)
#undef SLMT_ROWS_LAUNCH
    default: return fail(SLMT_ERR_INVALID, "paged decode: no whole-row kernel for this shape");
  }
}

}  // namespace slmt
