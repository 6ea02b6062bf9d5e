// Batched paged 4-bit decode attention on the matrix cores, head_dim 64 or 128
// with 4 or 8 query heads per KV head (reference kernel it replaces:
// kv_dequant_decode_per_token_paged_kernel, kernels/kv_dequant_kernels.cuh:671-801,
// batched over the whole decode step instead of launched per request).
//
// Why matrix cores for a GEMV-shaped decode: with 4-bit codes every cache byte
// carries 2 x G multiply-adds per product (QK and PV), and the vector ALUs do
// at most 2 per lane-instruction with fp16 x code exactness (v_dot2 issues at
// ~5 cycles per wave64 on this part).  At G = 4 that puts the vector-ALU
// instruction stream above the HBM time; here both products run on MFMA and
// the vector ALUs only unpack codes and run the softmax.
//
// Work split, staging and merge are the whole-row kernel's (attention_rows.hip):
// a workgroup owns NKV consecutive KV heads of every cache row, one wave per 4
// query heads (WPK waves per KV head); 64-token tiles are copied with 16-byte
// direct loads into a 2-stage LDS ring two tiles ahead; work is split stream-K
// over the concatenated tile list and split sequences are merged by merge_kernel.
// At head_dim 128 with 8 query heads per KV head the two waves of a KV head
// split each tile's tokens instead (32 each, all 8 heads as two sets of B
// columns), so the nibble unpacking of K and V is done once per token rather
// than once per wave; the second wave's sums join the first's through LDS at
// each segment end.  At head_dim 64 the split measured slower (the extra
// softmax reductions and the join cost more than the unpacking saved) and the
// two waves take 4 heads each over the whole tile.
//
// QK, exact: v_mfma_i32_16x16x64_i8.  The fp16 query of each head is scaled by a
// power of two to a 31-bit integer Q (every fp16 value above 2^-21 of the head's
// largest is exact) and split into four signed 8-bit limbs, Q = sum_x L_x 2^(8x);
// the 16 rows of A are (head h, limb x), the columns of B 16 tokens whose codes
// are unpacked from nibbles to bytes.  Integer accumulation is exact, and each
// lane of C then holds all four limbs of one (head, token): limbs 0 + 1 and
// 2 + 3 join in int32, the two halves in one fp32 fma, with no cross-lane
// traffic.  q.K = step * (Q.n) 2^-S + min * sum(q).
//
// PV: v_mfma_f32_16x16x32_f16 with A = V^T (rows: 16 V bytes, one of their two
// nibbles; k: 32 tokens) and B = the fp16 weights (columns: the wave's 4 heads).
// A lane's V bytes of one token are one ds_read_u16 (head_dim 64) or ds_read_b32
// (128), two tokens are packed with one v_perm, and each nibble becomes an fp16
// subnormal n * 2^-24 (or 16 n * 2^-24) with one AND, which the matrix core
// multiplies exactly by the weight.  Weights w = fp16(p * step) go into the B
// columns of the wave's heads; the columns the heads leave free carry each
// weight's remainder, fp16((p * step - w) * 2^11), so a column pair holds
// p * step to ~22 bits down to 2^-25 and to within 2^-36 below (a lone fp16
// weight loses precision below 2^-14 and vanishes below 2^-25: a long tail
// behind a dominant token would drop out).  The pair is joined once per
// segment; the softmax sums use p itself, and the per-token min enters once per
// token as sum(p * min).
#include "attention_kernel.h"

#include <hip/hip_ext.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <type_traits>

namespace slmt {
namespace mrows {

using namespace attn;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) const uint64_t lds_u64;

template <int D, int NKV, int WPK>
struct Shape {
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static_assert(NKV % 2 == 0, "sub-rows must be a whole number of 16-byte units");
  static constexpr int TT = 64;                 // tokens per tile
  static constexpr int SLOT = D + 8;            // bytes of one KV head in a cache row
  static constexpr int NS = 2;                  // LDS ring stages
  static constexpr int WAVES = NKV * WPK;
  static constexpr int THREADS = WAVES * 64;
  static constexpr int UPR = NKV * SLOT / 16;   // 16-byte units of a sub-row
  static constexpr int RP = UPR | 1;            // units of a staged row (odd: rows spread over the banks)
  static constexpr int RSTRIDE = RP * 16;
  static constexpr int RW = TT / WAVES;         // rows copied per wave
  static_assert(TT % WAVES == 0 && RW <= 16 && 16 % RW == 0, "a wave's rows must lie in one block");
  static constexpr int WUNITS = RW * RP;
  static constexpr int NOPS = (WUNITS + 63) / 64;
  static constexpr int LAST = WUNITS - 64 * (NOPS - 1);   // lanes of the wave's last load
  static constexpr int RB = TT / 16;            // QK row blocks (16 tokens)
  static constexpr int KB = D / 64;             // QK k-blocks (64 dims)
  static constexpr int CB = D / 64;             // PV blocks of 32 V bytes
  static constexpr int TH = TT / 32;            // PV token halves
  static constexpr int STAGE = TT * RSTRIDE;
  static constexpr int QOFF = NS * STAGE;       // one 1 KB query slot per wave
  // per-wave weights, fp16: 4 heads x TT tokens (or 8 heads x TT / 2 with the
  // token split), then their remainders in the same layout
  static constexpr int WSZ = 2 * 4 * TT * 2;
  static constexpr int WOFF = QOFF + WAVES * 1024;
  static constexpr int ZOFF = WOFF + WAVES * WSZ;   // 128 zero bytes (B operand of unused columns)
  static constexpr int MOFF = ZOFF + 128;
  static constexpr int STASH = 256;             // sequence lengths kept in LDS
  static constexpr int SOFF = MOFF + 32 * 4;
  // Two waves per KV head split each tile's tokens and take all of the KV head's
  // 8 query heads; at a segment end the second wave hands its (m, l, PV sums)
  // to the first through this buffer: per KV head 64 lanes x D/4 floats + 3 x 8.
  static constexpr int CBW = (D / 4) * 64 * 4 + 3 * 8 * 4;
  static constexpr int COFF = SOFF + STASH * 4;
  static constexpr bool TS = WPK == 2 && D == 128;   // token split (see mfma_kernel)
  // Non-temporal tile loads, except with two KV heads per workgroup at head_dim
  // 64: there the halves of a cache row go to different workgroups, and the
  // 64-byte line that straddles them is read by both; with the default policy
  // it stays in L2 for the second reader (traffic 1.22 -> 1.12 x algorithmic,
  // 20.2 -> 19.5 us at 32 q / 4 KV heads, batch 32, 4096 keys).
  static constexpr bool NT = !(D == 64 && NKV == 2);
  static constexpr int LDS = COFF + (TS ? NKV * CBW : 0);
  static_assert(LDS <= 160 * 1024, "LDS ring too large");
};

// The weights' reference sits kRefMargin (base 2) above the largest score seen:
// weights stay below 2^-kRefMargin (so p * step never exceeds the fp16 step), and
// the reference moves, with its rescale of the sums, only when a score passes it.
// Placed at the maximum itself it moved in most tiles of a short range (any of a
// wave's 4 or 8 heads growing): 21.4 -> 21.0 us per step at 32 q / 4 KV heads,
// head_dim 64, batch 32, 4096 keys.
constexpr float kRefMargin = 4.0f;

// log2(e) / sqrt(D)
template <int D>
constexpr float kC = D == 128 ? 1.4426950408889634f / 11.313708498984761f : 1.4426950408889634f / 8.0f;

// PV k-slot e (e < 8) of lane group g covers token ktok(g, e) of a 32-token
// half: 8 m + 4 (g & 1) + 2 (g >> 1) + s for e = 2 m + s.  The rows that the
// two half-waves read at once (groups 0, 1 and 2, 3) are 4 apart, 16 banks
// apart with an odd-unit row stride, so the V reads are conflict-free.  wpos
// is the inverse: the token's position 8 g + e in the weight scratch, so the 8
// k-slots of a lane group are 16 contiguous bytes.
__device__ __forceinline__ int ktok(int g, int e) { return 8 * (e >> 1) + 4 * (g & 1) + 2 * (g >> 1) + (e & 1); }
__device__ __forceinline__ int wpos(int t) {
  const int u = t & 7;
  const int g = ((u >> 2) & 1) | (((u >> 1) & 1) << 1);
  return 8 * g + 2 * (t >> 3) + (u & 1);
}

template <int D, int NKV, int WPK>
__global__ void __launch_bounds__(NKV * WPK * 64) mfma_kernel(const AttnParams p) {
  using S = Shape<D, NKV, WPK>;
  constexpr int TT = S::TT, SLOT = S::SLOT, RB = S::RB, KB = S::KB, CB = S::CB, TH = S::TH;
  // Token split (two waves per KV head): wave `half` of a KV head takes tokens
  // 32 half .. 32 half + 31 of every tile for all 8 query heads of the KV head
  // (two sets of 4), so the K unpacking and the V operands are built once per
  // token instead of once per wave.
  constexpr bool TS = S::TS;
  constexpr int NSET = TS ? 2 : 1;         // sets of 4 query heads per wave
  constexpr int RBW = TS ? RB / 2 : RB;    // QK row blocks per wave
  constexpr int THW = TS ? 1 : TH;         // PV token halves per wave
  constexpr int TTW = TT / (TS ? 2 : 1);   // tokens per wave and tile
  constexpr int HPW = 4 * NSET;            // query heads per wave
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
  const int half = TS ? (wave & 1) : 0;                           // token half (token split)
  int* misc = reinterpret_cast<int*>(smem + S::MOFF);
  uint8_t* const wscr = smem + S::WOFF + wave * S::WSZ;
  if (tid < 32) reinterpret_cast<uint32_t*>(smem + S::ZOFF)[tid] = 0u;   // published by schedule_range's barriers

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
  // 64: lanes qp >= 8 re-read dims 8(qp - 8) ..); the slot holds (head h, dim d)
  // at byte 64 (d / 8) + 16 h + 2 (d % 8)
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
      if (k < S::NOPS - 1 || S::LAST == 64 || lane < S::LAST) lds_load16<S::NT>(d.base, goff[k], d.dst + k * 1024);
    }
  };
  auto issue = [&](int t, int st) -> int {
    const Pending d = fetch(t, st);
    loads(d, std::integral_constant<int, 0>{}, std::integral_constant<int, S::NOPS>{});
    return d.info;
  };
  const uint32_t qslot = lds_smem + S::QOFF + wave * 1024;
  auto issue_q = [&](int b) { lds_load16(p.q + (int64_t)b * p.q_seq_stride, qoff, qslot); };

  // ---------------------------------------------------------------- lane roles
  // col = lane & 15, grp = lane >> 4.
  //  QK A: row col = 4 h + x is limb x of head h (h = col >> 2), k-set grp.
  //  QK B: column col (token 16 rb + col), k-set grp.
  //  QK C and softmax: column col, rows 4 grp + x: the lane holds the four limbs
  //    of head grp for token 16 rb + col of each row block.
  //  PV A: row col (V byte 32 cb + 2 col, and the next byte), k-set grp;
  //    PV B / C: column col (head col for col < 4), C rows 4 grp + r.
  const int col = lane & 15, grp = lane >> 4;
  const int hq = col >> 2, lx = col & 3;
  // first of the 16 dims that k-block kb of lane group grp covers (QK)
  auto kbase = [&](int kb) { return 64 * kb + 16 * grp; };
  const uint8_t* const qsl = smem + S::QOFF + wave * 1024;

  v4i qb[NSET][KB];                    // A operand: limb lx of head set st's head hq, k-set grp
  // m_run: the weights' reference, in score units (see softmax); dq: its margin
  float qa[NSET], qs[NSET], mq[NSET], m_run[NSET], l_run[NSET], vmt[NSET], dq[NSET];
#pragma unroll
  for (int st = 0; st < NSET; ++st) {
    qa[st] = qs[st] = mq[st] = 0.f;
    m_run[st] = -INFINITY;
    l_run[st] = vmt[st] = 0.f;
  }
  floatx4 acc[CB][4];                  // PV: [block][E.lo, E.hi, O.lo, O.hi]

  // Value of head grp for the softmax lanes, from lane 4 grp (which holds head
  // grp in the query operand's layout).
  const int soft_src = 16 * grp;   // byte address of lane 4 grp
  auto for_soft_lane = [&](float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(soft_src, __builtin_bit_cast(int, v)));
  };
  // Query of head set st for a new segment: read the lane's 16 dims per k-block
  // straight from the query slot (with the token split, set st's heads are in
  // the slot of wave 2 kvw + st; else in the wave's own), scale head hq to
  // 31-bit integers, and cut limb lx.
  auto begin_set = [&](int st) __attribute__((always_inline)) {
    m_run[st] = -INFINITY;
    l_run[st] = 0.f;
    vmt[st] = 0.f;
    const uint8_t* const qs_slot = TS ? smem + S::QOFF + (2 * kvw + st) * 1024 : qsl;
    float qv[KB][16];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        // dims kbase(kb) + 8 u .. + 7
        const uint4 w = *reinterpret_cast<const uint4*>(qs_slot + 64 * ((kbase(kb) >> 3) + u) + 16 * hq);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          qv[kb][8 * u + 2 * i] = h2f((uint16_t)(ws[i] & 0xffffu));
          qv[kb][8 * u + 2 * i + 1] = h2f((uint16_t)(ws[i] >> 16));
        }
      }
    float amax = 0.f;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(qv[kb][i]));
    {
      float a, b;
      swap16(amax, a, b);
      amax = fmaxf(a, b);
      swap32(amax, a, b);
      amax = fmaxf(a, b);
    }
    // amax * 2^sc in [2^29, 2^30): |Q| < 2^30, so the top limb fits 8 bits
    const int sc = amax > 0.f ? 30 - __builtin_amdgcn_frexp_expf(amax) : 0;
    const int sh = 8 * lx;
    const uint32_t xm = lx < 3 ? 0x80u : 0u;
    float qsum = 0.f;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      uint32_t bytes[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float f = __builtin_rintf(__builtin_amdgcn_ldexpf(qv[kb][i], sc));
        const int Q = (int)f;
        qsum += f;
        // balanced digits: Q + 0x808080 = sum d_x 2^(8x), limb x = d_x - 128 (x < 3), top = the rest
        bytes[i] = ((uint32_t)((Q + 0x808080) >> sh) & 0xffu) ^ xm;
      }
      // operand byte 4 dw + m is dim 8 (dw >> 1) + 2 m + (dw & 1) of the lane's 16
      uint32_t dw[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int b0 = 8 * (d >> 1) + (d & 1);
        dw[d] = bytes[b0] | (bytes[b0 + 2] << 8) | (bytes[b0 + 4] << 16) | (bytes[b0 + 6] << 24);
      }
      qb[st][kb] = v4i{(int)dw[0], (int)dw[1], (int)dw[2], (int)dw[3]};
    }
    {
      float a, b;
      swap16(qsum, a, b);
      qsum = a + b;
      swap32(qsum, a, b);
      qsum = a + b;
    }
    qs[st] = for_soft_lane(qsum);
    qa[st] = for_soft_lane(__builtin_amdgcn_ldexpf(kC<D>, -sc));
    dq[st] = kRefMargin * __builtin_amdgcn_rcpf(qa[st]);
  };
  auto begin = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[c][k] = floatx4{0.f, 0.f, 0.f, 0.f};
    begin_set(0);
    if constexpr (NSET == 2) begin_set(1);
  };

  // ---------------------------------------------------------------- tile data
  // LDS reads of one tile for this lane: QK A rows (packed), the rulers of the
  // lane's softmax tokens, and the V byte pairs of its PV k-slots.
  // K: lane (row col, group grp) reads bytes [8 grp, 8 grp + 8) of each 32-byte
  // half (k-block) of its row's codes, so that k-block kb is dims 64 kb ..
  // 64 kb + 63 in order.  These 8-byte reads are free of LDS bank conflicts at
  // the staged row strides; 8-byte reads 16 bytes apart, and pair reads
  // (ds_read2_b64) of 8-byte halves 8 or 32 bytes apart, cost 2, 8 and 8
  // conflict cycles each.
  // V: lane (row col, group grp) reads bytes [4 col, 4 col + 4) (head_dim 64:
  // [2 col, 2 col + 2)) of the V codes of its 8 k-slot tokens.
  // With the token split, the wave reads only its half of the tile's tokens
  // (row blocks and token half of the wave's 32 tokens).
  struct TileRegs {
    uint32_t k[RBW][2 * KB];    // packed codes: k-block kb in words 2 kb, 2 kb + 1
    uint2 rl[RBW];              // rulers of the lane's softmax tokens
    uint32_t v[THW][8];         // V codes of the k-slots, per token half
  };
  auto read_tile = [&](const uint8_t* Sb0, TileRegs& R) {
    const uint8_t* const Sb = Sb0 + 32 * half * S::RSTRIDE;
#pragma unroll
    for (int rb = 0; rb < RBW; ++rb) {
      const uint8_t* row = Sb + (16 * rb + col) * S::RSTRIDE;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        // the second k-block's address passes through an empty asm, which keeps
        // the compiler from merging the two reads into one pair read
        const lds_u64* src = (const lds_u64*)(row + 32 * kb + 8 * grp);
        if (kb > 0) asm("" : "+v"(src));
        const uint64_t w = *src;
        R.k[rb][2 * kb] = (uint32_t)w;
        R.k[rb][2 * kb + 1] = (uint32_t)(w >> 32);
      }
    }
#pragma unroll
    for (int rb = 0; rb < RBW; ++rb) R.rl[rb] = *reinterpret_cast<const uint2*>(Sb + (16 * rb + col) * S::RSTRIDE + D);
#pragma unroll
    for (int th = 0; th < THW; ++th)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint8_t* src = Sb + (32 * th + ktok(grp, e)) * S::RSTRIDE + D / 2;
        if constexpr (D == 128) R.v[th][e] = *reinterpret_cast<const uint32_t*>(src + 4 * col);
        else R.v[th][e] = *reinterpret_cast<const uint16_t*>(src + 2 * col);
      }
  };

  // QK of one tile: 16 tokens x (head, limb) per row block, exact int32.
  // C[st RBW + rb]: row block rb of the wave's tokens against head set st.
  auto qk = [&](const TileRegs& R, v4i (&C)[RB]) {
#pragma unroll
    for (int i = 0; i < RB; ++i) C[i] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int rb = 0; rb < RBW; ++rb) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const uint32_t x0 = R.k[rb][2 * kb], x1 = R.k[rb][2 * kb + 1];
        const v4i a{(int)(x0 & 0x0F0F0F0Fu), (int)((x0 >> 4) & 0x0F0F0F0Fu), (int)(x1 & 0x0F0F0F0Fu),
                    (int)((x1 >> 4) & 0x0F0F0F0Fu)};
#pragma unroll
        for (int st = 0; st < NSET; ++st)
          C[st * RBW + rb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qb[st][kb], a, C[st * RBW + rb], 0, 0, 0);
      }
    }
  };

  // Limb combine: C[r] of lane (col, grp) holds limbs 0..3 of head grp for
  // token 16 rb + col (r = st RBW + rb).  Each limb sum is below 2^18 in
  // magnitude (128 dims x 128 x 15), so limbs 0 + 1 and 2 + 3 join exactly in
  // int32 and s = lo + 2^16 hi = Q.n rounds once per half and once in the fma.
  auto combine = [&](const v4i (&C)[RB], float (&s)[4]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int lo = (int)((uint32_t)C[r][0] + ((uint32_t)C[r][1] << 8));
      const int hi = (int)((uint32_t)C[r][2] + ((uint32_t)C[r][3] << 8));
      s[r] = __builtin_fmaf((float)hi, 65536.0f, (float)lo);
    }
  };

  // Sum / max over the 16 lanes of head grp (one row of the wave).
  auto head_max = [&](float v) {
    v = fmaxf(v, dpp_f<DPP_ROW_ROR8>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_ROR4>(v));
    v = fmaxf(v, dpp_f<DPP_QUAD_XOR2>(v));
    return fmaxf(v, dpp_f<DPP_QUAD_XOR1>(v));
  };
  auto head_sum = [&](float v) {
    v += dpp_f<DPP_ROW_ROR8>(v);
    v += dpp_f<DPP_ROW_ROR4>(v);
    v += dpp_f<DPP_QUAD_XOR2>(v);
    return v + dpp_f<DPP_QUAD_XOR1>(v);
  };
  // value of head `col` (0..3) for the PV lanes: from lane 16 (col & 3), which
  // holds head col & 3 (one cross-lane read; four lane reads and a per-lane
  // choice among them compiled to a branch chain)
  const int pv_src = 64 * (col & 3);
  auto for_pv_lane = [&](float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(pv_src, __builtin_bit_cast(int, v)));
  };
  // value of head `col` (0..HPW-1) for the PV lanes: head col & 3 of set col >> 2
  auto for_pv_lane_set = [&](const float (&v)[NSET]) {
    if constexpr (NSET == 1) {
      return for_pv_lane(v[0]);
    } else {
      const float a = for_pv_lane(v[0]), b = for_pv_lane(v[1]);
      return (col & 4) ? b : a;
    }
  };

  // Softmax of one tile and its weights into the scratch.  Tokens past the
  // sequence end get u = -inf (weight 0) and zero rulers.  Score r is row block
  // r % RBW of the wave's tokens for head set r / RBW.
  auto softmax = [&](const TileRegs& R, const float (&s)[4], int nvalid) {
    float u[4];
    uint32_t vr[RBW];                  // V rulers (min, step) of the lane's tokens, fp16 pair
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int st = r / RBW, rb = r % RBW;
      const uint32_t kr = R.rl[rb].x;
      u[r] = __builtin_fmaf(s[r], h2f((uint16_t)(kr >> 16)), h2f((uint16_t)(kr & 0xffffu)) * qs[st]);
    }
#pragma unroll
    for (int rb = 0; rb < RBW; ++rb) vr[rb] = R.rl[rb].y;
    if (nvalid < TT) {
      // the sequence's last tile: slots past its end may hold anything (a
      // reused block), so they get u = -inf and their rulers must not reach
      // the sums
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rb = r % RBW;
        u[r] = 32 * half + 16 * rb + col < nvalid ? u[r] : -INFINITY;
      }
#pragma unroll
      for (int rb = 0; rb < RBW; ++rb) vr[rb] = 32 * half + 16 * rb + col < nvalid ? vr[rb] : 0u;
    }
    float alpha[NSET];
    bool grew = false;
#pragma unroll
    for (int st = 0; st < NSET; ++st) {
      float tl = u[st * RBW];
#pragma unroll
      for (int rb = 1; rb < RBW; ++rb) tl = fmaxf(tl, u[st * RBW + rb]);
      alpha[st] = 1.f;
      if (__builtin_amdgcn_ballot_w64(tl > m_run[st])) {
        const float tmax = head_max(tl);
        const bool grow = tmax > m_run[st];
        const float mnew = tmax + dq[st];
        alpha[st] = grow ? __builtin_amdgcn_exp2f((m_run[st] - mnew) * qa[st]) : 1.f;   // 0 from -inf
        l_run[st] *= alpha[st];
        vmt[st] *= alpha[st];
        m_run[st] = grow ? mnew : m_run[st];
        mq[st] = m_run[st] * qa[st];
        grew = true;
      }
    }
    if (grew) {
      const float ap = for_pv_lane_set(alpha);
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[c][k] *= ap;
    }
    uint32_t wv[4], wr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int st = r / RBW, rb = r % RBW;
      // tokens past the end give exp2(-inf) = 0 (mq is finite: the first half's
      // token 0 is valid in every tile, and a second half without valid tokens
      // keeps the previous finite mq or 0)
      const float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(u[r], qa[st], -mq[st]));
      const float vstep = h2f((uint16_t)(vr[rb] >> 16));
      const _Float16 wh = (_Float16)(pr * vstep);
      // remainder in units of 2^-11: at most half an ulp of a weight below
      // 65504 (16), so it never overflows; normal down to remainders of 2^-25
      const float rem = __builtin_fmaf(pr, vstep, -(float)wh);
      l_run[st] += pr;
      vmt[st] = __builtin_fmaf(pr, h2f((uint16_t)(vr[rb] & 0xffffu)), vmt[st]);
      wv[r] = __builtin_bit_cast(uint16_t, wh);
      wr[r] = __builtin_bit_cast(uint16_t, (_Float16)(rem * 2048.0f));
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int st = r / RBW, rb = r % RBW;
      uint16_t* wh = reinterpret_cast<uint16_t*>(wscr) + (4 * st + grp) * TTW;
      // token 16 rb + col of the wave's tokens: token half rb >> 1, local 16 (rb & 1) + col
      const int at = 32 * (rb >> 1) + wpos(16 * (rb & 1) + col);
      wh[at] = (uint16_t)wv[r];
      wh[HPW * TTW + at] = (uint16_t)wr[r];   // the remainder column of the same head
    }
  };

  // PV of one tile from its V byte pairs and the weights in the scratch.
  auto pv = [&](const TileRegs& R) {
    wave_lds_sync();
    half8 bw[THW];
#pragma unroll
    for (int th = 0; th < THW; ++th) {
      // columns HPW + h hold head h's remainders (zeros past 2 HPW)
      const uint8_t* src =
          col < 2 * HPW ? wscr + (col * TTW + 32 * th + 8 * grp) * 2 : smem + S::ZOFF + 64 * th + 16 * grp;
      bw[th] = *reinterpret_cast<const half8*>(src);
    }
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int th = 0; th < THW; ++th) {
        uint32_t el[4], eh[4], ol[4], oh[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          // [E_t, O_t, E_t', O_t'] of the k-slot pair 2d, 2d + 1: bytes 2c, 2c + 1
          // of the two tokens' V words
          const uint32_t x = __builtin_amdgcn_perm(R.v[th][2 * d + 1], R.v[th][2 * d],
                                                   c == 0 ? 0x05040100u : 0x07060302u);
          const uint32_t y = x >> 8;
          el[d] = x & 0x000F000Fu;
          eh[d] = x & 0x00F000F0u;
          ol[d] = y & 0x000F000Fu;
          oh[d] = y & 0x00F000F0u;
        }
        const uint4 e0 = make_uint4(el[0], el[1], el[2], el[3]), e1 = make_uint4(eh[0], eh[1], eh[2], eh[3]);
        const uint4 o0 = make_uint4(ol[0], ol[1], ol[2], ol[3]), o1 = make_uint4(oh[0], oh[1], oh[2], oh[3]);
        acc[c][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, e0), bw[th], acc[c][0], 0, 0, 0);
        acc[c][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, e1), bw[th], acc[c][1], 0, 0, 0);
        acc[c][2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, o0), bw[th], acc[c][2], 0, 0, 0);
        acc[c][3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, o1), bw[th], acc[c][3], 0, 0, 0);
      }
  };

  // End of a segment of sequence b whose first tile is seg_first (a whole
  // sequence when `whole`): write the output or a partial piece.  Lane (col <
  // 4, grp) holds head col and C row i = 4 grp + r of block c, i.e. V bytes
  // 4 i + 2 c (E) and 4 i + 2 c + 1 (O) (head_dim 64: 2 i, 2 i + 1), dims
  // 8 i + 4 c + (0: E.lo, 1: E.hi, 2: O.lo, 3: O.hi) (head_dim 64: 4 i + ...).
  // The stores are issued one iteration later (flush, right after that
  // iteration's wait for its tile): stores count in the same in-order vector
  // memory counter as the tile loads, and stores issued behind tile t+2's loads
  // would make the next wait hold for those loads too.
  float ov[CB][4][4];
  float2 pml = make_float2(0.f, 0.f);
  int pk = 0;                          // pending stores: 0 none, 1 output, 2 partial piece
  int64_t pofs = 0, pmlofs = 0;
  auto finish = [&](int b, int seg_first, bool whole, bool last_of_seq) __attribute__((always_inline)) {
    float lh[NSET], vh[NSET], mh[NSET];
#pragma unroll
    for (int st = 0; st < NSET; ++st) {
      lh[st] = head_sum(l_run[st]);
      vh[st] = head_sum(vmt[st]);
      mh[st] = m_run[st] * qa[st];
    }
    float lt = for_pv_lane_set(lh);
    float vt = for_pv_lane_set(vh);
    float mt = for_pv_lane_set(mh);
    const int h = hw + (col & (HPW - 1));   // lanes col >= HPW hold no output
    if constexpr (TS) {
      // The second wave of the pair hands its sums to the first, which scales
      // both by exp2(m - max) and stores the 8 heads; the second stores nothing.
      float* const cb = reinterpret_cast<float*>(smem + S::COFF + kvw * S::CBW);
      float* const cml = cb + (D / 4) * 64;
      if (half == 1) {
#pragma unroll
        for (int c = 0; c < CB; ++c)
#pragma unroll
          for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int r = 0; r < 4; ++r) cb[((4 * c + k) * 4 + r) * 64 + lane] = acc[c][k][r];
        if (grp == 0 && col < 8) {
          cml[col] = mt;
          cml[8 + col] = lt;
          cml[16 + col] = vt;
        }
      }
      lds_barrier();
      if (half == 1) {
        pk = 0;
        return;
      }
      const float m1 = cml[col & 7], l1 = cml[8 + (col & 7)], v1 = cml[16 + (col & 7)];
      const float M = fmaxf(mt, m1);            // mt is finite: token 0 of every tile is the first wave's
      const float f0 = __builtin_amdgcn_exp2f(mt - M), f1 = __builtin_amdgcn_exp2f(m1 - M);   // m1 = -inf gives 0
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[c][k][r] = __builtin_fmaf(acc[c][k][r], f0, f1 * cb[((4 * c + k) * 4 + r) * 64 + lane]);
      lt = __builtin_fmaf(lt, f0, f1 * l1);
      vt = __builtin_fmaf(vt, f0, f1 * v1);
      mt = M;
    }
    // join each head's column with its remainder column, HPW lanes up
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float lo = HPW == 4 ? dpp_f<DPP_ROW_SHL4>(acc[c][k][r]) : dpp_f<DPP_ROW_ROR8>(acc[c][k][r]);
          acc[c][k][r] = __builtin_fmaf(lo, 0x1p-11f, acc[c][k][r]);
        }
    const bool final_out = whole && last_of_seq;
    const float rL = final_out ? __builtin_amdgcn_rcpf(lt) : 1.0f;
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ov[c][r][0] = (acc[c][0][r] * 16777216.0f + vt) * rL;   // 2^24: nibble-as-subnormal scale
        ov[c][r][1] = (acc[c][1][r] * 1048576.0f + vt) * rL;    // (16 n) 2^-24 -> n
        ov[c][r][2] = (acc[c][2][r] * 16777216.0f + vt) * rL;
        ov[c][r][3] = (acc[c][3][r] * 1048576.0f + vt) * rL;
      }
    if (final_out) {
      pk = 1;
      pofs = (int64_t)b * p.out_seq_stride + (int64_t)h * p.out_head_stride;
    } else {
      const int slot = (seg_first == lo) ? 0 : 1;
      const int64_t pbase = ((int64_t)wg * 2 + slot) * p.H;
      pk = 2;
      pofs = (pbase + h) * D;
      pmlofs = (pbase + h) * 2;
      pml = make_float2(mt, lt);
    }
  };
  auto flush = [&]() __attribute__((always_inline)) {
    if (pk == 0) return;
    if (col < HPW) {
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int d = (D == 128 ? 8 : 4) * (4 * grp + r) + 4 * c;
          const float* o = ov[c][r];
          if (pk == 1) {
            if (p.out_f16) {
              uint2 v;
              v.x = (uint32_t)f2h(o[0]) | ((uint32_t)f2h(o[1]) << 16);
              v.y = (uint32_t)f2h(o[2]) | ((uint32_t)f2h(o[3]) << 16);
              *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.out) + pofs + d) = v;
            } else {
              *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.out) + pofs + d) = make_float4(o[0], o[1], o[2], o[3]);
            }
          } else {
            *reinterpret_cast<float4*>(p.part_o + pofs + d) = make_float4(o[0], o[1], o[2], o[3]);
          }
        }
      if (pk == 2 && grp == 0) *reinterpret_cast<float2*>(p.part_ml + pmlofs) = pml;
    }
    pk = 0;
  };

  // ---------------------------------------------------------------- pipeline
  // Two LDS stages; tile t lives in stage (t - lo) & 1 and is issued two
  // iterations ahead (the second tile one iteration ahead).  Iteration t:
  //   wait for this wave's loads of tile t (tile t+1's may still fly), then a
  //   barrier: tile t is complete in LDS;
  //   read what this lane needs of tile t into registers (and, at a segment
  //   start, set up the segment's query); QK on the matrix cores while the V
  //   reads land;
  //   a second barrier: every wave is done reading the stage, which now takes
  //   tile t+2 (after the query rows of tile t+1 when that starts a segment);
  //   combine, softmax, PV, and the end of a segment that ends at tile t.
  // The loads of one tile are followed by at most the next tile's query load
  // and loads (and output stores, issued behind no later load, which only
  // make the wait stricter), so waiting until NOPS operations remain covers
  // tile t and its query.
  build(lo);
  int sinfo[2];
  issue_q(rng.b);
  // Only the first tile before the loop: with the second one requested at the
  // same time, the whole chip's first burst is twice as large and a
  // workgroup's first tile lands anywhere within it (5.6 to 8.8 us at batch
  // 64); the second tile goes out as soon as the first has landed (-0.45 us
  // per step at batch 64, 32 q / 8 KV heads).
  sinfo[0] = issue(lo, 0);
  sinfo[1] = 0;
  int seg_first = lo;
  bool seg_whole = (sinfo[0] >> 7) & 1;

  auto iteration = [&](int t, auto stage) {
    constexpr int st = decltype(stage)::value;
    constexpr int so = st ^ 1;
    if (t == lo) {
      vm_wait_n<0>();
      if (lo + 1 < hi) sinfo[1] = issue(lo + 1, 1);   // stage 1 is still free
    } else if (t + 1 < hi) {
      vm_wait_n<S::NOPS>();
    } else {
      vm_wait_n<0>();
    }
    lds_barrier();
    flush();
    const int info = sinfo[st];
    const bool first_of_seq = (info >> 7) & 1;
    const bool seg_start = t == lo || first_of_seq;
    if (seg_start) {
      if (t != lo) {
        seg_first = t;
        seg_whole = true;
      }
      begin();
    }
    TileRegs R;
    read_tile(smem + st * S::STAGE + kvw * SLOT, R);
    lds_barrier();
    // tile t+2 into this stage, in parts spread over the rest of the
    // iteration: before the QK products, after the combine and after PV.  With
    // eight KV heads of one wave each (batch 64, 32 q / 8 KV heads, 64 tokens
    // of 1,104-byte rows) nothing goes before the products and half after
    // each of the other two points: 55.0 against 55.4 us per launch.  At the
    // other shapes thirds measured best (at 64 q / 8 KV heads, batch 8,
    // 32K-128K keys, the late split cost 1-3 us; issuing everything before the
    // products cost 2-6 us at both).
    constexpr bool LATE = D == 128 && NKV == 8 && WPK == 1;
    constexpr int K1 = LATE ? 0 : (S::NOPS + 2) / 3;
    constexpr int K2 = LATE ? (S::NOPS + 1) / 2 : (2 * S::NOPS + 2) / 3;
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
    v4i C[RB];
    qk(R, C);
    float s[4];
    combine(C, s);
    if (more) loads(nx, IC1{}, IC2{});
    softmax(R, s, (info & 63) + 1);
    pv(R);
    if (more) loads(nx, IC2{}, IC3{});
    const bool last_of_seq = (info >> 6) & 1;
    if (last_of_seq || t == hi - 1) finish(info >> 8, seg_first, seg_whole, last_of_seq);
  };
  for (int t = lo; t < hi; t += 2) {
    iteration(t, std::integral_constant<int, 0>{});
    if (t + 1 < hi) iteration(t + 1, std::integral_constant<int, 1>{});
  }
  flush();
  // Split sequences are merged, and empty sequences zeroed, by merge_kernel,
  // launched after this kernel on the same stream.
}

// Merge of the split sequences (and zeros for empty ones), launched after the
// decode kernel on the same stream: split_merge in attention_kernel.h.
template <int D>
__global__ void __launch_bounds__(128) merge_kernel(const AttnParams p) {
  split_merge<D, 64>(p);
}

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
template <int D, int NKV, int WPK>
static const char* kernel_name() {
  static const std::string n = "mfma_kernel<" + std::to_string(D) + "," + std::to_string(NKV) + "," +
                               std::to_string(WPK) + "> (matrix cores)";
  return n.c_str();
}

template <int D, int NKV, int WPK>
static int launch(AttnParams p, int groups, hipStream_t stream) {
  using S = Shape<D, NKV, WPK>;
  auto kern = mfma_kernel<D, NKV, WPK>;
  const int per_cu = blocks_per_cu(reinterpret_cast<const void*>(kern), S::THREADS, S::LDS);
  const int cus = device_cu_count();
  int W = std::max(1, cus * std::max(1, per_cu) / groups);
  if (W > p.W) W = p.W;          // the workspace holds partials for p.W workgroups
  p.W = W;
  p.nthreads = S::THREADS;
  p.heads_per_group = 4 * S::WAVES;
  hipEvent_t ev0, ev1;
  if (kernel_timing_events(&ev0, &ev1, kernel_name<D, NKV, WPK>()))
    hipExtLaunchKernelGGL(kern, dim3(W, groups), dim3(S::THREADS), S::LDS, stream, ev0, ev1, 0, p);
  else
    hipLaunchKernelGGL(kern, dim3(W, groups), dim3(S::THREADS), S::LDS, stream, p);
  if (int rc = check_launch("paged decode")) return rc;
  if (p.B > 0) {
    constexpr int MH = split_merge_heads<D>();
    hipLaunchKernelGGL((merge_kernel<D>), dim3(p.B, (p.H + MH - 1) / MH), dim3(128), 0, stream, p);
    return check_launch("paged decode merge");
  }
  return 0;
}

}  // namespace mrows

// The matrix-core kernel serves whole-row shapes whose 64-token tile splits
// into whole blocks per wave (4 or 8 waves per workgroup).  SLMT_PAGED_DECODE=valu
// selects the vector-ALU whole-row kernel instead.
bool mfma_rows_enabled(int D, int nkv, int wpk) {
  const int waves = nkv * wpk;
  if ((D != 64 && D != 128) || (waves != 4 && waves != 8)) return false;
  const char* e = std::getenv("SLMT_PAGED_DECODE");
  return !(e && std::strcmp(e, "valu") == 0);
}

#define SLMT_MROWS_CONFIGS(X) \
  X(128, 8, 1) X(128, 4, 1) X(128, 4, 2) X(128, 2, 2) X(64, 8, 1) X(64, 4, 1) X(64, 4, 2) X(64, 2, 2)
#define SLMT_MROWS_KEY(d, a, b) ((d) * 100 + (a) * 10 + (b))

int launch_attention_mfma(int D, int nkv, int wpk, int groups, const AttnParams& p, hipStream_t stream) {
  switch (SLMT_MROWS_KEY(D, nkv, wpk)) {
#define SLMT_MROWS_LAUNCH(d, a, b) case SLMT_MROWS_KEY(d, a, b): return mrows::launch<d, a, b>(p, groups, stream);
    SLMT_MROWS_CONFIGS(SLMT_MROWS_LAUNCH)
#undef SLMT_MROWS_LAUNCH
    default: return fail(SLMT_ERR_INVALID, "paged decode: no matrix-core kernel for this shape");
  }
}

}  // namespace slmt
