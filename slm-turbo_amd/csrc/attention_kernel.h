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
// * Work split: the tokens of all sequences are cut into tiles (32 tokens on
//   the direct-load path, 16 otherwise); the concatenated tile list is
//   divided evenly over W workgroups ("stream-K").  A workgroup walks its
//   tile range, which may cover the end of one sequence, whole sequences and
//   the start of another.  A sequence split over several workgroups is
//   merged by the last workgroup to finish its piece (log-sum-exp merge of
//   (m, l, o) partials; arrival counter per sequence), so one launch
//   produces the final output.  Arrivals are counted once the workgroup has
//   finished its whole range, so the load pipeline never drains in the
//   middle of it.
// * Staging, paged fast path (power-of-two block >= 16 tokens, 4 query heads
//   per KV head): each wave owns one KV head and a private LDS ring of
//   DSTAGE stages.  A 32-token tile of that head is two runs of 16
//   consecutive slots; the wave copies the K/V bytes and rulers of those
//   slots straight into its ring with 16-byte direct loads
//   (global_load_lds_dwordx4, no VGPRs), DSTAGE-1 tiles ahead, and waits for
//   them with an exact vmcnt -- no workgroup barrier anywhere in the loop.
//   The query rows of a new sequence ride in the same ring.  Block-table
//   entries for 64 tiles at a time are gathered into per-lane descriptors
//   and read back with readlane, so the loop issues no table loads.
// * Staging, general path (other layouts): the next tile's 8-byte chunks are
//   held in registers while the current one is computed, double-buffered.
// * QK (lane = token p x query head g of the wave's 4 heads): the fp16 query
//   is used exactly, scaled by a power of two; each key dword becomes four
//   fp16 pairs of subnormal integer codes (four masks) that v_dot2c_f32_f16
//   multiplies exactly with the matching query pairs, accumulating in fp32
//   (key_pairs / query_pairs below).  The per-token affine dequant is folded
//   in algebraically: q.K = step * q.n + min * sum(q).  The per-channel
//   layout multiplies the query by k_scale first and carries the product as
//   an fp16 pair plus its fp16 remainder (two products per pair).
// * Softmax: online, base 2 (log2(e)/sqrt(D) folded into the score scale),
//   per-tile max via DPP row rotations and permlane16/32 swaps.
// * PV (lane = packed byte j, i.e. dims 2j and 2j+1, for all 4 heads):
//   v_dot2c_f32_f16 over token pairs.  The two tokens' bytes are packed into
//   one dword (bytes at bits 0 and 16) and read as an fp16 pair of
//   subnormals, (lo + 16 hi) * 2^-24, which the instruction multiplies
//   exactly; a second product with the low nibbles alone (one AND) separates
//   the two dims.  Weights are p * step in fp16; the softmax sums use the
//   probability each fp16 weight stands for, so the output is an exact
//   weighted mean of the dequantized rows; accumulation is fp32; the
//   per-token min enters once per token as sum(p * min).
#pragma once

#include "slmt_internal.h"

#include <type_traits>

namespace slmt {
namespace attn {

constexpr int TILE = 16;           // tokens per tile, register-staged path
constexpr int DTILE = 32;          // tokens per tile, direct-load path
constexpr int WSCR = 1024;         // per-wave LDS scratch bytes (query pairs / weights)
constexpr int MAX_THREADS = 512;   // 8 waves: up to 256 VGPRs per wave
constexpr int MAXP = 5;            // 8-byte chunks prefetched per thread (general path)
constexpr int DSTAGE = 3;          // LDS ring depth of the direct-load path
constexpr int DHEADS = 32;         // query heads (4 per wave) per workgroup, direct-load path
constexpr int QSLOT = 1024;        // LDS bytes of one wave's query rows in a ring slot

__device__ __forceinline__ float readlane_f(float x, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }
// Lane i's 32-bit word, zero-extended when widened (the builtin returns a
// signed int, which would sign-extend the low word of an address).
__device__ __forceinline__ uint32_t readlane_u32(uint32_t x, int i) {
  return (uint32_t)__builtin_amdgcn_readlane((int)x, i);
}

__device__ __forceinline__ float fdot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
}

// Two bytes at bits 0-7 and 16-23 (zero elsewhere): one v_perm_b32.
__device__ __forceinline__ uint32_t pack_pair(uint32_t b0, uint32_t b1) {
  return __builtin_amdgcn_perm(b1, b0, 0x0C040C00u);
}

// QK on the exact fp16 query.  A key dword x holds dims 8i..8i+7 (dim 8i+j in
// nibble j).  Four masks turn it into fp16 pairs of subnormal integers,
//   (n0, n4), (16 n1, 16 n5), (n2, n6), (16 n3, 16 n7)   (value = bits * 2^-24),
// and v_dot2c_f32_f16 multiplies each pair exactly with the matching query
// pair, (q0, q4), (q1/16, q5/16), (q2, q6), (q3/16, q7/16), accumulating in
// fp32.  The query is first scaled by a power of two so that max|q| lies in
// [2^14, 2^15): every scaled value and every q/16 is then an fp16 number
// whose product with a code is exact, and only values below 2^-24 of max|q|
// lose bits.  The dot is therefore q.n * 2^-24 (scaled) to fp32 accuracy.
__device__ __forceinline__ void key_pairs(uint32_t x, uint32_t (&P)[4]) {
  const uint32_t y = x >> 8;
  P[0] = x & 0x000F000Fu;
  P[1] = x & 0x00F000F0u;
  P[2] = y & 0x000F000Fu;
  P[3] = y & 0x00F000F0u;
}
__device__ __forceinline__ uint32_t half_pair(float a, float b) {
  return (uint32_t)f2h(a) | ((uint32_t)f2h(b) << 16);
}
// Query pairs of dims 8i..8i+7 (qs already scaled), in key_pairs' order.
__device__ __forceinline__ void query_pairs(const float (&qs)[8], uint32_t (&Q)[4]) {
  Q[0] = half_pair(qs[0], qs[4]);
  Q[1] = half_pair(qs[1] * 0.0625f, qs[5] * 0.0625f);
  Q[2] = half_pair(qs[2], qs[6]);
  Q[3] = half_pair(qs[3] * 0.0625f, qs[7] * 0.0625f);
}
// Exponent e such that amax * 2^e lies in [2^14, 2^15) (0 for amax == 0).
// Scores are then kept as u = step * dot + min * sum(q_scaled) * 2^-24, i.e.
// q.K * 2^(e - 24), so the base-2 logit is u * log2(e)/sqrt(D) * 2^(24 - e).
__device__ __forceinline__ int query_exponent(float amax) {
  return amax > 0.f ? 15 - __builtin_amdgcn_frexp_expf(amax) : 0;
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

// Direct-load pipeline wait: until at most N of this wave's vector memory
// operations are outstanding.  Its direct loads retire in issue order, so
// every load older than the newest N has landed in LDS.  The asm is a
// compiler memory barrier: no LDS access moves across it.
template <int N>
__device__ __forceinline__ void vm_wait_n() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Wait until tile t's loads have landed when `ahead` later tiles (OPS loads
// each, plus possibly query loads) have been issued after it: at most
// OPS * ahead operations may still be outstanding.  Extra later operations
// only make the wait stricter.
template <int OPS>
__device__ __forceinline__ void vm_wait_tiles(int ahead) {   // ahead wave-uniform, 0 .. DSTAGE-2
  static_assert(DSTAGE >= 2 && DSTAGE <= 4, "one case per possible look-ahead");
  if (DSTAGE > 3 && ahead >= 2) vm_wait_n<2 * OPS>();
  else if (DSTAGE > 2 && ahead >= 1) vm_wait_n<OPS>();
  else vm_wait_n<0>();
}

// One 16-byte direct load per lane: global (sbase + voff) -> LDS byte address
// lds + 16 * lane.  Issued from asm so that the compiler's wait insertion
// does not treat every later LDS read as a possible alias of the load (it
// would wait for all of them); completion is tracked by vm_wait_barrier.
// M0 carries the LDS base; nothing else in these kernels uses M0.  The loads
// are non-temporal (nt): every cache byte is read once per decode step, and
// the streaming policy keeps it from displacing useful lines in L2 and the
// Infinity Cache (measured: 13 % less time for the load stream of a 303 MB
// cache).  NT = false keeps the default policy, for data that a second
// workgroup reads too.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <bool NT = true>
__device__ __forceinline__ void lds_load16(const void* sbase, uint32_t voff, uint32_t lds) {
  // the base and the LDS address are wave-uniform; readfirstlane keeps them in
  // SGPRs even where the compiler has them in VGPRs (divergent code)
  const uint64_t b = reinterpret_cast<uint64_t>(sbase);
  const uint64_t bs = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b) |
                      ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32)) << 32);
  if constexpr (NT)
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff),
                 "s"(reinterpret_cast<const void*>(bs)), "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff),
                 "s"(reinterpret_cast<const void*>(bs)), "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// Partial results cross workgroups (and XCDs) through the workspace.  They
// are written and read with relaxed agent-scope atomics, which the hardware
// performs coherently at device scope (write-through / past the per-XCD L2),
// so publishing them needs only a wait for the stores to complete -- no L2
// write-back or invalidate, which a release/acquire fence would issue.
__device__ __forceinline__ void store_pair_agent(float* dst, float a, float b) {
  const uint64_t v = (uint64_t)__builtin_bit_cast(uint32_t, a) | ((uint64_t)__builtin_bit_cast(uint32_t, b) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(dst), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 load_pair_agent(const float* src) {
  const uint64_t v = __hip_atomic_load(reinterpret_cast<const uint64_t*>(src), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__builtin_bit_cast(float, (uint32_t)v), __builtin_bit_cast(float, (uint32_t)(v >> 32)));
}
// Wait for all of this wave's vector memory operations (the agent-scope
// partial stores among them) to complete.
__device__ __forceinline__ void vm_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Scalar (SMEM) loads of wave-uniform table entries.  Reading through the
// constant address space makes the compiler use s_load, which is counted by
// lgkmcnt and so never waits on the vector loads that stream the cache.
typedef const __attribute__((address_space(4))) int32_t c_i32;
typedef const __attribute__((address_space(4))) int64_t c_i64;
__device__ __forceinline__ int32_t sload_i32(const void* base, int64_t idx) {
  return ((c_i32*)base)[idx];
}
__device__ __forceinline__ int64_t sload_i64(const void* base, int64_t idx) {
  return ((c_i64*)base)[idx];
}

// Length of sequence b; `b` must be wave-uniform (scalar load).
__device__ __forceinline__ int seq_len_of(const AttnParams& p, int b) {
  if (b >= p.B) return 0;
  int L = p.seq_lens ? sload_i32(p.seq_lens, b) : (p.causal_rows ? min(p.fixed_len, b + 1) : p.fixed_len);
  return L < 0 ? 0 : L;
}
// Same for a per-lane b (vector load).
__device__ __forceinline__ int seq_len_lane(const AttnParams& p, int b) {
  if (b >= p.B) return 0;
  int L = p.seq_lens ? p.seq_lens[b] : (p.causal_rows ? min(p.fixed_len, b + 1) : p.fixed_len);
  return L < 0 ? 0 : L;
}
template <int TT>
__device__ __forceinline__ int tiles_of(int L) { return (L + TT - 1) / TT; }

// First tile of workgroup w when T tiles are split over Weff workgroups.
__device__ __forceinline__ int range_start(int w, int T, int Weff) {
  return (int)(((long long)w * T) / Weff);
}
// Workgroup whose range holds tile t.
__device__ __forceinline__ int range_owner(int t, int T, int Weff) {
  return (int)((((long long)t + 1) * Weff - 1) / T);
}

// Walks the concatenated tile list.  Lnext, the length of sequence b+1, is
// loaded when the cursor enters b, so crossing into b+1 does not wait on it.
struct Cursor {
  int b, tb, Tb, Lb, Pb;   // sequence, tile in sequence, tiles/length of b, first global tile of b
  int Lnext;
};

template <int TT>
__device__ __forceinline__ void cursor_next(const AttnParams& p, Cursor& c) {
  c.tb++;
  if (c.tb >= c.Tb) {
    c.Pb += c.Tb;
    c.tb = 0;
    c.b++;
    c.Lb = c.Lnext;
    c.Tb = tiles_of<TT>(c.Lb);
    while (c.Tb == 0 && c.b < p.B) {
      c.b++;
      c.Lb = seq_len_of(p, c.b);
      c.Tb = tiles_of<TT>(c.Lb);
    }
    c.Lnext = seq_len_of(p, c.b + 1);
  }
}

// Physical block of logical block idx of sequence b (wave-uniform arguments).
__device__ __forceinline__ int64_t block_of(const AttnParams& p, int b, int idx) {
  const int64_t e = (int64_t)b * p.bt_stride + idx;
  if (p.bt64) return sload_i64(p.block_tables, e);
  return sload_i32(p.block_tables, e);
}
// Same for a per-lane block index (vector load).
__device__ __forceinline__ int64_t block_of_lane(const AttnParams& p, int b, int idx) {
  const int64_t e = (int64_t)b * p.bt_stride + idx;
  if (p.bt64) return reinterpret_cast<const int64_t*>(p.block_tables)[e];
  return reinterpret_cast<const int32_t*>(p.block_tables)[e];
}

// Stream-K schedule shared by the attention kernels: the concatenated tile
// list of all sequences (TT tokens per tile) split evenly over the effective
// workgroup count.  Every thread of the workgroup calls it; it writes zeros
// for sequences of length 0 (spread over the workgroups, heads [h0, h1)) and
// returns false when this workgroup has no tiles.  misc: LDS scratch of at
// least 24 ints.
struct TileRange {
  int T, Weff, lo, hi;   // total tiles, workgroups in use, this workgroup's [lo, hi)
  int b, Pb;             // sequence holding tile lo and its first global tile
};

// Writes zeros for the sequences of length 0 that workgroup blockIdx.x owns
// (every Weff-th sequence), heads [h0, h1).
template <int D>
__device__ void zero_empty(const AttnParams& p, int h0, int h1, int Weff) {
  const int tid = threadIdx.x, NT = blockDim.x;
  for (int b = blockIdx.x; b < p.B; b += Weff) {
    if (seq_len_of(p, b) == 0) {
      for (int e = tid; e < (h1 - h0) * D; e += NT) {
        const int h = h0 + e / D, d = e % D;
        const int64_t o = (int64_t)b * p.out_seq_stride + (int64_t)h * p.out_head_stride + d;
        if (p.out_f16) reinterpret_cast<uint16_t*>(p.out)[o] = 0;
        else reinterpret_cast<float*>(p.out)[o] = 0.0f;
      }
    }
  }
}

// ZERO: zero the empty sequences' outputs here; otherwise the caller calls
// zero_empty itself once it has a range (always done here when no workgroup
// has tiles).  stash (LDS, optional): receives the lengths of sequences
// 0 .. stash_n - 1, visible to the whole workgroup on return.
template <int TT, int D, bool ZERO = true>
__device__ bool schedule_range(const AttnParams& p, int* misc, int h0, int h1, TileRange& r, int* stash = nullptr,
                               int stash_n = 0) {
  const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
  const int NT = blockDim.x, nwaves = NT >> 6;
  // exclusive scan of the per-sequence tile counts (threads own contiguous chunks)
  int my_excl, mysum = 0;
  const int chunk = (p.B + NT - 1) / NT;
  const int cb0 = min(p.B, tid * chunk), cb1 = min(p.B, cb0 + chunk);
  for (int b = cb0; b < cb1; ++b) {
    const int L = seq_len_lane(p, b);
    if (b < stash_n) stash[b] = L;
    mysum += tiles_of<TT>(L);
  }
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
    r.T = uniform(misc[nwaves]);
  }
  r.Weff = max(1, min(p.W, (r.T + p.min_tiles - 1) / p.min_tiles));
  const int wg = blockIdx.x;
  if (wg >= r.Weff) return false;
  if (ZERO || r.T == 0) zero_empty<D>(p, h0, h1, r.Weff);
  if (r.T == 0) return false;
  r.lo = range_start(wg, r.T, r.Weff);
  r.hi = range_start(wg + 1, r.T, r.Weff);
  // locate the sequence holding tile lo (lengths from the stash where it holds
  // them: this thread wrote them above, and a global re-read would add a
  // dependent round trip to every workgroup's start)
  if (r.lo >= my_excl && r.lo < my_excl + mysum) {
    int run = my_excl;
    for (int b = cb0; b < cb1; ++b) {
      const int t = tiles_of<TT>(b < stash_n ? stash[b] : seq_len_lane(p, b));
      if (r.lo < run + t) {
        misc[20] = b;
        misc[21] = run;
        break;
      }
      run += t;
    }
  }
  lds_barrier();
  r.b = uniform(misc[20]);
  r.Pb = uniform(misc[21]);
  return true;
}

// Last-arriver merge of sequence b (tiles [Pb, Pb + Tb) of T over Weff
// workgroups): combines the (m, l, o) partials of every piece and writes the
// output of heads [h0, h1).  Pieces are read agent-coherently (past this
// XCD's L2) after the arrival counter showed that all of them were
// published.  A work item is one pair of dims, consecutive items on
// consecutive lanes (each load instruction reads whole 64-byte lines); a
// thread merges IPT items at once, MB pieces per batch, with all of a batch's
// loads issued together, and updates the running maximum once per batch.  For
// the per-channel layout the V scale/zero are applied to the merged average.
// The arrival counter is re-armed at the end.
template <int D, int MODE>
__device__ void merge_sequence(const AttnParams& p, int b, int Pb, int Tb, int T, int Weff, int h0, int h1,
                               int group) {
  static_assert(D % 2 == 0, "work items of 2 dims");
  constexpr int MB = 4, IPT = 4;
  auto load2 = [&](const float* src) -> float2 { return load_pair_agent(src); };
  const int tid = threadIdx.x, NT = blockDim.x, G = p.G;
  const int w_first = range_owner(Pb, T, Weff);
  const int w_last = range_owner(Pb + Tb - 1, T, Weff);
  const int first_slot = (range_start(w_first, T, Weff) == Pb) ? 0 : 1;
  const int total = (h1 - h0) * (D / 2);
  for (int e0 = tid; e0 < total; e0 += NT * IPT) {
    int hh[IPT], dd[IPT];
    float M[IPT], Lsum[IPT];
    float2 O[IPT];
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
      const int e = min(e0 + k * NT, total - 1);   // past the end: a repeat of the last item, not written
      hh[k] = h0 + e / (D / 2);
      dd[k] = (e - (e / (D / 2)) * (D / 2)) * 2;
      M[k] = -INFINITY;
      Lsum[k] = 0.f;
      O[k] = make_float2(0.f, 0.f);
    }
    for (int w0 = w_first; w0 <= w_last; w0 += MB) {
      float2 ml[MB][IPT], o[MB][IPT];
#pragma unroll
      for (int i = 0; i < MB; ++i) {
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
          ml[i][k] = make_float2(-INFINITY, 0.f);
          o[i][k] = make_float2(0.f, 0.f);
        }
        if (w0 + i <= w_last) {               // uniform: the batch's pieces only
          const int w = w0 + i;
          const int64_t base = ((int64_t)w * 2 + (w == w_first ? first_slot : 0)) * p.H;
#pragma unroll
          for (int k = 0; k < IPT; ++k) {
            ml[i][k] = load2(p.part_ml + (base + hh[k]) * 2);
            o[i][k] = load2(p.part_o + (base + hh[k]) * D + dd[k]);
          }
        }
      }
#pragma unroll
      for (int k = 0; k < IPT; ++k) {
        float Mn = M[k];
#pragma unroll
        for (int i = 0; i < MB; ++i) Mn = fmaxf(Mn, ml[i][k].x);
        const float a = __builtin_amdgcn_exp2f(M[k] - Mn);   // 0 for the first batch (M = -inf)
        Lsum[k] *= a;
        O[k].x *= a;
        O[k].y *= a;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          const float sc = __builtin_amdgcn_exp2f(ml[i][k].x - Mn);   // 0 past the last piece
          Lsum[k] += sc * ml[i][k].y;
          O[k].x += sc * o[i][k].x;
          O[k].y += sc * o[i][k].y;
        }
        M[k] = Mn;
      }
    }
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
      if (e0 + k * NT >= total) continue;
      const int h = hh[k], d = dd[k];
      const float rL = __builtin_amdgcn_rcpf(Lsum[k]);
      float r[2] = {O[k].x * rL, O[k].y * rL};
      if constexpr (MODE == SRC_CHANNEL) {
        if (p.use_quant) {
          const int64_t kvg = h / G;
#pragma unroll
          for (int j = 0; j < 2; ++j) r[j] = h2f(p.vr0[kvg * D + d + j]) * (r[j] - h2f(p.vr1[kvg * D + d + j]));
        }
      }
      const int64_t off = (int64_t)b * p.out_seq_stride + (int64_t)h * p.out_head_stride + d;
      if (p.out_f16) {
        reinterpret_cast<uint16_t*>(p.out)[off] = f2h(r[0]);
        reinterpret_cast<uint16_t*>(p.out)[off + 1] = f2h(r[1]);
      } else {
        reinterpret_cast<float*>(p.out)[off] = r[0];
        reinterpret_cast<float*>(p.out)[off + 1] = r[1];
      }
    }
  }
  if (tid == 0)
    __hip_atomic_store(p.counters + (int64_t)group * p.B + b, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Heads per workgroup of the separate merge: 128 threads, one pair of dims
// each, so a workgroup covers 256 / D heads (one head, looped, past D = 256).
template <int D>
constexpr int split_merge_heads() { return D >= 256 ? 1 : 256 / D; }

// Body of the separate merge kernel that the whole-row decode kernels launch
// after themselves on the same stream (so their partial stores are visible):
// one workgroup of 128 threads per (sequence b = blockIdx.x, heads
// [split_merge_heads<D>() * blockIdx.y, ...)).  It recomputes the stream-K
// split of the decode launch (the same tile counts, total T and workgroup
// count Weff from the same parameters) and, when the sequence spans several
// workgroups, combines their (m, l, o) partials.  Empty sequences get zeros.
// A thread owns one pair of dims of one head and issues the loads of up to
// MB pieces together, so a sequence split over at most MB workgroups costs a
// single round trip after the lengths; the running maximum is updated once
// per batch of MB pieces.
template <int D, int TT>
__device__ void split_merge(const AttnParams& p) {
  constexpr int MH = split_merge_heads<D>(), MB = 16, PAIRS = D / 2, NT = 128;
  static_assert(D % 2 == 0, "work items of 2 dims");
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h0 = blockIdx.y * MH, h1 = min(p.H, h0 + MH);
  __shared__ int red[5];
  int pre = 0, tot = 0;   // tiles before sequence b and in total
  for (int i = tid; i < p.B; i += NT) {
    const int Li = seq_len_lane(p, i);
    const int t = tiles_of<TT>(Li);
    tot += t;
    pre += i < b ? t : 0;
    if (i == b) red[4] = Li;   // the sequence's own length, from the same loads
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    pre += __shfl_xor(pre, o, 64);
    tot += __shfl_xor(tot, o, 64);
  }
  if (lane == 0) {
    red[wave] = pre;
    red[2 + wave] = tot;
  }
  __syncthreads();
  const int Pb = red[0] + red[1], T = red[2] + red[3], L = red[4];
  const int total = (h1 - h0) * PAIRS;
  auto store = [&](int h, int d, float r0, float r1) {
    const int64_t off = (int64_t)b * p.out_seq_stride + (int64_t)h * p.out_head_stride + d;
    if (p.out_f16) {
      reinterpret_cast<uint16_t*>(p.out)[off] = f2h(r0);
      reinterpret_cast<uint16_t*>(p.out)[off + 1] = f2h(r1);
    } else {
      reinterpret_cast<float*>(p.out)[off] = r0;
      reinterpret_cast<float*>(p.out)[off + 1] = r1;
    }
  };
  if (L == 0) {
    for (int e = tid; e < total; e += NT) store(h0 + e / PAIRS, (e % PAIRS) * 2, 0.f, 0.f);
    return;
  }
  const int Tb = tiles_of<TT>(L);
  const int Weff = max(1, min(p.W, (T + p.min_tiles - 1) / p.min_tiles));
  const int w_first = range_owner(Pb, T, Weff), w_last = range_owner(Pb + Tb - 1, T, Weff);
  if (w_first == w_last) return;   // one workgroup wrote the output
  const int first_slot = (range_start(w_first, T, Weff) == Pb) ? 0 : 1;
  for (int e = tid; e < total; e += NT) {
    const int h = h0 + e / PAIRS, d = (e % PAIRS) * 2;
    float M = -INFINITY, Ls = 0.f, O0 = 0.f, O1 = 0.f;
    for (int w0 = w_first; w0 <= w_last; w0 += MB) {
      float2 ml[MB], o[MB];
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        ml[i] = make_float2(-INFINITY, 0.f);
        o[i] = make_float2(0.f, 0.f);
        const int w = w0 + i;
        if (w <= w_last) {   // uniform: the batch's pieces only
          const int64_t slot = ((int64_t)w * 2 + (w == w_first ? first_slot : 0)) * p.H + h;
          ml[i] = *reinterpret_cast<const float2*>(p.part_ml + slot * 2);
          o[i] = *reinterpret_cast<const float2*>(p.part_o + slot * D + d);
        }
      }
      float Mn = M;
#pragma unroll
      for (int i = 0; i < MB; ++i) Mn = fmaxf(Mn, ml[i].x);
      const float a = __builtin_amdgcn_exp2f(M - Mn);   // 0 for the first batch (M = -inf)
      Ls *= a;
      O0 *= a;
      O1 *= a;
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        const float sc = __builtin_amdgcn_exp2f(ml[i].x - Mn);   // 0 past the last piece
        Ls += sc * ml[i].y;
        O0 += sc * o[i].x;
        O1 += sc * o[i].y;
      }
      M = Mn;
    }
    const float rL = __builtin_amdgcn_rcpf(Ls);
    store(h, d, O0 * rL, O1 * rL);
  }
}

// Tile loader of the general path: chunk c of a tile is 8 bytes; a thread
// owns chunks tid + k*NT.  The first MAXP chunks of a thread are prefetched
// into registers; further chunks (very wide rows) are copied at commit time.
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
        const int64_t phys = block_of_lane(p, b, (int)blk);
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

  __device__ void issue(const AttnParams& p, int NT, int total, int cpr, int row_lds, int kv_lo, int b, int tok0,
                        int Lb) {
#pragma unroll
    for (int k = 0; k < MAXP; ++k) {
      const int c = (int)threadIdx.x + k * NT;
      dst[k] = -1;
      if (c < total) {
        bool ok;
        int off;
        reg[k] = fetch(p, c, cpr, row_lds, kv_lo, b, tok0, Lb, off, ok);
        dst[k] = ok ? off : -1;
      }
    }
  }

  __device__ void commit(const AttnParams& p, int NT, uint8_t* stage, int total, int cpr, int row_lds, int kv_lo,
                         int b, int tok0, int Lb) {
#pragma unroll
    for (int k = 0; k < MAXP; ++k)
      if (dst[k] >= 0) *reinterpret_cast<uint2*>(stage + dst[k]) = reg[k];
    for (int c = (int)threadIdx.x + MAXP * NT; c < total; c += NT) {
      bool ok;
      int off;
      const uint2 v = fetch(p, c, cpr, row_lds, kv_lo, b, tok0, Lb, off, ok);
      if (ok) *reinterpret_cast<uint2*>(stage + off) = v;
    }
  }
};

// LDS geometry of a register-staged launch; the host computes the same
// numbers for the dynamic LDS size.
struct LdsGeom {
  int row_bytes, row_lds, stage_bytes;
  int wscr, misc, total;                  // byte offsets / total size
};

__host__ __device__ inline LdsGeom lds_geom(int nkv, int D, int waves) {
  LdsGeom g;
  g.row_bytes = nkv * (D + 8);
  // rows padded to an odd multiple of 8 bytes: conflict-free K reads
  g.row_lds = g.row_bytes + ((g.row_bytes & 15) == 0 ? 8 : 0);
  g.stage_bytes = (TILE * g.row_lds + 15) & ~15;
  g.wscr = 2 * g.stage_bytes;
  g.misc = g.wscr + waves * WSCR;
  g.total = g.misc + 32 * (int)sizeof(int);
  return g;
}

// Direct-load path (paged cache, the 4 query heads of every wave sharing one
// KV head): a wave copies its KV head's slot of each of the tile's 32 cache
// rows.  A slot is D+8 = 8 mod 16 bytes, so it starts 0 or 8 bytes into a
// 16-byte unit and spans dma_units(D) units; with an even number of KV heads
// (cache rows a multiple of 16 bytes) the widened slot never leaves its row.
// Rows 0-15 and 16-31 of a tile are 16 consecutive slots of one block each;
// the one load whose 64 units straddle the two halves is issued twice, each
// time for the lanes of one half.
__host__ __device__ constexpr int dma_units(int D) { return (D + 8 + 8 + 15) / 16; }
__host__ __device__ constexpr int dma_ops(int D) { return (DTILE * dma_units(D) + 63) / 64; }
__host__ __device__ constexpr int dma_split(int D) {   // load holding unit 16*units, or -1 if on a boundary
  return (16 * dma_units(D)) % 64 ? (16 * dma_units(D)) / 64 : -1;
}
__host__ __device__ constexpr int dma_issues(int D) { return dma_ops(D) + (dma_split(D) >= 0 ? 1 : 0); }

// Per-wave LDS region of the direct-load path: DSTAGE tile stages of
// dma_ops(D) KB, DSTAGE query slots, the query-pair/weight scratch; misc follows
// the last wave's region.
struct DmaGeom {
  int stage_bytes, wave_bytes, qslots, wscr, misc, total;
};

__host__ __device__ inline DmaGeom dma_geom(int D, int waves) {
  DmaGeom g;
  g.stage_bytes = dma_ops(D) * 1024;
  g.qslots = DSTAGE * g.stage_bytes;
  g.wscr = g.qslots + DSTAGE * QSLOT;
  g.wave_bytes = g.wscr + WSCR;
  g.misc = waves * g.wave_bytes;
  g.total = g.misc + 32 * (int)sizeof(int);
  return g;
}

// Per-lane state and per-tile math of one wave: 4 query heads of the
// workgroup's head group, TOK (16 or 32) tokens per tile.  In QK a lane owns
// query head g = lane & 3 and tokens p, p + 16, ... (p = lane >> 2).
template <int D, int MODE, bool SHARED, int TOK>
struct Heads {
  static constexpr int SLOT = D + 8;
  static constexpr int KD = D / 8;              // key dwords per token (8 dims each)
  static constexpr int VB = D / 2;              // value bytes per token
  static constexpr int NQ = TOK / 16;           // tokens per QK lane
  static constexpr int PH = (D == 64) ? 2 : 1;  // PV token phases (two half-waves for D = 64)
  static constexpr int PAIRS = TOK / 2 / PH;    // token pairs per PV lane per tile
  static constexpr float kC = 1.4426950408889634f /
      (D == 64 ? 8.0f : (D == 128 ? 11.313708498984761f : 8.94427190999916f));  // log2(e)/sqrt(D)

  int qp, qg, hq, kvl, pj, pph, jj;
  bool hvalid;
  int kvw[4];
  bool hw[4];
  // Query pairs of this lane's head for every key dword (key_pairs order);
  // the per-channel layout folds k_scale into the query, q' = q * s exactly
  // in fp32, and carries it as an fp16 high part and its fp16 remainder.
  static constexpr int QP = MODE == SRC_CHANNEL ? 8 : 4;
  uint32_t qpr[KD][QP];
  // m_run: the weight reference of the lane's head in base-2 logits (the
  // running max, or kRefDrop / 2 above a later tile's max more than kRefDrop
  // below it); m_top: the running max.
  float qa, qb, m_run, m_top, l_run, vmt;
  float acc[4][2];   // per head: sum w*lo, sum w*(lo + 16 hi), in units of 2^-24

  __device__ void setup(int lane, int wave, int h0, int h1, int G, int kv_lo) {
    qp = lane >> 2;
    qg = lane & 3;
    hq = h0 + wave * 4 + qg;
    hvalid = hq < h1;
    kvl = hvalid ? hq / G - kv_lo : 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int h = h0 + wave * 4 + g;
      hw[g] = h < h1;
      kvw[g] = hw[g] ? h / G - kv_lo : 0;
    }
    pj = (PH == 2) ? (lane & 31) : lane;
    pph = (PH == 2) ? (lane >> 5) : 0;
    jj = min(pj, VB - 1);
  }

  // Start a sequence: scale this lane's 8 query dims (for the per-channel
  // layout already multiplied by k_scale; zv = k_zero) by the head's power of
  // two and lay out the query pairs of the head's key dwords.
  __device__ void begin(const float (&qv)[8], const float (&zv)[8], uint8_t* wscr) {
    m_run = m_top = -INFINITY;
    l_run = 0.f;
    vmt = 0.f;
#pragma unroll
    for (int g = 0; g < 4; ++g) acc[g][0] = acc[g][1] = 0.f;
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(qv[i]));
    amax = red16_max(amax);
    const int ex = query_exponent(amax);
    float qs[8], qsum = 0.f, qzsum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      qs[i] = __builtin_amdgcn_ldexpf(qv[i], ex);
      qsum += qs[i];
      if constexpr (MODE == SRC_CHANNEL) qzsum = __builtin_fmaf(qs[i], zv[i], qzsum);
    }
    uint32_t pr[8];
    {
      uint32_t hp[4];
      query_pairs(qs, hp);
#pragma unroll
      for (int k = 0; k < 4; ++k) pr[k] = hp[k];
    }
    if constexpr (MODE == SRC_CHANNEL) {
      float rs[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) rs[i] = qs[i] - h2f(f2h(qs[i]));   // exact remainder
      uint32_t lp[4];
      query_pairs(rs, lp);
#pragma unroll
      for (int k = 0; k < 4; ++k) pr[4 + k] = lp[k];
    }
    qsum = red16_sum(qsum);
    if constexpr (MODE == SRC_CHANNEL) qzsum = red16_sum(qzsum);
    // The table holds 4 pairs per (head, key dword): one pass per group of 4.
    uint32_t* wl = reinterpret_cast<uint32_t*>(wscr);
#pragma unroll
    for (int part = 0; part < QP / 4; ++part) {
      wave_lds_sync();                   // previous table / weight reads of this wave are done
      if (qp < KD)
        *reinterpret_cast<uint4*>(wl + (qg * KD + qp) * 4) =
            make_uint4(pr[4 * part], pr[4 * part + 1], pr[4 * part + 2], pr[4 * part + 3]);
      wave_lds_sync();
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) {
        const uint4 v = *reinterpret_cast<const uint4*>(wl + (qg * KD + kd) * 4);
        qpr[kd][4 * part] = v.x;
        qpr[kd][4 * part + 1] = v.y;
        qpr[kd][4 * part + 2] = v.z;
        qpr[kd][4 * part + 3] = v.w;
      }
    }
    // base-2 logit = dot * qa + (ruler terms); the dot is in units of 2^-24
    qa = __builtin_amdgcn_ldexpf(kC, 24 - ex);
    if constexpr (MODE == SRC_CHANNEL) qb = -__builtin_amdgcn_ldexpf(kC * qzsum, -ex);
    else qb = __builtin_amdgcn_ldexpf(kC * qsum, -ex);
  }

  // Score of token row `row` of the tile for this lane's head (base-2 units),
  // and its V rulers for the weights.
  __device__ float score(const uint8_t* S, int row_lds, int row, float& vmin, float& vstep) const {
    const uint8_t* kb = S + row * row_lds + kvl * SLOT;
    float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KD / 2; ++j) {
      const uint2 w = *reinterpret_cast<const uint2*>(kb + 8 * j);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t P[4];
        key_pairs(h ? w.y : w.x, P);
#pragma unroll
        for (int k = 0; k < QP; ++k) a[k & 3] = fdot2(P[k & 3], qpr[2 * j + h][k], a[k & 3]);
      }
    }
    const float x = (a[0] + a[1]) + (a[2] + a[3]);   // q.n * 2^(e - 24)
    if constexpr (MODE == SRC_CHANNEL) {
      vmin = vstep = 0.f;
      return __builtin_fmaf(x, qa, qb);
    } else {
      const uint2 rr = *reinterpret_cast<const uint2*>(kb + D);
      const float kmin = h2f((uint16_t)(rr.x & 0xffffu));
      const float kstep = h2f((uint16_t)(rr.x >> 16));
      vmin = h2f((uint16_t)(rr.y & 0xffffu));
      vstep = h2f((uint16_t)(rr.y >> 16));
      return __builtin_fmaf(x * qa, kstep, kmin * qb);
    }
  }

  // One TOK-token tile staged at S (rows row_lds bytes apart, the staged KV
  // heads side by side); tokens tok0 + p >= Lb are masked.
  __device__ void tile(const uint8_t* S, int row_lds, int tok0, int Lb, uint8_t* wscr) {
    // ---- QK
    float s2[NQ], vmin[NQ], vstep[NQ];
    bool tvalid[NQ];
    float tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      s2[i] = score(S, row_lds, qp + 16 * i, vmin[i], vstep[i]);
      tvalid[i] = hvalid && (tok0 + qp + 16 * i < Lb);
      s2[i] = tvalid[i] ? s2[i] : -INFINITY;
      tmax = fmaxf(tmax, s2[i]);
    }
    // ---- online softmax (reference per head; rescale only when the tile's
    // max exceeds it or lies more than kRefDrop below it)
    tmax = red16_max(tmax);
    const bool grow = tmax > m_run;
    // down to half the threshold above the tile's max (finite: the head has
    // a valid token here), at most kRefFloor below the running max
    const bool drop = !grow && tmax > -INFINITY && tmax < m_run - kRefDrop;
    if (__builtin_amdgcn_ballot_w64(grow || drop)) {
      const float m_new = grow ? tmax : drop ? fmaxf(tmax + 0.5f * kRefDrop, m_top - kRefFloor) : m_run;
      const float alpha = grow || drop ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.f;   // 0 when growing from -inf
      m_top = fmaxf(m_top, tmax);
      l_run *= alpha;
      vmt *= alpha;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float ag = readlane_f(alpha, g);
        acc[g][0] *= ag;
        acc[g][1] *= ag;
      }
      m_run = m_new;
    }
    const float msafe = (m_run == -INFINITY) ? 0.f : m_run;
    // P.V multiplies the codes by fp16 weights; the softmax sums take the
    // probability each fp16 weight stands for (per token: w / step, steps
    // below 2^-10 keep p; per channel: the fp16 p itself), so the output is
    // an exact weighted mean of the dequantized rows.
    uint16_t wv[NQ];
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const float pr = __builtin_amdgcn_exp2f(s2[i] - msafe);   // 0 for masked tokens
      if constexpr (MODE == SRC_CHANNEL) {
        wv[i] = f2h(pr);
        l_run += h2f(wv[i]);
      } else {
        const float st = tvalid[i] ? vstep[i] : 0.f;
        const float mn = tvalid[i] ? vmin[i] : 0.f;
        wv[i] = f2h(pr * st);
        const float pp = st >= 0x1p-10f ? h2f(wv[i]) * __builtin_amdgcn_rcpf(st) : pr;
        l_run += pp;
        vmt = __builtin_fmaf(pp, mn, vmt);
      }
    }
    // weights as fp16 pairs: wscr[pair][head] = (w(2i), w(2i+1))
    wave_lds_sync();                     // query-pair / weight reads of this wave are done
#pragma unroll
    for (int i = 0; i < NQ; ++i)
      reinterpret_cast<uint16_t*>(wscr)[(((qp + 16 * i) >> 1) * 4 + qg) * 2 + (qp & 1)] = wv[i];
    wave_lds_sync();
    // ---- PV
#pragma unroll
    for (int i = 0; i < PAIRS; ++i) {
      const int pr2 = pph * PAIRS + i;
      const uint4 wq = *reinterpret_cast<const uint4*>(wscr + pr2 * 16);
      if constexpr (SHARED) {
        const uint8_t* vb = S + kvw[0] * SLOT + VB + jj;
        const uint32_t tw = pack_pair(vb[(2 * pr2) * row_lds], vb[(2 * pr2 + 1) * row_lds]);
        const uint32_t vlo = tw & 0x000F000Fu;
        acc[0][0] = fdot2(wq.x, vlo, acc[0][0]);
        acc[0][1] = fdot2(wq.x, tw, acc[0][1]);
        acc[1][0] = fdot2(wq.y, vlo, acc[1][0]);
        acc[1][1] = fdot2(wq.y, tw, acc[1][1]);
        acc[2][0] = fdot2(wq.z, vlo, acc[2][0]);
        acc[2][1] = fdot2(wq.z, tw, acc[2][1]);
        acc[3][0] = fdot2(wq.w, vlo, acc[3][0]);
        acc[3][1] = fdot2(wq.w, tw, acc[3][1]);
      } else {
        const uint32_t wgs[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint8_t* vb = S + kvw[g] * SLOT + VB + jj;
          const uint32_t tw = pack_pair(vb[(2 * pr2) * row_lds], vb[(2 * pr2 + 1) * row_lds]);
          acc[g][0] = fdot2(wgs[g], tw & 0x000F000Fu, acc[g][0]);
          acc[g][1] = fdot2(wgs[g], tw, acc[g][1]);
        }
      }
    }
  }

  // End of a segment: lt/vt per head (lane g holds head g's values) and the
  // un-normalized outputs o[g][0..1] of dims 2*pj, 2*pj+1 (valid in the
  // writer lanes): o = sum p*(step*n) ... + sum p*min.
  __device__ void reduce(float& lt, float& vt, float (&o)[4][2]) const {
    lt = red16_sum(l_run);
    vt = (MODE == SRC_CHANNEL) ? 0.f : red16_sum(vmt);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float lo = acc[g][0], full = acc[g][1];
      if constexpr (PH == 2) {
        float a, b2;
        swap32(lo, a, b2);
        lo = a + b2;
        swap32(full, a, b2);
        full = a + b2;
      }
      const float vg = readlane_f(vt, g);
      o[g][0] = lo * 16777216.0f + vg;            // 2^24: nibble-as-subnormal scale
      o[g][1] = (full - lo) * 1048576.0f + vg;    // (16 hi) * 2^-24 -> hi
    }
  }
  __device__ bool writer() const { return (PH == 1 || pph == 0) && pj < VB; }
};

// DMA: paged cache, block_size a power of two >= 16, an even number of KV
// heads (cache rows a multiple of 16 bytes) on a 16-byte aligned base, the 4
// heads of every wave sharing a KV head (plan_attention and launch_attention
// check).
template <int D, int MODE, bool SHARED, bool DMA>
__global__ void __launch_bounds__(MAX_THREADS) attention_kernel(const AttnParams p) {
  constexpr int TT = DMA ? DTILE : TILE;   // tokens per tile
  using HeadsT = Heads<D, MODE, SHARED, TT>;
  static_assert(!DMA || SHARED, "direct loads copy one KV head per wave");
  constexpr int KD = HeadsT::KD;
  constexpr int VB = HeadsT::VB;
  static_assert(!DMA || MODE == SRC_PAGED, "direct loads serve the paged layout only");

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = uniform(tid >> 6);
  const int NT = p.nthreads;
  const int nwaves = NT >> 6;
  const int group = blockIdx.y;
  const int G = p.G;
  const int h0 = group * p.heads_per_group;
  const int h1 = min(p.H, h0 + p.heads_per_group);
  const int kv_lo = h0 / G;
  const int nkv = (h1 - 1) / G - kv_lo + 1;
  // this wave's heads [hw0, min(h1, hwa + 4)) (none for trailing waves of a short last group)
  const int hw0 = h0 + 4 * wave;
  const bool active = hw0 < h1;
  const int hwa = active ? hw0 : h1 - 1;
  const LdsGeom geo = lds_geom(nkv, D, nwaves);
  const DmaGeom dgeo = dma_geom(D, nwaves);
  constexpr int UNITS = dma_units(D), OPS = dma_ops(D), SPLIT = dma_split(D), ISSUES = dma_issues(D);
  // direct-load path: this wave's KV head, its slot's place in the widened
  // slice (kv_w * SLOT = a0 + koff) and the wave's LDS region
  const int kv_w = hwa / G;
  const int a0 = (kv_w * (D + 8)) & ~15, koff = kv_w * (D + 8) - a0;
  uint8_t* const wbase = smem + wave * dgeo.wave_bytes;
  const int row_lds = DMA ? UNITS * 16 : geo.row_lds;
  uint8_t* wscr = DMA ? wbase + dgeo.wscr : smem + geo.wscr + wave * WSCR;
  // misc[0..16]: wave sums of the tile scan; misc[20..27]: broadcast slots
  int* misc = reinterpret_cast<int*>(smem + (DMA ? dgeo.misc : geo.misc));

  // ---------------------------------------------------------------- schedule
  TileRange rng;
  if (!schedule_range<TT, D>(p, misc, h0, h1, rng)) return;
  const int T = rng.T, Weff = rng.Weff, lo = rng.lo, hi = rng.hi;
  const int wg = blockIdx.x;
  Cursor cc;
  cc.b = rng.b;
  cc.Pb = rng.Pb;
  cc.Lb = seq_len_of(p, cc.b);
  cc.Tb = tiles_of<TT>(cc.Lb);
  cc.tb = lo - cc.Pb;
  cc.Lnext = seq_len_of(p, cc.b + 1);

  HeadsT hd;
  hd.setup(lane, wave, h0, h1, G, DMA ? kv_w : kv_lo);

  // ---------------------------------------------------------------- loaders
  // Direct loads: load k of this wave fills 1 KB of its stage; lane l of it
  // moves 16-byte unit u = 64k + l of the wave's slice, tile row r = u / UNITS,
  // column u % UNITS.  Rows 0-15 come from one block (base0), rows 16-31 from
  // another (base1); tokens are cache_row bytes apart.  Units past the 32 rows
  // re-read row 16's first unit into unused LDS.
  const int cache_row = p.cache_kv * (D + 8);
  uint32_t goff[OPS];
  bool split_hi = false;                      // lane of load SPLIT belongs to rows 16-31
  uint32_t qoff = 0;                          // this lane's query byte offset within a sequence
  const uint32_t lds_wave = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)wbase;
  if constexpr (DMA) {
#pragma unroll
    for (int k = 0; k < OPS; ++k) {
      const int u = 64 * k + lane;
      const int r = u / UNITS, c = u - r * UNITS;
      goff[k] = (uint32_t)(r < DTILE ? (r & 15) * cache_row + a0 + c * 16 : a0);
      if (k == SPLIT) split_hi = r >= 16;
    }
    qoff = (hd.hvalid && hd.qp < KD) ? (uint32_t)((hd.hq * p.q_head_stride + hd.qp * 8) * 2) : 0u;
  }
  // DMA: this wave's slice of the tile (rows 0-15 at base0, 16-31 at base1)
  // into ring slot st, plus its query rows of sequence qb (qb >= 0) at a
  // sequence start; exactly ISSUES (+1) loads per call.
  const int64_t blk_bytes = (int64_t)p.block_size * cache_row;
  auto dma_tile = [&](const uint8_t* base0, const uint8_t* base1, int st, int qb) {
    if (!active) return;
    const uint32_t dst = lds_wave + st * dgeo.stage_bytes;
#pragma unroll
    for (int k = 0; k < OPS; ++k) {
      if (k == SPLIT) {
        if (!split_hi) lds_load16(base0, goff[k], dst + k * 1024);
        if (split_hi) lds_load16(base1, goff[k], dst + k * 1024);
      } else {
        lds_load16((64 * k) / UNITS < 16 ? base0 : base1, goff[k], dst + k * 1024);
      }
    }
    if (qb >= 0) lds_load16(p.q + (int64_t)qb * p.q_seq_stride, qoff, lds_wave + dgeo.qslots + st * QSLOT);
  };

  using LoaderT = Loader<D, MODE>;
  LoaderT ld;
  const int cpr = LoaderT::chunks_per_row(nkv);
  const int total_chunks = TT * cpr;

  // Partial pieces whose arrival is counted after the range (at most two:
  // the range's first and last segments): sequence, first tile, tiles.
  int npend = 0;
  int pb0 = 0, pP0 = 0, pT0 = 0, pb1 = 0, pP1 = 0, pT1 = 0;

  // Writes the finished segment [seg_first_tile, t] of sequence c.b.
  auto finish_segment = [&](const Cursor& c, int seg_first_tile, int t) {
    float lt, vt, o[4][2];
    hd.reduce(lt, vt, o);
    const bool complete = (seg_first_tile == c.Pb) && (t == c.Pb + c.Tb - 1);
    const bool wr = hd.writer();
    const int d0 = 2 * hd.pj;
    if (complete) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (!hd.hw[g] || !wr) continue;
        const int h = h0 + wave * 4 + g;
        const float L = readlane_f(lt, g);
        const float rL = __builtin_amdgcn_rcpf(L);
        float r0 = o[g][0] * rL, r1 = o[g][1] * rL;
        if constexpr (MODE == SRC_CHANNEL) {
          if (p.use_quant) {
            const int64_t kvg = h / G;
            r0 = h2f(p.vr0[kvg * D + d0]) * (r0 - h2f(p.vr1[kvg * D + d0]));
            r1 = h2f(p.vr0[kvg * D + d0 + 1]) * (r1 - h2f(p.vr1[kvg * D + d0 + 1]));
          }
        }
        const int64_t off = (int64_t)c.b * p.out_seq_stride + (int64_t)h * p.out_head_stride + d0;
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
        if (!hd.hw[g] || !wr) continue;
        const int h = h0 + wave * 4 + g;
        store_pair_agent(p.part_o + (pbase + h) * D + d0, o[g][0], o[g][1]);
        if (hd.pj == 0) store_pair_agent(p.part_ml + (pbase + h) * 2, readlane_f(hd.m_run, g), readlane_f(lt, g));
      }
      if (npend == 0) {
        pb0 = c.b;
        pP0 = c.Pb;
        pT0 = c.Tb;
      } else {
        pb1 = c.b;
        pP1 = c.Pb;
        pT1 = c.Tb;
      }
      ++npend;
    }
  };

  // Starts the segment of cursor c: query pairs from its 8 dims.
  auto begin_segment = [&](const Cursor& c, const uint8_t* qlds) {
    float qv[8], zv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) qv[i] = zv[i] = 0.f;
    const bool dvalid = hd.hvalid && (hd.qp < KD);
    if (dvalid) {
      uint4 w;
      if constexpr (DMA) {
        w = *reinterpret_cast<const uint4*>(qlds + lane * 16);
      } else {
        const uint16_t* qrow =
            p.q + (int64_t)c.b * p.q_seq_stride + (int64_t)hd.hq * p.q_head_stride + hd.qp * 8;
        w = *reinterpret_cast<const uint4*>(qrow);
      }
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        qv[2 * i] = h2f((uint16_t)(ws[i] & 0xffffu));
        qv[2 * i + 1] = h2f((uint16_t)(ws[i] >> 16));
      }
      if constexpr (MODE == SRC_CHANNEL) {
        if (p.use_quant) {
          const int64_t kvg = kv_lo + hd.kvl;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            qv[i] *= h2f(p.kr0[kvg * D + hd.qp * 8 + i]);          // q' = q * k_scale
            zv[i] = h2f(p.kr1[kvg * D + hd.qp * 8 + i]);           // k_zero
          }
        }
      }
    }
    hd.begin(qv, zv, wscr);
  };

  int seg_first_tile = lo;

  if constexpr (DMA) {
    // ---------------------------------------------------------------- direct-load pipeline
    // Every wave runs its own ring of DSTAGE slots (no workgroup barriers):
    // tiles lo .. lo+DSTAGE-2 are issued up front; iteration t waits for tile
    // t, issues tile t+DSTAGE-1 into the slot tile t-1 used, computes tile t.
    //
    // Tile descriptors are built 64 tiles at a time, lane i for tile
    // dchunk + i: the slot bases of rows 0-15 and 16-31 and the sequence
    // whose query rows ride with the tile (-1 if none).  An issue then reads
    // them with v_readlane instead of walking the block table in scalar code.
    // Block-table entries are read as their low 32 bits (physical blocks are
    // below 2^31: the host checks num_blocks), so 32- and 64-bit tables share
    // the path.
    const int esh = p.bt64 ? 3 : 2;
    const uint8_t* btab = reinterpret_cast<const uint8_t*>(p.block_tables);
    uint32_t d0lo = 0, d0hi = 0, d1lo = 0, d1hi = 0;
    int dq = -1;
    int dchunk = lo;
    // c: cursor at tile `first` (global index)
    auto build = [&](const Cursor& c, int first) {
      const int t = first + lane;
      int b = c.b, P = c.Pb, Tb = c.Tb, L = c.Lb;
      int mb = -1, mtb = 0, mL = 0;
      for (;;) {
        if (t >= P && t < P + Tb) {
          mb = b;
          mtb = t - P;
          mL = L;
        }
        P += Tb;
        if (!__builtin_amdgcn_ballot_w64(t >= P && t < hi) || b + 1 >= p.B) break;
        ++b;
        L = b == c.b + 1 ? c.Lnext : seq_len_of(p, b);
        Tb = tiles_of<TT>(L);
      }
      uint64_t base0 = reinterpret_cast<uint64_t>(p.cache), base1 = base0;
      dq = -1;
      if (mb >= 0 && t < hi) {
        const int tok0 = mtb * DTILE;
        const bool upper = tok0 + 16 < mL;
        const int64_t row_e = (int64_t)mb * p.bt_stride;
        const int32_t e0 = *reinterpret_cast<const int32_t*>(btab + ((row_e + (tok0 >> p.block_shift)) << esh));
        const int32_t e1 =
            upper ? *reinterpret_cast<const int32_t*>(btab + ((row_e + ((tok0 + 16) >> p.block_shift)) << esh)) : e0;
        base0 += (uint64_t)(uint32_t)e0 * (uint64_t)blk_bytes + (uint64_t)((tok0 & (p.block_size - 1)) * cache_row);
        base1 = upper ? reinterpret_cast<uint64_t>(p.cache) + (uint64_t)(uint32_t)e1 * (uint64_t)blk_bytes +
                            (uint64_t)(((tok0 + 16) & (p.block_size - 1)) * cache_row)
                      : base0;
        dq = (mtb == 0 || t == lo) ? mb : -1;
      }
      d0lo = (uint32_t)base0;
      d0hi = (uint32_t)(base0 >> 32);
      d1lo = (uint32_t)base1;
      d1hi = (uint32_t)(base1 >> 32);
      dchunk = first;
    };
    auto issue_desc = [&](int t, int st) {
      const int i = t - dchunk;
      const uint64_t b0 = (uint64_t)readlane_u32(d0lo, i) | ((uint64_t)readlane_u32(d0hi, i) << 32);
      const uint64_t b1 = (uint64_t)readlane_u32(d1lo, i) | ((uint64_t)readlane_u32(d1hi, i) << 32);
      dma_tile(reinterpret_cast<const uint8_t*>(b0), reinterpret_cast<const uint8_t*>(b1), st,
               __builtin_amdgcn_readlane(dq, i));
    };
    Cursor dc = cc;                                 // cursor of the next tile to issue
    build(dc, lo);
    for (int j = 0; j < DSTAGE - 1 && lo + j < hi; ++j) {
      issue_desc(lo + j, (lo + j) % DSTAGE);
      cursor_next<TT>(p, dc);
    }
    int st = lo % DSTAGE;                           // ring slot of tile t
    for (int t = lo; t < hi; ++t) {
      // alternate the two waves of a SIMD (waves w and w+4) in priority
      if (((t - lo) & 7) == 0) {
        if ((((t - lo) >> 3) + (wave >> 2)) & 1) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
      }
      vm_wait_tiles<ISSUES>(min(DSTAGE - 2, hi - 1 - t));
      const int tn = t + DSTAGE - 1;
      if (tn < hi) {
        if (tn - dchunk >= 64) build(dc, tn);
        issue_desc(tn, st == 0 ? DSTAGE - 1 : st - 1);
        cursor_next<TT>(p, dc);
      }
      const bool seg_start = (t == lo) || (cc.tb == 0);
      const bool seg_end = (t == hi - 1) || (cc.tb == cc.Tb - 1);
      if (seg_start) {
        seg_first_tile = t;
        begin_segment(cc, wbase + dgeo.qslots + st * QSLOT);
      }
      hd.tile(wbase + st * dgeo.stage_bytes + koff, row_lds, cc.tb * TT, cc.Lb, wscr);
      if (seg_end) finish_segment(cc, seg_first_tile, t);
      if (t + 1 < hi) cursor_next<TT>(p, cc);
      st = st + 1 == DSTAGE ? 0 : st + 1;
    }
    __builtin_amdgcn_s_setprio(0);
  } else {
    // ---------------------------------------------------------------- register-staged pipeline
    Cursor lc = cc;                          // loader cursor runs one tile ahead
    ld.issue(p, NT, total_chunks, cpr, row_lds, kv_lo, lc.b, lc.tb * TILE, lc.Lb);
    ld.commit(p, NT, smem, total_chunks, cpr, row_lds, kv_lo, lc.b, lc.tb * TILE, lc.Lb);
    if (lo + 1 < hi) {
      cursor_next<TT>(p, lc);
      ld.issue(p, NT, total_chunks, cpr, row_lds, kv_lo, lc.b, lc.tb * TILE, lc.Lb);
    }
    lds_barrier();
    for (int t = lo; t < hi; ++t) {
      const int buf = (t - lo) & 1;
      const bool seg_start = (t == lo) || (cc.tb == 0);
      const bool seg_end = (t == hi - 1) || (cc.tb == cc.Tb - 1);
      if (seg_start) {
        seg_first_tile = t;
        begin_segment(cc, nullptr);
      }
      hd.tile(smem + buf * geo.stage_bytes, row_lds, cc.tb * TILE, cc.Lb, wscr);
      if (seg_end) finish_segment(cc, seg_first_tile, t);
      if (t + 1 < hi) {
        cursor_next<TT>(p, cc);
        // tile t+1 is in registers (issued by the loader cursor); commit it
        ld.commit(p, NT, smem + (buf ^ 1) * geo.stage_bytes, total_chunks, cpr, row_lds, kv_lo, lc.b,
                  lc.tb * TILE, lc.Lb);
        if (t + 2 < hi) {
          cursor_next<TT>(p, lc);
          ld.issue(p, NT, total_chunks, cpr, row_lds, kv_lo, lc.b, lc.tb * TILE, lc.Lb);
        }
        lds_barrier();
      }
    }
  }

  // ---------------------------------------------------------------- arrivals and merges
  if (npend == 0) return;
  // Every wave waits for its own partial stores (agent-coherent) before the
  // arrival is counted; the barrier then covers all waves of the workgroup.
  vm_drain();
  __syncthreads();
  auto arrive = [&](int b, int Pb, int Tb) -> int {
    const int pieces = range_owner(Pb + Tb - 1, T, Weff) - range_owner(Pb, T, Weff) + 1;
    const int prev = __hip_atomic_fetch_add(p.counters + (int64_t)group * p.B + b, 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    return (prev == pieces - 1) ? 1 : 0;
  };
  if (tid == 0) {
    misc[24] = arrive(pb0, pP0, pT0);
    misc[25] = npend > 1 ? arrive(pb1, pP1, pT1) : 0;
  }
  __syncthreads();
  // The last piece to arrive merges every piece of the sequence.
  auto merge = [&](int b, int Pb, int Tb) { merge_sequence<D, MODE>(p, b, Pb, Tb, T, Weff, h0, h1, group); };
  if (misc[24]) merge(pb0, pP0, pT0);
  if (misc[25]) merge(pb1, pP1, pT1);
  (void)VB;
}

}  // namespace attn

// Launch one instantiation (defined in the per-mode translation units).
int launch_attention_paged(int D, bool shared, bool dma, const AttnParams& p, dim3 grid, dim3 block,
                           size_t lds, hipStream_t stream);
int launch_attention_contig(int mode, int D, const AttnParams& p, dim3 grid, dim3 block, size_t lds,
                            hipStream_t stream);

}  // namespace slmt
