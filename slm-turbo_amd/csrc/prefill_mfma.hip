// Per-channel 4-bit prefill attention on the matrix cores (gfx950 MFMA), head_dim 64
// and 128 (reference kernel it replaces: kv_dequant_prefill_kernel,
// kernels/kv_dequant_kernels.cuh:293-502).
//
// Prefill is GEMM-shaped (every key meets up to 64 query rows of a tile), so
// unlike the decode it runs on the matrix cores.  A workgroup takes 64 query rows
// of one query head (of two, for long prefills), one wave per 16 rows of a head,
// and walks the 64-key tiles the rows can see.  Everything is kept transposed,
// so a lane owns one query column from the scores to the output:
//   S^T = K Q'^T     (v_mfma_f32_16x16x32_f16: A = K rows, B = the lane's query)
//   P^T = exp2(S^T - m)      (online softmax per query column)
//   O^T += V^T P^T   (v_mfma_f32_16x16x32_f16: B = the lane's P^T blocks as they are)
//
// Exactness of the operands (a nibble becomes the fp16 1024 + code by one OR with
// the pattern 0x6400; subtracting an integer below 2048 from it is exact):
// * K enters as its codes n.  The reference's q.k = sum q_d s_d (n_d - z_d), and
//   sum q_d s_d z_d is the same for every key of a query row, so it cancels in
//   the softmax and is never formed.
// * The per-channel K scale and the softmax scale log2(e) / sqrt(D) fold into
//   the query: q'_d = q_d * log2(e) / sqrt(D) * s_d in fp32, split into an fp16
//   high part and the fp16 rounding of the remainder; two products per block
//   keep ~22 bits of q'.
// * V enters as n - zr, zr the zero point rounded and clamped to 0..15 (the
//   reference quantizer's zero points are such integers), and the finished row
//   is o_d = s_d * (sum p (n - zr) / l - (z_d - zr_d)) in fp32.
// * P enters in fp16 (relative 2^-11 per weight), as the decode's weights do, and
//   the row sums l are a product of the same fp16 weights with a block of ones,
//   so numerator and denominator see the same rounded weights.
// use_quant = 0 takes the raw codes (scale 1, zero 0).  Causal row m sees keys
// n <= m; keys past S are masked.  S = 0 yields NaN rows (0/0), as the
// reference's kernels do.
//
// A workgroup takes 64 query rows of one query head (4 waves), or of two query
// heads of the same KV head (8 waves) for long prefills; the first four waves
// stage the tiles for all of them.
// Staging: the workgroup converts each tile into a 2-stage LDS ring: K as
// [key][dim] fp16 rows of D*2+32 bytes, V^T as [dim][key] fp16 rows of 160 bytes
// with the keys in the order the P.V product takes them, so that every operand
// read, K and V^T, is one conflict-free 16-byte read (see Geo).  The next tile's
// codes are loaded into registers two tiles ahead and written to LDS after the
// current tile's products; one barrier per tile.  Within a tile, all K operand
// reads are issued before the first QK product and all V^T operand reads
// before the softmax, so LDS latency hides behind the products and the
// exponentials instead of stalling each product.
#include "slmt_internal.h"

#include <type_traits>

namespace slmt {
namespace prefill {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

struct Params {
  const uint16_t* q;                       // [H, M, D] fp16
  const uint8_t* kp;                       // [KV_t, S, D/2] codes
  const uint8_t* vp;
  const uint16_t *ks, *kz, *vs, *vz;       // [KV_t, D] fp16 scale / zero point
  float* out;                              // [H, M, D]
  int H, G, M, S, causal, use_quant, qblocks;
  int vr_aligned;                          // V scale and zero point 8-byte aligned
};

constexpr int BM = 64;   // query rows per workgroup
constexpr int BN = 64;   // keys per tile

template <int D>
struct Geo {
  // Bytes of a staged K row: 32 bytes of padding.  The LDS serves a 16-byte read
  // for lanes 0-7 and 16-23 (then 8-15 and 24-31, ...) together, over 64 banks;
  // the K operand read puts rows 16 n + 0..7 at word offset 0 and 4 of a row in
  // one such group, and only a row stride of 8 (mod 16) words keeps those 16
  // four-bank spans apart.  Rows of 16 bytes of padding (36 or 68 words) cost
  // 4 conflict cycles per read.
  static constexpr int KROW = D * 2 + 32;
  // Bytes of a staged V^T row (keys in the order vpos gives, 32 bytes of
  // padding): the P.V operand of a lane is 16 contiguous bytes, one 16-byte read
  // (an 8-byte pair read moves half the bytes per cycle), conflict-free at a
  // stride of 40 words like the K rows.
  static constexpr int VROW = BN * 2 + 32;
  static constexpr int KBYTES = BN * KROW;
  static constexpr int STAGE = KBYTES + D * VROW;
  static constexpr int LDS = 2 * STAGE;
  static constexpr int KW = D / 64;         // 8-byte K words per staging thread (K: 4 threads per key)
  static constexpr int VW = D / 64;         // V dwords per key per staging thread (V: 8 threads per key pair)
};

__device__ __forceinline__ float hf(uint16_t h) { return h2f(h); }

// Position of key k (of a 64-key tile) in a V^T row: key 32 h + 16 u + 4 g + i
// (i < 4) sits at 32 h + 8 g + 4 u + i, so that the 8 keys of lane group g in
// the P.V product of half h (keys 32 h + 4 g + i, then 32 h + 16 + 4 g + i)
// are contiguous.  Even keys stay even: a key pair stays one 4-byte word.
__device__ __forceinline__ int vpos(int k) { return (k & 32) | ((k & 12) << 1) | ((k & 16) >> 2) | (k & 3); }

// fp16 pairs (1024 + low nibble, 1024 + high nibble) of byte i of x, minus zc
__device__ __forceinline__ uint32_t nib_pair(uint32_t lo_all, uint32_t hi_all, int i, half2v zc) {
  const uint32_t w = __builtin_amdgcn_perm(hi_all, lo_all, 0x0C000C00u | ((4u + i) << 16) | (uint32_t)i) | 0x64006400u;
  const half2v r = __builtin_bit_cast(half2v, w) - zc;
  return __builtin_bit_cast(uint32_t, r);
}

// HP query heads of one KV head per workgroup (4 waves each, the same 64 query
// rows): the K/V tiles are staged once, by the first four waves, for all of them.
// Head_dim 64 is held to 128 VGPRs, four waves per SIMD (two 8-wave workgroups
// per CU).
template <int D, int HP>
__global__ void __launch_bounds__(256 * HP) __attribute__((amdgpu_waves_per_eu(D == 64 ? 4 : 1))) prefill_kernel(const Params p) {
  using GG = Geo<D>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, w = (tid >> 6) & 3;
  const bool stager = tid < 256;                              // uniform per wave
  const int hgroups = p.H / HP;
  const int h = (blockIdx.x % hgroups) * HP + (tid >> 8);
  const int qb = p.qblocks - 1 - (int)(blockIdx.x / hgroups);   // the longest query blocks first
  const int kv = h / p.G;
  const int m0 = qb * BM;
  const int col = lane & 15, grp = lane >> 4;
  const int m = m0 + 16 * w + col;                          // this lane's query row
  const int mq = min(m, p.M - 1);
  const int kend = p.causal ? min(p.S, m0 + BM) : p.S;
  const int ntiles = (kend + BN - 1) / BN;
  const bool quant = p.use_quant != 0;

  // ---- the lane's query column, scaled per channel and by log2(e) / sqrt(D) (so
  // the scores come out as base-2 logits), split hi / lo (B operand of S^T)
  const float sc = 1.4426950408889634f * __builtin_amdgcn_rsqf((float)D);
  half8 qh[D / 32], ql[D / 32];
  {
    // The rulers are read whether or not use_quant is set (the pointers are
    // always valid), so that every load of the prologue is issued before the
    // first wait; under a per-element branch each load waited for the previous.
    const uint16_t* qrow = p.q + ((int64_t)h * p.M + mq) * D;
    uint4 raw[D / 32];
    uint16_t ksr[D / 32][8];
#pragma unroll
    for (int j = 0; j < D / 32; ++j) {
      raw[j] = *reinterpret_cast<const uint4*>(qrow + 32 * j + 8 * grp);
#pragma unroll
      for (int e = 0; e < 8; ++e) ksr[j][e] = p.ks[(int64_t)kv * D + 32 * j + 8 * grp + e];
    }
#pragma unroll
    for (int j = 0; j < D / 32; ++j) {
      const uint32_t wds[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float x = hf((uint16_t)(wds[e >> 1] >> (16 * (e & 1)))) * sc;
        x *= quant ? hf(ksr[j][e]) : 1.0f;
        const _Float16 hi = (_Float16)x;
        qh[j][e] = hi;
        ql[j][e] = (_Float16)(x - (float)hi);
      }
    }
  }

  // ---- staging roles
  // K: thread (key kk, quarter ku): dims D/4 * ku .. + D/4 - 1.  Staging wave v
  // takes keys 16 v .. 16 v + 15, lane l key 16 v + (l & 15) and quarter l >> 4:
  // the lanes of a quarter write consecutive rows, and the wave's loads cover
  // its 16 keys' codes contiguously.
  const int kk = (tid & 15) + 16 * ((tid >> 6) & 3), ku = (tid >> 4) & 3;
  const half2v kzc = half2v{(_Float16)1024.0f, (_Float16)1024.0f};
  // V: thread (key pair vk, byte group vb (+ 8)): dims 8 vb .. 8 vb + 7, each with
  // 1024 + its rounded zero point.  Staging wave v takes all 32 key pairs of the
  // tile for byte groups 2 v and 2 v + 1 (lane l: key pair l & 31, byte group
  // 2 v + (l >> 5)); its V^T stores then cover two rows' 32 words each, which
  // the LDS writes without bank conflicts.
  const int vk = lane & 31, vb = 2 * ((tid >> 6) & 3) + (lane >> 5);
  const int vcol = 2 * vpos(2 * vk);   // byte offset of the pair in a V^T row
  // zero points rounded and clamped to 0..15 (all loads first, as above)
  auto zround = [&](uint16_t z) { return quant ? fminf(fmaxf(__builtin_rintf(hf(z)), 0.f), 15.f) : 0.f; };
  // (1024 + zero) of dims 2b and 2b + 1 of the thread's 8, one register per pair;
  // the packed subtractions below take one half of it for both lanes (op_sel)
  half2v vzc[GG::VW][4];
  {
    uint16_t zr[GG::VW][8];
#pragma unroll
    for (int r = 0; r < GG::VW; ++r)
#pragma unroll
      for (int i = 0; i < 8; ++i) zr[r][i] = p.vz[(int64_t)kv * D + 8 * (vb + 8 * r) + i];
#pragma unroll
    for (int r = 0; r < GG::VW; ++r)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        vzc[r][b][0] = (_Float16)(1024.0f + zround(zr[r][2 * b]));
        vzc[r][b][1] = (_Float16)(1024.0f + zround(zr[r][2 * b + 1]));
      }
  }
  // The KV head's code planes from scalar registers, the lane's place in them as
  // 32-bit offsets (a plane is S * D / 2 < 2^32 bytes): scalar base plus vector
  // offset loads, and no 64-bit per-lane pointers held across the loop.
  const int kvs = __builtin_amdgcn_readfirstlane(kv);
  const uint8_t* const kbase = p.kp + (int64_t)kvs * p.S * (D / 2);
  const uint8_t* const vbase = p.vp + (int64_t)kvs * p.S * (D / 2);
  // Two register slots of codes: tile k is loaded into slot k % 2 two tiles
  // before it is computed, and written to LDS one tile before.
  uint2 kx[2][GG::KW];
  uint32_t vx[2][GG::VW][2];
  const uint32_t koff0 = (uint32_t)(kk * (D / 2) + ku * (D / 8));
  const uint32_t voff0 = (uint32_t)(2 * vk * (D / 2) + 4 * vb);
  auto load = [&](int t, auto slot) {   // the tile's codes (keys past S re-read key S - 1)
    constexpr int sl = decltype(slot)::value;
    if (!stager) return;
    if ((t + 1) * BN <= p.S) {             // uniform: every key of the tile lies before S
      const uint32_t off = (uint32_t)t * BN * (D / 2);
#pragma unroll
      for (int i = 0; i < GG::KW; ++i) kx[sl][i] = *reinterpret_cast<const uint2*>(kbase + (koff0 + off + 8 * i));
#pragma unroll
      for (int r = 0; r < GG::VW; ++r) {
        vx[sl][r][0] = *reinterpret_cast<const uint32_t*>(vbase + (voff0 + off + 32 * r));
        vx[sl][r][1] = *reinterpret_cast<const uint32_t*>(vbase + (voff0 + off + D / 2 + 32 * r));
      }
      return;
    }
    const int key = min(t * BN + kk, p.S - 1);
    const uint32_t ko = (uint32_t)(key * (D / 2) + ku * (D / 8));
#pragma unroll
    for (int i = 0; i < GG::KW; ++i) kx[sl][i] = *reinterpret_cast<const uint2*>(kbase + (ko + 8 * i));
    const int k0 = min(t * BN + 2 * vk, p.S - 1), k1 = min(t * BN + 2 * vk + 1, p.S - 1);
#pragma unroll
    for (int r = 0; r < GG::VW; ++r) {
      vx[sl][r][0] = *reinterpret_cast<const uint32_t*>(vbase + (uint32_t)(k0 * (D / 2) + 4 * (vb + 8 * r)));
      vx[sl][r][1] = *reinterpret_cast<const uint32_t*>(vbase + (uint32_t)(k1 * (D / 2) + 4 * (vb + 8 * r)));
    }
  };
  auto store = [&](auto slot) {  // slot's codes -> fp16 (code - zero) in LDS stage `slot`
    constexpr int sl = decltype(slot)::value;
    if (!stager) return;
    uint8_t* Ks = smem + sl * GG::STAGE;
    uint8_t* Vs = Ks + GG::KBYTES;
    uint32_t kw[D / 8];
#pragma unroll
    for (int i = 0; i < GG::KW; ++i) {
      const uint32_t ws2[2] = {kx[sl][i].x, kx[sl][i].y};
#pragma unroll
      for (int hw = 0; hw < 2; ++hw) {
        const uint32_t lo = ws2[hw] & 0x0F0F0F0Fu, hi = (ws2[hw] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int pi = 8 * i + 4 * hw + b;     // dim pair index within the thread's quarter
          kw[pi] = nib_pair(lo, hi, b, kzc);
        }
      }
    }
    uint4* kd = reinterpret_cast<uint4*>(Ks + kk * GG::KROW + ku * (D / 2));
#pragma unroll
    for (int i = 0; i < D / 32; ++i) kd[i] = make_uint4(kw[4 * i], kw[4 * i + 1], kw[4 * i + 2], kw[4 * i + 3]);
#pragma unroll
    for (int r = 0; r < GG::VW; ++r) {
      const uint32_t lo0 = vx[sl][r][0] & 0x0F0F0F0Fu, hi0 = (vx[sl][r][0] >> 4) & 0x0F0F0F0Fu;
      const uint32_t lo1 = vx[sl][r][1] & 0x0F0F0F0Fu, hi1 = (vx[sl][r][1] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int d = 8 * (vb + 8 * r) + 2 * b;  // dims d (low nibbles) and d + 1 (high nibbles)
        const uint32_t sel = 0x0C000C00u | ((4u + b) << 16) | (uint32_t)b;
        const half2v ze = __builtin_shufflevector(vzc[r][b], vzc[r][b], 0, 0);
        const half2v zo = __builtin_shufflevector(vzc[r][b], vzc[r][b], 1, 1);
        const half2v e = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(lo1, lo0, sel) | 0x64006400u) - ze;
        const half2v o = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(hi1, hi0, sel) | 0x64006400u) - zo;
        *reinterpret_cast<uint32_t*>(Vs + d * GG::VROW + vcol) = __builtin_bit_cast(uint32_t, e);
        *reinterpret_cast<uint32_t*>(Vs + (d + 1) * GG::VROW + vcol) = __builtin_bit_cast(uint32_t, o);
      }
    }
  };

  floatx4 o[D / 16];
#pragma unroll
  for (int c = 0; c < D / 16; ++c) o[c] = floatx4{0.f, 0.f, 0.f, 0.f};
  // the row sums l come out of the matrix cores as a product with a block of
  // ones, from the same fp16 weights the output uses
  floatx4 ol = floatx4{0.f, 0.f, 0.f, 0.f};
  const half8 ones = half8{(_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f,
                           (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f};
  // The products of S^T accumulate onto -m, m = the column's running maximum
  // (0 before the first tile), so the scores come out of the matrix cores as
  // base-2 logits relative to it and need no subtraction per score.  The C
  // operand is this persistent register block, rewritten only when the maximum
  // moves; it also is the running maximum's only copy.
  floatx4 cinit = floatx4{0.f, 0.f, 0.f, 0.f};

  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  // The staging waves' tile loads are issued unconditionally (the last tile
  // again where no tile t + 2 is left), and the loop below is instantiated
  // separately for staging and other waves: the compiler's memory-counter waits
  // are merged conservatively over paths that issue no loads, and with either
  // branch the staging store of tile t + 1 waited for the loads of tile t + 2
  // as well, which were issued in the same iteration.
  if (ntiles > 0) {
    load(0, S0{});
    load(min(1, ntiles - 1), S1{});
    store(S0{});
  }
  __syncthreads();
  // iteration t: tile t is in LDS stage t % 2, tile t + 1 in register slot (t + 1) % 2
  auto iteration = [&](int t, auto slot, auto role) {
    constexpr int sl = decltype(slot)::value;
    constexpr bool ST = decltype(role)::value;
    using Next = std::integral_constant<int, sl ^ 1>;
    if constexpr (ST) load(min(t + 2, ntiles - 1), slot);   // slot sl held tile t, already in LDS
    const uint8_t* Ks = smem + sl * GG::STAGE;
    const uint8_t* Vs = Ks + GG::KBYTES;
    // S^T: keys 16 n + 4 grp + i of this tile against the lane's query
    // (all K operand reads are issued before the first product)
    half8 ka[4][D / 32];
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int j = 0; j < D / 32; ++j)
        ka[n][j] = *reinterpret_cast<const half8*>(Ks + (16 * n + col) * GG::KROW + (32 * j + 8 * grp) * 2);
    __builtin_amdgcn_sched_barrier(0);
    floatx4 s[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      s[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[n][0], qh[0], cinit, 0, 0, 0);
      s[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[n][0], ql[0], s[n], 0, 0, 0);
#pragma unroll
      for (int j = 1; j < D / 32; ++j) {
        s[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[n][j], qh[j], s[n], 0, 0, 0);
        s[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[n][j], ql[j], s[n], 0, 0, 0);
      }
    }
    // The V^T operands of the tile, read now so that their LDS latency hides
    // behind the softmax: dims 16 c + col, keys 32 hh + 4 grp + i and
    // 32 hh + 16 + 4 grp + i (i < 4), positions 32 hh + 8 grp .. + 7 of the row.
    half8 va[D / 16][2];
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
        va[c][hh] = *reinterpret_cast<const half8*>(Vs + (16 * c + col) * GG::VROW + (32 * hh + 8 * grp) * 2);
    // Keys past S or past a causal row are masked.  A tile whose keys all lie
    // before S and at or before the wave's first row (m0 + 16 w) needs no mask:
    // the test is uniform over the wave.
    const int kt0 = t * BN;
    // the wave's first row as a scalar (no vector register held across the loop)
    const int wrow0 = m0 + __builtin_amdgcn_readfirstlane(16 * w);
    const bool whole = kt0 + BN <= p.S && (!p.causal || kt0 + BN - 1 <= wrow0);
    float tmax = -INFINITY;
    if (whole) {
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i) tmax = fmaxf(tmax, s[n][i]);
    } else {
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kt0 + 16 * n + 4 * grp + i;
          const bool ok = key < p.S && (!p.causal || key <= m);
          const float v = ok ? s[n][i] : -INFINITY;
          s[n][i] = v;
          tmax = fmaxf(tmax, v);
        }
    }
    // The reference maximum moves only when some column's maximum exceeds it by
    // more than 2^8 (base-2 logits): the weights then stay below 256, well inside
    // fp16, and the running sums are rescaled rarely (alpha = 0 from the initial
    // -inf, 1 where a column's maximum did not grow).  Key 0 is visible to every
    // row, so the first tile sets a finite maximum.  The test runs on the lane's
    // own 16 scores (some lane exceeds iff some column does); the column maximum
    // across the four lane groups is formed only when it fires.  s holds
    // logit - off, and off = m_run once m_run is finite.
    const float off = -cinit[0];
    const float m_run = t == 0 ? -INFINITY : off;
    if (__builtin_amdgcn_ballot_w64(tmax > (t == 0 ? -INFINITY : 8.0f))) {
      // across the four lane groups (rows of 16 lanes) that hold the column
      float a, b;
      swap16(tmax, a, b);
      tmax = fmaxf(a, b);
      swap32(tmax, a, b);
      tmax = fmaxf(a, b);
      const float m_new = fmaxf(m_run, tmax + off);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      ol *= alpha;
#pragma unroll
      for (int c = 0; c < D / 16; ++c) o[c] *= alpha;
      const float rebase = m_new - off;
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i) s[n][i] -= rebase;
      cinit = floatx4{-m_new, -m_new, -m_new, -m_new};
    }
    half4 pb[4];
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i) pb[n][i] = (_Float16)__builtin_amdgcn_exp2f(s[n][i]);
    // O^T: dims 16 c + 4 grp + i.  One product covers 32 keys: the lane's 8
    // k slots are keys 32 hh + 4 grp + i and 32 hh + 16 + 4 grp + i (i < 4), the
    // same keys in the V^T operand (A) and in the weights (B = pb[2 hh], pb[2 hh + 1])
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const half8 b = __builtin_shufflevector(pb[2 * hh], pb[2 * hh + 1], 0, 1, 2, 3, 4, 5, 6, 7);
        o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[c][hh], b, o[c], 0, 0, 0);
      }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const half8 b = __builtin_shufflevector(pb[2 * hh], pb[2 * hh + 1], 0, 1, 2, 3, 4, 5, 6, 7);
      ol = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, b, ol, 0, 0, 0);
    }
    if constexpr (ST) {
      if (t + 1 < ntiles) store(Next{});
    }
    __syncthreads();
  };
  auto run = [&](auto role) {
    for (int t = 0; t < ntiles; t += 2) {
      iteration(t, S0{}, role);
      if (t + 1 < ntiles) iteration(t + 1, S1{}, role);
    }
  };
  if (stager) run(std::true_type{});
  else run(std::false_type{});

  // every row of the ones product holds the column's whole sum
  const float rl = 1.0f / ol[0];
  if (m < p.M) {
    float* orow = p.out + ((int64_t)h * p.M + m) * D;
    // The V scale and zero point of the lane's dims 16 c + 4 grp + (0..3), all
    // loaded before the first output store: the compiler cannot move loads
    // through other pointers above a store, and loaded per dim between the
    // stores they were 2 x D/4 dependent round trips per lane (-6 % at 4096
    // queries, head_dim 128; -16 % on the short prefills).  8-byte loads where
    // the rulers are 8-byte aligned.
    uint2 zq[D / 16], sq[D / 16];
    if (quant) {
      const uint16_t* const zr0 = p.vz + (int64_t)kv * D + 4 * grp;
      const uint16_t* const sr0 = p.vs + (int64_t)kv * D + 4 * grp;
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
        if (p.vr_aligned) {
          zq[c] = *reinterpret_cast<const uint2*>(zr0 + 16 * c);
          sq[c] = *reinterpret_cast<const uint2*>(sr0 + 16 * c);
        } else {
          zq[c] = make_uint2(zr0[16 * c] | ((uint32_t)zr0[16 * c + 1] << 16), zr0[16 * c + 2] | ((uint32_t)zr0[16 * c + 3] << 16));
          sq[c] = make_uint2(sr0[16 * c] | ((uint32_t)sr0[16 * c + 1] << 16), sr0[16 * c + 2] | ((uint32_t)sr0[16 * c + 3] << 16));
        }
      }
    }
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[i] = o[c][i] * rl;
        if (quant) {
          const uint32_t zw = i < 2 ? zq[c].x : zq[c].y, sw = i < 2 ? sq[c].x : sq[c].y;
          const float z = hf((uint16_t)(i & 1 ? zw >> 16 : zw & 0xffffu));
          const float zr = fminf(fmaxf(__builtin_rintf(z), 0.f), 15.f);   // zround of this dim
          v[i] = (v[i] - (z - zr)) * hf((uint16_t)(i & 1 ? sw >> 16 : sw & 0xffffu));
        }
      }
      *reinterpret_cast<float2*>(orow + 16 * c + 4 * grp) = make_float2(v[0], v[1]);
      *reinterpret_cast<float2*>(orow + 16 * c + 4 * grp + 2) = make_float2(v[2], v[3]);
    }
  }
}

template <int D, int HP>
int launch_hp(const Params& p, hipStream_t stream) {
  static const bool lds_ok = [] {   // above 64 KB of LDS (head_dim 128) needs the attribute
    return hipFuncSetAttribute(reinterpret_cast<const void*>(prefill_kernel<D, HP>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, Geo<D>::LDS) == hipSuccess;
  }();
  if (!lds_ok) return fail(SLMT_ERR_HIP, "prefill: could not grant the kernel its LDS");
  const int grid = p.qblocks * (p.H / HP);
  hipLaunchKernelGGL((prefill_kernel<D, HP>), dim3(grid), dim3(256 * HP), Geo<D>::LDS, stream, p);
  return check_launch("prefill");
}

// Two query heads per workgroup where a KV head has an even number of them and
// the grid stays above 256 such workgroups (long prefills): the staging work per
// query row halves.  Short prefills keep one head per workgroup and twice the
// workgroups.
template <int D>
int launch(const Params& p, hipStream_t stream) {
  if (p.G % 2 == 0 && (int64_t)p.qblocks * (p.H / 2) > 256) return launch_hp<D, 2>(p, stream);
  return launch_hp<D, 1>(p, stream);
}

}  // namespace prefill

bool prefill_mfma_supported(int D) { return D == 64 || D == 128; }

int launch_prefill_mfma(const void* q, const void* kp, const void* ks, const void* kz, const void* vp, const void* vs,
                        const void* vz, int H, int G, int M, int S, int D, int causal, int use_quant, float* out,
                        hipStream_t stream) {
  prefill::Params p;
  p.q = reinterpret_cast<const uint16_t*>(q);
  p.kp = reinterpret_cast<const uint8_t*>(kp);
  p.vp = reinterpret_cast<const uint8_t*>(vp);
  p.ks = reinterpret_cast<const uint16_t*>(ks);
  p.kz = reinterpret_cast<const uint16_t*>(kz);
  p.vs = reinterpret_cast<const uint16_t*>(vs);
  p.vz = reinterpret_cast<const uint16_t*>(vz);
  p.out = out;
  p.H = H;
  p.G = G;
  p.M = M;
  p.S = S;
  p.causal = causal ? 1 : 0;
  p.use_quant = use_quant ? 1 : 0;
  p.vr_aligned = (reinterpret_cast<uintptr_t>(vs) & 7) == 0 && (reinterpret_cast<uintptr_t>(vz) & 7) == 0;
  p.qblocks = (M + prefill::BM - 1) / prefill::BM;
  if (M <= 0) return SLMT_OK;
  if ((int64_t)p.qblocks * H > 0x7fffffff) return fail(SLMT_ERR_UNSUPPORTED, "prefill: too many query blocks");
  if (D == 64) return prefill::launch<64>(p, stream);
  if (D == 128) return prefill::launch<128>(p, stream);
  return fail(SLMT_ERR_UNSUPPORTED, "prefill: the matrix-core kernel takes head_dim 64 or 128");
}

}  // namespace slmt
