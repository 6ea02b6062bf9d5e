// Single-sequence per-channel 4-bit decode, split over (KV head, key chunk)
// workgroups (reference kernel it replaces for head_dim 64 / 128 and up to 8
// query heads per KV head: kv_dequant_decode_kernel,
// kernels/kv_dequant_kernels.cuh:113-275).
//
// The reference's op-level decode is one query row over a short context (tens
// of KB to a few MB of packed K/V), so the call is bound by latency, not by
// bandwidth: the design minimises the chain of dependent memory round trips
// and the work on it.  A single wave issues a vector instruction only every
// ~8 cycles, so the per-wave work must be short: one workgroup of four waves
// per (KV head kv, chunk of CT keys), each wave CT/4 keys:
//   * the G query heads of kv, scaled per channel (q'_d = q_d * k_scale_d), go
//     to LDS;
//   * QK, 16 keys per round: lane (key t, quarter c) dots its quarter of the
//     key codes with every head in fp32 and the quad adds the quarters.  The
//     zero point's term sum_d q'_d k_zero_d is the same for every key of a head,
//     so it cancels in the softmax and is never formed; the rest is exact fp32
//     on exact integer codes;
//   * softmax over the wave's keys per head (wave reductions), weights to LDS;
//   * PV: lane = V byte (two dims): sum over the wave's keys of p * code;
//   * the four waves' (m, l, acc) are combined by log-sum-exp in LDS, wave w
//     keeping heads w, w + 4;
//   * one chunk: the waves write the output, o_d = v_scale_d (acc_d / l - v_zero_d).
//     Several chunks: (m, l, acc) partials go to the workspace with agent-scope
//     stores and the last chunk of kv to arrive (agent-scope counter) merges
//     them and resets the counter to zero.
// use_quant = 0 attends over the raw codes.  Keys are loaded once, coalesced
// (4 lanes per key row); V rows are staged in LDS for the byte-wise PV.
#include "attention_kernel.h"

namespace slmt {
namespace chan {

using namespace attn;

struct Params {
  const uint16_t* q;                        // [H, 1, D] fp16
  const uint8_t* kp;                        // [KV_t, S, D/2]
  const uint8_t* vp;
  const uint16_t *ks, *vs, *vz;             // [KV_t, D] fp16
  float* out;                               // [H, 1, D]
  float* part;                              // [KV][nchunks][GT][D + 2] partials
  int* counters;                            // [KV] arrival counters (left at zero)
  int G, S, CT, nchunks, use_quant;
};

constexpr int MAX_CT = 256;     // keys per workgroup
constexpr int NW = 4;           // waves per workgroup; wave w takes keys [w CT/4, (w+1) CT/4) of the chunk

__device__ __forceinline__ float wave_sum(float x) {
  x += dpp_f<DPP_QUAD_XOR1>(x);
  x += dpp_f<DPP_QUAD_XOR2>(x);
  x += dpp_f<DPP_ROW_ROR4>(x);
  x += dpp_f<DPP_ROW_ROR8>(x);
  float a, b;
  swap16(x, a, b);
  x = a + b;
  swap32(x, a, b);
  return a + b;
}

template <int D, int GT>
__global__ void __launch_bounds__(64 * NW) split_kernel(const Params p) {
  constexpr int QB = D / 8;                 // key bytes per quarter lane
  constexpr int VB = D / 2;                 // V bytes per key
  constexpr int NB = D == 128 ? 64 : 32;    // lanes holding a head's output (dims 2b, 2b+1)
  constexpr int HPW = (GT + NW - 1) / NW;   // heads each wave combines and writes
  __shared__ __attribute__((aligned(16))) float qs[GT * D];     // q' of the GT heads (zero past G)
  __shared__ __attribute__((aligned(16))) float sp[MAX_CT * 8];  // scores, then weights: [key][head]
  __shared__ __attribute__((aligned(16))) uint8_t vt[MAX_CT * VB];
  __shared__ float wml[NW][GT][2];                                // each wave's (m, l) per head
  __shared__ __attribute__((aligned(16))) float2 wacc[NW][GT][64]; // each wave's PV sums per lane
  __shared__ float sw[HPW * NW][64];                              // merge coefficients per chunk
  __shared__ int last;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int chunk = blockIdx.x, kv = blockIdx.y;
  const int tok0 = chunk * p.CT;
  const int ntok = min(p.CT, p.S - tok0);   // >= 1: the host launches ceil(S / CT) chunks
  const int CTW = p.CT / NW;                // keys per wave, a multiple of 16
  const int wk0 = wave * CTW;               // this wave's first key within the chunk
  const int wn = max(0, min(CTW, ntok - wk0));
  const bool quant = p.use_quant != 0;
  const int h0 = kv * p.G;

  // round r's codes: lane (key t, quarter c) loads its quarter of key t's K and
  // V rows; round 0's loads fly while q' is prepared.  Keys past the wave's
  // re-read the chunk's last key (their scores are never stored and their V
  // rows never read): selecting zeros instead made each load wait before the
  // next was issued.
  const int t = lane >> 2, c = lane & 3;
  const uint8_t* kbase = p.kp + ((int64_t)kv * p.S + tok0 + wk0) * VB + c * QB;
  const uint8_t* vbase = p.vp + ((int64_t)kv * p.S + tok0 + wk0) * VB + c * QB;
  struct Codes {
    uint2 k[QB / 8], v[QB / 8];
  };
  auto load_round = [&](int r) -> Codes {
    Codes cd;
    const int j = min(wk0 + 16 * r + t, ntok - 1) - wk0;   // a key of the chunk
#pragma unroll
    for (int i = 0; i < QB / 8; ++i) {
      cd.k[i] = *reinterpret_cast<const uint2*>(kbase + (int64_t)j * VB + 8 * i);
      cd.v[i] = *reinterpret_cast<const uint2*>(vbase + (int64_t)j * VB + 8 * i);
    }
    return cd;
  };
  Codes cur = load_round(0);

  // q' and this lane's V rulers for the output dims 2b, 2b+1.  Every load is
  // issued first, unconditionally (rows past G re-read the last head's, the
  // rulers are read without use_quant): under per-element branches each load
  // waited for the one before it.
  const int b = lane % NB, par = lane / NB, step = 64 / NB;
  constexpr int QN = (GT * D + 64 * NW - 1) / (64 * NW);   // q' elements per thread
  uint16_t qraw[QN], kraw[QN], vsr[2], vzw[2];
#pragma unroll
  for (int u = 0; u < QN; ++u) {
    const int i = min(tid + u * 64 * NW, GT * D - 1);
    const int h = min(i / D, p.G - 1), d = i % D;
    qraw[u] = p.q[(int64_t)(h0 + h) * D + d];
    kraw[u] = p.ks[(int64_t)kv * D + d];
  }
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    vsr[e] = p.vs[(int64_t)kv * D + 2 * b + e];
    vzw[e] = p.vz[(int64_t)kv * D + 2 * b + e];
  }
  float vsc[2] = {1.f, 1.f}, vzr[2] = {0.f, 0.f};
  if (quant) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      vsc[e] = h2f(vsr[e]);
      vzr[e] = h2f(vzw[e]);
    }
  }
#pragma unroll
  for (int u = 0; u < QN; ++u) {
    const int i = tid + u * 64 * NW;
    if (i < GT * D) {
      const float x = h2f(qraw[u]) * (quant ? h2f(kraw[u]) : 1.f);
      qs[i] = i / D < p.G ? x : 0.f;
    }
  }
  __syncthreads();

  // ---- QK, 16 keys per round; V rows staged on the way
  for (int r = 0; r * 16 < wn; ++r) {
    const int jw = 16 * r + t;              // key within the wave's keys
    const int j = wk0 + jw;                 // key within the chunk
    if (r > 0) cur = load_round(r);
    uint32_t kw[QB / 4];
#pragma unroll
    for (int i = 0; i < QB / 8; ++i) {
      *reinterpret_cast<uint2*>(vt + j * VB + c * QB + 8 * i) = cur.v[i];
      kw[2 * i] = cur.k[i].x;
      kw[2 * i + 1] = cur.k[i].y;
    }
    float dot[GT];
#pragma unroll
    for (int h = 0; h < GT; ++h) dot[h] = 0.f;
#pragma unroll
    for (int w = 0; w < QB / 4; ++w) {
      float n[8];
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) {
        const uint32_t byte = (kw[w] >> (8 * bb)) & 0xFFu;
        n[2 * bb] = (float)(byte & 15u);
        n[2 * bb + 1] = (float)(byte >> 4);
      }
      const int d0 = c * (D / 4) + 8 * w;
#pragma unroll
      for (int h = 0; h < GT; ++h) {
        const float4 qa = *reinterpret_cast<const float4*>(&qs[h * D + d0]);
        const float4 qb = *reinterpret_cast<const float4*>(&qs[h * D + d0 + 4]);
        float s = dot[h];
        s = __builtin_fmaf(qa.x, n[0], s);
        s = __builtin_fmaf(qa.y, n[1], s);
        s = __builtin_fmaf(qa.z, n[2], s);
        s = __builtin_fmaf(qa.w, n[3], s);
        s = __builtin_fmaf(qb.x, n[4], s);
        s = __builtin_fmaf(qb.y, n[5], s);
        s = __builtin_fmaf(qb.z, n[6], s);
        s = __builtin_fmaf(qb.w, n[7], s);
        dot[h] = s;
      }
    }
#pragma unroll
    for (int h = 0; h < GT; ++h) {
      float s = dot[h];
      s += dpp_f<DPP_QUAD_XOR1>(s);
      s += dpp_f<DPP_QUAD_XOR2>(s);
      if ((h & 3) == c && jw < wn) sp[j * 8 + h] = s;
    }
  }
  __syncthreads();

  // ---- softmax per head over the wave's keys (base 2)
  const float kscale = 1.4426950408889634f * __builtin_amdgcn_rsqf((float)D);
  float mh[GT], lh[GT];
#pragma unroll
  for (int h = 0; h < GT; ++h) {
    float mx = -INFINITY;
    for (int j = lane; j < wn; j += 64) mx = fmaxf(mx, sp[(wk0 + j) * 8 + h] * kscale);
    mx = wave_max(mx);
    float ls = 0.f;
    for (int j = lane; j < wn; j += 64) {
      const float e = __builtin_amdgcn_exp2f(sp[(wk0 + j) * 8 + h] * kscale - mx);
      sp[(wk0 + j) * 8 + h] = e;
      ls += e;
    }
    mh[h] = mx;
    lh[h] = wave_sum(ls);
  }
  __syncthreads();

  // ---- PV over the wave's keys: lane = V byte (dims 2b, 2b+1); head_dim 64:
  // lanes 32-63 take the odd keys
  float acc[GT][2];
#pragma unroll
  for (int h = 0; h < GT; ++h) acc[h][0] = acc[h][1] = 0.f;
  for (int jw = par; jw < wn; jw += step) {
    const int j = wk0 + jw;
    const uint32_t byte = vt[j * VB + b];
    const float nlo = (float)(byte & 15u), nhi = (float)(byte >> 4);
    float w[8];
    *reinterpret_cast<float4*>(w) = *reinterpret_cast<const float4*>(&sp[j * 8]);
    if (GT > 4) *reinterpret_cast<float4*>(w + 4) = *reinterpret_cast<const float4*>(&sp[j * 8 + 4]);
#pragma unroll
    for (int h = 0; h < GT; ++h) {
      acc[h][0] = __builtin_fmaf(w[h], nlo, acc[h][0]);
      acc[h][1] = __builtin_fmaf(w[h], nhi, acc[h][1]);
    }
  }
  if (D == 64) {
#pragma unroll
    for (int h = 0; h < GT; ++h) {
      float a0, a1;
      swap32(acc[h][0], a0, a1);
      acc[h][0] = a0 + a1;
      swap32(acc[h][1], a0, a1);
      acc[h][1] = a0 + a1;
    }
  }

  // ---- the chunk's four waves combined (log-sum-exp) in LDS; wave w then
  // owns heads w, w + NW, ...
#pragma unroll
  for (int h = 0; h < GT; ++h) {
    wacc[wave][h][lane] = make_float2(acc[h][0], acc[h][1]);
    if (lane == 0) {
      wml[wave][h][0] = mh[h];
      wml[wave][h][1] = lh[h];
    }
  }
  __syncthreads();
  float cm[HPW], cl[HPW];
  float2 ca[HPW];
#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    const int h = wave + NW * k;
    cm[k] = -INFINITY;
    cl[k] = 0.f;
    ca[k] = make_float2(0.f, 0.f);
    if (h < GT) {
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < NW; ++w) M = fmaxf(M, wml[w][h][0]);
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float mw = wml[w][h][0];
        const float f = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);   // waves without keys: 0
        cl[k] += f * wml[w][h][1];
        const float2 a = wacc[w][h][lane];
        ca[k].x += f * a.x;
        ca[k].y += f * a.y;
      }
      cm[k] = M;
    }
  }

  auto write_out = [&](int h, float o0, float o1) {   // o: sum p * code / l, dims 2b, 2b+1
    const int d = 2 * b;
    if (quant) {
      o0 = (o0 - vzr[0]) * vsc[0];
      o1 = (o1 - vzr[1]) * vsc[1];
    }
    *reinterpret_cast<float2*>(p.out + (int64_t)(h0 + h) * D + d) = make_float2(o0, o1);
  };

  if (p.nchunks == 1) {
    if (lane < NB) {
#pragma unroll
      for (int k = 0; k < HPW; ++k) {
        const int h = wave + NW * k;
        if (h < GT && h < p.G) write_out(h, ca[k].x / cl[k], ca[k].y / cl[k]);
      }
    }
    return;
  }

  // ---- partials, arrival, and the last arriver's merge
  float* mypart = p.part + ((int64_t)kv * p.nchunks + chunk) * GT * (D + 2);
#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    const int h = wave + NW * k;
    if (h < GT) {
      if (lane < NB) store_pair_agent(mypart + h * (D + 2) + 2 * b, ca[k].x, ca[k].y);
      if (lane == 0) store_pair_agent(mypart + h * (D + 2) + D, cm[k], cl[k]);
    }
  }
  vm_drain();
  __syncthreads();
  if (tid == 0) {
    const int prev = __hip_atomic_fetch_add(p.counters + kv, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = prev == p.nchunks - 1;
  }
  __syncthreads();
  if (!last) return;
  // (m, l) of every chunk at once: lane k loads chunk k's for the wave's heads;
  // the merge coefficients exp2(m_k - M) / L go to LDS
  const float* kvpart = p.part + (int64_t)kv * p.nchunks * GT * (D + 2);
#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    const int h = wave + NW * k;
    if (h >= GT) continue;
    float mk = -INFINITY, lk = 0.f;
    if (lane < p.nchunks) {
      const float2 ml = load_pair_agent(kvpart + ((int64_t)lane * GT + h) * (D + 2) + D);
      mk = ml.x;
      lk = ml.y;
    }
    const float M = wave_max(mk);
    const float w = lane < p.nchunks ? __builtin_amdgcn_exp2f(mk - M) : 0.f;
    const float L = wave_sum(w * lk);
    sw[k * NW + wave][lane] = w / L;
  }
  __syncthreads();
  // outputs: lane b owns dims 2b, 2b+1 (head_dim 64: lanes 32-63 take the odd
  // chunks); the partial outputs are loaded 8 at a time before they are used
#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    const int h = wave + NW * k;
    if (h >= GT || h >= p.G) continue;
    const float* cf = sw[k * NW + wave];
    float o0 = 0.f, o1 = 0.f;
    for (int k0 = par; k0 < p.nchunks; k0 += 8 * step) {
      float2 ov[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int kk = k0 + i * step;
        ov[i] = kk < p.nchunks ? load_pair_agent(kvpart + ((int64_t)kk * GT + h) * (D + 2) + 2 * b) : make_float2(0.f, 0.f);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int kk = k0 + i * step;
        const float f = kk < p.nchunks ? cf[kk] : 0.f;
        o0 = __builtin_fmaf(f, ov[i].x, o0);
        o1 = __builtin_fmaf(f, ov[i].y, o1);
      }
    }
    if (D == 64) {
      float a0, a1;
      swap32(o0, a0, a1);
      o0 = a0 + a1;
      swap32(o1, a0, a1);
      o1 = a0 + a1;
    }
    if (lane < NB) write_out(h, o0, o1);
  }
  if (tid == 0) __hip_atomic_store(p.counters + kv, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int D, int GT>
int launch(const Params& p, int KV, hipStream_t stream) {
  hipLaunchKernelGGL((split_kernel<D, GT>), dim3(p.nchunks, KV), dim3(64 * NW), 0, stream, p);
  return check_launch("per-channel decode");
}

}  // namespace chan

int launch_decode_channel_split(const void* q, const void* kp, const void* ks, const void* kz, const void* vp,
                                const void* vs, const void* vz, int H, int G, int S, int D, int use_quant, float* out,
                                void* workspace, int64_t ws_bytes, hipStream_t stream) {
  (void)kz;   // the key zero point cancels in the softmax
  if ((D != 64 && D != 128) || G < 1 || G > 8 || S < 1) return SLMT_ERR_UNSUPPORTED;
  const int KV = H / G;
  // chunk size: workgroups of four waves, each wave a multiple of 16 keys; the
  // smallest power of two from 64 keys per workgroup that gives at most 32
  // chunks per KV head (the merge reads every chunk's partials) and at most
  // 256 workgroups; past 16384 keys the general kernel takes over (64 chunks)
  int ct = 64;
  while (ct < chan::MAX_CT) {
    const int n = (S + ct - 1) / ct;
    if (n <= 32 && n * KV <= 256) break;
    ct *= 2;
  }
  const int nchunks = (S + ct - 1) / ct;
  if (nchunks > 64) return SLMT_ERR_UNSUPPORTED;
  const int GT = G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : 8;
  const int64_t part_bytes = (int64_t)KV * nchunks * GT * (D + 2) * 4;
  const int64_t part_off = kWsCounterInts * 4;
  if (nchunks > 1 && (workspace == nullptr || ws_bytes < part_off + part_bytes || KV > kWsCounterInts))
    return SLMT_ERR_UNSUPPORTED;
  chan::Params p;
  p.q = reinterpret_cast<const uint16_t*>(q);
  p.kp = reinterpret_cast<const uint8_t*>(kp);
  p.vp = reinterpret_cast<const uint8_t*>(vp);
  p.ks = reinterpret_cast<const uint16_t*>(ks);
  p.vs = reinterpret_cast<const uint16_t*>(vs);
  p.vz = reinterpret_cast<const uint16_t*>(vz);
  p.out = out;
  p.counters = reinterpret_cast<int*>(workspace);
  p.part = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + part_off);
  p.G = G;
  p.S = S;
  p.CT = ct;
  p.nchunks = nchunks;
  p.use_quant = use_quant ? 1 : 0;
#define SLMT_CHAN_CASE(d, gt) \
  if (D == d && GT == gt) return chan::launch<d, gt>(p, KV, stream);
  SLMT_CHAN_CASE(64, 1) SLMT_CHAN_CASE(64, 2) SLMT_CHAN_CASE(64, 4) SLMT_CHAN_CASE(64, 8)
  SLMT_CHAN_CASE(128, 1) SLMT_CHAN_CASE(128, 2) SLMT_CHAN_CASE(128, 4) SLMT_CHAN_CASE(128, 8)
#undef SLMT_CHAN_CASE
  return SLMT_ERR_UNSUPPORTED;
}

}  // namespace slmt
