// rf_attention.hip — single-query causal GQA attention over the KV cache.
//
// Replaces compute::attention_reference (core/src/compute.rs:461-547) behind
// ops::attention_checked (runtime/src/ops.rs:49-69).  Semantics: query head h
// reads KV head h * kvh / qh; positions 0..hist-1 come from the history
// [pos][kvh][hd], position hist is the current K/V; score = dot / sqrt(hd);
// softmax over hist+1 positions; out = sum_p softmax_p * V_p.
//
// Flash-decoding on gfx950: the positions are split into `nsplit` chunks per
// KV head.  A workgroup (4 wavefronts) owns one (chunk, KV head) pair and all
// G = qh/kvh query heads that share it, so each K/V row is read from HBM once
// for the whole group.  Sixteen lanes cooperate on one position (each holds
// hd/16 consecutive dims: 512 contiguous bytes per position for hd = 128), so
// a wavefront streams four positions per step.  Scores go to LDS, the chunk's
// max and exp-sum are workgroup reductions, then V is accumulated with the
// same lane mapping.  Each chunk writes (o, m, l); a combine kernel merges
// the chunks with the usual max-rescaling.
//
// Model mode (d_pos != null) fuses the decode-step glue: RoPE (half-split,
// core/src/compute.rs:446-456) is applied to q and the current k from a
// host-built cos/sin table, and the rotated k and the raw v are written into
// the cache slot `hist` (kv_cache.rs:381-412).  No workgroup of the launch
// reads that slot, so the write does not race with the reads.
#include "rf_kernels.h"

namespace rf {

constexpr int ATT_THREADS = 256;
constexpr int ATT_MAX_CHUNK = 1024;

__device__ __forceinline__ uint32_t att_chunk(uint32_t total, uint32_t nsplit) {
  uint32_t c = (total + nsplit - 1) / nsplit;
  return (c + 15u) & ~15u;
}

// Rotated element d of a head vector v (half-split RoPE, cs = [half][2] cos/sin).
__device__ __forceinline__ float rope_elem(const float* v, const float* cs, uint32_t d, uint32_t hd) {
  const uint32_t half = hd >> 1;
  if (d < half) {
    const float c = cs[2 * d], s = cs[2 * d + 1];
    return v[d] * c - v[d + half] * s;
  }
  const uint32_t i = d - half;
  const float c = cs[2 * i], s = cs[2 * i + 1];
  return v[i] * s + v[d] * c;
}

template <int G, int DPL>
__global__ __launch_bounds__(ATT_THREADS) void attn_split(AttnArgs a) {
  constexpr int HD = DPL * 16;
  __shared__ __align__(16) float sc[G][ATT_MAX_CHUNK];
  __shared__ __align__(16) float kcur[HD];
  __shared__ float mh[G], lh[G];
  __shared__ __align__(16) float ored[4][G][HD];

  const uint32_t g = blockIdx.y, sp = blockIdx.x;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t hist = a.d_pos ? (uint32_t)(*a.d_pos) : a.hist;
  const uint32_t total = hist + 1;
  const uint32_t chunk = att_chunk(total, a.nsplit);
  const uint32_t p0 = sp * chunk;
  if (p0 >= total) return;
  const uint32_t p1 = min(total, p0 + chunk);
  const uint32_t npos = p1 - p0;
  const uint32_t nsplit_used = (total + chunk - 1) / chunk;
  const uint32_t kvw = a.kvh * HD;
  const float* cs = a.rope ? a.rope + (size_t)hist * HD : nullptr;  // [half][2] for this position

  // Current k of this KV head (rotated in model mode), and the cache write.
  for (uint32_t d = tid; d < (uint32_t)HD; d += ATT_THREADS) {
    const float* kc = a.k_cur + g * HD;
    const float kv = cs ? rope_elem(kc, cs, d, HD) : kc[d];
    kcur[d] = kv;
    if (a.k_store && sp == 0) {
      a.k_store[(size_t)hist * kvw + g * HD + d] = kv;
      a.v_store[(size_t)hist * kvw + g * HD + d] = a.v_cur[g * HD + d];
    }
  }

  const uint32_t sl = lane & 15u, slot = wave * 4u + (lane >> 4);
  const uint32_t d0 = sl * DPL;
  float qr[G][DPL];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float* qv = a.q + (size_t)(g * G + h) * HD;
#pragma unroll
    for (int i = 0; i < DPL; ++i) qr[h][i] = cs ? rope_elem(qv, cs, d0 + i, HD) : qv[d0 + i];
  }
  __syncthreads();

  // Pass 1: scores.
  for (uint32_t j = slot; j < npos; j += 16u) {
    const uint32_t p = p0 + j;
    const float* kp = (p < hist) ? a.k_hist + (size_t)p * kvw + g * HD + d0 : kcur + d0;
    float kv[DPL];
#pragma unroll
    for (int i = 0; i < DPL; i += 4) {
      const float4 v4 = *reinterpret_cast<const float4*>(kp + i);
      kv[i] = v4.x; kv[i + 1] = v4.y; kv[i + 2] = v4.z; kv[i + 3] = v4.w;
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < DPL; ++i) s = fmaf(qr[h][i], kv[i], s);
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
      if (sl == 0) sc[h][j] = s / a.denom;
    }
  }
  __syncthreads();

  // Chunk max and exp-sum per head (one wavefront per head).
  for (uint32_t h = wave; h < (uint32_t)G; h += 4u) {
    float m = -INFINITY;
    for (uint32_t j = lane; j < npos; j += 64u) m = fmaxf(m, sc[h][j]);
    m = rf_wave_max(m);
    float l = 0.f;
    for (uint32_t j = lane; j < npos; j += 64u) {
      const float e = expf(sc[h][j] - m);
      sc[h][j] = e;
      l += e;
    }
    l = rf_wave_sum(l);
    if (lane == 0) { mh[h] = m; lh[h] = l; }
  }
  __syncthreads();

  // Pass 2: o[h] = sum_p e[h][p] * V_p.
  float o[G][DPL];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < DPL; ++i) o[h][i] = 0.f;
  for (uint32_t j = slot; j < npos; j += 16u) {
    const uint32_t p = p0 + j;
    const float* vp = (p < hist) ? a.v_hist + (size_t)p * kvw + g * HD + d0 : a.v_cur + g * HD + d0;
    float vv[DPL];
#pragma unroll
    for (int i = 0; i < DPL; i += 4) {
      const float4 v4 = *reinterpret_cast<const float4*>(vp + i);
      vv[i] = v4.x; vv[i + 1] = v4.y; vv[i + 2] = v4.z; vv[i + 3] = v4.w;
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float e = sc[h][j];
#pragma unroll
      for (int i = 0; i < DPL; ++i) o[h][i] = fmaf(e, vv[i], o[h][i]);
    }
  }
  // Reduce the four 16-lane groups of each wavefront, then the four wavefronts.
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      float v = o[h][i];
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      o[h][i] = v;
    }
  if (lane < 16u) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int i = 0; i < DPL; ++i) ored[wave][h][d0 + i] = o[h][i];
  }
  __syncthreads();
  for (uint32_t t = tid; t < (uint32_t)(G * HD); t += ATT_THREADS) {
    const uint32_t h = t / HD, d = t % HD;
    const float v = ored[0][h][d] + ored[1][h][d] + ored[2][h][d] + ored[3][h][d];
    const uint32_t qhead = g * G + h;
    if (nsplit_used == 1) {
      a.out[(size_t)qhead * HD + d] = v / lh[h];
    } else {
      float* w = a.ws + ((size_t)sp * a.qh + qhead) * (HD + 2);
      w[d] = v;
      if (d == 0) { w[HD] = mh[h]; w[HD + 1] = lh[h]; }
    }
  }
}

// Merge the per-chunk (o, m, l) of every query head.  One workgroup per head.
__global__ __launch_bounds__(256) void attn_combine(AttnArgs a) {
  const uint32_t qhead = blockIdx.x, hd = a.hd;
  const uint32_t hist = a.d_pos ? (uint32_t)(*a.d_pos) : a.hist;
  const uint32_t total = hist + 1;
  const uint32_t chunk = att_chunk(total, a.nsplit);
  const uint32_t ns = (total + chunk - 1) / chunk;
  if (ns == 1) return;
  float m = -INFINITY;
  for (uint32_t s = 0; s < ns; ++s) m = fmaxf(m, a.ws[((size_t)s * a.qh + qhead) * (hd + 2) + hd]);
  float l = 0.f;
  for (uint32_t s = 0; s < ns; ++s) {
    const float* w = a.ws + ((size_t)s * a.qh + qhead) * (hd + 2);
    l = fmaf(w[hd + 1], expf(w[hd] - m), l);
  }
  for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) {
    float acc = 0.f;
    for (uint32_t s = 0; s < ns; ++s) {
      const float* w = a.ws + ((size_t)s * a.qh + qhead) * (hd + 2);
      acc = fmaf(w[d], expf(w[hd] - m), acc);
    }
    a.out[(size_t)qhead * hd + d] = acc / l;
  }
}

// Any-shape fallback (tiny heads, large GQA groups): one workgroup per query
// head, scores in the workspace ([qh][total]), plain loops.
__global__ __launch_bounds__(256) void attn_naive(AttnArgs a) {
  __shared__ float red[256];
  __shared__ float bcast;
  const uint32_t h = blockIdx.x, tid = threadIdx.x;
  const uint32_t hist = a.d_pos ? (uint32_t)(*a.d_pos) : a.hist, total = hist + 1;
  const uint32_t hd = a.hd, g = h * a.kvh / a.qh, kvw = a.kvh * hd;
  const float* cs = a.rope ? a.rope + (size_t)hist * hd : nullptr;
  float* sc = a.ws + (size_t)h * total;
  const float* qv = a.q + (size_t)h * hd;
  const float* kc = a.k_cur + g * hd;
  if (a.k_store && h * a.kvh % a.qh == 0) {  // first query head of each KV group writes the slot
    for (uint32_t d = tid; d < hd; d += 256u) {
      a.k_store[(size_t)hist * kvw + g * hd + d] = cs ? rope_elem(kc, cs, d, hd) : kc[d];
      a.v_store[(size_t)hist * kvw + g * hd + d] = a.v_cur[g * hd + d];
    }
  }
  float mx = -INFINITY;
  for (uint32_t p = tid; p < total; p += 256u) {
    const float* kp = p < hist ? a.k_hist + (size_t)p * kvw + g * hd : nullptr;
    float s = 0.f;
    for (uint32_t d = 0; d < hd; ++d) {
      const float qd = cs ? rope_elem(qv, cs, d, hd) : qv[d];
      const float kd = kp ? kp[d] : (cs ? rope_elem(kc, cs, d, hd) : kc[d]);
      s = fmaf(qd, kd, s);
    }
    s = s / a.denom;
    sc[p] = s;
    mx = fmaxf(mx, s);
  }
  red[tid] = mx;
  __syncthreads();
  if (tid == 0) {
    float m = -INFINITY;
    for (int i = 0; i < 256; ++i) m = fmaxf(m, red[i]);
    bcast = m;
  }
  __syncthreads();
  const float m = bcast;
  float l = 0.f;
  for (uint32_t p = tid; p < total; p += 256u) {
    const float e = expf(sc[p] - m);
    sc[p] = e;
    l += e;
  }
  __syncthreads();
  red[tid] = l;
  __syncthreads();
  if (tid == 0) {
    float s = 0.f;
    for (int i = 0; i < 256; ++i) s += red[i];
    bcast = s;
  }
  __syncthreads();
  const float lsum = bcast;
  for (uint32_t d = tid; d < hd; d += 256u) {
    float acc = 0.f;
    for (uint32_t p = 0; p < total; ++p) {
      const float vd = p < hist ? a.v_hist[(size_t)p * kvw + g * hd + d] : a.v_cur[g * hd + d];
      acc = fmaf(sc[p], vd, acc);
    }
    a.out[(size_t)h * hd + d] = acc / lsum;
  }
}

bool attention_supported(uint32_t qh, uint32_t kvh, uint32_t hd) {
  if (kvh == 0 || qh % kvh != 0) return false;
  const uint32_t G = qh / kvh;
  const bool g_ok = G == 1 || G == 2 || G == 4 || G == 8;
  const bool hd_ok = hd == 64 || hd == 128 || hd == 256;
  return g_ok && hd_ok && G * (hd / 16) <= 64;
}

uint32_t attention_splits(uint32_t total, uint32_t kvh) {
  const uint32_t by_len = (total + 63) / 64;
  const uint32_t want = (512 + kvh - 1) / kvh;
  const uint32_t min_for_lds = (total + ATT_MAX_CHUNK - 1) / ATT_MAX_CHUNK;
  uint32_t n = by_len < want ? by_len : want;
  if (n < min_for_lds) n = min_for_lds;
  return n < 1 ? 1 : n;
}

template <int G, int DPL>
static void launch_split_t(const AttnArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((attn_split<G, DPL>), dim3(a.nsplit, a.kvh), dim3(ATT_THREADS), 0, st, a);
}

hipError_t launch_attention_naive(const AttnArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(attn_naive, dim3(a.qh), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t st) {
  if (!attention_supported(a.qh, a.kvh, a.hd)) return launch_attention_naive(a, st);
  const uint32_t G = a.qh / a.kvh, dpl = a.hd / 16;
#define RF_ATT(GG, DD) if (G == GG && dpl == DD) launch_split_t<GG, DD>(a, st);
  RF_ATT(1, 4) RF_ATT(1, 8) RF_ATT(1, 16) RF_ATT(2, 4) RF_ATT(2, 8) RF_ATT(2, 16)
  RF_ATT(4, 4) RF_ATT(4, 8) RF_ATT(4, 16) RF_ATT(8, 4) RF_ATT(8, 8)
#undef RF_ATT
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (a.nsplit > 1) {
    hipLaunchKernelGGL(attn_combine, dim3(a.qh), dim3(a.hd < 256 ? a.hd : 256), 0, st, a);
    e = hipGetLastError();
  }
  return e;
}

}  // namespace rf
