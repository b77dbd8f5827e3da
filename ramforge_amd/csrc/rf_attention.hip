// rf_attention.hip — single-query causal GQA attention over the KV cache.
//
// Replaces compute::attention_reference (core/src/compute.rs:461-547) behind
// ops::attention_checked (runtime/src/ops.rs:49-69).  Semantics: query head h
// reads KV head h * kvh / qh; positions 0..hist-1 come from the history
// [pos][kvh][hd], position hist is the current K/V; score = dot / sqrt(hd);
// softmax over hist+1 positions; out = sum_p softmax_p * V_p.
//
// Flash-decoding on gfx950, one launch per call:
//   * The positions are cut into chunks of at least 64 (one chunk per
//     workgroup and KV head).  A workgroup (4 wavefronts) owns one
//     (chunk, KV head) pair and all G = qh/kvh query heads that share it, so
//     every K/V row is read from HBM once for the whole group.
//   * Sixteen lanes cooperate on one position (hd/16 dims each, taken four
//     at a time so that every load of the 16 lanes reads 256 contiguous
//     bytes of the row); a wavefront covers four
//     positions per step and every lane issues the loads of four steps before
//     it uses any of them, so a 64-position chunk is one round trip per pass.
//   * The G partial dot products of a position are summed over the 16 lanes
//     with a transposing butterfly (log2(G) exchange steps that halve the
//     heads each lane holds, then plain steps): 5 shuffles for G = 4 instead
//     of 16.
//   * Scores go to LDS; the chunk max and exp-sum are per-head wavefront
//     reductions.  For V each lane owns hd/64 dims and each wavefront 16 of
//     every 64 positions, so the weighted sum needs no cross-lane step; the
//     four wavefronts are summed through LDS.
//   * Each chunk writes (o, m, l) of its G heads; a second kernel (one
//     wavefront per query head) merges the chunks with the usual
//     max-rescaling.  (Merging inside the split
//     kernel through arrival counters needs device-scope release fences,
//     which write back the per-XCD L2 on gfx950 and cost far more than the
//     second launch.)
//
// Model mode (d_pos != null) fuses the decode-step glue: RoPE (half-split,
// core/src/compute.rs:446-456) is applied to q and the current k from a
// host-built cos/sin table, and the rotated k and the raw v are written into
// the cache slot `hist` (kv_cache.rs:381-412).  No workgroup of the launch
// reads that slot from memory (the current position is taken from LDS), so
// the write does not race with the reads.
#include "rf_kernels.h"

namespace rf {

constexpr uint32_t ATT_MAX_CHUNK = 1024;  // positions of one chunk (LDS score rows)
constexpr int ATT_UNROLL = 4;
constexpr uint32_t ATT_MAX_SPLITS = 256;

typedef float f32x4 __attribute__((ext_vector_type(4)));

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

// Sum of s[h] over the 16 lanes of a position group (one DPP row) for every
// h < N.  Each exchange level hands half of the heads a lane holds to its
// partner across bit OFF and keeps the other half; after log2(N) levels a
// lane holds one head, summed by plain exchanges over the remaining bits.
// `head` accumulates which head the lane ends with; lanes with
// (lane & (16/N - 1)) == 0 hold distinct heads.
template <int N, int OFF>
__device__ __forceinline__ float head_reduce16(float* s, uint32_t lane, uint32_t& head) {
  if constexpr (N > 1) {
    constexpr int half = N / 2;
    const bool hi = (lane & OFF) != 0;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      const float send = hi ? s[i] : s[i + half];
      const float keep = hi ? s[i + half] : s[i];
      s[i] = keep + rf_xchg16<OFF>(send);
    }
    if (hi) head += half;
    return head_reduce16<half, OFF / 2>(s, lane, head);
  } else if constexpr (OFF >= 1) {
    s[0] += rf_xchg16<OFF>(s[0]);
    return head_reduce16<1, OFF / 2>(s, lane, head);
  } else {
    return s[0];
  }
}

template <int N>
__device__ __forceinline__ void load_few(float* dst, const float* src) {
  if constexpr (N == 1) {
    dst[0] = __builtin_nontemporal_load(src);
  } else {
    typedef float vec __attribute__((ext_vector_type(N)));
    const vec v = __builtin_nontemporal_load(reinterpret_cast<const vec*>(src));
#pragma unroll
    for (int i = 0; i < N; ++i) dst[i] = v[i];
  }
}

// n dims of a K row for one lane: four consecutive floats from every 64
// (src points at the lane's first float of the row).
__device__ __forceinline__ void load_dims(float* dst, const float* src, int n) {
  const f32x4* p = reinterpret_cast<const f32x4*>(src);
#pragma unroll
  for (int i = 0; i < n / 4; ++i) {
    const f32x4 v = __builtin_nontemporal_load(p + 16 * i);
    dst[4 * i] = v.x; dst[4 * i + 1] = v.y; dst[4 * i + 2] = v.z; dst[4 * i + 3] = v.w;
  }
}

// Raw buffer loads over one chunk's rows of one KV head: offsets past the
// region read as zeros, so the loads of a round's positions past the chunk
// need no clamping (and fetch nothing).
typedef __amdgpu_buffer_rsrc_t AttRsrc;
constexpr int ATT_RSRC_WORD3 = 0x00020000;  // raw buffer, 32-bit data
constexpr int ATT_AUX_NT = 2;               // streaming loads
__device__ __forceinline__ AttRsrc att_rsrc(const float* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, (int32_t)bytes, ATT_RSRC_WORD3);
}
// n dims of a K row for one lane (four consecutive floats from every 64) at
// byte offset off of the region
__device__ __forceinline__ void load_dims_buf(float* dst, AttRsrc r, uint32_t off, int n) {
#pragma unroll
  for (int i = 0; i < n / 4; ++i) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off + 256u * i, 0, ATT_AUX_NT);
    dst[4 * i] = __uint_as_float(v[0]); dst[4 * i + 1] = __uint_as_float(v[1]);
    dst[4 * i + 2] = __uint_as_float(v[2]); dst[4 * i + 3] = __uint_as_float(v[3]);
  }
}
template <int N>
__device__ __forceinline__ void load_few_buf(float* dst, AttRsrc r, uint32_t off) {
  if constexpr (N == 1) {
    dst[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, ATT_AUX_NT));
  } else if constexpr (N == 2) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, ATT_AUX_NT);
    dst[0] = __uint_as_float(v[0]); dst[1] = __uint_as_float(v[1]);
  } else {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, ATT_AUX_NT);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = __uint_as_float(v[i]);
  }
}

// W wavefronts per workgroup: one round of loads covers 16 W positions
// (4 W position slots of 16 lanes, U positions each in pass 1; 16 rows per
// wavefront in pass 2), so a chunk of up to 16 W positions is one memory round
// trip per pass.  PERQ: one workgroup per query head (G = 1) instead of per
// KV head, so short contexts spread over qh workgroups; the query heads of a
// group read the same K/V rows (from L2 or HBM) and the group's first head
// writes the cache slot.
template <int G, int DPL, int W, bool PERQ>
__global__ __launch_bounds__(64 * W) void attn_split(AttnArgs a) {
  static_assert(!PERQ || G == 1, "one query head per workgroup");
  constexpr int HD = DPL * 16;
  constexpr uint32_t NTH = 64u * W, NSLOT = 4u * W;
  constexpr int U = DPL <= 8 ? ATT_UNROLL : ATT_UNROLL / 2;  // register budget for hd = 256
  constexpr uint32_t RV = 16;                                 // V rows per wavefront and round
  // (Holding a whole 256-position chunk in flight, 8 K positions per lane
  // and 32 V rows per wavefront, measured slower at 2048-8000 positions.)
  constexpr uint32_t WMASK = 16u / G - 1u;
  __shared__ __align__(16) float sc[G][ATT_MAX_CHUNK];
  __shared__ __align__(16) float qs[G][HD];
  __shared__ __align__(16) float kcur[HD];
  __shared__ __align__(16) float vcur[HD];
  __shared__ float mh[G], lh[G];
  __shared__ __align__(16) float ored[W][G][HD];

  // g: the KV head; qg: the first query head of this workgroup
  const uint32_t qg = PERQ ? blockIdx.y : blockIdx.y * G;
  const uint32_t g = PERQ ? blockIdx.y / (a.qh / a.kvh) : blockIdx.y, sp = blockIdx.x;
  const bool writes_slot = sp == 0 && (!PERQ || qg % (a.qh / a.kvh) == 0);
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  // token batch (prefill): query z of a.ntok at position hist + z, whose own
  // k / v are already in the cache row hist + z
  const uint32_t z = blockIdx.z;
  const uint32_t hist = (a.d_pos ? (uint32_t)(*a.d_pos) : a.hist) + z;
  const uint32_t kvw = a.kvh * HD;
  const float* qz = a.q + (size_t)z * a.qh * HD;
  const float* kcur_p = a.ntok ? a.k_hist + (size_t)hist * kvw : a.k_cur;
  const float* vcur_p = a.ntok ? a.v_hist + (size_t)hist * kvw : a.v_cur;
  float* outz = a.out + (size_t)z * a.qh * HD;
  float* wsz = a.ws + (size_t)z * a.nsplit * a.qh * att_rec(HD);
  const uint32_t total = hist + 1;
  const uint32_t chunk = att_chunk(total, a.nsplit);
  const uint32_t p0 = sp * chunk;
  if (p0 >= total) return;
  const uint32_t p1 = min(total, p0 + chunk);
  const uint32_t npos = p1 - p0;
  const uint32_t nmain = min(p1, hist) - p0;  // positions read from the cache
  const bool has_cur = p1 == total;           // the current position is the last one
  const uint32_t ns = (total + chunk - 1) / chunk;
  const float* cs = a.rope ? a.rope + (size_t)hist * HD : nullptr;  // [half][2] for this position
  const uint32_t sl = lane & 15u, slot = wave * 4u + (lane >> 4);
  // Lane sl of a position holds dims kdim(i) = 64 (i / 4) + 4 sl + i % 4, so
  // each 16-byte load of the 16 lanes covers 256 contiguous bytes of the row.
  const uint32_t d0 = sl * 4u;
  // K and V rows p0 .. p0 + nmain - 1 of KV head g: a region ending with the
  // last row's head segment; rows past it (a round's tail) read as zeros
  const uint32_t rbytes = nmain ? ((nmain - 1u) * kvw + HD) * 4u : 0u;
  const AttRsrc kr = att_rsrc(a.k_hist + (size_t)p0 * kvw + g * HD, rbytes);
  const AttRsrc vr = att_rsrc(a.v_hist + (size_t)p0 * kvw + g * HD, rbytes);
  // Pass 2 maps lanes to dims instead: lane l owns dims [l*DPW, (l+1)*DPW) of
  // every V row and wavefront w the rows w*16 .. w*16+15 of each 64-row batch,
  // so the weighted V sum needs no cross-lane reduction.
  constexpr int DPW = HD / 64;

  // Loads first: the prologue's operands (q of the G heads, the current k
  // and v, the cos/sin row), then the first batch of K rows, then of V rows,
  // all before any is used.  A wavefront's loads complete in order, so the
  // prologue waits for its own operands only, pass 1 for K and not V, and a
  // 64-position chunk still takes one memory round trip.  Indices are
  // clamped: every load is in bounds.  Element t of [q heads..., k, v] is
  // handled by thread t % NTH.
  constexpr uint32_t NE = (G + 2) * HD, NP = (NE + NTH - 1) / NTH, HALF = HD / 2;
  float va[NP], vp[NP], c0[NP], c1[NP];
#pragma unroll
  for (uint32_t i = 0; i < NP; ++i) {
    const uint32_t t = min(tid + i * NTH, NE - 1u), r = t / HD, d = t % HD;
    const float* src = r < (uint32_t)G ? qz + (size_t)(qg + r) * HD : (r == (uint32_t)G ? kcur_p : vcur_p) + g * HD;
    const uint32_t ci = d < HALF ? d : d - HALF;
    va[i] = src[d];
    vp[i] = src[d < HALF ? d + HALF : d - HALF];
    c0[i] = cs ? cs[2 * ci] : 1.f;
    c1[i] = cs ? cs[2 * ci + 1] : 0.f;
  }
  __builtin_amdgcn_sched_barrier(0);
  float kv[U][DPL], vv[RV][DPW];
#pragma unroll
  for (int u = 0; u < U; ++u) load_dims_buf(kv[u], kr, ((slot + NSLOT * u) * kvw + d0) * 4u, DPL);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < (int)RV; ++k) load_few_buf<DPW>(vv[k], vr, ((wave * RV + k) * kvw + lane * DPW) * 4u);
  __builtin_amdgcn_sched_barrier(0);

  // Rotated q of the G heads, the current k (rotated) and v, and the slot write.
#pragma unroll
  for (uint32_t i = 0; i < NP; ++i) {
    const uint32_t t = tid + i * NTH, r = t / HD, d = t % HD;
    if (t >= NE) break;
    // half-split rotation in the RoPE kernel's operation order
    const float rot = d < HALF ? va[i] * c0[i] - vp[i] * c1[i] : vp[i] * c1[i] + va[i] * c0[i];
    if (r < (uint32_t)G) {
      qs[r][d] = cs ? rot : va[i];
    } else if (r == (uint32_t)G) {
      const float kr = cs ? rot : va[i];
      kcur[d] = kr;
      if (a.k_store && writes_slot) a.k_store[(size_t)hist * kvw + g * HD + d] = kr;
    } else {
      vcur[d] = va[i];
      if (a.v_store && writes_slot) a.v_store[(size_t)hist * kvw + g * HD + d] = va[i];
    }
  }
  __syncthreads();

  float qr[G][DPL];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < DPL; ++i) qr[h][i] = qs[h][64 * (i / 4) + d0 + i % 4];

  // Pass 1: scores.
  for (uint32_t j0 = 0; j0 < nmain; j0 += NSLOT * U) {
    if (j0 > 0) {
#pragma unroll
      for (int u = 0; u < U; ++u) load_dims_buf(kv[u], kr, ((j0 + slot + NSLOT * u) * kvw + d0) * 4u, DPL);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float s[G];
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc = fmaf(qr[h][i], kv[u][i], acc);
        s[h] = acc;
      }
      uint32_t hh = 0;
      const float r = head_reduce16<G, 8>(s, lane, hh);
      const uint32_t j = j0 + slot + NSLOT * u;
      if (j < nmain && (lane & WMASK) == 0) sc[hh][j] = r / a.denom;
    }
  }
  if (has_cur && wave == 0) {
    float s[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < DPL; ++i) acc = fmaf(qr[h][i], kcur[64 * (i / 4) + d0 + i % 4], acc);
      s[h] = acc;
    }
    uint32_t hh = 0;
    const float r = head_reduce16<G, 8>(s, lane, hh);
    if (slot == 0 && (lane & WMASK) == 0) sc[hh][nmain] = r / a.denom;
  }
  __syncthreads();

  // Chunk max and exp-sum per head (one wavefront per head).  The weights
  // of the last round's positions past the chunk are zeroed: pass 2 adds
  // their (zero) V rows without a mask.
  const uint32_t rend = (npos + RV * W - 1) / (RV * W) * (RV * W);
  for (uint32_t h = wave; h < (uint32_t)G; h += W) {
    float m = -INFINITY;
    for (uint32_t j = lane; j < npos; j += 64u) m = fmaxf(m, sc[h][j]);
    m = rf_wave_max(m);
    float l = 0.f;
    for (uint32_t j = lane; j < npos; j += 64u) {
      const float e = expf(sc[h][j] - m);
      sc[h][j] = e;
      l += e;
    }
    for (uint32_t j = npos + lane; j < rend; j += 64u) sc[h][j] = 0.f;
    l = rf_wave_sum(l);
    if (lane == 0) { mh[h] = m; lh[h] = l; }
  }
  __syncthreads();

  // Pass 2: o[h] = sum_p e[h][p] * V_p, RV W rows per batch.
  float o[G][DPW];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < DPW; ++i) o[h][i] = 0.f;
  // Rows past the chunk hold zeros and zero weights (the current position's
  // row, read from vcur below, among them): adding them changes no bit, as o
  // is never -0.
  for (uint32_t j0 = 0; j0 < nmain; j0 += RV * W) {
    if (j0 > 0) {
#pragma unroll
      for (int k = 0; k < (int)RV; ++k) load_few_buf<DPW>(vv[k], vr, ((j0 + wave * RV + k) * kvw + lane * DPW) * 4u);
    }
    // weights of this wavefront's rows, four at a time with 16-byte LDS reads
    // (j0 + RV w is a multiple of 16, and j0 + RV (w + 1) <= ATT_MAX_CHUNK
    // since j0 < nmain <= chunk <= ATT_MAX_CHUNK, a multiple of RV W)
#pragma unroll
    for (int q4 = 0; q4 < (int)RV / 4; ++q4) {
      float e[G][4];
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float4 w4 = *reinterpret_cast<const float4*>(&sc[h][j0 + wave * RV + 4u * q4]);
        e[h][0] = w4.x; e[h][1] = w4.y; e[h][2] = w4.z; e[h][3] = w4.w;
      }
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
          for (int i = 0; i < DPW; ++i) o[h][i] = fmaf(e[h][k], vv[4 * q4 + k][i], o[h][i]);
    }
  }
  if (has_cur && wave == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float e = sc[h][nmain];
#pragma unroll
      for (int i = 0; i < DPW; ++i) o[h][i] = fmaf(e, vcur[lane * DPW + i], o[h][i]);
    }
  }
  // Sum the W wavefronts.
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < DPW; ++i) ored[wave][h][lane * DPW + i] = o[h][i];
  __syncthreads();
  for (uint32_t t = tid; t < (uint32_t)(G * HD); t += NTH) {
    const uint32_t h = t / HD, d = t % HD;
    float v = ored[0][h][d];
#pragma unroll
    for (int w = 1; w < W; ++w) v += ored[w][h][d];
    const uint32_t qhead = qg + h;
    if (ns == 1) {
      outz[(size_t)qhead * HD + d] = v / lh[h];
    } else {
      float* w = wsz + ((size_t)sp * a.qh + qhead) * att_rec(HD);
      w[d] = v;
      if (d == 0) { w[HD] = mh[h]; w[HD + 1] = lh[h]; }
    }
  }
}

// One-pass (online-softmax) form of attn_split for decode steps: every
// 16-lane slot streams K and V rows of its positions (U per round, K and V in
// the same lane-to-dims layout) and keeps a running maximum, exp-sum and
// weighted V sum per query head, rescaled once per round by exp2(m - m');
// scores are scaled by log2(e) / sqrt(hd) through q, so exp2 gives the
// reference's exp(score - max) (compute.rs:363-384, 461-547) up to rounding.
// The W x 4 slots are combined once at the end (lane exchanges, then LDS).
// There is no score array, no chunk-length limit and one workgroup barrier
// after the prologue.  Records are written as attn_split writes them (m in
// natural-log units), so attn_merge and the merging o-projection read either.
template <int G, int DPL, int W, bool PERQ>
__global__ __launch_bounds__(64 * W) void attn_flash(AttnArgs a) {
  static_assert(!PERQ || G == 1, "one query head per workgroup");
  constexpr int HD = DPL * 16;
  constexpr uint32_t NTH = 64u * W, NSLOT = 4u * W;
  // positions per slot and round: K, V (2 U DPL) and q, o (2 G DPL) within
  // about 128 registers
  constexpr int U = DPL * (8 + 2 * G) <= 128 ? 4 : 2;
  constexpr float LOG2E = 1.4426950408889634f, LN2 = 0.6931471805599453f;
  __shared__ __align__(16) float qs[G][HD];
  __shared__ __align__(16) float kcur[HD];
  __shared__ __align__(16) float vcur[HD];
  __shared__ __align__(16) float po[W][G][HD];
  __shared__ float pm[W][G], pl[W][G];

  const uint32_t qg = PERQ ? blockIdx.y : blockIdx.y * G;
  const uint32_t g = PERQ ? blockIdx.y / (a.qh / a.kvh) : blockIdx.y, sp = blockIdx.x;
  const bool writes_slot = sp == 0 && (!PERQ || qg % (a.qh / a.kvh) == 0);
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t hist = a.d_pos ? (uint32_t)(*a.d_pos) : a.hist;
  const uint32_t kvw = a.kvh * HD;
  const uint32_t total = hist + 1;
  const uint32_t chunk = att_chunk(total, a.nsplit);
  const uint32_t p0 = sp * chunk;
  if (p0 >= total) return;
  const uint32_t p1 = min(total, p0 + chunk);
  const uint32_t nmain = min(p1, hist) - p0;  // positions read from the cache
  const bool has_cur = p1 == total;
  const uint32_t ns = (total + chunk - 1) / chunk;
  const float* cs = a.rope ? a.rope + (size_t)hist * HD : nullptr;
  const uint32_t sl = lane & 15u, slot = wave * 4u + (lane >> 4);
  const uint32_t d0 = sl * 4u;  // dims 64 (i / 4) + d0 + i % 4 of K and V rows
  const float* kb = a.k_hist + (size_t)p0 * kvw + g * HD + d0;
  const float* vb = a.v_hist + (size_t)p0 * kvw + g * HD + d0;

  // Loads first: prologue operands, then the first round of K and V rows.
  constexpr uint32_t NE = (G + 2) * HD, NP = (NE + NTH - 1) / NTH, HALF = HD / 2;
  float va[NP], vp[NP], c0[NP], c1[NP];
#pragma unroll
  for (uint32_t i = 0; i < NP; ++i) {
    const uint32_t t = min(tid + i * NTH, NE - 1u), r = t / HD, d = t % HD;
    const float* src = r < (uint32_t)G ? a.q + (size_t)(qg + r) * HD : (r == (uint32_t)G ? a.k_cur : a.v_cur) + g * HD;
    const uint32_t ci = d < HALF ? d : d - HALF;
    va[i] = src[d];
    vp[i] = src[d < HALF ? d + HALF : d - HALF];
    c0[i] = cs ? cs[2 * ci] : 1.f;
    c1[i] = cs ? cs[2 * ci + 1] : 0.f;
  }
  __builtin_amdgcn_sched_barrier(0);
  float kv[U][DPL], vv[U][DPL];
  auto issue = [&](uint32_t j0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t j = min(j0 + slot + NSLOT * u, nmain - 1u);
      load_dims(kv[u], kb + (size_t)j * kvw, DPL);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t j = min(j0 + slot + NSLOT * u, nmain - 1u);
      load_dims(vv[u], vb + (size_t)j * kvw, DPL);
    }
  };
  if (nmain > 0) issue(0);
  __builtin_amdgcn_sched_barrier(0);

  // Rotated q of the G heads, the current k (rotated) and v, and the slot write.
#pragma unroll
  for (uint32_t i = 0; i < NP; ++i) {
    const uint32_t t = tid + i * NTH, r = t / HD, d = t % HD;
    if (t >= NE) break;
    const float rot = d < HALF ? va[i] * c0[i] - vp[i] * c1[i] : vp[i] * c1[i] + va[i] * c0[i];
    if (r < (uint32_t)G) {
      qs[r][d] = cs ? rot : va[i];
    } else if (r == (uint32_t)G) {
      const float kr = cs ? rot : va[i];
      kcur[d] = kr;
      if (a.k_store && writes_slot) a.k_store[(size_t)hist * kvw + g * HD + d] = kr;
    } else {
      vcur[d] = va[i];
      if (a.v_store && writes_slot) a.v_store[(size_t)hist * kvw + g * HD + d] = va[i];
    }
  }
  __syncthreads();

  const float qscale = LOG2E / a.denom;
  float qr[G][DPL];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < DPL; ++i) qr[h][i] = qs[h][64 * (i / 4) + d0 + i % 4] * qscale;
  float m[G], l[G], o[G][DPL];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) o[h][i] = 0.f;
  }
  // Scores of U positions (invalid ones -inf), then one rescale per head.
  auto consume = [&](const float (&kk)[U][DPL], const float (&vw)[U][DPL], uint32_t j0, uint32_t nvalid) {
    float s[U][G];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool ok = j0 + slot + NSLOT * u < nvalid;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc = fmaf(qr[h][i], kk[u][i], acc);
        acc = rf_row16_sum(acc);
        s[u][h] = ok ? acc : -INFINITY;
      }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float mx = m[h];
#pragma unroll
      for (int u = 0; u < U; ++u) mx = fmaxf(mx, s[u][h]);
      if (mx == -INFINITY) continue;  // nothing valid yet in this slot
      const float corr = __builtin_amdgcn_exp2f(m[h] - mx);  // exp2(-inf) = 0
      l[h] *= corr;
#pragma unroll
      for (int i = 0; i < DPL; ++i) o[h][i] *= corr;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float p = __builtin_amdgcn_exp2f(s[u][h] - mx);
        l[h] += p;
#pragma unroll
        for (int i = 0; i < DPL; ++i) o[h][i] = fmaf(p, vw[u][i], o[h][i]);
      }
      m[h] = mx;
    }
  };
  for (uint32_t j0 = 0; j0 < nmain; j0 += NSLOT * U) {
    if (j0 > 0) issue(j0);
    consume(kv, vv, j0, nmain);
  }
  if (has_cur) {  // the current position: slot 0 with k and v from LDS
    float kk[U][DPL], vw[U][DPL];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < DPL; ++i) {
        kk[u][i] = kcur[64 * (i / 4) + d0 + i % 4];
        vw[u][i] = vcur[64 * (i / 4) + d0 + i % 4];
      }
    consume(kk, vw, 0, 1);  // only slot 0, u = 0 is valid
  }
  // The four slots of the wavefront, then the W wavefronts.
#pragma unroll
  for (uint32_t off = 16; off <= 32; off *= 2) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float mo = __shfl_xor(m[h], off), lo = __shfl_xor(l[h], off);
      const float mx = fmaxf(m[h], mo);
      const float fs = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[h] - mx);
      const float fo = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mo - mx);
      l[h] = l[h] * fs + lo * fo;
#pragma unroll
      for (int i = 0; i < DPL; ++i) o[h][i] = o[h][i] * fs + __shfl_xor(o[h][i], off) * fo;
      m[h] = mx;
    }
  }
  if (lane < 16u) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int i = 0; i < DPL; ++i) po[wave][h][64 * (i / 4) + d0 + i % 4] = o[h][i];
      if (lane == 0) { pm[wave][h] = m[h]; pl[wave][h] = l[h]; }
    }
  }
  __syncthreads();
  for (uint32_t t = tid; t < (uint32_t)(G * HD); t += NTH) {
    const uint32_t h = t / HD, d = t % HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) M = fmaxf(M, pm[w][h]);
    float acc = 0.f, lsum = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = pm[w][h] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(pm[w][h] - M);
      acc = fmaf(po[w][h][d], f, acc);
      lsum = fmaf(pl[w][h], f, lsum);
    }
    const uint32_t qhead = qg + h;
    if (ns == 1) {
      a.out[(size_t)qhead * HD + d] = acc / lsum;
    } else {
      float* w = a.ws + ((size_t)sp * a.qh + qhead) * att_rec(HD);
      w[d] = acc;
      if (d == 0) { w[HD] = M * LN2; w[HD + 1] = lsum; }
    }
  }
}

// Merge the chunk records (o, m, l) of one query head: one wavefront per
// head, lane l owning dims [l DPW, (l + 1) DPW).  The first 32 records (all
// of them up to 32 chunks) are requested together with the (m, l) pairs,
// before any arithmetic; the factors exp(m_s - M) go through LDS to every
// lane.
template <int DPW>
__global__ __launch_bounds__(64) void attn_merge(AttnArgs a) {
  constexpr uint32_t HD = 64u * DPW, B = 32, MPL = ATT_MAX_SPLITS / 64;  // (m, l) pairs per lane
  __shared__ float fac[ATT_MAX_SPLITS];
  const uint32_t qhead = blockIdx.x, lane = threadIdx.x;
  const uint32_t z = blockIdx.z;  // token batch: see attn_split
  const uint32_t hist = (a.d_pos ? (uint32_t)(*a.d_pos) : a.hist) + z;
  const uint32_t total = hist + 1;
  const uint32_t chunk = att_chunk(total, a.nsplit);
  const uint32_t ns = (total + chunk - 1) / chunk;  // 1 < ns <= nsplit <= ATT_MAX_SPLITS
  if (ns == 1) return;
  const size_t rec = att_rec(HD), stride = (size_t)a.qh * rec;
  const float* base = a.ws + (size_t)z * a.nsplit * stride + (size_t)qhead * rec;
  float pre[B][DPW];
#pragma unroll
  for (uint32_t s = 0; s < B; ++s) load_few<DPW>(pre[s], base + (size_t)min(s, ns - 1u) * stride + lane * DPW);
  float ms[MPL], ls[MPL];
#pragma unroll
  for (uint32_t k = 0; k < MPL; ++k) {
    const uint32_t s = lane + 64u * k;
    ms[k] = s < ns ? base[s * stride + HD] : -INFINITY;
    ls[k] = s < ns ? base[s * stride + HD + 1] : 0.f;
  }
  float m = ms[0];
#pragma unroll
  for (uint32_t k = 1; k < MPL; ++k) m = fmaxf(m, ms[k]);
  m = rf_wave_max(m);
  float l = 0.f;
#pragma unroll
  for (uint32_t k = 0; k < MPL; ++k) {
    const uint32_t s = lane + 64u * k;
    if (s < ns) {
      const float f = expf(ms[k] - m);
      fac[s] = f;
      l = fmaf(ls[k], f, l);
    }
  }
  l = rf_wave_sum(l);
  __syncthreads();  // (one wavefront) the factors are in LDS
  float acc[DPW];
#pragma unroll
  for (int i = 0; i < DPW; ++i) acc[i] = 0.f;
#pragma unroll
  for (uint32_t s = 0; s < B; ++s)
    if (s < ns) {
#pragma unroll
      for (int i = 0; i < DPW; ++i) acc[i] = fmaf(fac[s], pre[s][i], acc[i]);
    }
  for (uint32_t s0 = B; s0 < ns; s0 += 16u) {
    float v[16][DPW];
#pragma unroll
    for (uint32_t j = 0; j < 16; ++j) load_few<DPW>(v[j], base + (size_t)min(s0 + j, ns - 1u) * stride + lane * DPW);
#pragma unroll
    for (uint32_t j = 0; j < 16; ++j)
      if (s0 + j < ns) {
#pragma unroll
        for (int i = 0; i < DPW; ++i) acc[i] = fmaf(fac[s0 + j], v[j][i], acc[i]);
      }
  }
  float* o = a.out + (size_t)z * a.qh * HD + (size_t)qhead * HD + lane * DPW;
#pragma unroll
  for (int i = 0; i < DPW; ++i) o[i] = acc[i] / l;
}


// Batched-prefill attention on the matrix cores (FlashAttention-style): a
// workgroup owns TT tiles of 16 consecutive prompt tokens, the G query heads
// of one KV head (one wavefront per head and tile) and one position split,
// and reads each K / V row of its positions once for all 16 TT G query rows
// (the decode kernel with a token dimension reads them once per token).  Per
// tile of 16 positions:
//   * S^T = K Q^T on v_mfma_f32_16x16x4f32 (f32 products, f32 sums): lane l
//     supplies K[position l % 16][dim] and q[token l % 16][dim] for the dims of
//     its group l / 16 (HD / 4 consecutive dims each; the dims are summed in
//     two interleaved chains), so the result lane holds the scores of token
//     l % 16 at positions 4 (l / 16) + v, v = 0..3;
//   * online softmax per token (running maximum m, exp-sum l, output rescaled
//     by exp(m - m')), each token's maximum reduced over its 4 lanes;
//   * O^T += V^T P^T, four MFMAs per 16 dims: MFMA t takes positions
//     4 k + t (k = l / 16), the order in which the lane already holds P, so
//     the scores never move between lanes; V is staged transposed in LDS.
// K and V tiles are staged through LDS (double-buffered, one barrier per
// tile); rows past the split read as zeros through a bounded buffer resource.
// Token z (position hist + z) attends positions 0 .. hist + z in the split's
// range [sp c, (sp + 1) c) with c = att_chunk(hist + z + 1, nsplit), the
// chunking attn_merge reads, and writes the same chunk records (m in
// natural-log units) or, when its positions fit one chunk, its output.
// Scores are dot / denom (division) and exp is expf, as in attn_split; only
// the order of the sums differs.
constexpr uint32_t APF_TOK = 16;  // tokens per wavefront = positions per tile
template <int G, int HD, int TT>
__global__ __launch_bounds__(64 * G * TT) void attn_prefill(AttnArgs a) {
  constexpr uint32_t KS = HD / 4;              // dims per lane group (k steps of S)
  constexpr uint32_t DT = HD / 16;             // 16-dim tiles of O^T
  constexpr uint32_t KP = HD + 4;              // LDS row stride of the K tile (floats)
  constexpr uint32_t VP = APF_TOK + 4;         // LDS row stride of the V^T tile
  constexpr uint32_t NTH = 64u * G * TT;
  constexpr uint32_t NCH = APF_TOK * HD / 4;   // 16-byte chunks of one K (or V) tile
  constexpr uint32_t CPT = (NCH + NTH - 1) / NTH;
  __shared__ __align__(16) float kt[2][APF_TOK * KP];
  __shared__ __align__(16) float vt[2][HD * VP];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t r = lane & 15u, gq = lane >> 4;
  // wavefront w: query head w % G of KV head g, tokens z0 .. z0 + 15 (tile w / G of the workgroup's TT)
  const uint32_t sp = blockIdx.x, g = blockIdx.y, zw = blockIdx.z * APF_TOK * TT;
  const uint32_t z0 = zw + (wave / G) * APF_TOK;
  const uint32_t qhead = g * G + wave % G, kvw = a.kvh * HD;
  const uint32_t zl = min(a.ntok, z0 + APF_TOK) - 1u;  // this tile's last token (or the prompt's)
  const uint32_t z = z0 + r;
  const bool zok = z < a.ntok;
  // this token's range in split sp, and the union over the workgroup's tokens
  // (chunks never shrink with the token: first start .. last end)
  const uint32_t tot = a.hist + (zok ? z : zl) + 1u, ch = att_chunk(tot, a.nsplit);
  const uint32_t r0 = sp * ch, r1 = min(tot, r0 + ch);
  const uint32_t zwl = min(a.ntok, zw + APF_TOK * TT) - 1u;
  const uint32_t totl = a.hist + zwl + 1u, chl = att_chunk(totl, a.nsplit);
  const uint32_t lo = sp * att_chunk(a.hist + zw + 1u, a.nsplit), hi = min(totl, sp * chl + chl);
  if (lo >= hi) return;  // uniform: no token of the tile has positions in this split
  // K / V rows 0 .. hi - 1 of KV head g; rows past hi read as zeros
  const uint32_t rb = ((hi - 1u) * kvw + HD) * 4u;
  const AttRsrc kr = att_rsrc(a.k_hist + g * HD, rb), vr = att_rsrc(a.v_hist + g * HD, rb);

  // q of token z (the tile's last token for rows past the prompt), dims gq KS ..
  float qv[KS];
  {
    const float* qp = a.q + ((size_t)(zok ? z : zl) * a.qh + qhead) * HD + gq * KS;
#pragma unroll
    for (uint32_t i = 0; i < KS / 4; ++i) {
      const float4 v = *reinterpret_cast<const float4*>(qp + 4 * i);
      qv[4 * i] = v.x; qv[4 * i + 1] = v.y; qv[4 * i + 2] = v.z; qv[4 * i + 3] = v.w;
    }
  }
  // staging: chunk c = tid + NTH i of a tile: row c / (HD / 4), dims 4 (c % (HD / 4)) ..
  float4 kreg[CPT], vreg[CPT];
  auto fetch = [&](uint32_t p) {
#pragma unroll
    for (uint32_t i = 0; i < CPT; ++i) {
      const uint32_t c = min(tid + NTH * i, NCH - 1u), row = c / (HD / 4), c4 = c % (HD / 4);
      const uint32_t off = ((p + row) * kvw + 4u * c4) * 4u;
      const auto k4 = __builtin_amdgcn_raw_buffer_load_b128(kr, off, 0, ATT_AUX_NT);
      const auto v4 = __builtin_amdgcn_raw_buffer_load_b128(vr, off, 0, ATT_AUX_NT);
      kreg[i] = make_float4(__uint_as_float(k4[0]), __uint_as_float(k4[1]), __uint_as_float(k4[2]), __uint_as_float(k4[3]));
      vreg[i] = make_float4(__uint_as_float(v4[0]), __uint_as_float(v4[1]), __uint_as_float(v4[2]), __uint_as_float(v4[3]));
    }
  };
  auto stage = [&](uint32_t b) {
#pragma unroll
    for (uint32_t i = 0; i < CPT; ++i) {
      const uint32_t c = tid + NTH * i, row = c / (HD / 4), c4 = c % (HD / 4);
      if (c < NCH) {
        *reinterpret_cast<float4*>(&kt[b][row * KP + 4u * c4]) = kreg[i];
        float* vd = &vt[b][(4u * c4) * VP + row];
        vd[0] = vreg[i].x; vd[VP] = vreg[i].y; vd[2 * VP] = vreg[i].z; vd[3 * VP] = vreg[i].w;
      }
    }
  };

  f32x4 o[DT];
#pragma unroll
  for (uint32_t d = 0; d < DT; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  fetch(lo);
  stage(0);
  __syncthreads();
  uint32_t b = 0;
  for (uint32_t p = lo; p < hi; p += APF_TOK, b ^= 1u) {
    const bool more = p + APF_TOK < hi;
    if (more) fetch(p + APF_TOK);
    // S^T: two chains over the lane group's dims
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    const float* kp = &kt[b][r * KP + gq * KS];
#pragma unroll
    for (uint32_t i = 0; i < KS / 4; ++i) {
      const float4 k4 = *reinterpret_cast<const float4*>(kp + 4 * i);
      const float kk[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
      for (uint32_t e = 0; e < 4; ++e)
        acc[e & 1u] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[e], qv[4 * i + e], acc[e & 1u], 0, 0, 0);
    }
    // scores of token z at positions p + 4 gq + v, masked to its range
    float sv[4], mx = -INFINITY;
#pragma unroll
    for (uint32_t v = 0; v < 4; ++v) {
      const uint32_t pos = p + 4u * gq + v;
      const float sc = (acc[0][v] + acc[1][v]) / a.denom;
      sv[v] = (zok && pos >= r0 && pos < r1) ? sc : -INFINITY;
      mx = fmaxf(mx, sv[v]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mn = fmaxf(m, mx);
    float pv[4];
    if (mn == -INFINITY) {  // nothing of this token's range yet
#pragma unroll
      for (uint32_t v = 0; v < 4; ++v) pv[v] = 0.f;
    } else {
      const float al = expf(m - mn);  // m = -inf: 0
      float ps = 0.f;
#pragma unroll
      for (uint32_t v = 0; v < 4; ++v) {
        pv[v] = expf(sv[v] - mn);
        ps += pv[v];
      }
      l = fmaf(l, al, ps);
#pragma unroll
      for (uint32_t d = 0; d < DT; ++d)
#pragma unroll
        for (uint32_t v = 0; v < 4; ++v) o[d][v] *= al;
      m = mn;
    }
    // O^T += V^T P^T: MFMA t takes positions 4 gq + t
#pragma unroll
    for (uint32_t d = 0; d < DT; ++d) {
      const float4 v4 = *reinterpret_cast<const float4*>(&vt[b][(16u * d + r) * VP + 4u * gq]);
      o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4.x, pv[0], o[d], 0, 0, 0);
      o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4.y, pv[1], o[d], 0, 0, 0);
      o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4.z, pv[2], o[d], 0, 0, 0);
      o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4.w, pv[3], o[d], 0, 0, 0);
    }
    if (more) stage(b ^ 1u);  // its last readers were the previous tile's, before the last barrier
    __syncthreads();
  }
  // the token's exp-sum over its four lane groups
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (!zok || r0 >= r1) return;
  const uint32_t ns = (tot + ch - 1u) / ch;
  // lane holds O^T[16 d + 4 gq + v][token z]
  if (ns == 1) {
    float* op = a.out + ((size_t)z * a.qh + qhead) * HD + 4u * gq;
#pragma unroll
    for (uint32_t d = 0; d < DT; ++d)
      *reinterpret_cast<float4*>(op + 16u * d) = make_float4(o[d][0] / l, o[d][1] / l, o[d][2] / l, o[d][3] / l);
  } else {
    float* w = a.ws + (((size_t)z * a.nsplit + sp) * a.qh + qhead) * att_rec(HD);
#pragma unroll
    for (uint32_t d = 0; d < DT; ++d)
      *reinterpret_cast<float4*>(w + 16u * d + 4u * gq) = make_float4(o[d][0], o[d][1], o[d][2], o[d][3]);
    if (gq == 0) { w[HD] = m; w[HD + 1] = l; }
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

bool attention_supported(uint32_t qh, uint32_t kvh, uint32_t hd, uint64_t total) {
  if (kvh == 0 || qh % kvh != 0) return false;
  if (total > (uint64_t)ATT_MAX_SPLITS * ATT_MAX_CHUNK) return false;
  const uint32_t G = qh / kvh;
  const bool g_ok = G == 1 || G == 2 || G == 4 || G == 8;
  const bool hd_ok = hd == 64 || hd == 128 || hd == 256;
  return g_ok && hd_ok && G * (hd / 16) <= 64;
}

// Chunks per KV head: 64 positions each while that keeps the launch within
// about 256 workgroups (one per CU), longer chunks beyond (at most
// ATT_MAX_SPLITS chunks of at most ATT_MAX_CHUNK positions).  Timed on
// 32 q / 8 KV heads, hd 128, split + merge per layer: 256 workgroups beat
// 1024 at every length from 256 to 8192 positions (9.3 vs 13.2 us at 512,
// 20.5 vs 24.5 us at 8192) and 512 beat neither (27.9 us at 8000 against
// 18.9 for 256); workgroups of chunks past the end still cost their dispatch.
uint32_t attention_splits(uint32_t total, uint32_t kvh) {
  uint32_t n = (total + ATT_MIN_CHUNK - 1) / ATT_MIN_CHUNK;
  uint32_t cap = 256u / (kvh ? kvh : 1u);
  if (cap > ATT_MAX_SPLITS) cap = ATT_MAX_SPLITS;
  if (cap < 1) cap = 1;
  if (n > cap) n = cap;
  const uint32_t lo = (total + ATT_MAX_CHUNK - 1) / ATT_MAX_CHUNK;
  if (n < lo) n = lo;
  return n < 1 ? 1 : n;
}

// Launch regimes of single-query attention, each one fixed shape so that one
// captured graph serves every position in it.  cap = the largest context the
// caller will use (the model's KV capacity; the API passes the context
// itself).  Workgroups target about 256 (one per CU) and chunks of at least
// 64 positions.  Timed per layer on 32 q / 8 KV heads, hd 128, split + merge,
// graph replay over 32 layers of K/V:
//   0  context <= 64: one workgroup per query head, one chunk, no merge
//      (4.7-5.6 us; per KV head 5.4-6.7);
//   1  <= 64 Sq (Sq = min(256 / qh, 8) chunks): per query head, 64-position chunks,
//      4 wavefronts (96-512 positions: 7.4-7.8 us; per KV head 9.1-9.5);
//   2  <= 128 Sq: per query head, 8 wavefronts (1024 positions: 9.6 vs 10.1);
//   3  <= 64 Skv (Skv = attention_splits(cap)): per KV head, 4 wavefronts;
//   4  beyond: per KV head, 8 wavefronts.
// The workgroups of one chunk's query heads sit nsplit apart in dispatch
// order, so with nsplit a multiple of 8 they land on one XCD and the re-reads
// of that chunk's K/V by the G heads of a group hit its L2.  Past ~1K
// positions those re-reads (G x the K/V bytes through L2) cost more than the
// per-query-head layout gains, so regimes 3-4 read each K/V row once per KV
// head; Sq stops at 8 so the per-query-head regimes end by 1024 positions.
static uint32_t regime_sq(uint32_t qh) {
  const uint32_t s = qh >= 256 ? 1u : 256u / qh;
  return s > 8 ? 8u : s;
}
static uint32_t regime_skv(uint64_t cap, uint32_t kvh) {
  return attention_splits((uint32_t)(cap < 0xFFFFFFFFull ? cap : 0xFFFFFFFFull), kvh);
}
// Regime 0's longest context (one chunk per query head, no merge): 64, or
// rf_tune_attention_single's 128 / 256 (8 wavefronts above 64).  Timed in
// the 8B decode at positions 40-168 (graph replay, one-pass kernel): 64
// gives 536 tok/s, 128 529, 256 520 (two passes of the split kernel with
// the merging o-projection beat one longer chunk there).
static uint32_t g_single_max = ATT_MIN_CHUNK;
void set_attention_single(uint32_t n) { g_single_max = n; }
uint32_t attention_single() { return g_single_max; }

AttnShape attention_regime_shape(int r, uint32_t qh, uint32_t kvh, uint64_t cap) {
  const uint32_t sq = regime_sq(qh);
  const uint32_t skv = regime_skv(cap, kvh);
  switch (r) {
    case 0: return AttnShape{1, 1, g_single_max > ATT_MIN_CHUNK ? 8u : 4u};
    case 1: return AttnShape{1, sq, 4};
    case 2: return AttnShape{1, sq, 8};
    case 3: return AttnShape{0, skv, 4};
    default: return AttnShape{0, skv, 8};
  }
}
int attention_regime(uint64_t total, uint32_t qh, uint32_t kvh, uint64_t cap) {
  const uint64_t sq = regime_sq(qh);
  if (total <= g_single_max) return 0;
  if (total <= ATT_MIN_CHUNK * sq) return 1;
  if (total <= 2 * ATT_MIN_CHUNK * sq) return 2;
  return total <= ATT_MIN_CHUNK * (uint64_t)regime_skv(cap, kvh) ? 3 : 4;
}

uint64_t attention_ws_floats(uint32_t nsplit, uint32_t qh, uint32_t hd) {
  return (uint64_t)nsplit * qh * att_rec(hd);
}

// Which decode launches (ntok == 0) take the one-pass kernel
// (rf_tune_attention_kernel): 1 (default) those per query head, 2 all, 0
// none; prefill batches take the two-pass kernel.  Timed in the 8B Q8_0
// decode (graph replay, attention group per layer incl. the merge kernel):
// positions 32-96 (per query head) 4.47 against 4.89 us, 540 against 536
// tok/s; about 2048 positions (per KV head, G = 4) 13.8 against 12.1 us;
// about 8100 positions 19.9 against 19.5 us.  With four query heads per
// slot the one-pass kernel needs all four scores in every lane (16 row sums
// per four positions) and 218 registers; the two-pass kernel transposes the
// four sums in 5 exchanges and owns V dims per lane.
static int g_att_kernel = 1;
void set_attention_kernel(int mode) { g_att_kernel = mode; }
int attention_kernel() { return g_att_kernel; }

template <int G, int DPL, int W, bool PERQ = false>
static void launch_split_t(const AttnArgs& a, hipStream_t st) {
  if (a.ntok == 0 && (g_att_kernel == 2 || (g_att_kernel == 1 && PERQ))) {
    RF_KLAUNCH((attn_flash<G, DPL, W, PERQ>), dim3(a.nsplit, PERQ ? a.qh : a.kvh, 1), dim3(64 * W), 0, st, a);
    return;
  }
  RF_KLAUNCH((attn_split<G, DPL, W, PERQ>), dim3(a.nsplit, PERQ ? a.qh : a.kvh, a.ntok ? a.ntok : 1),
                     dim3(64 * W), 0, st, a);
}

// Wavefronts per workgroup for chunks of up to `chunk` positions (one round
// of loads per pass covers 16 W positions).  Timed on 32 q / 8 KV heads, hd
// 128, split + merge per layer, graph replay over 32 layers of K/V: W = 8
// wins once chunks pass 64 positions (8192 positions, 32 chunks: 19.3 vs
// 20.6 us; 4096: 13.8 vs 15.0 us) and loses below (64 positions: 6.0 vs
// 5.6 us); W = 16 (1024 threads, 128 VGPRs) spills and was slower everywhere.
uint32_t attention_waves(uint32_t chunk, uint32_t) { return chunk <= 64 ? 4u : 8u; }
uint32_t att_chunk_positions(uint64_t total, uint32_t nsplit) { return att_chunk((uint32_t)total, nsplit); }
static_assert(ATT_PREFILL_CHUNK == ATT_MAX_CHUNK, "prefill chunks are the kernel's longest");

hipError_t launch_attention_naive(const AttnArgs& a, hipStream_t st) {
  RF_KLAUNCH(attn_naive, dim3(a.qh), dim3(256), 0, st, a);
  return hipGetLastError();
}

// Token batches on the matrix-core kernel (rf_tune_prefill_attention):
// G = 1, 2, 4 or 8 query heads per KV head, head_dim 64 or 128, cache
// offsets within 32 bits, and more than APF_MIN_TOTAL positions.  Timed on
// the 8B Q8_0 prompt (32 / 8 heads, hd 128), whole prompt: 8000 tokens
// 998 ms against 1520 ms with the split kernel, 2048 tokens 209 against 224
// ms, but 512 tokens 49.5 against 47.8 ms: for short contexts the split
// kernel's workgroup per token and KV head (K / V from L2) is quicker.
// Mode 2 takes the kernel at every length (tests of short prompts).
constexpr uint64_t APF_MIN_TOTAL = 1024;
static int g_apf = 1;
void set_prefill_attention_mfma(int mode) { g_apf = mode; }
int prefill_attention_mfma() { return g_apf; }
bool prefill_attention_mfma_supported(uint32_t qh, uint32_t kvh, uint32_t hd, uint64_t total) {
  if (g_apf == 0 || kvh == 0 || qh % kvh || (g_apf == 1 && total <= APF_MIN_TOTAL)) return false;
  const uint32_t G = qh / kvh;
  return (G == 1 || G == 2 || G == 4 || G == 8) && (hd == 64 || hd == 128) &&
         total * kvh * hd * 4 < (1ull << 31);
}
// Position splits of a prefill launch on that kernel: at least enough
// workgroups (16-token tiles x KV heads x splits) for 256 CUs, and about 256
// positions per split past that, at most 32 and no more than chunks of
// ATT_MIN_CHUNK positions give (att_chunk's smallest chunk).
// Token tiles per workgroup: two for G <= 4 (the workgroup's K / V tiles
// serve 32 tokens; 8000-token 8B prompt 965 against 997 ms with one), one
// for G = 8 (512 threads already).
template <int G> constexpr int apf_tiles() { return G <= 4 ? 2 : 1; }
uint32_t prefill_attention_mfma_splits(uint64_t total, uint64_t ntok, uint32_t kvh) {
  const uint64_t per = APF_TOK * 2;  // workgroups of two token tiles (G = 8: one; more splits then)
  const uint64_t tiles = (ntok + per - 1) / per * (kvh ? kvh : 1);
  uint64_t n = (256 + tiles - 1) / tiles;
  const uint64_t by_len = (total + 255) / 256, most = (total + ATT_MIN_CHUNK - 1) / ATT_MIN_CHUNK;
  if (n < by_len) n = by_len;
  if (n > 32) n = 32;
  if (n > most) n = most;
  return (uint32_t)(n < 1 ? 1 : n);
}

template <int G, int HD>
static void launch_apf_t(const AttnArgs& a, hipStream_t st) {
  constexpr int TT = apf_tiles<G>();
  RF_KLAUNCH((attn_prefill<G, HD, TT>), dim3(a.nsplit, a.kvh, (a.ntok + TT * APF_TOK - 1) / (TT * APF_TOK)),
             dim3(64 * G * TT), 0, st, a);
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t st) {
  if (a.nsplit < 1 || a.nsplit > ATT_MAX_SPLITS) return hipErrorInvalidValue;
  const uint32_t G = a.qh / a.kvh, dpl = a.hd / 16;
  if (a.ntok && !a.per_q && prefill_attention_mfma_supported(a.qh, a.kvh, a.hd, (uint64_t)a.hist + a.ntok)) {
    switch (G * 1000 + a.hd) {
      case 1064: launch_apf_t<1, 64>(a, st); break;
      case 1128: launch_apf_t<1, 128>(a, st); break;
      case 2064: launch_apf_t<2, 64>(a, st); break;
      case 2128: launch_apf_t<2, 128>(a, st); break;
      case 4064: launch_apf_t<4, 64>(a, st); break;
      case 4128: launch_apf_t<4, 128>(a, st); break;
      case 8064: launch_apf_t<8, 64>(a, st); break;
      default: launch_apf_t<8, 128>(a, st); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nsplit == 1 || a.defer_merge) return e;
    const dim3 mg(a.qh, 1, a.ntok);
    if (a.hd == 64) RF_KLAUNCH(attn_merge<1>, mg, dim3(64), 0, st, a);
    else RF_KLAUNCH(attn_merge<2>, mg, dim3(64), 0, st, a);
    return hipGetLastError();
  }
  // API mode knows the context on the host; model mode passes the regime's W.
  const uint32_t w = a.waves ? a.waves : attention_waves(att_chunk(a.hist + 1, a.nsplit), G * a.hd);
  if (w != 4 && w != 8) return hipErrorInvalidValue;
  bool done = false;
  if (a.per_q) {  // one workgroup per query head: G = 1 kernels, any GQA ratio
    switch (dpl * 2 + (w == 8 ? 1 : 0)) {
      case 8: launch_split_t<1, 4, 4, true>(a, st); break;
      case 9: launch_split_t<1, 4, 8, true>(a, st); break;
      case 16: launch_split_t<1, 8, 4, true>(a, st); break;
      case 17: launch_split_t<1, 8, 8, true>(a, st); break;
      case 32: launch_split_t<1, 16, 4, true>(a, st); break;
      case 33: launch_split_t<1, 16, 8, true>(a, st); break;
      default: return hipErrorInvalidValue;
    }
    done = true;
  }
#define RF_ATT(GG, DD)                                          \
  if (!done && G == GG && dpl == DD) {                          \
    if (w == 4) launch_split_t<GG, DD, 4>(a, st);               \
    else launch_split_t<GG, DD, 8>(a, st);                      \
    done = true;                                                \
  }
  RF_ATT(1, 4) RF_ATT(1, 8) RF_ATT(1, 16) RF_ATT(2, 4) RF_ATT(2, 8) RF_ATT(2, 16)
  RF_ATT(4, 4) RF_ATT(4, 8) RF_ATT(4, 16) RF_ATT(8, 4) RF_ATT(8, 8)
#undef RF_ATT
  if (!done) return hipErrorInvalidValue;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.nsplit == 1 || a.defer_merge) return e;
  const dim3 mg(a.qh, 1, a.ntok ? a.ntok : 1);
  switch (a.hd) {
    case 64: RF_KLAUNCH(attn_merge<1>, mg, dim3(64), 0, st, a); break;
    case 128: RF_KLAUNCH(attn_merge<2>, mg, dim3(64), 0, st, a); break;
    default: RF_KLAUNCH(attn_merge<4>, mg, dim3(64), 0, st, a); break;  // 256 (attention_supported)
  }
  return hipGetLastError();
}

// Loads this file's code object on the current device (HIP defers that to a
// kernel's first use, which may otherwise fall inside a stream capture).
hipError_t load_module_attention() {
  hipFuncAttributes fa;
  return hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(attn_merge<2>));
}

}  // namespace rf
