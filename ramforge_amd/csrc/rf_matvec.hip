// rf_matvec.hip — batch-1 dequant-dot matvec for GGUF block formats (gfx950).
//
// Replaces the CPU kernels behind compute_dispatch::matvec_backend
// (runtime/src/compute_dispatch.rs:40-58): quant::matvec_<fmt>
// (core/src/quant.rs:898-1489) and CpuBackend::matvec for F32
// (runtime/src/backend.rs:173-218).  Layout is the reference's: raw GGUF
// bytes, row-major [out][in], y[o] = sum_i W[o,i] x[i] (core/src/compute.rs:7-14).
//
// Work decomposition (batch-1 matvec is HBM-bound, so no MFMA):
//   * A workgroup owns a tile of `rows_per_tile` consecutive rows.  The tile is
//     one contiguous byte range of the weight matrix; it is copied into LDS
//     with 16-byte coalesced global loads (the only HBM traffic for W).
//   * Thread t owns unit u = t % units (32 consecutive inputs) for the rows
//     g, g + rg, g + 2rg, ... of the tile (g = t / units).  Its 32 x values
//     live in registers and are reused for every row it computes.
//   * Each thread decodes its unit from LDS (nibbles/int8 + scales in
//     registers) and produces one partial per row; partials are reduced
//     through LDS and a 64-lane shuffle reduction, one row per wavefront.
//   * Optional fusions for the decode step: RMSNorm of x as a prologue (the
//     workgroup's units cover x exactly once, so sum(x^2) is a workgroup
//     reduction of values already in registers), a residual add epilogue, and
//     a dual gate/up tile with a SiLU(gate)*up epilogue.
#include "rf_kernels.h"

#include <mutex>

namespace rf {

// Copy `bytes` from global `src` to LDS `dst` (16-byte aligned), all threads.
__device__ __forceinline__ void copy_tile(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src,
                                          uint32_t bytes, uint32_t tid, uint32_t nth) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  if ((reinterpret_cast<uintptr_t>(src) & 15u) == 0) {
    const uint32_t n16 = bytes >> 4;
    const u32x4* s4 = reinterpret_cast<const u32x4*>(src);
    u32x4* d4 = reinterpret_cast<u32x4*>(dst);
    constexpr int UNR = 8;
    for (uint32_t base = 0; n16 && base < n16; base += nth * UNR) {
      u32x4 r[UNR];
#pragma unroll
      for (int j = 0; j < UNR; ++j) {  // unconditional (clamped) loads keep them all in flight
        const uint32_t i = min(base + j * nth + tid, n16 - 1u);
        r[j] = __builtin_nontemporal_load(s4 + i);
      }
#pragma unroll
      for (int j = 0; j < UNR; ++j) {
        const uint32_t i = base + j * nth + tid;
        if (i < n16) d4[i] = r[j];
      }
    }
    for (uint32_t i = (n16 << 4) + tid; i < bytes; i += nth) dst[i] = src[i];
  } else if ((reinterpret_cast<uintptr_t>(src) & 3u) == 0) {
    const uint32_t n4 = bytes >> 2;
    const uint32_t* s = reinterpret_cast<const uint32_t*>(src);
    uint32_t* d = reinterpret_cast<uint32_t*>(dst);
    for (uint32_t i = tid; i < n4; i += nth) d[i] = s[i];
    for (uint32_t i = (n4 << 2) + tid; i < bytes; i += nth) dst[i] = src[i];
  } else {
    for (uint32_t i = tid; i < bytes; i += nth) dst[i] = src[i];
  }
}

// x[32u .. 32u+31] with eight unconditional 16-byte loads (u < units always
// holds, so every thread reads in bounds).  The host guarantees 16-byte
// aligned x and norm weights for the tiled kernels: a data-dependent branch
// around these loads makes the compiler drain the memory counter behind the
// in-flight tile loads, which costs more than the whole decode.
__device__ __forceinline__ void load_xunit(XUnit& xu, const float* __restrict__ x, uint32_t u) {
  const float4* p = reinterpret_cast<const float4*>(x + 32u * u);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 v = p[i];
    xu.v[4 * i] = v.x; xu.v[4 * i + 1] = v.y; xu.v[4 * i + 2] = v.z; xu.v[4 * i + 3] = v.w;
  }
}

// Norm weights of unit u (same addressing as load_xunit).
__device__ __forceinline__ void load_nwunit(float (&nw)[32], const float* __restrict__ w, uint32_t u) {
  const float4* p = reinterpret_cast<const float4*>(w + 32u * u);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 v = p[i];
    nw[4 * i] = v.x; nw[4 * i + 1] = v.y; nw[4 * i + 2] = v.z; nw[4 * i + 3] = v.w;
  }
}

// RMSNorm prologue (core/src/compute.rs:291-319: x / sqrt(mean(x^2) + eps) * w),
// with the reciprocal of the rms.  Threads of row group 0 hold every unit of x
// exactly once, so sum(x^2) is a workgroup reduction of register values.  The
// weights arrive in registers (loaded with x, ahead of the weight tiles).
__device__ __forceinline__ void norm_xunit(XUnit& xu, const float (&nw)[32], bool first_group, uint32_t in_dim,
                                           float eps, float* wsum, uint32_t tid, uint32_t nth) {
  float ss = 0.f;
  if (first_group) {
#pragma unroll
    for (int i = 0; i < 32; ++i) ss = fmaf(xu.v[i], xu.v[i], ss);
  }
  ss = rf_wave_sum(ss);
  if ((tid & 63u) == 0) wsum[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
  for (uint32_t i = 0; i < (nth >> 6); ++i) tot += wsum[i];
  const float inv = 1.0f / sqrtf(tot / (float)in_dim + eps);
#pragma unroll
  for (int i = 0; i < 32; ++i) xu.v[i] = xu.v[i] * inv * nw[i];
}

__device__ __forceinline__ void finish_xunit(XUnit& xu) {
  float lo = 0.f, hi = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) { lo += xu.v[i]; hi += xu.v[16 + i]; }
  xu.sum_lo = lo;
  xu.sum_hi = hi;
  xu.sum = lo + hi;
}

// Contribution of unit `sub` of the block at `blk`: the dot, or for a unit of
// x holding an infinity or NaN the kind of the reference's terms
// (unit_kinds), so the row sums come out as the reference's NaN / +-inf.
// Only the formats with a min term need that: their dot subtracts
// dmin m sum(x), which turns the reference's infinite terms into inf - inf.
// The signed-code dots (and F32) multiply each code by x, which gives the
// reference's infinities and NaNs by itself.
template <uint32_t T>
constexpr bool has_min_term() { return T == T_Q4_K || T == T_Q5_K || T == T_Q2_K; }

template <uint32_t T>
__device__ __forceinline__ float unit_dot(const uint8_t* b, uint32_t blk, uint32_t sub, const XUnit& x, bool finite) {
  if constexpr (has_min_term<T>()) return finite ? Fmt<T>::dot(b, blk, sub, x) : unit_kinds<T>(b, blk, sub, x);
  else return Fmt<T>::dot(b, blk, sub, x);
}

template <uint32_t T, int EPI>
__global__ __launch_bounds__(1024) void matvec_tiled(MvArgs a) {
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ float wsum[16];
  constexpr uint32_t UPB = Fmt<T>::QK / 32u;  // units per block
  const uint32_t tid = threadIdx.x, nth = blockDim.x;
  const uint32_t bid = blockIdx.x;
  const int s = (a.nseg > 2 && bid >= a.seg[2].tile_begin) ? 2 : ((a.nseg > 1 && bid >= a.seg[1].tile_begin) ? 1 : 0);
  const uint8_t* w = s == 0 ? a.seg[0].w : (s == 1 ? a.seg[1].w : a.seg[2].w);
  float* y = s == 0 ? a.seg[0].y : (s == 1 ? a.seg[1].y : a.seg[2].y);
  const float* res = s == 0 ? a.seg[0].res : (s == 1 ? a.seg[1].res : a.seg[2].res);
  const uint32_t seg_rows = s == 0 ? a.seg[0].rows : (s == 1 ? a.seg[1].rows : a.seg[2].rows);
  const uint32_t tile_begin = s == 0 ? a.seg[0].tile_begin : (s == 1 ? a.seg[1].tile_begin : a.seg[2].tile_begin);

  const uint32_t r0 = (bid - tile_begin) * a.rows_per_tile;
  const uint32_t nrows = min(a.rows_per_tile, seg_rows - r0);
  const uint32_t row_bytes = a.row_bytes;
  const uint32_t tile_bytes = nrows * row_bytes;

  copy_tile(lds, w + (size_t)r0 * row_bytes, tile_bytes, tid, nth);
  if (EPI == EPI_SWIGLU) copy_tile(lds + a.tile_stride, a.w_up + (size_t)r0 * row_bytes, tile_bytes, tid, nth);

  const uint32_t units = a.units;
  const uint32_t u = tid % units, g = tid / units;
  const bool active = g < a.rg;
  XUnit xu;
  load_xunit(xu, a.x, u);
  if (a.norm_w != nullptr) {
    float nw[32];
    load_nwunit(nw, a.norm_w, u);
    norm_xunit(xu, nw, active && g == 0, a.in_dim, a.eps, wsum, tid, nth);
  } else {
    __syncthreads();
  }
  finish_xunit(xu);
  const bool xfin = !has_min_term<T>() || unit_finite(xu);

  const uint32_t blk = (u / UPB) * Fmt<T>::BS, sub = u % UPB;
  constexpr int MAXR = 8;
  float part[MAXR], part2[MAXR];
#pragma unroll
  for (int k = 0; k < MAXR; ++k) {
    part[k] = 0.f;
    part2[k] = 0.f;
    const uint32_t r = g + k * a.rg;
    if (active && r < nrows) {
      part[k] = unit_dot<T>(lds, r * row_bytes + blk, sub, xu, xfin);
      if (EPI == EPI_SWIGLU) part2[k] = unit_dot<T>(lds + a.tile_stride, r * row_bytes + blk, sub, xu, xfin);
    }
  }
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int k = 0; k < MAXR; ++k) {
    const uint32_t r = g + k * a.rg;
    if (active && r < nrows) {
      red[r * units + u] = part[k];
      if (EPI == EPI_SWIGLU) red[(nrows + r) * units + u] = part2[k];
    }
  }
  __syncthreads();
  const uint32_t lane = tid & 63u, wave = tid >> 6, nwaves = nth >> 6;
  for (uint32_t r = wave; r < nrows; r += nwaves) {
    float v = 0.f, v2 = 0.f;
    for (uint32_t i = lane; i < units; i += 64u) {
      v += red[r * units + i];
      if (EPI == EPI_SWIGLU) v2 += red[(nrows + r) * units + i];
    }
    v = rf_wave_sum(v);
    if (EPI == EPI_SWIGLU) v2 = rf_wave_sum(v2);
    if (lane == 0) {
      const uint32_t o = r0 + r;
      if (EPI == EPI_STORE) {
        y[o] = v;
      } else if (EPI == EPI_RESIDUAL) {
        y[o] = res[o] + v;  // add_reference(hidden, proj) (compute.rs:321-327)
      } else {
        // silu_reference then mul_reference (compute.rs:337-350, 329-335)
        const float sg = v / (1.0f + expf(-v));
        y[o] = sg * v2;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Persistent streaming variant (the decode hot path).  A grid of about
// (CUs x workgroups-per-CU) workgroups walks the tiles of all segments; each
// workgroup loads its x slice (and applies the fused RMSNorm) once, and keeps
// the next tile's 16-byte words in registers while it decodes the current
// tile from LDS, so every workgroup always has one tile of HBM reads in
// flight.  Requires 16-byte aligned rows (row_bytes % 16 == 0) and weight
// bases; the dual (gate/up) tile is the gate rows followed by the up rows.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int PF = 8;  // prefetch words (16 B) per thread per tile

struct TileRef {
  const u32x4* p0;  // first range (gate / plain rows)
  const u32x4* p1;  // second range (up rows) or null
  uint32_t n0, n;   // words in the first range, total words
  uint32_t r0, nrows;
  int seg;
};

__device__ __forceinline__ TileRef tile_ref(const MvArgs& a, uint32_t tile, bool dual) {
  TileRef t;
  t.seg = (a.nseg > 2 && tile >= a.seg[2].tile_begin) ? 2 : ((a.nseg > 1 && tile >= a.seg[1].tile_begin) ? 1 : 0);
  const uint8_t* w = t.seg == 0 ? a.seg[0].w : (t.seg == 1 ? a.seg[1].w : a.seg[2].w);
  const uint32_t rows = t.seg == 0 ? a.seg[0].rows : (t.seg == 1 ? a.seg[1].rows : a.seg[2].rows);
  const uint32_t tb = t.seg == 0 ? a.seg[0].tile_begin : (t.seg == 1 ? a.seg[1].tile_begin : a.seg[2].tile_begin);
  t.r0 = (tile - tb) * a.rows_per_tile;
  t.nrows = min(a.rows_per_tile, rows - t.r0);
  const uint32_t words = t.nrows * a.row_bytes / 16u;
  t.p0 = reinterpret_cast<const u32x4*>(w + (size_t)t.r0 * a.row_bytes);
  t.n0 = words;
  t.p1 = dual ? reinterpret_cast<const u32x4*>(a.w_up + (size_t)t.r0 * a.row_bytes) : nullptr;
  t.n = dual ? 2 * words : words;
  return t;
}

// Branch-free on purpose: every slot issues one load (indices past the tile
// are clamped to its last word and never stored).  A guarded load, or an
// if/else between the gate and up ranges, makes the compiler drain the memory
// counter before each load and serialises the prefetch.
__device__ __forceinline__ void tile_prefetch(u32x4 (&r)[PF], const TileRef& t, uint32_t tid, uint32_t nth) {
#pragma unroll
  for (int j = 0; j < PF; ++j) {
    const uint32_t i = min(j * nth + tid, t.n - 1u);
    const u32x4* src = i < t.n0 ? t.p0 + i : t.p1 + (i - t.n0);
    r[j] = __builtin_nontemporal_load(src);
  }
}

__device__ __forceinline__ void tile_store(const u32x4 (&r)[PF], uint8_t* lds, uint32_t n, uint32_t tid,
                                           uint32_t nth) {
  u32x4* d = reinterpret_cast<u32x4*>(lds);
#pragma unroll
  for (int j = 0; j < PF; ++j) {
    const uint32_t i = j * nth + tid;
    if (i < n) d[i] = r[j];
  }
}

template <uint32_t T, int EPI>
__global__ __launch_bounds__(512) void matvec_stream(MvArgs a) {
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ float wsum[8];
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  constexpr uint32_t UPB = Fmt<T>::QK / 32u;
  const uint32_t tid = threadIdx.x, nth = blockDim.x;
  const uint32_t ntiles = a.ntiles;
  uint32_t tile = blockIdx.x;
  const uint32_t units = a.units;
  const uint32_t u = tid % units, g = tid / units;
  const bool active = g < a.rg;
  // x and the norm weights are requested first (L2-resident, they return
  // before the weight tile), so the RMSNorm prologue overlaps the tile fetch.
  // Without a norm the x slice is loaded twice instead of branching around
  // the loads.
  XUnit xu;
  load_xunit(xu, a.x, u);
  float nw[32];
  load_nwunit(nw, a.norm_w != nullptr ? a.norm_w : a.x, u);
  u32x4 pf[PF];
  TileRef cur{};
  if (tile < ntiles) {
    cur = tile_ref(a, tile, DUAL);
    tile_prefetch(pf, cur, tid, nth);
  }
  if (a.norm_w != nullptr) norm_xunit(xu, nw, active && g == 0, a.in_dim, a.eps, wsum, tid, nth);
  finish_xunit(xu);
  const bool xfin = !has_min_term<T>() || unit_finite(xu);

  const uint32_t row_bytes = a.row_bytes;
  const uint32_t blk = (u / UPB) * Fmt<T>::BS, sub = u % UPB;
  float* red = reinterpret_cast<float*>(lds + a.red_offset);
  const uint32_t lane = tid & 63u, wave = tid >> 6, nwaves = nth >> 6;
  constexpr int MAXR = 8;

  for (; tile < ntiles; tile += gridDim.x) {
    tile_store(pf, lds, cur.n, tid, nth);
    __syncthreads();
    const TileRef t = cur;
    const uint32_t next = tile + gridDim.x;
    if (next < ntiles) {
      cur = tile_ref(a, next, DUAL);
      tile_prefetch(pf, cur, tid, nth);
    }
    const uint32_t nrows = t.nrows;
#pragma unroll
    for (int k = 0; k < MAXR; ++k) {
      const uint32_t r = g + k * a.rg;
      if (active && r < nrows) {
        red[r * units + u] = unit_dot<T>(lds, r * row_bytes + blk, sub, xu, xfin);
        if (DUAL)
          red[(nrows + r) * units + u] = unit_dot<T>(lds + nrows * row_bytes, r * row_bytes + blk, sub, xu, xfin);
      }
    }
    __syncthreads();
    float* y = t.seg == 0 ? a.seg[0].y : (t.seg == 1 ? a.seg[1].y : a.seg[2].y);
    const float* res = t.seg == 0 ? a.seg[0].res : (t.seg == 1 ? a.seg[1].res : a.seg[2].res);
    for (uint32_t r = wave; r < nrows; r += nwaves) {
      float v = 0.f, v2 = 0.f;
      for (uint32_t i = lane; i < units; i += 64u) {
        v += red[r * units + i];
        if (DUAL) v2 += red[(nrows + r) * units + i];
      }
      v = rf_wave_sum(v);
      if (DUAL) v2 = rf_wave_sum(v2);
      if (lane == 0) {
        const uint32_t o = t.r0 + r;
        if (EPI == EPI_STORE) {
          y[o] = v;
        } else if (EPI == EPI_RESIDUAL) {
          y[o] = res[o] + v;
        } else {
          const float sg = v / (1.0f + expf(-v));
          y[o] = sg * v2;
        }
      }
    }
  }
}

// General fallback: one wavefront per row, bit-exact unit decode straight from
// global memory.  Used when a row has more than 1024 units (in_dim > 32768)
// or for F32 rows whose length is not a multiple of 32.
template <uint32_t T>
__global__ __launch_bounds__(256) void matvec_rowwise(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                      float* __restrict__ y, uint32_t in_dim, uint32_t rows,
                                                      uint32_t row_bytes) {
  const uint32_t lane = threadIdx.x & 63u, r = blockIdx.x * 4u + (threadIdx.x >> 6);
  if (r >= rows) return;
  const uint8_t* row = w + (size_t)r * row_bytes;
  float acc = 0.f;
  constexpr uint32_t UPB = Fmt<T>::QK / 32u;
  float deq[32];
  for (uint32_t u = lane; u < in_dim / 32u; u += 64u) {
    Fmt<T>::dequant(row, (u / UPB) * Fmt<T>::BS, u % UPB, deq);
#pragma unroll
    for (int i = 0; i < 32; ++i) acc = fmaf(deq[i], x[32u * u + i], acc);
  }
  acc = rf_wave_sum(acc);
  if (lane == 0) y[r] = acc;
}

// F32 rows need no decode; Fmt<T_F32>::dequant is only referenced by the
// rowwise kernel for quantized types.
template <>
__global__ __launch_bounds__(256) void matvec_rowwise<T_F32>(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                            float* __restrict__ y, uint32_t in_dim, uint32_t rows,
                                                            uint32_t row_bytes) {
  const uint32_t lane = threadIdx.x & 63u, r = blockIdx.x * 4u + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* wr = reinterpret_cast<const float*>(w + (size_t)r * row_bytes);
  float acc = 0.f;
  for (uint32_t i = lane; i < in_dim; i += 64u) acc = fmaf(wr[i], x[i], acc);
  acc = rf_wave_sum(acc);
  if (lane == 0) y[r] = acc;
}

// ------------------------------------------------------------------ host side

static uint32_t block_elems(uint32_t t) {
  switch (t) {
    case T_Q4_0: case T_Q5_0: case T_Q8_0: return 32;
    case T_Q2_K: case T_Q3_K: case T_Q4_K: case T_Q5_K: case T_Q6_K: case T_Q8_K: return 256;
    case T_F32: return 1;
    default: return 0;
  }
}

static uint32_t block_bytes(uint32_t t) {
  switch (t) {
    case T_Q4_0: return 18; case T_Q5_0: return 22; case T_Q8_0: return 34;
    case T_Q2_K: return 84; case T_Q3_K: return 110; case T_Q4_K: return 144;
    case T_Q5_K: return 176; case T_Q6_K: return 210; case T_Q8_K: return 292;
    case T_F32: return 4;
    default: return 0;
  }
}

bool type_geometry(uint32_t t, uint64_t* qk, uint64_t* bs) {
  const uint32_t a = block_elems(t), b = block_bytes(t);
  if (a == 0) return false;
  if (qk) *qk = a;
  if (bs) *bs = b;
  return true;
}

static uint32_t g_tile_target = 32768;  // LDS bytes per one-shot matvec tile (tunable)
static bool g_stream_enabled = true;    // persistent streaming kernel where eligible
static uint32_t g_stream_tile_cap = 57344;  // bytes of one streaming tile (tunable)
void set_matvec_stream_tile(uint32_t bytes) { g_stream_tile_cap = bytes < 2048 ? 2048 : (bytes > 57344 ? 57344 : bytes); }
void set_matvec_tile_bytes(uint32_t bytes) { g_tile_target = bytes < 4096 ? 4096 : (bytes > 61440 ? 61440 : bytes); }
uint32_t matvec_tile_bytes() { return g_tile_target; }
void set_matvec_stream(bool on) { g_stream_enabled = on; }
bool matvec_stream() { return g_stream_enabled; }

MvPlan plan_matvec(uint32_t t, uint64_t in_dim, bool dual) {
  MvPlan p{};
  const uint64_t units = in_dim / 32;
  const uint64_t rb = in_dim / block_elems(t) * block_bytes(t);
  p.row_bytes = (uint32_t)rb;
  if (in_dim % 32 != 0 || units == 0 || units > 1024) {
    p.tiled = false;
    return p;
  }
  p.tiled = true;
  p.units = (uint32_t)units;
  const uint64_t per_matrix = dual ? g_tile_target / 2 : g_tile_target;
  uint64_t max_rows = per_matrix / rb;
  if (max_rows < 1) max_rows = 1;
  uint64_t rg = units >= 256 ? 1 : 256 / units;
  uint64_t rpt;
  if (rg > max_rows) {  // short rows but a small tile budget: fewer row groups
    rg = max_rows;
    rpt = 1;
  } else {
    rpt = max_rows / rg;
    if (rpt > 8) rpt = 8;
  }
  p.rg = (uint32_t)rg;
  p.rows_per_tile = (uint32_t)(p.rg * rpt);
  p.threads = (uint32_t)(((units * p.rg) + 63) / 64 * 64);
  p.tile_stride = (uint32_t)((p.rows_per_tile * rb + 15) / 16 * 16);
  const uint64_t tile = (uint64_t)p.tile_stride * (dual ? 2 : 1);
  const uint64_t red = (uint64_t)p.rows_per_tile * units * 4 * (dual ? 2 : 1);
  const uint64_t lds = (tile > red ? tile : red) + 16;
  if (lds > 65536 - 512) {  // with the static LDS it would not fit 64 KiB: rowwise kernel
    p.tiled = false;
    return p;
  }
  p.lds_bytes = (uint32_t)lds;

  // Persistent streaming plan: one prefetch of PF 16-byte words per thread
  // bounds the tile; aim for >= 2 workgroups per CU (160 KiB LDS per CU).
  p.stream = false;
  const uint64_t sthreads = (units * rg + 63) / 64 * 64;
  if (rb % 16 == 0 && sthreads <= 512) {
    uint64_t tile_cap = 16ull * PF * sthreads;
    if (tile_cap > g_stream_tile_cap) tile_cap = g_stream_tile_cap;
    const uint64_t per_row = rb * (dual ? 2 : 1);
    uint64_t rows = tile_cap / per_row;
    if (rows > rg * 8) rows = rg * 8;
    if (rows >= 1) {
      const uint64_t tile_bytes = rows * per_row;
      const uint64_t red_off = (tile_bytes + 16 + 15) / 16 * 16;
      const uint64_t s_lds = red_off + rows * units * 4 * (dual ? 2 : 1);
      if (s_lds <= 65536 - 512) {
        p.stream = true;
        p.s_rows_per_tile = (uint32_t)rows;
        p.s_threads = (uint32_t)sthreads;
        p.s_red_offset = (uint32_t)red_off;
        p.s_lds_bytes = (uint32_t)s_lds;
        uint64_t by_lds = 163840 / (s_lds + 256);
        uint64_t by_waves = 16 / (sthreads / 64);  // ~4 waves per SIMD at ~120 VGPRs
        uint64_t w = by_lds < by_waves ? by_lds : by_waves;
        p.s_wgs_per_cu = (uint32_t)(w < 1 ? 1 : w);
      }
    }
  }
  return p;
}

static int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    hipDeviceProp_t prop;
    cached[dev] = hipGetDeviceProperties(&prop, dev) == hipSuccess ? prop.multiProcessorCount : 256;
  }
  return cached[dev];
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <uint32_t T, int EPI>
static hipError_t launch_tiled_t(const MvArgs& a, uint32_t grid, const MvPlan& p, hipStream_t st) {
  RF_KLAUNCH((matvec_tiled<T, EPI>), dim3(grid), dim3(p.threads), p.lds_bytes, st, a);
  return hipGetLastError();
}

// Resident workgroups per CU of one persistent kernel instance (registers,
// LDS and waves all counted by the runtime), cached per shape.  0 when the
// query would run while st is being captured (setup_outside_capture).
template <uint32_t T, int EPI>
static uint32_t stream_occupancy(uint32_t threads, uint32_t lds, hipStream_t st) {
  static std::mutex mu;
  std::lock_guard<std::mutex> lock(mu);
  static uint32_t cache_threads[8] = {0}, cache_lds[8] = {0}, cache_val[8] = {0};
  for (int i = 0; i < 8; ++i)
    if (cache_threads[i] == threads && cache_lds[i] == lds) return cache_val[i];
  if (setup_outside_capture(st) != hipSuccess) return 0;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, matvec_stream<T, EPI>, (int)threads, (size_t)lds) !=
          hipSuccess || n < 1)
    n = 1;
  for (int i = 0; i < 8; ++i)
    if (cache_threads[i] == 0) {
      cache_threads[i] = threads;
      cache_lds[i] = lds;
      cache_val[i] = (uint32_t)n;
      break;
    }
  return (uint32_t)n;
}

template <uint32_t T, int EPI>
static hipError_t launch_stream_t(const MvArgs& a, uint32_t tiles, const MvPlan& p, hipStream_t st) {
  // balanced persistent grid: every workgroup walks k tiles
  const uint32_t occ = stream_occupancy<T, EPI>(p.s_threads, p.s_lds_bytes, st);
  if (occ == 0) return hipErrorStreamCaptureUnsupported;
  const uint64_t max_grid = (uint64_t)cu_count() * occ;
  const uint64_t k = (tiles + max_grid - 1) / max_grid;
  const uint32_t grid = (uint32_t)((tiles + k - 1) / k);
  RF_KLAUNCH((matvec_stream<T, EPI>), dim3(grid), dim3(p.s_threads), p.s_lds_bytes, st, a);
  return hipGetLastError();
}

// ------------------------------------------------ lane kernel (Q8_0)
// GGUF rows read straight into registers, realigned there: one row per
// wavefront at a time, lane l owning blocks l, l + 64, ... of the row.  A
// 34-byte block at byte 34 b starts 0 (even b) or 2 (odd b) bytes into a
// dword: the lane loads the 9 dwords covering it with raw buffer loads
// (dword alignment; offsets past the row return zeros) and takes the codes
// as dwords 1..8 (odd b) or shifts them down by two bytes with v_alignbyte
// (even b).  No LDS tile and no barrier in the row loop: x sits in LDS once
// per workgroup of four wavefronts, about two rows per wavefront.  Signed
// codes times x, the block scale once per block, as the other kernels
// (quant.rs:977-1029 up to the order of the sums).  Rows must start on
// dwords (an even block count per row, a dword-aligned base).
// Timed against the LDS-tiled streaming kernel (graph replay, weights
// rotated over >= 1.2 GiB): Q8_0 4096 x 4096 8.9 against 11.0 us; but
// slower for wider rows (Q8_0 28672 x 8192 67 against 57 us) and for Q4_0
// (14336 x 4096 21 against 17 us, 18-byte blocks: two loads per 32
// weights), and a persistent grid of 8-wavefront workgroups with two blocks
// per lane (always dword aligned) was slower still (12.2 us at 4096 x
// 4096), so it takes Q8_0 rows of up to 4096 inputs only.
typedef __amdgpu_buffer_rsrc_t MvRsrc;
constexpr int MV_RSRC_WORD3 = 0x00020000;
constexpr uint32_t MVL_WAVES = 4;
constexpr uint32_t MVL_MAX_IN = 4096;

// BPL blocks per lane and row (ceil(blocks / 64)); NB rows in flight per
// wavefront (the next row's dwords requested before this row is summed).
template <int BPL, int NB>
__global__ __launch_bounds__(64 * MVL_WAVES) void matvec_lanes(const uint8_t* __restrict__ w,
                                                               const float* __restrict__ x, float* __restrict__ y,
                                                               uint32_t in_dim, uint32_t rows, uint32_t row_bytes) {
  constexpr uint32_t BS = 34, NDW = 9;
  extern __shared__ __align__(16) float xs[];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t nblk = in_dim / 32u;
  const uint32_t stride = gridDim.x * MVL_WAVES;
  uint32_t dw[NB][BPL][NDW];
  auto fetch = [&](uint32_t (&d)[BPL][NDW], uint32_t r) {
    const bool live = r < rows;  // wave-uniform: past the last row every load returns zeros
    const MvRsrc rs = __builtin_amdgcn_make_buffer_rsrc((void*)(w + (size_t)(live ? r : 0u) * row_bytes), 0,
                                                        live ? (int32_t)row_bytes : 0, MV_RSRC_WORD3);
#pragma unroll
    for (int k = 0; k < BPL; ++k) {
      const uint32_t off = (BS * (lane + 64u * k)) & ~3u;
      const auto v0 = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
      const auto v1 = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16u, 0, 0);
      d[k][0] = v0[0]; d[k][1] = v0[1]; d[k][2] = v0[2]; d[k][3] = v0[3];
      d[k][4] = v1[0]; d[k][5] = v1[1]; d[k][6] = v1[2]; d[k][7] = v1[3];
      d[k][8] = __builtin_amdgcn_raw_buffer_load_b32(rs, off + 32u, 0, 0);
    }
  };
  uint32_t r = blockIdx.x * MVL_WAVES + wave;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) fetch(dw[nb], r + (uint32_t)nb * stride);
  // x into LDS behind the first rows' loads
  for (uint32_t i = tid; i < in_dim / 4u; i += 64u * MVL_WAVES)
    reinterpret_cast<float4*>(xs)[i] = reinterpret_cast<const float4*>(x)[i];
  __syncthreads();
  auto finish = [&](const uint32_t (&d)[BPL][NDW], uint32_t rr) {
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < BPL; ++k) {
      const uint32_t b = lane + 64u * k;
      if (b < nblk) {
        const bool odd = (b & 1u) != 0u;
        const uint32_t h = odd ? d[k][0] >> 16 : d[k][0] & 0xFFFFu;
        const float* xb = xs + 32u * b;
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t c = odd ? d[k][i + 1] : __builtin_amdgcn_alignbyte(d[k][i + 1], d[k][i], 2);
          const float4 xv = *reinterpret_cast<const float4*>(xb + 4 * i);
          s = fmaf(rf_sb(c, 0), xv.x, s);
          s = fmaf(rf_sb(c, 1), xv.y, s);
          s = fmaf(rf_sb(c, 2), xv.z, s);
          s = fmaf(rf_sb(c, 3), xv.w, s);
        }
        acc += rf_half_to_float_fast(h) * s;
      }
    }
    acc = rf_wave_sum(acc);
    if (lane == 0 && rr < rows) y[rr] = acc;
  };
  for (; r < rows; r += (uint32_t)NB * stride) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      finish(dw[nb], r + (uint32_t)nb * stride);
      fetch(dw[nb], r + (uint32_t)(nb + NB) * stride);
    }
  }
}

// Whether the lane kernel takes this launch: Q8_0 rows of an even block
// count (dword-aligned rows) and at most MVL_MAX_IN inputs, a dword-aligned
// base and 16-byte aligned x.
static bool lanes_ok(uint32_t t, uint64_t in_dim, const void* w, const float* x) {
  if (t != T_Q8_0 || in_dim == 0 || in_dim % 64 != 0 || in_dim > MVL_MAX_IN) return false;
  return (reinterpret_cast<uintptr_t>(w) & 3u) == 0 && aligned16(x);
}

static int g_lanes_enabled = 1;
void set_matvec_lanes(bool on) { g_lanes_enabled = on ? 1 : 0; }
bool matvec_lanes_on() { return g_lanes_enabled != 0; }

template <int BPL>
static hipError_t launch_lanes_b(const MvSegDesc& s, const float* x, uint64_t in_dim, hipStream_t st) {
  constexpr int NB = 2;
  static std::mutex mu;
  static uint32_t occ = 0;
  const uint32_t lds = (uint32_t)in_dim * 4u;
  {
    std::lock_guard<std::mutex> lock(mu);
    if (occ == 0) {
      if (setup_outside_capture(st) != hipSuccess) return hipErrorStreamCaptureUnsupported;
      int n = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, matvec_lanes<BPL, NB>, 64 * MVL_WAVES,
                                                       (size_t)MVL_MAX_IN * 4u) != hipSuccess || n < 1)
        n = 1;
      occ = (uint32_t)n;
    }
  }
  const uint64_t rows = s.rows;
  const uint64_t want = (rows + MVL_WAVES * NB - 1) / (MVL_WAVES * NB);  // about NB rows per wavefront
  const uint64_t cap = (uint64_t)cu_count() * occ;
  const uint32_t grid = (uint32_t)std::max<uint64_t>(1, std::min(want, cap));
  const uint32_t row_bytes = (uint32_t)(in_dim / 32u * 34u);
  RF_KLAUNCH((matvec_lanes<BPL, NB>), dim3(grid), dim3(64 * MVL_WAVES), lds, st, static_cast<const uint8_t*>(s.w),
             x, s.y, (uint32_t)in_dim, (uint32_t)rows, row_bytes);
  return hipGetLastError();
}

static hipError_t launch_lanes(const MvSegDesc& s, const float* x, uint64_t in_dim, hipStream_t st) {
  return in_dim <= 2048 ? launch_lanes_b<1>(s, x, in_dim, st) : launch_lanes_b<2>(s, x, in_dim, st);
}

template <int EPI>
static hipError_t launch_tiled_e(uint32_t t, const MvArgs& a, uint32_t grid, const MvPlan& p, hipStream_t st,
                                 bool stream) {
#define RF_MV(TT) \
  case TT: return stream ? launch_stream_t<TT, EPI>(a, grid, p, st) : launch_tiled_t<TT, EPI>(a, grid, p, st);
  switch (t) {
    RF_MV(T_Q8_0) RF_MV(T_Q4_0) RF_MV(T_Q5_0) RF_MV(T_Q4_K) RF_MV(T_Q5_K) RF_MV(T_Q6_K) RF_MV(T_Q2_K)
    RF_MV(T_Q3_K) RF_MV(T_Q8_K) RF_MV(T_F32)
    default: return hipErrorInvalidValue;
  }
#undef RF_MV
}

hipError_t launch_matvec_segments(uint32_t t, const MvSegDesc* segs, int nseg, const float* x,
                                  const float* norm_w, float eps, uint64_t in_dim, int epi,
                                  hipStream_t st) {
  if (nseg < 1 || nseg > 3) return hipErrorInvalidValue;
  const bool dual = epi == EPI_SWIGLU;
  MvPlan p = plan_matvec(t, in_dim, dual);
  // The tiled kernels read x and the norm weights as 16-byte vectors; other
  // pointers take the rowwise kernel (plain store epilogue only).
  const bool x_vec = aligned16(x) && (norm_w == nullptr || aligned16(norm_w));
  if (!p.tiled || !x_vec) {
    if (norm_w != nullptr || epi != EPI_STORE) return hipErrorInvalidValue;
    for (int i = 0; i < nseg; ++i) {
      const uint32_t rows = (uint32_t)segs[i].rows;
      if (rows == 0) continue;
      dim3 grid((rows + 3) / 4);
      switch (t) {
#define RF_ROWWISE(TT) case TT: RF_KLAUNCH(matvec_rowwise<TT>, grid, dim3(256), 0, st, static_cast<const uint8_t*>(segs[i].w), x, segs[i].y, (uint32_t)in_dim, rows, p.row_bytes); break;
        RF_ROWWISE(T_Q8_0) RF_ROWWISE(T_Q4_0) RF_ROWWISE(T_Q5_0) RF_ROWWISE(T_Q4_K) RF_ROWWISE(T_Q5_K)
        RF_ROWWISE(T_Q6_K) RF_ROWWISE(T_Q2_K) RF_ROWWISE(T_Q3_K) RF_ROWWISE(T_Q8_K) RF_ROWWISE(T_F32)
#undef RF_ROWWISE
        default: return hipErrorInvalidValue;
      }
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  if (g_lanes_enabled && epi == EPI_STORE && norm_w == nullptr && nseg == 1 && segs[0].rows > 0 &&
      segs[0].rows <= 0xFFFFFFFFull && lanes_ok(t, in_dim, segs[0].w, x))
    return launch_lanes(segs[0], x, in_dim, st);
  bool stream = p.stream && g_stream_enabled;
  for (int i = 0; i < nseg && stream; ++i)
    stream = aligned16(segs[i].w) && (!dual || aligned16(segs[i].w_up));
  const uint32_t rpt = stream ? p.s_rows_per_tile : p.rows_per_tile;
  MvArgs a{};
  uint32_t tiles = 0;
  for (int i = 0; i < nseg; ++i) {
    a.seg[i].w = static_cast<const uint8_t*>(segs[i].w);
    a.seg[i].y = segs[i].y;
    a.seg[i].res = segs[i].res;
    a.seg[i].rows = (uint32_t)segs[i].rows;
    a.seg[i].tile_begin = tiles;
    tiles += (uint32_t)((segs[i].rows + rpt - 1) / rpt);
  }
  if (tiles == 0) return hipSuccess;
  a.nseg = (uint32_t)nseg;
  a.x = x;
  a.norm_w = norm_w;
  a.eps = eps;
  a.in_dim = (uint32_t)in_dim;
  a.units = p.units;
  a.rg = p.rg;
  a.rows_per_tile = p.rows_per_tile;
  a.row_bytes = p.row_bytes;
  a.tile_stride = p.tile_stride;
  a.w_up = dual ? static_cast<const uint8_t*>(segs[0].w_up) : nullptr;
  const uint32_t grid = tiles;  // one-shot kernel: one workgroup per tile
  if (stream) {
    a.rows_per_tile = rpt;
    a.ntiles = tiles;
    a.red_offset = p.s_red_offset;
  }
  switch (epi) {
    case EPI_STORE: return launch_tiled_e<EPI_STORE>(t, a, grid, p, st, stream);
    case EPI_RESIDUAL: return launch_tiled_e<EPI_RESIDUAL>(t, a, grid, p, st, stream);
    case EPI_SWIGLU: return launch_tiled_e<EPI_SWIGLU>(t, a, grid, p, st, stream);
    default: return hipErrorInvalidValue;
  }
}

// Loads this file's code object on the current device (HIP defers that to a
// kernel's first use, which may otherwise fall inside a stream capture) and
// caches the device's CU count the launchers read.
hipError_t load_module_matvec() {
  (void)cu_count();
  hipFuncAttributes fa;
  return hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(matvec_rowwise<T_F32>));
}

}  // namespace rf
