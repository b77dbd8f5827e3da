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

// ------------------------------------------------ wave-staged kernel (Q8_0, Q4_0, Q4_K, Q6_K)
// GGUF rows staged per wavefront: each wavefront owns whole rows (row i,
// i + G, ... for G wavefronts in the grid), loads the bytes of its next row
// (or of its next chunk of at most 8 KiB, for longer rows) with 16-byte
// loads that are contiguous across lanes, writes them into its own LDS
// region and reads the blocks back from there.  The next item's loads are in
// flight while the current one is summed; no barrier after the prologue (a
// wavefront's LDS writes and reads complete in order).  x sits in LDS once
// per workgroup.  Each lane takes eight weights of a block per step: four
// lanes per 32-element block (16 blocks per step), 32 lanes per 256-element
// super-block (2 per step).
//   Q8_0: lane p of a block takes codes 8p..8p+7 (bytes 2+8p.., realigned
//   with v_alignbyte; a block starts 0 or 2 bytes into a dword) times
//   x[8p..8p+7]; Q4_0: bytes 2+4p..2+4p+3, low nibbles times x[4p..4p+3],
//   high nibbles times x[16+4p..16+4p+3]; Q4_K / Q6_K: elements 8p..8p+7 of
//   the super-block, with the sub-block's scale (and min).
// Signed codes times x, the block scale once per block and lane, as the
// other kernels (quant.rs:977-1029 up to the order of the sums); a code of 0
// meets an infinite x as the reference's 0 * inf = NaN term does.  Q4_K
// subtracts dmin m sum(x) of its eight elements; with an infinity or NaN in
// x it takes the kind of the reference's terms instead (unit_kinds).
// Timed under graph replay with >= 1.2 GiB of rotated copies against the
// lane kernel it replaced (registers only, lane = block, 34-byte strided
// loads): Q8_0 4096 x 4096 6.4 against 8.6 us, 1024 x 4096 4.0 against 5.3,
// 14336 x 4096 14.3 against 20.4; Q4_0 14336 x 4096 10.7 us and 4096 x 14336
// 14.0 against 17.1 and 16.6 for the LDS-tiled streaming kernel.  Two items
// in flight per wavefront, two rows per item sharing the x reads and a
// contiguous eight-element lane mapping for Q4_0 were slower.
typedef __amdgpu_buffer_rsrc_t MvRsrc;
constexpr int MV_RSRC_WORD3 = 0x00020000;
constexpr uint32_t MVW_CHUNK = 8192;  // most bytes one item stages
constexpr uint32_t MVW_LDS = 160 * 1024 - 256;  // dynamic LDS; the rest for static use (__syncthreads_or)

struct WvArgs {
  const uint8_t* w;
  const float* x;
  float* y;
  uint32_t in_dim, rows, row_bytes;
  uint32_t region;  // LDS bytes per wavefront: an item's bytes + 16, rounded to 16
  uint32_t nch;     // items (chunks) per row
  uint32_t cblk;    // blocks per chunk; a multiple of the blocks per step when nch > 1
};

// x in LDS: element e at float e + 4 (e / 64), so that the 16-byte reads of
// lanes 16 or 32 floats apart fall on different banks.
__device__ __forceinline__ uint32_t wv_xi(uint32_t e) { return e + ((e >> 6) << 2); }
// LDS bytes of x; min-term formats also keep the sum of every 16 elements
// after it.
__host__ __device__ constexpr uint32_t wv_x_bytes(uint32_t in_dim, bool sums) {
  return in_dim * 4u + (in_dim / 64u) * 16u + (sums ? in_dim / 16u * 4u : 0u);
}

// x values of one lane for one block: N float4.
template <int N>
struct WvX {
  float4 v[N];
};

// x of lane p when the lane takes elements 4N p .. 4N p + 4N - 1 of the block
// whose first element is e0.
template <int N>
__device__ __forceinline__ void wv_xload(const float* xs, uint32_t e0, uint32_t p, WvX<N>& x) {
#pragma unroll
  for (int i = 0; i < N; ++i) x.v[i] = *reinterpret_cast<const float4*>(xs + wv_xi(e0 + 4u * (N * p + i)));
}

template <int N>
__device__ __forceinline__ bool wv_finite(const WvX<N>& x) {
  bool ok = true;
#pragma unroll
  for (int i = 0; i < N; ++i)
    ok = ok && fabsf(x.v[i].x) <= 3.40282347e38f && fabsf(x.v[i].y) <= 3.40282347e38f &&
         fabsf(x.v[i].z) <= 3.40282347e38f && fabsf(x.v[i].w) <= 3.40282347e38f;
  return ok;
}

template <int N>
__device__ __forceinline__ float wv_xsum(const WvX<N>& x) {
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) t += (x.v[i].x + x.v[i].y) + (x.v[i].z + x.v[i].w);
  return t;
}

// Kind of the terms w_i x_i (NaN, +inf, -inf, or 0 when all are finite).
template <int N>
__device__ __forceinline__ float wv_kinds(const float (&w)[4 * N], const WvX<N>& x) {
  bool nan = false, pinf = false, ninf = false;
#pragma unroll
  for (int i = 0; i < 4 * N; ++i) {
    const float4& q = x.v[i / 4];
    const float xv = (i & 3) == 0 ? q.x : ((i & 3) == 1 ? q.y : ((i & 3) == 2 ? q.z : q.w));
    const float t = w[i] * xv;
    nan = nan || t != t;
    pinf = pinf || t == __builtin_inff();
    ninf = ninf || t == -__builtin_inff();
  }
  if (nan || (pinf && ninf)) return __builtin_nanf("");
  return pinf ? __builtin_inff() : (ninf ? -__builtin_inff() : 0.f);
}

// sum over four signed bytes of c times x
__device__ __forceinline__ float wv_dot4s(uint32_t c, const float4& x, float t) {
  t = fmaf(rf_sb(c, 0), x.x, t); t = fmaf(rf_sb(c, 1), x.y, t);
  t = fmaf(rf_sb(c, 2), x.z, t); t = fmaf(rf_sb(c, 3), x.w, t);
  return t;
}
// sum over four unsigned bytes of n times x
__device__ __forceinline__ float wv_dot4u(uint32_t n, const float4& x, float t) {
  t = fmaf(rf_ub(n, 0), x.x, t); t = fmaf(rf_ub(n, 1), x.y, t);
  t = fmaf(rf_ub(n, 2), x.z, t); t = fmaf(rf_ub(n, 3), x.w, t);
  return t;
}

// Per format: QK elements and BS bytes per block, EPL elements per lane
// (QK / EPL lanes per block), MIN for a min term; xload, dot (and kinds for
// MIN) of lane p's share of the block at LDS byte o.
template <uint32_t T>
struct WvFmt;
template <>
struct WvFmt<T_Q8_0> {
  static constexpr uint32_t BS = 34, QK = 32, EPL = 8;
  static constexpr bool MIN = false;
  using X = WvX<2>;
  __device__ static void xload(const float* xs, uint32_t e0, uint32_t p, X& x) { wv_xload<2>(xs, e0, p, x); }
  __device__ static float dot(const uint8_t* wr, uint32_t o, const X& x, uint32_t p, float) {
    const uint32_t h = *reinterpret_cast<const uint16_t*>(wr + o);
    const uint32_t oc = o + 2u + 8u * p;  // a block starts 0 or 2 bytes into a dword
    const uint32_t* w = reinterpret_cast<const uint32_t*>(wr + (oc & ~3u));
    const uint32_t d0 = w[0], d1 = w[1], d2 = w[2], sh = oc & 3u;
    const float t = wv_dot4s(__builtin_amdgcn_alignbyte(d2, d1, sh), x.v[1],
                             wv_dot4s(__builtin_amdgcn_alignbyte(d1, d0, sh), x.v[0], 0.f));
    return rf_half_to_float_fast(h) * t;
  }
};
template <>
struct WvFmt<T_Q4_0> {
  static constexpr uint32_t BS = 18, QK = 32, EPL = 8;
  static constexpr bool MIN = false;
  using X = WvX<2>;
  // lane p: x[4p..4p+3] (low nibbles of bytes 4p..) and x[16+4p..] (high)
  __device__ static void xload(const float* xs, uint32_t e0, uint32_t p, X& x) {
    x.v[0] = *reinterpret_cast<const float4*>(xs + wv_xi(e0 + 4u * p));
    x.v[1] = *reinterpret_cast<const float4*>(xs + wv_xi(e0 + 16u + 4u * p));
  }
  __device__ static float dot(const uint8_t* wr, uint32_t o, const X& x, uint32_t p, float) {
    const uint32_t h = *reinterpret_cast<const uint16_t*>(wr + o);
    const uint32_t oc = o + 2u + 4u * p;
    const uint32_t* w = reinterpret_cast<const uint32_t*>(wr + (oc & ~3u));
    const uint32_t c = __builtin_amdgcn_alignbyte(w[1], w[0], oc & 3u);
    // (nibble - 8) moved to the top of each byte: the int8 16 (nibble - 8)
    const uint32_t lo = rf_opaque(rf_top_signed(c, 4)), hi = rf_opaque(rf_top_signed(c >> 4, 4));
    return rf_half_to_float_fast(h) * (wv_dot4s(hi, x.v[1], wv_dot4s(lo, x.v[0], 0.f)) * 0.0625f);
  }
};
// quant.rs:186-255: d @0, dmin @2, scales[12] @4, qs[128] @16; sub-block s
// uses qs[32(s/2) + l], low nibble if s even, high if odd; (d*sc)*q - dmin*m.
// Lane p: sub-block s = p / 2, elements 16(p % 2).. of it (one 16-byte read).
template <>
struct WvFmt<T_Q4_K> {
  static constexpr uint32_t BS = 144, QK = 256, EPL = 16;
  static constexpr bool MIN = true;
  using X = WvX<4>;
  __device__ static void xload(const float* xs, uint32_t e0, uint32_t p, X& x) { wv_xload<4>(xs, e0, p, x); }
  __device__ static void codes(const uint8_t* wr, uint32_t o, uint32_t p, float& d1, float& m1, uint32_t (&n)[4]) {
    const uint32_t s = p >> 1;
    const uint32_t dd = *reinterpret_cast<const uint32_t*>(wr + o);
    // get_scale_min_k4 (quant.rs:216-226) from the three scale bytes lane s
    // needs: s < 4: sc = b[s] & 63, m = b[s+4] & 63; else sc = (b[s+4] & 15) |
    // (b[s-4] >> 6) << 4, m = (b[s+4] >> 4) | (b[s] >> 6) << 4
    const bool lo4 = s < 4u;
    const uint8_t* sb = wr + o + 4u;
    const uint32_t u = sb[lo4 ? s : s + 4u], v = sb[lo4 ? s + 4u : s - 4u], w = sb[s];
    const uint32_t sc = lo4 ? (u & 63u) : ((u & 15u) | ((v >> 6) << 4));
    const uint32_t m = lo4 ? (v & 63u) : ((u >> 4) | ((w >> 6) << 4));
    d1 = rf_half_to_float_fast(dd & 0xFFFFu) * (float)sc;
    m1 = rf_half_to_float_fast(dd >> 16) * (float)m;
    const uint4 q = *reinterpret_cast<const uint4*>(wr + o + 16u + 32u * (s >> 1) + 16u * (p & 1u));
    const uint32_t sh = (s & 1u) * 4u;
    n[0] = rf_opaque((q.x >> sh) & 0x0F0F0F0Fu);
    n[1] = rf_opaque((q.y >> sh) & 0x0F0F0F0Fu);
    n[2] = rf_opaque((q.z >> sh) & 0x0F0F0F0Fu);
    n[3] = rf_opaque((q.w >> sh) & 0x0F0F0F0Fu);
  }
  // xsum: the sum of the lane's sixteen x values
  __device__ static float dot(const uint8_t* wr, uint32_t o, const X& x, uint32_t p, float xsum) {
    float d1, m1;
    uint32_t n[4];
    codes(wr, o, p, d1, m1, n);
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) t = wv_dot4u(n[i], x.v[i], t);
    return fmaf(d1, t, -m1 * xsum);
  }
  __device__ static float kinds(const uint8_t* wr, uint32_t o, const X& x, uint32_t p) {
    float d1, m1;
    uint32_t n[4];
    codes(wr, o, p, d1, m1, n);
    float w[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i] = d1 * rf_ub(n[i / 4], i & 3) - m1;
    return wv_kinds<4>(w, x);
  }
};
// quant.rs:347-407: ql[128] @0, qh[64] @128, scales i8[16] @192, d f16 @208.
// Element e = 128 hf + 32 k + l: low 4 bits from ql[64hf + 32(k&1) + l]
// (nibble k>>1), high 2 bits from qh[32hf + l] >> 2k, scale
// scales[8hf + 2k + l/16]; (d*sc)*(q-32).  Lane p: elements 8p..8p+7 (one
// l/16 group, one scale).
template <>
struct WvFmt<T_Q6_K> {
  static constexpr uint32_t BS = 210, QK = 256, EPL = 8;
  static constexpr bool MIN = false;
  using X = WvX<2>;
  __device__ static void xload(const float* xs, uint32_t e0, uint32_t p, X& x) { wv_xload<2>(xs, e0, p, x); }
  __device__ static float dot(const uint8_t* wr, uint32_t o, const X& x, uint32_t p, float) {
    const uint32_t hf = p >> 4, k = (p >> 2) & 3u, l0 = 8u * (p & 3u);
    const float d = rf_half_to_float_fast(*reinterpret_cast<const uint16_t*>(wr + o + 208u));
    const float sc = (float)*reinterpret_cast<const int8_t*>(wr + o + 192u + 8u * hf + 2u * k + (l0 >> 4));
    uint32_t ql[2], qh[2];
    rf_lds_words<2>(wr, o + 64u * hf + 32u * (k & 1u) + l0, ql);
    rf_lds_words<2>(wr, o + 128u + 32u * hf + l0, qh);
    const uint32_t nsh = (k >> 1) * 4u, hsh = 2u * k;
    // 4 (q - 32) as int8 bytes: exact products
    const uint32_t c0 =
        rf_opaque(rf_top_signed(((ql[0] >> nsh) & 0x0F0F0F0Fu) | (((qh[0] >> hsh) & 0x03030303u) << 4), 6));
    const uint32_t c1 =
        rf_opaque(rf_top_signed(((ql[1] >> nsh) & 0x0F0F0F0Fu) | (((qh[1] >> hsh) & 0x03030303u) << 4), 6));
    return d * (sc * (wv_dot4s(c1, x.v[1], wv_dot4s(c0, x.v[0], 0.f)) * 0.25f));
  }
};

// NQ 16-byte loads per lane and item (NQ * 1024 >= the item's bytes).  XR:
// rows of at most 4096 inputs (one item each) with each lane's x of all
// steps held in registers, read from LDS once per wavefront; otherwise x is
// read from LDS per step.
template <uint32_t T, int NQ, bool XR>
__global__ __launch_bounds__(512) void matvec_wave(WvArgs a) {
  using F = WvFmt<T>;
  using X = typename F::X;
  // lanes per block, blocks per step, steps of a 4096-input row
  constexpr uint32_t BS = F::BS, PL = F::QK / F::EPL, SB = 64u / PL;
  constexpr int XS = XR ? (int)(4096u / (64u * F::EPL)) : 1;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  extern __shared__ __align__(16) uint8_t mvw_sm[];
  const float* xs = reinterpret_cast<const float*>(mvw_sm);
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t nw = blockDim.x >> 6;
  float* xsum16 = reinterpret_cast<float*>(mvw_sm + wv_x_bytes(a.in_dim, false));
  uint8_t* wr = mvw_sm + wv_x_bytes(a.in_dim, F::MIN) + wave * a.region;
  const uint32_t G = gridDim.x * nw;
  const uint32_t chb = a.cblk * BS;  // bytes of a full chunk
  auto item_bytes = [&](uint32_t c) { return c + 1u < a.nch ? chb : a.row_bytes - c * chb; };
  u32x4 buf[NQ];
  auto fetch = [&](uint32_t r, uint32_t c) {
    const bool live = r < a.rows;  // wave-uniform; past the last row every load returns zeros
    const uint8_t* base = a.w + (live ? (uint64_t)r * a.row_bytes + (uint64_t)c * chb : 0u);
    const MvRsrc rs = __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, live ? (int32_t)item_bytes(c) : 0,
                                                        MV_RSRC_WORD3);
#pragma unroll
    for (int i = 0; i < NQ; ++i)  // streamed once: non-temporal
      buf[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, 16u * (lane + 64u * i), 0, 2);
  };
  // item k of this wavefront: row r0 + (k / nch) G, chunk k % nch
  uint32_t r = blockIdx.x * nw + wave, c = 0;
  fetch(r, c);
  for (uint32_t i = tid; i < a.in_dim / 4u; i += blockDim.x) {
    const float4 v = reinterpret_cast<const float4*>(a.x)[i];
    *reinterpret_cast<float4*>(mvw_sm + 4u * wv_xi(4u * i)) = v;
  }
  __syncthreads();
  int bad = 0;  // an infinity or NaN in x (min-term formats)
  if constexpr (F::MIN) {  // sums of 16 elements, and whether x is finite
    for (uint32_t g = tid; g < a.in_dim / 16u; g += blockDim.x) {
      WvX<4> v;
      wv_xload<4>(xs, 0u, g, v);
      xsum16[g] = wv_xsum(v);
      bad |= !wv_finite(v);
    }
    bad = __syncthreads_or(bad);
  }
  const uint32_t p = lane % PL, bl = lane / PL;
  X xr[XS];
  float xsr[XS];
  if constexpr (XR) {
    const uint32_t last = a.in_dim / F::QK - 1u;
#pragma unroll
    for (int k = 0; k < XS; ++k) {
      F::xload(xs, F::QK * min(SB * k + bl, last), p, xr[k]);
      if constexpr (F::MIN) xsr[k] = wv_xsum(xr[k]);
    }
  }
  // lane's share of block bk of the item
  auto term = [&](uint32_t bk, const X& x, float xsum) -> float {
    if constexpr (F::MIN) {
      if (bad && !wv_finite(x)) return F::kinds(wr, BS * bk, x, p);
    }
    return F::dot(wr, BS * bk, x, p, xsum);
  };
  float acc = 0.f;
  while (r < a.rows) {
    const uint32_t nb = item_bytes(c);
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const uint32_t o = 16u * (lane + 64u * i);
      if (o < nb) *reinterpret_cast<u32x4*>(wr + o) = buf[i];
    }
    const uint32_t rn = c + 1u < a.nch ? r : r + G, cn = c + 1u < a.nch ? c + 1u : 0u;
    fetch(rn, cn);
    const uint32_t nbk = nb / BS;
    if constexpr (XR) {
#pragma unroll
      for (int k = 0; k < XS; ++k) {
        const uint32_t bk = SB * k + bl;
        if (SB * k < nbk && bk < nbk) acc += term(bk, xr[k], F::MIN ? xsr[k] : 0.f);
      }
    } else {
      const uint32_t b0 = c * a.cblk, nfull = nbk / SB * SB;
#pragma unroll 2
      for (uint32_t j = 0; j < nfull; j += SB) {
        F::xload(xs, F::QK * (b0 + j + bl), p, xr[0]);
        acc += term(j + bl, xr[0], F::MIN ? xsum16[(F::QK * (b0 + j + bl) + F::EPL * p) / 16u] : 0.f);
      }
      const uint32_t bk = nfull + bl;
      if (nfull < nbk && bk < nbk) {
        F::xload(xs, F::QK * (b0 + bk), p, xr[0]);
        acc += term(bk, xr[0], F::MIN ? xsum16[(F::QK * (b0 + bk) + F::EPL * p) / 16u] : 0.f);
      }
    }
    if (cn == 0u) {
      const float v = rf_wave_sum(acc);
      if (lane == 0) a.y[r] = v;
      acc = 0.f;
    }
    r = rn;
    c = cn;
  }
}

// Whether the wave-staged kernel takes this launch: Q8_0 / Q4_0 / Q6_K rows
// and Q4_K rows of at most 4096 inputs, of an even block count
// (dword-aligned rows), a dword-aligned base, 16-byte aligned x, and x plus
// four wavefronts' regions within the LDS.  (Q4_K at 4096 x 14336 took 24.4
// us against 19.1 on the streaming kernel.)
static bool wave_ok(uint32_t t, uint64_t in_dim, const void* w, const float* x) {
  const uint64_t qk = t == T_Q8_0 || t == T_Q4_0 ? 32 : (t == T_Q4_K || t == T_Q6_K ? 256 : 0);
  if (qk == 0 || in_dim == 0 || in_dim % (2 * qk) != 0) return false;
  if (t == T_Q4_K && in_dim > 4096) return false;
  if ((reinterpret_cast<uintptr_t>(w) & 3u) != 0 || !aligned16(x)) return false;
  return wv_x_bytes((uint32_t)in_dim, true) + 4u * (MVW_CHUNK + 16u) <= MVW_LDS;
}

static int g_wave_enabled = 1;
void set_matvec_wave(bool on) { g_wave_enabled = on ? 1 : 0; }
bool matvec_wave_on() { return g_wave_enabled != 0; }

// Resident workgroups per CU for (kernel, threads, LDS), cached; the first
// query for a kernel also raises its dynamic LDS limit.  Both run outside
// captures only (hipErrorStreamCaptureUnsupported inside one).
template <uint32_t T, int NQ, bool XR>
static hipError_t wave_occupancy(uint32_t threads, uint32_t lds, hipStream_t st, uint32_t* occ) {
  static std::mutex mu;
  std::lock_guard<std::mutex> lock(mu);
  static uint32_t key[16] = {0}, val[16] = {0};
  static bool attr = false;
  const uint32_t k = threads << 20 | lds;
  for (int i = 0; i < 16; ++i)
    if (key[i] == k) {
      *occ = val[i];
      return hipSuccess;
    }
  hipError_t e = setup_outside_capture(st);
  if (e != hipSuccess) return e;
  if (!attr) {
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(matvec_wave<T, NQ, XR>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)MVW_LDS);
    if (e != hipSuccess) return e;
    attr = true;
  }
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, matvec_wave<T, NQ, XR>, (int)threads, (size_t)lds) !=
          hipSuccess || n < 1)
    n = 1;
  for (int i = 0; i < 16; ++i)
    if (key[i] == 0) {
      key[i] = k;
      val[i] = (uint32_t)n;
      break;
    }
  *occ = (uint32_t)n;
  return hipSuccess;
}

template <uint32_t T, int NQ, bool XR>
static hipError_t launch_wave_q(const WvArgs& a, hipStream_t st) {
  const uint32_t ncu = (uint32_t)cu_count();
  // eight wavefronts per workgroup unless there are fewer rows than that
  // per CU; whole workgroups per CU, about two rows per wavefront
  uint32_t nw = a.rows >= 8u * ncu ? 8u : 4u;
  const uint32_t xb = wv_x_bytes(a.in_dim, WvFmt<T>::MIN);
  uint32_t lds = xb + nw * a.region;
  if (lds > MVW_LDS) {
    nw = 4u;
    lds = xb + nw * a.region;
  }
  uint32_t occ = 0;
  const hipError_t e = wave_occupancy<T, NQ, XR>(64u * nw, lds, st, &occ);
  if (e != hipSuccess) return e;
  uint32_t grid;
  if ((uint64_t)a.rows <= (uint64_t)nw * ncu) {
    grid = (a.rows + nw - 1) / nw;
  } else {
    const uint64_t k = ((uint64_t)a.rows + 2ull * nw * ncu - 1) / (2ull * nw * ncu);
    grid = (uint32_t)(std::min<uint64_t>(k, occ) * ncu);
  }
  RF_KLAUNCH((matvec_wave<T, NQ, XR>), dim3(grid), dim3(64u * nw), lds, st, a);
  return hipGetLastError();
}

// x in registers pays for its per-wavefront load from about three rows per
// wavefront of an eight-wavefront workgroup per CU on (Q8_0 14336 x 4096:
// 13.3 against 15.5 us; Q4_0 4096 x 4096, two rows per wavefront: 5.8
// against 5.5 us).
constexpr uint32_t MVW_XR_ROWS_PER_WAVE = 3;

template <uint32_t T>
static hipError_t launch_wave_t(const WvArgs& a, hipStream_t st) {
  const uint32_t nq = (std::min(a.row_bytes, a.cblk * WvFmt<T>::BS) + 1023u) / 1024u;
  if (a.nch == 1 && a.in_dim <= 4096 && a.rows >= MVW_XR_ROWS_PER_WAVE * 8u * (uint32_t)cu_count()) {
    switch (nq) {
      case 1: return launch_wave_q<T, 1, true>(a, st);
      case 2: return launch_wave_q<T, 2, true>(a, st);
      case 3: return launch_wave_q<T, 3, true>(a, st);
      case 4: return launch_wave_q<T, 4, true>(a, st);
      default: return launch_wave_q<T, 5, true>(a, st);
    }
  }
  switch (nq) {
    case 1: return launch_wave_q<T, 1, false>(a, st);
    case 2: return launch_wave_q<T, 2, false>(a, st);
    case 3: return launch_wave_q<T, 3, false>(a, st);
    case 4: return launch_wave_q<T, 4, false>(a, st);
    case 5: return launch_wave_q<T, 5, false>(a, st);
    case 6: return launch_wave_q<T, 6, false>(a, st);
    default: return launch_wave_q<T, 8, false>(a, st);
  }
}

template <uint32_t T>
static hipError_t launch_wave_f(const MvSegDesc& s, const float* x, uint64_t in_dim, hipStream_t st) {
  constexpr uint32_t bs = WvFmt<T>::BS, sb = 64u / (WvFmt<T>::QK / WvFmt<T>::EPL);
  const uint32_t nblk = (uint32_t)(in_dim / WvFmt<T>::QK);
  WvArgs a{};
  a.w = static_cast<const uint8_t*>(s.w);
  a.x = x;
  a.y = s.y;
  a.in_dim = (uint32_t)in_dim;
  a.rows = (uint32_t)s.rows;
  a.row_bytes = nblk * bs;
  if (a.row_bytes <= MVW_CHUNK) {
    a.nch = 1;
    a.cblk = nblk;
  } else {  // chunks of about equal size, whole steps
    const uint32_t n = (a.row_bytes + MVW_CHUNK - 1) / MVW_CHUNK;
    a.cblk = ((nblk + n - 1) / n + sb - 1) / sb * sb;
    if (a.cblk * bs > MVW_CHUNK) a.cblk = MVW_CHUNK / bs / sb * sb;
    a.nch = (nblk + a.cblk - 1) / a.cblk;
  }
  a.region = (std::min(a.row_bytes, a.cblk * bs) + 16u + 15u) & ~15u;
  return launch_wave_t<T>(a, st);
}

static hipError_t launch_wave(uint32_t t, const MvSegDesc& s, const float* x, uint64_t in_dim, hipStream_t st) {
  switch (t) {
    case T_Q8_0: return launch_wave_f<T_Q8_0>(s, x, in_dim, st);
    case T_Q4_0: return launch_wave_f<T_Q4_0>(s, x, in_dim, st);
    case T_Q4_K: return launch_wave_f<T_Q4_K>(s, x, in_dim, st);
    case T_Q6_K: return launch_wave_f<T_Q6_K>(s, x, in_dim, st);
    default: return hipErrorInvalidValue;
  }
}

// ------------------------------------------------ F32 rows, per wavefront
// F32 weights need no decode and are naturally aligned: a wavefront owns
// rows (rows r, r + G, ... of G wavefronts) and reads each in items of up to
// NQ 256-float chunks, lane l taking floats 4l, 4l + 256, ... of the item
// with 16-byte loads straight into registers, times the same floats of x
// from LDS (zero-padded to whole items); two register sets alternate, so the
// next item's loads are in flight while the current one is summed.  Each
// lane sums its floats in order, then the wavefront sums the lanes (the
// reference's AVX2 kernel keeps 8 lanes of FMA partials, backend.rs:173-218,
// simd.rs:21-45: the same sum up to the order of the additions).
constexpr uint32_t MVF_NQ = 8;  // 256-float chunks per item

struct F32WArgs {
  const float* w;
  const float* x;
  float* y;
  uint32_t in_dim, rows, nch;  // nch = items per row
};

__global__ __launch_bounds__(512) void matvec_f32_wave(F32WArgs a) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  constexpr uint32_t ICH = MVF_NQ * 256u;  // floats per item
  extern __shared__ __align__(16) float mvf_x[];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t nw = blockDim.x >> 6, G = gridDim.x * nw;
  f32x4 buf[2][MVF_NQ];
  auto fetch = [&](f32x4 (&b)[MVF_NQ], uint32_t r, uint32_t c) {
    const bool live = r < a.rows;  // wave-uniform; past the last row every load returns zeros
    const uint32_t first = c * ICH, n = live ? min(ICH, a.in_dim - first) : 0u;
    const MvRsrc rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.w + (live ? (uint64_t)r * a.in_dim + first : 0u)), 0, (int32_t)(n * 4u), MV_RSRC_WORD3);
#pragma unroll
    for (int i = 0; i < (int)MVF_NQ; ++i)  // streamed once: non-temporal
      b[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, 16u * (lane + 64u * i), 0, 2));
  };
  uint32_t r = blockIdx.x * nw + wave, c = 0;
  fetch(buf[0], r, c);
  const uint32_t npad = a.nch * ICH;
  for (uint32_t i = tid; i < npad / 4u; i += blockDim.x)
    reinterpret_cast<float4*>(mvf_x)[i] =
        4u * i < a.in_dim ? reinterpret_cast<const float4*>(a.x)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
  __syncthreads();
  float acc = 0.f;
  auto next = [&](uint32_t& rr, uint32_t& cc) {
    if (++cc == a.nch) {
      cc = 0;
      rr += G;
    }
  };
  auto consume = [&](const f32x4 (&b)[MVF_NQ], uint32_t rr, uint32_t cc) {
#pragma unroll
    for (int i = 0; i < (int)MVF_NQ; ++i) {
      const float4 xv = *reinterpret_cast<const float4*>(mvf_x + cc * ICH + 4u * (lane + 64u * i));
      acc = fmaf(b[i].x, xv.x, acc);
      acc = fmaf(b[i].y, xv.y, acc);
      acc = fmaf(b[i].z, xv.z, acc);
      acc = fmaf(b[i].w, xv.w, acc);
    }
    if (cc + 1u == a.nch) {
      const float v = rf_wave_sum(acc);
      if (lane == 0) a.y[rr] = v;
      acc = 0.f;
    }
  };
  while (r < a.rows) {
    uint32_t r1 = r, c1 = c;
    next(r1, c1);
    fetch(buf[1], r1, c1);
    consume(buf[0], r, c);
    if (r1 >= a.rows) break;
    uint32_t r2 = r1, c2 = c1;
    next(r2, c2);
    fetch(buf[0], r2, c2);
    consume(buf[1], r1, c1);
    r = r2;
    c = c2;
  }
}

static bool f32_wave_ok(uint64_t in_dim, const void* w, const float* x) {
  if (in_dim == 0 || in_dim % 4 != 0 || in_dim > 16384) return false;
  return aligned16(w) && aligned16(x);
}

static hipError_t launch_f32_wave(const MvSegDesc& s, const float* x, uint64_t in_dim, hipStream_t st) {
  F32WArgs a{};
  a.w = static_cast<const float*>(s.w);
  a.x = x;
  a.y = s.y;
  a.in_dim = (uint32_t)in_dim;
  a.rows = (uint32_t)s.rows;
  a.nch = (uint32_t)((in_dim + MVF_NQ * 256u - 1) / (MVF_NQ * 256u));
  const uint32_t lds = a.nch * MVF_NQ * 256u * 4u;
  const uint32_t ncu = (uint32_t)cu_count();
  const uint32_t nw = a.rows >= 8u * ncu ? 8u : 4u;
  static std::mutex mu;
  static uint32_t key[8] = {0}, val[8] = {0};
  uint32_t occ = 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    const uint32_t k = nw << 20 | lds;
    for (int i = 0; i < 8 && !occ; ++i)
      if (key[i] == k) occ = val[i];
    if (!occ) {
      const hipError_t e = setup_outside_capture(st);
      if (e != hipSuccess) return e;
      int n = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, matvec_f32_wave, (int)(64u * nw), (size_t)lds) !=
              hipSuccess || n < 1)
        n = 1;
      occ = (uint32_t)n;
      for (int i = 0; i < 8; ++i)
        if (key[i] == 0) {
          key[i] = k;
          val[i] = occ;
          break;
        }
    }
  }
  uint32_t grid;
  if ((uint64_t)a.rows <= (uint64_t)nw * ncu) {
    grid = (a.rows + nw - 1) / nw;
  } else {
    const uint64_t k = ((uint64_t)a.rows + 2ull * nw * ncu - 1) / (2ull * nw * ncu);
    grid = (uint32_t)(std::min<uint64_t>(k, occ) * ncu);
  }
  RF_KLAUNCH(matvec_f32_wave, dim3(grid), dim3(64u * nw), lds, st, a);
  return hipGetLastError();
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
  if (g_wave_enabled && epi == EPI_STORE && norm_w == nullptr && nseg == 1 && segs[0].rows > 0 &&
      segs[0].rows <= 0x7FFFFFFFull) {
    if (wave_ok(t, in_dim, segs[0].w, x)) return launch_wave(t, segs[0], x, in_dim, st);
    if (t == T_F32 && f32_wave_ok(in_dim, segs[0].w, x)) return launch_f32_wave(segs[0], x, in_dim, st);
  }
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
