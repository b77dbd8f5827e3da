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
    for (uint32_t base = 0; base < n16; base += nth * UNR) {
      u32x4 r[UNR];
#pragma unroll
      for (int j = 0; j < UNR; ++j) {
        const uint32_t i = base + j * nth + tid;
        if (i < n16) r[j] = __builtin_nontemporal_load(s4 + i);
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

__device__ __forceinline__ void load_xunit(XUnit& xu, const float* __restrict__ x, uint32_t u, bool active) {
  if (!active) {
#pragma unroll
    for (int i = 0; i < 32; ++i) xu.v[i] = 0.f;
    return;
  }
  const float* p = x + 32u * u;
  if ((reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 v = reinterpret_cast<const float4*>(p)[i];
      xu.v[4 * i] = v.x; xu.v[4 * i + 1] = v.y; xu.v[4 * i + 2] = v.z; xu.v[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) xu.v[i] = p[i];
  }
}

__device__ __forceinline__ void finish_xunit(XUnit& xu) {
  float lo = 0.f, hi = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) { lo += xu.v[i]; hi += xu.v[16 + i]; }
  xu.sum_lo = lo;
  xu.sum_hi = hi;
  xu.sum = lo + hi;
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
  load_xunit(xu, a.x, u, active);

  if (a.norm_w != nullptr) {
    // RMSNorm prologue (core/src/compute.rs:291-319: x / sqrt(mean(x^2) + eps) * w).
    float ss = 0.f;
    if (active && g == 0) {
#pragma unroll
      for (int i = 0; i < 32; ++i) ss = fmaf(xu.v[i], xu.v[i], ss);
    }
    ss = rf_wave_sum(ss);
    if ((tid & 63u) == 0) wsum[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
    for (uint32_t i = 0; i < (nth >> 6); ++i) tot += wsum[i];
    const float rms = sqrtf(tot / (float)a.in_dim + a.eps);
    const float inv = 1.0f / rms;
    if (active) {
      const float* nw = a.norm_w + 32u * u;
#pragma unroll
      for (int i = 0; i < 32; ++i) xu.v[i] = xu.v[i] * inv * nw[i];
    }
  } else {
    __syncthreads();
  }
  finish_xunit(xu);

  const uint32_t blk = (u / UPB) * Fmt<T>::BS, sub = u % UPB;
  constexpr int MAXR = 8;
  float part[MAXR], part2[MAXR];
#pragma unroll
  for (int k = 0; k < MAXR; ++k) {
    part[k] = 0.f;
    part2[k] = 0.f;
    const uint32_t r = g + k * a.rg;
    if (active && r < nrows) {
      part[k] = Fmt<T>::dot(lds, r * row_bytes + blk, sub, xu);
      if (EPI == EPI_SWIGLU) part2[k] = Fmt<T>::dot(lds + a.tile_stride, r * row_bytes + blk, sub, xu);
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

static uint32_t g_tile_target = 32768;  // LDS bytes per matvec tile (tunable)
void set_matvec_tile_bytes(uint32_t bytes) { g_tile_target = bytes < 4096 ? 4096 : (bytes > 61440 ? 61440 : bytes); }
uint32_t matvec_tile_bytes() { return g_tile_target; }

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
  p.rg = units >= 256 ? 1u : (uint32_t)(256 / units);
  const uint64_t per_matrix = dual ? g_tile_target / 2 : g_tile_target;
  uint64_t rpt = per_matrix / (p.rg * rb);
  if (rpt < 1) rpt = 1;
  if (rpt > 8) rpt = 8;
  p.rows_per_tile = (uint32_t)(p.rg * rpt);
  p.threads = (uint32_t)(((units * p.rg) + 63) / 64 * 64);
  p.tile_stride = (uint32_t)((p.rows_per_tile * rb + 15) / 16 * 16);
  const uint64_t tile = (uint64_t)p.tile_stride * (dual ? 2 : 1);
  const uint64_t red = (uint64_t)p.rows_per_tile * units * 4 * (dual ? 2 : 1);
  p.lds_bytes = (uint32_t)((tile > red ? tile : red) + 16);
  return p;
}

template <uint32_t T, int EPI>
static hipError_t launch_tiled_t(const MvArgs& a, uint32_t grid, const MvPlan& p, hipStream_t st) {
  hipLaunchKernelGGL((matvec_tiled<T, EPI>), dim3(grid), dim3(p.threads), p.lds_bytes, st, a);
  return hipGetLastError();
}

template <int EPI>
static hipError_t launch_tiled_e(uint32_t t, const MvArgs& a, uint32_t grid, const MvPlan& p, hipStream_t st) {
  switch (t) {
    case T_Q8_0: return launch_tiled_t<T_Q8_0, EPI>(a, grid, p, st);
    case T_Q4_0: return launch_tiled_t<T_Q4_0, EPI>(a, grid, p, st);
    case T_Q5_0: return launch_tiled_t<T_Q5_0, EPI>(a, grid, p, st);
    case T_Q4_K: return launch_tiled_t<T_Q4_K, EPI>(a, grid, p, st);
    case T_Q5_K: return launch_tiled_t<T_Q5_K, EPI>(a, grid, p, st);
    case T_Q6_K: return launch_tiled_t<T_Q6_K, EPI>(a, grid, p, st);
    case T_Q2_K: return launch_tiled_t<T_Q2_K, EPI>(a, grid, p, st);
    case T_Q3_K: return launch_tiled_t<T_Q3_K, EPI>(a, grid, p, st);
    case T_Q8_K: return launch_tiled_t<T_Q8_K, EPI>(a, grid, p, st);
    case T_F32: return launch_tiled_t<T_F32, EPI>(a, grid, p, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_matvec_segments(uint32_t t, const MvSegDesc* segs, int nseg, const float* x,
                                  const float* norm_w, float eps, uint64_t in_dim, int epi,
                                  hipStream_t st) {
  if (nseg < 1 || nseg > 3) return hipErrorInvalidValue;
  const bool dual = epi == EPI_SWIGLU;
  MvPlan p = plan_matvec(t, in_dim, dual);
  if (!p.tiled) {
    if (norm_w != nullptr || epi != EPI_STORE) return hipErrorInvalidValue;
    for (int i = 0; i < nseg; ++i) {
      const uint32_t rows = (uint32_t)segs[i].rows;
      if (rows == 0) continue;
      dim3 grid((rows + 3) / 4);
      switch (t) {
#define RF_ROWWISE(TT) case TT: hipLaunchKernelGGL(matvec_rowwise<TT>, grid, dim3(256), 0, st, static_cast<const uint8_t*>(segs[i].w), x, segs[i].y, (uint32_t)in_dim, rows, p.row_bytes); break;
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
  MvArgs a{};
  uint32_t tiles = 0;
  for (int i = 0; i < nseg; ++i) {
    a.seg[i].w = static_cast<const uint8_t*>(segs[i].w);
    a.seg[i].y = segs[i].y;
    a.seg[i].res = segs[i].res;
    a.seg[i].rows = (uint32_t)segs[i].rows;
    a.seg[i].tile_begin = tiles;
    tiles += (uint32_t)((segs[i].rows + p.rows_per_tile - 1) / p.rows_per_tile);
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
  switch (epi) {
    case EPI_STORE: return launch_tiled_e<EPI_STORE>(t, a, tiles, p, st);
    case EPI_RESIDUAL: return launch_tiled_e<EPI_RESIDUAL>(t, a, tiles, p, st);
    case EPI_SWIGLU: return launch_tiled_e<EPI_SWIGLU>(t, a, tiles, p, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rf
