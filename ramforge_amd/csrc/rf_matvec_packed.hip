// rf_matvec_packed.hip — batch-1 matvec on the device-native ("packed")
// layout of Q8_0 and Q4_0 matrices (gfx950).
//
// Same arithmetic as quant::matvec_q8_0 / matvec_q4_0 (core/src/quant.rs:
// 913-1029): y[o] = sum over blocks of d_b * sum_i q_i x_i with the
// reference's codes and f16 scales; only the memory layout differs.
//
// Packed layout of a [rows][in] matrix (same byte count as the GGUF payload):
//   codes : rows x CRB bytes, row-major (CRB = in for Q8_0, in/2 for Q4_0;
//           Q4_0 keeps the GGUF nibble order of each block's 16 bytes)
//   scales: rows x (in/32) f16 scale bits, row-major, after all codes.
// GGUF interleaves a 2-byte scale with every 32 (Q8_0) or 16 (Q4_0) code
// bytes, so its blocks are never 16-byte aligned.  Split apart, the code
// bytes of a row are one aligned stream that a wavefront reads with 16-byte
// loads straight into registers.
//
// Work decomposition: lane l of a wavefront owns bytes [1024c + 16l, +16) of
// "chunk" c of a row (16 Q8_0 codes or 32 Q4_0 codes); one 16-byte load per
// lane moves 1 KiB per instruction.  x (times the norm weights when the
// RMSNorm prologue is fused) and the sums of its 16-element units are staged
// in LDS once per workgroup, so no register holds x between steps.  A wavefront
// owns U whole rows (every chunk), so no partial sum crosses wavefronts and
// the main loop has no barrier; a step is U rows x LPW chunks and the next
// step's codes are requested before the current one is decoded (two register
// buffers).  Row sums are DPP row reductions plus readlane.  Fusions as in
// rf_matvec.hip: RMSNorm prologue, residual or SiLU(gate)*up epilogue, up to
// three output segments.
#include "rf_kernels.h"

#include <mutex>

namespace rf {

typedef uint32_t nv_u32x4 __attribute__((ext_vector_type(4)));

// Tasks (row groups) per wavefront whose residual is staged in LDS.
constexpr uint32_t PK_RES_SLOTS = 8;
// Word 3 of a raw (untyped, stride 0) buffer resource on gfx9-family parts,
// and the cache-policy operand of a streaming (nt) load.
constexpr int PK_RSRC_WORD3 = 0x00020000;
constexpr int PK_AUX_NT = 2;
// Upper bound of the kernel's static LDS (norm partials and staged
// residuals: 16 + 16 * PK_RES_SLOTS floats at 1024 threads).
constexpr uint64_t PK_STATIC_LDS = 1024;

template <uint32_t T> struct Pk;
template <> struct Pk<T_Q8_0> {
  static constexpr uint32_t CB = 32;   // code bytes per 32 elements
  static constexpr uint32_t EPL = 16;  // elements per 16-byte lane load
};
template <> struct Pk<T_Q4_0> {
  static constexpr uint32_t CB = 16;
  static constexpr uint32_t EPL = 32;
};

// The workgroup stages x while its first step's codes are in flight.  x sits
// in LDS permuted so that the 16-byte reads of a step are consecutive across
// lanes (no bank conflicts): element 4i + k of lane l's slice of chunk c (EPL
// elements per slice) is stored at c * 64 * EPL + 256 i + 4 l + k.
// Codes and scales of one step: U rows x LPW chunks (twice with the "up" matrix).
template <int U, int LPW, bool DUAL>
struct PkStep {
  nv_u32x4 q[U][LPW], q2[DUAL ? U : 1][LPW];
  uint32_t s[U][LPW], s2[DUAL ? U : 1][LPW];
};

// NB step buffers per wavefront: NB - 1 steps are in flight while one is
// decoded.
template <uint32_t T, int EPI, bool NORM, int U, int LPW, int NB, int NT>
__global__ __launch_bounds__(NT) void matvec_packed(PkArgs a) {
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  constexpr uint32_t EPL = Pk<T>::EPL, EPB = 32u / Pk<T>::CB, NW = NT / 64;
  extern __shared__ __align__(16) float xl[];  // [nchunk * 64 * EPL] x, then [nchunk * 64 * EPL / 16] unit sums
  __shared__ float wsum[NW];
  __shared__ float resl[EPI == EPI_RESIDUAL ? NW : 1][PK_RES_SLOTS][U];
  static_assert(sizeof(wsum) + sizeof(resl) <= PK_STATIC_LDS, "static LDS above the planner's reservation");
  // The wavefront index through readfirstlane: rows, segments and their
  // pointers are then scalar values, so no vector load (whose wait would also
  // wait for the codes in flight) is spent on them.
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t in = a.in_dim, nb = in / 32u, crb = in / EPB;
  const uint32_t nchunk = (crb + 1023u) / 1024u, nstep = (nchunk + LPW - 1) / LPW;
  float* xsum_l = xl + nchunk * 64u * EPL;

  auto seg_of = [&](uint32_t v) -> PkSeg {
    return (a.nseg > 2 && v >= a.seg[2].row_begin) ? a.seg[2]
                                                   : ((a.nseg > 1 && v >= a.seg[1].row_begin) ? a.seg[1] : a.seg[0]);
  };

  const uint32_t ntask = (a.rows_total + U - 1) / U;
  const uint32_t gstride = gridDim.x * NW;

  typedef PkStep<U, LPW, DUAL> Step;
  Step buf[NB];
  // Codes and scales through raw buffer loads: one resource per row (scalar
  // base, range = the row's bytes), the lane's byte offset in a VGPR.  Offsets
  // past the row (the tail of a partial chunk) and every load of a fetch past
  // the last task (range 0) return zeros without touching memory, so fetches
  // are issued unconditionally and the compiler's wait counts stay exact: a
  // consume waits for its own step only, never for the prefetch behind it.
  auto fetch = [&](Step& B, uint32_t t, uint32_t st) {
    const bool live = t < ntask;  // wave-uniform
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t v = min(t * U + u, a.rows_total - 1u);
      const PkSeg g = seg_of(v);
      const uint32_t r = v - g.row_begin;
      const int32_t nc = live ? (int32_t)crb : 0, ns2 = live ? (int32_t)(nb * 2u) : 0;
      const auto rc = __builtin_amdgcn_make_buffer_rsrc((void*)(g.codes + (size_t)r * crb), 0, nc, PK_RSRC_WORD3);
      const auto rs = __builtin_amdgcn_make_buffer_rsrc((void*)(g.scales + (size_t)r * nb), 0, ns2, PK_RSRC_WORD3);
      __amdgpu_buffer_rsrc_t rc2, rs2;
      if constexpr (DUAL) {
        rc2 = __builtin_amdgcn_make_buffer_rsrc((void*)(g.codes_up + (size_t)r * crb), 0, nc, PK_RSRC_WORD3);
        rs2 = __builtin_amdgcn_make_buffer_rsrc((void*)(g.scales_up + (size_t)r * nb), 0, ns2, PK_RSRC_WORD3);
      }
#pragma unroll
      for (int l = 0; l < LPW; ++l) {
        const uint32_t b = (st * LPW + l) * 1024u + 16u * lane, sb = (b * EPB / 32u) * 2u;
        B.q[u][l] = __builtin_amdgcn_raw_buffer_load_b128(rc, b, 0, PK_AUX_NT);
        B.s[u][l] = __builtin_amdgcn_raw_buffer_load_b16(rs, sb, 0, 0);
        if constexpr (DUAL) {
          B.q2[u][l] = __builtin_amdgcn_raw_buffer_load_b128(rc2, b, 0, PK_AUX_NT);
          B.s2[u][l] = __builtin_amdgcn_raw_buffer_load_b16(rs2, sb, 0, 0);
        }
      }
    }
  };

  auto advance = [&](uint32_t& tt, uint32_t& ss) {
    if (++ss == nstep) { ss = 0; tt += gstride; }
  };
  // The first NB - 1 steps are requested before the prologue.
  uint32_t ct = blockIdx.x * NW + wave, cs = 0, ft = ct, fs = 0;
#pragma unroll
  for (int b = 0; b < NB - 1; ++b) {
    fetch(buf[b], ft, fs);
    advance(ft, fs);
  }

  // Prologue, one round of loads and one barrier.  Thread j (then j + NT, ...)
  // owns unit j: 16 consecutive elements, one lane slice of a Q8_0 chunk or
  // half of a Q4_0 one.  It writes the unit into LDS and the unit's sum.
  // With NORM, rms_norm_reference (core/src/compute.rs:291-319) is
  // x / sqrt(mean(x^2) + eps) * w; LDS holds x * w and every row sum is
  // scaled by 1 / sqrt(mean(x^2) + eps) in the epilogue (the same value up to
  // rounding), so the mean's reduction shares the prologue's barrier.
  constexpr uint32_t UPS = EPL / 16u;  // units per lane slice
  const uint32_t nunit = nchunk * 64u * UPS;
  {
    const float4* x4 = reinterpret_cast<const float4*>(a.x);
    const float4* w4 = reinterpret_cast<const float4*>(a.norm_w);
    float ss = 0.f;
    for (uint32_t j = tid; j < nunit; j += NT) {
      const uint32_t js = j / UPS, h = j % UPS;
      const uint32_t e = ((js >> 6) * 1024u + 16u * (js & 63u)) * EPB + 16u * h;
      float s = 0.f;
      if (e < in) {
        float4 v[4], w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          v[k] = x4[e / 4u + k];
          if (NORM) w[k] = w4[e / 4u + k];
        }
        float* dst = xl + (js >> 6) * 64u * EPL + 4u * h * 256u + 4u * (js & 63u);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if (NORM) {
            ss = fmaf(v[k].x, v[k].x, ss); ss = fmaf(v[k].y, v[k].y, ss);
            ss = fmaf(v[k].z, v[k].z, ss); ss = fmaf(v[k].w, v[k].w, ss);
            v[k].x *= w[k].x; v[k].y *= w[k].y; v[k].z *= w[k].z; v[k].w *= w[k].w;
          }
          *reinterpret_cast<float4*>(dst + 256 * k) = v[k];
          s += v[k].x; s += v[k].y; s += v[k].z; s += v[k].w;
        }
      }
      xsum_l[j] = s;
    }
    if (NORM) {
      ss = rf_wave_sum(ss);
      if (lane == 0) wsum[wave] = ss;
    }
    // EPI_RESIDUAL: the residual of every row this wavefront will finish
    // (at most PK_RES_SLOTS tasks; the launch sizes the grid for that), so
    // the epilogue reads LDS instead of waiting on a load queued behind codes.
    if constexpr (EPI == EPI_RESIDUAL) {
      for (uint32_t k = 0; k < PK_RES_SLOTS; ++k) {
        const uint32_t t = ct + k * gstride;
        if (t >= ntask) break;
        if (lane < (uint32_t)U) {
          const uint32_t vr = t * U + lane;
          float r = 0.f;
          if (vr < a.rows_total) {
            const PkSeg g = seg_of(vr);
            r = g.res[vr - g.row_begin];
          }
          resl[wave][k][lane] = r;
        }
      }
    }
  }
  __syncthreads();
  float inv = 1.f;
  if (NORM) {
    float tot = 0.f;
#pragma unroll
    for (uint32_t i = 0; i < NW; ++i) tot += wsum[i];
    inv = 1.0f / sqrtf(tot / (float)in + a.eps);
  }

  float acc[U], acc2[U];
#pragma unroll
  for (int u = 0; u < U; ++u) { acc[u] = 0.f; acc2[u] = 0.f; }
  uint32_t done = 0;  // tasks this wavefront has finished

  auto consume = [&](const Step& B, uint32_t tt, uint32_t ss) {
#pragma unroll
    for (int l = 0; l < LPW; ++l) {
      // Lanes past the end of the row (a partial last chunk, or a chunk past
      // nchunk when LPW does not divide it) decode zeros against a clamped,
      // in-bounds slice of x and keep their sums by a select.
      const uint32_t c = ss * LPW + l, cx = c < nchunk ? c : nchunk - 1u;
      const bool valid = c * 1024u + 16u * lane < crb;
      const float* xp = xl + cx * 64u * EPL + 4u * lane;
      float s[U], s2[U];
#pragma unroll
      for (int u = 0; u < U; ++u) { s[u] = 0.f; s2[u] = 0.f; }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (T == T_Q8_0) {
          const float4 xv = *reinterpret_cast<const float4*>(xp + 256 * i);
          const float xe[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const uint32_t w = B.q[u][l][i] ^ 0x80808080u;  // q + 128 as unsigned bytes
#pragma unroll
            for (int k = 0; k < 4; ++k) s[u] = fmaf(rf_ub(w, k), xe[k], s[u]);
            if constexpr (DUAL) {
              const uint32_t w2 = B.q2[u][l][i] ^ 0x80808080u;
#pragma unroll
              for (int k = 0; k < 4; ++k) s2[u] = fmaf(rf_ub(w2, k), xe[k], s2[u]);
            }
          }
        } else {
          // byte j: low nibble -> element j, high nibble -> element j + 16 (quant.rs:84-113)
          const float4 xv = *reinterpret_cast<const float4*>(xp + 256 * i);
          const float4 xw = *reinterpret_cast<const float4*>(xp + 256 * (i + 4));
          const float xe[4] = {xv.x, xv.y, xv.z, xv.w}, xh[4] = {xw.x, xw.y, xw.z, xw.w};
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const uint32_t lo = rf_opaque(B.q[u][l][i] & 0x0F0F0F0Fu), hi = rf_opaque((B.q[u][l][i] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              s[u] = fmaf(rf_ub(lo, k), xe[k], s[u]);
              s[u] = fmaf(rf_ub(hi, k), xh[k], s[u]);
            }
            if constexpr (DUAL) {
              const uint32_t lo2 = rf_opaque(B.q2[u][l][i] & 0x0F0F0F0Fu),
                             hi2 = rf_opaque((B.q2[u][l][i] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
              for (int k = 0; k < 4; ++k) {
                s2[u] = fmaf(rf_ub(lo2, k), xe[k], s2[u]);
                s2[u] = fmaf(rf_ub(hi2, k), xh[k], s2[u]);
              }
            }
          }
        }
      }
      const float xs = UPS == 1 ? xsum_l[cx * 64u + lane]
                                : xsum_l[(cx * 64u + lane) * 2u] + xsum_l[(cx * 64u + lane) * 2u + 1u];
      constexpr float bias = T == T_Q8_0 ? -128.f : -8.f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float t = fmaf(rf_half_to_float_fast(B.s[u][l]), fmaf(bias, xs, s[u]), acc[u]);
        acc[u] = valid ? t : acc[u];
        if constexpr (DUAL) {
          const float t2 = fmaf(rf_half_to_float_fast(B.s2[u][l]), fmaf(bias, xs, s2[u]), acc2[u]);
          acc2[u] = valid ? t2 : acc2[u];
        }
      }
    }
    if (ss + 1u == nstep) {  // the task's rows are complete
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float v = rf_wave_sum(acc[u]) * inv;
        const float v2 = DUAL ? rf_wave_sum(acc2[u]) * inv : 0.f;
        acc[u] = 0.f;
        acc2[u] = 0.f;
        const uint32_t vr = tt * U + u;  // wave-uniform
        if (lane == (uint32_t)u && vr < a.rows_total) {
          const PkSeg g = seg_of(vr);
          const uint32_t o = vr - g.row_begin;
          if (EPI == EPI_STORE) {
            g.y[o] = v;
          } else if (EPI == EPI_RESIDUAL) {
            // add_reference (compute.rs:321-327); the launch keeps done < PK_RES_SLOTS
            g.y[o] = (done < PK_RES_SLOTS ? resl[wave][done][u] : g.res[o]) + v;
          } else {
            g.y[o] = v / (1.0f + expf(-v)) * v2;  // silu_reference * up (compute.rs:337-350)
          }
        }
      }
      ++done;
    }
  };
  // Buffer b holds step k with k % NB == b: the step NB - 1 ahead goes into
  // the buffer freed by the previous step.
  // The only exit is the uniform check at the top of each step, so every
  // buffer is consumed (its loads waited for) before it is refilled.
  for (;;) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (ct >= ntask) return;
      fetch(buf[(b + NB - 1) % NB], ft, fs);
      advance(ft, fs);
      consume(buf[b], ct, cs);
      advance(ct, cs);
    }
  }
}

// GGUF blocks -> packed layout, one thread per block (install-time only).
template <uint32_t T>
__global__ __launch_bounds__(256) void pack_blocks(const uint8_t* __restrict__ raw, uint8_t* __restrict__ packed,
                                                   uint64_t rows, uint32_t nb) {
  constexpr uint32_t BS = Fmt<T>::BS, CB = Pk<T>::CB;
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * nb) return;
  const uint8_t* b = raw + i * BS;
  uint16_t* scales = reinterpret_cast<uint16_t*>(packed + rows * nb * CB);
  scales[i] = (uint16_t)rf_ld_u16(b);
  uint8_t* codes = packed + i * CB;  // row r, block j -> r * nb * CB + j * CB == i * CB
#pragma unroll
  for (uint32_t k = 0; k < CB; ++k) codes[k] = b[2 + k];
}

// ------------------------------------------------------------------ host side

bool packed_type(uint32_t t) { return t == T_Q8_0 || t == T_Q4_0; }

static uint32_t pk_lds_limit() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 65536;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || n < 65536)
      n = 65536;
    cached[dev] = n;
  }
  return (uint32_t)cached[dev];
}

static uint64_t pk_nchunk(uint32_t t, uint64_t in_dim) {
  const uint64_t crb = in_dim * (t == T_Q8_0 ? 32u : 16u) / 32u;
  return (crb + 1023) / 1024;
}

PkPlan plan_packed(uint32_t t, uint64_t in_dim) {
  PkPlan p{};
  if (!packed_type(t) || in_dim == 0 || in_dim % 32 != 0 || in_dim > (1u << 24)) return p;
  const uint64_t nchunk = pk_nchunk(t, in_dim), epl = t == T_Q8_0 ? 16 : 32;
  const uint64_t lds = (nchunk * 64 * epl + nchunk * 64 * (epl / 16)) * 4;
  if (lds + PK_STATIC_LDS > pk_lds_limit()) return p;
  p.ok = true;
  p.lds_bytes = (uint32_t)lds;
  return p;
}

static int pk_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Resident workgroups per CU of one kernel at one LDS size; the caller keeps
// one cache per kernel (a few distinct sizes per model).
struct PkOccCache {
  std::mutex mu;
  uint32_t keys[16];
  int vals[16];
  int n = 0;
  uint32_t attr = 0;  // dynamic LDS the kernel has been opened up to (above 64 KiB)
};
static int pk_occupancy(PkOccCache& c, const void* kern, int nt, uint32_t lds) {
  std::lock_guard<std::mutex> lock(c.mu);
  for (int i = 0; i < c.n; ++i)
    if (c.keys[i] == lds) return c.vals[i];
  if (lds > 65536 && lds > c.attr) {
    if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) return 0;
    c.attr = lds;
  }
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, nt, lds) != hipSuccess || occ < 1) occ = 1;
  if (c.n < 16) {
    c.keys[c.n] = lds;
    c.vals[c.n] = occ;
    ++c.n;
  }
  return occ;
}

template <uint32_t T, int EPI, bool NORM, int LPW, int NB, int NT>
static hipError_t launch_pk(const PkArgs& a, uint32_t lds, hipStream_t st) {
  constexpr int U = 1;
  static PkOccCache cache;
  auto kern = matvec_packed<T, EPI, NORM, U, LPW, NB, NT>;
  const int occ = pk_occupancy(cache, reinterpret_cast<const void*>(kern), NT, lds);
  if (occ < 1) return hipErrorInvalidConfiguration;
  const uint64_t tasks = (a.rows_total + U - 1) / U, nw = NT / 64;
  const uint64_t want = (tasks + nw - 1) / nw, cap = (uint64_t)pk_cu_count() * occ;
  uint64_t grid = want < cap ? want : cap;
  if (EPI == EPI_RESIDUAL) {  // at most PK_RES_SLOTS tasks per wavefront (residuals staged in LDS)
    const uint64_t need = (tasks + nw * PK_RES_SLOTS - 1) / (nw * PK_RES_SLOTS);
    if (grid < need) grid = need;
  }
  hipLaunchKernelGGL(kern, dim3((uint32_t)grid), dim3(NT), lds, st, a);
  return hipGetLastError();
}

// Launch shape, from timing the 8B projections (Q8_0 and Q4_0; 4096 and
// 14336 inputs): one row per wavefront; LPW = chunks per step, up to 4 (2 for
// gate/up, whose step loads two matrices); 1024-thread workgroups when x fills
// more than 40 KB of LDS (two resident workgroups then still give 32
// wavefronts per CU), else 512.
template <uint32_t T, int EPI, bool NORM>
static hipError_t launch_pk_l(const PkArgs& a, uint32_t lds, hipStream_t st) {
  const uint64_t nchunk = pk_nchunk(T, a.in_dim);
  const uint32_t pref = EPI == EPI_SWIGLU ? 2 : 4;
  uint32_t lpw = 1;
  while (lpw * 2 <= pref && lpw * 2 <= nchunk) lpw *= 2;
  const bool big = lds > 40960;
  switch (lpw * 2 + (big ? 1 : 0)) {
    case 2: return launch_pk<T, EPI, NORM, 1, 2, 512>(a, lds, st);
    case 3: return launch_pk<T, EPI, NORM, 1, 2, 1024>(a, lds, st);
    case 4: return launch_pk<T, EPI, NORM, 2, 2, 512>(a, lds, st);
    case 5: return launch_pk<T, EPI, NORM, 2, 2, 1024>(a, lds, st);
    case 8: return launch_pk<T, EPI, NORM, 4, 2, 512>(a, lds, st);
    case 9: return launch_pk<T, EPI, NORM, 4, 2, 1024>(a, lds, st);
    default: return hipErrorInvalidValue;
  }
}

template <uint32_t T>
static hipError_t launch_pk_t(const PkArgs& a, uint32_t lds, int epi, bool norm, hipStream_t st) {
  switch (epi * 2 + (norm ? 1 : 0)) {
    case EPI_STORE * 2: return launch_pk_l<T, EPI_STORE, false>(a, lds, st);
    case EPI_STORE * 2 + 1: return launch_pk_l<T, EPI_STORE, true>(a, lds, st);
    case EPI_RESIDUAL * 2: return launch_pk_l<T, EPI_RESIDUAL, false>(a, lds, st);
    case EPI_RESIDUAL * 2 + 1: return launch_pk_l<T, EPI_RESIDUAL, true>(a, lds, st);
    case EPI_SWIGLU * 2: return launch_pk_l<T, EPI_SWIGLU, false>(a, lds, st);
    case EPI_SWIGLU * 2 + 1: return launch_pk_l<T, EPI_SWIGLU, true>(a, lds, st);
    default: return hipErrorInvalidValue;
  }
}

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

hipError_t launch_matvec_packed(uint32_t t, const PkSegDesc* segs, int nseg, const float* x, const float* norm_w,
                                float eps, uint64_t in_dim, int epi, hipStream_t st) {
  const PkPlan p = plan_packed(t, in_dim);
  if (!p.ok || nseg < 1 || nseg > 3) return hipErrorInvalidValue;
  if (!al16(x) || (norm_w && !al16(norm_w))) return hipErrorInvalidValue;
  const bool dual = epi == EPI_SWIGLU;
  const uint64_t cb = t == T_Q8_0 ? 32 : 16, crb = in_dim * cb / 32, nb = in_dim / 32;
  PkArgs a{};
  uint64_t total = 0;
  for (int i = 0; i < nseg; ++i) {
    const PkSegDesc& d = segs[i];
    if (d.row_start + d.rows > d.matrix_rows) return hipErrorInvalidValue;
    const uint8_t* base = static_cast<const uint8_t*>(d.packed);
    a.seg[i].codes = base + d.row_start * crb;
    a.seg[i].scales = reinterpret_cast<const uint16_t*>(base + d.matrix_rows * crb) + d.row_start * nb;
    if (dual) {
      const uint8_t* up = static_cast<const uint8_t*>(d.packed_up);
      if (!up) return hipErrorInvalidValue;
      a.seg[i].codes_up = up + d.row_start * crb;
      a.seg[i].scales_up = reinterpret_cast<const uint16_t*>(up + d.matrix_rows * crb) + d.row_start * nb;
    }
    if (!al16(a.seg[i].codes) || (dual && !al16(a.seg[i].codes_up))) return hipErrorInvalidValue;
    a.seg[i].y = d.y;
    a.seg[i].res = d.res;
    a.seg[i].row_begin = (uint32_t)total;
    total += d.rows;
  }
  if (total == 0) return hipSuccess;
  if (total > 0xFFFFFFFFull) return hipErrorInvalidValue;
  a.nseg = (uint32_t)nseg;
  a.rows_total = (uint32_t)total;
  a.x = x;
  a.norm_w = norm_w;
  a.eps = eps;
  a.in_dim = (uint32_t)in_dim;
  switch (t) {
    case T_Q8_0: return launch_pk_t<T_Q8_0>(a, p.lds_bytes, epi, norm_w != nullptr, st);
    case T_Q4_0: return launch_pk_t<T_Q4_0>(a, p.lds_bytes, epi, norm_w != nullptr, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_pack(uint32_t t, const void* raw, void* packed, uint64_t rows, uint64_t in_dim, hipStream_t st) {
  if (!packed_type(t) || in_dim % 32 != 0) return hipErrorInvalidValue;
  const uint64_t nb = in_dim / 32, n = rows * nb;
  if (n == 0) return hipSuccess;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (t == T_Q8_0)
    hipLaunchKernelGGL(pack_blocks<T_Q8_0>, grid, dim3(256), 0, st, static_cast<const uint8_t*>(raw),
                       static_cast<uint8_t*>(packed), rows, (uint32_t)nb);
  else
    hipLaunchKernelGGL(pack_blocks<T_Q4_0>, grid, dim3(256), 0, st, static_cast<const uint8_t*>(raw),
                       static_cast<uint8_t*>(packed), rows, (uint32_t)nb);
  return hipGetLastError();
}

}  // namespace rf
