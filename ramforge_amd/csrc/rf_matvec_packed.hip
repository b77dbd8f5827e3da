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
// loads straight into registers (1 KiB per load instruction): no LDS staging,
// no barrier in the main loop.
//
// Work decomposition: lane l of a wavefront owns bytes [1024c + 16l, +16) of
// "chunk" c of every row (16 Q8_0 codes or 32 Q4_0 codes = one block) and
// keeps the matching x elements in registers.  A wavefront covers LPW chunks;
// `kw` wavefronts cover a row (kw in {1, 2, 4}); a 256-thread workgroup holds
// 4/kw row groups.  Each row group takes U rows per step; the next step's
// codes are requested before the current step is decoded (two register
// buffers).  Row sums are DPP row reductions plus readlane; with kw > 1 the
// wavefront partials meet in LDS.  Fusions as in rf_matvec.hip: RMSNorm
// prologue, residual or SiLU(gate)*up epilogue, up to three output segments.
#include "rf_kernels.h"

#include <mutex>

namespace rf {

typedef uint32_t nv_u32x4 __attribute__((ext_vector_type(4)));

template <uint32_t T> struct Pk;
template <> struct Pk<T_Q8_0> {
  static constexpr uint32_t CB = 32;   // code bytes per 32 elements
  static constexpr uint32_t EPL = 16;  // elements per 16-byte lane load
  __device__ static float dot(const nv_u32x4& q, const float* x, float xsum) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t b = q[i] ^ 0x80808080u;  // q + 128 as unsigned bytes
#pragma unroll
      for (int k = 0; k < 4; ++k) s = fmaf(rf_ub(b, k), x[4 * i + k], s);
    }
    return fmaf(-128.f, xsum, s);
  }
};
template <> struct Pk<T_Q4_0> {
  static constexpr uint32_t CB = 16;
  static constexpr uint32_t EPL = 32;
  // byte j: low nibble -> element j, high nibble -> element j + 16 (quant.rs:84-113)
  __device__ static float dot(const nv_u32x4& q, const float* x, float xsum) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = rf_opaque(q[i] & 0x0F0F0F0Fu), hi = rf_opaque((q[i] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        s = fmaf(rf_ub(lo, k), x[4 * i + k], s);
        s = fmaf(rf_ub(hi, k), x[16 + 4 * i + k], s);
      }
    }
    return fmaf(-8.f, xsum, s);
  }
};

template <uint32_t T, int EPI, bool NORM, int LPW, int U>
__global__ __launch_bounds__(256) void matvec_packed(PkArgs a) {
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  constexpr uint32_t EPL = Pk<T>::EPL;
  __shared__ float part[2][4][2 * U];
  __shared__ float ssq[4];
  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
  const uint32_t kw = a.kw, kwi = w % kw, rgi = w / kw, nrg = 4u / kw;
  const uint32_t in = a.in_dim, nb = in / 32u;

  // This lane's code bytes and x elements in each of its LPW chunks.
  uint32_t boff[LPW], eoff[LPW];
  bool ok[LPW];
#pragma unroll
  for (int l = 0; l < LPW; ++l) {
    const uint32_t b = (kwi * LPW + l) * 1024u + 16u * lane;
    const uint32_t e = b * (32u / Pk<T>::CB);
    ok[l] = e < in;
    eoff[l] = ok[l] ? e : in - EPL;  // clamped: every load stays in bounds
    boff[l] = eoff[l] / (32u / Pk<T>::CB);
  }

  // Row v of all segments -> its segment, chosen with selects (a dynamic
  // index into the kernel-argument array would be copied to scratch).
  auto seg_of = [&](uint32_t v) -> PkSeg {
    return (a.nseg > 2 && v >= a.seg[2].row_begin) ? a.seg[2]
                                                   : ((a.nseg > 1 && v >= a.seg[1].row_begin) ? a.seg[1] : a.seg[0]);
  };
  const uint32_t crb = in * Pk<T>::CB / 32u;

  nv_u32x4 qa[U][LPW], qb[U][LPW], q2a[U][LPW], q2b[U][LPW];
  uint32_t sa[U][LPW], sb[U][LPW], s2a[U][LPW], s2b[U][LPW];
  auto fetch = [&](nv_u32x4 (&q)[U][LPW], uint32_t (&sc)[U][LPW], nv_u32x4 (&q2)[U][LPW],
                   uint32_t (&sc2)[U][LPW], uint32_t v0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t v = min(v0 + u, a.rows_total - 1u);
      const PkSeg g = seg_of(v);
      const uint32_t r = v - g.row_begin;
#pragma unroll
      for (int l = 0; l < LPW; ++l) {
        q[u][l] = __builtin_nontemporal_load(reinterpret_cast<const nv_u32x4*>(g.codes + (size_t)r * crb + boff[l]));
        sc[u][l] = g.scales[(size_t)r * nb + eoff[l] / 32u];
        if (DUAL) {
          q2[u][l] = __builtin_nontemporal_load(
              reinterpret_cast<const nv_u32x4*>(g.codes_up + (size_t)r * crb + boff[l]));
          sc2[u][l] = g.scales_up[(size_t)r * nb + eoff[l] / 32u];
        }
      }
    }
  };

  // Loop over workgroup batches of nrg * U rows: every wavefront of the
  // workgroup runs the same number of iterations (barriers below).
  const uint32_t step = gridDim.x * nrg * U;
  uint32_t wb = blockIdx.x * nrg * U;
  const uint32_t off = rgi * U;
  if (wb < a.rows_total) fetch(qa, sa, q2a, s2a, wb + off);  // weights first, then x

  float xs[LPW][EPL], xsum[LPW];
#pragma unroll
  for (int l = 0; l < LPW; ++l) {
    const float4* xp = reinterpret_cast<const float4*>(a.x + eoff[l]);
#pragma unroll
    for (int i = 0; i < (int)EPL / 4; ++i) {
      const float4 v = xp[i];
      xs[l][4 * i] = v.x; xs[l][4 * i + 1] = v.y; xs[l][4 * i + 2] = v.z; xs[l][4 * i + 3] = v.w;
    }
  }
  if (NORM) {
    // rms_norm_reference (core/src/compute.rs:291-319): x / sqrt(mean(x^2) + eps) * w
    float nwr[LPW][EPL];
#pragma unroll
    for (int l = 0; l < LPW; ++l) {
      const float4* np = reinterpret_cast<const float4*>(a.norm_w + eoff[l]);
#pragma unroll
      for (int i = 0; i < (int)EPL / 4; ++i) {
        const float4 v = np[i];
        nwr[l][4 * i] = v.x; nwr[l][4 * i + 1] = v.y; nwr[l][4 * i + 2] = v.z; nwr[l][4 * i + 3] = v.w;
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int l = 0; l < LPW; ++l)
      if (ok[l])
#pragma unroll
        for (int i = 0; i < (int)EPL; ++i) ss = fmaf(xs[l][i], xs[l][i], ss);
    ss = rf_wave_sum(ss);
    if (kw > 1) {
      if (lane == 0) ssq[w] = ss;
      __syncthreads();
      ss = 0.f;
      for (uint32_t k = 0; k < kw; ++k) ss += ssq[rgi * kw + k];
    }
    const float inv = 1.0f / sqrtf(ss / (float)in + a.eps);
#pragma unroll
    for (int l = 0; l < LPW; ++l)
#pragma unroll
      for (int i = 0; i < (int)EPL; ++i) xs[l][i] = xs[l][i] * inv * nwr[l][i];
  }
#pragma unroll
  for (int l = 0; l < LPW; ++l) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < (int)EPL; ++i) s += xs[l][i];
    xsum[l] = s;
  }

  int buf = 0;
  auto consume = [&](const nv_u32x4 (&q)[U][LPW], const uint32_t (&sc)[U][LPW], const nv_u32x4 (&q2)[U][LPW],
                     const uint32_t (&sc2)[U][LPW], uint32_t v0) {
    float v[U], v2[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float acc = 0.f, acc2 = 0.f;
#pragma unroll
      for (int l = 0; l < LPW; ++l) {
        if (!ok[l]) continue;
        acc = fmaf(rf_half_to_float(sc[u][l]), Pk<T>::dot(q[u][l], xs[l], xsum[l]), acc);
        if (DUAL) acc2 = fmaf(rf_half_to_float(sc2[u][l]), Pk<T>::dot(q2[u][l], xs[l], xsum[l]), acc2);
      }
      v[u] = rf_wave_sum(acc);
      v2[u] = DUAL ? rf_wave_sum(acc2) : 0.f;
    }
    if (kw > 1) {
      if (lane == 0)
#pragma unroll
        for (int u = 0; u < U; ++u) {
          part[buf][w][u] = v[u];
          if (DUAL) part[buf][w][U + u] = v2[u];
        }
      __syncthreads();
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float t = 0.f, t2 = 0.f;
        for (uint32_t k = 0; k < kw; ++k) {
          t += part[buf][rgi * kw + k][u];
          if (DUAL) t2 += part[buf][rgi * kw + k][U + u];
        }
        v[u] = t;
        v2[u] = t2;
      }
      buf ^= 1;  // the other buffer is written next step: no second barrier
    }
    if (kwi == 0 && lane < (uint32_t)U) {
      float mine = 0.f, mine2 = 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (lane == (uint32_t)u) { mine = v[u]; mine2 = v2[u]; }
      const uint32_t vr = v0 + lane;
      if (vr < a.rows_total) {
        const PkSeg g = seg_of(vr);
        const uint32_t o = vr - g.row_begin;
        if (EPI == EPI_STORE) {
          g.y[o] = mine;
        } else if (EPI == EPI_RESIDUAL) {
          g.y[o] = g.res[o] + mine;  // add_reference (compute.rs:321-327)
        } else {
          g.y[o] = mine / (1.0f + expf(-mine)) * mine2;  // silu_reference * up (compute.rs:337-350)
        }
      }
    }
  };
  while (wb < a.rows_total) {
    const uint32_t w1 = wb + step;
    if (w1 < a.rows_total) fetch(qb, sb, q2b, s2b, w1 + off);
    consume(qa, sa, q2a, s2a, wb + off);
    if (w1 >= a.rows_total) break;
    const uint32_t w2 = w1 + step;
    if (w2 < a.rows_total) fetch(qa, sa, q2a, s2a, w2 + off);
    consume(qb, sb, q2b, s2b, w1 + off);
    wb = w2;
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

PkPlan plan_packed(uint32_t t, uint64_t in_dim) {
  PkPlan p{};
  if (!packed_type(t) || in_dim == 0 || in_dim % 32 != 0 || in_dim > (1u << 24)) return p;
  const uint32_t cb = t == T_Q8_0 ? 32u : 16u;
  const uint64_t crb = in_dim * cb / 32;
  const uint32_t nchunk = (uint32_t)((crb + 1023) / 1024);
  uint32_t lpw, kw;
  if (nchunk <= 1) { lpw = 1; kw = 1; }
  else if (nchunk <= 2) { lpw = 2; kw = 1; }
  else if (nchunk <= 8) { lpw = 2; kw = (nchunk + 1) / 2; }
  else { lpw = 4; kw = (nchunk + 3) / 4; }
  if (t == T_Q4_0 && lpw == 4) { lpw = 2; kw = (nchunk + 1) / 2; }  // 32 x floats per chunk: keep 64
  if (kw == 3) kw = 4;
  if (kw > 4) return p;
  p.ok = true;
  p.lpw = lpw;
  p.kw = kw;
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

template <uint32_t T, int EPI, bool NORM, int LPW, int U>
static hipError_t launch_pk(const PkArgs& a, hipStream_t st) {
  static std::mutex mu;
  static int occ_cache = 0;
  int occ;
  {
    std::lock_guard<std::mutex> lock(mu);
    if (!occ_cache) {
      int n = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, matvec_packed<T, EPI, NORM, LPW, U>, 256, 0) !=
              hipSuccess || n < 1)
        n = 1;
      occ_cache = n;
    }
    occ = occ_cache;
  }
  const uint32_t nrg = 4u / a.kw;
  const uint64_t batches = (a.rows_total + (uint64_t)nrg * U - 1) / ((uint64_t)nrg * U);
  const uint64_t cap = (uint64_t)pk_cu_count() * occ;
  const uint32_t grid = (uint32_t)(batches < cap ? batches : cap);
  hipLaunchKernelGGL((matvec_packed<T, EPI, NORM, LPW, U>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

// Rows per step U against chunks per lane LPW: two register buffers of
// U x LPW x (16 B codes, twice for gate/up) plus LPW x EPL x floats stay
// within about 190 VGPRs (chosen by timing the 8B projections: the spread
// between the candidates was within 15%).
template <uint32_t T, int EPI, int LPW>
constexpr int pk_rows_per_step() {
  constexpr bool dual = EPI == EPI_SWIGLU;
  if (LPW >= 4) return dual ? 1 : 2;
  if (LPW == 2) return (T == T_Q4_0 && dual) ? 1 : 2;
  return dual ? 2 : 4;
}

template <uint32_t T, int EPI, bool NORM>
static hipError_t launch_pk_l(const PkArgs& a, uint32_t lpw, hipStream_t st) {
  switch (lpw) {
    case 1: return launch_pk<T, EPI, NORM, 1, pk_rows_per_step<T, EPI, 1>()>(a, st);
    case 2: return launch_pk<T, EPI, NORM, 2, pk_rows_per_step<T, EPI, 2>()>(a, st);
    case 4:
      if constexpr (T == T_Q8_0) return launch_pk<T, EPI, NORM, 4, pk_rows_per_step<T, EPI, 4>()>(a, st);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

template <uint32_t T>
static hipError_t launch_pk_t(const PkArgs& a, uint32_t lpw, int epi, bool norm, hipStream_t st) {
  switch (epi * 2 + (norm ? 1 : 0)) {
    case EPI_STORE * 2: return launch_pk_l<T, EPI_STORE, false>(a, lpw, st);
    case EPI_STORE * 2 + 1: return launch_pk_l<T, EPI_STORE, true>(a, lpw, st);
    case EPI_RESIDUAL * 2: return launch_pk_l<T, EPI_RESIDUAL, false>(a, lpw, st);
    case EPI_RESIDUAL * 2 + 1: return launch_pk_l<T, EPI_RESIDUAL, true>(a, lpw, st);
    case EPI_SWIGLU * 2: return launch_pk_l<T, EPI_SWIGLU, false>(a, lpw, st);
    case EPI_SWIGLU * 2 + 1: return launch_pk_l<T, EPI_SWIGLU, true>(a, lpw, st);
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
  a.kw = p.kw;
  switch (t) {
    case T_Q8_0: return launch_pk_t<T_Q8_0>(a, p.lpw, epi, norm_w != nullptr, st);
    case T_Q4_0: return launch_pk_t<T_Q4_0>(a, p.lpw, epi, norm_w != nullptr, st);
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
