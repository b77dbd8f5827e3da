// rf_elementwise.hip — decode-step glue kernels, bit-exact dequant and the
// seeded synthetic payload generator.
//
// RMSNorm, add, mul, SiLU, SwiGLU, softmax: core/src/compute.rs:291-384.
// RoPE: core/src/compute.rs:389-456 (cos/sin built on the host with the same
// f32 expression and libm, so the device only does the rotation).
// Greedy argmax: runtime/src/sampling.rs:45-57 (first maximum wins).
// Row decode: core/src/quant.rs:615-868, tensor.rs:801-866.
#include "rf_kernels.h"

namespace rf {

// ---------------------------------------------------------------- RMSNorm
// Single workgroup; the sum of squares is a tree reduction (the reference sums
// sequentially), the normalisation keeps the reference's x / rms * w order.
__global__ __launch_bounds__(1024) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                       uint32_t n, float eps, float* __restrict__ y) {
  __shared__ float part[16];
  const uint32_t tid = threadIdx.x;
  float ss = 0.f;
  for (uint32_t i = tid; i < n; i += blockDim.x) ss = fmaf(x[i], x[i], ss);
  ss = rf_wave_sum(ss);
  if ((tid & 63u) == 0) part[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
  for (uint32_t i = 0; i < (blockDim.x >> 6); ++i) tot += part[i];
  const float rms = sqrtf(tot / (float)n + eps);
  for (uint32_t i = tid; i < n; i += blockDim.x) y[i] = x[i] / rms * w[i];
}

hipError_t launch_rmsnorm(const float* x, const float* w, uint64_t n, float eps, float* y, hipStream_t st) {
  RF_KLAUNCH(rmsnorm_kernel, dim3(1), dim3(1024), 0, st, x, w, (uint32_t)n, eps, y);
  return hipGetLastError();
}

// ---------------------------------------------------------------- binary ops
__global__ void binary_kernel(int op, const float* __restrict__ a, const float* __restrict__ b, uint64_t n,
                              float* __restrict__ out) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float av = a[i], bv = b[i];
  if (op == BIN_ADD) out[i] = av + bv;
  else if (op == BIN_MUL) out[i] = av * bv;
  else out[i] = av / (1.0f + expf(-av)) * bv;  // swiglu_reference (compute.rs:354-361)
}

hipError_t launch_binary(int op, const float* a, const float* b, uint64_t n, float* out, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const uint32_t gb = grid_blocks(n, 256);
  if (!gb) return hipErrorInvalidValue;
  RF_KLAUNCH(binary_kernel, dim3(gb), dim3(256), 0, st, op, a, b, n, out);
  return hipGetLastError();
}

__global__ void silu_kernel(const float* __restrict__ x, uint64_t n, float* __restrict__ y) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  y[i] = v / (1.0f + expf(-v));
}

hipError_t launch_silu(const float* x, uint64_t n, float* y, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const uint32_t gb = grid_blocks(n, 256);
  if (!gb) return hipErrorInvalidValue;
  RF_KLAUNCH(silu_kernel, dim3(gb), dim3(256), 0, st, x, n, y);
  return hipGetLastError();
}

__global__ void bias_add_kernel(float* __restrict__ v, const float* __restrict__ b, uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) v[i] += b[i];
}

hipError_t launch_bias_add(float* v, const float* b, uint64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const uint32_t gb = grid_blocks(n, 256);
  if (!gb) return hipErrorInvalidValue;
  RF_KLAUNCH(bias_add_kernel, dim3(gb), dim3(256), 0, st, v, b, n);
  return hipGetLastError();
}

// ---------------------------------------------------------------- softmax
__global__ __launch_bounds__(1024) void softmax_kernel(float* __restrict__ v, uint32_t n) {
  __shared__ float part[16];
  __shared__ float bc;
  const uint32_t tid = threadIdx.x, nw = blockDim.x >> 6;
  float m = -INFINITY;
  for (uint32_t i = tid; i < n; i += blockDim.x) m = fmaxf(m, v[i]);
  m = rf_wave_max(m);
  if ((tid & 63u) == 0) part[tid >> 6] = m;
  __syncthreads();
  if (tid == 0) {
    float mm = -INFINITY;
    for (uint32_t i = 0; i < nw; ++i) mm = fmaxf(mm, part[i]);
    bc = mm;
  }
  __syncthreads();
  m = bc;
  float s = 0.f;
  for (uint32_t i = tid; i < n; i += blockDim.x) {
    const float e = expf(v[i] - m);
    v[i] = e;
    s += e;
  }
  s = rf_wave_sum(s);
  __syncthreads();
  if ((tid & 63u) == 0) part[tid >> 6] = s;
  __syncthreads();
  if (tid == 0) {
    float t = 0.f;
    for (uint32_t i = 0; i < nw; ++i) t += part[i];
    bc = t;
  }
  __syncthreads();
  s = bc;
  for (uint32_t i = tid; i < n; i += blockDim.x) v[i] = v[i] / s;
}

hipError_t launch_softmax(float* v, uint64_t n, hipStream_t st) {
  RF_KLAUNCH(softmax_kernel, dim3(1), dim3(1024), 0, st, v, (uint32_t)n);
  return hipGetLastError();
}

// ---------------------------------------------------------------- RoPE
// cs = [hd/2][2] cos/sin for the position; q [qh][hd], k [kvh][hd] in place.
__global__ void rope_kernel(float* __restrict__ q, float* __restrict__ k, RopeCS t, uint32_t hd, uint32_t qh,
                            uint32_t kvh) {
  const uint32_t half = hd >> 1;
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;  // pair index over all heads
  const uint32_t nq = qh * half, nk = kvh * half;
  if (i >= nq + nk) return;
  float* v = i < nq ? q : k;
  const uint32_t j = i < nq ? i : i - nq;
  const uint32_t head = j / half, p = j % half;
  float* hv = v + (size_t)head * hd;
  const float c = t.cs[2 * p], s = t.cs[2 * p + 1];
  const float a = hv[p], b = hv[p + half];
  hv[p] = a * c - b * s;
  hv[p + half] = a * s + b * c;
}

hipError_t launch_rope_pair(float* q, float* k, const RopeCS& cs, uint32_t hd, uint32_t qh, uint32_t kvh,
                            hipStream_t st) {
  const uint32_t n = (qh + kvh) * (hd / 2);
  if (n == 0) return hipSuccess;
  RF_KLAUNCH(rope_kernel, dim3((n + 255) / 256), dim3(256), 0, st, q, k, cs, hd, qh, kvh);
  return hipGetLastError();
}

// ---------------------------------------------------------------- argmax
// Two stages.  Candidate (v, i) beats (bv, bi) iff v > bv or (v == bv and
// i < bi); NaN never wins.  That selects the lowest index holding the maximum
// of the non-NaN values, which is what the reference's strict `>` scan from
// logits[0] returns whenever logits[0] is not NaN; a NaN logits[0] makes the
// reference return 0, handled explicitly in the final stage.
__device__ __forceinline__ void amax_merge(float& bv, uint32_t& bi, float v, uint32_t i) {
  if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

__global__ __launch_bounds__(256) void argmax_stage1(const float* __restrict__ x, uint64_t n,
                                                     float* __restrict__ pv, uint32_t* __restrict__ pi) {
  float bv = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
    amax_merge(bv, bi, x[i], (uint32_t)i);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const uint32_t oi = __shfl_xor(bi, o, 64);
    amax_merge(bv, bi, ov, oi);
  }
  __shared__ float sv[4];
  __shared__ uint32_t si[4];
  if ((threadIdx.x & 63u) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) amax_merge(bv, bi, sv[w], si[w]);
    pv[blockIdx.x] = bv;
    pi[blockIdx.x] = bi;
  }
}

__global__ __launch_bounds__(64) void argmax_stage2(const float* __restrict__ x, const float* __restrict__ pv,
                                                    const uint32_t* __restrict__ pi, uint32_t np,
                                                    uint32_t* __restrict__ out, uint32_t* __restrict__ ring,
                                                    const int32_t* __restrict__ d_pos) {
  float bv = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
  for (uint32_t i = threadIdx.x; i < np; i += 64u) amax_merge(bv, bi, pv[i], pi[i]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const uint32_t oi = __shfl_xor(bi, o, 64);
    amax_merge(bv, bi, ov, oi);
  }
  if (threadIdx.x == 0) {
    const uint32_t r = (isnan(x[0]) || bi == 0xFFFFFFFFu) ? 0u : bi;
    *out = r;
    if (ring) ring[*d_pos] = r;
  }
}

// argmax_stage2 for the device decode loop, with the embedding row of the
// chosen token decoded into `hidden` by the same workgroup (the reference
// reads the row for the sampled token, persistent.rs:80-205): 256 threads, a
// 32-element unit (or element, for F32 / F16 / BF16 tables) each at a time.
template <uint32_t T>
__global__ __launch_bounds__(256) void argmax_embed_kernel(const float* __restrict__ x, const float* __restrict__ pv,
                                                           const uint32_t* __restrict__ pi, uint32_t np,
                                                           uint32_t* __restrict__ out, uint32_t* __restrict__ ring,
                                                           const int32_t* __restrict__ d_pos,
                                                           const uint8_t* __restrict__ embd, uint32_t in_dim,
                                                           uint64_t row_bytes, float* __restrict__ hidden) {
  __shared__ float sv[4];
  __shared__ uint32_t si[4];
  __shared__ uint32_t tok;
  const uint32_t tid = threadIdx.x;
  float bv = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
  for (uint32_t i = tid; i < np; i += 256u) amax_merge(bv, bi, pv[i], pi[i]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const uint32_t oi = __shfl_xor(bi, o, 64);
    amax_merge(bv, bi, ov, oi);
  }
  if ((tid & 63u) == 0) { sv[tid >> 6] = bv; si[tid >> 6] = bi; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w) amax_merge(bv, bi, sv[w], si[w]);
    const uint32_t r = (isnan(x[0]) || bi == 0xFFFFFFFFu) ? 0u : bi;
    *out = r;
    if (ring) ring[*d_pos] = r;
    tok = r;
  }
  __syncthreads();
  const uint8_t* row = embd + (uint64_t)tok * row_bytes;  // tok < n, the table's rows
  if constexpr (T == T_F32 || T == T_F16 || T == T_BF16) {
    for (uint32_t c = tid; c < in_dim; c += 256u) {
      if (T == T_F32) {
        float f;
        __builtin_memcpy(&f, row + 4u * c, 4);
        hidden[c] = f;
      } else {
        const uint32_t h = rf_ld_u16(row + 2u * c);
        hidden[c] = T == T_F16 ? rf_half_to_float(h) : rf_bf16_to_float(h);
      }
    }
  } else {
    constexpr uint32_t UPB = Fmt<T>::QK / 32u;
    for (uint32_t u = tid; u < in_dim / 32u; u += 256u) {
      float vals[32];
      Fmt<T>::dequant(row, (u / UPB) * Fmt<T>::BS, u % UPB, vals);
#pragma unroll
      for (int i = 0; i < 32; ++i) hidden[32u * u + i] = vals[i];
    }
  }
}

uint32_t argmax_partials(uint64_t n) {
  uint64_t b = (n + 1023) / 1024;
  if (b < 1) b = 1;
  if (b > 256) b = 256;
  return (uint32_t)b;
}

hipError_t launch_argmax(const float* logits, uint64_t n, uint32_t* out, float* ws_val, uint32_t* ws_idx,
                         uint32_t* ring, const int32_t* d_pos, hipStream_t st) {
  const uint32_t np = argmax_partials(n);
  RF_KLAUNCH(argmax_stage1, dim3(np), dim3(256), 0, st, logits, n, ws_val, ws_idx);
  RF_KLAUNCH(argmax_stage2, dim3(1), dim3(64), 0, st, logits, ws_val, ws_idx, np, out, ring, d_pos);
  return hipGetLastError();
}

hipError_t launch_argmax_embed(const float* logits, uint64_t n, uint32_t* out, float* ws_val, uint32_t* ws_idx,
                               uint32_t* ring, const int32_t* d_pos, uint32_t et, const void* embd, uint64_t in_dim,
                               float* hidden, hipStream_t st) {
  if (n == 0 || in_dim == 0 || in_dim > 0xFFFFFFFFull) return hipErrorInvalidValue;
  uint64_t qk = 1, bs = 4;
  if (et == T_F16 || et == T_BF16) bs = 2;
  else if (et != T_F32 && !type_geometry(et, &qk, &bs)) return hipErrorInvalidValue;
  if (in_dim % qk != 0 || (et != T_F32 && et != T_F16 && et != T_BF16 && in_dim % 32 != 0)) return hipErrorInvalidValue;
  const uint64_t row_bytes = in_dim / qk * bs;
  const uint32_t np = argmax_partials(n);
  RF_KLAUNCH(argmax_stage1, dim3(np), dim3(256), 0, st, logits, n, ws_val, ws_idx);
  const uint8_t* e = static_cast<const uint8_t*>(embd);
  const uint32_t d = (uint32_t)in_dim;
  switch (et) {
#define RF_AE(TT)                                                                                                   \
  case TT:                                                                                                          \
    RF_KLAUNCH(argmax_embed_kernel<TT>, dim3(1), dim3(256), 0, st, logits, ws_val, ws_idx, np, out, ring,  \
                       d_pos, e, d, row_bytes, hidden);                                                           \
    break;
    RF_AE(T_F32) RF_AE(T_F16) RF_AE(T_BF16) RF_AE(T_Q4_0) RF_AE(T_Q5_0) RF_AE(T_Q8_0) RF_AE(T_Q2_K) RF_AE(T_Q3_K)
    RF_AE(T_Q4_K) RF_AE(T_Q5_K) RF_AE(T_Q6_K) RF_AE(T_Q8_K)
#undef RF_AE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------- dequant rows
template <uint32_t T>
__global__ void dequant_kernel(const uint8_t* __restrict__ w, uint32_t in_dim, uint64_t rows, uint64_t row_bytes,
                               float* __restrict__ out, const uint32_t* __restrict__ token, uint64_t token_rows) {
  constexpr uint32_t UPB = Fmt<T>::QK / 32u;
  const uint32_t units = in_dim / 32u;
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= rows * units) return;
  const uint64_t r = t / units;
  const uint32_t u = (uint32_t)(t % units);
  uint64_t src_row = r;
  if (token) {
    src_row = token[r];
    if (src_row >= token_rows) src_row = 0;  // the host validated ids it knows; a device id is clamped
  }
  const uint8_t* row = w + src_row * row_bytes;
  float vals[32];
  Fmt<T>::dequant(row, (u / UPB) * Fmt<T>::BS, u % UPB, vals);
  float* o = out + r * in_dim + 32u * u;
#pragma unroll
  for (int i = 0; i < 32; ++i) o[i] = vals[i];
}

// F32 / F16 / BF16 rows (tensor.rs:801-866): element-wise.
__global__ void decode_plain_kernel(uint32_t t, const uint8_t* __restrict__ w, uint64_t in_dim, uint64_t rows,
                                    float* __restrict__ out, const uint32_t* __restrict__ token, uint64_t token_rows) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * in_dim) return;
  const uint64_t r = i / in_dim, c = i % in_dim;
  uint64_t src_row = r;
  if (token) {
    src_row = token[r];
    if (src_row >= token_rows) src_row = 0;
  }
  const uint64_t e = src_row * in_dim + c;
  if (t == T_F32) {
    float f;
    __builtin_memcpy(&f, w + 4 * e, 4);
    out[i] = f;
  } else {
    const uint32_t h = rf_ld_u16(w + 2 * e);
    out[i] = t == T_F16 ? rf_half_to_float(h) : rf_bf16_to_float(h);
  }
}

hipError_t launch_dequant_rows(uint32_t t, const void* wv, uint64_t in_dim, uint64_t rows, float* out,
                               const uint32_t* token_index, uint64_t token_rows, hipStream_t st) {
  const uint8_t* w = static_cast<const uint8_t*>(wv);
  if (rows == 0 || in_dim == 0) return hipSuccess;
  if (t == T_F32 || t == T_F16 || t == T_BF16) {
    const uint64_t n = rows * in_dim;
    const uint32_t gb = n / rows == in_dim ? grid_blocks(n, 256) : 0u;
    if (!gb) return hipErrorInvalidValue;
    RF_KLAUNCH(decode_plain_kernel, dim3(gb), dim3(256), 0, st, t, w, in_dim, rows,
                       out, token_index, token_rows);
    return hipGetLastError();
  }
  uint64_t qk = 0, bs = 0;
  if (!type_geometry(t, &qk, &bs)) return hipErrorInvalidValue;
  const uint64_t row_bytes = in_dim / qk * bs;
  const uint64_t n = rows * (in_dim / 32);
  const uint32_t gb = n / rows == in_dim / 32 ? grid_blocks(n, 256) : 0u;
  if (!gb || in_dim > 0xFFFFFFFFull) return hipErrorInvalidValue;
  const dim3 grid(gb), blk(256);
  switch (t) {
#define RF_DQ(TT) case TT: RF_KLAUNCH(dequant_kernel<TT>, grid, blk, 0, st, w, (uint32_t)in_dim, rows, row_bytes, out, token_index, token_rows); break;
    RF_DQ(T_Q4_0) RF_DQ(T_Q5_0) RF_DQ(T_Q8_0) RF_DQ(T_Q2_K) RF_DQ(T_Q3_K) RF_DQ(T_Q4_K) RF_DQ(T_Q5_K)
    RF_DQ(T_Q6_K) RF_DQ(T_Q8_K)
#undef RF_DQ
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------- position
__global__ void advance_pos_kernel(int32_t* p) { *p += 1; }

hipError_t launch_advance_pos(int32_t* d_pos, hipStream_t st) {
  RF_KLAUNCH(advance_pos_kernel, dim3(1), dim3(1), 0, st, d_pos);
  return hipGetLastError();
}

__global__ void set_u32_kernel(uint32_t* p, uint32_t v) { *p = v; }
__global__ void set_i32_kernel(int32_t* p, int32_t v) { *p = v; }
__global__ void fill_kernel(float* p, float v, uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

hipError_t launch_set_u32(uint32_t* p, uint32_t v, hipStream_t st) {
  RF_KLAUNCH(set_u32_kernel, dim3(1), dim3(1), 0, st, p, v);
  return hipGetLastError();
}

hipError_t launch_set_i32(int32_t* p, int32_t v, hipStream_t st) {
  RF_KLAUNCH(set_i32_kernel, dim3(1), dim3(1), 0, st, p, v);
  return hipGetLastError();
}

hipError_t launch_fill(float* p, float v, uint64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const uint32_t gb = grid_blocks(n, 256);
  if (!gb) return hipErrorInvalidValue;
  RF_KLAUNCH(fill_kernel, dim3(gb), dim3(256), 0, st, p, v, n);
  return hipGetLastError();
}

// ---------------------------------------------------------------- synthetic payloads
// Counter-based generator: word i of stream s is SplitMix64 output i.  Normal
// deviates are Irwin-Hall(12) sums, exact in binary64, and the f16 rounding is
// integer-only, so host and device produce identical bytes.
__device__ __forceinline__ uint64_t synth_u64(uint64_t seed, uint64_t index) {
  uint64_t z = seed + (index + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ double synth_normal(uint64_t s, uint64_t j) {
  uint64_t acc = 0;
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    const uint64_t r = synth_u64(s, 6 * j + (uint64_t)k);
    acc += (r & 0xFFFFFFFFull) + (r >> 32);
  }
  return __dmul_rn((double)acc, 1.0 / 4294967296.0) - 6.0;
}

__device__ __forceinline__ uint32_t f32_to_f16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 16) & 0x8000u, exp = (u >> 23) & 0xFFu;
  uint32_t mant = u & 0x7FFFFFu;
  if (exp == 0xFFu) return sign | 0x7C00u | (mant ? 0x200u : 0u);
  const int e = (int)exp - 127 + 15;
  if (e >= 31) return sign | 0x7C00u;
  if (e <= 0) {
    if (e < -10) return sign;
    mant |= 0x800000u;
    const int shift = 14 - e;
    uint32_t hm = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (hm & 1u))) hm++;
    return sign | hm;
  }
  uint32_t h = sign | ((uint32_t)e << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return h;
}

__device__ __forceinline__ uint32_t synth_scale(uint64_t s, uint64_t j, double mul) {
  return f32_to_f16_rne((float)__dmul_rn(fabs(synth_normal(s, j)), mul));
}

// K-quant min scale: the block's d as the reference decodes it, times the
// format's mean code r, encoded so that it decodes to that value again (an
// f16 subnormal decodes at half its IEEE value, so it is encoded doubled).
// Weights d sc q - dmin m of uniform codes and scales are then zero-mean.
__device__ __forceinline__ uint32_t synth_min(uint32_t dbits, float r) {
  const float v = rf_half_to_float(dbits) * r;
  uint32_t h = f32_to_f16_rne(v);
  if ((h & 0x7C00u) == 0 && (h & 0x3FFu) != 0) {
    const uint32_t h2 = f32_to_f16_rne(2.0f * v);
    if ((h2 & 0x7C00u) == 0) h = h2;
    // between the largest decoded subnormal (1023 2^-25) and the smallest
    // normal (2^-14) nothing decodes: the nearer of the two
    else h = (v - 1023.0f * 0x1p-25f < 0x1p-14f - v) ? 0x03FFu : 0x0400u;
  }
  return h;
}

__device__ __forceinline__ void put16(uint8_t* p, uint32_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

__device__ __forceinline__ void synth_fill(uint64_t s, uint64_t wpb, uint64_t b, uint8_t* out, uint32_t n) {
  for (uint32_t i = 0; i < n; i += 8) {
    const uint64_t r = synth_u64(s, wpb * b + i / 8);
    for (uint32_t k = 0; k < 8 && i + k < n; ++k) out[i + k] = (uint8_t)(r >> (8 * k));
  }
}

__global__ void synth_kernel(uint32_t t, uint64_t ss, uint64_t sc, uint64_t first, uint64_t nblk, double mul,
                             uint8_t* __restrict__ out, uint32_t bs) {
  const uint64_t k = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= nblk) return;
  const uint64_t b = first + k;
  uint8_t* p = out + k * bs;
  switch (t) {
    case T_F32: {
      const float v = (float)__dmul_rn(synth_normal(ss, b), mul);
      __builtin_memcpy(p, &v, 4);
      break;
    }
    case T_Q8_0: {
      put16(p, synth_scale(ss, b, mul));
      for (int j = 0; j < 32; ++j) {
        const uint64_t r = synth_u64(sc, 8 * b + (uint64_t)(j / 4));
        const uint32_t c16 = (uint32_t)((r >> (16 * (j % 4))) & 0xFFFFu);
        p[2 + j] = (uint8_t)(int8_t)((int)((c16 * 255u) >> 16) - 127);
      }
      break;
    }
    case T_Q4_0: put16(p, synth_scale(ss, b, mul)); synth_fill(sc, 2, b, p + 2, 16); break;
    case T_Q5_0: put16(p, synth_scale(ss, b, mul)); synth_fill(sc, 3, b, p + 2, 20); break;
    case T_Q4_K: {
      const uint32_t d = synth_scale(ss, 2 * b, mul);
      put16(p, d);
      put16(p + 2, synth_min(d, 7.5f));
      synth_fill(sc, 18, b, p + 4, 140);
      break;
    }
    case T_Q5_K: {
      const uint32_t d = synth_scale(ss, 2 * b, mul);
      put16(p, d);
      put16(p + 2, synth_min(d, 15.5f));
      synth_fill(sc, 22, b, p + 4, 172);
      break;
    }
    case T_Q6_K:
      synth_fill(sc, 26, b, p, 208);
      put16(p + 208, synth_scale(ss, 2 * b, mul));
      break;
    case T_Q2_K:
      synth_fill(sc, 10, b, p, 80);
      {
        const uint32_t d = synth_scale(ss, 2 * b, mul);
        put16(p + 80, d);
        put16(p + 82, synth_min(d, 1.5f));
      }
      break;
    case T_Q3_K:
      synth_fill(sc, 14, b, p, 108);
      put16(p + 108, synth_scale(ss, 2 * b, mul));
      break;
    case T_Q8_K: {
      const float d = (float)__dmul_rn(fabs(synth_normal(ss, 2 * b)), mul);
      __builtin_memcpy(p, &d, 4);
      synth_fill(sc, 32, b, p + 4, 256);
      for (int g = 0; g < 16; ++g) {
        int s = 0;
        for (int i = 0; i < 16; ++i) s += (int8_t)p[4 + 16 * g + i];
        put16(p + 260 + 2 * g, (uint32_t)(uint16_t)(int16_t)s);
      }
      break;
    }
    default: break;
  }
}

static uint64_t host_synth_u64(uint64_t seed, uint64_t index) {
  uint64_t z = seed + (index + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

hipError_t launch_synth(uint32_t t, uint64_t seed, uint64_t first, uint64_t nblk, double mul, void* dst,
                        hipStream_t st) {
  uint64_t qk = 0, bs = 0;
  if (!type_geometry(t, &qk, &bs)) return hipErrorInvalidValue;
  if (nblk == 0) return hipSuccess;
  const uint64_t ss = host_synth_u64(seed ^ 0xA5A5A5A5A5A5A5A5ull, 0);
  const uint64_t sc = host_synth_u64(seed ^ 0x3C3C3C3C3C3C3C3Cull, 0);
  const uint32_t gb = grid_blocks(nblk, 256);
  if (!gb) return hipErrorInvalidValue;
  RF_KLAUNCH(synth_kernel, dim3(gb), dim3(256), 0, st, t, ss, sc, first, nblk,
                     mul, static_cast<uint8_t*>(dst), (uint32_t)bs);
  return hipGetLastError();
}

// Loads this file's code object on the current device (HIP defers that to a
// kernel's first use, which may otherwise fall inside a stream capture).
hipError_t load_module_elementwise() {
  hipFuncAttributes fa;
  return hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(set_u32_kernel));
}

}  // namespace rf
