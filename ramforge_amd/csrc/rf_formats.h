// rf_formats.h — GGUF block formats on gfx950.
//
// Two views of every executable format (support.rs:266-282):
//   * dequant_unit: the bit-exact decode of 32 consecutive elements, written
//     with the reference's own operation order (core/src/quant.rs:84-612) so
//     the floats are identical to BlockXxx::dequantize.
//   * dot_unit: the dequant-dot used by the matvec kernels.  It returns the
//     contribution of one 32-element unit to y[row] = sum_i W[row,i] x[i] as
//     sum_i q_i x_i times the sub-block scale: the signed codes (times an
//     exact power of two) are converted to float, so every product q_i x_i
//     is exact up to its own rounding and a zero code adds nothing, as the
//     reference's (q * d) * x does.  The K-quants with a min (Q4_K, Q5_K,
//     Q2_K) subtract dmin * m * sum(x) of the sub-block, the format's own
//     offset.  Only the association and summation order differ from
//     sum (q*d)*x_i.
//
// A "unit" is 32 consecutive elements of a row.  In every format unit u of a
// row covers x[32u, 32u+32): Q4_0/Q5_0/Q8_0 blocks are one unit, the 256-
// element K-quant super-blocks are eight units each.  `blk` is the byte
// offset of the unit's block inside the buffer `b` (LDS for the matvec, any
// 4-byte-aligned buffer with 4 readable bytes of slack for rf_lds_*).
#pragma once

#include "rf_device.h"

namespace rf {

enum : uint32_t {
  T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q5_0 = 6, T_Q8_0 = 8, T_Q2_K = 10, T_Q3_K = 11,
  T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_Q8_K = 15, T_BF16 = 30
};

// x registers of one unit: v[32] plus partial sums the formats need.
struct XUnit {
  float v[32];
  float sum;      // sum of all 32
  float sum_lo;   // sum of v[0..16)
  float sum_hi;   // sum of v[16..32)
};

template <uint32_t T> struct Fmt;

// ---------------------------------------------------------------- Q8_0 (34 B)
// quant.rs:155-182: d f16 @0, qs i8[32] @2; value = q * d.
template <> struct Fmt<T_Q8_0> {
  static constexpr uint32_t QK = 32, BS = 34;
  __device__ static float dot(const uint8_t* b, uint32_t blk, uint32_t /*sub*/, const XUnit& x) {
    const float d = rf_half_to_float(rf_lds_u32(b, blk) & 0xFFFFu);
    uint32_t w[8];
    rf_lds_words<8>(b, blk + 2, w);
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) acc = fmaf(rf_sb(w[i], k), x.v[4 * i + k], acc);
    return d * acc;
  }
  __device__ static void dequant(const uint8_t* b, uint32_t blk, uint32_t, float* out) {
    const float d = rf_half_to_float(rf_ld_u16(b + blk));
    for (int i = 0; i < 32; ++i) out[i] = (float)(int8_t)b[blk + 2 + i] * d;
  }
};

// ---------------------------------------------------------------- Q4_0 (18 B)
// quant.rs:84-113: d f16 @0, qs[16] @2; elem j = lo(qs[j]) - 8, elem 16+j = hi(qs[j]) - 8.
template <> struct Fmt<T_Q4_0> {
  static constexpr uint32_t QK = 32, BS = 18;
  __device__ static float dot(const uint8_t* b, uint32_t blk, uint32_t, const XUnit& x) {
    const float d = rf_half_to_float(rf_lds_u32(b, blk) & 0xFFFFu);
    uint32_t w[4];
    rf_lds_words<4>(b, blk + 2, w);
    float acc = 0.f;  // 16 (nibble - 8) as int8 bytes: exact products
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = rf_opaque(rf_top_signed(w[i], 4)), hi = rf_opaque(rf_top_signed(w[i] >> 4, 4));
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc = fmaf(rf_sb(lo, k), x.v[4 * i + k], acc);
        acc = fmaf(rf_sb(hi, k), x.v[16 + 4 * i + k], acc);
      }
    }
    return d * (acc * 0.0625f);
  }
  __device__ static void dequant(const uint8_t* b, uint32_t blk, uint32_t, float* out) {
    const float d = rf_half_to_float(rf_ld_u16(b + blk));
    for (int j = 0; j < 16; ++j) {
      const uint32_t byte = b[blk + 2 + j];
      out[j] = (float)((int)(byte & 0x0Fu) - 8) * d;
      out[16 + j] = (float)((int)(byte >> 4) - 8) * d;
    }
  }
};

// ---------------------------------------------------------------- Q5_0 (22 B)
// quant.rs:117-151: d @0, qh u32 @2, qs[16] @6; elem e gets bit e of qh as bit 4.
template <> struct Fmt<T_Q5_0> {
  static constexpr uint32_t QK = 32, BS = 22;
  __device__ static float dot(const uint8_t* b, uint32_t blk, uint32_t, const XUnit& x) {
    const float d = rf_half_to_float(rf_lds_u32(b, blk) & 0xFFFFu);
    const uint32_t qh = rf_lds_u32(b, blk + 2);
    uint32_t w[4];
    rf_lds_words<4>(b, blk + 6, w);
    float acc = 0.f;  // 8 (q - 16) as int8 bytes: exact products
    // bit k of a nibble to bit 4 of byte k (k * 7 + k = 8 k, then << 4)
    auto spread = [](uint32_t nib) { return ((nib * 0x00204081u) & 0x01010101u) << 4; };
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = (w[i] & 0x0F0F0F0Fu) | spread((qh >> (4 * i)) & 0xFu);
      const uint32_t hi = ((w[i] >> 4) & 0x0F0F0F0Fu) | spread((qh >> (4 * i + 16)) & 0xFu);
      const uint32_t sl = rf_opaque(rf_top_signed(lo, 5)), sh = rf_opaque(rf_top_signed(hi, 5));
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc = fmaf(rf_sb(sl, k), x.v[4 * i + k], acc);
        acc = fmaf(rf_sb(sh, k), x.v[16 + 4 * i + k], acc);
      }
    }
    return d * (acc * 0.125f);
  }
  __device__ static void dequant(const uint8_t* b, uint32_t blk, uint32_t, float* out) {
    const float d = rf_half_to_float(rf_ld_u16(b + blk));
    const uint32_t qh = rf_ld_u16(b + blk + 2) | (rf_ld_u16(b + blk + 4) << 16);
    for (int j = 0; j < 16; ++j) {
      const uint32_t byte = b[blk + 6 + j];
      const uint32_t xh0 = ((qh >> j) << 4) & 0x10u;
      const uint32_t xh1 = (qh >> (j + 12)) & 0x10u;
      out[j] = (float)((int)((byte & 0x0Fu) | xh0) - 16) * d;
      out[16 + j] = (float)((int)((byte >> 4) | xh1) - 16) * d;
    }
  }
};

// get_scale_min of Q4_K / Q5_K (quant.rs:216-226, 283-291); sc = 12 bytes at `off`.
__device__ __forceinline__ void rf_scale_min_k4(const uint8_t* b, uint32_t off, uint32_t j,
                                                uint32_t& d, uint32_t& m) {
  uint32_t s[3];
  rf_lds_words<3>(b, off, s);
  auto byte = [&](uint32_t i) -> uint32_t { return (s[i >> 2] >> (8 * (i & 3))) & 0xFFu; };
  if (j < 4) {
    d = byte(j) & 63u;
    m = byte(j + 4) & 63u;
  } else {
    d = (byte(j + 4) & 0xFu) | ((byte(j - 4) >> 6) << 4);
    m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
  }
}

// ---------------------------------------------------------------- Q4_K (144 B)
// quant.rs:186-255: d @0, dmin @2, scales[12] @4, qs[128] @16.  Sub-block s
// (elements 32s..32s+31) uses qs[32(s/2) + l], low nibble if s even, high if
// odd, value (d*sc)*q - dmin*m.
template <> struct Fmt<T_Q4_K> {
  static constexpr uint32_t QK = 256, BS = 144;
  __device__ static float dot(const uint8_t* b, uint32_t blk, uint32_t s, const XUnit& x) {
    const uint32_t dd = rf_lds_u32(b, blk);
    const float d = rf_half_to_float(dd & 0xFFFFu), dmin = rf_half_to_float(dd >> 16);
    uint32_t sc, m;
    rf_scale_min_k4(b, blk + 4, s, sc, m);
    uint32_t w[8];
    rf_lds_words<8>(b, blk + 16 + 32 * (s >> 1), w);
    const uint32_t sh = (s & 1u) * 4u;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t n = rf_opaque((w[i] >> sh) & 0x0F0F0F0Fu);
#pragma unroll
      for (int k = 0; k < 4; ++k) acc = fmaf(rf_ub(n, k), x.v[4 * i + k], acc);
    }
    return fmaf(d * (float)sc, acc, -(dmin * (float)m) * x.sum);
  }
  __device__ static void dequant(const uint8_t* b, uint32_t blk, uint32_t s, float* out) {
    const float d = rf_half_to_float(rf_ld_u16(b + blk)), dmin = rf_half_to_float(rf_ld_u16(b + blk + 2));
    const uint8_t* sc = b + blk + 4;
    uint32_t scv, mv;
    if (s < 4) { scv = sc[s] & 63u; mv = sc[s + 4] & 63u; }
    else { scv = (sc[s + 4] & 0xFu) | ((sc[s - 4] >> 6) << 4); mv = (sc[s + 4] >> 4) | ((sc[s] >> 6) << 4); }
    const float d1 = d * (float)scv, m1 = dmin * (float)mv;
    const uint8_t* qs = b + blk + 16 + 32 * (s >> 1);
    for (int l = 0; l < 32; ++l) {
      const uint32_t q = (s & 1u) ? (qs[l] >> 4) : (qs[l] & 0x0Fu);
      out[l] = d1 * (float)q - m1;
    }
  }
};

// ---------------------------------------------------------------- Q5_K (176 B)
// quant.rs:259-343: d @0, dmin @2, scales[12] @4, qh[32] @16, qs[128] @48.
// High bit of element l in sub-block s = bit (s) of qh[8(s/2) + l/8]
// (the reference indexes qh[q_offset/4 + l/8] with masks 1<<2j / 2<<2j).
template <> struct Fmt<T_Q5_K> {
  static constexpr uint32_t QK = 256, BS = 176;
  __device__ static float dot(const uint8_t* b, uint32_t blk, uint32_t s, const XUnit& x) {
    const uint32_t dd = rf_lds_u32(b, blk);
    const float d = rf_half_to_float(dd & 0xFFFFu), dmin = rf_half_to_float(dd >> 16);
    uint32_t sc, m;
    rf_scale_min_k4(b, blk + 4, s, sc, m);
    const uint32_t j = s >> 1;
    const uint32_t qh = rf_lds_u32(b, blk + 16 + 8 * j);  // bytes qh[8j .. 8j+3]
    uint32_t w[8];
    rf_lds_words<8>(b, blk + 48 + 32 * j, w);
    const uint32_t sh = (s & 1u) * 4u;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t n = rf_opaque((w[i] >> sh) & 0x0F0F0F0Fu);
      // element l = 4i + k reads byte l/8 = i/2 of qh, bit s
      const uint32_t hb = (qh >> (8 * (i >> 1) + s)) & 1u;
      const uint32_t nh = n | (hb * 0x10101010u);
#pragma unroll
      for (int k = 0; k < 4; ++k) acc = fmaf(rf_ub(nh, k), x.v[4 * i + k], acc);
    }
    return fmaf(d * (float)sc, acc, -(dmin * (float)m) * x.sum);
  }
  __device__ static void dequant(const uint8_t* b, uint32_t blk, uint32_t s, float* out) {
    const float d = rf_half_to_float(rf_ld_u16(b + blk)), dmin = rf_half_to_float(rf_ld_u16(b + blk + 2));
    const uint8_t* sc = b + blk + 4;
    uint32_t scv, mv;
    if (s < 4) { scv = sc[s] & 63u; mv = sc[s + 4] & 63u; }
    else { scv = (sc[s + 4] & 0xFu) | ((sc[s - 4] >> 6) << 4); mv = (sc[s + 4] >> 4) | ((sc[s] >> 6) << 4); }
    const float d1 = d * (float)scv, m1 = dmin * (float)mv;
    const uint32_t j = s >> 1, u = (s & 1u) ? (2u << (2 * j)) : (1u << (2 * j));
    const uint8_t* qh = b + blk + 16;
    const uint8_t* qs = b + blk + 48 + 32 * j;
    for (int l = 0; l < 32; ++l) {
      const uint32_t q = (s & 1u) ? (qs[l] >> 4) : (qs[l] & 0x0Fu);
      const uint32_t high = (qh[(32 * j) / 4 + l / 8] & u) ? 16u : 0u;
      out[l] = d1 * (float)(q + high) - m1;
    }
  }
};

// ---------------------------------------------------------------- Q6_K (210 B)
// quant.rs:347-407: ql[128] @0, qh[64] @128, scales i8[16] @192, d f16 @208.
// Unit s = 4*hf + k covers elements 128hf + 32k + l: low 4 bits from
// ql[64hf + 32(k&1) + l] (nibble k>>1), high 2 bits from qh[32hf + l] >> 2k,
// scale scales[8hf + 2k + l/16]; value (d*sc)*(q-32).
template <> struct Fmt<T_Q6_K> {
  static constexpr uint32_t QK = 256, BS = 210;
  __device__ static float dot(const uint8_t* b, uint32_t blk, uint32_t s, const XUnit& x) {
    const uint32_t hf = s >> 2, k = s & 3u;
    const float d = rf_half_to_float(rf_lds_u32(b, blk + 208) & 0xFFFFu);
    const uint32_t scw = rf_lds_u32(b, blk + 192 + 8 * hf + 2 * k);
    const float sc_lo = (float)(int8_t)(scw & 0xFFu), sc_hi = (float)(int8_t)((scw >> 8) & 0xFFu);
    uint32_t ql[8], qh[8];
    rf_lds_words<8>(b, blk + 64 * hf + 32 * (k & 1u), ql);
    rf_lds_words<8>(b, blk + 128 + 32 * hf, qh);
    const uint32_t nsh = (k >> 1) * 4u, hsh = 2u * k;
    float acc_lo = 0.f, acc_hi = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // 4 (q - 32) as int8 bytes: exact products
      const uint32_t q =
          rf_opaque(rf_top_signed(((ql[i] >> nsh) & 0x0F0F0F0Fu) | (((qh[i] >> hsh) & 0x03030303u) << 4), 6));
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if (i < 4) acc_lo = fmaf(rf_sb(q, kk), x.v[4 * i + kk], acc_lo);
        else acc_hi = fmaf(rf_sb(q, kk), x.v[4 * i + kk], acc_hi);
      }
    }
    return d * (fmaf(sc_lo, acc_lo, sc_hi * acc_hi) * 0.25f);
  }
  __device__ static void dequant(const uint8_t* b, uint32_t blk, uint32_t s, float* out) {
    const uint32_t hf = s >> 2, k = s & 3u;
    const float d = rf_half_to_float(rf_ld_u16(b + blk + 208));
    const uint8_t* ql = b + blk + 64 * hf + 32 * (k & 1u);
    const uint8_t* qh = b + blk + 128 + 32 * hf;
    const int8_t* sc = reinterpret_cast<const int8_t*>(b + blk + 192 + 8 * hf + 2 * k);
    for (int l = 0; l < 32; ++l) {
      const uint32_t lo = (k >> 1) ? (ql[l] >> 4) : (ql[l] & 0x0Fu);
      const int q = (int)(lo | (((qh[l] >> (2 * k)) & 3u) << 4)) - 32;
      out[l] = d * (float)sc[l / 16] * (float)q;
    }
  }
};

// ---------------------------------------------------------------- Q2_K (84 B)
// quant.rs:411-473: scales[16] @0, qs[64] @16, d @80, dmin @82.  Unit s =
// 4n + k covers elements 128n + 32k + l: q = (qs[32n + l] >> 2k) & 3, scale
// byte scales[8n + 2k + l/16]; value (d*(sc&15))*q - dmin*(sc>>4).
template <> struct Fmt<T_Q2_K> {
  static constexpr uint32_t QK = 256, BS = 84;
  __device__ static float dot(const uint8_t* b, uint32_t blk, uint32_t s, const XUnit& x) {
    const uint32_t n = s >> 2, k = s & 3u;
    const uint32_t dd = rf_lds_u32(b, blk + 80);
    const float d = rf_half_to_float(dd & 0xFFFFu), dmin = rf_half_to_float(dd >> 16);
    const uint32_t scw = rf_lds_u32(b, blk + 8 * n + 2 * k);
    const uint32_t s0 = scw & 0xFFu, s1 = (scw >> 8) & 0xFFu;
    uint32_t w[8];
    rf_lds_words<8>(b, blk + 16 + 32 * n, w);
    float acc_lo = 0.f, acc_hi = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t q = (w[i] >> (2 * k)) & 0x03030303u;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if (i < 4) acc_lo = fmaf(rf_ub(q, kk), x.v[4 * i + kk], acc_lo);
        else acc_hi = fmaf(rf_ub(q, kk), x.v[4 * i + kk], acc_hi);
      }
    }
    const float r_lo = fmaf(d * (float)(s0 & 15u), acc_lo, -(dmin * (float)(s0 >> 4)) * x.sum_lo);
    const float r_hi = fmaf(d * (float)(s1 & 15u), acc_hi, -(dmin * (float)(s1 >> 4)) * x.sum_hi);
    return r_lo + r_hi;
  }
  __device__ static void dequant(const uint8_t* b, uint32_t blk, uint32_t s, float* out) {
    const uint32_t n = s >> 2, k = s & 3u;
    const float d = rf_half_to_float(rf_ld_u16(b + blk + 80)), dmin = rf_half_to_float(rf_ld_u16(b + blk + 82));
    const uint8_t* qs = b + blk + 16 + 32 * n;
    for (int h = 0; h < 2; ++h) {
      const uint32_t sc = b[blk + 8 * n + 2 * k + h];
      const float dl = d * (float)(sc & 0xFu), ml = dmin * (float)(sc >> 4);
      for (int l = 0; l < 16; ++l) {
        const uint32_t q = (qs[16 * h + l] >> (2 * k)) & 3u;
        out[16 * h + l] = dl * (float)q - ml;
      }
    }
  }
};

// Q3_K 6-bit scale j (0..7) as the reference unpacks it (quant.rs:508-541):
// only scales[0..8) are ever used (see Fmt<T_Q3_K>).
__device__ __forceinline__ int rf_q3k_scale(uint32_t s0_3, uint32_t s4_7, uint32_t s8_11, uint32_t j) {
  if (j < 4) {
    const uint32_t lo = (s0_3 >> (8 * j)) & 0xFu, hi = (s8_11 >> (8 * j)) & 3u;
    return (int)(lo | (hi << 4));
  }
  const uint32_t jj = j - 4;
  const uint32_t lo = (s4_7 >> (8 * jj)) & 0xFu, hi = (s8_11 >> (8 * jj + 2)) & 3u;
  return (int)(lo | (hi << 4));
}

// ---------------------------------------------------------------- Q3_K (110 B)
// quant.rs:477-575: hmask[32] @0, qs[64] @32, scales[12] @96, d @108.  Unit
// s = 4n + j covers elements 128n + 32j + l: q = ((qs[32n + l] >> 2j) & 3) -
// (hmask[l] bit (4n+j) ? 0 : 4); the reference takes the scale from
// scales[j] for l < 16 and scales[j+4] for l >= 16 in BOTH halves n.
template <> struct Fmt<T_Q3_K> {
  static constexpr uint32_t QK = 256, BS = 110;
  __device__ static float dot(const uint8_t* b, uint32_t blk, uint32_t s, const XUnit& x) {
    const uint32_t n = s >> 2, j = s & 3u;
    const float d = rf_half_to_float(rf_lds_u32(b, blk + 108) & 0xFFFFu);
    uint32_t sw[3];
    rf_lds_words<3>(b, blk + 96, sw);
    const float sc_lo = (float)(rf_q3k_scale(sw[0], sw[1], sw[2], j) - 32);
    const float sc_hi = (float)(rf_q3k_scale(sw[0], sw[1], sw[2], j + 4) - 32);
    uint32_t w[8], hm[8];
    rf_lds_words<8>(b, blk + 32 + 32 * n, w);
    rf_lds_words<8>(b, blk, hm);
    const uint32_t bit = 4 * n + j;
    float acc_lo = 0.f, acc_hi = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // 32 (t - 4) as int8 bytes: exact products
      const uint32_t t =
          rf_opaque(rf_top_signed(((w[i] >> (2 * j)) & 0x03030303u) | (((hm[i] >> bit) & 0x01010101u) << 2), 3));
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if (i < 4) acc_lo = fmaf(rf_sb(t, kk), x.v[4 * i + kk], acc_lo);
        else acc_hi = fmaf(rf_sb(t, kk), x.v[4 * i + kk], acc_hi);
      }
    }
    return d * (fmaf(sc_lo, acc_lo, sc_hi * acc_hi) * 0.03125f);
  }
  __device__ static void dequant(const uint8_t* b, uint32_t blk, uint32_t s, float* out) {
    const uint32_t n = s >> 2, j = s & 3u;
    const float d = rf_half_to_float(rf_ld_u16(b + blk + 108));
    const uint8_t* sc = b + blk + 96;
    auto w32 = [&](int o) { return (uint32_t)sc[o] | ((uint32_t)sc[o + 1] << 8) | ((uint32_t)sc[o + 2] << 16) | ((uint32_t)sc[o + 3] << 24); };
    const uint32_t a0 = w32(0), a1 = w32(4), a2 = w32(8);
    const uint8_t* qs = b + blk + 32 + 32 * n;
    const uint8_t* hm = b + blk;
    const uint32_t m = 1u << (4 * n + j);
    for (int h = 0; h < 2; ++h) {
      const int scv = rf_q3k_scale(a0, a1, a2, j + 4 * h) - 32;
      const float dl = d * (float)scv;
      for (int l = 0; l < 16; ++l) {
        int q = (int)((qs[16 * h + l] >> (2 * j)) & 3u);
        q -= (hm[16 * h + l] & m) ? 0 : 4;
        out[16 * h + l] = dl * (float)q;
      }
    }
  }
};

// ---------------------------------------------------------------- Q8_K (292 B)
// quant.rs:579-612: d f32 @0, qs i8[256] @4, bsums @260; value d * q.
template <> struct Fmt<T_Q8_K> {
  static constexpr uint32_t QK = 256, BS = 292;
  __device__ static float dot(const uint8_t* b, uint32_t blk, uint32_t s, const XUnit& x) {
    const float d = __uint_as_float(rf_lds_u32(b, blk));
    uint32_t w[8];
    rf_lds_words<8>(b, blk + 4 + 32 * s, w);
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) acc = fmaf(rf_sb(w[i], k), x.v[4 * i + k], acc);
    return d * acc;
  }
  __device__ static void dequant(const uint8_t* b, uint32_t blk, uint32_t s, float* out) {
    float d;
    __builtin_memcpy(&d, b + blk, 4);
    for (int i = 0; i < 32; ++i) out[i] = d * (float)(int8_t)b[blk + 4 + 32 * s + i];
  }
};

// ---------------------------------------------------------------- F32
template <> struct Fmt<T_F32> {
  static constexpr uint32_t QK = 32, BS = 128;  // a "block" is one 32-float unit
  __device__ static float dot(const uint8_t* b, uint32_t blk, uint32_t, const XUnit& x) {
    const float4* p = reinterpret_cast<const float4*>(b + blk);
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 w = p[i];
      acc = fmaf(w.x, x.v[4 * i], acc);
      acc = fmaf(w.y, x.v[4 * i + 1], acc);
      acc = fmaf(w.z, x.v[4 * i + 2], acc);
      acc = fmaf(w.w, x.v[4 * i + 3], acc);
    }
    return acc;
  }
};

// A unit of x holding an infinity or NaN: in place of the dot, the kind of
// the reference's terms (q * d) * x_i with each weight decoded bit-exactly
// (dequant): NaN when a term is NaN or infinities of both signs occur, else
// the one infinity.  Adding such values reproduces the reference's row
// result for any summation order: finite units do not change an infinity,
// and +inf + -inf and NaN + anything are NaN.
template <uint32_t T>
__device__ float unit_kinds(const uint8_t* b, uint32_t blk, uint32_t sub, const XUnit& x) {
  float deq[32];
  Fmt<T>::dequant(b, blk, sub, deq);
  bool nan = false, pinf = false, ninf = false;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const float t = deq[i] * x.v[i];
    nan = nan || t != t;
    pinf = pinf || t == __builtin_inff();
    ninf = ninf || t == -__builtin_inff();
  }
  if (nan || (pinf && ninf)) return __builtin_nanf("");
  return pinf ? __builtin_inff() : (ninf ? -__builtin_inff() : 0.f);
}

__device__ __forceinline__ bool unit_finite(const XUnit& x) {
  bool ok = true;
#pragma unroll
  for (int i = 0; i < 32; ++i) ok = ok && fabsf(x.v[i]) <= 3.40282347e38f;
  return ok;
}

}  // namespace rf
