// rf_matvec_packed.hip — batch-1 matvec on the device-native ("packed")
// layout of Q8_0, Q4_0, Q4_K and Q6_K matrices (gfx950).
//
// Same arithmetic as quant::matvec_q8_0 / matvec_q4_0 / matvec_q4_k /
// matvec_q6_k (core/src/quant.rs:898-1327): y[o] = sum over blocks of the
// block's decoded weights times x, with the reference's codes and scales;
// only the memory layout differs.
//
// Packed layout of a [rows][in] matrix: the bytes of every block are split
// into regions, each stored for all rows, row-major (same byte count as the
// GGUF payload):
//   Q8_0 / Q4_0: codes (32 / 16 bytes per block; Q4_0 keeps the GGUF nibble
//                order), f16 scales (2 bytes per block)
//   Q4_K:        codes (qs, 128 bytes per block), header (d, dmin, the 12
//                6-bit scale/min bytes: 16 bytes per block)
//   Q6_K:        ql (128), qh (64), int8 scales (16), f16 d (2 per block)
// GGUF interleaves these, so its blocks are never 16-byte aligned.  Split
// apart, the code bytes of a row are one aligned stream that a wavefront reads
// with 16-byte loads straight into registers.
//
// Work decomposition: lane l of a wavefront owns bytes [1024c + 16l, +16) of
// "chunk" c of a row's codes (16 Q8_0 codes, or 32 codes of the 4-/6-bit
// formats); one 16-byte load per lane moves 1 KiB per instruction.  The 16
// or 32 weights of a lane meet one or two 16-element "units" of x: Q4_0's low
// nibbles are elements j, its high nibbles j + 16; Q4_K's are 32 apart (two
// sub-blocks of a 64-element group); Q6_K's 64 apart.  x (times the norm
// weights when the RMSNorm prologue is fused) and the sum of every unit are
// staged in LDS once per workgroup, so no register holds x between steps.  A
// wavefront owns U whole rows (every chunk), so no partial sum crosses
// wavefronts and the main loop has no barrier; a step is U rows x LPW chunks
// and the next step's codes are requested before the current one is decoded
// (NB register buffers).  Row sums are DPP row reductions plus readlane.
// Fusions as in rf_matvec.hip: RMSNorm prologue, residual or SiLU(gate)*up
// epilogue, up to three output segments.
#include "rf_kernels.h"

#include <algorithm>
#include <cstdio>
#include <mutex>
#include <type_traits>

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

typedef __amdgpu_buffer_rsrc_t PkRsrc;

// ---------------------------------------------------------------- formats
//
// PkFmt<T>:
//   QK, EPB      block elements, elements per byte of the code region
//   NREG         regions; row_bytes(k, in) = bytes of region k per row
//   Meta         what a lane loads besides its 16 code bytes
//   fetch        loads of one lane at code byte b of the row
//   unit_elem    first element of unit h of the lane whose codes start at b
//   word         decode code word i against x words (units 0 and 1)
//   finish       scale the unit sums into the chunk's contribution
//   INTX         codes are summed against x's int8 digit planes (idot,
//                ifinish) instead of decoded to float (word, finish)
// Lane constants (which sub-block / half a lane's 16 bytes fall in) depend
// only on b % 128 = 16 (lane % 8), because every chunk starts at a multiple of
// 1024 bytes.

template <uint32_t T> struct PkFmt;

// x digits of one unit (matvec_packed's prologue): x = s X with the int32
// X = 2^24 a + 2^16 b + 2^8 c + e in balanced int8 digits (PK_PLANES planes);
// S[p] = sum of codes times digit plane p, exact in int32 (|S| < 2^18).  The
// unit's value is s times S[0] 2^24 + S[1] 2^16 + S[2] 2^8 + S[3]: the pairs
// are joined exactly in int32 (|S[0] 2^8 + S[1]| < 2^26), then two
// conversions and one fma round, each at most 2^-24 relative.
constexpr int PK_PLANES = 4;
__device__ __forceinline__ float pk_digits(const int* S) {
  const int hi = S[0] * 256 + S[1], lo = S[2] * 256 + S[3];
  return fmaf((float)hi, 65536.f, (float)lo);
}

// Non-finite x (matvec_packed's fallback): the kind of the reference's
// term deq * x, as bit 0 NaN, bit 1 +inf, bit 2 -inf.
__device__ __forceinline__ uint32_t pk_term_kind(float deq, float x) {
  const float t = deq * x;
  return t != t ? 1u : (t == __builtin_inff() ? 2u : (t == -__builtin_inff() ? 4u : 0u));
}
__device__ __forceinline__ uint32_t pk_word_kinds(const float* deq, const float4& x) {
  return pk_term_kind(deq[0], x.x) | pk_term_kind(deq[1], x.y) | pk_term_kind(deq[2], x.z) |
         pk_term_kind(deq[3], x.w);
}

template <> struct PkFmt<T_Q8_0> {
  static constexpr uint32_t QK = 32, EPB = 1, NREG = 2;
  static constexpr bool INTX = true;
  __host__ __device__ static uint64_t row_bytes(int k, uint64_t in) { return k == 0 ? in : in / 32 * 2; }
  typedef uint32_t Meta;  // f16 scale bits
  struct Lane {
    __device__ explicit Lane(uint32_t) {}
  };
  __device__ static void fetch(nv_u32x4& q, Meta& m, const PkRsrc* r, uint32_t b) {
    q = __builtin_amdgcn_raw_buffer_load_b128(r[0], b, 0, PK_AUX_NT);
    m = __builtin_amdgcn_raw_buffer_load_b16(r[1], (b >> 5) << 1, 0, 0);  // block b/32, 2 bytes each
  }
  __device__ static uint32_t unit_elem(uint32_t b, uint32_t) { return b; }
  // signed codes times x, each product exact up to its own rounding (a zero
  // code adds exactly nothing, as the reference's (q * d) * x does)
  __device__ static void word(const Lane&, uint32_t q, const Meta&, int, const float4& xv, const float4&,
                              float& s0, float&) {
    s0 = fmaf(rf_sb(q, 0), xv.x, s0); s0 = fmaf(rf_sb(q, 1), xv.y, s0);
    s0 = fmaf(rf_sb(q, 2), xv.z, s0); s0 = fmaf(rf_sb(q, 3), xv.w, s0);
  }
  __device__ static float finish(const Lane&, const Meta& m, float s0, float, float, float) {
    return rf_half_to_float_fast(m) * s0;
  }
  // the codes are signed bytes: one dot4 per word and digit plane
  __device__ static void idot(const Lane&, const nv_u32x4& q, const nv_u32x4* P, int (*S)[PK_PLANES]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int p = 0; p < PK_PLANES; ++p)
        S[0][p] = __builtin_amdgcn_sdot4((int)q[i], (int)P[p][i], S[0][p], false);
  }
  __device__ static float ifinish(const Lane&, const Meta& m, int (*S)[PK_PLANES], const float2* u) {
    return rf_half_to_float_fast(m) * (u[0].x * pk_digits(S[0]));
  }
  // word i's terms, each weight decoded as the reference does (quant.rs:177-181: q * d)
  __device__ static uint32_t kinds(const Lane&, uint32_t q, const Meta& m, int, const float4& xv, const float4&) {
    const float d = rf_half_to_float_fast(m);
    float deq[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) deq[k] = (float)(int8_t)((q >> (8 * k)) & 0xFFu) * d;
    return pk_word_kinds(deq, xv);
  }
};

template <> struct PkFmt<T_Q4_0> {
  static constexpr uint32_t QK = 32, EPB = 2, NREG = 2;
  static constexpr bool INTX = true;
  __host__ __device__ static uint64_t row_bytes(int k, uint64_t in) { return k == 0 ? in / 2 : in / 32 * 2; }
  typedef uint32_t Meta;
  struct Lane {
    __device__ explicit Lane(uint32_t) {}
  };
  __device__ static void fetch(nv_u32x4& q, Meta& m, const PkRsrc* r, uint32_t b) {
    q = __builtin_amdgcn_raw_buffer_load_b128(r[0], b, 0, PK_AUX_NT);
    m = __builtin_amdgcn_raw_buffer_load_b16(r[1], (b >> 4) << 1, 0, 0);  // block b/16
  }
  // byte j: low nibble -> element j, high nibble -> element j + 16 (quant.rs:84-113)
  __device__ static uint32_t unit_elem(uint32_t b, uint32_t h) { return 2u * b + 16u * h; }
  // The signed codes nibble - 8 as int8 bytes 16 (nibble - 8): products with
  // x are exact up to their own rounding (no -8 sum(x) correction to cancel
  // against), and the factor 16 comes off exactly in finish.  (Converting
  // each nibble with v_cvt_off_f32_i4 instead, (nibble ^ 8) / 16 with the
  // byte picked by SDWA, saves two instructions per word but timed the same:
  // 14336 x 4096 9.52 against 9.47 us, 4096 x 14336 10.60 against 10.56.)
  __device__ static void word(const Lane&, uint32_t q, const Meta&, int, const float4& xv, const float4& xw,
                              float& s0, float& s1) {
    const uint32_t lo = rf_opaque(rf_top_signed(q, 4)), hi = rf_opaque(rf_top_signed(q >> 4, 4));
    s0 = fmaf(rf_sb(lo, 0), xv.x, s0); s0 = fmaf(rf_sb(lo, 1), xv.y, s0);
    s0 = fmaf(rf_sb(lo, 2), xv.z, s0); s0 = fmaf(rf_sb(lo, 3), xv.w, s0);
    s1 = fmaf(rf_sb(hi, 0), xw.x, s1); s1 = fmaf(rf_sb(hi, 1), xw.y, s1);
    s1 = fmaf(rf_sb(hi, 2), xw.z, s1); s1 = fmaf(rf_sb(hi, 3), xw.w, s1);
  }
  __device__ static float finish(const Lane&, const Meta& m, float s0, float s1, float, float) {
    return rf_half_to_float_fast(m) * ((s0 + s1) * 0.0625f);
  }
  // the same int8 bytes 16 (nibble - 8) against the digits: exact int32 sums
  __device__ static void idot(const Lane&, const nv_u32x4& q, const nv_u32x4* P, int (*S)[PK_PLANES]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = rf_opaque(rf_top_signed(q[i], 4)), hi = rf_opaque(rf_top_signed(q[i] >> 4, 4));
#pragma unroll
      for (int p = 0; p < PK_PLANES; ++p) {
        S[0][p] = __builtin_amdgcn_sdot4((int)lo, (int)P[p][i], S[0][p], false);
        S[1][p] = __builtin_amdgcn_sdot4((int)hi, (int)P[PK_PLANES + p][i], S[1][p], false);
      }
    }
  }
  __device__ static float ifinish(const Lane&, const Meta& m, int (*S)[PK_PLANES], const float2* u) {
    const float s = fmaf(u[0].x, pk_digits(S[0]), u[1].x * pk_digits(S[1]));
    return rf_half_to_float_fast(m) * (s * 0.0625f);
  }
  // (nibble - 8) * d, low nibbles against unit 0, high against unit 1 (quant.rs:104-112)
  __device__ static uint32_t kinds(const Lane&, uint32_t q, const Meta& m, int, const float4& xv, const float4& xw) {
    const float d = rf_half_to_float_fast(m);
    float lo[4], hi[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      lo[k] = (float)((int)((q >> (8 * k)) & 0xFu) - 8) * d;
      hi[k] = (float)((int)((q >> (8 * k + 4)) & 0xFu) - 8) * d;
    }
    return pk_word_kinds(lo, xv) | pk_word_kinds(hi, xw);
  }
};

// Q4_K (quant.rs:186-255): a 256-element block is 4 groups of 64; byte l of
// group g holds element 64g + l (low nibble, sub-block 2g) and 64g + 32 + l
// (high nibble, sub-block 2g + 1).  A lane's 16 bytes are half hh of group g
// (g = (lane % 8) / 2, hh = lane % 2).  Sub-block j has 6-bit scale and min
// per get_scale_min (quant.rs:216-226); value d*sc*q - dmin*m.
template <> struct PkFmt<T_Q4_K> {
  static constexpr uint32_t QK = 256, EPB = 2, NREG = 2;
  static constexpr bool INTX = false;
  __host__ __device__ static uint64_t row_bytes(int k, uint64_t in) { return k == 0 ? in / 2 : in / 256 * 16; }
  typedef nv_u32x4 Meta;  // d | dmin << 16, then scale bytes 0-3, 4-7, 8-11
  struct Lane {
    uint32_t sh;  // bit offset of sub-block 2g's byte in its scale word
    bool hi;      // g >= 2: the 4+2-bit form
    __device__ explicit Lane(uint32_t lane) {
      const uint32_t g = (lane & 7u) >> 1;
      sh = 16u * (g & 1u);
      hi = g >= 2u;
    }
  };
  __device__ static void fetch(nv_u32x4& q, Meta& m, const PkRsrc* r, uint32_t b) {
    q = __builtin_amdgcn_raw_buffer_load_b128(r[0], b, 0, PK_AUX_NT);
    m = __builtin_amdgcn_raw_buffer_load_b128(r[1], (b >> 7) << 4, 0, 0);
  }
  __device__ static uint32_t unit_elem(uint32_t b, uint32_t h) {
    const uint32_t o = b & 127u;
    return (b >> 7) * 256u + 64u * (o >> 5) + 16u * ((o >> 4) & 1u) + 32u * h;
  }
  // unsigned nibbles: the min term dmin * m * sum(x) is part of the format
  __device__ static void word(const Lane&, uint32_t q, const Meta&, int, const float4& xv, const float4& xw,
                              float& s0, float& s1) {
    const uint32_t lo = rf_opaque(q & 0x0F0F0F0Fu), hi = rf_opaque((q >> 4) & 0x0F0F0F0Fu);
    s0 = fmaf(rf_ub(lo, 0), xv.x, s0); s0 = fmaf(rf_ub(lo, 1), xv.y, s0);
    s0 = fmaf(rf_ub(lo, 2), xv.z, s0); s0 = fmaf(rf_ub(lo, 3), xv.w, s0);
    s1 = fmaf(rf_ub(hi, 0), xw.x, s1); s1 = fmaf(rf_ub(hi, 1), xw.y, s1);
    s1 = fmaf(rf_ub(hi, 2), xw.z, s1); s1 = fmaf(rf_ub(hi, 3), xw.w, s1);
  }
  __device__ static float finish(const Lane& L, const Meta& m, float s0, float s1, float xs0, float xs1) {
    // sub-blocks j = 2g (+0) and 2g + 1 (+8 bits): for j < 4 sc = S[j] & 63,
    // m = S[j+4] & 63; else sc = (S[j+4] & 15) | (S[j-4] >> 6) << 4,
    // m = (S[j+4] >> 4) | (S[j] >> 6) << 4  (S = the 12 scale bytes)
    uint32_t sc[2], mn[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint32_t s = L.sh + 8u * k;
      const uint32_t a = (m.y >> s) & 0xFFu, c = (m.z >> s) & 0xFFu, e = (m.w >> s) & 0xFFu;
      sc[k] = L.hi ? ((e & 15u) | ((a >> 6) << 4)) : (a & 63u);
      mn[k] = L.hi ? ((e >> 4) | ((c >> 6) << 4)) : (c & 63u);
    }
    const float d = rf_half_to_float_fast(m.x & 0xFFFFu), dmin = rf_half_to_float_fast(m.x >> 16);
    const float r0 = fmaf(d * (float)sc[0], s0, -(dmin * (float)mn[0]) * xs0);
    return fmaf(d * (float)sc[1], s1, fmaf(-(dmin * (float)mn[1]), xs1, r0));
  }
  // d1 * q - m1 with d1 = d * sc, m1 = dmin * m (quant.rs:228-254), no fused multiply-add
  __device__ static uint32_t kinds(const Lane& L, uint32_t q, const Meta& m, int, const float4& xv, const float4& xw) {
    const float d = rf_half_to_float_fast(m.x & 0xFFFFu), dmin = rf_half_to_float_fast(m.x >> 16);
    uint32_t out = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t s = L.sh + 8u * h;
      const uint32_t a = (m.y >> s) & 0xFFu, c = (m.z >> s) & 0xFFu, e = (m.w >> s) & 0xFFu;
      const uint32_t sc = L.hi ? ((e & 15u) | ((a >> 6) << 4)) : (a & 63u);
      const uint32_t mn = L.hi ? ((e >> 4) | ((c >> 6) << 4)) : (c & 63u);
      const float d1 = d * (float)sc, m1 = dmin * (float)mn;
      float deq[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float prod = d1 * (float)((q >> (8 * k + 4 * h)) & 0xFu);
        deq[k] = __fsub_rn(prod, m1);
      }
      out |= pk_word_kinds(deq, h ? xw : xv);
    }
    return out;
  }
};

// Q6_K (quant.rs:347-407): per 128-element half hf, byte r < 64 of ql holds
// element 128hf + r (low nibble) and 128hf + 64 + r (high nibble); their two
// high bits are bits 2k and 2k + 4 of qh[32hf + r % 32], k = r / 32; scales
// sc[8hf + 2k + (r % 32) / 16] and the same + 4; value d*sc*(q - 32).  A
// lane's 16 bytes sit at r = 16 (lane % 4) of half hf = (lane % 8) / 4.
template <> struct PkFmt<T_Q6_K> {
  static constexpr uint32_t QK = 256, EPB = 2, NREG = 4;
  static constexpr bool INTX = false;
  __host__ __device__ static uint64_t row_bytes(int k, uint64_t in) {
    return k == 0 ? in / 2 : k == 1 ? in / 4 : k == 2 ? in / 256 * 16 : in / 256 * 2;
  }
  struct Meta {
    nv_u32x4 qh, sc;
    uint32_t d;
  };
  struct Lane {
    uint32_t qsh;  // 2k: shift of the low unit's high bits
    uint32_t bsh;  // bit offset of the low unit's scale byte in its word
    bool hf;       // half 1: scale words 2 and 3 instead of 0 and 1
    __device__ explicit Lane(uint32_t lane) {
      qsh = 2u * ((lane & 3u) >> 1);
      bsh = 8u * (qsh + (lane & 1u));
      hf = (lane & 4u) != 0;
    }
  };
  __device__ static void fetch(nv_u32x4& q, Meta& m, const PkRsrc* r, uint32_t b) {
    const uint32_t blk = b >> 7, o = b & 127u;
    q = __builtin_amdgcn_raw_buffer_load_b128(r[0], b, 0, PK_AUX_NT);
    m.qh = __builtin_amdgcn_raw_buffer_load_b128(r[1], blk * 64u + 32u * (o >> 6) + (o & 31u), 0, PK_AUX_NT);
    m.sc = __builtin_amdgcn_raw_buffer_load_b128(r[2], blk * 16u, 0, 0);
    m.d = __builtin_amdgcn_raw_buffer_load_b16(r[3], blk * 2u, 0, 0);
  }
  __device__ static uint32_t unit_elem(uint32_t b, uint32_t h) {
    const uint32_t o = b & 127u;
    return (b >> 7) * 256u + 128u * (o >> 6) + (o & 63u) + 64u * h;
  }
  __device__ static void word(const Lane& L, uint32_t q, const Meta& m, int i, const float4& xv, const float4& xw,
                              float& s0, float& s1) {
    // the 6-bit codes q - 32 as int8 bytes 4 (q - 32): exact products, the
    // factor 4 comes off exactly in finish
    const uint32_t h = m.qh[i];
    const uint32_t lo = rf_opaque(rf_top_signed((q & 0x0F0F0F0Fu) | (((h >> L.qsh) & 0x03030303u) << 4), 6));
    const uint32_t hi =
        rf_opaque(rf_top_signed(((q >> 4) & 0x0F0F0F0Fu) | (((h >> (L.qsh + 4u)) & 0x03030303u) << 4), 6));
    s0 = fmaf(rf_sb(lo, 0), xv.x, s0); s0 = fmaf(rf_sb(lo, 1), xv.y, s0);
    s0 = fmaf(rf_sb(lo, 2), xv.z, s0); s0 = fmaf(rf_sb(lo, 3), xv.w, s0);
    s1 = fmaf(rf_sb(hi, 0), xw.x, s1); s1 = fmaf(rf_sb(hi, 1), xw.y, s1);
    s1 = fmaf(rf_sb(hi, 2), xw.z, s1); s1 = fmaf(rf_sb(hi, 3), xw.w, s1);
  }
  __device__ static float finish(const Lane& L, const Meta& m, float s0, float s1, float, float) {
    const uint32_t w0 = L.hf ? m.sc.z : m.sc.x, w1 = L.hf ? m.sc.w : m.sc.y;
    const float sc0 = (float)(int32_t)(int8_t)((w0 >> L.bsh) & 0xFFu);
    const float sc1 = (float)(int32_t)(int8_t)((w1 >> L.bsh) & 0xFFu);
    const float d = rf_half_to_float_fast(m.d);
    return d * (fmaf(sc0, s0, sc1 * s1) * 0.25f);
  }
  // (d * sc) * (q - 32) (quant.rs:376-406)
  __device__ static uint32_t kinds(const Lane& L, uint32_t q, const Meta& m, int i, const float4& xv,
                                   const float4& xw) {
    const uint32_t h = m.qh[i];
    const uint32_t w0 = L.hf ? m.sc.z : m.sc.x, w1 = L.hf ? m.sc.w : m.sc.y;
    const float d = rf_half_to_float_fast(m.d);
    const float ds0 = d * (float)(int32_t)(int8_t)((w0 >> L.bsh) & 0xFFu);
    const float ds1 = d * (float)(int32_t)(int8_t)((w1 >> L.bsh) & 0xFFu);
    float lo[4], hi[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t sh = 8u * k;
      const int ql = (int)(((q >> sh) & 0xFu) | (((h >> (L.qsh + sh)) & 3u) << 4));
      const int qh = (int)(((q >> (sh + 4u)) & 0xFu) | (((h >> (L.qsh + 4u + sh)) & 3u) << 4));
      lo[k] = ds0 * (float)(ql - 32);
      hi[k] = ds1 * (float)(qh - 32);
    }
    return pk_word_kinds(lo, xv) | pk_word_kinds(hi, xw);
  }
};

// Codes and metadata of one step: U rows x LPW chunks (twice with the "up" matrix).
template <uint32_t T, int U, int LPW, bool DUAL>
struct PkStep {
  nv_u32x4 q[U][LPW], q2[DUAL ? U : 1][LPW];
  typename PkFmt<T>::Meta m[U][LPW], m2[DUAL ? U : 1][LPW];
};

// The workgroup stages x while its first steps' codes are in flight.  x sits
// in LDS permuted so that the 16-byte reads of a step are consecutive across
// lanes (no bank conflicts): element 4i + k of unit h of lane l's slice of
// chunk c (EPL = 16 or 32 elements per slice) is stored at
// c * 64 * EPL + 256 (4h + i) + 4 l + k.  NB step buffers per wavefront: NB - 1
// steps are in flight while one is decoded.  ALLF: every step of the
// wavefront (its tasks times the steps of a row at most NB) is requested
// before the prologue and none after it, so a launch makes one memory round
// trip.
//
// MRG: x is merged from single-query attention's chunk records in the
// prologue (the merge the attention's own merge kernel does, so that launch
// is saved): per head, M = max of the chunks' m, factors f_c = exp(m_c - M),
// L = sum of l_c f_c and x = (sum of f_c o_c) / L, taken as a product with
// 1 / L.  Each thread merges half a unit (8 elements) over all chunks; the
// launch sees to 2 nunit <= NT and at most 8 chunks.
template <uint32_t T, int EPI, bool NORM, int U, int LPW, int NB, int NT, bool IX, bool ALLF = false,
          bool MRG = false>
__global__ __launch_bounds__(NT) void matvec_packed(PkArgs a) {
  typedef PkFmt<T> F;
  constexpr bool IXE = F::INTX && IX;  // digit planes instead of float x
  static_assert(!MRG || (!IXE && !NORM && EPI == EPI_RESIDUAL && ALLF), "merged x: one float-x residual step");
  // Non-finite x needs a fallback only where a decode does not multiply each
  // signed code by x: the digit planes, and Q4_K's min term (d sc sum(q x) -
  // dmin m sum(x) gives inf - inf where the reference's (d sc q - dmin m) x
  // is an infinity).  The signed-code float decodes of Q8_0, Q4_0 and Q6_K
  // produce the reference's NaN / +-inf rows by themselves: a code times an
  // infinity is the reference's term up to a positive power of two, and
  // finite terms cannot change an infinite or NaN sum.
  constexpr bool KINDS = IXE || T == T_Q4_K;
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  constexpr uint32_t EPB = F::EPB, UPS = EPB, EPL = 16u * UPS, NW = NT / 64;
  extern __shared__ __align__(16) float xl[];  // [nchunk * 64 * EPL] x, then [nchunk * 64 * UPS] unit sums
  __shared__ float wsum[NW];
  __shared__ uint32_t wbad[NW];  // the wavefront staged a non-finite x element
  __shared__ float resl[EPI == EPI_RESIDUAL ? NW : 1][PK_RES_SLOTS][U];
  static_assert(sizeof(wsum) + sizeof(wbad) + sizeof(resl) <= PK_STATIC_LDS,
                "static LDS above the planner's reservation");
  // The wavefront index through readfirstlane: rows, segments and their
  // pointers are then scalar values, so no vector load (whose wait would also
  // wait for the codes in flight) is spent on them.
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // MRG: the position first, before any store of the kernel (so that it is a
  // scalar load: nothing this kernel writes comes before it)
  const uint32_t m_posv = MRG ? (uint32_t)(*a.m_pos) : 0u;
  if (a.advance != nullptr && blockIdx.x == 0 && tid == 0) *a.advance += 1;
  const uint32_t in = a.in_dim, crb = in / EPB;
  const uint32_t nchunk = (crb + 1023u) / 1024u, nstep = (nchunk + LPW - 1) / LPW;
  float* xsum_l = xl + nchunk * 64u * EPL;
  // INTX: digit planes (plane p of unit h of lane l in chunk c at byte
  // ((c UPS + h) PK_PLANES + p) 1024 + 16 l), then (scale, scale * sum of X)
  // of unit j at float2 j.  The launch sizes LDS for the larger of this and
  // the float layout, which the kernel falls back to for a non-finite x.
  uint8_t* xdig = reinterpret_cast<uint8_t*>(xl);
  float2* xinfo = reinterpret_cast<float2*>(xdig + nchunk * UPS * (1024u * PK_PLANES));
  const typename F::Lane LC(lane);

  auto seg_of = [&](uint32_t v) -> PkSeg {
    return (a.nseg > 2 && v >= a.seg[2].row_begin) ? a.seg[2]
                                                   : ((a.nseg > 1 && v >= a.seg[1].row_begin) ? a.seg[1] : a.seg[0]);
  };

  const uint32_t ntask = (a.rows_total + U - 1) / U;
  const uint32_t gstride = gridDim.x * NW;

  typedef PkStep<T, U, LPW, DUAL> Step;
  Step buf[NB];
  // Raw buffer loads: one resource per row and region (scalar base, range =
  // the row's bytes), the lane's byte offset in a VGPR.  Offsets past the row
  // (the tail of a partial chunk) and every load of a fetch past the last task
  // (range 0) return zeros without touching memory, so fetches are issued
  // unconditionally and the compiler's wait counts stay exact: a consume waits
  // for its own step only, never for the prefetch behind it.
  auto fetch = [&](Step& B, uint32_t t, uint32_t st) {
    const bool live = t < ntask;  // wave-uniform
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t v = min(t * U + u, a.rows_total - 1u);
      const PkSeg g = seg_of(v);
      const uint32_t r = v - g.row_begin;
      PkRsrc rr[F::NREG], rr2[F::NREG];
#pragma unroll
      for (int k = 0; k < (int)F::NREG; ++k) {
        const uint32_t rb = (uint32_t)F::row_bytes(k, in);
        const int32_t n = live ? (int32_t)rb : 0;
        rr[k] = __builtin_amdgcn_make_buffer_rsrc((void*)(g.reg[k] + (size_t)r * rb), 0, n, PK_RSRC_WORD3);
        if constexpr (DUAL)
          rr2[k] = __builtin_amdgcn_make_buffer_rsrc((void*)(g.reg_up[k] + (size_t)r * rb), 0, n, PK_RSRC_WORD3);
      }
#pragma unroll
      for (int l = 0; l < LPW; ++l) {
        const uint32_t b = (st * LPW + l) * 1024u + 16u * lane;
        F::fetch(B.q[u][l], B.m[u][l], rr, b);
        if constexpr (DUAL) F::fetch(B.q2[u][l], B.m2[u][l], rr2, b);
      }
    }
  };

  auto advance = [&](uint32_t& tt, uint32_t& ss) {
    if (++ss == nstep) { ss = 0; tt += gstride; }
  };
  // Prologue, one round of loads and one barrier.  Thread j (then j + NT, ...)
  // owns unit j: 16 consecutive elements of x, unit j % UPS of lane slice
  // j / UPS.  It writes the unit into LDS and the unit's sum.  With NORM,
  // rms_norm_reference (core/src/compute.rs:291-319) is
  // x / sqrt(mean(x^2) + eps) * w; LDS holds x * w and every row sum is
  // scaled by 1 / sqrt(mean(x^2) + eps) in the epilogue (the same value up to
  // rounding), so the mean's reduction shares the prologue's barrier.
  const uint32_t nunit = nchunk * 64u * UPS;
  const float4* x4 = reinterpret_cast<const float4*>(a.x);
  const float4* w4 = reinterpret_cast<const float4*>(a.norm_w);
  // The 16 elements of unit j (times the norm weights), their squares summed
  // into ss; false for the zero padding past the row.
  auto load_unit = [&](uint32_t j, float* v, float& ss, bool sq) -> bool {
    const uint32_t js = j / UPS, h = j % UPS;
    const uint32_t b = (js >> 6) * 1024u + 16u * (js & 63u);
    if (b >= crb) return false;
    const uint32_t e = F::unit_elem(b, h);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float4 xv = x4[e / 4u + k];
      v[4 * k] = xv.x; v[4 * k + 1] = xv.y; v[4 * k + 2] = xv.z; v[4 * k + 3] = xv.w;
      if (NORM) {
        const float4 wv = w4[e / 4u + k];
        if (sq) {
          ss = fmaf(xv.x, xv.x, ss); ss = fmaf(xv.y, xv.y, ss);
          ss = fmaf(xv.z, xv.z, ss); ss = fmaf(xv.w, xv.w, ss);
        }
        v[4 * k] *= wv.x; v[4 * k + 1] *= wv.y; v[4 * k + 2] *= wv.z; v[4 * k + 3] *= wv.w;
      }
    }
    return true;
  };
  // Float layout: unit j (values v, or the zero padding past the row when
  // !have) in its permuted LDS slots and its sum.  Returns false for a
  // non-finite element.
  auto put_float = [&](uint32_t j, const float* v, bool have, bool check) -> bool {
    const uint32_t js = j / UPS, h = j % UPS;
    float s = 0.f;
    bool fin = true;
    if (have) {
      float* dst = xl + (js >> 6) * 64u * EPL + 4u * h * 256u + 4u * (js & 63u);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        *reinterpret_cast<float4*>(dst + 256 * k) = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
        s += v[4 * k]; s += v[4 * k + 1]; s += v[4 * k + 2]; s += v[4 * k + 3];
      }
      if (check) {
#pragma unroll
        for (int k = 0; k < 16; ++k) fin = fin && fabsf(v[k]) <= 3.40282347e38f;
      }
    }
    xsum_l[j] = s;
    return fin;
  };
  auto stage_float = [&](uint32_t j, float& ss, bool sq, bool check) -> bool {
    float v[16];
    const bool have = load_unit(j, v, ss, sq);
    return put_float(j, v, have, check);
  };
  // Digit layout: with 2^E above the unit's largest |x|, X = rint(x 2^(30 - E))
  // (|X| < 2^30) in balanced base-256 digits X = 2^24 a + 2^16 b + 2^8 c + e
  // (a in [-64, 64]); codes times digits then sum exactly in int32.  Each
  // element is off by at most 2^(E - 31), i.e. x keeps 30 bits below the
  // unit's largest element.  E is at least -96 so the scale 2^(E - 30) is a
  // normal float.  Returns false for a non-finite element (the kernel then
  // restages x as floats).
  auto stage_digits = [&](uint32_t j, float& ss) -> bool {
    const uint32_t js = j / UPS, h = j % UPS;
    nv_u32x4 pl[PK_PLANES] = {};
    float2 info = make_float2(0.f, 0.f);
    float v[16];
    bool fin = true;
    if (load_unit(j, v, ss, true)) {
      float mx = 0.f;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        mx = fmaxf(mx, fabsf(v[k]));
        fin = fin && fabsf(v[k]) <= 3.40282347e38f;
      }
      int ex = 0;
      (void)frexpf(mx, &ex);
      ex = ex < -96 ? -96 : ex;
      long long sx = 0;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int X = fin ? (int)rintf(ldexpf(v[k], 30 - ex)) : 0;
        const int d0 = (int)(int8_t)(X & 0xFF), X1 = (X - d0) >> 8;
        const int c0 = (int)(int8_t)(X1 & 0xFF), X2 = (X1 - c0) >> 8;
        const int b0 = (int)(int8_t)(X2 & 0xFF), a0 = (X2 - b0) >> 8;
        sx += X;
        const int sh = 8 * (k & 3);
        pl[0][k >> 2] |= (uint32_t)(a0 & 0xFF) << sh;
        pl[1][k >> 2] |= (uint32_t)(b0 & 0xFF) << sh;
        pl[2][k >> 2] |= (uint32_t)(c0 & 0xFF) << sh;
        pl[3][k >> 2] |= (uint32_t)(d0 & 0xFF) << sh;
      }
      const float sc = ldexpf(1.f, ex - 30);
      info = make_float2(sc, sc * (float)sx);
    }
    uint8_t* dst = xdig + (((js >> 6) * UPS + h) * PK_PLANES) * 1024u + 16u * (js & 63u);
#pragma unroll
    for (int p = 0; p < PK_PLANES; ++p) *reinterpret_cast<nv_u32x4*>(dst + 1024u * p) = pl[p];
    xinfo[j] = info;
    return fin;
  };

  // MRG: the (m, l) pair of record tid, then this thread's half of its unit
  // (thread t: unit t / 2, elements 8 (t % 2) .. + 7) from every chunk, all
  // before the weights.  Only the valid chunks' records are read (a uniform
  // count); with a single chunk the attention wrote x itself.
  uint32_t m_ns = 1, m_head = 0;
  float2 mlv = make_float2(0.f, 0.f);
  float4 mo[MRG ? 8 : 1][2];
  if constexpr (MRG) {
    const uint32_t total = m_posv + 1u, chunk = att_chunk(total, a.m_nsplit);
    m_ns = (total + chunk - 1u) / chunk;
    const uint32_t rec = att_rec(1u << a.m_hd_log2), hmask = (1u << a.m_hd_log2) - 1u;
    const PkRsrc wsr =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.mws, 0, (int32_t)(m_ns * a.m_qh * rec * 4u), PK_RSRC_WORD3);
    // lanes 8 h .. 8 h + 7: head h's (m, l) of chunks 0..7 (m = -inf, l = 0
    // past the valid ones)
    mlv = make_float2(-INFINITY, 0.f);
    if (m_ns > 1u && (tid >> 3) < a.m_qh && (tid & 7u) < m_ns) {
      const uint32_t r = (tid & 7u) * a.m_qh + (tid >> 3);
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(wsr, (r * rec + hmask + 1u) * 4u, 0, 0);
      mlv = make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
    }
    const uint32_t j = tid >> 1, js = j / UPS, hh = j % UPS;
    const uint32_t b = (js >> 6) * 1024u + 16u * (js & 63u);
    const uint32_t e = (j < nunit && b < crb ? F::unit_elem(b, hh) : 0u) + 8u * (tid & 1u);
    m_head = e >> a.m_hd_log2;
    if (m_ns == 1u) {
      const float4* xs = reinterpret_cast<const float4*>(a.x) + e / 4u;
      mo[0][0] = xs[0];
      mo[0][1] = xs[1];
    } else {
      const uint32_t off = ((m_head * rec) + (e & hmask)) * 4u, cstride = a.m_qh * rec * 4u;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        if ((uint32_t)c < m_ns) {  // uniform
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(wsr, off + c * cstride + 16u * k, 0, 0);
            mo[c][k] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                                   __uint_as_float(v[3]));
          }
        }
      }
    }
  }
  // x first: the raw loads of this thread's first unit are issued before
  // any weight step, so the prologue's wait for them does not also wait for
  // the codes requested behind them (a wavefront's loads complete in order).
  float4 xr[4], wr[4];
  bool xin = false;
  if constexpr (!IXE && !MRG) {
    const uint32_t js = tid / UPS, h = tid % UPS;
    const uint32_t b = (js >> 6) * 1024u + 16u * (js & 63u);
    xin = tid < nunit && b < crb;
    if (xin) {
      const uint32_t e = F::unit_elem(b, h);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        xr[k] = x4[e / 4u + k];
        if (NORM) wr[k] = w4[e / 4u + k];
      }
    }
  }
  // (Loading the first task's residual here too, before the weights, made
  // the 8B down projection 2.5 us slower.)
  __builtin_amdgcn_sched_barrier(0);
  // The first NB - 1 steps (ALLF: all NB) are requested before the prologue.
  uint32_t ct = blockIdx.x * NW + wave, cs = 0, ft = ct, fs = 0;
#pragma unroll
  for (int b = 0; b < (ALLF ? NB : NB - 1); ++b) {
    fetch(buf[b], ft, fs);
    advance(ft, fs);
  }

  bool finite = true;
  if constexpr (MRG) {
    // The merge's per-record work once per workgroup: each group of 8 lanes
    // holds one head's chunks, so M = the largest m, the factors exp(m - M)
    // and L = the sum of l times factor (a fixed butterfly order) take three
    // lane exchanges each; the factors and 1 / L go to LDS behind the unit
    // sums.  Each thread then sums factor times o over the chunks for its 8
    // elements, scales by 1 / L and stages them.
    float* fac = xsum_l + nunit;                 // [nsplit][qh]
    float* invl = fac + a.m_nsplit * a.m_qh;     // [qh]
    if (m_ns > 1u) {
      float M = mlv.x;
      M = fmaxf(M, __shfl_xor(M, 1));
      M = fmaxf(M, __shfl_xor(M, 2));
      M = fmaxf(M, __shfl_xor(M, 4));
      const float f = expf(mlv.x - M);  // 0 past the valid chunks
      float L = mlv.y * f;
      L += __shfl_xor(L, 1);
      L += __shfl_xor(L, 2);
      L += __shfl_xor(L, 4);
      const uint32_t h = tid >> 3, c = tid & 7u;
      if (h < a.m_qh) {
        if (c < m_ns) fac[c * a.m_qh + h] = f;
        if (c == 0u) invl[h] = 1.0f / L;
      }
      __syncthreads();
    }
    const uint32_t j = tid >> 1, half = tid & 1u, js = j / UPS, hh = j % UPS;
    const bool have = j < nunit && (js >> 6) * 1024u + 16u * (js & 63u) < crb;
    float v[8];
    if (m_ns == 1u) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        v[4 * k] = mo[0][k].x; v[4 * k + 1] = mo[0][k].y; v[4 * k + 2] = mo[0][k].z; v[4 * k + 3] = mo[0][k].w;
      }
    } else {
      const float f0 = fac[m_head];  // chunk 0 (m_ns >= 2)
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        v[4 * k] = f0 * mo[0][k].x; v[4 * k + 1] = f0 * mo[0][k].y;
        v[4 * k + 2] = f0 * mo[0][k].z; v[4 * k + 3] = f0 * mo[0][k].w;
      }
#pragma unroll
      for (int c = 1; c < 8; ++c) {
        if ((uint32_t)c < m_ns) {
          const float f = fac[c * a.m_qh + m_head];
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            v[4 * k] = fmaf(f, mo[c][k].x, v[4 * k]);
            v[4 * k + 1] = fmaf(f, mo[c][k].y, v[4 * k + 1]);
            v[4 * k + 2] = fmaf(f, mo[c][k].z, v[4 * k + 2]);
            v[4 * k + 3] = fmaf(f, mo[c][k].w, v[4 * k + 3]);
          }
        }
      }
      const float r = invl[m_head];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] *= r;
    }
    // the unit's slots (put_float's layout): this half's two float4; the
    // unit's sum (the two halves, adjacent lanes) where the format reads it
    if (have) {
      float* dst = xl + (js >> 6) * 64u * EPL + 4u * hh * 256u + 4u * (js & 63u) + 512u * half;
#pragma unroll
      for (int k = 0; k < 2; ++k)
        *reinterpret_cast<float4*>(dst + 256 * k) = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
    }
    if constexpr (T == T_Q4_K) {
      float s8 = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) s8 += v[k];
      const float s16 = s8 + __shfl_xor(s8, 1);
      if (j < nunit && half == 0u) xsum_l[j] = have ? s16 : 0.f;
    }
    if constexpr (KINDS) {
      bool fin = true;
#pragma unroll
      for (int k = 0; k < 8; ++k) fin = fin && fabsf(v[k]) <= 3.40282347e38f;
      finite = !have || fin;
    }
  }
  {
    float ss = 0.f;
    for (uint32_t j = tid; j < (MRG ? 0u : nunit); j += NT) {
      if constexpr (IXE) {
        finite = stage_digits(j, ss) && finite;
      } else if (j == tid) {  // the unit loaded above (load_unit's arithmetic)
        float v[16];
        if (xin) {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const float4 xv = xr[k];
            v[4 * k] = xv.x; v[4 * k + 1] = xv.y; v[4 * k + 2] = xv.z; v[4 * k + 3] = xv.w;
            if (NORM) {
              const float4 wv = wr[k];
              ss = fmaf(xv.x, xv.x, ss); ss = fmaf(xv.y, xv.y, ss);
              ss = fmaf(xv.z, xv.z, ss); ss = fmaf(xv.w, xv.w, ss);
              v[4 * k] *= wv.x; v[4 * k + 1] *= wv.y; v[4 * k + 2] *= wv.z; v[4 * k + 3] *= wv.w;
            }
          }
        }
        finite = put_float(j, v, xin, KINDS) && finite;
      } else {
        finite = stage_float(j, ss, true, KINDS) && finite;
      }
    }
    if (NORM) {
      ss = rf_wave_sum(ss);
      if (lane == 0) wsum[wave] = ss;
    }
    if constexpr (KINDS) {
      const bool bad = __ballot(!finite) != 0;
      if (lane == 0) wbad[wave] = bad ? 1u : 0u;
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
  // A non-finite x element (every workgroup sees the same x, so all of them
  // agree): every row sum is then non-finite.  The reference adds the terms
  // deq * x of a row in order (quant.rs:977-1029): NaN when a term is NaN or
  // terms of both infinite signs occur, else the one infinity.  That depends
  // on the terms only, not on their order, so each row's terms are classified
  // with the reference's own weight decode instead of summed (an overflow of
  // finite partial sums, which the reference's order could turn into NaN, is
  // not reproduced).
  bool bad = false;
  if constexpr (KINDS) {
#pragma unroll
    for (uint32_t i = 0; i < NW; ++i) bad = bad || wbad[i] != 0u;
  }
  float inv = 1.f;
  if (NORM) {
    float tot = 0.f;
#pragma unroll
    for (uint32_t i = 0; i < NW; ++i) tot += wsum[i];
    inv = 1.0f / sqrtf(tot / (float)in + a.eps);
  }
  if constexpr (KINDS) {
  if (bad) {
    if constexpr (IXE) {  // the digit layout holds no floats: stage them
      float unused = 0.f;
      for (uint32_t j = tid; j < nunit; j += NT) (void)stage_float(j, unused, false, false);
      __syncthreads();
    }
    for (uint32_t t = blockIdx.x * NW + wave; t < ntask; t += gstride) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t v = t * U + u;
        if (v >= a.rows_total) break;
        const PkSeg g = seg_of(v);
        const uint32_t r = v - g.row_begin;
        PkRsrc rr[F::NREG], rr2[F::NREG];
#pragma unroll
        for (int k = 0; k < (int)F::NREG; ++k) {
          const uint32_t rb = (uint32_t)F::row_bytes(k, in);
          rr[k] = __builtin_amdgcn_make_buffer_rsrc((void*)(g.reg[k] + (size_t)r * rb), 0, (int32_t)rb, PK_RSRC_WORD3);
          if constexpr (DUAL)
            rr2[k] = __builtin_amdgcn_make_buffer_rsrc((void*)(g.reg_up[k] + (size_t)r * rb), 0, (int32_t)rb,
                                                       PK_RSRC_WORD3);
        }
        uint32_t kd = 0, kd2 = 0;
        for (uint32_t c = 0; c < nchunk; ++c) {
          const uint32_t b = c * 1024u + 16u * lane;
          nv_u32x4 q, q2;
          typename F::Meta m, m2;
          F::fetch(q, m, rr, b);
          if constexpr (DUAL) F::fetch(q2, m2, rr2, b);
          if (b < crb) {
            const float* xp = xl + c * 64u * EPL + 4u * lane;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float4 xv = *reinterpret_cast<const float4*>(xp + 256 * i);
              const float4 xw = UPS == 2 ? *reinterpret_cast<const float4*>(xp + 256 * (i + 4)) : xv;
              kd |= F::kinds(LC, q[i], m, i, xv, xw);
              if constexpr (DUAL) kd2 |= F::kinds(LC, q2[i], m2, i, xv, xw);
            }
          }
        }
        auto value = [&](uint32_t k) {
          const bool nan = __ballot((k & 1u) != 0) != 0, pinf = __ballot((k & 2u) != 0) != 0,
                     ninf = __ballot((k & 4u) != 0) != 0;
          return (nan || (pinf && ninf) || !(pinf || ninf)) ? __builtin_nanf("")
                                                             : (pinf ? __builtin_inff() : -__builtin_inff());
        };
        // with the fused RMSNorm, 1 / rms is 0 (or NaN) here: every row is NaN,
        // as the reference's x / rms (inf / inf at the infinity) makes it
        const float y0 = value(kd) * inv, y1 = DUAL ? value(kd2) * inv : 0.f;
        if (lane == 0) {
          const uint32_t o = v - g.row_begin;
          if (EPI == EPI_STORE) g.y[o] = y0;
          else if (EPI == EPI_RESIDUAL) g.y[o] = g.res[o] + y0;
          else g.y[o] = y0 / (1.0f + expf(-y0)) * y1;
        }
      }
    }
    return;
  }
  }

  float acc[U], acc2[U];
#pragma unroll
  for (int u = 0; u < U; ++u) { acc[u] = 0.f; acc2[u] = 0.f; }
  uint32_t done = 0;  // tasks this wavefront has finished

  // One step: decode LPW chunks of U rows against x (digit planes when
  // MODE::value, else floats), then finish the rows when the task ends.
  auto consume = [&](auto mode, const Step& B, uint32_t tt, uint32_t ss) {
    constexpr bool DIG = IXE && decltype(mode)::value;
#pragma unroll
    for (int l = 0; l < LPW; ++l) {
      // Lanes past the end of the row (a partial last chunk, or a chunk past
      // nchunk when LPW does not divide it) decode zeros against a clamped,
      // in-bounds slice of x and keep their sums by a select.
      const uint32_t c = ss * LPW + l, cx = c < nchunk ? c : nchunk - 1u;
      const bool valid = c * 1024u + 16u * lane < crb;
      if constexpr (DIG) {
        if constexpr (IXE) {  // only formats with idot / ifinish
        nv_u32x4 P[PK_PLANES * UPS];
        float2 ui[UPS];
#pragma unroll
        for (uint32_t h = 0; h < UPS; ++h) {
#pragma unroll
          for (uint32_t p = 0; p < (uint32_t)PK_PLANES; ++p)
            P[PK_PLANES * h + p] =
                *reinterpret_cast<const nv_u32x4*>(xdig + ((cx * UPS + h) * PK_PLANES + p) * 1024u + 16u * lane);
          ui[h] = xinfo[(cx * 64u + lane) * UPS + h];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          int S[UPS][PK_PLANES] = {};
          F::idot(LC, B.q[u][l], P, S);
          const float f = F::ifinish(LC, B.m[u][l], S, ui);
          acc[u] = valid ? acc[u] + f : acc[u];
          if constexpr (DUAL) {
            int S2[UPS][PK_PLANES] = {};
            F::idot(LC, B.q2[u][l], P, S2);
            const float f2 = F::ifinish(LC, B.m2[u][l], S2, ui);
            acc2[u] = valid ? acc2[u] + f2 : acc2[u];
          }
        }
        }
      } else {
        const float* xp = xl + cx * 64u * EPL + 4u * lane;
        float s0[U], s1[U], t0[U], t1[U];
#pragma unroll
        for (int u = 0; u < U; ++u) { s0[u] = 0.f; s1[u] = 0.f; t0[u] = 0.f; t1[u] = 0.f; }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 xv = *reinterpret_cast<const float4*>(xp + 256 * i);
          float4 xw = xv;
          if (UPS == 2) xw = *reinterpret_cast<const float4*>(xp + 256 * (i + 4));
#pragma unroll
          for (int u = 0; u < U; ++u) {
            F::word(LC, B.q[u][l][i], B.m[u][l], i, xv, xw, s0[u], s1[u]);
            if constexpr (DUAL) F::word(LC, B.q2[u][l][i], B.m2[u][l], i, xv, xw, t0[u], t1[u]);
          }
        }
        const uint32_t ui = (cx * 64u + lane) * UPS;
        const float xs0 = xsum_l[ui], xs1 = UPS == 2 ? xsum_l[ui + 1u] : 0.f;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float f = F::finish(LC, B.m[u][l], s0[u], s1[u], xs0, xs1);
          acc[u] = valid ? acc[u] + f : acc[u];
          if constexpr (DUAL) {
            const float f2 = F::finish(LC, B.m2[u][l], t0[u], t1[u], xs0, xs1);
            acc2[u] = valid ? acc2[u] + f2 : acc2[u];
          }
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
  // the buffer freed by the previous step.  The only exit is the uniform
  // check at the top of each step, so every buffer is consumed (its loads
  // waited for) before it is refilled.
  auto run = [&](auto mode) {
    if constexpr (ALLF) {  // at most NB steps per wavefront (the launch sees to it)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (ct >= ntask) return;
        consume(mode, buf[b], ct, cs);
        advance(ct, cs);
      }
      return;
    }
    for (;;) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (ct >= ntask) return;
        fetch(buf[(b + NB - 1) % NB], ft, fs);
        advance(ft, fs);
        consume(mode, buf[b], ct, cs);
        advance(ct, cs);
      }
    }
  };
  run(std::integral_constant<bool, IXE>());
}

// GGUF blocks -> packed layout, one thread per block (install-time only).
// Block i (row-major over rows and blocks) lands at i * (region bytes per
// block) in every region.
template <uint32_t T>
__global__ __launch_bounds__(256) void pack_blocks(const uint8_t* __restrict__ raw, uint8_t* __restrict__ packed,
                                                   uint64_t nblocks) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nblocks) return;
  constexpr uint32_t BS = Fmt<T>::BS;
  const uint8_t* b = raw + i * BS;
  auto copy = [&](uint8_t* dst, const uint8_t* src, uint32_t n) {
    for (uint32_t k = 0; k < n; ++k) dst[k] = src[k];
  };
  if constexpr (T == T_Q8_0 || T == T_Q4_0) {
    constexpr uint32_t CB = BS - 2;
    copy(packed + nblocks * CB + 2 * i, b, 2);  // f16 scale
    copy(packed + i * CB, b + 2, CB);           // codes
  } else if constexpr (T == T_Q4_K) {
    copy(packed + nblocks * 128 + 16 * i, b, 16);  // d, dmin, scales[12]
    copy(packed + i * 128, b + 16, 128);           // qs
  } else {
    uint8_t* qh = packed + nblocks * 128;
    uint8_t* sc = qh + nblocks * 64;
    uint8_t* d = sc + nblocks * 16;
    copy(packed + i * 128, b, 128);  // ql
    copy(qh + i * 64, b + 128, 64);
    copy(sc + i * 16, b + 192, 16);
    copy(d + i * 2, b + 208, 2);
  }
}

// ------------------------------------------------------------------ host side

bool packed_type(uint32_t t) { return t == T_Q8_0 || t == T_Q4_0 || t == T_Q4_K || t == T_Q6_K; }

static uint32_t pk_qk(uint32_t t) { return (t == T_Q4_K || t == T_Q6_K) ? 256u : 32u; }
static uint32_t pk_epb(uint32_t t) { return t == T_Q8_0 ? 1u : 2u; }

// Region k of format t: bytes per row.
static uint64_t pk_row_bytes(uint32_t t, int k, uint64_t in) {
  switch (t) {
    case T_Q8_0: return PkFmt<T_Q8_0>::row_bytes(k, in);
    case T_Q4_0: return PkFmt<T_Q4_0>::row_bytes(k, in);
    case T_Q4_K: return PkFmt<T_Q4_K>::row_bytes(k, in);
    default: return PkFmt<T_Q6_K>::row_bytes(k, in);
  }
}
static int pk_nreg(uint32_t t) { return t == T_Q6_K ? 4 : 2; }

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

static uint64_t pk_nchunk(uint32_t t, uint64_t in_dim) { return (in_dim / pk_epb(t) + 1023) / 1024; }

PkPlan plan_packed(uint32_t t, uint64_t in_dim) {
  PkPlan p{};
  if (!packed_type(t) || in_dim == 0 || in_dim % pk_qk(t) != 0 || in_dim > (1u << 24)) return p;
  const uint64_t nchunk = pk_nchunk(t, in_dim), ups = pk_epb(t), epl = 16 * ups;
  const uint64_t lds = (nchunk * 64 * epl + nchunk * 64 * ups) * 4;
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
// one cache per kernel (a few distinct sizes per model).  A miss runs the
// one-time setup (dynamic LDS attribute, occupancy query) and is refused (-1)
// while st is being captured.
struct PkOccCache {
  std::mutex mu;
  uint32_t keys[16];
  int vals[16];
  int n = 0;
  uint32_t attr = 0;  // dynamic LDS the kernel has been opened up to (above 64 KiB)
};
static int pk_occupancy(PkOccCache& c, const void* kern, int nt, uint32_t lds, hipStream_t st) {
  std::lock_guard<std::mutex> lock(c.mu);
  for (int i = 0; i < c.n; ++i)
    if (c.keys[i] == lds) return c.vals[i];
  if (setup_outside_capture(st) != hipSuccess) return -1;
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

// Name of the matvec_packed instance the calling thread launched (or, in a
// planning pass, would launch) last, spelled as the profiler's kernel trace
// spells it, so that a measurement can be matched to the kernel that ran.
static thread_local char t_last_kernel[128];
template <uint32_t T, int EPI, bool NORM, int U, int LPW, int NB, int NT, bool IX, bool ALLF, bool MRG>
static void note_kernel() {
  auto b = [](bool v) { return v ? "true" : "false"; };
  snprintf(t_last_kernel, sizeof t_last_kernel, "void rf::matvec_packed<%uu, %d, %s, %d, %d, %d, %d, %s, %s, %s>(rf::PkArgs)",
           T, EPI, b(NORM), U, LPW, NB, NT, b(IX), b(ALLF), b(MRG));
}
const char* last_packed_kernel() { return t_last_kernel; }
void clear_last_packed_kernel() { t_last_kernel[0] = 0; }

// x as digit planes on the launches with >= 24 KiB of codes per wavefront
// (1), on every Q8_0 / Q4_0 launch whose LDS holds them (2), or float x
// everywhere (0, default): rf_tune_matvec_digits.  Measured A/B on one box,
// 8B gate/up: 3 planes 21.6-21.9 us; 4 planes 22.3-22.5 us; float x
// 22.4-22.5 us.  With 4 planes the digits no longer pay, so float x, which
// is the reference's arithmetic up to summation order, is the default.
static int g_digits = 0;
void set_matvec_digits(int mode) { g_digits = mode; }
int matvec_digits() { return g_digits; }

// LDS of the digit-plane variant: PK_PLANES bytes per element and a float2
// per 16-element unit, which also holds the float layout it falls back to.
static uint64_t pk_digit_lds(uint32_t t, uint64_t in_dim) {
  const uint64_t nchunk = pk_nchunk(t, in_dim), ups = pk_epb(t);
  return nchunk * ups * (1024u * PK_PLANES) + nchunk * 64u * ups * 8u;
}

// Grid: a whole number k of workgroups per CU (a CU with one workgroup more
// than its neighbours sets the launch time), k just large enough for about
// four rows per wavefront, at most the occupancy.  Timed on the 8B and 70B
// shapes against the fullest grid (CUs x occupancy): Q/K/V 6144x4096 8.3 vs
// 9.3 us (Q8_0), 6.3 vs 7.1 us (Q4_0); Q4_0 gate/up 15.8 vs 16.8 us; the
// other shapes within 0.2 us.
// Workgroups: whole rounds of one per CU, enough for about `per` tasks per
// wavefront, at most the kernel's occupancy.  Q8_0 gate/up launches and rows
// of up to 2048 inputs aim at 2 (8B gate/up: 768 workgroups, its occupancy,
// instead of 512, 21.5 against 21.9 us back to back, decode 545 against 540
// tok/s; the d-2048 model's gate/up 8.57 against 8.69 us); the 8B's other
// launches keep 4 (with 2: Q/K/V 7.75 against 7.30 us), and so do the other
// formats' gate/up (with 2: Q4_K 17.26 / Q4_0 16.15 against 17.30 / 16.17 us,
// Q6_K 20.72 against 20.61).
static uint64_t pk_grid(uint64_t tasks, uint64_t nw, int occ, int epi, uint64_t per = 4) {
  const uint64_t cus = (uint64_t)pk_cu_count();
  const uint64_t want = (tasks + nw - 1) / nw;
  uint64_t k = (tasks + cus * nw * per - 1) / (cus * nw * per);
  if (k < 1) k = 1;
  if (k > (uint64_t)occ) k = (uint64_t)occ;
  uint64_t grid = cus * k < want ? cus * k : want;
  if (epi == EPI_RESIDUAL) {  // at most PK_RES_SLOTS tasks per wavefront (residuals staged in LDS)
    const uint64_t need = (tasks + nw * PK_RES_SLOTS - 1) / (nw * PK_RES_SLOTS);
    if (grid < need) grid = need;
  }
  return grid;
}

template <uint32_t T, int EPI, bool NORM, int LPW, int NB, int NT>
static hipError_t launch_pk(const PkArgs& a, uint32_t lds, hipStream_t st) {
  constexpr int U = 1;
  static PkOccCache cache, cache_ix;  // one per kernel variant
  auto kern = matvec_packed<T, EPI, NORM, U, LPW, NB, NT, false>;
  const int occ = pk_occupancy(cache, reinterpret_cast<const void*>(kern), NT, lds, st);
  if (occ < 0) return hipErrorStreamCaptureUnsupported;
  if (occ < 1) return hipErrorInvalidConfiguration;
  const uint64_t tasks = (a.rows_total + U - 1) / U, nw = NT / 64;
  uint64_t grid = pk_grid(tasks, nw, occ, EPI, ((EPI == EPI_SWIGLU && T == T_Q8_0) || a.in_dim <= 2048) ? 2 : 4);
  // Q8_0 / Q4_0 take the int8 digit planes of x when a wavefront's rows hold
  // at least 24 KiB of codes: their split costs each workgroup a longer
  // prologue, which the cheaper decode repays only over that many bytes
  // (timed: gate/up 14336x4096 x2 21.7-21.9 vs 22.7-22.9 us, the 70B-shape
  // 28672x8192 42.0 vs 43.5 us, the 8B output rows -3%; Q/K/V, o-proj and a
  // single 14336x4096 Q4_0 matrix 0.15-1.5 us slower with them).  The digit
  // variant has its own LDS size, occupancy and grid.
  if constexpr (PkFmt<T>::INTX) {
    const uint64_t rows_pw = (tasks * U + grid * nw - 1) / (grid * nw);
    const uint64_t code_bytes = rows_pw * a.in_dim / PkFmt<T>::EPB * (EPI == EPI_SWIGLU ? 2 : 1);
    const uint64_t lds_ix = pk_digit_lds(T, a.in_dim);
    const bool want = g_digits == 2 || (g_digits == 1 && code_bytes >= 24576);
    if (want && lds_ix + PK_STATIC_LDS <= pk_lds_limit()) {
      auto kix = matvec_packed<T, EPI, NORM, U, LPW, NB, NT, true>;
      const int occ_ix = pk_occupancy(cache_ix, reinterpret_cast<const void*>(kix), NT, (uint32_t)lds_ix, st);
      if (occ_ix < 0) return hipErrorStreamCaptureUnsupported;
      if (occ_ix < 1) return hipErrorInvalidConfiguration;
      note_kernel<T, EPI, NORM, U, LPW, NB, NT, true, false, false>();
      RF_KLAUNCH(kix, dim3((uint32_t)pk_grid(tasks, nw, occ_ix, EPI)), dim3(NT), (uint32_t)lds_ix, st, a);
      return hipGetLastError();
    }
  }
  note_kernel<T, EPI, NORM, U, LPW, NB, NT, false, false, false>();
  RF_KLAUNCH(kern, dim3((uint32_t)grid), dim3(NT), lds, st, a);
  return hipGetLastError();
}

// All-in-flight launches (matvec_packed<..., ALLF>): when a row fits one
// step (LPW = the row's chunks) and the grid gives every wavefront one row,
// the wavefront requests it before the x prologue.  rf_tune_packed_inflight
// switches them off (0) or on (1, default).
static int g_inflight = 1;
void set_packed_inflight(int mode) { g_inflight = mode; }
int packed_inflight() { return g_inflight; }

template <uint32_t T, int EPI, bool NORM, int LPW, int NB>
static hipError_t launch_pk_all_nb(const PkArgs& a, uint32_t lds, uint64_t grid, hipStream_t st) {
  note_kernel<T, EPI, NORM, 1, LPW, NB, 512, false, true, false>();
  RF_KLAUNCH((matvec_packed<T, EPI, NORM, 1, LPW, NB, 512, false, true>), dim3((uint32_t)grid), dim3(512),
                     lds, st, a);
  return hipGetLastError();
}

// One row per wavefront: the grid is a wavefront per row when the NB = 1
// instance's occupancy holds that many and the two-step ring would give at
// most 2 rows per wavefront (measured on the 8B shapes, Q8_0, A/B on one box:
// o-proj 4096x4096 7.1 -> 6.6 us; Q/K/V with one row per wavefront in 768
// workgroups 8.73 against 8.44 us for the ring's 3 rows in 256; with 1.5
// rows per wavefront 8.33 against 8.21; the 14336-wide down projection 15.5
// against 13.7 us, its x staged in twice as many workgroups, so neither
// takes this shape; nor do Q8_0 rows of 2048 inputs, two chunks (the d-2048
// model's Q/K/V 4.19 / 4.25 against 4.07 / 4.08 us, decode 2,175 against
// 2,181 tok/s), or of 8192, eight chunks (its down projection: 6.3 against
// 5.9 us)).  *done stays false otherwise.
template <uint32_t T, int EPI, bool NORM, int LPW>
static hipError_t launch_pk_all(const PkArgs& a, uint32_t lds, hipStream_t st, bool* done) {
  *done = false;
  static PkOccCache cache;
  auto k1 = matvec_packed<T, EPI, NORM, 1, LPW, 1, 512, false, true>;
  const int occ = pk_occupancy(cache, reinterpret_cast<const void*>(k1), 512, lds, st);
  if (occ < 0) return hipErrorStreamCaptureUnsupported;
  if (occ < 1) return hipSuccess;
  const uint64_t nw = 8, cus = (uint64_t)pk_cu_count(), tasks = a.rows_total;
  const uint64_t grid = (tasks + nw - 1) / nw;
  // the ring's grid would give at most 2 rows per wavefront (o-proj); at 3
  // (Q/K/V) the ring's 256 workgroups beat 768 one-row ones
  if (grid > cus * (uint64_t)occ || tasks > 2 * cus * nw) return hipSuccess;
  *done = true;
  return launch_pk_all_nb<T, EPI, NORM, LPW, 1>(a, lds, grid, st);
}

// The single-step launch above with x merged from attention chunk records
// (matvec_packed<..., MRG>): Q8_0 rows of 2 or 4 chunks, Q4_0 / Q4_K / Q6_K rows of 1 or 2,
// with the MRG kernel's own occupancy and LDS (x, its unit sums, then the
// records' factors and the heads' 1 / L).
// hipErrorNotSupported when the shape does not take it;
// with launch false it only says so.
static bool pk_merge_shape(uint32_t t, uint64_t in_dim, uint32_t nsplit, uint32_t qh, uint32_t hd, uint32_t* lds) {
  const PkPlan p = plan_packed(t, in_dim);
  if (!p.ok || !g_inflight) return false;
  if (t == T_Q8_0 || t == T_Q4_0) {
    if (g_digits == 2) return false;  // digit planes everywhere: no float-x launch
  }
  const uint64_t nchunk = pk_nchunk(t, in_dim);
  if (!((t == T_Q8_0 && (nchunk == 2 || nchunk == 4)) || ((t == T_Q4_0 || t == T_Q4_K || t == T_Q6_K) && nchunk <= 2)))
    return false;
  if (hd < 16 || (hd & (hd - 1)) != 0 || (uint64_t)qh * hd != in_dim) return false;
  if (nsplit < 1 || nsplit > 8 || qh > 64) return false;  // 8 lanes per head's chunk records
  if (2 * nchunk * 64 * pk_epb(t) > 512) return false;  // two threads per unit of 16 elements
  const uint64_t l = p.lds_bytes + (uint64_t)nsplit * qh * 4 + (uint64_t)qh * 4;  // factors, 1 / L
  if (l + PK_STATIC_LDS > pk_lds_limit()) return false;
  *lds = (uint32_t)l;
  return true;
}

template <uint32_t T, int LPW>
static hipError_t launch_pk_merge(const PkArgs& a, uint32_t lds, bool launch, hipStream_t st) {
  static PkOccCache cache;
  auto k = matvec_packed<T, EPI_RESIDUAL, false, 1, LPW, 1, 512, false, true, true>;
  const int occ = pk_occupancy(cache, reinterpret_cast<const void*>(k), 512, lds, st);
  if (occ < 0) return hipErrorStreamCaptureUnsupported;
  const uint64_t nw = 8, cus = (uint64_t)pk_cu_count(), tasks = a.rows_total;
  const uint64_t grid = (tasks + nw - 1) / nw;
  if (occ < 1 || grid > cus * (uint64_t)occ || tasks > 2 * cus * nw) return hipErrorNotSupported;
  if (!launch) return hipSuccess;
  note_kernel<T, EPI_RESIDUAL, false, 1, LPW, 1, 512, false, true, true>();
  RF_KLAUNCH(k, dim3((uint32_t)grid), dim3(512), lds, st, a);
  return hipGetLastError();
}

// LPW = the row's chunks (one step per row): Q8_0 rows of 2048 or 4096
// inputs, Q4_0 / Q4_K / Q6_K rows of up to 4096 (Q6_K: 110 VGPRs; an
// all-Q6_K 8B model decodes at 534 against 517 tok/s with the merge kernel).
static hipError_t launch_pk_merge_t(uint32_t t, const PkArgs& a, uint32_t lds, bool launch, hipStream_t st) {
  const uint64_t nchunk = pk_nchunk(t, a.in_dim);
  switch (t) {
    case T_Q8_0:
      return nchunk == 4 ? launch_pk_merge<T_Q8_0, 4>(a, lds, launch, st) : launch_pk_merge<T_Q8_0, 2>(a, lds, launch, st);
    case T_Q4_0:
      return nchunk == 2 ? launch_pk_merge<T_Q4_0, 2>(a, lds, launch, st) : launch_pk_merge<T_Q4_0, 1>(a, lds, launch, st);
    case T_Q4_K:
      return nchunk == 2 ? launch_pk_merge<T_Q4_K, 2>(a, lds, launch, st) : launch_pk_merge<T_Q4_K, 1>(a, lds, launch, st);
    case T_Q6_K:
      return nchunk == 2 ? launch_pk_merge<T_Q6_K, 2>(a, lds, launch, st) : launch_pk_merge<T_Q6_K, 1>(a, lds, launch, st);
    default: return hipErrorNotSupported;
  }
}

hipError_t pk_merge_supported(uint32_t t, uint64_t in_dim, uint64_t rows, uint32_t nsplit, uint32_t qh, uint32_t hd,
                              hipStream_t st) {
  uint32_t lds = 0;
  if (rows == 0 || rows > 0xFFFFFFFFull || !pk_merge_shape(t, in_dim, nsplit, qh, hd, &lds))
    return hipErrorNotSupported;
  PkArgs a{};
  a.rows_total = (uint32_t)rows;
  a.in_dim = (uint32_t)in_dim;
  return launch_pk_merge_t(t, a, lds, false, st);
}

// Launch shape, from timing the 8B projections (Q8_0 and Q4_0; 4096 and
// 14336 inputs): one row per wavefront; LPW = chunks per step, up to 4 (2 for
// gate/up, whose step loads two matrices; Q6_K, with three more loads per
// chunk, one less doubling); 1024-thread workgroups when x fills more than
// 40 KB of LDS (two resident workgroups then still give 32 wavefronts per
// CU), else 512 (always 512 for Q6_K gate/up).  Two step buffers: a third
// for the 8B logits rows (97 instead of 77 VGPRs) took them from 85.3 to
// 89.1 us; steps of 8 chunks for the 14336-wide down projection (119
// VGPRs) from 12.5 to 14.1 us.
template <uint32_t T, int EPI, bool NORM>
static hipError_t launch_pk_l(const PkArgs& a, uint32_t lds, hipStream_t st) {
  const uint64_t nchunk = pk_nchunk(T, a.in_dim);
  // All-in-flight shapes: single-matrix float-x launches whose rows are 4
  // chunks (Q8_0) or 2 (Q4_0, Q4_K): in_dim 4096.
  if constexpr (EPI != EPI_SWIGLU && T != T_Q6_K) {
    bool done = false;
    hipError_t e = hipSuccess;
    if (g_inflight && !(PkFmt<T>::INTX && g_digits == 2)) {
      if constexpr (T == T_Q8_0) {
        if (nchunk == 4) e = launch_pk_all<T, EPI, NORM, 4>(a, lds, st, &done);
      } else {
        if (nchunk == 2) e = launch_pk_all<T, EPI, NORM, 2>(a, lds, st, &done);
      }
    }
    if (done || e != hipSuccess) return e;
  }
  uint32_t pref = EPI == EPI_SWIGLU ? 2 : 4;
  if (T == T_Q6_K) pref /= 2;
  uint32_t lpw = 1;
  while (lpw * 2 <= pref && lpw * 2 <= nchunk) lpw *= 2;
  // Q6_K gate/up keeps 512 threads: its two streams of four regions do not
  // fit the 128 VGPRs of a 1024-thread workgroup (that form spilled to
  // scratch), so it is never instantiated.
  constexpr bool WIDE = !(T == T_Q6_K && EPI == EPI_SWIGLU);
  const bool big = WIDE && lds > 40960;
  switch (lpw * 2 + (big ? 1 : 0)) {
    case 2: return launch_pk<T, EPI, NORM, 1, 2, 512>(a, lds, st);
    case 3:
      if constexpr (WIDE) return launch_pk<T, EPI, NORM, 1, 2, 1024>(a, lds, st);
      return hipErrorInvalidValue;
    case 4: return launch_pk<T, EPI, NORM, 2, 2, 512>(a, lds, st);
    case 5:
      if constexpr (WIDE) return launch_pk<T, EPI, NORM, 2, 2, 1024>(a, lds, st);
      return hipErrorInvalidValue;
    case 8:
      if constexpr (T != T_Q6_K && EPI != EPI_SWIGLU) return launch_pk<T, EPI, NORM, 4, 2, 512>(a, lds, st);
      return hipErrorInvalidValue;
    case 9:
      if constexpr (T != T_Q6_K && EPI != EPI_SWIGLU) return launch_pk<T, EPI, NORM, 4, 2, 1024>(a, lds, st);
      return hipErrorInvalidValue;
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
                                float eps, uint64_t in_dim, int epi, hipStream_t st, int32_t* advance,
                                const PkMerge* mrg) {
  const PkPlan p = plan_packed(t, in_dim);
  if (!p.ok || nseg < 1 || nseg > 3) return hipErrorInvalidValue;
  uint32_t mlds = 0;
  if (mrg) {
    if (epi != EPI_RESIDUAL || norm_w || nseg != 1 || !mrg->ws || !mrg->d_pos ||
        (reinterpret_cast<uintptr_t>(mrg->ws) & 15u) != 0)
      return hipErrorInvalidValue;
    if (!pk_merge_shape(t, in_dim, mrg->nsplit, mrg->qh, mrg->hd, &mlds)) return hipErrorNotSupported;
  }
  if (!al16(x) || (norm_w && !al16(norm_w))) return hipErrorInvalidValue;
  const bool dual = epi == EPI_SWIGLU;
  const int nreg = pk_nreg(t);
  PkArgs a{};
  uint64_t total = 0;
  for (int i = 0; i < nseg; ++i) {
    const PkSegDesc& d = segs[i];
    if (d.row_start + d.rows > d.matrix_rows) return hipErrorInvalidValue;
    if (dual && !d.packed_up) return hipErrorInvalidValue;
    uint64_t off = 0;  // region k starts after regions 0..k-1 of all matrix rows
    for (int k = 0; k < nreg; ++k) {
      const uint64_t rb = pk_row_bytes(t, k, in_dim);
      a.seg[i].reg[k] = static_cast<const uint8_t*>(d.packed) + off + d.row_start * rb;
      if (dual) a.seg[i].reg_up[k] = static_cast<const uint8_t*>(d.packed_up) + off + d.row_start * rb;
      off += d.matrix_rows * rb;
    }
    // 16-byte loads from region 0 (and Q4_K's headers, Q6_K's qh and scales)
    for (int k = 0; k < nreg; ++k) {
      const bool wide = k == 0 || t == T_Q4_K || (t == T_Q6_K && k < 3);
      if (wide && (!al16(a.seg[i].reg[k]) || (dual && !al16(a.seg[i].reg_up[k])))) return hipErrorInvalidValue;
    }
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
  a.advance = advance;
  if (mrg) {
    a.mws = mrg->ws;
    a.m_pos = mrg->d_pos;
    a.m_nsplit = mrg->nsplit;
    a.m_qh = mrg->qh;
    a.m_hd_log2 = (uint32_t)__builtin_ctz(mrg->hd);
    return launch_pk_merge_t(t, a, mlds, true, st);
  }
  switch (t) {
    case T_Q8_0: return launch_pk_t<T_Q8_0>(a, p.lds_bytes, epi, norm_w != nullptr, st);
    case T_Q4_0: return launch_pk_t<T_Q4_0>(a, p.lds_bytes, epi, norm_w != nullptr, st);
    case T_Q4_K: return launch_pk_t<T_Q4_K>(a, p.lds_bytes, epi, norm_w != nullptr, st);
    case T_Q6_K: return launch_pk_t<T_Q6_K>(a, p.lds_bytes, epi, norm_w != nullptr, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_pack(uint32_t t, const void* raw, void* packed, uint64_t rows, uint64_t in_dim, hipStream_t st) {
  if (!packed_type(t) || in_dim % pk_qk(t) != 0) return hipErrorInvalidValue;
  const uint64_t n = rows * (in_dim / pk_qk(t));
  if (n == 0) return hipSuccess;
  const uint32_t gb = n / rows == in_dim / pk_qk(t) ? grid_blocks(n, 256) : 0u;
  if (!gb) return hipErrorInvalidValue;
  const dim3 grid(gb);
  const uint8_t* r = static_cast<const uint8_t*>(raw);
  uint8_t* o = static_cast<uint8_t*>(packed);
  switch (t) {
    case T_Q8_0: RF_KLAUNCH(pack_blocks<T_Q8_0>, grid, dim3(256), 0, st, r, o, n); break;
    case T_Q4_0: RF_KLAUNCH(pack_blocks<T_Q4_0>, grid, dim3(256), 0, st, r, o, n); break;
    case T_Q4_K: RF_KLAUNCH(pack_blocks<T_Q4_K>, grid, dim3(256), 0, st, r, o, n); break;
    default: RF_KLAUNCH(pack_blocks<T_Q6_K>, grid, dim3(256), 0, st, r, o, n); break;
  }
  return hipGetLastError();
}

// Loads this file's code object on the current device (HIP defers that to a
// kernel's first use, which may otherwise fall inside a stream capture) and
// caches the device limits the launchers read.
hipError_t load_module_packed() {
  (void)pk_cu_count();
  (void)pk_lds_limit();
  hipFuncAttributes fa;
  return hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(pack_blocks<T_Q8_0>));
}

}  // namespace rf
