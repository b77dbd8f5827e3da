// rf_device.h — device helpers shared by the gfx950 kernels.
//
// All kernels are compiled with -ffp-contract=off: a multiply followed by an
// add stays two roundings unless fmaf() is written explicitly.  Dequantisation
// relies on that to stay bit-identical with the reference decoders, which never
// fuse (Rust does not contract floating-point expressions).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define RF_WAVE 64

// GGUF half -> float exactly as core/src/quant.rs:40-65 decodes it.  Normal,
// infinite and NaN halves decode to their IEEE value (NaN payload kept, not
// quieted).  The reference's subnormal branch normalises with a test-then-shift
// loop that counts one shift too many, so a subnormal half with fraction f
// decodes to f * 2^-25 — half its IEEE value.  f * 2^-25 is computed exactly
// here (f < 1024 is exact in binary32 and the scale is a power of two), which
// yields the same bits as the reference.
__device__ __forceinline__ float rf_half_to_float(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu;
  const uint32_t frac = h & 0x3FFu;
  if (exp == 0u) {
    const float v = (float)frac * 0x1p-25f;
    return __uint_as_float(__float_as_uint(v) | sign);
  }
  const uint32_t e32 = (exp == 0x1Fu) ? 0xFFu : exp + 112u;
  return __uint_as_float(sign | (e32 << 23) | (frac << 13));
}

// rf_half_to_float through the hardware conversion: the same value for every
// non-NaN input (a subnormal converts exactly to f * 2^-24 and is halved; a
// NaN keeps its payload but comes back quiet).  For hot loops that decode a
// block scale per lane.
__device__ __forceinline__ float rf_half_to_float_fast(uint32_t h) {
  const float f = (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  return (h & 0x7C00u) ? f : f * 0.5f;
}

__device__ __forceinline__ float rf_bf16_to_float(uint32_t h) { return __uint_as_float(h << 16); }

// Unaligned little-endian loads from a byte pointer (any alignment), byte-wise.
__device__ __forceinline__ uint32_t rf_ld_u16(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8);
}

// 32-bit word at byte offset `off` of an LDS buffer whose base is 4-byte
// aligned; `off` may have any alignment.  Reads the two aligned words that
// cover it and shifts with v_alignbyte.  The LDS buffer must be readable for 4
// bytes past the last byte requested.
__device__ __forceinline__ uint32_t rf_lds_u32(const uint8_t* lds, uint32_t off) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(lds + (off & ~3u));
  return __builtin_amdgcn_alignbyte(w[1], w[0], off & 3u);
}

// N consecutive 32-bit words starting at byte offset `off` (any alignment).
template <int N>
__device__ __forceinline__ void rf_lds_words(const uint8_t* lds, uint32_t off, uint32_t (&out)[N]) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(lds + (off & ~3u));
  const uint32_t sh = off & 3u;
  uint32_t raw[N + 1];
#pragma unroll
  for (int i = 0; i < N + 1; ++i) raw[i] = w[i];
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], sh);
}

// Cross-lane data movement inside a 16-lane row with DPP (a VALU operand
// modifier: no LDS round trip, unlike ds_bpermute behind __shfl_xor).
// rf_xchg16<OFF>(v) returns v of a partner lane whose index differs from
// this lane's in bit OFF: quad permutations for OFF = 1, 2 (lane ^ 1,
// lane ^ 2), the half-row mirror (lane ^ 7) for OFF = 4 and the row mirror
// (lane ^ 15) for OFF = 8.  Every lane of the wavefront must be active.
template <int OFF>
__device__ __forceinline__ float rf_xchg16(float v) {
  static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8, "DPP partner bit");
  constexpr int ctrl = OFF == 1 ? 0xB1 : OFF == 2 ? 0x4E : OFF == 4 ? 0x141 : 0x140;
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, true));
}

// Sum (max) over the 16 lanes of each row; every lane gets its row's value.
__device__ __forceinline__ float rf_row16_sum(float v) {
  v += rf_xchg16<1>(v);
  v += rf_xchg16<2>(v);
  v += rf_xchg16<4>(v);
  v += rf_xchg16<8>(v);
  return v;
}

__device__ __forceinline__ float rf_row16_max(float v) {
  v = fmaxf(v, rf_xchg16<1>(v));
  v = fmaxf(v, rf_xchg16<2>(v));
  v = fmaxf(v, rf_xchg16<4>(v));
  v = fmaxf(v, rf_xchg16<8>(v));
  return v;
}

__device__ __forceinline__ float rf_lane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Wavefront sum / max (all 64 lanes active); the result is uniform.
__device__ __forceinline__ float rf_wave_sum(float v) {
  v = rf_row16_sum(v);
  return (rf_lane(v, 0) + rf_lane(v, 16)) + (rf_lane(v, 32) + rf_lane(v, 48));
}

__device__ __forceinline__ float rf_wave_max(float v) {
  v = rf_row16_max(v);
  return fmaxf(fmaxf(rf_lane(v, 0), rf_lane(v, 16)), fmaxf(rf_lane(v, 32), rf_lane(v, 48)));
}

// Hides a value from the optimiser (empty asm, value stays in a VGPR).  A
// packed-nibble word w & 0x0F0F0F0F passed through it keeps its four bytes
// in one register, so each element costs one v_cvt_f32_ubyte{k}; without it
// the mask is folded into a per-element bit-field extract plus a convert.
__device__ __forceinline__ uint32_t rf_opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Unsigned byte k of a word converted to float (v_cvt_f32_ubyte{k}).
__device__ __forceinline__ float rf_ub(uint32_t w, int k) { return (float)((w >> (8 * k)) & 0xFFu); }
// Signed byte k of a word converted to float (one v_cvt_f32_i32 with an SDWA
// sign-extended byte operand).
__device__ __forceinline__ float rf_sb(uint32_t w, int k) { return (float)(int8_t)((w >> (8 * k)) & 0xFFu); }
// Signed codes c in [-2^(b-1), 2^(b-1)) stored as b-bit fields (offset
// binary, c + 2^(b-1)) in the low bits of each byte of w, moved to the top
// of the byte with the sign bit restored: every byte becomes the int8
// 2^(8-b) c, so rf_sb gives the code times an exact power of two.
__device__ __forceinline__ uint32_t rf_top_signed(uint32_t w, int b) {
  const uint32_t top = 0x01010101u * (0xFFu << (8 - b) & 0xFFu);
  return ((w << (8 - b)) & top) ^ 0x80808080u;
}
