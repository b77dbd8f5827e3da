// rf_prefill.hip — batched prompt prefill: the projections of a chunk of
// prompt tokens as one quantized GEMM on the matrix cores, RMSNorm and RoPE +
// K/V cache store per token.
//
// The reference forwards prompt tokens one at a time (inference.rs:580-592,
// ModelExecutor::execute_layer per token, model_executor.rs:102-236); this
// file computes the same per-token arithmetic for up to MM_MAX_TOKENS tokens
// per launch, so each weight byte is read once per chunk instead of once per
// token.
//
// GEMM (mm_packed): Y[t][r] = sum_k W[r][k] X[t][k] on the packed layout of
// Q8_0 / Q4_0 / Q4_K / Q6_K (rf_matvec_packed.hip).  Per 32-element step the
// weight codes are small integers (Q8_0 -128..127, Q4_0 -8..7, Q4_K 0..15,
// Q6_K -32..31), exact in bf16; x (f32) is split into three bf16 pieces
// hi + mid + lo that carry its 24-bit significand (|x - hi - mid - lo| <=
// 2^-26 |x|).  Each product code * piece is exact in f32, so three
// v_mfma_f32_16x16x32_bf16 give the step's partial dot sum_k q_k x_k at f32
// accuracy; the block scale is then applied in f32 as the reference applies
// it per element (quant.rs:977-1327):
//   Q8_0  d * sum q x                      ((q * d) * x summed, quant.rs:977-1029)
//   Q4_0  d * sum (q - 8) x                (quant.rs:875-975)
//   Q4_K  (d*sc) * sum q x - (dmin*m) * sum x   ((d1*q - m1) * x, quant.rs:1085-1137)
//   Q6_K  (d*sc) * sum q x per 16 elements (quant.rs:1195-1327)
// Only the summation order differs from the reference's sequential loop.
//
// MFMA operand layout (16x16x32, A = x tile, B = weight tile): lane l holds
// A row (token) l % 16 and B column (weight row) l % 16, elements 8 (l / 16)
// .. + 7 of the step for both; the result lane l holds D[token 4 (l / 16) + i]
// [row l % 16], i = 0..3, so every value a lane accumulates belongs to its own
// weight row and takes that row's scale.
//
// Workgroup: 12 or 8 wavefronts (mm_pick_wide) x 32 rows (two 16-row tiles)
// x all tokens of the chunk (NTT tiles of 16), over a range of 128-element k
// slices (split-K).
// Each x slice is split once per workgroup while it is staged: three bf16
// planes in LDS (16-byte skew per token row: the 16 token rows of an A read
// fall in distinct banks), read as MFMA operands by all the wavefronts.
// Two slice buffers: the next slice's x (from L2) is loaded while the
// current slice is computed, the weights (from HBM, straight to registers)
// one or two slices ahead (the workgroup shape's ring depth).
// Partial sums of the splits land in a workspace and mm_reduce adds them in
// a fixed order (deterministic) and applies the epilogue.
#include <algorithm>

#include "rf_device.h"
#include "rf_kernels.h"

namespace rf {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t MM_KS = 128;           // k elements per staged x slice
constexpr uint32_t MM_ST = MM_KS / 32;    // 32-element steps per slice
constexpr uint32_t MM_XB = MM_KS + 8;     // LDS bf16 per token row of one x plane (16-byte skew)

struct MmSeg {
  const uint8_t* reg[PK_MAX_REGIONS];  // regions at the segment's first row
  uint32_t rows;                       // rows of the segment
  uint32_t group_begin;                // first workgroup (blockIdx.x) of the segment
  uint32_t col;                        // first partial column of the segment
};
struct MmArgs {
  MmSeg seg[3];
  uint32_t nseg;
  const float* x;  // [n][ldx]
  float* part;     // [nsplit][n][mtot]
  uint32_t n, ldx, in_dim, mtot, nslices, spp;
};

__device__ __forceinline__ uint32_t mm_byte(uint2 w, int k) { return ((k < 4 ? w.x : w.y) >> (8 * (k & 3))) & 0xFFu; }

__device__ __forceinline__ bf16x8 mm_codes(const float (&v)[8]) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (__bf16)v[i];
  return r;
}

// Every load of the GEMM is a raw buffer load over one segment's region (all
// its rows) or over x: an offset at or past the region's size returns zeros
// and reads nothing, so the loads of a partial slice, of the rows past a
// segment and of the slices past a split are issued unconditionally.  (With
// those loads behind branches the compiler could not count the loads in
// flight and waited for all of them before each slice's MFMAs: the next
// slice's prefetched weights and x arrived before the current slice could
// start.)
typedef __amdgpu_buffer_rsrc_t MmRsrc;
constexpr int MM_RSRC_WORD3 = 0x00020000;  // raw buffer, 32-bit data (as the decode kernel's)
constexpr uint32_t MM_OOR = 0xFFFFFFF0u;   // past every region the host allows (< 2^31 bytes)

__device__ __forceinline__ MmRsrc mm_rsrc(const void* base, uint64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int32_t)bytes, MM_RSRC_WORD3);
}
__device__ __forceinline__ uint2 mm_ld8(MmRsrc r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint4 mm_ld16(MmRsrc r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t mm_ld2(MmRsrc r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// The MM_ST f16 scales of a slice of one row, kept as loaded: scale j in
// half j & 1 of word j >> 1, taken out only when step j uses it (mm_scale).
// SC8 (K a multiple of 128: whole slices, the four scales 8-byte aligned): one
// 8-byte load; else one 2-byte load per step.  Splitting the halves right
// after the load made every wavefront wait there for all its loads in flight,
// the weights of the slices ahead included; two registers instead of four
// also make room for a third wavefront per SIMD.
template <bool SC8>
__device__ __forceinline__ void mm_load_scales(MmRsrc r, uint32_t off, uint32_t nst, uint2& sc) {
  static_assert(MM_ST == 4, "four scales per slice");
  if constexpr (SC8) {
    sc = mm_ld8(r, nst ? off : MM_OOR);
  } else {
    uint32_t h[MM_ST];
#pragma unroll
    for (uint32_t j = 0; j < MM_ST; ++j) h[j] = mm_ld2(r, j < nst ? off + 2u * j : MM_OOR);
    sc = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
  }
}

__device__ __forceinline__ uint32_t mm_scale(uint2 sc, int j) {
  const uint32_t w = j < 2 ? sc.x : sc.y;
  return (j & 1) ? w >> 16 : w & 0xFFFFu;
}

// Bytes of one row in region k of the packed layout (rf_matvec_packed.hip).
__host__ __device__ inline uint64_t mm_row_bytes(uint32_t t, int k, uint64_t K) {
  switch (t) {
    case T_Q8_0: return k == 0 ? K : K / 32 * 2;
    case T_Q4_0: return k == 0 ? K / 2 : K / 32 * 2;
    case T_Q4_K: return k == 0 ? K / 2 : K / 256 * 16;
    default: return k == 0 ? K / 2 : k == 1 ? K / 4 : k == 2 ? K / 256 * 16 : K / 256 * 2;
  }
}

// Per-format weight slice (MM_KS elements of one row) of one lane (element
// group g) and its decode into the B operand of step j.  nst = 0 (a slice
// past the split) loads nothing.
template <uint32_t T> struct MmW;

// Q8_0: two steps per 16-byte load.  For steps 2p and 2p + 1 of a slice the
// lanes of groups 0-1 load codes 16 (g & 1) .. + 15 of block 2p and groups 2-3
// the same codes of block 2p + 1: 64 contiguous bytes of each of 16 rows per
// instruction, half the load instructions of one 8-byte load per step.
// prep(p) swaps the upper 32 lanes' first half with the lower 32 lanes'
// second half (v_permlane32_swap), after which .xy is step 2p's operand and
// .zw step 2p + 1's; lane group g then holds codes 8 mm_kperm(g) .. + 7 of
// its block, and the x operand is read in the same K order.
__device__ __forceinline__ uint32_t mm_kperm(uint32_t g) { return ((g & 1u) << 1) | (g >> 1); }

template <> struct MmW<T_Q8_0> {
  static constexpr uint32_t NREG = 2;
  uint4 c[MM_ST / 2];
  uint2 sc;
  template <bool SC8>
  __device__ void load(const MmRsrc* rs, uint32_t row, uint32_t sl, uint32_t g, uint32_t nst, uint32_t K) {
    const uint32_t cb = row * K + sl * MM_KS + 32u * (g >> 1) + 16u * (g & 1u);
#pragma unroll
    for (uint32_t p = 0; p < MM_ST / 2; ++p) c[p] = mm_ld16(rs[0], 2u * p + (g >> 1) < nst ? cb + 64u * p : MM_OOR);
    mm_load_scales<SC8>(rs[1], (row * (K / 32u) + sl * MM_ST) * 2u, nst, sc);
  }
  __device__ void prep(int p) {
    const auto s0 = __builtin_amdgcn_permlane32_swap(c[p].x, c[p].z, false, false);
    const auto s1 = __builtin_amdgcn_permlane32_swap(c[p].y, c[p].w, false, false);
    c[p] = make_uint4(s0[0], s1[0], s0[1], s1[1]);
  }
  __device__ void step(int j, uint32_t, bf16x8& b, float& d) const {
    const uint4 w = c[j >> 1];
    const uint2 q = (j & 1) ? make_uint2(w.z, w.w) : make_uint2(w.x, w.y);
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = (float)(int)(int8_t)mm_byte(q, k);
    b = mm_codes(v);
    d = rf_half_to_float_fast(mm_scale(sc, j));
  }
};

template <> struct MmW<T_Q4_0> {
  static constexpr uint32_t NREG = 2;
  uint2 c[MM_ST];
  uint2 sc;
  template <bool SC8>
  __device__ void load(const MmRsrc* rs, uint32_t row, uint32_t sl, uint32_t g, uint32_t nst, uint32_t K) {
    const uint32_t blk = row * (K / 32u) + sl * MM_ST;
    const uint32_t cb = blk * 16u + 8u * (g & 1u);
#pragma unroll
    for (uint32_t j = 0; j < MM_ST; ++j) c[j] = mm_ld8(rs[0], j < nst ? cb + 16u * j : MM_OOR);
    mm_load_scales<SC8>(rs[1], blk * 2u, nst, sc);
  }
  // elements 8g..8g+7 of a block: low nibbles of bytes 0-7 / 8-15 (g = 0, 1),
  // high nibbles of the same bytes (g = 2, 3): value nibble - 8
  __device__ void step(int j, uint32_t g, bf16x8& b, float& d) const {
    const int sh = 4 * (int)(g >> 1);
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = (float)((int)((mm_byte(c[j], k) >> sh) & 15u) - 8);
    b = mm_codes(v);
    d = rf_half_to_float_fast(mm_scale(sc, j));
  }
};

// A slice is half a 256-element block: sub-blocks 4 hh .. 4 hh + 3.
template <> struct MmW<T_Q4_K> {
  static constexpr uint32_t NREG = 2;
  uint2 c[2];  // qs bytes 32 (2 hh + i) + 8g .. + 7: sub-blocks 4 hh + 2i (low nibbles), + 1 (high)
  uint4 h;     // d | dmin << 16, scale bytes 0-3, 4-7, 8-11
  uint32_t hh;
  template <bool>
  __device__ void load(const MmRsrc* rs, uint32_t row, uint32_t sl, uint32_t g, uint32_t nst, uint32_t K) {
    const uint32_t blk = row * (K / 256u) + (sl >> 1);
    hh = sl & 1u;
    const uint32_t cb = blk * 128u + 64u * hh + 8u * g;
#pragma unroll
    for (int i = 0; i < 2; ++i) c[i] = mm_ld8(rs[0], nst ? cb + 32u * i : MM_OOR);
    h = mm_ld16(rs[1], nst ? blk * 16u : MM_OOR);
  }
  __device__ uint32_t sbyte(uint32_t i) const {
    const uint32_t w = i < 4 ? h.y : (i < 8 ? h.z : h.w);
    return (w >> (8 * (i & 3u))) & 0xFFu;
  }
  // get_scale_min (quant.rs:216-226) of sub-block 4 hh + j
  __device__ void step(int j, uint32_t, bf16x8& b, float& d1, float& m1) const {
    const int sh = 4 * (j & 1);
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = (float)((mm_byte(c[j >> 1], k) >> sh) & 15u);
    b = mm_codes(v);
    // hh is uniform and j a compile-time index: every byte index is static
    const uint32_t ju = (uint32_t)j, q = 4u + ju;
    uint32_t sc, m;
    if (hh == 0) {
      sc = sbyte(ju) & 63u;
      m = sbyte(ju + 4) & 63u;
    } else {
      sc = (sbyte(q + 4) & 0xFu) | ((sbyte(q - 4) >> 6) << 4);
      m = (sbyte(q + 4) >> 4) | ((sbyte(q) >> 6) << 4);
    }
    const float d = rf_half_to_float_fast(h.x & 0xFFFFu), dmin = rf_half_to_float_fast(h.x >> 16);
    d1 = d * (float)sc;
    m1 = dmin * (float)m;
  }
};

// A slice is one 128-element half hh of a block: steps qq = 0..3 cover
// elements 128 hh + 32 qq + l, l = 0..31 (quant.rs:376-406).
template <> struct MmW<T_Q6_K> {
  static constexpr uint32_t NREG = 4;
  uint2 ql[2];  // [p]: ql bytes 64 hh + 32 p + 8g .. + 7
  uint2 qh;     // qh bytes 32 hh + 8g .. + 7
  uint4 sc;     // 16 int8 scales
  uint32_t d, hh;
  template <bool>
  __device__ void load(const MmRsrc* rs, uint32_t row, uint32_t sl, uint32_t g, uint32_t nst, uint32_t K) {
    const uint32_t blk = row * (K / 256u) + (sl >> 1);
    hh = sl & 1u;
    const uint32_t lb = blk * 128u + 64u * hh + 8u * g;
#pragma unroll
    for (int i = 0; i < 2; ++i) ql[i] = mm_ld8(rs[0], nst ? lb + 32u * i : MM_OOR);
    qh = mm_ld8(rs[1], nst ? blk * 64u + 32u * hh + 8u * g : MM_OOR);
    sc = mm_ld16(rs[2], nst ? blk * 16u : MM_OOR);
    d = mm_ld2(rs[3], nst ? blk * 2u : MM_OOR);
  }
  __device__ float scale(uint32_t i) const {
    const uint32_t w = i < 4 ? sc.x : (i < 8 ? sc.y : (i < 12 ? sc.z : sc.w));
    return (float)(int)(int8_t)((w >> (8 * (i & 3u))) & 0xFFu);
  }
  // q = (ql nibble qq / 2 of byte 64 hh + 32 (qq & 1) + l) | (qh bits 2qq of byte 32 hh + l) << 4, minus 32.
  // Elements l < 16 (groups 0, 1) take scale 8 hh + 2qq, the rest 8 hh + 2qq + 1:
  // b0 holds groups 0-1 (zeros in 2-3), b1 groups 2-3.
  __device__ void step(int qq, uint32_t g, bf16x8& b0, bf16x8& b1, float& d0, float& d1) const {
    const uint2 l = ql[qq & 1];
    const int lsh = 4 * (qq >> 1), hsh = 2 * qq;
    const bool first = g < 2u;
    float v0[8], v1[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int q = (int)(((mm_byte(l, k) >> lsh) & 15u) | (((mm_byte(qh, k) >> hsh) & 3u) << 4)) - 32;
      v0[k] = first ? (float)q : 0.f;
      v1[k] = first ? 0.f : (float)q;
    }
    b0 = mm_codes(v0);
    b1 = mm_codes(v1);
    const float dd = rf_half_to_float_fast(d);
    const uint32_t q2 = 2u * (uint32_t)qq;  // hh uniform, qq compile-time: static indices
    d0 = dd * (hh == 0 ? scale(q2) : scale(8u + q2));
    d1 = dd * (hh == 0 ? scale(q2 + 1u) : scale(9u + q2));
  }
};

// x = hi + mid + lo, each the round-to-nearest bf16 of what remains.
__device__ __forceinline__ void mm_split3(float x, __bf16& hi, __bf16& mid, __bf16& lo) {
  hi = (__bf16)x;
  const float r1 = x - (float)hi;
  mid = (__bf16)r1;
  lo = (__bf16)(r1 - (float)mid);
}

// Two workgroup shapes: wavefronts per workgroup (32 weight rows each) and
// how many slices of weights are in registers at once (DEPTH 3: loaded two
// slices ahead, 2: one).  The x tile (104 KB at 64 tokens) allows one
// workgroup per CU, so the wavefronts of one workgroup are all the latency
// hiding there is.  Wide, 12 wavefronts with a two-slice ring, fits 168
// VGPRs (three per SIMD) and ran Q4_K at 64 tokens 12-32% faster than
// narrow, 8 with a three-slice ring (gate/up 87.5 -> 77.1 us, down 48.2 ->
// 41.1, Q/K/V 29.5 -> 20.0).  Its 384-row workgroups leave too few for some
// shapes (4096 rows: 11, filling 176 of 256 CUs), so each launch takes the
// shape whose split fills the chip better (mm_pick_wide).  Q6_K's four weight
// regions do not fit the wide register budget (63 VGPRs spilled): narrow.
constexpr uint32_t MM_ROWS_NARROW = 8 * 32, MM_ROWS_WIDE = 12 * 32;

template <uint32_t T, int NTT, int NW, int DEPTH, bool SC8>
__global__ __launch_bounds__(64 * NW) void mm_packed(MmArgs a) {
  // Two x slice buffers, each three bf16 planes [3][NT][MM_XB] and (Q4_K)
  // step sums [MM_ST][NT]: slice s + 1 is loaded (x and weights) while slice
  // s is computed, then split into the other buffer; one barrier per slice.
  extern __shared__ __align__(16) __bf16 xsb[];
  constexpr uint32_t NT = NTT * 16, PLANE = NT * MM_XB;
  constexpr uint32_t BUF = 3 * PLANE + (T == T_Q4_K ? MM_ST * NT * 2 : 0);  // bf16 elements per buffer
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t r16 = lane & 15u, g = lane >> 4;
  const uint32_t gx = T == T_Q8_0 ? mm_kperm(g) : g;  // K order of the weight operand's lane groups
  MmSeg s = a.seg[0];
  if (a.nseg > 1 && blockIdx.x >= a.seg[1].group_begin) s = a.seg[1];
  if (a.nseg > 2 && blockIdx.x >= a.seg[2].group_begin) s = a.seg[2];
  const uint32_t row_base = (blockIdx.x - s.group_begin) * (NW * 32u) + wave * 32u;
  uint32_t rowc[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) rowc[rt] = min(row_base + 16u * rt + r16, s.rows - 1u);  // loads stay in bounds
  const uint32_t K = a.in_dim, n = a.n;
  const uint32_t sl0 = blockIdx.y * a.spp, sl1 = min(a.nslices, sl0 + a.spp);
  // staging: thread -> (token st_t, 32-element block st_b, half st_h) of a slice
  const uint32_t st_t = tid >> 3, st_b = (tid >> 1) & 3u, st_h = tid & 1u;
  // steps of slice sl of this split (0 past the split's last slice)
  auto nsteps = [&](uint32_t sl) { return sl < sl1 ? min(MM_ST, (K - sl * MM_KS) / 32u) : 0u; };
  MmRsrc rs[MmW<T>::NREG];
#pragma unroll
  for (int k = 0; k < (int)MmW<T>::NREG; ++k) rs[k] = mm_rsrc(s.reg[k], (uint64_t)s.rows * mm_row_bytes(T, k, K));
  const MmRsrc xr = mm_rsrc(a.x, (uint64_t)n * a.ldx * 4u);
  auto fetch_x = [&](uint32_t sl, float4 (&xv)[4]) {
    const bool live = st_t < n && st_b < nsteps(sl);
    const uint32_t off = (st_t * a.ldx + sl * MM_KS + 32u * st_b + 16u * st_h) * 4u;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(xr, live ? off + 16u * q : MM_OOR, 0, 0);
      xv[q] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
    }
  };
  auto put_x = [&](uint32_t buf, const float4 (&xv)[4]) {
    if (st_t >= NT) return;  // whole groups of 8 threads (one token row)
    __bf16* dst = xsb + buf * BUF + st_t * MM_XB + 32u * st_b + 16u * st_h;
    float sum = 0.f;
    bf16x8 hv[2], mv[2], lv[2];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float e[4] = {xv[q].x, xv[q].y, xv[q].z, xv[q].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        __bf16 h, m, l;
        mm_split3(e[i], h, m, l);
        hv[q >> 1][4 * (q & 1) + i] = h;
        mv[q >> 1][4 * (q & 1) + i] = m;
        lv[q >> 1][4 * (q & 1) + i] = l;
        sum += e[i];
      }
    }
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      *reinterpret_cast<bf16x8*>(dst + 8 * v) = hv[v];
      *reinterpret_cast<bf16x8*>(dst + PLANE + 8 * v) = mv[v];
      *reinterpret_cast<bf16x8*>(dst + 2 * PLANE + 8 * v) = lv[v];
    }
    if constexpr (T == T_Q4_K) {
      sum += __shfl_xor(sum, 1);  // the partner half is in this thread group
      if (st_h == 0) reinterpret_cast<float*>(xsb + buf * BUF + 3 * PLANE)[st_b * NT + st_t] = sum;
    }
  };

  f32x4 acc[2][NTT];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int nt = 0; nt < NTT; ++nt) acc[rt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Weights DEPTH - 1 slices ahead, x one slice ahead.  The ring of weight
  // registers rotates by unrolling the slice loop DEPTH times (a copy of the
  // registers would wait for the loads that fill them).
  static_assert(DEPTH == 2 || DEPTH == 3, "weight ring of two or three slices");
  typedef MmW<T> Wt[2];
  auto load_w = [&](Wt& w, uint32_t sl) {
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) w[rt].template load<SC8>(rs, rowc[rt], sl, g, nsteps(sl), K);
  };
  float4 xv[4];
  // Slice sl with weights w: the next slice's x and the weights of slice
  // sl + DEPTH - 1 (into the buffer slice sl - 1 used) are requested first.
  auto run_slice = [&](uint32_t sl, Wt& w, Wt& refill) {
    const uint32_t cb = (sl - sl0) & 1u, nst = nsteps(sl);
    const bool more = sl + 1 < sl1;
    fetch_x(sl + 1, xv);
    load_w(refill, sl + DEPTH - 1);
    const __bf16* xb = xsb + cb * BUF;
    const float* ss = reinterpret_cast<const float*>(xb + 3 * PLANE);
#pragma unroll
    for (int j = 0; j < (int)MM_ST; ++j) {
      if ((uint32_t)j >= nst) break;
      bf16x8 b[2], b2[2];
      float d[2], e[2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        if constexpr (T == T_Q8_0) {
          if ((j & 1) == 0) w[rt].prep(j >> 1);
        }
        if constexpr (T == T_Q4_K) w[rt].step(j, g, b[rt], d[rt], e[rt]);
        else if constexpr (T == T_Q6_K) w[rt].step(j, g, b[rt], b2[rt], d[rt], e[rt]);
        else w[rt].step(j, g, b[rt], d[rt]);
      }
      // All A operands of the step, then the hi / mid / lo MFMAs of every
      // (row tile, token tile) pair in turn: each MFMA's accumulator input
      // was written 2 NTT (4 NTT for Q6_K) MFMAs earlier, so the chains
      // overlap instead of waiting on each other.
      bf16x8 ax[3][NTT];
#pragma unroll
      for (int nt = 0; nt < NTT; ++nt) {
        const __bf16* ap = xb + (nt * 16u + r16) * MM_XB + 32u * j + 8u * gx;
#pragma unroll
        for (int p = 0; p < 3; ++p) ax[p][nt] = *reinterpret_cast<const bf16x8*>(ap + p * PLANE);
      }
      constexpr int NB = T == T_Q6_K ? 2 : 1;
      f32x4 tmp[NB][2][NTT];
#pragma unroll
      for (int p = 0; p < 3; ++p)
#pragma unroll
        for (int h = 0; h < NB; ++h)
#pragma unroll
          for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int nt = 0; nt < NTT; ++nt) {
              const bf16x8& bw = h == 0 ? b[rt] : b2[rt];
              tmp[h][rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  ax[p][nt], bw, p == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : tmp[h][rt][nt], 0, 0, 0);
            }
#pragma unroll
      for (int nt = 0; nt < NTT; ++nt) {
        float4 sx = make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (T == T_Q4_K) sx = *reinterpret_cast<const float4*>(&ss[j * NT + nt * 16u + 4u * g]);
        const float sxa[4] = {sx.x, sx.y, sx.z, sx.w};
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          f32x4& c = acc[rt][nt];
          const f32x4& t0 = tmp[0][rt][nt];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if constexpr (T == T_Q6_K) c[i] = fmaf(e[rt], tmp[NB - 1][rt][nt][i], fmaf(d[rt], t0[i], c[i]));
            else if constexpr (T == T_Q4_K) c[i] = fmaf(-e[rt], sxa[i], fmaf(d[rt], t0[i], c[i]));
            else c[i] = fmaf(d[rt], t0[i], c[i]);
          }
        }
      }
    }
    if (more) put_x(cb ^ 1u, xv);  // the other buffer's last reader was slice sl - 1, before the last barrier
    __syncthreads();
  };
  Wt wa, wb, wc;
  fetch_x(sl0, xv);
  load_w(wa, sl0);
  if constexpr (DEPTH == 3) load_w(wb, sl0 + 1);
  put_x(0, xv);
  __syncthreads();
  if constexpr (DEPTH == 2) {
    for (uint32_t sl = sl0; sl < sl1; sl += 2) {
      run_slice(sl, wa, wb);
      if (sl + 1 < sl1) run_slice(sl + 1, wb, wa);
    }
  } else {
    for (uint32_t sl = sl0; sl < sl1; sl += 3) {
      run_slice(sl, wa, wc);
      if (sl + 1 < sl1) run_slice(sl + 1, wb, wa);
      if (sl + 2 < sl1) run_slice(sl + 2, wc, wb);
    }
  }
  float* out = a.part + (size_t)blockIdx.y * n * a.mtot + s.col;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const uint32_t r = row_base + 16u * rt + r16;
    if (r >= s.rows) continue;
#pragma unroll
    for (int nt = 0; nt < NTT; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t t = nt * 16u + 4u * g + i;
        if (t < n) out[(size_t)t * a.mtot + r] = acc[rt][nt][i];
      }
  }
}

// Sum of the split partials in split order, then the epilogue:
//   EPI_STORE     y = v (+ bias: the reference adds it after the matvec)
//   EPI_RESIDUAL  y = res + v
//   EPI_SWIGLU    y = silu(v_gate) * v_up  (segment 0 gate, segment 1 up)
struct MmRedSeg {
  float* y;
  const float* res;
  const float* bias;
  uint32_t rows, col, ld;
};
struct MmRedArgs {
  MmRedSeg seg[3];
  uint32_t nseg, nsplit, n, mtot, mcols;
  int epi;
  const float* part;
};

// Sums of the n split partials p[s][0], p[s][stride], ... of NS streams, each
// in split order.  The loads of a batch (MM_RED_BATCH / NS splits of every
// stream) are issued before any of its adds (indices past the last split are
// clamped to it: L2 hits, never added), so a batch costs one memory round
// trip instead of one per split.
constexpr uint32_t MM_RED_BATCH = 16;
__device__ __forceinline__ float4 add4(float4 v, float4 q) {
  return make_float4(v.x + q.x, v.y + q.y, v.z + q.z, v.w + q.w);
}
__device__ __forceinline__ float add4(float v, float q) { return v + q; }
template <int NS, typename V>
__device__ __forceinline__ void mm_split_sums(const V* const (&p)[NS], size_t stride, uint32_t n, V (&v)[NS]) {
  constexpr uint32_t B = MM_RED_BATCH / NS;
#pragma unroll
  for (int i = 0; i < NS; ++i) v[i] = p[i][0];
  for (uint32_t k0 = 1; k0 < n; k0 += B) {
    V q[NS][B];
#pragma unroll
    for (int i = 0; i < NS; ++i)
#pragma unroll
      for (uint32_t j = 0; j < B; ++j) q[i][j] = p[i][min(k0 + j, n - 1u) * stride];
#pragma unroll
    for (int i = 0; i < NS; ++i)
#pragma unroll
      for (uint32_t j = 0; j < B; ++j)
        if (k0 + j < n) v[i] = add4(v[i], q[i][j]);
  }
}

__global__ __launch_bounds__(256) void mm_reduce(MmRedArgs a) {
  const uint64_t e = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (e >= (uint64_t)a.n * a.mcols) return;
  const uint32_t t = (uint32_t)(e / a.mcols), c = (uint32_t)(e % a.mcols);
  MmRedSeg s = a.seg[0];
  if (a.nseg > 1 && c >= a.seg[1].col) s = a.seg[1];
  if (a.nseg > 2 && c >= a.seg[2].col) s = a.seg[2];
  const uint32_t r = c - s.col;
  const size_t stride = (size_t)a.n * a.mtot;
  const size_t o = (size_t)t * s.ld + r;
  const float* pv = a.part + (size_t)t * a.mtot + c;
  if (a.epi == EPI_SWIGLU) {
    const float* p2[2] = {pv, a.part + (size_t)t * a.mtot + a.seg[1].col + r};
    float vu[2];
    mm_split_sums<2>(p2, stride, a.nsplit, vu);
    s.y[o] = vu[0] / (1.0f + expf(-vu[0])) * vu[1];  // silu_reference * up (compute.rs:337-361)
    return;
  }
  // the residual (unused otherwise: the output's own element) requested with the partials
  const float rr = (a.epi == EPI_RESIDUAL ? s.res : s.y)[o];
  const float* p1[1] = {pv};
  float v[1];
  mm_split_sums<1>(p1, stride, a.nsplit, v);
  if (a.epi == EPI_RESIDUAL) {
    s.y[o] = rr + v[0];
  } else {
    s.y[o] = s.bias ? v[0] + s.bias[r] : v[0];
  }
}

// mm_reduce for four consecutive columns per thread (16-byte loads and
// stores), when every segment boundary, row stride and pointer allows it
// (mm_reduce_vec4).  Each column is summed in split order and finished
// exactly as in mm_reduce: the same bits, a quarter of the memory
// instructions.
__global__ __launch_bounds__(256) void mm_reduce4(MmRedArgs a) {
  const uint64_t e = ((uint64_t)blockIdx.x * 256u + threadIdx.x) * 4u;
  if (e >= (uint64_t)a.n * a.mcols) return;
  const uint32_t t = (uint32_t)(e / a.mcols), c = (uint32_t)(e % a.mcols);
  MmRedSeg s = a.seg[0];
  if (a.nseg > 1 && c >= a.seg[1].col) s = a.seg[1];
  if (a.nseg > 2 && c >= a.seg[2].col) s = a.seg[2];
  const uint32_t r = c - s.col;
  const size_t stride = (size_t)a.n * a.mtot / 4;  // float4 units (mtot % 4 == 0)
  const size_t o = (size_t)t * s.ld + r;
  const float4* pv = reinterpret_cast<const float4*>(a.part + (size_t)t * a.mtot + c);
  float4 out;
  if (a.epi == EPI_SWIGLU) {
    const float4* p2[2] = {pv, reinterpret_cast<const float4*>(a.part + (size_t)t * a.mtot + a.seg[1].col + r)};
    float4 vu[2];
    mm_split_sums<2>(p2, stride, a.nsplit, vu);
    const float4 v = vu[0], u = vu[1];
    out = make_float4(v.x / (1.0f + expf(-v.x)) * u.x, v.y / (1.0f + expf(-v.y)) * u.y,
                      v.z / (1.0f + expf(-v.z)) * u.z, v.w / (1.0f + expf(-v.w)) * u.w);
  } else {
    // the residual (unused otherwise: the output's own elements) requested with the partials
    const float4 rr = *reinterpret_cast<const float4*>((a.epi == EPI_RESIDUAL ? s.res : s.y) + o);
    const float4* p1[1] = {pv};
    float4 v[1];
    mm_split_sums<1>(p1, stride, a.nsplit, v);
    out = v[0];
    if (a.epi == EPI_RESIDUAL) {
      out = make_float4(rr.x + v[0].x, rr.y + v[0].y, rr.z + v[0].z, rr.w + v[0].w);
    } else if (s.bias) {
      const float4 b = *reinterpret_cast<const float4*>(s.bias + r);
      out = make_float4(v[0].x + b.x, v[0].y + b.y, v[0].z + b.z, v[0].w + b.w);
    }
  }
  *reinterpret_cast<float4*>(s.y + o) = out;
}

// mm_reduce4's EPI_RESIDUAL for one segment of rows <= 4096 V columns,
// fused with the RMSNorm that follows it: one workgroup per token row,
// thread tid owning columns 4 (tid + 1024 i).  y = res + the partials in
// split order (mm_reduce4's bits), then xn = y / rms(y) * w with
// rms_norm_reference's arithmetic (compute.rs:291-319); the sum of squares
// runs over the row's slots and wavefronts in a fixed order.
template <int V>
__global__ __launch_bounds__(1024) void mm_reduce_norm(MmRedArgs a, const float* __restrict__ w, float eps,
                                                      float* __restrict__ xn) {
  __shared__ float part[16];
  const uint32_t t = blockIdx.x, tid = threadIdx.x;
  const MmRedSeg s = a.seg[0];
  const uint32_t cols = s.rows;
  const size_t stride = (size_t)a.n * a.mtot / 4;  // float4 units (mtot % 4 == 0)
  const float4* pv[V];
  float4 rr[V], v[V];
  uint32_t c[V];
#pragma unroll
  for (int i = 0; i < V; ++i) {
    c[i] = 4u * (tid + 1024u * i);
    const uint32_t cc = c[i] < cols ? c[i] : 0u;  // slots past the row: in bounds, unused
    pv[i] = reinterpret_cast<const float4*>(a.part + (size_t)t * a.mtot + s.col + cc);
    rr[i] = *reinterpret_cast<const float4*>(s.res + (size_t)t * s.ld + cc);
  }
  mm_split_sums<V>(pv, stride, a.nsplit, v);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const float4 y = make_float4(rr[i].x + v[i].x, rr[i].y + v[i].y, rr[i].z + v[i].z, rr[i].w + v[i].w);
    v[i] = y;
    if (c[i] < cols) {
      *reinterpret_cast<float4*>(s.y + (size_t)t * s.ld + c[i]) = y;
      ss = fmaf(y.x, y.x, ss);
      ss = fmaf(y.y, y.y, ss);
      ss = fmaf(y.z, y.z, ss);
      ss = fmaf(y.w, y.w, ss);
    }
  }
  ss = rf_wave_sum(ss);
  if ((tid & 63u) == 0) part[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < 16; ++k) tot += part[k];
  const float rms = sqrtf(tot / (float)cols + eps);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    if (c[i] >= cols) break;
    const float4 wv = *reinterpret_cast<const float4*>(w + c[i]);
    *reinterpret_cast<float4*>(xn + (size_t)t * s.ld + c[i]) =
        make_float4(v[i].x / rms * wv.x, v[i].y / rms * wv.y, v[i].z / rms * wv.z, v[i].w / rms * wv.w);
  }
}

// mm_reduce4 for a Q/K/V launch with its RoPE epilogue (MmRope): item j of
// token t is either four rotation pairs (i0 .. i0 + 3, i0 + hd/2 .. + 3) of a
// q or k head, summed in split order with the bias added as mm_reduce4 does,
// rotated as rope_kv_rows_kernel rotates them and stored into qr or the K
// cache row, or four v columns stored into the V cache row.  The same bits as
// the two launches it replaces.
__global__ __launch_bounds__(256) void mm_reduce_rope(MmRedArgs a, MmRope p) {
  const uint32_t half = p.hd >> 1, g4 = half / 4u;
  const uint32_t nrot = (p.qh + p.kvh) * g4, per = nrot + p.kvh * p.hd / 4u;
  const uint64_t e = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (e >= (uint64_t)a.n * per) return;
  const uint32_t t = (uint32_t)(e / per), j = (uint32_t)(e % per);
  const size_t stride = (size_t)a.n * a.mtot / 4;  // float4 units (mtot % 4 == 0)
  const float* row = a.part + (size_t)t * a.mtot;
  const uint32_t qd = p.qh * p.hd, kvd = p.kvh * p.hd, pos = p.pos0 + t;
  if (j >= nrot) {  // four v columns
    const uint32_t r = 4u * (j - nrot);
    const float4* pv[1] = {reinterpret_cast<const float4*>(row + a.seg[2].col + r)};
    float4 v[1];
    mm_split_sums<1>(pv, stride, a.nsplit, v);
    float4 o = v[0];
    if (a.seg[2].bias) {
      const float4 b = *reinterpret_cast<const float4*>(a.seg[2].bias + r);
      o = make_float4(v[0].x + b.x, v[0].y + b.y, v[0].z + b.z, v[0].w + b.w);
    }
    *reinterpret_cast<float4*>(p.vc + (size_t)pos * kvd + r) = o;
    return;
  }
  const uint32_t hr = j / g4, i0 = 4u * (j % g4);  // head row (q heads, then k heads), first pair
  const bool isq = hr < p.qh;
  const uint32_t col = isq ? a.seg[0].col : a.seg[1].col;
  const float* bias = isq ? a.seg[0].bias : a.seg[1].bias;
  const uint32_t r0 = (isq ? hr : hr - p.qh) * p.hd + i0;  // row of the segment; its partner r0 + half
  const float4* pv[2] = {reinterpret_cast<const float4*>(row + col + r0),
                         reinterpret_cast<const float4*>(row + col + r0 + half)};
  float4 v[2];
  mm_split_sums<2>(pv, stride, a.nsplit, v);
  if (bias) {
    const float4 b0 = *reinterpret_cast<const float4*>(bias + r0), b1 = *reinterpret_cast<const float4*>(bias + r0 + half);
    v[0] = make_float4(v[0].x + b0.x, v[0].y + b0.y, v[0].z + b0.z, v[0].w + b0.w);
    v[1] = make_float4(v[1].x + b1.x, v[1].y + b1.y, v[1].z + b1.z, v[1].w + b1.w);
  }
  // cos, sin of pairs i0 .. i0 + 3
  const float4 ca = *reinterpret_cast<const float4*>(p.rope + (size_t)pos * p.hd + 2u * i0);
  const float4 cb = *reinterpret_cast<const float4*>(p.rope + (size_t)pos * p.hd + 2u * i0 + 4u);
  const float x0[4] = {v[0].x, v[0].y, v[0].z, v[0].w}, x1[4] = {v[1].x, v[1].y, v[1].z, v[1].w};
  const float c[4] = {ca.x, ca.z, cb.x, cb.z}, sn[4] = {ca.y, ca.w, cb.y, cb.w};
  float lo[4], hi[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    lo[k] = x0[k] * c[k] - x1[k] * sn[k];
    hi[k] = x0[k] * sn[k] + x1[k] * c[k];
  }
  float* dst = isq ? p.qr + (size_t)t * qd + hr * p.hd : p.kc + (size_t)pos * kvd + (hr - p.qh) * p.hd;
  *reinterpret_cast<float4*>(dst + i0) = make_float4(lo[0], lo[1], lo[2], lo[3]);
  *reinterpret_cast<float4*>(dst + i0 + half) = make_float4(hi[0], hi[1], hi[2], hi[3]);
}

static bool mm_reduce_vec4(const MmRedArgs& r) {
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (r.mcols % 4 || r.mtot % 4 || !al(r.part)) return false;
  for (uint32_t i = 0; i < r.nseg; ++i) {
    const MmRedSeg& s = r.seg[i];
    if (s.col % 4 || s.rows % 4 || s.ld % 4 || !al(s.y) || (s.res && !al(s.res)) || (s.bias && !al(s.bias)))
      return false;
  }
  return true;
}

// ------------------------------------------------------------------ host side

static uint32_t mm_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v < 1) v = 256;
    cached[dev] = v;
  }
  return (uint32_t)cached[dev];
}

bool mm_supported(uint32_t t, uint64_t in_dim) {
  if (!packed_type(t) || in_dim == 0 || in_dim > (1u << 24)) return false;
  const uint64_t qk = (t == T_Q4_K || t == T_Q6_K) ? 256 : 32;
  return in_dim % qk == 0;
}

// Split-K shape: whole slices per split, at least two slices per workgroup
// and at most K / 4 partial floats per row (sp * n <= K / 4: the partial sums
// stay below about the weights' bytes); among those the fewest splits whose
// workgroups fill whole rounds of one workgroup per CU (104 KB of LDS at 64
// tokens) within 85% of the best split count's fill (each split adds a
// workgroup prologue and partial traffic: gate/up at 16 splits spent 23 us
// in the reduce alone, at 2 splits 5 us).
static void mm_shape(uint64_t groups, uint64_t in_dim, uint64_t n, uint32_t* nsplit, uint32_t* spp,
                     uint32_t* nslices, double* fill = nullptr) {
  const uint64_t ns = (in_dim + MM_KS - 1) / MM_KS;
  const uint64_t target = mm_cu_count();
  uint64_t spmax = ns >= 2 ? ns / 2 : 1;
  const uint64_t by_bytes = in_dim / (4 * (n ? n : 1));
  if (spmax > by_bytes) spmax = by_bytes;
  if (spmax < 1) spmax = 1;
  auto util = [&](uint64_t sp, uint64_t* per_out) {
    const uint64_t per = (ns + sp - 1) / sp, eff = (ns + per - 1) / per, w = groups * eff;
    *per_out = per;
    return w < target ? (double)w / target : (double)w / (double)(((w + target - 1) / target) * target);
  };
  double best = 0.0;
  uint64_t per = ns;
  for (uint64_t sp = 1; sp <= spmax; ++sp) best = std::max(best, util(sp, &per));
  uint64_t best_per = ns;
  double chosen = util(1, &per);
  for (uint64_t sp = 1; sp <= spmax; ++sp)
    if (util(sp, &per) >= 0.85 * best) {
      best_per = per;
      chosen = util(sp, &per);
      break;
    }
  if (fill) *fill = chosen;
  *spp = (uint32_t)best_per;
  *nsplit = (uint32_t)((ns + best_per - 1) / best_per);
  *nslices = (uint32_t)ns;
}

static uint64_t mm_groups(const MmSegDesc* segs, int nseg, uint64_t rows_per_group) {
  uint64_t g = 0;
  for (int i = 0; i < nseg; ++i) g += (segs[i].rows + rows_per_group - 1) / rows_per_group;
  return g;
}

// Partial-sum floats of a launch of exactly n tokens, for either workgroup size.
uint64_t mm_part_floats_at(const uint64_t* rows, int nseg, uint64_t in_dim, uint64_t n) {
  MmSegDesc d[3] = {};
  uint64_t mtot = 0;
  for (int i = 0; i < nseg && i < 3; ++i) {
    d[i].rows = rows[i];
    mtot += rows[i];
  }
  uint64_t most = 0;
  for (uint64_t rpg : {MM_ROWS_NARROW, MM_ROWS_WIDE}) {
    uint32_t nsplit, spp, ns;
    mm_shape(mm_groups(d, nseg, rpg), in_dim, n, &nsplit, &spp, &ns);
    if ((uint64_t)nsplit * n > most) most = (uint64_t)nsplit * n;
  }
  return most * mtot;
}

// Partial-sum floats a launch of up to n tokens may need, for either
// workgroup size (the split count depends on the token count and on the
// workgroups a launch has).
uint64_t mm_part_floats(const uint64_t* rows, int nseg, uint64_t in_dim, uint64_t n) {
  uint64_t most = 0;
  for (uint64_t k = 1; k <= n; ++k) most = std::max(most, mm_part_floats_at(rows, nseg, in_dim, k));
  return most;
}

static int mm_ntt(uint64_t n) { return (int)((n + 15) / 16); }

template <uint32_t T, int NTT, int NW, int DEPTH, bool SC8>
static hipError_t mm_launch_t(const MmArgs& a, dim3 grid, hipStream_t st) {
  const uint32_t lds = 2u * (3u * NTT * 16u * MM_XB * 2u + (T == T_Q4_K ? MM_ST * NTT * 16u * 4u : 0u));
  static bool opened = false;
  if (!opened) {
    if (setup_outside_capture(st) != hipSuccess) return hipErrorStreamCaptureUnsupported;
    if (lds > 65536) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(mm_packed<T, NTT, NW, DEPTH, SC8>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
    }
    opened = true;
  }
  RF_KLAUNCH((mm_packed<T, NTT, NW, DEPTH, SC8>), grid, dim3(64 * NW), lds, st, a);
  return hipGetLastError();
}

template <uint32_t T, int NW, int DEPTH, bool SC8>
static hipError_t mm_launch_ntt(const MmArgs& a, dim3 grid, int ntt, hipStream_t st) {
  switch (ntt) {
    case 1: return mm_launch_t<T, 1, NW, DEPTH, SC8>(a, grid, st);
    case 2: return mm_launch_t<T, 2, NW, DEPTH, SC8>(a, grid, st);
    case 3: return mm_launch_t<T, 3, NW, DEPTH, SC8>(a, grid, st);
    case 4: return mm_launch_t<T, 4, NW, DEPTH, SC8>(a, grid, st);
    default: return hipErrorInvalidValue;
  }
}

template <uint32_t T, bool SC8>
static hipError_t mm_launch_sc(const MmArgs& a, dim3 grid, int ntt, bool wide, hipStream_t st) {
  if constexpr (T == T_Q6_K) {
    return mm_launch_ntt<T, 8, 2, SC8>(a, grid, ntt, st);  // a three-slice ring spills at 64 tokens
  } else {
    if (wide) return mm_launch_ntt<T, 12, 2, SC8>(a, grid, ntt, st);
    return mm_launch_ntt<T, 8, 3, SC8>(a, grid, ntt, st);
  }
}

// SC8 (Q8_0 / Q4_0 with K a multiple of 128 and 8-byte aligned scale rows):
// one 8-byte scale load per slice; the K-quants keep their scales in the
// block headers and take one instantiation.
template <uint32_t T>
static hipError_t mm_launch_shape(const MmArgs& a, dim3 grid, int ntt, bool wide, bool sc8, hipStream_t st) {
  if constexpr (T == T_Q8_0 || T == T_Q4_0) {
    if (sc8) return mm_launch_sc<T, true>(a, grid, ntt, wide, st);
  }
  return mm_launch_sc<T, false>(a, grid, ntt, wide, st);
}

// The wide shape unless its split fills the CUs clearly worse than the narrow
// one (at least 95% of the narrow shape's fill), never for Q6_K.
static bool mm_pick_wide(uint32_t t, const MmSegDesc* segs, int nseg, uint64_t in_dim, uint64_t n) {
  if (t == T_Q6_K) return false;
  uint32_t nsplit, spp, ns;
  double fw = 0.0, fn = 0.0;
  mm_shape(mm_groups(segs, nseg, MM_ROWS_WIDE), in_dim, n, &nsplit, &spp, &ns, &fw);
  mm_shape(mm_groups(segs, nseg, MM_ROWS_NARROW), in_dim, n, &nsplit, &spp, &ns, &fn);
  return fw >= 0.95 * fn;
}

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

hipError_t launch_matmul_packed(uint32_t t, const MmSegDesc* segs, int nseg, const float* x, uint64_t ldx,
                                uint64_t n, uint64_t in_dim, int epi, float* part, uint64_t part_floats,
                                hipStream_t st, const float* norm_w, float eps, float* xn, const MmRope* rope) {
  if (norm_w && (epi != EPI_RESIDUAL || nseg != 1 || !xn)) return hipErrorInvalidValue;
  if (rope) {  // q, k, v segments of one launch, 16-byte rows and tables
    const uint64_t hd = rope->hd;
    const uintptr_t al = reinterpret_cast<uintptr_t>(rope->rope) | reinterpret_cast<uintptr_t>(rope->qr) |
                         reinterpret_cast<uintptr_t>(rope->kc) | reinterpret_cast<uintptr_t>(rope->vc);
    if (epi != EPI_STORE || norm_w || nseg != 3 || hd == 0 || hd % 8 != 0 || (al & 15u) != 0 ||
        segs[0].rows != (uint64_t)rope->qh * hd || segs[1].rows != (uint64_t)rope->kvh * hd ||
        segs[2].rows != (uint64_t)rope->kvh * hd)
      return hipErrorInvalidValue;
  }
  if (!mm_supported(t, in_dim) || nseg < 1 || nseg > 3 || n == 0 || n > MM_MAX_TOKENS) return hipErrorInvalidValue;
  if (!al16(x) || ldx % 4 != 0 || ldx < in_dim || !part) return hipErrorInvalidValue;
  if (epi == EPI_SWIGLU && (nseg != 2 || segs[0].rows != segs[1].rows)) return hipErrorInvalidValue;
  const int nreg = t == T_Q6_K ? 4 : 2;
  auto row_bytes = [&](int k) -> uint64_t { return mm_row_bytes(t, k, in_dim); };
  // the kernel addresses each segment's regions and x through 32-bit buffer
  // offsets, with offsets from MM_OOR on reading as zeros
  if ((uint64_t)n * ldx * 4 >= (1ull << 31)) return hipErrorInvalidValue;
  bool sc8 = in_dim % MM_KS == 0;
  const bool wide = mm_pick_wide(t, segs, nseg, in_dim, n);
  const uint64_t rpg = wide ? MM_ROWS_WIDE : MM_ROWS_NARROW;
  MmArgs a{};
  MmRedArgs r{};
  uint64_t mtot = 0, groups = 0;
  for (int i = 0; i < nseg; ++i) {
    const MmSegDesc& d = segs[i];
    if (d.rows == 0 || d.row_start + d.rows > d.matrix_rows || !d.packed || !d.y) return hipErrorInvalidValue;
    uint64_t off = 0;
    for (int k = 0; k < nreg; ++k) {
      const uint64_t rb = row_bytes(k);
      a.seg[i].reg[k] = static_cast<const uint8_t*>(d.packed) + off + d.row_start * rb;
      off += d.matrix_rows * rb;
    }
    for (int k = 0; k < nreg; ++k)
      if (d.rows * row_bytes(k) >= (1ull << 31)) return hipErrorInvalidValue;
    sc8 = sc8 && (reinterpret_cast<uintptr_t>(a.seg[i].reg[1]) & 7u) == 0;
    // 8-byte code loads; Q4_K headers and Q6_K scales as 16 bytes
    if ((reinterpret_cast<uintptr_t>(a.seg[i].reg[0]) & 7u) != 0) return hipErrorInvalidValue;
    if (t == T_Q4_K && !al16(a.seg[i].reg[1])) return hipErrorInvalidValue;
    if (t == T_Q6_K && (((reinterpret_cast<uintptr_t>(a.seg[i].reg[1]) & 7u) != 0) || !al16(a.seg[i].reg[2])))
      return hipErrorInvalidValue;
    a.seg[i].rows = (uint32_t)d.rows;
    a.seg[i].group_begin = (uint32_t)groups;
    a.seg[i].col = (uint32_t)mtot;
    r.seg[i] = MmRedSeg{d.y, d.res, d.bias, (uint32_t)d.rows, (uint32_t)mtot, (uint32_t)d.ld};
    if (epi == EPI_RESIDUAL && !d.res) return hipErrorInvalidValue;
    groups += (d.rows + rpg - 1) / rpg;
    mtot += d.rows;
  }
  if (mtot > 0xFFFFFFFFull || groups > 0x7FFFFFFFull) return hipErrorInvalidValue;
  uint32_t nsplit, spp, nslices;
  mm_shape(groups, in_dim, n, &nsplit, &spp, &nslices);
  if ((uint64_t)nsplit * n * mtot > part_floats) return hipErrorInvalidValue;
  a.nseg = (uint32_t)nseg;
  a.x = x;
  a.part = part;
  a.n = (uint32_t)n;
  a.ldx = (uint32_t)ldx;
  a.in_dim = (uint32_t)in_dim;
  a.mtot = (uint32_t)mtot;
  a.nslices = nslices;
  a.spp = spp;
  const dim3 grid((uint32_t)groups, nsplit);
  const int ntt = mm_ntt(n);
  r.nseg = (uint32_t)nseg;
  r.nsplit = nsplit;
  r.n = (uint32_t)n;
  r.mtot = (uint32_t)mtot;
  r.mcols = epi == EPI_SWIGLU ? (uint32_t)segs[0].rows : (uint32_t)mtot;
  r.epi = epi;
  r.part = part;
  if (rope && !mm_reduce_vec4(r)) return hipErrorInvalidValue;  // before any launch
  hipError_t e;
  switch (t) {
    case T_Q8_0: e = mm_launch_shape<T_Q8_0>(a, grid, ntt, wide, sc8, st); break;
    case T_Q4_0: e = mm_launch_shape<T_Q4_0>(a, grid, ntt, wide, sc8, st); break;
    case T_Q4_K: e = mm_launch_shape<T_Q4_K>(a, grid, ntt, wide, false, st); break;
    default: e = mm_launch_shape<T_Q6_K>(a, grid, ntt, wide, false, st); break;
  }
  if (e != hipSuccess) return e;
  const uint64_t total = (uint64_t)n * r.mcols;
  const bool al = ((reinterpret_cast<uintptr_t>(norm_w) | reinterpret_cast<uintptr_t>(xn)) & 15u) == 0;
  if (norm_w && al && mm_reduce_vec4(r) && r.mcols <= 8192) {
    if (r.mcols <= 4096) RF_KLAUNCH(mm_reduce_norm<1>, dim3((uint32_t)n), dim3(1024), 0, st, r, norm_w, eps, xn);
    else RF_KLAUNCH(mm_reduce_norm<2>, dim3((uint32_t)n), dim3(1024), 0, st, r, norm_w, eps, xn);
    return hipGetLastError();
  }
  if (rope) {
    const uint64_t items = n * ((uint64_t)(rope->qh + rope->kvh) * rope->hd / 8 + (uint64_t)rope->kvh * rope->hd / 4);
    RF_KLAUNCH(mm_reduce_rope, dim3((uint32_t)((items + 255) / 256)), dim3(256), 0, st, r, *rope);
    return hipGetLastError();
  }
  if (mm_reduce_vec4(r))
    RF_KLAUNCH(mm_reduce4, dim3((uint32_t)((total / 4 + 255) / 256)), dim3(256), 0, st, r);
  else
    RF_KLAUNCH(mm_reduce, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, st, r);
  e = hipGetLastError();
  if (e != hipSuccess || !norm_w) return e;
  const MmSegDesc& d = segs[0];
  return launch_rmsnorm_rows(d.y, norm_w, d.rows, n, d.ld, eps, xn, st);
}

// ------------------------------------------------------- per-token glue

// RMSNorm of `rows` rows of length n (stride ld), x / rms * w as
// rms_norm_reference (compute.rs:291-319); one workgroup per row.  Rows of up
// to 8192 elements (n % 4 == 0, 16-byte aligned) stay in registers between
// the sum of squares and the scaling, read with 16-byte loads.
template <int V>
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           uint32_t n, uint32_t ld, float eps,
                                                           float* __restrict__ y) {
  __shared__ float part[4];
  const uint32_t tid = threadIdx.x;
  const float* xr = x + (size_t)blockIdx.x * ld;
  float* yr = y + (size_t)blockIdx.x * ld;
  float ss = 0.f;
  float4 v[V > 0 ? V : 1];
  if constexpr (V > 0) {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const uint32_t k = 4u * (tid + 256u * i);
      v[i] = k < n ? *reinterpret_cast<const float4*>(xr + k) : make_float4(0.f, 0.f, 0.f, 0.f);
      ss = fmaf(v[i].x, v[i].x, ss);
      ss = fmaf(v[i].y, v[i].y, ss);
      ss = fmaf(v[i].z, v[i].z, ss);
      ss = fmaf(v[i].w, v[i].w, ss);
    }
  } else {
    for (uint32_t i = tid; i < n; i += 256u) ss = fmaf(xr[i], xr[i], ss);
  }
  ss = rf_wave_sum(ss);
  if ((tid & 63u) == 0) part[tid >> 6] = ss;
  __syncthreads();
  const float tot = part[0] + part[1] + part[2] + part[3];
  const float rms = sqrtf(tot / (float)n + eps);
  if constexpr (V > 0) {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const uint32_t k = 4u * (tid + 256u * i);
      if (k >= n) break;
      const float4 wv = *reinterpret_cast<const float4*>(w + k);
      *reinterpret_cast<float4*>(yr + k) =
          make_float4(v[i].x / rms * wv.x, v[i].y / rms * wv.y, v[i].z / rms * wv.z, v[i].w / rms * wv.w);
    }
  } else {
    for (uint32_t i = tid; i < n; i += 256u) yr[i] = xr[i] / rms * w[i];
  }
}

hipError_t launch_rmsnorm_rows(const float* x, const float* w, uint64_t n, uint64_t rows, uint64_t ld, float eps,
                               float* y, hipStream_t st) {
  if (rows == 0) return hipSuccess;
  const bool vec = n % 4 == 0 && ld % 4 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                                                   reinterpret_cast<uintptr_t>(y)) & 15u) == 0;
  const dim3 grid((uint32_t)rows), blk(256);
  if (vec && n <= 4096) RF_KLAUNCH(rmsnorm_rows_kernel<4>, grid, blk, 0, st, x, w, (uint32_t)n, (uint32_t)ld, eps, y);
  else if (vec && n <= 8192) RF_KLAUNCH(rmsnorm_rows_kernel<8>, grid, blk, 0, st, x, w, (uint32_t)n, (uint32_t)ld, eps, y);
  else RF_KLAUNCH(rmsnorm_rows_kernel<0>, grid, blk, 0, st, x, w, (uint32_t)n, (uint32_t)ld, eps, y);
  return hipGetLastError();
}

// Token z at position pos0 + z (blockIdx.x), head row blockIdx.y of [q heads,
// k heads, v heads]: q heads rotated into qr[z], k heads rotated into the K
// cache row, v copied into the V cache row (rope_reference,
// compute.rs:389-456, with the host cos/sin table; the rotation is written in
// the same operation order as the decode attention kernel's).  One
// wavefront per head row.
__global__ __launch_bounds__(64) void rope_kv_rows_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                          const float* __restrict__ v, const float* __restrict__ rope,
                                                          uint32_t pos0, uint32_t qh, uint32_t kvh, uint32_t hd,
                                                          float* __restrict__ qr, float* __restrict__ kc,
                                                          float* __restrict__ vc) {
  const uint32_t z = blockIdx.x, hr = blockIdx.y, pos = pos0 + z, half = hd >> 1;
  const uint32_t qd = qh * hd, kvd = kvh * hd;
  if (hr >= qh + kvh) {  // v head
    const uint32_t o = (hr - qh - kvh) * hd;
    for (uint32_t d = threadIdx.x; d < hd; d += 64u) vc[(size_t)pos * kvd + o + d] = v[(size_t)z * kvd + o + d];
    return;
  }
  const bool isq = hr < qh;
  const uint32_t o = (isq ? hr : hr - qh) * hd;
  const float* src = isq ? q + (size_t)z * qd + o : k + (size_t)z * kvd + o;
  float* dst = isq ? qr + (size_t)z * qd + o : kc + (size_t)pos * kvd + o;
  const float* cs = rope + (size_t)pos * hd;
  for (uint32_t d = threadIdx.x; d < hd; d += 64u) {
    const uint32_t ci = d < half ? d : d - half;
    const float va = src[d], vp = src[d < half ? d + half : d - half];
    const float c0 = cs[2 * ci], c1 = cs[2 * ci + 1];
    dst[d] = d < half ? va * c0 - vp * c1 : vp * c1 + va * c0;
  }
}

hipError_t launch_rope_kv_rows(const float* q, const float* k, const float* v, const float* rope, uint64_t pos0,
                               uint64_t ntok, uint32_t qh, uint32_t kvh, uint32_t hd, float* qr, float* kc,
                               float* vc, hipStream_t st) {
  if (ntok == 0) return hipSuccess;
  RF_KLAUNCH(rope_kv_rows_kernel, dim3((uint32_t)ntok, qh + 2 * kvh), dim3(64), 0, st, q, k, v, rope,
                     (uint32_t)pos0, qh, kvh, hd, qr, kc, vc);
  return hipGetLastError();
}

// Loads this file's code object on the current device (HIP defers that to a
// kernel's first use, which may otherwise fall inside a stream capture) and
// caches the device's CU count the launchers read.
hipError_t load_module_prefill() {
  (void)mm_cu_count();
  hipFuncAttributes fa;
  return hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(mm_reduce));
}

}  // namespace rf
