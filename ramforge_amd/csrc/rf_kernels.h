// rf_kernels.h — kernel argument structs and host-side launchers (internal).
#pragma once

#include "rf_formats.h"

namespace rf {

enum { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2 };

// Planning pass: while set on the calling thread, the launchers do all their
// host-side work (dispatch, the one-time kernel setup of dynamic LDS and
// occupancy) but launch nothing.  The model runs a decode step this way
// before it captures one, so no setup call falls inside the capture.
extern thread_local bool g_plan_only;
#define RF_KLAUNCH(...)                                   \
  do {                                                    \
    if (!::rf::g_plan_only) hipLaunchKernelGGL(__VA_ARGS__); \
  } while (0)

// hipSuccess, or hipErrorStreamCaptureUnsupported when st is being captured:
// a launcher's one-time kernel setup (hipFuncSetAttribute, occupancy
// queries) runs outside stream captures only.
hipError_t setup_outside_capture(hipStream_t st);

// Workgroups of `per` threads that cover n > 0 items, or 0 when that exceeds
// the 2^31 - 1 workgroups of a grid dimension: the launcher then fails
// instead of covering a truncated range.
inline uint32_t grid_blocks(uint64_t n, uint32_t per) {
  const uint64_t b = (n + per - 1) / per;
  return b > 0x7FFFFFFFull ? 0u : (uint32_t)b;
}

struct MvSeg {
  const uint8_t* w;
  float* y;
  const float* res;
  uint32_t rows;
  uint32_t tile_begin;
};

struct MvArgs {
  MvSeg seg[3];
  uint32_t nseg;
  const float* x;
  const float* norm_w;
  float eps;
  uint32_t in_dim, units, rg, rows_per_tile, row_bytes, tile_stride;
  const uint8_t* w_up;
  uint32_t ntiles;      // persistent kernel: tiles over all segments
  uint32_t red_offset;  // persistent kernel: LDS byte offset of the reduction area
};

struct MvPlan {
  bool tiled;
  uint32_t units, rg, rows_per_tile, threads, row_bytes, tile_stride, lds_bytes;
  // persistent streaming kernel (chosen when rows and bases are 16-byte aligned)
  bool stream;
  uint32_t s_rows_per_tile, s_threads, s_lds_bytes, s_red_offset, s_wgs_per_cu;
};

// One output segment of a (possibly multi-matrix) matvec launch.  All
// segments of one launch share the input vector, in_dim and ggml type.
struct MvSegDesc {
  const void* w;      // first byte of the segment's first row
  const void* w_up;   // EPI_SWIGLU: the paired "up" matrix (same rows)
  float* y;
  const float* res;   // EPI_RESIDUAL: y = res + W x
  uint64_t rows;
};

bool type_geometry(uint32_t t, uint64_t* qk, uint64_t* bs);
MvPlan plan_matvec(uint32_t t, uint64_t in_dim, bool dual);
void set_matvec_tile_bytes(uint32_t bytes);
void set_matvec_stream_tile(uint32_t bytes);
uint32_t matvec_tile_bytes();
void set_matvec_stream(bool on);
bool matvec_stream();
// Plain (store, no norm, one segment) Q8_0 / Q4_0 matvecs on GGUF bytes take
// the wave-staged kernel (rf_tune_matvec_kernel 2, default).
void set_matvec_wave(bool on);
bool matvec_wave_on();
// Packed Q8_0 / Q4_0 launches take x as int8 digit planes when a wavefront's
// rows hold >= 24 KiB of codes (1), always (2), or never (0).
void set_matvec_digits(int mode);
int matvec_digits();
// Packed launches whose rows fit one step and leave at most 4 rows per
// wavefront request all of them before the prologue (1) or use the two-step
// ring (0).
void set_packed_inflight(int mode);
int packed_inflight();
hipError_t launch_matvec_segments(uint32_t t, const MvSegDesc* segs, int nseg, const float* x,
                                  const float* norm_w, float eps, uint64_t in_dim, int epi,
                                  hipStream_t st);

// Matvec on the packed (device-native) layout of Q8_0, Q4_0, Q4_K and Q6_K
// (rf_matvec_packed.hip): the bytes of each block are split into regions,
// each stored for all rows, row-major: Q8_0 / Q4_0 codes, f16 scales; Q4_K
// codes, 16-byte headers (d, dmin, 12 scale bytes); Q6_K low bits (ql), high
// bits (qh), 16 int8 scales, f16 d.  Same byte count as the GGUF payload.
constexpr int PK_MAX_REGIONS = 4;
struct PkSeg {
  const uint8_t* reg[PK_MAX_REGIONS];     // each region at the segment's first row (codes first)
  const uint8_t* reg_up[PK_MAX_REGIONS];  // EPI_SWIGLU: the "up" matrix
  float* y;
  const float* res;
  uint32_t row_begin;  // first row of the segment among all segments
};
struct PkArgs {
  PkSeg seg[3];
  uint32_t nseg, rows_total;
  const float* x;
  const float* norm_w;
  float eps;
  uint32_t in_dim;
  int32_t* advance;  // non-null: workgroup 0 adds 1 to *advance (the model's device position)
  // Merged x (matvec_packed<..., MRG>): x is the merge of single-query
  // attention's chunk records (o[hd], m, l at mws[(c * m_qh + h) * att_rec(hd)],
  // hd = 2^m_hd_log2, m_nsplit chunks per head, the chunk count following
  // from *m_pos as in the attention kernels); with one chunk, x itself holds
  // the output.
  const float* mws;
  const int32_t* m_pos;
  uint32_t m_nsplit, m_qh, m_hd_log2;
};
// Chunk records of the attention launch that precedes an o-projection which
// merges them (launch_matvec_packed's mrg argument).
struct PkMerge {
  const float* ws;
  const int32_t* d_pos;
  uint32_t nsplit, qh, hd;
};
struct PkPlan {
  bool ok;
  uint32_t lds_bytes;  // x and its slice sums staged in LDS
};
struct PkSegDesc {
  const void* packed;     // packed matrix base (codes of row 0)
  const void* packed_up;  // EPI_SWIGLU: packed "up" matrix, same shape
  uint64_t matrix_rows;   // rows of the whole packed matrix (locates the scales)
  uint64_t row_start;     // first row of this segment within the matrix
  uint64_t rows;
  float* y;
  const float* res;
};
bool packed_type(uint32_t t);
PkPlan plan_packed(uint32_t t, uint64_t in_dim);
// advance: optional device counter the launch increments once (nothing in
// the launch reads it).
hipError_t launch_matvec_packed(uint32_t t, const PkSegDesc* segs, int nseg, const float* x, const float* norm_w,
                                float eps, uint64_t in_dim, int epi, hipStream_t st, int32_t* advance = nullptr,
                                const PkMerge* mrg = nullptr);
// hipSuccess when launch_matvec_packed can merge attention chunk records into
// x for this projection (EPI_RESIDUAL, no norm, one segment of `rows` rows):
// the single-step launch of Q8_0 / Q4_0 / Q4_K with in_dim = qh * hd, hd a
// power of two from 16, at most 8 chunks and 64 query heads;
// hipErrorNotSupported when it cannot; hipErrorStreamCaptureUnsupported when
// answering needs the kernel's one-time setup while st is being captured.
hipError_t pk_merge_supported(uint32_t t, uint64_t in_dim, uint64_t rows, uint32_t nsplit, uint32_t qh, uint32_t hd,
                              hipStream_t st);
// The matvec_packed instance the calling thread launched last (also in a
// planning pass), as the kernel trace names it; "" after a clear or when the
// last launch was not a packed one.
const char* last_packed_kernel();
void clear_last_packed_kernel();
// GGUF payload [rows][in_dim] -> packed layout (distinct buffers).
hipError_t launch_pack(uint32_t t, const void* raw, void* packed, uint64_t rows, uint64_t in_dim, hipStream_t st);

// Bit-exact row decode: rows [0, rows) of `w` (row_bytes each) -> out[rows][in_dim].
// If token_index != nullptr, output row r is row token_index[r] of `w`.
hipError_t launch_dequant_rows(uint32_t t, const void* w, uint64_t in_dim, uint64_t rows,
                               float* out, const uint32_t* token_index, uint64_t token_rows,
                               hipStream_t st);

// Split-K single-query attention (see rf_attention.hip).
struct AttnArgs {
  const float* q;        // [qh][hd]
  const float* k_hist;   // [hist][kvh][hd] (or the model's cache base)
  const float* v_hist;
  const float* k_cur;    // [kvh][hd]
  const float* v_cur;
  float* out;            // [qh][hd]
  float* ws;             // chunk records [nsplit][qh][att_rec(hd)]
  const float* rope;     // model mode: [cap][hd/2][2] cos/sin table, else null
  float* k_store;        // model mode: cache slot base (k_cache), else null
  float* v_store;
  const int32_t* d_pos;  // model mode: device position (== hist), else null
  uint32_t hist;         // API mode history length
  uint32_t qh, kvh, hd, nsplit;
  uint32_t waves;        // wavefronts per chunk workgroup (4 or 8); 0: chosen from hist
  uint32_t per_q;        // nonzero: one workgroup per query head and chunk (short contexts)
  uint32_t defer_merge;  // nonzero: no merge launch (the o-projection merges the chunk records)
  uint32_t ntok;         // nonzero: a batch of ntok queries (prefill): query z at position
                         // hist + z, q / out [ntok][qh][hd], ws [ntok][nsplit][qh][att_rec(hd)]; every
                         // query's own k / v already in the cache (k_hist / v_hist) and rotated
  float denom;           // sqrt(hd) as the reference computes it
};
hipError_t launch_attention(const AttnArgs& a, hipStream_t st);
// Token batches (ntok > 0) run attn_prefill, the matrix-core kernel, where
// supported (rf_tune_prefill_attention: 0 never, 1 past 1024 positions, 2
// always); its launches take prefill_attention_mfma_splits position splits.
void set_prefill_attention_mfma(int mode);
int prefill_attention_mfma();
bool prefill_attention_mfma_supported(uint32_t qh, uint32_t kvh, uint32_t hd, uint64_t total);
uint32_t prefill_attention_mfma_splits(uint64_t total, uint64_t ntok, uint32_t kvh);
// Decode launches that take the one-pass online-softmax kernel (attn_flash):
// 1 (default) those per query head, 2 all, 0 none (attn_split, scores in LDS).
void set_attention_kernel(int mode);
int attention_kernel();
// Any-shape kernel; its workspace is [qh][hist + 1] floats.
hipError_t launch_attention_naive(const AttnArgs& a, hipStream_t st);
uint32_t attention_splits(uint32_t total_positions, uint32_t kvh);
uint32_t attention_waves(uint32_t chunk, uint32_t g_hd);
// Positions per chunk of a `nsplit`-chunk launch over `total` positions.
uint32_t att_chunk_positions(uint64_t total, uint32_t nsplit);
constexpr uint64_t ATT_PREFILL_CHUNK = 1024;  // longest chunk of the split kernel
constexpr uint32_t ATT_MIN_CHUNK = 64;        // 16 position slots x 4 loads in flight
// Positions per chunk of an nsplit-chunk split over `total` positions (a
// multiple of 16, at least ATT_MIN_CHUNK); the chunk count is
// ceil(total / chunk).  Shared by the attention kernels and the o-projection
// that merges their chunk records.
__host__ __device__ __forceinline__ uint32_t att_chunk(uint32_t total, uint32_t nsplit) {
  uint32_t c = (total + nsplit - 1) / nsplit;
  c = (c + 15u) & ~15u;
  return c < ATT_MIN_CHUNK ? ATT_MIN_CHUNK : c;
}
// Floats per chunk record of the split kernel: o[hd], m, l and two unused
// floats, so that records (hd a multiple of 4) start on 16-byte boundaries.
__host__ __device__ constexpr uint32_t att_rec(uint32_t hd) { return hd + 4; }
struct AttnShape {
  uint32_t per_q, nsplit, waves;
};
constexpr int ATT_REGIMES = 5;
int attention_regime(uint64_t total, uint32_t qh, uint32_t kvh, uint64_t cap);
void set_attention_single(uint32_t n);
uint32_t attention_single();
AttnShape attention_regime_shape(int regime, uint32_t qh, uint32_t kvh, uint64_t cap);
uint64_t attention_ws_floats(uint32_t nsplit, uint32_t qh, uint32_t hd);
// The split kernel handles this shape for up to `total_positions` positions.
bool attention_supported(uint32_t qh, uint32_t kvh, uint32_t hd, uint64_t total_positions);

// Batched prefill (rf_prefill.hip): Y[t][r] = sum_k W[r][k] X[t][k] for up to
// MM_MAX_TOKENS tokens on the packed layout, on the matrix cores, with split-K
// partials in `part` and the epilogue of the decode matvec (EPI_SWIGLU:
// segment 0 gate, segment 1 up, output in segment 0's y).
constexpr uint64_t MM_MAX_TOKENS = 64;
struct MmSegDesc {
  const void* packed;    // packed matrix base
  uint64_t matrix_rows;  // rows of the whole packed matrix (locates its regions)
  uint64_t row_start;    // first row of this segment within the matrix
  uint64_t rows;
  float* y;              // [n][ld]
  const float* res;      // EPI_RESIDUAL: [n][ld]
  const float* bias;     // EPI_STORE: added per row, or null
  uint64_t ld;
};
bool mm_supported(uint32_t t, uint64_t in_dim);
uint64_t mm_part_floats(const uint64_t* rows, int nseg, uint64_t in_dim, uint64_t n);
uint64_t mm_part_floats_at(const uint64_t* rows, int nseg, uint64_t in_dim, uint64_t n);
// norm_w (EPI_RESIDUAL, one segment): also xn = RMSNorm(y) * norm_w per token
// row (stride ld), the norm that follows a residual projection; fused into
// the split-K reduce where the rows allow it, else a separate launch.
// RoPE epilogue of a Q/K/V launch (EPI_STORE, segments q, k, v of qh hd,
// kvh hd and kvh hd rows): the split-K reduce rotates q into qr[token] and k
// into K cache row pos0 + token and copies v into V cache row pos0 + token,
// with rope_kv_rows_kernel's arithmetic (the segments' own outputs are not
// written).  rope = the [position][hd / 2][cos, sin] table.
struct MmRope {
  const float* rope;
  uint32_t pos0, qh, kvh, hd;
  float* qr;
  float* kc;
  float* vc;
};
hipError_t launch_matmul_packed(uint32_t t, const MmSegDesc* segs, int nseg, const float* x, uint64_t ldx,
                                uint64_t n, uint64_t in_dim, int epi, float* part, uint64_t part_floats,
                                hipStream_t st, const float* norm_w = nullptr, float eps = 0.f,
                                float* xn = nullptr, const MmRope* rope = nullptr);
hipError_t launch_rmsnorm_rows(const float* x, const float* w, uint64_t n, uint64_t rows, uint64_t ld, float eps,
                               float* y, hipStream_t st);
hipError_t launch_rope_kv_rows(const float* q, const float* k, const float* v, const float* rope, uint64_t pos0,
                               uint64_t ntok, uint32_t qh, uint32_t kvh, uint32_t hd, float* qr, float* kc,
                               float* vc, hipStream_t st);

// Elementwise (rf_elementwise.hip).
hipError_t launch_rmsnorm(const float* x, const float* w, uint64_t n, float eps, float* y, hipStream_t st);
hipError_t launch_binary(int op, const float* a, const float* b, uint64_t n, float* out, hipStream_t st);
hipError_t launch_silu(const float* x, uint64_t n, float* y, hipStream_t st);
hipError_t launch_softmax(float* v, uint64_t n, hipStream_t st);
// cos/sin pairs of one position passed by value (hd <= 512).
struct RopeCS {
  float cs[512];
};
hipError_t launch_rope_pair(float* q, float* k, const RopeCS& cs, uint32_t hd, uint32_t qh, uint32_t kvh, hipStream_t st);
hipError_t launch_bias_add(float* v, const float* b, uint64_t n, hipStream_t st);
// Writes the index to *out and, if ring != null, also to ring[*d_pos].
hipError_t launch_argmax(const float* logits, uint64_t n, uint32_t* out, float* ws_val, uint32_t* ws_idx,
                         uint32_t* ring, const int32_t* d_pos, hipStream_t st);
// launch_argmax whose final stage also decodes row *out of the embedding
// table (ggml type embd_type, [rows][in_dim], GGUF layout) into `hidden`.
hipError_t launch_argmax_embed(const float* logits, uint64_t n, uint32_t* out, float* ws_val, uint32_t* ws_idx,
                               uint32_t* ring, const int32_t* d_pos, uint32_t embd_type, const void* embd,
                               uint64_t in_dim, float* hidden, hipStream_t st);
uint32_t argmax_partials(uint64_t n);
hipError_t launch_synth(uint32_t t, uint64_t seed, uint64_t first_block, uint64_t n_blocks, double mul,
                        void* dst, hipStream_t st);
hipError_t launch_advance_pos(int32_t* d_pos, hipStream_t st);
hipError_t launch_set_u32(uint32_t* p, uint32_t v, hipStream_t st);
hipError_t launch_set_i32(int32_t* p, int32_t v, hipStream_t st);
hipError_t launch_fill(float* p, float v, uint64_t n, hipStream_t st);

enum { BIN_ADD = 0, BIN_MUL = 1, BIN_SWIGLU = 2 };

// Per-file code-object loads (one per .hip file with kernels), called at
// context creation so that no capture sees a first-use load.
hipError_t load_module_attention();
hipError_t load_module_elementwise();
hipError_t load_module_matvec();
hipError_t load_module_packed();
hipError_t load_module_prefill();

}  // namespace rf
