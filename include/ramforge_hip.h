/*
 * ramforge_hip.h — C ABI of the MI355X (gfx950) decode-step tier for RAMforge.
 *
 * The library replaces RAMforge's legacy CPU decode hot path: the GGUF block
 * matvec and single-query GQA attention, the per-layer composition around them
 * and the device-memory side of the layer-lifetime contract.  The signatures
 * are plain C (pointers, sizes, status codes) so a Rust `extern "C"` block can
 * bind them one-to-one.  Reference paths are relative to
 * crates/ramforge-{core,runtime}/src of RAMforge.
 *
 * Conventions (mirroring the reference's Rust API):
 *   - Every call returns int32_t: RF_OK (0) or an RF_ERR_* code.  The message
 *     of the last failure on the calling thread is read with rf_last_error();
 *     messages keep the reference's wording ("row truncated", "not divisible",
 *     "arity mismatch", "exceeds out_dim", "insufficient memory", ...).
 *   - Arguments are validated before anything is written or launched: on
 *     error the outputs are untouched (quant.rs:1718-1730, 1788-1806).
 *   - Tensors passed to compute calls are DEVICE pointers; shapes use the
 *     reference's conventions (matvec kernels take out_dim/in_dim as quant.rs
 *     does; the weight bytes are the raw GGUF payload, row-major [out][in]).
 *   - `stream` is a hipStream_t; NULL selects the context's compute stream.
 *     Compute calls are asynchronous with respect to the host.
 *   - Workspaces: rf_attention_decode, rf_matmul_packed and rf_matvec_packed
 *     with a misaligned x use context-owned workspaces.  rf_ctx_reserve sizes
 *     them up front (rf_attention_workspace_bytes / rf_matmul_workspace_bytes
 *     give the bytes a shape needs) and, with fixed = 1, turns any later call
 *     that would need more into an RF_ERR_INVALID error: then no entry point
 *     allocates or synchronises on the hot path.  Without a fixed reservation
 *     the first call that needs a workspace (or a larger one) allocates it,
 *     synchronising the device before freeing a smaller one; that growth is
 *     refused while the stream is being captured, and graphs captured before
 *     a workspace was replaced are refused by rf_graph_replay.  Calls that
 *     share a workspace must be ordered (one stream, or events).
 *   - A context is driven from one host thread at a time (the reference
 *     engine calls from one thread, parallelism is internal); the ledger
 *     calls (rf_vram_*) and rf_last_error are safe from any thread.
 */
#ifndef RAMFORGE_HIP_H
#define RAMFORGE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RF_OK 0
#define RF_ERR_INVALID 1     /* shape / argument error (reference: Err(String)) */
#define RF_ERR_BUDGET 2      /* VRAM ledger refused a charge (MemoryError)     */
#define RF_ERR_HIP 3         /* HIP runtime failure                            */
#define RF_ERR_UNSUPPORTED 4 /* type or shape outside what the kernels cover   */
#define RF_ERR_IO 5          /* a byte source's read failed (DataSourceError)  */

/* ggml type ids: core/src/types.rs:238-292 (GgmlType::from_u32). */
#define RF_TYPE_F32 0u
#define RF_TYPE_F16 1u
#define RF_TYPE_Q4_0 2u
#define RF_TYPE_Q5_0 6u
#define RF_TYPE_Q8_0 8u
#define RF_TYPE_Q2_K 10u
#define RF_TYPE_Q3_K 11u
#define RF_TYPE_Q4_K 12u
#define RF_TYPE_Q5_K 13u
#define RF_TYPE_Q6_K 14u
#define RF_TYPE_Q8_K 15u
#define RF_TYPE_BF16 30u

/* matvec row_count value meaning "all rows from row_start" (Rust `None`). */
#define RF_ALL_ROWS UINT64_MAX

typedef struct rf_ctx rf_ctx;
typedef struct rf_model rf_model;
typedef void *rf_stream_t; /* hipStream_t */

/* ------------------------------------------------------------------ errors */

/* Copies the calling thread's last error message (NUL-terminated, truncated
 * to cap) and returns its full length. */
size_t rf_last_error(char *buf, size_t cap);
/* Library version string. */
const char *rf_version(void);

/* --------------------------------------------------------------- context */

/* Creates a context on HIP device `device` with a device-memory ledger of
 * `vram_budget_bytes` (0 = the device's total memory).  The ledger is the
 * device-domain MemoryBudget (core/src/memory.rs:30-384) that the GPU
 * residency tier charges; the context also owns one compute stream and two
 * copy streams at default priority (rf_ctx_copy_stream returns the first; the
 * streaming tier splits a layer's uploads over both).  Replaces CpuBackend::new
 * (runtime/src/backend.rs:72-84) as the compute backend handle. */
int32_t rf_ctx_create(int32_t device, uint64_t vram_budget_bytes, rf_ctx **out);
void rf_ctx_destroy(rf_ctx *ctx);
int32_t rf_ctx_synchronize(rf_ctx *ctx);
/* Grows the context's workspaces to at least these sizes now (charges
 * "workspace:attention", "workspace:matmul", "workspace:scratch"; 0 leaves one
 * as it is).  staging_bytes serves rf_matvec_packed / rf_matmul_packed with an
 * x that is not 16-byte aligned: 4 * in_dim (times min(n_tokens, 64) for the
 * matmul).  fixed != 0: later calls never grow a workspace; one that would
 * need more fails with RF_ERR_INVALID.  No counterpart in the reference,
 * whose CPU kernels allocate per call (ops.rs:49-69 returns a fresh Vec). */
int32_t rf_ctx_reserve(rf_ctx *ctx, uint64_t attention_bytes, uint64_t matmul_bytes, uint64_t staging_bytes,
                       int32_t fixed);
/* Workspace bytes of rf_attention_decode for every context of up to
 * max_positions (hist_len + 1) positions with this head shape, and of
 * rf_matmul_packed for one call of this shape (0: none needed). */
uint64_t rf_attention_workspace_bytes(uint64_t max_positions, uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim);
uint64_t rf_matmul_workspace_bytes(uint64_t out_dim, uint64_t in_dim, uint64_t n_tokens);
rf_stream_t rf_ctx_compute_stream(rf_ctx *ctx);
rf_stream_t rf_ctx_copy_stream(rf_ctx *ctx);
/* Device name and compute-unit count (for reports). */
int32_t rf_ctx_device_info(rf_ctx *ctx, char *name, size_t cap, int32_t *compute_units);

/* ------------------------------------------------- VRAM ledger + buffers */

/* MemoryBudget::allocate (memory.rs:93-122) followed by hipMalloc: the charge
 * is reserved before the allocation and rolled back if hipMalloc fails.
 * Errors: zero size, duplicate name, insufficient budget. */
int32_t rf_vram_alloc(rf_ctx *ctx, const char *charge, uint64_t bytes, void **out);
/* hipFree of the buffer registered under `charge`, then MemoryBudget::release
 * (memory.rs:133-152): the physical free precedes the logical release. */
int32_t rf_vram_release(rf_ctx *ctx, const char *charge);
/* memory.rs:286-325: renames every charge starting with old_prefix. */
int32_t rf_vram_rename_prefix(rf_ctx *ctx, const char *old_prefix, const char *new_prefix);
/* Charge size (RF_ERR_INVALID if absent), used / total / peak bytes. */
int32_t rf_vram_charge(rf_ctx *ctx, const char *charge, uint64_t *bytes);
uint64_t rf_vram_used(rf_ctx *ctx);
uint64_t rf_vram_total(rf_ctx *ctx);
uint64_t rf_vram_peak(rf_ctx *ctx);

/* Pinned host staging buffers (hipHostMalloc). */
int32_t rf_pinned_alloc(rf_ctx *ctx, uint64_t bytes, void **out);
int32_t rf_pinned_free(rf_ctx *ctx, void *ptr);

/* Copies.  rf_upload_async is hipMemcpyAsync host->device on `stream`
 * (pinned sources overlap with compute when issued on the copy stream). */
int32_t rf_upload_async(rf_ctx *ctx, void *dst, const void *src, uint64_t bytes, rf_stream_t stream);
int32_t rf_upload(rf_ctx *ctx, void *dst, const void *src, uint64_t bytes);
int32_t rf_download(rf_ctx *ctx, void *dst, const void *src, uint64_t bytes);
int32_t rf_memset(rf_ctx *ctx, void *dst, int32_t value, uint64_t bytes);
/* Device -> device copy on `stream` (hipMemcpyAsync); no reference
 * counterpart (the reference moves layer bytes host-side only). */
int32_t rf_copy_async(rf_ctx *ctx, void *dst, const void *src, uint64_t bytes, rf_stream_t stream);

/* Events for stream ordering and timing. */
int32_t rf_event_create(rf_ctx *ctx, void **event);
int32_t rf_event_destroy(rf_ctx *ctx, void *event);
int32_t rf_event_record(rf_ctx *ctx, void *event, rf_stream_t stream);
int32_t rf_stream_wait_event(rf_ctx *ctx, rf_stream_t stream, void *event);
int32_t rf_event_elapsed_ms(rf_ctx *ctx, void *start, void *stop, float *ms);
int32_t rf_event_synchronize(rf_ctx *ctx, void *event);

/* --------------------------------------------------------------- matvec */

/* y = W x for one GGUF tensor, kernel shape [out_dim, in_dim].
 * Replaces quant::matvec_<fmt> / matvec_<fmt>_row_range (core/src/quant.rs:
 * 898-1489) and, for RF_TYPE_F32, CpuBackend::matvec (runtime/src/backend.rs:
 * 173-218), i.e. everything compute_dispatch::matvec_backend routes to
 * (runtime/src/compute_dispatch.rs:40-58).  Rows [row_start, row_start +
 * row_count) are computed into the LOCAL y (y[0] <-> row_start,
 * quant.rs:907-912); row_count = RF_ALL_ROWS means through out_dim.
 * w_bytes is the size of the buffer behind w (validated like the
 * reference's w_bytes.len()).  x has in_dim floats, y has row_count floats. */
int32_t rf_matvec(rf_ctx *ctx, uint32_t ggml_type, const void *w, uint64_t w_bytes, uint64_t out_dim,
                  uint64_t in_dim, const float *x, float *y, uint64_t row_start, uint64_t row_count,
                  rf_stream_t stream);

/* Repack cache of rf_matvec (off by default; no counterpart in the
 * reference).  The reference's matvec seam is handed the same immutable
 * tensor bytes every token (compute_dispatch.rs:40-58 over a loaded
 * TensorData); with the cache on, rf_matvec's first call on a Q8_0, Q4_0,
 * Q4_K or Q6_K tensor packs all out_dim rows into a device copy in the
 * packed layout (below), and later calls with the same pointer, type,
 * out_dim and in_dim run the packed kernel on it.  Results are those of
 * rf_matvec_packed.  max_bytes bounds the copies (least recently used
 * evicted first); each is charged to the ledger as "workspace:repack:<n>"
 * and a tensor that does not fit runs uncached.  max_bytes = 0 turns the
 * cache off and frees it.  Eviction synchronises the device.  No entry is
 * added while the stream is being captured into a graph or once
 * rf_ctx_reserve has fixed the workspaces; a capture uses the entries whose
 * pack has completed by rf_capture_begin, and rf_graph_replay refuses such a
 * graph after any entry has been dropped (it may hold the freed copy).  A
 * graph captured by other means must not be replayed after a drop.
 * The caller's bytes must stay unchanged while cached: after changing or
 * freeing them, call rf_matvec_cache_forget on their range, which drops every
 * entry whose source bytes overlap [base, base + bytes). */
int32_t rf_matvec_cache(rf_ctx *ctx, uint64_t max_bytes);
int32_t rf_matvec_cache_forget(rf_ctx *ctx, const void *base, uint64_t bytes);
int32_t rf_matvec_cache_stats(rf_ctx *ctx, uint64_t *entries, uint64_t *bytes, uint64_t *hits,
                              uint64_t *misses);

/* Device-native ("packed") layout of Q8_0, Q4_0, Q4_K and Q6_K tensors, used
 * by the model for its weights.  No counterpart in the reference, which reads
 * GGUF blocks as stored; the arithmetic of rf_matvec_packed is that of
 * quant::matvec_q8_0 / matvec_q4_0 / matvec_q4_k / matvec_q6_k
 * (quant.rs:898-1327).  Layout of a [rows][in_dim] tensor, same byte count as
 * the GGUF payload: each block is cut into byte ranges ("regions") and every
 * region is stored for all blocks of all rows, row-major, one region after
 * the other:
 *   Q8_0: codes (bytes 2-33), f16 scale (0-1)
 *   Q4_0: codes (bytes 2-17, GGUF nibble order), f16 scale (0-1)
 *   Q4_K: qs (bytes 16-143), header d, dmin, scales[12] (0-15)
 *   Q6_K: ql (0-127), qh (128-191), scales (192-207), d (208-209)
 * rf_pack_weights converts a GGUF payload (raw and packed must not overlap);
 * rf_packed_supported(type, in_dim) is 1 when the packed kernel covers the
 * shape (in_dim a whole number of blocks, and the row's x staged in one
 * workgroup's LDS: about 4 bytes per element of in_dim, up to the current
 * device's limit, 160 KiB on gfx950, so in_dim <= 37888 for Q8_0 and <= 36864
 * for the others there, 14336 for all on a 64 KiB device). */
int32_t rf_packed_supported(uint32_t ggml_type, uint64_t in_dim);
int32_t rf_pack_weights(rf_ctx *ctx, uint32_t ggml_type, const void *raw, uint64_t raw_bytes, uint64_t rows,
                        uint64_t in_dim, void *packed, uint64_t packed_bytes, rf_stream_t stream);
/* rf_matvec on a packed tensor: same arguments, validation, row-range and
 * error rules (packed_bytes plays the role of w_bytes). */
int32_t rf_matvec_packed(rf_ctx *ctx, uint32_t ggml_type, const void *packed, uint64_t packed_bytes,
                         uint64_t out_dim, uint64_t in_dim, const float *x, float *y, uint64_t row_start,
                         uint64_t row_count, rf_stream_t stream);
/* Batched matvec for prompt prefill: y[t][o] = sum_i W[o][i] x[t][i] for
 * n_tokens rows of x ([n_tokens][in_dim]) on a packed tensor, into
 * y[n_tokens][out_dim].  No counterpart in the reference, which runs the
 * matvec once per prompt token (inference.rs:580-592); each y row is the
 * matvec of quant::matvec_q8_0 / _q4_0 / _q4_k / _q6_k (quant.rs:898-1327)
 * to f32 accuracy (summation order aside), computed on the matrix cores
 * (bf16 MFMA on exact integer codes and a three-piece bf16 split of x).
 * in_dim must be a whole number of blocks; validation as rf_matvec_packed
 * (packed_bytes >= out_dim rows). */
int32_t rf_matmul_packed(rf_ctx *ctx, uint32_t ggml_type, const void *packed, uint64_t packed_bytes,
                         uint64_t out_dim, uint64_t in_dim, const float *x, uint64_t n_tokens, float *y,
                         rf_stream_t stream);

/* Bit-exact row decode: rows [row_start, row_start + row_count) of a
 * [rows, in_dim] GGUF tensor into out[row_count][in_dim].  Replaces
 * dequantize_row_<fmt> (quant.rs:615-868) and decode_row_to_f32
 * (core/src/tensor.rs:801-866, incl. F32/F16/BF16). */
int32_t rf_dequantize_rows(rf_ctx *ctx, uint32_t ggml_type, const void *w, uint64_t w_bytes,
                           uint64_t in_dim, uint64_t row_start, uint64_t row_count, float *out,
                           rf_stream_t stream);

/* ------------------------------------------------------------ attention */

/* Single-token causal GQA attention: out[q_heads][head_dim].  Replaces
 * ops::attention_checked (runtime/src/ops.rs:49-69) ->
 * compute::attention_reference (core/src/compute.rs:461-547).  k_hist/v_hist
 * hold hist_len positions in [pos][kv_heads][head_dim] layout (KvCache,
 * runtime/src/kv_cache.rs:452-481); k_cur/v_cur are [kv_heads][head_dim];
 * q and k_cur are already rotated (RoPE is a separate call, as in
 * model_executor.rs:196-204).  Unlike the reference the output is written to
 * a caller-owned buffer instead of a fresh Vec. */
int32_t rf_attention_decode(rf_ctx *ctx, const float *q, const float *k_hist, const float *v_hist,
                            const float *k_cur, const float *v_cur, uint32_t hist_len, uint32_t q_heads,
                            uint32_t kv_heads, uint32_t head_dim, float *out, rf_stream_t stream);

/* rf_attention_decode for callers that cannot allocate device memory (code
 * under graph capture, serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  Same arguments, validation and results; the
 * split records (or score rows) live in a static device array of
 * RF_ATTENTION_NOALLOC_SCRATCH_BYTES per GPU instead of the context workspace,
 * so no call allocates, frees or synchronises.  A call whose shape needs more
 * scratch than that fails with RF_ERR_INVALID: with hd 128 that is about
 * 65536 positions at 32 query heads.  Every call on one GPU shares that GPU's
 * array: calls that may overlap on one GPU (several streams or contexts
 * without ordering between them) race and must not be issued. */
#define RF_ATTENTION_NOALLOC_SCRATCH_BYTES (8ull << 20)
int32_t rf_attention_decode_noalloc(rf_ctx *ctx, const float *q, const float *k_hist, const float *v_hist,
                                    const float *k_cur, const float *v_cur, uint32_t hist_len, uint32_t q_heads,
                                    uint32_t kv_heads, uint32_t head_dim, float *out, rf_stream_t stream);

/* ---------------------------------------------------------- elementwise */

/* ops::apply_rope -> compute::rope_reference (runtime/src/ops.rs:9-20,
 * core/src/compute.rs:389-456): half-split RoPE in place on q[q_heads][hd]
 * and k[kv_heads][hd].  cos/sin are computed on the host with the
 * reference's f32 expression and libm. */
int32_t rf_rope(rf_ctx *ctx, float *q, float *k, uint64_t position, uint32_t head_dim, uint32_t q_heads,
                uint32_t kv_heads, float theta, rf_stream_t stream);
/* compute::rms_norm_reference (compute.rs:291-319); ComputeBackend::rmsnorm. */
int32_t rf_rmsnorm(rf_ctx *ctx, const float *x, const float *weight, uint64_t n, float eps, float *out,
                   rf_stream_t stream);
/* add_reference / mul_reference / silu_reference / swiglu_reference
 * (compute.rs:321-361). */
int32_t rf_add(rf_ctx *ctx, const float *a, const float *b, uint64_t n, float *out, rf_stream_t stream);
/* In-place bias add v[i] += bias[i], the qwen2 Q/K/V bias step of
 * ModelExecutor::execute_layer (runtime/src/model_executor.rs:161-194). */
int32_t rf_bias_add(rf_ctx *ctx, float *v, const float *bias, uint64_t n, rf_stream_t stream);
int32_t rf_mul(rf_ctx *ctx, const float *a, const float *b, uint64_t n, float *out, rf_stream_t stream);
int32_t rf_silu(rf_ctx *ctx, const float *x, uint64_t n, float *out, rf_stream_t stream);
int32_t rf_swiglu(rf_ctx *ctx, const float *gate, const float *up, uint64_t n, float *out, rf_stream_t stream);
/* softmax_reference in place (compute.rs:363-384). */
int32_t rf_softmax(rf_ctx *ctx, float *values, uint64_t n, rf_stream_t stream);
/* Greedy Sampler::sample_checked (runtime/src/sampling.rs:45-57): the first
 * maximum wins; the index is written to DEVICE memory out_index. */
int32_t rf_argmax(rf_ctx *ctx, const float *logits, uint64_t n, uint32_t *out_index, rf_stream_t stream);

/* ------------------------------------------------- synthetic payloads */

/* Writes n_blocks GGUF blocks of ggml_type (F32: n_blocks floats) generated
 * from `seed` starting at global block index first_block, on the device.
 * Scale fields are f16(|n| * scale_mul) with n an Irwin-Hall(12) normal,
 * except the min scale of Q4_K / Q5_K / Q2_K: the block's decoded d times the
 * mean code (7.5 / 15.5 / 1.5), so that the weights are zero-mean.  Q8_0
 * codes are uniform in [-127, 127]; the other codes are uniform bytes.
 * Bench and test input generator; it has no counterpart in the reference. */
int32_t rf_synth_blocks(rf_ctx *ctx, uint32_t ggml_type, uint64_t seed, uint64_t first_block, uint64_t n_blocks,
                        double scale_mul, void *dst, uint64_t dst_bytes, rf_stream_t stream);

/* ---------------------------------------------------------------- model */

/* LlamaConfig (runtime/src/model.rs:26-37). */
typedef struct {
    uint64_t vocab_size;
    uint64_t context_length;
    uint64_t embedding_length;
    uint64_t block_count;
    uint64_t feed_forward_length;
    uint64_t head_count;
    uint64_t head_count_kv;
    uint64_t head_dim;
    float rms_eps;
    float rope_freq_base;
} rf_model_config;

/* A dense llama/qwen2 decoder whose weights live in VRAM (charges
 * "layer:{i}:{tensor}", "persistent:{tensor}", "kv_cache", "tmp:forward"),
 * executing StreamingLlamaModel::forward_single_streaming
 * (streaming_model.rs:909-1305) with ModelExecutor::execute_layer
 * (model_executor.rs:102-236) per layer, compute_logits
 * (streaming_model.rs:1334-1370) and the greedy loop of
 * InferenceEngine::generate_impl (inference.rs:445-759).  kv_capacity is the
 * KV cache capacity in tokens (<= context_length), allocated and charged
 * ("kv_cache:k", "kv_cache:v") at creation unless rf_model_kv_growth is
 * used; the attention workspaces and regimes are sized for it either way. */
int32_t rf_model_create(rf_ctx *ctx, const rf_model_config *cfg, uint64_t kv_capacity, rf_model **out);
void rf_model_destroy(rf_model *model);
/* Chunked KV growth (KvCache::GROW_CHUNK_TOKENS and grow_to_with_budget,
 * kv_cache.rs:49, 297-356, as inference.rs:478-496 and 666-687 use them):
 * the cache is reallocated to initial_tokens (1..=kv_capacity; only on an
 * empty cache) and from then on grows whenever a forward, prefill or decode
 * step needs a position past it, to the next multiple of 256 positions, at
 * most kv_capacity (rf_model_generate: at most the positions its prompt and
 * max_tokens need, starting from exactly the prompt's length).  Each growth
 * charges the replacement "kv_cache:{k,v}:growth" while the old buffers are
 * still charged, evicting streamed layers first when the budget is short;
 * on failure (RF_ERR_BUDGET, or the device allocation's error) the cache and
 * its charges are unchanged.  Growth drops captured decode graphs (they are
 * captured again at the next step). */
int32_t rf_model_kv_growth(rf_model *model, uint64_t initial_tokens);
/* rf_model_create with the KV cache allocated (and charged) for
 * initial_tokens positions only and growth enabled from the start, as the
 * reference sizes a new cache for the prompt (KvCache::new_with_budget,
 * inference.rs:478-496); kv_capacity bounds the growth. */
int32_t rf_model_create_growing(rf_ctx *ctx, const rf_model_config *cfg, uint64_t kv_capacity,
                                uint64_t initial_tokens, rf_model **out);
/* Positions the KV cache holds now (KvCache::capacity_tokens). */
int32_t rf_model_kv_capacity(rf_model *model, uint64_t *tokens);
/* Which kernels the model runs (no counterpart in the reference, which has
 * one CPU path; for tests and tools that must know which path they cover):
 * split_attention = 1 when decode attention runs the split-K kernel
 * (32/8/... query-KV head ratios with head_dim 64, 128 or 256), 0 for the
 * any-shape kernel; regime = the split kernel's launch regime (0-4) of a
 * decode step at position pos (0 for the any-shape kernel);
 * batched_prefill = 1 when rf_model_prefill (and rf_model_generate after
 * rf_model_set_prefill(1)) forwards prompts as batched GEMMs with the
 * tensors installed now, 0 when it falls back to one forward per token. */
int32_t rf_model_paths(rf_model *model, uint64_t pos, int32_t *split_attention, int32_t *regime,
                       int32_t *batched_prefill);

/* Installs tensor `name` (GGUF names: token_embd.weight, output_norm.weight,
 * output.weight, blk.{i}.{attn_norm,attn_q,attn_k,attn_v,attn_output,
 * ffn_norm,ffn_gate,ffn_up,ffn_down}.weight, blk.{i}.attn_{q,k,v}.bias) of
 * ggml shape [ne0 = in, ne1 = out] from host bytes (uploaded through a
 * pinned staging buffer on the copy stream). */
int32_t rf_model_set_tensor(rf_model *model, const char *name, uint32_t ggml_type, uint64_t ne0, uint64_t ne1,
                            const void *host_data, uint64_t nbytes);
/* Same, generating the payload on the device with rf_synth_blocks(seed,
 * scale_mul); F32 tensors may instead be a constant (constant != NaN). */
int32_t rf_model_synth_tensor(rf_model *model, const char *name, uint32_t ggml_type, uint64_t ne0, uint64_t ne1,
                              uint64_t seed, double scale_mul, float constant);
/* Resets the KV cache (seq_len = 0). */
int32_t rf_model_reset(rf_model *model);
uint64_t rf_model_seq_len(rf_model *model);

/* One forward pass for `token` at `pos` (must equal seq_len); optionally
 * copies the output-normed hidden state to host final_hidden[embedding]. */
int32_t rf_model_forward(rf_model *model, uint32_t token, uint64_t pos, float *final_hidden);
/* Logits of the last forward to host logits[vocab]. */
int32_t rf_model_logits(rf_model *model, float *logits);
/* Greedy generation: prompt tokens forwarded one at a time, then up to
 * max_tokens greedy tokens with the reference's stop rules (EOS when eos >= 0,
 * max tokens without a terminal forward, context length). */
int32_t rf_model_generate(rf_model *model, const uint32_t *prompt, uint64_t prompt_len, uint64_t max_tokens,
                          int64_t eos, uint32_t *out_tokens, uint64_t *n_out);
/* One decode step on the device (logits -> argmax -> embedding of the chosen
 * token -> forward), without host synchronisation: the token id stays in
 * device memory.  Used by the throughput benchmark after the prompt. */
int32_t rf_model_decode_steps(rf_model *model, uint64_t steps);
/* Copies the last `n` greedy tokens produced by rf_model_decode_steps. */
int32_t rf_model_read_tokens(rf_model *model, uint32_t *out, uint64_t n);
/* Batched prompt prefill: forwards tokens[0..n) at positions seq_len ..
 * seq_len + n - 1 in chunks of 64 tokens, each chunk through every layer
 * with the projections as rf_matmul_packed GEMMs, per-token RMSNorm, RoPE,
 * K/V cache writes and causal attention over the cache.  Same result as n
 * rf_model_forward calls (the reference's prompt loop, inference.rs:580-592)
 * to f32 accuracy; afterwards the model is where those calls leave it
 * (rf_model_logits, rf_model_decode_steps continue from the last token).
 * Models whose projections are not all in the packed layout (or whose
 * attention shape needs the any-shape kernel) are forwarded one token at a
 * time instead.  final_hidden as rf_model_forward, for the last token.  No
 * counterpart in the reference. */
int32_t rf_model_prefill(rf_model *model, const uint32_t *tokens, uint64_t n, float *final_hidden);
/* rf_model_generate forwards the prompt with rf_model_prefill (1) or one
 * token at a time as the reference does (0, default). */
int32_t rf_model_set_prefill(rf_model *model, int32_t batched);
/* Enables capture of one decode step into a hipGraph that is replayed by
 * rf_model_decode_steps (1) or eager launches (0, default). */
int32_t rf_model_use_graph(rf_model *model, int32_t enable);

/* VRAM residency tier with layer streaming (device side of load_layer,
 * release_layer and LayerCache: streaming_model.rs:555-873,
 * layer_cache.rs:74-268).  Must be called before any blk.* tensor is
 * installed.  Afterwards every block tensor is kept in pinned host memory (in
 * the device layout) and a forward pass uploads each layer it needs on the
 * copy stream: charges "layer:{i}:{tensor}" are made before the buffers are
 * allocated (all released again if one fails), the next layer's upload
 * overlaps the current layer's kernels, and a computed layer enters an LRU
 * cache of at most layer_cache_bytes (charges renamed "cache:layer:{i}:*",
 * least recently used layers evicted first; buffers are freed before their
 * charges are released).  A layer that cannot be cached is released after
 * the pass.  Loads evict cached layers until the context's VRAM budget holds
 * them; when even an empty cache leaves too little, the pass fails with
 * RF_ERR_BUDGET ("insufficient memory").  Graph replay and kernel timing are
 * unavailable in this mode. */
int32_t rf_model_enable_streaming(rf_model *model, uint64_t layer_cache_bytes);
/* Layer cache eviction policy: 0 = least recently used (LayerCache, the
 * default); 1 = the layer needed furthest in the future of the layer cycle
 * (optimal for decoding's in-order scan; a just-computed layer that would be
 * needed later than every cached one is released instead of cached).  No
 * counterpart in the reference for policy 1. */
int32_t rf_model_set_cache_policy(rf_model *model, int32_t policy);
/* Units of layer streaming per layer: 1 = the whole layer (the reference's
 * LayerCache entry, the default); 2 = the attention tensors with both norms,
 * then the feed-forward matrices (gate, up, down); 3 = the attention part,
 * then gate and up, then down.  Each unit is loaded, cached and evicted on
 * its own, so a budget that holds part of a layer keeps that part; the pass
 * acquires each unit while the previous one's kernels run.  Charges keep
 * their names ("layer:{i}:{tensor}", "cache:layer:{i}:{tensor}"); residency
 * stats and the cache count units.  Needs layer streaming; releases every
 * resident unit.  No counterpart in the reference. */
int32_t rf_model_set_stream_units(rf_model *model, int32_t per_layer);
/* out[6]: cache hits, misses (layer uploads), evictions, bytes uploaded,
 * bytes and layers currently cached. */
int32_t rf_model_residency_stats(rf_model *model, uint64_t *out);
/* Pinned host memory the model holds: host copies of streamed block tensors,
 * streamed persistent weights (mapped) and the byte source's two staging
 * buffers.  No counterpart in the reference. */
int32_t rf_model_host_bytes(rf_model *model, uint64_t *pinned);

/* Reads `length` bytes at `offset` of a model's byte source (its GGUF file or
 * the virtual concatenation of its shards: DataSource::read_range_into,
 * core/src/datasource.rs:574-700) into dst; returns 0 on success, any other
 * value is reported as RF_ERR_IO. */
typedef int32_t (*rf_read_fn)(void *user, uint64_t offset, uint64_t length, void *dst);
/* Streamed layers read from a byte source instead of pinned host copies
 * (the device side of load_layer's reads, streaming_model.rs:581-847): only
 * with layer streaming enabled and before any rf_model_set_tensor_source.
 * Two pinned staging buffers of staging_bytes each (>= 4096) are the host
 * memory the reads use; `read` is called on the thread that runs the forward
 * pass, one range at a time, and, with read-ahead on (rf_model_set_read_ahead;
 * the default for rf_file_source_read), also from the model's worker thread. */
int32_t rf_model_set_reader(rf_model *model, rf_read_fn read, void *user, uint64_t staging_bytes);
/* Read-ahead of the byte source (1 on, 0 off):
 * a worker thread of the model reads the next layer the pass will load from
 * the source (the next host-only layer in layer order) into a pinned buffer
 * of one layer's source bytes (allocated at the first read-ahead) while the
 * calling thread queues the layers before it; the pass then uploads from
 * that buffer.  `read` is then also called from the worker thread, so it
 * must be thread-safe.  On by default when `read` is rf_file_source_read,
 * off for other readers.  A failed read-ahead is reported by the load that
 * needs it, as RF_ERR_IO.  No counterpart in the reference (its reads run
 * on the forward pass's thread). */
int32_t rf_model_set_read_ahead(rf_model *model, int32_t on);
/* A byte source over a model file, for rf_model_set_reader: pass
 * rf_file_source_read as `read` and the handle as `user`.  Each read of
 * [offset, offset + length) is split over up to `threads` threads (pieces of
 * at least 4 MiB), each a pread loop into its part of dst (GgufDataSource's
 * read_range, core/src/datasource.rs:574-700, is one pread loop; the split is
 * this build's own, for reads from the page cache at memory speed).  Returns
 * 0 or the failing piece's errno (EIO for a short read past the file's end). */
typedef struct rf_file_source rf_file_source;
int32_t rf_file_source_open(const char *path, uint32_t threads, rf_file_source **out);
void rf_file_source_close(rf_file_source *source);
int32_t rf_file_source_read(void *source, uint64_t offset, uint64_t length, void *dst);
/* Declares block tensor `name` (blk.*) at [offset, offset + nbytes) of the
 * byte source; nothing is read now.  Each load of its layer reads the layer's
 * tensors as ranges merged while the gaps are at most 4 KiB and the span fits
 * a staging buffer (build_layer_read_plan, layer_read.rs:6-160; a tensor
 * larger than a buffer is read in buffer-sized pieces), copies them to the
 * layer's device buffers and repacks (packed projections) or widens
 * (F16 / BF16) them on the device through a raw buffer charged
 * "workspace:layer_read", sized at declaration for the largest such tensor.
 * A failed read releases every charge the load made (RF_ERR_IO). */
int32_t rf_model_set_tensor_source(rf_model *model, const char *name, uint32_t ggml_type, uint64_t ne0,
                                   uint64_t ne1, uint64_t offset, uint64_t nbytes);
/* out[2]: reader calls and bytes read from the byte source. */
int32_t rf_model_read_stats(rf_model *model, uint64_t *out);
/* Persistent weights of a streaming model (persistent.rs:1-6, 466-470):
 * policy 0 (default) keeps token_embd.weight / output.weight resident when
 * its device bytes are at most a quarter of the context's VRAM budget
 * (should_keep_resident) and streams it otherwise; 1 streams both, 2 keeps
 * both resident; 3 streams token_embd.weight regardless of its size (a
 * decode step reads one of its rows, so the VRAM it would take holds cached
 * layers instead) and applies policy 0 to output.weight (no counterpart in
 * the reference; for models with an output projection: a tied one reads the
 * embedding for the logits).  A streamed one stays in mapped pinned host memory (in the
 * device layout) that the kernels read in place: the embedding gather reads
 * one row per token, the logits matvec every row (streamed_matvec_into,
 * persistent.rs:286-463), and no VRAM is charged for it.  Set before those
 * tensors load; applies only with layer streaming enabled. */
int32_t rf_model_set_persistent_policy(rf_model *model, int32_t policy);
/* Bit 0: token_embd.weight is streamed; bit 1: output.weight is streamed. */
int32_t rf_model_persistent_streamed(rf_model *model, uint32_t *mask);
/* Profiler of the real forward (the reference's per-event records around each
 * matvec, compute_dispatch.rs:48-56, profile.rs:7-23): with enable = 1 every
 * launch group of the forwards, logits and eager decode steps that follow is
 * bracketed by HIP events on the compute stream and its device time added to
 * a per-group total.  Eager launches only: refused while graph replay is on
 * (and rf_model_use_graph(model, 1) is refused while it is on).  Same results
 * either way. */
int32_t rf_model_profile(rf_model *model, int32_t enable);
/* ms[6] / counts[6]: accumulated device milliseconds and launches per group,
 * indexed RF_KERNEL_QKV - 1 .. RF_KERNEL_LOGITS - 1; reset != 0 zeroes them
 * after reading (waits for the recorded events). */
int32_t rf_model_profile_read(rf_model *model, double *ms, uint64_t *counts, int32_t reset);

/* Launch groups of one decode step (see rf_model_time_kernel). */
#define RF_KERNEL_QKV 1       /* attn RMSNorm + Q/K/V matvec (+ bias)      */
#define RF_KERNEL_ATTENTION 2 /* RoPE + split-K attention + K/V commit     */
#define RF_KERNEL_OPROJ 3     /* attn_output matvec + residual             */
#define RF_KERNEL_GATEUP 4    /* ffn RMSNorm + gate/up matvec + SiLU*up    */
#define RF_KERNEL_DOWN 5      /* ffn_down matvec + residual                */
#define RF_KERNEL_LOGITS 6    /* output RMSNorm + output projection        */

/* Times one launch group exactly as a decode step launches it: for every
 * layer in order (RF_KERNEL_LOGITS: the output projection), `reps` times,
 * back-to-back on the compute stream between two HIP events.  Returns the
 * average milliseconds per launch, the average algorithmic HBM bytes per
 * launch (weights + vectors read + written; attention: the K/V history at the
 * current position) and the number of launches.  Activations are overwritten
 * with meaningless values: call rf_model_reset before decoding again.  Used
 * for the profiler's per-event times (runtime/src/profile.rs:7-23). */
int32_t rf_model_time_kernel(rf_model *model, uint32_t kind, uint32_t reps, float *avg_ms,
                             uint64_t *bytes_per_launch, uint64_t *launches);
/* Name of the packed matvec kernel instance one launch group runs (layer 0;
 * the o-projection as it follows the attention at the current position),
 * spelled as the profiler's kernel trace spells it, e.g.
 * "void rf::matvec_packed<8u, 2, true, 1, 2, 2, 512, false, false, false>(rf::PkArgs)";
 * "" when the group launches no packed matvec.  Nothing is launched.  No
 * counterpart in the reference: it ties measurements to the kernel that
 * ran. */
int32_t rf_model_kernel_name(rf_model *model, uint32_t kind, char *buf, uint64_t cap);

/* ------------------------------------------------------- graph capture */

/* Records the calls the caller enqueues on the context's compute stream
 * between rf_capture_begin and rf_capture_end into a hipGraph (thread-local
 * capture: other threads are unaffected), and replays it.  No counterpart in
 * the reference; used to time kernels without host launch overhead.
 * rf_graph_replay launches the graph `reps` times on the compute stream and
 * reports the mean milliseconds per replay (HIP events).  A graph captured
 * before one of the context's workspaces was replaced (grown) refers to the
 * freed buffer: rf_graph_replay refuses it with RF_ERR_INVALID. */
int32_t rf_capture_begin(rf_ctx *ctx);
int32_t rf_capture_end(rf_ctx *ctx, void **graph);
int32_t rf_graph_replay(rf_ctx *ctx, void *graph, uint32_t reps, float *ms_per_replay);
int32_t rf_graph_destroy(rf_ctx *ctx, void *graph);

/* ------------------------------------------------------------- tuning */

/* LDS bytes per one-shot matvec tile (4096..61440); returns the value in effect. */
uint32_t rf_tune_matvec_tile_bytes(uint32_t bytes);
/* Matvec kernel family for GGUF bytes: 2 = plain Q8_0 / Q4_0 / Q6_K
 * matvecs and Q4_K ones of up to 4096 inputs (rf_matvec, no fused norm or
 * epilogue; rows of an even block count, 16-byte aligned x, 4-byte aligned
 * weights, at most about 29000 inputs) stage each row per wavefront in LDS
 * through 16-byte loads, and plain F32 ones (16-byte aligned, at most 16384
 * inputs) load rows per wavefront straight into registers; the rest as 1
 * (default);
 * 1 = persistent streaming kernel where rows and bases are
 * 16-byte aligned, LDS-staged row tiles; 0 = one-shot tile kernel
 * everywhere; other values only query.  Returns the mode in effect
 * (process-wide). */
int32_t rf_tune_matvec_kernel(int32_t mode);
/* x of the packed Q8_0 / Q4_0 matvec: 0 = float x everywhere (default), 1 =
 * int8 digit planes on launches whose wavefronts hold >= 24 KiB of codes, 2 =
 * digit planes on every launch whose workgroup LDS holds them (in_dim up to
 * about 36000); other values only query.  Returns the mode in effect (process-wide).  With digit
 * planes each 16-element unit of x (times the RMSNorm weights where fused) is
 * rounded to 30-bit fixed point below its largest element: element k of unit
 * u is off by at most 2^(E_u - 31), 2^E_u the power of two above the unit's
 * largest |x|, so a row sum is off by at most sum_u 2^(E_u - 31) sum_k |w_k|
 * beyond f32 rounding.  The reference multiplies f32 x by each decoded weight
 * (quant.rs:977-1029); mode 0 does the same, in another summation order.
 * An x holding an infinity or NaN gives, in every mode and format of the
 * packed matvec, the reference's non-finite row results: NaN where a term
 * (decoded weight times x) is NaN or infinities of both signs meet, else the
 * one infinity. */
int32_t rf_tune_matvec_digits(int32_t mode);
/* Packed matvec launch shape: 1 = a launch whose rows each fit one step
 * (in_dim 4096 of Q8_0 / Q4_0 / Q4_K, float x, one matrix) with a wavefront
 * per row requests its row before staging x (default), 0 = the two-step ring
 * everywhere; other values only query.  Same results either way.  Returns
 * the mode in effect (process-wide). */
int32_t rf_tune_packed_inflight(int32_t mode);
/* Decode attention at contexts split per query head (up to 1024 positions
 * with 32 query heads): 1 = the o-projection merges the chunk records of the
 * split kernel while staging its x, so no merge kernel is launched (default;
 * packed Q8_0 / Q4_0 / Q4_K o-projections of q_heads * head_dim up to 4096),
 * 0 = the merge kernel, then the o-projection; other values only query.  The
 * two differ in rounding only (the merge's sums in another order).  Applies
 * to steps enqueued or captured afterwards.  Returns the mode in effect
 * (process-wide). */
int32_t rf_tune_attention_merge(int32_t mode);
/* Decode-step attention kernel (rf_attention_decode and model decode
 * steps; batched prefill keeps the two-pass kernel): the one-pass kernel
 * with an online softmax (each position slot keeps a running maximum,
 * exp-sum and weighted V sum) for launches with one workgroup per query head
 * (short contexts; 1, default), for every launch (2), or for none (0: the
 * two-pass kernel, scores of a chunk in LDS, then V).  Both write the same
 * chunk records; they differ in rounding only.  Other values only query.
 * Returns the mode in effect (process-wide). */
int32_t rf_tune_attention_kernel(int32_t mode);
/* Longest context (64, 128 or 256 positions) that decode attention serves
 * with one chunk per query head (no chunk records to merge, so the
 * o-projection reads x directly); 8 wavefronts per workgroup above 64.
 * Other values only query.  Applies to steps enqueued or captured
 * afterwards.  Returns the value in effect (process-wide). */
int32_t rf_tune_attention_single(int32_t positions);
/* Batched-prefill attention: the matrix-core kernel (16-token tiles per KV
 * head, each K / V row read once per tile; G = 1, 2, 4 or 8 query heads per
 * KV head, head_dim 64 or 128) for chunks whose last token sees more than
 * 1024 positions (1, default), for every chunk (2), or never (0: the decode
 * split kernel with a token dimension, each K / V row read once per token).
 * They differ in rounding only.  Other values only query.  Returns the mode
 * in effect (process-wide). */
int32_t rf_tune_prefill_attention(int32_t mode);
/* Weight layout of models created afterwards: 1 = Q8_0 / Q4_0 / Q4_K / Q6_K
 * projection weights are repacked at install into the device-native layout
 * (default; the batched prefill needs it), 0 = kept as GGUF bytes; other
 * values only query.  Applies to tensors
 * installed after the call.  Returns the mode in effect (process-wide). */
int32_t rf_tune_packed_weights(int32_t mode);

#ifdef __cplusplus
}
#endif
#endif
