/*
 * ramforge_oracle.h — CPU restatement of RAMforge's legacy decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker and the timed
 * CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product path (ramforge_amd/) never links,
 * loads or calls it.
 *
 * Every function restates one reference function (Rust, read as text under
 * crates/) with the same loop order and the same f32 operation sequence.  The
 * library is compiled with -ffp-contract=off so no multiply-add is fused
 * unless the reference itself fuses it (the AVX2 F32 dot, simd.rs:21-45).
 *
 * Errors: functions return 0 on success, nonzero on failure; the message is
 * readable through orc_last_error() and follows the reference's wording so
 * tests can match the same substrings.  On failure no output is written.
 */
#ifndef RAMFORGE_ORACLE_H
#define RAMFORGE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (core/src/types.rs:238-292). */
enum {
    ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q5_0 = 6, ORC_Q8_0 = 8,
    ORC_Q2_K = 10, ORC_Q3_K = 11, ORC_Q4_K = 12, ORC_Q5_K = 13,
    ORC_Q6_K = 14, ORC_Q8_K = 15, ORC_BF16 = 30
};

#define ORC_ROW_COUNT_ALL ((size_t)-1)

const char *orc_last_error(void);

/* quant.rs:40-65 (bit-for-bit, including its subnormal handling). */
float orc_f16_to_f32(uint16_t bits);
/* tensor.rs:1044-1047 */
float orc_bf16_to_f32(uint16_t bits);

/* Block geometry: elements per block and bytes per block (quant.rs:24-37). */
int orc_block_geometry(uint32_t ggml_type, size_t *block_elems, size_t *block_bytes);

/* dequantize_row_<fmt> (quant.rs:615-868) and decode_row_to_f32 for F32/F16/BF16
 * (tensor.rs:801-866). */
int orc_dequantize_row(uint32_t ggml_type, const uint8_t *bytes, size_t nbytes,
                       size_t n_elements, float *out, size_t out_len);

/* quant::matvec_<fmt> with kernel shape [out, in] (quant.rs:898-1489): the
 * fused row-dots for Q4_0 / Q6_K and decode-then-dot for the rest. */
int orc_matvec_quant(uint32_t ggml_type, const uint8_t *w, size_t w_len,
                     size_t out_dim, size_t in_dim, const float *x, size_t x_len,
                     float *y, size_t y_len);

/* matvec_q4_0_row_range / matvec_q6_k_row_range (quant.rs:913-975, 1265-1327):
 * y is local, y[0] <-> row_start; row_count == ORC_ROW_COUNT_ALL means None. */
int orc_matvec_quant_row_range(uint32_t ggml_type, const uint8_t *w, size_t w_len,
                               size_t out_dim, size_t in_dim, const float *x,
                               size_t x_len, float *y, size_t y_len,
                               size_t row_start, size_t row_count);

/* compute::quantized_matvec_reference (compute.rs:185-229), shape [in, out]. */
int orc_quantized_matvec_reference(uint32_t ggml_type, const uint8_t *raw, size_t raw_len,
                                   size_t input, size_t output, const float *x,
                                   size_t x_len, float *y, size_t y_len);

/* compute::matvec_f32_reference / _row_range (compute.rs:105-180). */
int orc_matvec_f32_reference(const float *w, size_t w_len, size_t input, size_t output,
                             const float *x, size_t x_len, float *y, size_t y_len);
int orc_matvec_f32_reference_row_range(const float *w, size_t w_len, size_t input,
                                       size_t output, const float *x, size_t x_len,
                                       float *y, size_t y_len, size_t row_start,
                                       size_t row_count);

/* CpuBackend::matvec (backend.rs:173-218) with w_shape = [in, out]:
 * threads > 1 && out >= 4 -> per-row dot on `threads` workers; use_simd selects
 * the AVX2 8-lane FMA dot (simd.rs:21-45) instead of the scalar reference. */
int orc_backend_matvec_f32(const float *w, size_t w_len, size_t in_dim, size_t out_dim,
                           const float *x, size_t x_len, float *y, size_t y_len,
                           int threads, int use_simd);

/* compute_dispatch::matvec_backend (compute_dispatch.rs:40-58, 90-254) for a
 * tensor of ggml shape [in, out]: F32 -> backend matvec; Q4_0 / Q6_K ->
 * row chunks over `threads` when out >= 128; other formats single-threaded. */
int orc_dispatch_matvec(uint32_t ggml_type, const void *data, size_t data_len,
                        size_t in_dim, size_t out_dim, const float *x, size_t x_len,
                        float *y, size_t y_len, int threads, int use_simd);

/* Parity-run accelerator: split the rows of every format over n threads in
 * orc_dispatch_matvec (identical results; 0 restores the reference policy). */
void orc_set_parity_threads(int n);

/* compute.rs:291-384 */
int orc_rms_norm(const float *input, const float *weight, size_t n, float eps, float *out);
int orc_add(const float *a, const float *b, size_t n, float *out);
int orc_mul(const float *a, const float *b, size_t n, float *out);
int orc_silu(const float *input, size_t n, float *out);
int orc_swiglu(const float *gate, const float *up, size_t n, float *out);
int orc_softmax(float *values, size_t n);

/* compute.rs:389-456, half-split RoPE in place on q [qh][hd] and k [kvh][hd]. */
int orc_rope(float *q, size_t q_len, float *k, size_t k_len, size_t position,
             size_t head_dim, size_t query_heads, size_t kv_heads, float theta);

/* compute.rs:461-547: out has query_heads * head_dim floats. */
int orc_attention(const float *q, size_t q_len, const float *k_hist, const float *v_hist,
                  size_t hist_elems, const float *k_cur, const float *v_cur, size_t cur_len,
                  size_t history_len, size_t query_heads, size_t kv_heads, size_t head_dim,
                  float *out, size_t out_len);

/* Greedy Sampler::sample_checked (sampling.rs:40-57): first maximum wins. */
uint32_t orc_argmax(const float *logits, size_t n);

/* ---------------------------------------------------------------------------
 * Dense llama decode (model_executor.rs:102-236, streaming_model.rs:909-1370,
 * inference.rs:445-759) over caller-owned host tensors.
 * ------------------------------------------------------------------------- */
typedef struct {
    uint32_t type;       /* ggml type id */
    const void *data;    /* raw GGUF payload (F32 as float) */
    size_t nbytes;
    size_t ne0, ne1;     /* ggml shape [in, out]; 1-D tensors use ne1 = 1 */
} orc_tensor;

typedef struct {
    orc_tensor attn_norm, attn_q, attn_k, attn_v, attn_output;
    orc_tensor ffn_norm, ffn_gate, ffn_up, ffn_down;
    orc_tensor attn_q_bias, attn_k_bias, attn_v_bias; /* data == NULL when absent */
} orc_layer;

typedef struct {
    size_t vocab_size, context_length, embedding_length, block_count;
    size_t feed_forward_length, head_count, head_count_kv, head_dim;
    float rms_eps, rope_freq_base;
} orc_config;

typedef struct orc_model orc_model;

int orc_model_create(const orc_config *cfg, const orc_tensor *token_embd,
                     const orc_tensor *output_norm, const orc_tensor *output /* may be NULL */,
                     const orc_layer *layers, size_t kv_capacity, int threads, int use_simd,
                     orc_model **out);
void orc_model_destroy(orc_model *m);
int orc_model_reset(orc_model *m);
size_t orc_model_seq_len(const orc_model *m);
/* forward_single_streaming: final_hidden gets the output-normed hidden state. */
int orc_model_forward(orc_model *m, uint32_t token, size_t pos, float *final_hidden);
/* compute_logits into logits[vocab] from final_hidden. */
int orc_model_logits(orc_model *m, const float *final_hidden, float *logits);
/* generate_impl's greedy loop: prompt, then up to max_tokens greedy tokens.
 * eos < 0 disables the EOS stop.  Returns the number of tokens written.
 * If logits_trace is non-NULL it receives (vocab) floats per generated token. */
int orc_model_generate(orc_model *m, const uint32_t *prompt, size_t prompt_len,
                       size_t max_tokens, int64_t eos, uint32_t *out_tokens,
                       size_t *n_out, float *top2_margin);

/* ---------------------------------------------------------------------------
 * Seeded synthetic payloads shared bit-for-bit with the device generator.
 * ------------------------------------------------------------------------- */
uint64_t orc_synth_u64(uint64_t seed, uint64_t index);
/* Fill `n_blocks` blocks of `ggml_type` starting at global block index
 * `first_block` of the stream `seed` (same layout as the device generator). */
int orc_synth_blocks(uint32_t ggml_type, uint64_t seed, uint64_t first_block,
                     uint64_t n_blocks, double scale_sigma, uint8_t *out);

#ifdef __cplusplus
}
#endif
#endif
