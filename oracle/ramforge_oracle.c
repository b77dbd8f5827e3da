/*
 * ramforge_oracle.c — CPU restatement of RAMforge's legacy decode path.
 *
 * TEST INFRASTRUCTURE ONLY (see ramforge_oracle.h).  Parity checker and timed
 * CPU baseline; never part of the product path.
 *
 * Citations are to the reference tree (Rust, read as text):
 *   core/src/quant.rs, core/src/compute.rs, core/src/tensor.rs,
 *   runtime/src/{backend,simd,compute_dispatch,model_executor,streaming_model,
 *   inference,sampling,kv_cache}.rs
 * Paths are relative to crates/ramforge-{core,runtime}/src.
 *
 * Build: gcc -O2 -ffp-contract=off -fopenmp -mavx2 -mfma (oracle/Makefile).
 * Rust never contracts a*b+c into an FMA, so neither may this file, except
 * where the reference calls an FMA intrinsic itself (simd.rs:33).
 */
#include "ramforge_oracle.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static __thread char g_err[512];

static int fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return 1;
}

const char *orc_last_error(void) { return g_err; }

/* ------------------------------------------------------------------------ */
/* f16 / bf16                                                                */
/* ------------------------------------------------------------------------ */

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* quant.rs:40-65.  The subnormal branch counts `e` with a test-then-shift
 * loop, so a subnormal half decodes to frac * 2^-25 (half its IEEE value).
 * Restated exactly; device decoders must reproduce it. */
float orc_f16_to_f32(uint16_t bits) {
    uint32_t sign = (bits >> 15) & 1u;
    uint32_t exp = (bits >> 10) & 0x1Fu;
    uint32_t frac = bits & 0x3FFu;
    uint32_t out;
    if (exp == 0) {
        if (frac == 0) {
            out = sign << 31;
        } else {
            uint32_t e = 0, f = frac;
            while ((f & 0x400u) == 0) { f <<= 1; e += 1; }
            f &= 0x3FFu;
            uint32_t ex = 127u - 15u - e;
            out = (sign << 31) | (ex << 23) | (f << 13);
        }
    } else if (exp == 0x1F) {
        out = (sign << 31) | (0xFFu << 23) | (frac << 13);
    } else {
        out = (sign << 31) | ((exp + (127u - 15u)) << 23) | (frac << 13);
    }
    return bits_f32(out);
}

/* tensor.rs:1044-1047 */
float orc_bf16_to_f32(uint16_t bits) { return bits_f32((uint32_t)bits << 16); }

static inline float rd_f16(const uint8_t *p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }
static inline float rd_f32(const uint8_t *p) { float f; memcpy(&f, p, 4); return f; }

/* ------------------------------------------------------------------------ */
/* Block geometry (quant.rs:24-37) and names (types.rs)                      */
/* ------------------------------------------------------------------------ */

static const char *type_name(uint32_t t) {
    switch (t) {
    case ORC_F32: return "F32"; case ORC_F16: return "F16"; case ORC_BF16: return "BF16";
    case ORC_Q4_0: return "Q4_0"; case ORC_Q5_0: return "Q5_0"; case ORC_Q8_0: return "Q8_0";
    case ORC_Q2_K: return "Q2_K"; case ORC_Q3_K: return "Q3_K"; case ORC_Q4_K: return "Q4_K";
    case ORC_Q5_K: return "Q5_K"; case ORC_Q6_K: return "Q6_K"; case ORC_Q8_K: return "Q8_K";
    default: return "unknown";
    }
}

int orc_block_geometry(uint32_t t, size_t *qk, size_t *bs) {
    size_t a, b;
    switch (t) {
    case ORC_Q4_0: a = 32; b = 18; break;
    case ORC_Q5_0: a = 32; b = 22; break;
    case ORC_Q8_0: a = 32; b = 34; break;
    case ORC_Q2_K: a = 256; b = 84; break;
    case ORC_Q3_K: a = 256; b = 110; break;
    case ORC_Q4_K: a = 256; b = 144; break;
    case ORC_Q5_K: a = 256; b = 176; break;
    case ORC_Q6_K: a = 256; b = 210; break;
    case ORC_Q8_K: a = 256; b = 292; break;
    case ORC_F32: a = 1; b = 4; break;
    case ORC_F16: case ORC_BF16: a = 1; b = 2; break;
    default: return fail("no reference row layout registered for type %u", t);
    }
    if (qk) *qk = a;
    if (bs) *bs = b;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Block decoders (BlockXxx::dequantize)                                     */
/* ------------------------------------------------------------------------ */

/* quant.rs:104-112 */
static void deq_q4_0(const uint8_t *b, float *out) {
    float d = rd_f16(b);
    const uint8_t *qs = b + 2;
    for (int j = 0; j < 16; j++) {
        int q0 = (int)(qs[j] & 0x0F) - 8;
        int q1 = (int)(qs[j] >> 4) - 8;
        out[j] = (float)q0 * d;
        out[16 + j] = (float)q1 * d;
    }
}

/* quant.rs:140-150 */
static void deq_q5_0(const uint8_t *b, float *out) {
    float d = rd_f16(b);
    uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
    const uint8_t *qs = b + 6;
    for (int j = 0; j < 16; j++) {
        uint8_t xh0 = (uint8_t)(((qh >> j) << 4) & 0x10u);
        uint8_t xh1 = (uint8_t)((qh >> (j + 12)) & 0x10u);
        int q0 = (int)((qs[j] & 0x0F) | xh0) - 16;
        int q1 = (int)((qs[j] >> 4) | xh1) - 16;
        out[j] = (float)q0 * d;
        out[16 + j] = (float)q1 * d;
    }
}

/* quant.rs:177-181 */
static void deq_q8_0(const uint8_t *b, float *out) {
    float d = rd_f16(b);
    for (int i = 0; i < 32; i++) out[i] = (float)(int8_t)b[2 + i] * d;
}

/* quant.rs:216-226 (BlockQ4K::get_scale_min; Q5_K's copy is identical, 283-291) */
static void get_scale_min(const uint8_t *sc, int j, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = sc[j] & 63;
        *m = sc[j + 4] & 63;
    } else {
        *d = (uint8_t)((sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4));
        *m = (uint8_t)((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
    }
}

/* quant.rs:228-254 */
static void deq_q4_k(const uint8_t *b, float *out) {
    float d = rd_f16(b), dmin = rd_f16(b + 2);
    const uint8_t *scales = b + 4, *qs = b + 16;
    int y = 0, is = 0, qo = 0;
    for (int g = 0; g < 4; g++) {
        uint8_t sc0, m0, sc1, m1;
        get_scale_min(scales, is, &sc0, &m0);
        get_scale_min(scales, is + 1, &sc1, &m1);
        float d1 = d * (float)sc0, min1 = dmin * (float)m0;
        float d2 = d * (float)sc1, min2 = dmin * (float)m1;
        for (int l = 0; l < 32; l++) out[y + l] = d1 * (float)(qs[qo + l] & 0x0F) - min1;
        y += 32;
        for (int l = 0; l < 32; l++) out[y + l] = d2 * (float)(qs[qo + l] >> 4) - min2;
        y += 32;
        qo += 32;
        is += 2;
    }
}

/* quant.rs:293-342.  The high-bit byte is qh[q_offset/4 + l/8] (reference
 * indexing, not ggml's qh[l]). */
static void deq_q5_k(const uint8_t *b, float *out) {
    float d = rd_f16(b), dmin = rd_f16(b + 2);
    const uint8_t *scales = b + 4, *qh = b + 16, *qs = b + 48;
    int y = 0, is = 0, qo = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int g = 0; g < 4; g++) {
        uint8_t sc0, m0, sc1, m1;
        get_scale_min(scales, is, &sc0, &m0);
        get_scale_min(scales, is + 1, &sc1, &m1);
        float d1 = d * (float)sc0, min1 = dmin * (float)m0;
        float d2 = d * (float)sc1, min2 = dmin * (float)m1;
        for (int l = 0; l < 32; l++) {
            uint8_t q = qs[qo + l] & 0xF;
            uint8_t high = (qh[qo / 4 + l / 8] & u1) ? 16 : 0;
            out[y + l] = d1 * (float)(uint8_t)(q + high) - min1;
        }
        y += 32;
        for (int l = 0; l < 32; l++) {
            uint8_t q = qs[qo + l] >> 4;
            uint8_t high = (qh[qo / 4 + l / 8] & u2) ? 16 : 0;
            out[y + l] = d2 * (float)(uint8_t)(q + high) - min2;
        }
        y += 32;
        qo += 32;
        is += 2;
        u1 = (uint8_t)(u1 << 2);
        u2 = (uint8_t)(u2 << 2);
    }
}

/* quant.rs:376-406: out = (d * sc) * q. */
static void deq_q6_k(const uint8_t *b, float *out) {
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    float d = rd_f16(b + 208);
    int yp = 0, qlo = 0, qho = 0, sco = 0;
    for (int h = 0; h < 2; h++) {
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)(int8_t)((ql[qlo + l] & 0xF) | ((qh[qho + l] & 3) << 4)) - 32;
            int q2 = (int)(int8_t)((ql[qlo + 32 + l] & 0xF) | (((qh[qho + l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)(int8_t)((ql[qlo + l] >> 4) | (((qh[qho + l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)(int8_t)((ql[qlo + 32 + l] >> 4) | (((qh[qho + l] >> 6) & 3) << 4)) - 32;
            out[yp + l] = d * (float)sc[sco + is] * (float)q1;
            out[yp + l + 32] = d * (float)sc[sco + is + 2] * (float)q2;
            out[yp + l + 64] = d * (float)sc[sco + is + 4] * (float)q3;
            out[yp + l + 96] = d * (float)sc[sco + is + 6] * (float)q4;
        }
        yp += 128;
        qlo += 64;
        qho += 32;
        sco += 8;
    }
}

/* quant.rs:441-472 */
static void deq_q2_k(const uint8_t *b, float *out) {
    const uint8_t *scales = b, *qs = b + 16;
    float d = rd_f16(b + 80), dmin = rd_f16(b + 82);
    int y = 0, is = 0, qo = 0;
    for (int h = 0; h < 2; h++) {
        int shift = 0;
        for (int k = 0; k < 4; k++) {
            uint8_t sc = scales[is++];
            float dl = d * (float)(sc & 0xF), ml = dmin * (float)(sc >> 4);
            for (int l = 0; l < 16; l++) {
                int q = (qs[qo + l] >> shift) & 3;
                out[y + l] = dl * (float)q - ml;
            }
            y += 16;
            sc = scales[is++];
            dl = d * (float)(sc & 0xF);
            ml = dmin * (float)(sc >> 4);
            for (int l = 0; l < 16; l++) {
                int q = (qs[qo + 16 + l] >> shift) & 3;
                out[y + l] = dl * (float)q - ml;
            }
            y += 16;
            shift += 2;
        }
        qo += 32;
    }
}

/* quant.rs:508-574.  Both 128-element halves use scales[j] and scales[j+4]
 * (reference indexing, not ggml's running scale index). */
static void deq_q3_k(const uint8_t *b, float *out) {
    const uint8_t *hmask = b, *qs = b + 32, *scb = b + 96;
    float d = rd_f16(b + 108);
    uint32_t aux[4] = {0, 0, 0, 0};
    for (int i = 0; i < 3; i++)
        aux[i] = (uint32_t)scb[4 * i] | ((uint32_t)scb[4 * i + 1] << 8) |
                 ((uint32_t)scb[4 * i + 2] << 16) | ((uint32_t)scb[4 * i + 3] << 24);
    const uint32_t kmask1 = 0x03030303u, kmask2 = 0x0F0F0F0Fu;
    uint32_t tmp = aux[2], a0 = aux[0], a1 = aux[1];
    aux[2] = ((a0 >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4);
    aux[3] = ((a1 >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4);
    aux[0] = (a0 & kmask2) | (((tmp >> 0) & kmask1) << 4);
    aux[1] = (a1 & kmask2) | (((tmp >> 2) & kmask1) << 4);
    int8_t sc8[16];
    for (int i = 0; i < 4; i++)
        for (int k = 0; k < 4; k++) sc8[4 * i + k] = (int8_t)(uint8_t)(aux[i] >> (8 * k));
    int y = 0, qo = 0;
    uint8_t m = 1;
    for (int h = 0; h < 2; h++) {
        int shift = 0;
        for (int j = 0; j < 4; j++) {
            int sc = (int)sc8[j] - 32;
            float dl = d * (float)sc;
            for (int l = 0; l < 16; l++) {
                int q = (qs[qo + l] >> shift) & 3;
                q -= (hmask[l] & m) ? 0 : 4;
                out[y + l] = dl * (float)q;
            }
            y += 16;
            sc = (int)sc8[j + 4] - 32;
            dl = d * (float)sc;
            for (int l = 0; l < 16; l++) {
                int q = (qs[qo + 16 + l] >> shift) & 3;
                q -= (hmask[16 + l] & m) ? 0 : 4;
                out[y + l] = dl * (float)q;
            }
            y += 16;
            shift += 2;
            m = (uint8_t)(m << 1);
        }
        qo += 32;
    }
}

/* quant.rs:607-611 */
static void deq_q8_k(const uint8_t *b, float *out) {
    float d = rd_f32(b);
    for (int i = 0; i < 256; i++) out[i] = d * (float)(int8_t)b[4 + i];
}

typedef void (*deq_fn)(const uint8_t *, float *);

static deq_fn decoder_for(uint32_t t) {
    switch (t) {
    case ORC_Q4_0: return deq_q4_0; case ORC_Q5_0: return deq_q5_0; case ORC_Q8_0: return deq_q8_0;
    case ORC_Q2_K: return deq_q2_k; case ORC_Q3_K: return deq_q3_k; case ORC_Q4_K: return deq_q4_k;
    case ORC_Q5_K: return deq_q5_k; case ORC_Q6_K: return deq_q6_k; case ORC_Q8_K: return deq_q8_k;
    default: return NULL;
    }
}

static int is_quant(uint32_t t) { return decoder_for(t) != NULL; }

/* ------------------------------------------------------------------------ */
/* Row decode: dequantize_row_<fmt> (quant.rs:615-868), decode_row_to_f32    */
/* (tensor.rs:801-866)                                                       */
/* ------------------------------------------------------------------------ */

int orc_dequantize_row(uint32_t t, const uint8_t *bytes, size_t nbytes, size_t n, float *out,
                       size_t out_len) {
    if (t == ORC_F32 || t == ORC_F16 || t == ORC_BF16) {
        size_t w = (t == ORC_F32) ? 4 : 2;
        if (out_len != n) return fail("decode_row_to_f32: out buffer %zu != num_elements %zu", out_len, n);
        if (nbytes < n * w)
            return fail("%s row truncated: expected %zu bytes, got %zu", t == ORC_F32 ? "F32" : "F16/BF16", n * w, nbytes);
        for (size_t i = 0; i < n; i++) {
            if (t == ORC_F32) out[i] = rd_f32(bytes + 4 * i);
            else {
                uint16_t v = (uint16_t)(bytes[2 * i] | (bytes[2 * i + 1] << 8));
                out[i] = (t == ORC_F16) ? orc_f16_to_f32(v) : orc_bf16_to_f32(v);
            }
        }
        return 0;
    }
    deq_fn f = decoder_for(t);
    size_t qk, bs;
    if (!f || orc_block_geometry(t, &qk, &bs)) return fail("decode_row_to_f32: unsupported tensor type %s", type_name(t));
    if (n % qk != 0)
        return fail("%s row size %zu not divisible by block size %zu", type_name(t), n, qk);
    size_t nb = n / qk;
    if (nbytes < nb * bs)
        return fail("%s row truncated: expected %zu bytes, got %zu", type_name(t), nb * bs, nbytes);
    if (out_len < n) return fail("%s row output too short: %zu < %zu", type_name(t), out_len, n);
    float tmp[256];
    for (size_t i = 0; i < nb; i++) {
        f(bytes + i * bs, tmp);
        memcpy(out + i * qk, tmp, qk * sizeof(float));
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Quantized matvec kernels (kernel shape [out, in])                         */
/* ------------------------------------------------------------------------ */

/* quant.rs:875-895: interleaved low/high nibble accumulation per block. */
static float q4_0_row_dot(const uint8_t *row, size_t blocks, const float *x) {
    float sum = 0.0f;
    size_t xo = 0, off = 0;
    for (size_t b = 0; b < blocks; b++) {
        float d = rd_f16(row + off);
        off += 2;
        for (int j = 0; j < 16; j++) {
            uint8_t byte = row[off + j];
            int q0 = (int)(byte & 0x0F) - 8;
            int q1 = (int)(byte >> 4) - 8;
            sum += (float)q0 * d * x[xo + j];
            sum += (float)q1 * d * x[xo + 16 + j];
        }
        off += 16;
        xo += 32;
    }
    return sum;
}

/* quant.rs:1195-1252: sc = (scale as f32) * d, then sc * q * x, order l, l+32,
 * l+64, l+96. */
static float q6_k_row_dot(const uint8_t *row, size_t blocks, const float *x) {
    float sum = 0.0f;
    size_t xo = 0, off = 0;
    for (size_t b = 0; b < blocks; b++) {
        const uint8_t *ql = row + off, *qh = row + off + 128, *scales = row + off + 192;
        float d = rd_f16(row + off + 208);
        off += 210;
        int qlo = 0, qho = 0, sco = 0;
        for (int h = 0; h < 2; h++) {
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                uint8_t qhb = qh[qho + l], lo = ql[qlo + l], hi = ql[qlo + 32 + l];
                float sc1 = (float)(int8_t)scales[sco + is] * d;
                float sc2 = (float)(int8_t)scales[sco + is + 2] * d;
                float sc3 = (float)(int8_t)scales[sco + is + 4] * d;
                float sc4 = (float)(int8_t)scales[sco + is + 6] * d;
                int q1 = (int)(int8_t)((lo & 0x0F) | ((qhb & 0x03) << 4)) - 32;
                int q2 = (int)(int8_t)((hi & 0x0F) | (((qhb >> 2) & 0x03) << 4)) - 32;
                int q3 = (int)(int8_t)((lo >> 4) | (((qhb >> 4) & 0x03) << 4)) - 32;
                int q4 = (int)(int8_t)((hi >> 4) | (((qhb >> 6) & 0x03) << 4)) - 32;
                sum += sc1 * (float)q1 * x[xo + l];
                sum += sc2 * (float)q2 * x[xo + l + 32];
                sum += sc3 * (float)q3 * x[xo + l + 64];
                sum += sc4 * (float)q4 * x[xo + l + 96];
            }
            xo += 128;
            qlo += 64;
            qho += 32;
            sco += 8;
        }
    }
    return sum;
}

/* quant.rs:913-975 / 1265-1327 */
int orc_matvec_quant_row_range(uint32_t t, const uint8_t *w, size_t w_len, size_t out_dim,
                               size_t in_dim, const float *x, size_t x_len, float *y,
                               size_t y_len, size_t row_start, size_t row_count) {
    const char *nm = type_name(t);
    if (t != ORC_Q4_0 && t != ORC_Q6_K) return fail("row-range kernel exists only for Q4_0 and Q6_K, got %s", nm);
    if (x_len != in_dim)
        return fail("matvec input shape mismatch: W [%zu, %zu], x %zu", out_dim, in_dim, x_len);
    if (row_start > out_dim) return fail("%s row start %zu exceeds out_dim %zu", nm, row_start, out_dim);
    if (row_count == ORC_ROW_COUNT_ALL) row_count = out_dim - row_start;
    size_t row_end = row_start + row_count;
    if (row_end < row_start) return fail("%s row range overflow", nm);
    if (row_end > out_dim || y_len != row_count)
        return fail("%s row range %zu..%zu requires local y length %zu, got %zu for out_dim %zu", nm,
                    row_start, row_end, row_count, y_len, out_dim);
    size_t qk = (t == ORC_Q4_0) ? 32 : 256, bs = (t == ORC_Q4_0) ? 18 : 210;
    if (in_dim % qk != 0) return fail("%s in_dim %zu not divisible by %zu", nm, in_dim, qk);
    size_t bpr = in_dim / qk, rb = bpr * bs;
    if (w_len < out_dim * rb) return fail("%s weight truncated: expected %zu bytes, got %zu", nm, out_dim * rb, w_len);
    for (size_t i = row_start; i < row_end; i++) {
        const uint8_t *row = w + i * rb;
        y[i - row_start] = (t == ORC_Q4_0) ? q4_0_row_dot(row, bpr, x) : q6_k_row_dot(row, bpr, x);
    }
    return 0;
}

/* quant.rs:977-1029 (Q8_0) and the identical decode-then-dot bodies of
 * matvec_q5_0 1031-1083, matvec_q4_k 1085-1137, matvec_q5_k 1139-1191,
 * matvec_q2_k 1329-1381, matvec_q3_k 1383-1435, matvec_q8_k 1437-1489. */
static int matvec_decode_then_dot(uint32_t t, const uint8_t *w, size_t w_len, size_t out_dim,
                                  size_t in_dim, const float *x, size_t x_len, float *y,
                                  size_t y_len, size_t r0, size_t r1) {
    const char *nm = type_name(t);
    if (x_len != in_dim || y_len != out_dim)
        return fail("matvec shape mismatch: W [%zu, %zu], x %zu, y %zu", out_dim, in_dim, x_len, y_len);
    size_t qk, bs;
    orc_block_geometry(t, &qk, &bs);
    if (in_dim % qk != 0) return fail("%s in_dim %zu not divisible by %zu", nm, in_dim, qk);
    size_t rb = (in_dim / qk) * bs;
    if (w_len < out_dim * rb) return fail("%s weight truncated: expected %zu bytes, got %zu", nm, out_dim * rb, w_len);
    deq_fn f = decoder_for(t);
    float deq[256];
    for (size_t i = r0; i < r1; i++) {
        const uint8_t *row = w + i * rb;
        float sum = 0.0f;
        for (size_t b = 0; b < in_dim / qk; b++) {
            f(row + b * bs, deq);
            const float *xb = x + b * qk;
            for (size_t j = 0; j < qk; j++) sum += deq[j] * xb[j];
        }
        y[i] = sum;
    }
    return 0;
}

/* Parity-run accelerator (never used for the timed CPU baseline): when > 1,
 * orc_dispatch_matvec splits the rows of every format over this many threads.
 * Each row's arithmetic is unchanged, so results are identical to the
 * reference's single-threaded kernels. */
static int g_parity_threads = 0;
void orc_set_parity_threads(int n) { g_parity_threads = n; }

int orc_matvec_quant(uint32_t t, const uint8_t *w, size_t w_len, size_t out_dim, size_t in_dim,
                     const float *x, size_t x_len, float *y, size_t y_len) {
    if (!is_quant(t)) return fail("quantized matvec does not support type %s", type_name(t));
    if (t == ORC_Q4_0 || t == ORC_Q6_K)
        return orc_matvec_quant_row_range(t, w, w_len, out_dim, in_dim, x, x_len, y, y_len, 0, ORC_ROW_COUNT_ALL);
    if (g_parity_threads > 1 && out_dim >= 64) {
        int err = matvec_decode_then_dot(t, w, w_len, out_dim, in_dim, x, x_len, y, y_len, 0, 0);
        if (err) return err;
        int n = g_parity_threads;
#pragma omp parallel for num_threads(n) schedule(static) reduction(| : err)
        for (int c = 0; c < n; c++) {
            size_t r0 = out_dim * (size_t)c / (size_t)n, r1 = out_dim * (size_t)(c + 1) / (size_t)n;
            err |= matvec_decode_then_dot(t, w, w_len, out_dim, in_dim, x, x_len, y, y_len, r0, r1);
        }
        return err;
    }
    return matvec_decode_then_dot(t, w, w_len, out_dim, in_dim, x, x_len, y, y_len, 0, out_dim);
}

/* compute.rs:185-229 */
int orc_quantized_matvec_reference(uint32_t t, const uint8_t *raw, size_t raw_len, size_t input,
                                   size_t output, const float *x, size_t x_len, float *y,
                                   size_t y_len) {
    if (x_len != input || y_len != output)
        return fail("quantized matvec shape mismatch: shape [%zu, %zu], x %zu, y %zu", input, output, x_len, y_len);
    size_t qk, bs;
    if (!is_quant(t) || orc_block_geometry(t, &qk, &bs))
        return fail("no reference row layout registered for %s", type_name(t));
    if (input % qk != 0)
        return fail("%s input dimension %zu is not divisible by block width %zu", type_name(t), input, qk);
    size_t rb = (input / qk) * bs;
    if (raw_len < rb * output)
        return fail("quantized weight buffer truncated: expected %zu, got %zu", rb * output, raw_len);
    float *dec = (float *)malloc(input * sizeof(float));
    if (!dec) return fail("failed to reserve decoded quantized row");
    for (size_t o = 0; o < output; o++) {
        if (orc_dequantize_row(t, raw + o * rb, rb, input, dec, input)) { free(dec); return 1; }
        float sum = 0.0f;
        for (size_t i = 0; i < input; i++) sum += dec[i] * x[i];
        y[o] = sum;
    }
    free(dec);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* F32 matvec                                                                */
/* ------------------------------------------------------------------------ */

/* compute.rs:105-121 */
int orc_matvec_f32_reference(const float *w, size_t w_len, size_t input, size_t output,
                             const float *x, size_t x_len, float *y, size_t y_len) {
    if (w_len != input * output || x_len != input || y_len != output)
        return fail("matvec arity mismatch: shape [input=%zu, output=%zu] requires weights exactly %zu, x %zu, y %zu; got weights %zu, x %zu, y %zu",
                    input, output, input * output, input, output, w_len, x_len, y_len);
    for (size_t o = 0; o < output; o++) {
        const float *row = w + o * input;
        float sum = 0.0f;
        for (size_t i = 0; i < input; i++) sum += row[i] * x[i];
        y[o] = sum;
    }
    return 0;
}

/* compute.rs:126-180 */
int orc_matvec_f32_reference_row_range(const float *w, size_t w_len, size_t input, size_t output,
                                       const float *x, size_t x_len, float *y, size_t y_len,
                                       size_t row_start, size_t row_count) {
    if (row_start + row_count < row_start || row_start + row_count > output)
        return fail("row range %zu..%zu exceeds output dimension %zu", row_start, row_start + row_count, output);
    if (y_len != row_count) return fail("row-range output length mismatch: expected %zu, got %zu", row_count, y_len);
    if (x_len != input) return fail("row-range input length mismatch: expected %zu, got %zu", input, x_len);
    if (w_len != input * output) return fail("matrix weight buffer length mismatch: expected %zu, got %zu", input * output, w_len);
    for (size_t r = 0; r < row_count; r++) {
        const float *row = w + (row_start + r) * input;
        float sum = 0.0f;
        for (size_t i = 0; i < input; i++) sum += row[i] * x[i];
        y[r] = sum;
    }
    return 0;
}

/* simd.rs:21-45: 8 FMA lanes, store, `iter().sum()` of the lanes in order,
 * then a mul-then-add scalar remainder. */
static float dot_avx2_order(const float *a, const float *b, size_t len) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t i = 0;
    for (; i + 8 <= len; i += 8)
        for (int l = 0; l < 8; l++) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
    float total = -0.0f;
    for (int l = 0; l < 8; l++) total += acc[l];
    for (; i < len; i++) total += a[i] * b[i];
    return total;
}

/* simd.rs:17-19: `map(x*y).sum()`, sequential. */
static float dot_scalar(const float *a, const float *b, size_t len) {
    float total = -0.0f;
    for (size_t i = 0; i < len; i++) total += a[i] * b[i];
    return total;
}

/* simd.rs:48-54 */
static float dot_f32_avx2(const float *a, const float *b, size_t len) {
    return len >= 8 ? dot_avx2_order(a, b, len) : dot_scalar(a, b, len);
}

/* backend.rs:173-218 (matvec_rows_parallel 133-149, matvec_f32_avx2 simd.rs:62-83) */
int orc_backend_matvec_f32(const float *w, size_t w_len, size_t in_dim, size_t out_dim,
                           const float *x, size_t x_len, float *y, size_t y_len, int threads,
                           int use_simd) {
    if (x_len != in_dim || y_len != out_dim || w_len < in_dim * out_dim)
        return fail("backend matvec arity mismatch (ggml layout [in, out]): shape [%zu, %zu] implies in=%zu, out=%zu, but got w.len()=%zu, x.len()=%zu, y.len()=%zu",
                    in_dim, out_dim, in_dim, out_dim, w_len, x_len, y_len);
    if (threads > 1 && out_dim >= 4) {
#pragma omp parallel for num_threads(threads) schedule(static)
        for (size_t o = 0; o < out_dim; o++) {
            const float *row = w + o * in_dim;
            if (use_simd) {
                y[o] = dot_f32_avx2(row, x, in_dim);
            } else {
                float sum = 0.0f;
                for (size_t i = 0; i < in_dim; i++) sum += row[i] * x[i];
                y[o] = sum;
            }
        }
    } else if (use_simd && in_dim >= 8) {
        for (size_t o = 0; o < out_dim; o++) y[o] = dot_avx2_order(w + o * in_dim, x, in_dim);
    } else {
        for (size_t o = 0; o < out_dim; o++) {
            const float *row = w + o * in_dim;
            float sum = 0.0f;
            for (size_t i = 0; i < in_dim; i++) sum += row[i] * x[i];
            y[o] = sum;
        }
    }
    return 0;
}

/* compute_dispatch.rs:76-88 */
static size_t make_row_chunks(size_t out_dim, size_t n_chunks, size_t *starts, size_t *counts) {
    size_t n = n_chunks < out_dim ? n_chunks : out_dim;
    if (n < 1) n = 1;
    size_t base = out_dim / n, extra = out_dim % n, cur = 0;
    for (size_t i = 0; i < n; i++) {
        size_t c = base + (i < extra ? 1 : 0);
        starts[i] = cur;
        counts[i] = c;
        cur += c;
    }
    return n;
}

/* compute_dispatch.rs:40-58 (matvec_backend), 90-213 (row-parallel Q4_0 /
 * Q6_K when threads > 1 and out >= QUANT_PARALLEL_ROW_THRESHOLD = 128),
 * 219-254 (single-threaded compact kernels for the other formats). */
int orc_dispatch_matvec(uint32_t t, const void *data, size_t data_len, size_t in_dim, size_t out_dim,
                        const float *x, size_t x_len, float *y, size_t y_len, int threads,
                        int use_simd) {
    if (t == ORC_F32)
        return orc_backend_matvec_f32((const float *)data, data_len / 4, in_dim, out_dim, x, x_len, y,
                                      y_len, threads, use_simd);
    if (!is_quant(t))
        return fail("optimized quantized dispatch received unsupported tensor variant %s", type_name(t));
    const uint8_t *raw = (const uint8_t *)data;
    if ((t == ORC_Q4_0 || t == ORC_Q6_K) && g_parity_threads > 1 && threads < g_parity_threads) threads = g_parity_threads;
    if ((t == ORC_Q4_0 || t == ORC_Q6_K) && threads > 1 && out_dim >= 128) {
        size_t qk = (t == ORC_Q4_0) ? 32 : 256, bs = (t == ORC_Q4_0) ? 18 : 210;
        if (x_len != in_dim)
            return fail("matvec input shape mismatch: W [%zu, %zu], x %zu", out_dim, in_dim, x_len);
        if (y_len != out_dim)
            return fail("%s row range 0..%zu requires local y length %zu, got %zu for out_dim %zu",
                        type_name(t), out_dim, out_dim, y_len, out_dim);
        if (in_dim % qk != 0) return fail("%s in_dim %zu not divisible by %zu", type_name(t), in_dim, qk);
        size_t rb = (in_dim / qk) * bs;
        if (data_len < out_dim * rb)
            return fail("%s weight truncated: expected %zu bytes, got %zu", type_name(t), out_dim * rb, data_len);
        size_t *starts = (size_t *)malloc(sizeof(size_t) * (size_t)threads * 2);
        if (!starts) return fail("failed to allocate row chunks");
        size_t *counts = starts + threads;
        size_t n = make_row_chunks(out_dim, (size_t)threads, starts, counts);
        int err = 0;
#pragma omp parallel for num_threads(threads) schedule(static, 1) reduction(| : err)
        for (size_t c = 0; c < n; c++) {
            const uint8_t *wsub = raw + starts[c] * rb;
            err |= orc_matvec_quant_row_range(t, wsub, counts[c] * rb, counts[c], in_dim, x, x_len,
                                              y + starts[c], counts[c], 0, ORC_ROW_COUNT_ALL);
        }
        free(starts);
        return err;
    }
    return orc_matvec_quant(t, raw, data_len, out_dim, in_dim, x, x_len, y, y_len);
}

/* ------------------------------------------------------------------------ */
/* Elementwise ops (compute.rs:291-384)                                      */
/* ------------------------------------------------------------------------ */

/* compute.rs:291-319 */
int orc_rms_norm(const float *in, const float *w, size_t n, float eps, float *out) {
    if (n == 0) return fail("RMSNorm shape mismatch: input 0, weight 0, output 0");
    if (!isfinite(eps) || eps < 0.0f) return fail("RMSNorm epsilon must be finite and non-negative");
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss += in[i] * in[i];
    float rms = sqrtf(ss / (float)n + eps);
    for (size_t i = 0; i < n; i++) out[i] = in[i] / rms * w[i];
    return 0;
}

int orc_add(const float *a, const float *b, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = a[i] + b[i];
    return 0;
}

int orc_mul(const float *a, const float *b, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = a[i] * b[i];
    return 0;
}

/* compute.rs:337-350 */
int orc_silu(const float *in, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) {
        float v = in[i];
        out[i] = v / (1.0f + expf(-v));
    }
    return 0;
}

/* compute.rs:354-361 */
int orc_swiglu(const float *g, const float *u, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) {
        float v = g[i];
        out[i] = v / (1.0f + expf(-v)) * u[i];
    }
    return 0;
}

/* compute.rs:363-384 */
int orc_softmax(float *v, size_t n) {
    if (n == 0) return fail("softmax requires a non-empty vector");
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++) mx = fmaxf(mx, v[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        v[i] = expf(v[i] - mx);
        sum += v[i];
    }
    if (!isfinite(sum) || sum == 0.0f) return fail("softmax normalization is not finite");
    for (size_t i = 0; i < n; i++) v[i] /= sum;
    return 0;
}

/* compute.rs:446-456 */
static void rope_head(float *v, size_t len, size_t position, float theta) {
    size_t half = len / 2;
    for (size_t i = 0; i < half; i++) {
        float angle = powf(theta, -2.0f * (float)i / (float)len) * (float)position;
        float c = cosf(angle), s = sinf(angle);
        float a = v[i], b = v[i + half];
        v[i] = a * c - b * s;
        v[i + half] = a * s + b * c;
    }
}

/* compute.rs:389-444 */
int orc_rope(float *q, size_t q_len, float *k, size_t k_len, size_t pos, size_t hd, size_t qh,
             size_t kvh, float theta) {
    if (hd == 0 || hd % 2 != 0) return fail("RoPE head dimension must be non-zero and even");
    if (qh == 0 || kvh == 0) return fail("RoPE requires non-zero query and KV head counts");
    if (!isfinite(theta) || theta <= 0.0f) return fail("RoPE frequency base must be finite and positive");
    if (q_len != qh * hd || k_len != kvh * hd)
        return fail("RoPE shape mismatch: q %zu, k %zu, heads %zu:%zu, head_dim %zu", q_len, k_len, qh, kvh, hd);
    for (size_t h = 0; h < qh; h++) rope_head(q + h * hd, hd, pos, theta);
    for (size_t h = 0; h < kvh; h++) rope_head(k + h * hd, hd, pos, theta);
    return 0;
}

/* compute.rs:461-547 */
int orc_attention(const float *q, size_t q_len, const float *kh, const float *vh, size_t hist_elems,
                  const float *kc, const float *vc, size_t cur_len, size_t hist, size_t qhn,
                  size_t kvhn, size_t hd, float *out, size_t out_len) {
    if (qhn == 0 || kvhn == 0 || hd == 0)
        return fail("attention requires non-zero query heads, KV heads, and head dimension");
    if (qhn % kvhn != 0)
        return fail("GQA requires query_heads %zu to be divisible by kv_heads %zu", qhn, kvhn);
    size_t kvw = kvhn * hd, qw = qhn * hd;
    if (q_len != qw || hist_elems != hist * kvw || cur_len != kvw || out_len != qw)
        return fail("attention tensor shape mismatch");
    size_t total = hist + 1;
    /* Heads are independent; with parity threads (never for the timed CPU
     * baseline) they are spread over threads, each head's arithmetic and
     * order unchanged, so the output is bit-identical. */
    int nth = g_parity_threads > 1 ? g_parity_threads : 1;
    float *scores = (float *)malloc((size_t)nth * total * sizeof(float));
    if (!scores) return fail("failed to reserve attention scores");
    float *acc = (float *)calloc(qw, sizeof(float));
    if (!acc) { free(scores); return fail("failed to reserve attention output"); }
    float denom = sqrtf((float)hd);
    int err = 0;
#pragma omp parallel for num_threads(nth) schedule(static) reduction(| : err) if (nth > 1)
    for (size_t h = 0; h < qhn; h++) {
        float *sc = scores + (size_t)omp_get_thread_num() * total;
        size_t g = h * kvhn / qhn;
        const float *qv = q + h * hd;
        for (size_t p = 0; p < total; p++) {
            const float *kall = (p < hist) ? kh + p * kvw : kc;
            const float *kv = kall + g * hd;
            float dot = 0.0f;
            for (size_t i = 0; i < hd; i++) dot += qv[i] * kv[i];
            sc[p] = dot / denom;
        }
        if (orc_softmax(sc, total)) { err |= 1; continue; }
        float *oh = acc + h * hd;
        for (size_t p = 0; p < total; p++) {
            const float *vall = (p < hist) ? vh + p * kvw : vc;
            const float *vv = vall + g * hd;
            for (size_t i = 0; i < hd; i++) oh[i] += sc[p] * vv[i];
        }
    }
    if (err) { free(scores); free(acc); return 1; }
    memcpy(out, acc, qw * sizeof(float));
    free(scores);
    free(acc);
    return 0;
}

/* sampling.rs:45-57 */
uint32_t orc_argmax(const float *l, size_t n) {
    if (n == 0) return 0;
    size_t best = 0;
    float bv = l[0];
    for (size_t i = 1; i < n; i++)
        if (l[i] > bv) { bv = l[i]; best = i; }
    return (uint32_t)best;
}

/* ------------------------------------------------------------------------ */
/* Dense llama model                                                         */
/* ------------------------------------------------------------------------ */

struct orc_model {
    orc_config cfg;
    orc_tensor token_embd, output_norm, output;
    int has_output;
    orc_layer *layers;
    size_t kv_cap, seq_len;
    float *k_cache, *v_cache; /* [layer][cap][kvh][hd] (kv_cache.rs:20-34) */
    int threads, use_simd;
    /* scratch (streaming_model.rs:1006-1017) */
    float *hidden, *tmp, *q, *k, *v, *attn_out, *attn_proj, *gate, *up, *gate_silu, *gate_up, *ffn_out;
    float *staged_k, *staged_v, *norm_w;
};

static const float *f32_data(const orc_tensor *t, float *scratch, size_t n) {
    if (t->type == ORC_F32) return (const float *)t->data;
    if (orc_dequantize_row(t->type, (const uint8_t *)t->data, t->nbytes, n, scratch, n)) return NULL;
    return scratch;
}

int orc_model_create(const orc_config *cfg, const orc_tensor *te, const orc_tensor *on,
                     const orc_tensor *out, const orc_layer *layers, size_t kv_cap, int threads,
                     int use_simd, orc_model **res) {
    orc_model *m = (orc_model *)calloc(1, sizeof *m);
    if (!m) return fail("model allocation failed");
    m->cfg = *cfg;
    m->token_embd = *te;
    m->output_norm = *on;
    m->has_output = out != NULL && out->data != NULL;
    if (m->has_output) m->output = *out;
    m->layers = (orc_layer *)malloc(sizeof(orc_layer) * cfg->block_count);
    memcpy(m->layers, layers, sizeof(orc_layer) * cfg->block_count);
    m->kv_cap = kv_cap;
    m->threads = threads;
    m->use_simd = use_simd;
    size_t kvd = cfg->head_count_kv * cfg->head_dim, qd = cfg->head_count * cfg->head_dim;
    size_t d = cfg->embedding_length, f = cfg->feed_forward_length;
    size_t kv_elems = cfg->block_count * kv_cap * kvd;
    m->k_cache = (float *)calloc(kv_elems ? kv_elems : 1, sizeof(float));
    m->v_cache = (float *)calloc(kv_elems ? kv_elems : 1, sizeof(float));
    m->hidden = calloc(d, 4); m->tmp = calloc(d, 4); m->q = calloc(qd, 4);
    m->k = calloc(kvd, 4); m->v = calloc(kvd, 4); m->attn_out = calloc(qd, 4);
    m->attn_proj = calloc(d, 4); m->gate = calloc(f, 4); m->up = calloc(f, 4);
    m->gate_silu = calloc(f, 4); m->gate_up = calloc(f, 4); m->ffn_out = calloc(d, 4);
    m->staged_k = calloc(cfg->block_count * kvd, 4);
    m->staged_v = calloc(cfg->block_count * kvd, 4);
    m->norm_w = calloc(d > qd ? d : qd, 4);
    if (!m->k_cache || !m->v_cache || !m->staged_k || !m->staged_v || !m->norm_w) {
        orc_model_destroy(m);
        return fail("model scratch allocation failed");
    }
    *res = m;
    return 0;
}

void orc_model_destroy(orc_model *m) {
    if (!m) return;
    free(m->layers); free(m->k_cache); free(m->v_cache);
    free(m->hidden); free(m->tmp); free(m->q); free(m->k); free(m->v); free(m->attn_out);
    free(m->attn_proj); free(m->gate); free(m->up); free(m->gate_silu); free(m->gate_up);
    free(m->ffn_out); free(m->staged_k); free(m->staged_v); free(m->norm_w);
    free(m);
}

int orc_model_reset(orc_model *m) { m->seq_len = 0; return 0; }
size_t orc_model_seq_len(const orc_model *m) { return m->seq_len; }

static int mv(orc_model *m, const orc_tensor *t, const float *x, size_t xl, float *y, size_t yl) {
    return orc_dispatch_matvec(t->type, t->data, t->nbytes, t->ne0, t->ne1, x, xl, y, yl, m->threads, m->use_simd);
}

/* model_executor.rs:102-236 */
static int execute_layer(orc_model *m, size_t li, size_t pos) {
    const orc_config *c = &m->cfg;
    const orc_layer *L = &m->layers[li];
    size_t d = c->embedding_length, hd = c->head_dim, qd = c->head_count * hd, kvd = c->head_count_kv * hd;
    size_t f = c->feed_forward_length;
    const float *nw = f32_data(&L->attn_norm, m->norm_w, d);
    if (!nw) return 1;
    if (orc_rms_norm(m->hidden, nw, d, c->rms_eps, m->tmp)) return 1;
    if (mv(m, &L->attn_q, m->tmp, d, m->q, qd)) return 1;
    if (mv(m, &L->attn_k, m->tmp, d, m->k, kvd)) return 1;
    if (mv(m, &L->attn_v, m->tmp, d, m->v, kvd)) return 1;
    int nb = (L->attn_q_bias.data != NULL) + (L->attn_k_bias.data != NULL) + (L->attn_v_bias.data != NULL);
    if (nb == 3) {
        const float *bq = (const float *)L->attn_q_bias.data, *bk = (const float *)L->attn_k_bias.data,
                    *bv = (const float *)L->attn_v_bias.data;
        for (size_t i = 0; i < qd; i++) m->q[i] += bq[i];
        for (size_t i = 0; i < kvd; i++) m->k[i] += bk[i];
        for (size_t i = 0; i < kvd; i++) m->v[i] += bv[i];
    } else if (nb != 0) {
        return fail("internal error: incomplete Q/K/V bias set survived load of layer %zu", li);
    }
    if (orc_rope(m->q, qd, m->k, kvd, pos, hd, c->head_count, c->head_count_kv, c->rope_freq_base)) return 1;
    size_t hist = m->seq_len;
    const float *kh = m->k_cache + li * m->kv_cap * kvd, *vh = m->v_cache + li * m->kv_cap * kvd;
    if (orc_attention(m->q, qd, kh, vh, hist * kvd, m->k, m->v, kvd, hist, c->head_count,
                      c->head_count_kv, hd, m->attn_out, qd))
        return 1;
    if (mv(m, &L->attn_output, m->attn_out, qd, m->attn_proj, d)) return 1;
    orc_add(m->hidden, m->attn_proj, d, m->tmp);
    memcpy(m->hidden, m->tmp, d * 4);
    nw = f32_data(&L->ffn_norm, m->norm_w, d);
    if (!nw) return 1;
    if (orc_rms_norm(m->hidden, nw, d, c->rms_eps, m->tmp)) return 1;
    if (mv(m, &L->ffn_gate, m->tmp, d, m->gate, f)) return 1;
    if (mv(m, &L->ffn_up, m->tmp, d, m->up, f)) return 1;
    orc_silu(m->gate, f, m->gate_silu);
    orc_mul(m->gate_silu, m->up, f, m->gate_up);
    if (mv(m, &L->ffn_down, m->gate_up, f, m->ffn_out, d)) return 1;
    orc_add(m->hidden, m->ffn_out, d, m->tmp);
    memcpy(m->hidden, m->tmp, d * 4);
    return 0;
}

/* streaming_model.rs:909-1305 */
int orc_model_forward(orc_model *m, uint32_t token, size_t pos, float *final_hidden) {
    const orc_config *c = &m->cfg;
    size_t d = c->embedding_length, kvd = c->head_count_kv * c->head_dim;
    if (pos != m->seq_len)
        return fail("KV position/history mismatch: position %zu requires cache history %zu, got %zu", pos, pos, m->seq_len);
    if (m->seq_len >= m->kv_cap) return fail("KV cache full");
    /* token_embd is [n_embd, vocab]; the row is contiguous (tensor.rs:701-760) */
    if (token >= m->token_embd.ne1)
        return fail("token_id %u out of bounds for embedding with %zu rows", token, m->token_embd.ne1);
    size_t qk = 1, bs = 4;
    orc_block_geometry(m->token_embd.type, &qk, &bs);
    size_t rb = (d / qk) * bs;
    if (orc_dequantize_row(m->token_embd.type, (const uint8_t *)m->token_embd.data + (size_t)token * rb, rb, d,
                           m->hidden, d))
        return 1;
    for (size_t li = 0; li < c->block_count; li++) {
        if (execute_layer(m, li, pos)) return 1;
        memcpy(m->staged_k + li * kvd, m->k, kvd * 4);
        memcpy(m->staged_v + li * kvd, m->v, kvd * 4);
    }
    /* kv_cache.rs:381-421: commit every layer, then advance seq_len. */
    for (size_t li = 0; li < c->block_count; li++) {
        memcpy(m->k_cache + (li * m->kv_cap + m->seq_len) * kvd, m->staged_k + li * kvd, kvd * 4);
        memcpy(m->v_cache + (li * m->kv_cap + m->seq_len) * kvd, m->staged_v + li * kvd, kvd * 4);
    }
    m->seq_len += 1;
    const float *nw = f32_data(&m->output_norm, m->norm_w, d);
    if (!nw) return 1;
    return orc_rms_norm(m->hidden, nw, d, c->rms_eps, final_hidden);
}

/* streaming_model.rs:1334-1370: output.weight, else the tied token_embd. */
int orc_model_logits(orc_model *m, const float *final_hidden, float *logits) {
    const orc_tensor *w = m->has_output ? &m->output : &m->token_embd;
    return mv(m, w, final_hidden, m->cfg.embedding_length, logits, m->cfg.vocab_size);
}

/* inference.rs:580-707 (greedy, no tokenizer). */
int orc_model_generate(orc_model *m, const uint32_t *prompt, size_t plen, size_t max_tokens,
                       int64_t eos, uint32_t *out_tokens, size_t *n_out, float *margin) {
    size_t d = m->cfg.embedding_length, V = m->cfg.vocab_size, ctx = m->cfg.context_length;
    float *hidden = (float *)calloc(d, 4), *logits = (float *)calloc(V, 4);
    if (!hidden || !logits) { free(hidden); free(logits); return fail("generate scratch allocation failed"); }
    int rc = 0;
    size_t n = 0;
    for (size_t p = 0; p < plen && !rc; p++) rc = orc_model_forward(m, prompt[p], p, hidden);
    size_t cur = plen;
    for (size_t gi = 0; gi < max_tokens && !rc; gi++) {
        if ((rc = orc_model_logits(m, hidden, logits))) break;
        uint32_t next = orc_argmax(logits, V);
        if (margin) {
            float best = logits[next], second = -INFINITY;
            for (size_t i = 0; i < V; i++)
                if (i != next && logits[i] > second) second = logits[i];
            margin[gi] = best - second;
        }
        if (eos >= 0 && (int64_t)next == eos) break;
        out_tokens[n++] = next;
        size_t next_pos = cur + 1;
        if (gi + 1 >= max_tokens) break;
        if (next_pos >= ctx) break;
        if ((rc = orc_model_forward(m, next, cur, hidden))) break;
        cur = next_pos;
        if (cur >= ctx) break;
    }
    *n_out = n;
    free(hidden);
    free(logits);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* Seeded synthetic payloads (shared bit-for-bit with the device generator)  */
/* ------------------------------------------------------------------------ */

/* SplitMix64 output number `index` of the stream starting at `seed`. */
uint64_t orc_synth_u64(uint64_t seed, uint64_t index) {
    uint64_t z = seed + (index + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static uint64_t mix_seed(uint64_t seed, uint64_t salt) { return orc_synth_u64(seed ^ salt, 0); }

/* Irwin-Hall(12) approximation of N(0,1): exact in binary64. */
static double synth_normal(uint64_t s, uint64_t j) {
    uint64_t acc = 0;
    for (int k = 0; k < 6; k++) {
        uint64_t r = orc_synth_u64(s, 6 * j + (uint64_t)k);
        acc += (r & 0xFFFFFFFFull) + (r >> 32);
    }
    return (double)acc * (1.0 / 4294967296.0) - 6.0;
}

/* binary32 -> binary16, round to nearest even, integer-only. */
static uint16_t f32_to_f16_rne(float f) {
    uint32_t u = f32_bits(f);
    uint32_t sign = (u >> 16) & 0x8000u, exp = (u >> 23) & 0xFFu, mant = u & 0x7FFFFFu;
    if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0u));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mant |= 0x800000u;
        int shift = 14 - e;
        uint32_t hm = mant >> shift, rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (mant >> 13), rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

static uint16_t synth_scale_f16(uint64_t s, uint64_t j, double mul) {
    return f32_to_f16_rne((float)(fabs(synth_normal(s, j)) * mul));
}

static void put16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* K-quant min scale: the block's d as the reference decodes it
 * (orc_f16_to_f32), times the format's mean code r, encoded so that it
 * decodes to that value again (f16 subnormals decode at half their IEEE
 * value, so they are encoded doubled). */
static uint16_t synth_min_f16(uint16_t dbits, float r) {
    float v = orc_f16_to_f32(dbits) * r;
    uint16_t h = f32_to_f16_rne(v);
    if ((h & 0x7C00u) == 0 && (h & 0x3FFu) != 0) {
        uint16_t h2 = f32_to_f16_rne(2.0f * v);
        if ((h2 & 0x7C00u) == 0) h = h2;
        /* between the largest decoded subnormal (1023 2^-25) and the smallest
         * normal (2^-14) nothing decodes: the nearer of the two */
        else h = (v - 1023.0f * 0x1p-25f < 0x1p-14f - v) ? 0x03FFu : 0x0400u;
    }
    return h;
}

static void synth_bytes(uint64_t s, uint64_t words_per_block, uint64_t block, uint8_t *out, size_t n) {
    for (size_t i = 0; i < n; i++) {
        uint64_t r = orc_synth_u64(s, words_per_block * block + i / 8);
        out[i] = (uint8_t)(r >> (8 * (i % 8)));
    }
}

#define SALT_SCALE 0xA5A5A5A5A5A5A5A5ull
#define SALT_CODE 0x3C3C3C3C3C3C3C3Cull

/* Block layout of the synthetic generator (one block at global index b):
 *   Q8_0: d = f16(|n_b| * mul); q_j = ((16-bit chunk j%4 of word 8b+j/4) * 255 >> 16) - 127
 *   F32:  element b = (float)(n_b * mul)
 *   others: scale fields f16(|n| * mul) from normal 2b (d); the K-quant
 *           min scale dmin = the decoded d times the mean code (Q4_K 7.5,
 *           Q5_K 15.5, Q2_K 1.5; synth_min_f16), so that d*sc*q - dmin*m is
 *           zero-mean over uniform codes and scales;
 *           every other byte of the block from the code stream, words_per_block
 *           = ceil(payload / 8), byte i = byte (i % 8) of word (wpb * b + i / 8).
 *   Q8_K: d = (float)(|n_b| * mul) as f32, bsums = sums of 16-element groups. */
int orc_synth_blocks(uint32_t t, uint64_t seed, uint64_t first, uint64_t nblk, double mul, uint8_t *out) {
    uint64_t ss = mix_seed(seed, SALT_SCALE), sc = mix_seed(seed, SALT_CODE);
    size_t qk, bs;
    if (orc_block_geometry(t, &qk, &bs)) return 1;
    if (t == ORC_F16 || t == ORC_BF16) return fail("synthetic generator does not emit %s", type_name(t));
#pragma omp parallel for schedule(static)
    for (uint64_t k = 0; k < nblk; k++) {
        uint64_t b = first + k;
        uint8_t *p = out + k * bs;
        switch (t) {
        case ORC_F32: {
            float v = (float)(synth_normal(ss, b) * mul);
            memcpy(p, &v, 4);
            break;
        }
        case ORC_Q8_0:
            put16(p, synth_scale_f16(ss, b, mul));
            for (int j = 0; j < 32; j++) {
                uint64_t r = orc_synth_u64(sc, 8 * b + (uint64_t)(j / 4));
                uint32_t c16 = (uint32_t)((r >> (16 * (j % 4))) & 0xFFFFu);
                p[2 + j] = (uint8_t)(int8_t)((int)((c16 * 255u) >> 16) - 127);
            }
            break;
        case ORC_Q4_0: put16(p, synth_scale_f16(ss, b, mul)); synth_bytes(sc, 2, b, p + 2, 16); break;
        case ORC_Q5_0: put16(p, synth_scale_f16(ss, b, mul)); synth_bytes(sc, 3, b, p + 2, 20); break;
        case ORC_Q4_K: {
            uint16_t d = synth_scale_f16(ss, 2 * b, mul);
            put16(p, d);
            put16(p + 2, synth_min_f16(d, 7.5f));
            synth_bytes(sc, 18, b, p + 4, 140);
            break;
        }
        case ORC_Q5_K: {
            uint16_t d = synth_scale_f16(ss, 2 * b, mul);
            put16(p, d);
            put16(p + 2, synth_min_f16(d, 15.5f));
            synth_bytes(sc, 22, b, p + 4, 172);
            break;
        }
        case ORC_Q6_K:
            synth_bytes(sc, 26, b, p, 208);
            put16(p + 208, synth_scale_f16(ss, 2 * b, mul));
            break;
        case ORC_Q2_K:
            synth_bytes(sc, 10, b, p, 80);
            {
                uint16_t d = synth_scale_f16(ss, 2 * b, mul);
                put16(p + 80, d);
                put16(p + 82, synth_min_f16(d, 1.5f));
            }
            break;
        case ORC_Q3_K:
            synth_bytes(sc, 14, b, p, 108);
            put16(p + 108, synth_scale_f16(ss, 2 * b, mul));
            break;
        case ORC_Q8_K: {
            float d = (float)(fabs(synth_normal(ss, 2 * b)) * mul);
            memcpy(p, &d, 4);
            synth_bytes(sc, 32, b, p + 4, 256);
            for (int g = 0; g < 16; g++) {
                int s = 0;
                for (int i = 0; i < 16; i++) s += (int8_t)p[4 + 16 * g + i];
                put16(p + 260 + 2 * g, (uint16_t)(int16_t)s);
            }
            break;
        }
        default: break;
        }
    }
    return 0;
}
