/*
 * g4_oracle_matvec.c -- CPU restatement of gemma4-rs's mat-vec kernels over
 * GGUF weight formats (crates/llm-backend-cpu/src/matvec.rs, dequant.rs) and
 * the activations applied to their results (crates/llm-backend-cpu/src/ops.rs).
 *
 * TEST INFRASTRUCTURE ONLY: the oracle for the HIP backend, never part of it.
 * Built with -ffp-contract=off like the rest of the oracle: every product
 * and sum is its own rounded f32 operation, in the reference's order.
 */
#include "g4_oracle.h"

#include <math.h>
#include <stdio.h>
#include <string.h>

/* Rust's `Iterator::sum` for floats folds from -0.0. */
#define SUM_START_F (-0.0f)
#define SUM_START_D (-0.0)

/* half::f16 -> f32 (exact). */
float or_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {  /* subnormal: normalise */
            int e = -1;
            uint32_t m = man;
            do {
                ++e;
                m <<= 1;
            } while (!(m & 0x400u));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((m & 0x3ffu) << 13);
        }
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* half::f16::from_f32: round to nearest, ties to even; overflow to inf;
 * NaN stays NaN (quiet). */
uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t exp = (x >> 23) & 0xffu, man = x & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0));
    const int e = (int)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return sign;  /* below half the smallest subnormal */
        const uint32_t m = man | 0x800000u;
        const int shift = 14 - e;  /* to a 10-bit subnormal mantissa */
        uint32_t h = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u))) ++h;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  /* may carry into the exponent (to inf) */
    return (uint16_t)(sign | h);
}

/* matvec.rs:192-204 */
float or_bf16_to_f32(uint16_t b) {
    const uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t or_f32_to_bf16(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    if (isnan(value)) return (uint16_t)((bits >> 16) | 64u);
#ifdef G4_PLANT_BF16_TRUNC /* planted mistake: truncation */
    return (uint16_t)(bits >> 16);
#else
    return (uint16_t)((bits + (0x7fffu + ((bits >> 16) & 1u))) >> 16);
#endif
}

/* Rust's `f32 as i8`: saturating, NaN -> 0. */
static int8_t sat_i8(float v) {
    if (isnan(v)) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}

/* matvec.rs:35-53 (quantize_q8_0): per 32-value block, max|x| (NaN ignored,
 * as f32::max does), scale = max/127, stored as its f16 rounding; values
 * x * (1/scale) rounded half to even, saturated to i8. */
int or_quantize_q8_0(const float *x, size_t n, float *scales, int8_t *quants) {
    if (n % OR_Q8_BLOCK != 0) {
        char msg[96];
        snprintf(msg, sizeof msg, "Q8_0 activation length %zu is not a multiple of %d", n, OR_Q8_BLOCK);
        return or_fail(OR_ERR_COMPUTE, msg);
    }
    for (size_t b = 0; b < n / OR_Q8_BLOCK; ++b) {
        const float *blk = x + b * OR_Q8_BLOCK;
        float max = 0.0f;
        for (size_t i = 0; i < OR_Q8_BLOCK; ++i) max = fmaxf(max, fabsf(blk[i]));
        const float scale = max / 127.0f;
        const float inverse = scale == 0.0f ? 0.0f : 1.0f / scale;
#ifdef G4_PLANT_Q8_SCALE_F32 /* planted mistake: scale kept in f32 */
        scales[b] = scale;
#else
        scales[b] = or_f16_to_f32(or_f32_to_f16(scale));
#endif
#ifdef G4_PLANT_Q8_ROUND_AWAY /* planted mistake: half away from zero */
        for (size_t i = 0; i < OR_Q8_BLOCK; ++i) quants[b * OR_Q8_BLOCK + i] = sat_i8(roundf(blk[i] * inverse));
#else
        for (size_t i = 0; i < OR_Q8_BLOCK; ++i) quants[b * OR_Q8_BLOCK + i] = sat_i8(rintf(blk[i] * inverse));
#endif
    }
    return OR_OK;
}

/* dequant.rs:13-24 */
int or_dequant_q8_0(const uint8_t *bytes, size_t len, float *out) {
    if (len % OR_Q8_BYTES != 0) {
        char msg[96];
        snprintf(msg, sizeof msg, "Q8_0 data length %zu is not a multiple of %d", len, OR_Q8_BYTES);
        return or_fail(OR_ERR_COMPUTE, msg);
    }
    for (size_t b = 0; b < len / OR_Q8_BYTES; ++b) {
        const uint8_t *blk = bytes + b * OR_Q8_BYTES;
        const float scale = or_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (size_t i = 0; i < OR_Q8_BLOCK; ++i) out[b * OR_Q8_BLOCK + i] = (float)(int8_t)blk[2 + i] * scale;
    }
    return OR_OK;
}

/* matvec.rs:206-214 (check_shape): rows * row_len == len without overflow,
 * else the reference's message. */
static int shape_ok(size_t len, size_t rows, size_t row_len, const char *kind) {
    if ((row_len == 0 || rows <= SIZE_MAX / row_len) && rows * row_len == len) return 1;
    char msg[160];
    snprintf(msg, sizeof msg, "%s weight has %zu elements, expected %zu rows of %zu", kind, len, rows, row_len);
    or_fail(OR_ERR_COMPUTE, msg);
    return 0;
}

/* matvec.rs:186-190 (q8_0_row_len) */
static int q8_cols_ok(size_t cols) {
    if (cols % OR_Q8_BLOCK == 0) return 1;
    char msg[96];
    snprintf(msg, sizeof msg, "Q8_0 row length %zu is not a multiple of %d", cols, OR_Q8_BLOCK);
    or_fail(OR_ERR_COMPUTE, msg);
    return 0;
}

/* matvec.rs:138-151 (dot_q8_0): per block the exact integer dot, then
 * `dot as f32 * (w_scale * x_scale)`, the blocks summed in order. */
static float dot_q8_0(const uint8_t *row, size_t nb, const float *xs, const int8_t *xq) {
    float sum = SUM_START_F;
    for (size_t b = 0; b < nb; ++b) {
        const uint8_t *blk = row + b * OR_Q8_BYTES;
        const float ws = or_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        int32_t dot = 0;
        for (size_t i = 0; i < OR_Q8_BLOCK; ++i) dot += (int32_t)(int8_t)blk[2 + i] * (int32_t)xq[b * OR_Q8_BLOCK + i];
        sum += (float)dot * (ws * xs[b]);
    }
    return sum;
}

/* matvec.rs:55-62 */
int or_matvec_q8_0(const uint8_t *w, size_t w_len, size_t rows, size_t cols, const float *xs,
                   const int8_t *xq, float *out) {
    if (!q8_cols_ok(cols)) return OR_ERR_COMPUTE;
    const size_t nb = cols / OR_Q8_BLOCK, row_len = nb * OR_Q8_BYTES;
    if (!shape_ok(w_len, rows, row_len, "Q8_0")) return OR_ERR_COMPUTE;
    for (size_t r = 0; r < rows; ++r) out[r] = dot_q8_0(w + r * row_len, nb, xs, xq);
    return OR_OK;
}

/* ops.rs:79-81 */
float or_softcap(float value, float cap) {
#ifdef G4_PLANT_SOFTCAP /* planted mistake: cap applied outside only */
    return tanhf(value) * cap;
#else
    return tanhf(value * (1.0f / cap)) * cap;
#endif
}

/* ops.rs:85-89: 0.5 * x * (1 + tanh(sqrt(2/pi) * x * (1 + a * x * x))), left to right. */
float or_gelu_tanh(float x) {
#ifdef G4_PLANT_GELU_COEF /* planted mistake: cubic coefficient */
    const float sqrt_2_over_pi = 0.7978846f, coef_a = 0.0447f;
#else
    const float sqrt_2_over_pi = 0.7978846f, coef_a = 0.044715f;
#endif
    return 0.5f * x * (1.0f + tanhf(sqrt_2_over_pi * x * (1.0f + coef_a * x * x)));
}

/* ops.rs:95-103 */
float or_gelu_tanh_fp16_table(float x) {
    if (x <= -10.0f) return 0.0f;
    if (x >= 10.0f) return x;
    return or_f16_to_f32(or_f32_to_f16(or_gelu_tanh(or_f16_to_f32(or_f32_to_f16(x)))));
}

/* matvec.rs:64-81 with post = softcap (model.rs:447) */
int or_matvec_q8_0_softcap(const uint8_t *w, size_t w_len, size_t rows, size_t cols, const float *xs,
                           const int8_t *xq, float cap, float *out) {
    const int rc = or_matvec_q8_0(w, w_len, rows, cols, xs, xq, out);
    if (rc != OR_OK) return rc;
    for (size_t r = 0; r < rows; ++r) out[r] = or_softcap(out[r], cap);
    return OR_OK;
}

/* matvec.rs:83-102: gelu(gate_row . x) * (up_row . x) per row. */
int or_geglu_q8_0(const uint8_t *gate, const uint8_t *up, size_t w_len, size_t rows, size_t cols,
                  const float *xs, const int8_t *xq, int fp16_gelu, float *out) {
    if (!q8_cols_ok(cols)) return OR_ERR_COMPUTE;
    const size_t nb = cols / OR_Q8_BLOCK, row_len = nb * OR_Q8_BYTES;
    if (!shape_ok(w_len, rows, row_len, "Q8_0")) return OR_ERR_COMPUTE;
    for (size_t r = 0; r < rows; ++r) {
        const float g = dot_q8_0(gate + r * row_len, nb, xs, xq);
        const float u = dot_q8_0(up + r * row_len, nb, xs, xq);
        out[r] = (fp16_gelu ? or_gelu_tanh_fp16_table(g) : or_gelu_tanh(g)) * u;
    }
    return OR_OK;
}

/* matvec.rs:104-122, 153-176: f32 activations against dequantized blocks,
 * either in f32 (block dot summed in order, times the scale, blocks summed
 * in order) or with every sum in f64 and one final rounding. */
int or_matvec_q8_0_f32(const uint8_t *w, size_t w_len, size_t rows, size_t cols, const float *x,
                       int f64_sums, float *out) {
    if (!q8_cols_ok(cols)) return OR_ERR_COMPUTE;
    const size_t nb = cols / OR_Q8_BLOCK, row_len = nb * OR_Q8_BYTES;
    if (!shape_ok(w_len, rows, row_len, "Q8_0")) return OR_ERR_COMPUTE;
    for (size_t r = 0; r < rows; ++r) {
        const uint8_t *row = w + r * row_len;
        if (f64_sums) {
            double sum = SUM_START_D;
            for (size_t b = 0; b < nb; ++b) {
                const uint8_t *blk = row + b * OR_Q8_BYTES;
                const double scale = (double)or_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
                double dot = SUM_START_D;
                for (size_t i = 0; i < OR_Q8_BLOCK; ++i)
                    dot += (double)(int8_t)blk[2 + i] * (double)x[b * OR_Q8_BLOCK + i];
                sum += dot * scale;
            }
            out[r] = (float)sum;
        } else {
            float sum = SUM_START_F;
            for (size_t b = 0; b < nb; ++b) {
                const uint8_t *blk = row + b * OR_Q8_BYTES;
                const float scale = or_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
                float dot = SUM_START_F;
                for (size_t i = 0; i < OR_Q8_BLOCK; ++i) dot += (float)(int8_t)blk[2 + i] * x[b * OR_Q8_BLOCK + i];
                sum += dot * scale;
            }
            out[r] = sum;
        }
    }
    return OR_OK;
}

/* matvec.rs:124-130, 178-180: x rounded to bf16 first, then one sequential
 * f32 sum over the row. */
int or_matvec_bf16(const uint16_t *w, size_t w_len, size_t rows, size_t cols, const float *x, float *out) {
    if (!shape_ok(w_len, rows, cols, "BF16")) return OR_ERR_COMPUTE;
    for (size_t r = 0; r < rows; ++r) {
        float sum = SUM_START_F;
        for (size_t i = 0; i < cols; ++i) sum += or_bf16_to_f32(w[r * cols + i]) * or_bf16_to_f32(or_f32_to_bf16(x[i]));
        out[r] = sum;
    }
    return OR_OK;
}

/* matvec.rs:182-184: a sequential f32 sum per row (not ops.rs's 16-lane dot). */
int or_matvec_f32(const float *w, size_t w_len, size_t rows, size_t cols, const float *x, float *out) {
    if (!shape_ok(w_len, rows, cols, "f32")) return OR_ERR_COMPUTE;
    for (size_t r = 0; r < rows; ++r) {
        float sum = SUM_START_F;
        for (size_t i = 0; i < cols; ++i) sum += w[r * cols + i] * x[i];
        out[r] = sum;
    }
    return OR_OK;
}
