/*
 * g4_oracle.h -- CPU restatement of gemma4-rs's attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle that the HIP
 * attention backend is compared against.  Only the test suite, the smoke
 * check and the CPU-baseline leg of the benchmark may load it; the product
 * library never links, loads or calls it.
 *
 * Every function restates one reference function (file:line given beside
 * it, paths relative to the gemma4-rs repository root) with the same
 * floating-point operation order, so that it reproduces the reference's f32
 * arithmetic: 16-lane dot products, sequential softmax sum, sequential P.V,
 * f64-accumulated RMS norm, and RoPE angles built by repeated f32
 * multiplication.  Compiled with -ffp-contract=off (Rust never fuses a*b+c).
 *
 * Status codes mirror EngError (crates/llm-eng/src/error.rs:3-15).
 */
#ifndef G4_ORACLE_H
#define G4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    OR_OK = 0,
    OR_ERR_COMPUTE = 1,          /* EngError::Compute */
    OR_ERR_CONTEXT_TOO_LONG = 2, /* EngError::ContextTooLong{got,max} */
    OR_ERR_MISSING_LAYER = 3,    /* EngError::MissingLayer(layer) */
    OR_ERR_KV_LAYER_OUT_OF_RANGE = 10, /* KvShareError::LayerOutOfRange */
    OR_ERR_KV_TOO_MANY_SHARED = 11,    /* KvShareError::TooManySharedLayers */
    OR_ERR_KV_NO_EARLIER_SAME_KIND = 12 /* KvShareError::NoEarlierLayerOfSameKind */
};

/* Message of the last error raised on this thread (reference wording). */
const char *or_last_error(void);

/* ---- backend primitives: crates/llm-backend-cpu/src/ops.rs ---- */
float or_dot_f32(const float *a, const float *b, size_t n);                 /* ops.rs:65-76   */
int or_softmax_f32(const float *x, size_t n, float *out);                   /* ops.rs:105-127 */
int or_rms_norm(const float *x, size_t n, const float *weight, size_t weight_len,
                float eps, float *out);                                      /* ops.rs:45-56   */
int or_rope_neox(float *x, size_t len, size_t position, float base, size_t n_rot,
                 const float *freq_factors, size_t n_factors);               /* ops.rs:134-162 */

/* ---- model-level attention: crates/llm-gemma4/src/impl_/model.rs ---- */
/* attend_head (model.rs:326-343) over a contiguous [T][kv_width] image. Returns
 * OR_OK, or OR_ERR_COMPUTE when the softmax fails (the Rust returns an empty Vec). */
int or_attend_head(const float *q, const float *keys, const float *values, size_t T,
                   size_t kv_width, size_t head_dim, size_t n_heads, size_t n_kv_heads,
                   float scale, size_t head, float *out);
/* attend (model.rs:348-366) over a contiguous K/V image (the `concat` result). */
int or_attend(const float *q, size_t q_len, const float *keys, const float *values, size_t T,
              size_t n_heads, size_t n_kv_heads, float scale, float *out);
/* attend (model.rs:348-366) over per-position rows, including the `concat`
 * copy the reference makes.  threads == 1 runs the heads in order on the
 * caller; any other value hands them to the process-wide persistent pool as
 * map_items does (crates/llm-backend-cpu/src/pool.rs:145-197), whose size is
 * LLM_THREADS if set, else the online CPU count (pool.rs:86-110). */
int or_attend_rows(const float *q, size_t q_len, const float *const *key_rows,
                   const float *const *value_rows, size_t T, size_t n_heads, size_t n_kv_heads,
                   float scale, size_t threads, float *out);
/* A prompt chunk as the reference's token-at-a-time loop runs it
 * (crates/llm-gemma4/src/impl_/generate.rs:37-41, model.rs:407-410): query i
 * (q + i*q_len, at position pos0 + i) attends rows [b, pos0 + i + 1) of the
 * contiguous image keys/values (row t = position t), b = 0 when window == 0
 * else windowed_len's start (eng/mod.rs:10-12); out + i*q_len receives it.
 * Each query is or_attend; `threads` (>= 1) OS threads take queries in turn
 * (a checker's parallelism, not the reference's).  status[i] (may be NULL)
 * gets each query's result code; the call returns OR_ERR_COMPUTE if any
 * query failed. */
int or_attend_prefill(const float *q, size_t q_len, size_t N, const float *keys, const float *values,
                      size_t pos0, size_t window, size_t n_heads, size_t n_kv_heads, float scale,
                      size_t threads, int *status, float *out);
/* The same results as or_attend_prefill, bit for bit, from a cache-friendly
 * loop nest (a checker speed-up for long contexts): groups of consecutive
 * queries walk their keys together.  positions (NULL: pos0 + i) gives query
 * i's position, for checking a sample of a chunk's rows.  At most 64 heads. */
int or_attend_prefill_blocked(const float *q, size_t q_len, size_t N, const size_t *positions,
                              const float *keys, const float *values, size_t pos0, size_t window,
                              size_t n_heads, size_t n_kv_heads, float scale, size_t threads, int *status,
                              float *out);
/* f64 twin of attend: every product and sum in double, for the noise floor
 * |attend_f32 - attend_f64| that the tolerance policy falls back on. */
int or_attend_f64(const float *q, size_t q_len, const float *keys, const float *values, size_t T,
                  size_t n_heads, size_t n_kv_heads, double scale, double *out);

/* norm_heads (model.rs:283-290) and rope_heads (model.rs:295-304), in place. */
int or_norm_heads(float *x, size_t len, size_t head_dim, const float *weight, float eps);
int or_rope_heads(float *x, size_t len, size_t head_dim, size_t position, float base,
                  const float *freq_factors, size_t n_factors);

/* ---- policies: crates/llm-gemma4/src/idea/mod.rs, src/eng/mod.rs ---- */
int or_layer_attention_kind(size_t n_layers, size_t layer);    /* idea/mod.rs:148-156: 0 local, 1 global */
size_t or_head_dim(size_t n_layers, size_t layer, size_t head_dim_local,
                   size_t head_dim_global);                     /* idea/mod.rs:140-145 */
void or_proportional_rope_freq_factors(size_t head_dim, float p, float *out); /* idea/mod.rs:162-165 */
void or_windowed_len(size_t seq_len, size_t window, size_t *begin, size_t *end); /* eng/mod.rs:10-12 */
int or_kv_source_layer(size_t n_layers, size_t shared_kv_layers, size_t layer,
                       size_t *source);                         /* eng/mod.rs:71-90 */

/* ---- KvCache: crates/llm-eng/src/context_memory.rs:21-86 ---- */
/* Rows are `width` floats (n_kv_heads * head_dim of the owning layer). */
typedef struct or_kv_cache or_kv_cache;
or_kv_cache *or_kv_new(void);
void or_kv_free(or_kv_cache *c);
int or_kv_append(or_kv_cache *c, size_t layer, const float *k, const float *v,
                 size_t width);                                                  /* :44-51 */
/* keys/values point at `len` contiguous rows (the prefix of the layer's cache). */
int or_kv_view(const or_kv_cache *c, size_t layer, size_t len, const float **keys,
               const float **values, size_t *width);                             /* :53-69 */
void or_kv_clear(or_kv_cache *c);                                                /* :82-84 */

/* Gemma4HyperParams fields the attention segment reads (idea/mod.rs:15-34). */
typedef struct {
    size_t n_layers, n_heads, n_kv_heads, head_dim_local, head_dim_global;
    size_t sliding_window, shared_kv_layers;
    float local_rope_base, global_rope_base, rms_norm_eps;
} or_hparams;

/* Layer-attention segment of Gemma4CpuModel::layer (model.rs:386-411), from
 * the projected q/k/v onwards: q-norm, RoPE(q); for owner layers k-norm,
 * v-norm (no weight), RoPE(k), append; view(source, pos+1); window;
 * attend(scale 1.0).  q is [n_heads*head_dim], k and v [n_kv_heads*head_dim]
 * (ignored on shared layers); all three are modified in place.  Reports the
 * attended set as (source layer, [kv_begin, kv_end)). */
int or_layer_attention(or_kv_cache *c, const or_hparams *hp, size_t layer, size_t position,
                       float *q, float *k, float *v, const float *q_norm_w,
                       const float *k_norm_w, const float *rope_freqs, size_t n_freqs,
                       float *out, size_t *source_layer, size_t *kv_begin, size_t *kv_end);

/* Records `msg` as the last error and returns `code`. */
int or_fail(int code, const char *msg);

/* ---- mat-vecs over GGUF weight formats (crates/llm-backend-cpu/src/matvec.rs) ---- */
#define OR_Q8_BLOCK 32 /* values per Q8_0 block */
#define OR_Q8_BYTES 34 /* f16 scale + 32 int8 */
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);                                                 /* half::f16::from_f32 */
float or_bf16_to_f32(uint16_t b);                                                /* matvec.rs:192-194 */
uint16_t or_f32_to_bf16(float f);                                                /* matvec.rs:196-204 */
int or_quantize_q8_0(const float *x, size_t n, float *scales, int8_t *quants);  /* matvec.rs:35-53 */
int or_dequant_q8_0(const uint8_t *bytes, size_t len, float *out);              /* dequant.rs:13-24 */
int or_matvec_q8_0(const uint8_t *w, size_t w_len, size_t rows, size_t cols, const float *xs,
                   const int8_t *xq, float *out);                                /* matvec.rs:55-62 */
int or_matvec_q8_0_softcap(const uint8_t *w, size_t w_len, size_t rows, size_t cols,
                           const float *xs, const int8_t *xq, float cap, float *out); /* :64-81 */
int or_geglu_q8_0(const uint8_t *gate, const uint8_t *up, size_t w_len, size_t rows, size_t cols,
                  const float *xs, const int8_t *xq, int fp16_gelu, float *out); /* :83-102 */
int or_matvec_q8_0_f32(const uint8_t *w, size_t w_len, size_t rows, size_t cols, const float *x,
                       int f64_sums, float *out);                                /* :104-122 */
int or_matvec_bf16(const uint16_t *w, size_t w_len, size_t rows, size_t cols, const float *x,
                   float *out);                                                  /* :124-130 */
int or_matvec_f32(const float *w, size_t w_len, size_t rows, size_t cols, const float *x,
                  float *out);                                                   /* :132-136 */
float or_softcap(float value, float cap);                                        /* ops.rs:79-81 */
float or_gelu_tanh(float x);                                                     /* ops.rs:85-89 */
float or_gelu_tanh_fp16_table(float x);                                          /* ops.rs:95-103 */

/* ---- test and CPU-baseline helpers (not part of the reference) ---- */
size_t or_pool_threads(void);
/* Test inputs: for each of n_rows rows of row_width floats, norm_heads with
 * `weight` (NULL: none) and then, when base > 0, rope_heads at position
 * pos0 + row -- the preparation model.rs:395-404 applies to q and k rows. */
int or_prepare_rows(float *x, size_t n_rows, size_t row_width, size_t head_dim,
                    const float *weight, float eps, size_t pos0, float base,
                    const float *freq_factors, size_t n_factors);

#ifdef __cplusplus
}
#endif
#endif
