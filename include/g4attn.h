/*
 * g4attn.h -- C ABI of the MI355X (gfx950) attention backend for gemma4-rs.
 *
 * The backend replaces the engine's CPU attention seam: the private
 * `attend(q, keys, values, n_heads, n_kv_heads, scale)` that
 * Gemma4CpuModel::layer calls once per layer
 * (crates/llm-gemma4/src/impl_/model.rs:348-366, call site model.rs:410),
 * together with the primitives it is assembled from and the engine ports it
 * reads (ComputePort, ContextMemory, EngError).  Citations are file:line in
 * the gemma4-rs repository.
 *
 * Conventions
 *  - Every function returns a g4_status; 0 is success.  On failure
 *    g4_last_error() holds the message with the reference's wording and
 *    g4_last_error_fields() the numbers of ContextTooLong / MissingLayer.
 *    Nothing panics or aborts across the ABI.
 *  - "_dev" pointers are device (HBM) pointers owned by the caller; host
 *    pointers are marked "host".  No function keeps a pointer after it
 *    returns, except the KV-cache object, which owns its device rows.
 *  - stream is a hipStream_t (NULL = the null stream).  Device-pointer entry
 *    points are asynchronous and stream-ordered; their softmax failures are
 *    recorded on the device and reported by g4_check_status().  Host-pointer
 *    entry points synchronise and report failures directly.
 *  - A K/V cache is rows of n_kv_heads*head_dim f32, row t = position t,
 *    oldest first, as the reference's KvCache keeps them
 *    (crates/llm-eng/src/context_memory.rs:44-51, model.rs:312-321);
 *    `row_stride` is the distance between rows in floats.
 */
#ifndef G4ATTN_H
#define G4ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* EngError variants (crates/llm-eng/src/error.rs:3-15). */
typedef enum {
    G4_OK = 0,
    G4_ERR_CONTEXT_TOO_LONG = 1, /* EngError::ContextTooLong { got, max } */
    G4_ERR_MISSING_LAYER = 2,    /* EngError::MissingLayer(layer) */
    G4_ERR_MISSING_WEIGHT = 3,   /* EngError::MissingWeight(name) */
    G4_ERR_COMPUTE = 4,          /* EngError::Compute(message) */
    G4_ERR_MSG = 5               /* EngError::Msg(message) */
} g4_status;

typedef struct g4_ctx g4_ctx;           /* one per device */
typedef struct g4_kv_cache g4_kv_cache; /* device-resident ContextMemory */
typedef void *g4_stream;                /* hipStream_t */

/* Message of the last failure on the calling thread ("" if none). */
const char *g4_last_error(void);
/* ContextTooLong: *a = got, *b = max.  MissingLayer: *a = layer. */
void g4_last_error_fields(uint64_t *a, uint64_t *b);

/* ---------------------------------------------------------------- context */
int g4_init(int device, g4_ctx **ctx);
int g4_release(g4_ctx *ctx);
/* Waits for `stream`, then reports (and clears) any softmax failure the
 * device-pointer attention calls recorded since the last check, as
 * G4_ERR_COMPUTE "softmax input is not finite" (model.rs:362-364). */
int g4_check_status(g4_ctx *ctx, g4_stream stream);
/* Tuning: keys per split-K work item of the decode kernels, rounded up to a
 * multiple of 16 (0 = automatic). */
int g4_set_decode_chunk(g4_ctx *ctx, int64_t keys);
/* Tuning: 1 = prefill computes every product with f32 MFMAs; 0 (default) =
 * split-f16 MFMA products (each f32 operand as an f16 hi + lo pair, three
 * f16 products per f32 product, f32 accumulation) for every work unit whose
 * q rows and K/V rows are finite and below 2^15 in magnitude, f32 MFMAs for
 * the others.  Both match the f32 reference within its tolerance; the
 * engine has no counterpart (a backend precision knob). */
int g4_set_prefill_exact(g4_ctx *ctx, int exact);

/* ---------------------------------------------------------- device memory */
/* Caller-owned device buffers on the context's device, so that a binding
 * needs no other runtime: the device image of F32Buf
 * (crates/llm-backend-cpu/src/buffer.rs:1-26) and of the GGUF weight blobs
 * the mat-vecs read (crates/llm-eng/src/weight_store.rs:5-22).  The library
 * keeps no hidden copy of them.  0 bytes gives NULL. */
int g4_alloc(g4_ctx *ctx, size_t bytes, void **ptr_dev);
/* Frees a g4_alloc buffer after the device's queued work (NULL: no-op). */
int g4_free(g4_ctx *ctx, void *ptr_dev);
/* Synchronous copies of `bytes`, after all work queued on the device: host
 * to device, device to host, device to device. */
int g4_copy_to_device(g4_ctx *ctx, void *dst_dev, const void *src_host, size_t bytes);
int g4_copy_to_host(g4_ctx *ctx, void *dst_host, const void *src_dev, size_t bytes);
int g4_copy_on_device(g4_ctx *ctx, void *dst_dev, const void *src_dev, size_t bytes);
/* Waits for `stream` (NULL: the null stream).  g4_check_status waits too,
 * and also reports softmax failures. */
int g4_sync(g4_ctx *ctx, g4_stream stream);
/* Makes the context's device the calling thread's current HIP device.  The
 * device-pointer calls below run on the current device, as HIP calls do;
 * g4_init, g4_alloc, g4_copy_* and g4_sync make it current themselves. */
int g4_activate(g4_ctx *ctx);

/* ------------------------------------------------------ attention (hot path) */
/* attend (model.rs:348-366), host buffers: q[n_heads*head_dim] with
 * head_dim = q_len / n_heads, keys/values [T][n_kv_heads*head_dim] (the
 * `concat` image of model.rs:352-353), out[q_len].  Query head h reads KV head
 * h*n_kv_heads/n_heads (model.rs:329).  Synchronous. */
int g4_attend(g4_ctx *ctx, const float *q_host, size_t q_len, const float *keys_host,
              const float *values_host, size_t T, size_t n_heads, size_t n_kv_heads, float scale,
              float *out_host);

/* One decode step over cache rows [kv_begin, kv_end) of k_cache/v_cache:
 * the device form of `attend(q, &keys[range], &values[range], ...)` after
 * `context.view(source, pos+1)` and the window range (model.rs:407-410). */
int g4_attend_decode(g4_ctx *ctx, const float *q_dev, const float *k_cache_dev,
                     const float *v_cache_dev, int64_t row_stride, int64_t kv_begin,
                     int64_t kv_end, int n_heads, int n_kv_heads, int head_dim, float scale,
                     float *out_dev, g4_stream stream);

/* g4_attend_decode that allocates nothing.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The split
 * partials go to a static device array of 8 MiB + 64 KiB, one per GPU, whose
 * address g4_init resolves; a decode whose split plan needs more is refused
 * with G4_ERR_COMPUTE (any range with one KV head and 8 query heads fits).
 * Same arguments, results and stream semantics as g4_attend_decode.  Every
 * call on a GPU shares that GPU's array: calls that overlap in time on one
 * GPU (other streams, other contexts) race and must be serialised by the
 * caller. */
int g4_attend_decode_noalloc(g4_ctx *ctx, const float *q_dev, const float *k_cache_dev,
                             const float *v_cache_dev, int64_t row_stride, int64_t kv_begin,
                             int64_t kv_end, int n_heads, int n_kv_heads, int head_dim, float scale,
                             float *out_dev, g4_stream stream);

/* B independent decode steps in one launch (ragged lengths).  Sequence s
 * reads rows [kv_begin[s], kv_end[s]) of its cache, whose row 0 is row
 * seq_row0[s] of k_base/v_base (seq_row0 may be NULL: all zero).  The three
 * arrays are device arrays of B int64; max_kv_len (host) must bound every
 * kv_end[s]-kv_begin[s] (a longer range is reported as ContextTooLong by
 * g4_check_status).  q and out are [B][n_heads*head_dim].  No reference
 * counterpart: the engine is single-sequence (crates/llm-eng/src/schedule.rs:6-9);
 * each sequence's result equals attend over its own rows. */
int g4_attend_decode_batch(g4_ctx *ctx, int B, const float *q_dev, const float *k_base_dev,
                           const float *v_base_dev, int64_t row_stride,
                           const int64_t *seq_row0_dev, const int64_t *kv_begin_dev,
                           const int64_t *kv_end_dev, int64_t max_kv_len, int n_heads,
                           int n_kv_heads, int head_dim, float scale, float *out_dev,
                           g4_stream stream);

/* Chunked prefill: N queries at positions pos0..pos0+N-1, q and out
 * [N][n_heads*head_dim].  Query i sees exactly the rows a decode at position
 * p = pos0+i would: [0, p+1) when window == 0 (GlobalPolicy), else
 * [(p+1-window)+, p+1) (LocalWindowPolicy, crates/llm-gemma4/src/eng/mod.rs:10-36),
 * which is what the reference's token-at-a-time prompt loop computes
 * (crates/llm-gemma4/src/impl_/generate.rs:37-41, model.rs:250).  The cache
 * must hold rows up to pos0+N-1. */
int g4_attend_prefill(g4_ctx *ctx, const float *q_dev, const float *k_cache_dev,
                      const float *v_cache_dev, int64_t row_stride, int64_t pos0, int64_t N,
                      int64_t window, int n_heads, int n_kv_heads, int head_dim, float scale,
                      float *out_dev, g4_stream stream);

/* Work schedule of g4_attend_prefill's MFMA path (head_dim 256 or 512,
 * 8 query heads per KV head) on a GPU with num_cus compute units: position
 * blocks of 8 queries are cut into units of 16-key tiles, and workgroup w
 * (of n_bins per KV head) runs units bin_start[w] .. bin_start[w+1]-1 in
 * turn.  units (host) gets 4 int32 per unit: {block, first tile, end tile,
 * partial slot or -1 for a block computed by one unit}; bin_start (host)
 * n_bins+1 entries; counts (host) {n_units, n_bins, n_slots}.  Host only,
 * no device work; counts are filled even when the arrays are too small
 * (then G4_ERR_MSG).  No counterpart in the reference, whose prompt runs
 * token at a time (crates/llm-gemma4/src/impl_/generate.rs:37-41). */
int g4_prefill_schedule(int64_t pos0, int64_t N, int64_t window, int head_dim, int n_kv_heads, int num_cus,
                        int32_t *units, int64_t units_cap, int32_t *bin_start, int64_t bins_cap,
                        int32_t *counts);

/* ----------------------------------------- attention input preparation */
/* rms_norm (crates/llm-backend-cpu/src/ops.rs:45-56) applied to each of
 * n_rows rows of `width` floats (norm_heads, model.rs:283-290): f64 mean of
 * squares, x * (1/sqrt(mean+eps)) * weight[i]; weight_dev may be NULL (V). */
int g4_rms_norm_rows(g4_ctx *ctx, const float *x_dev, int64_t n_rows, int64_t width,
                     const float *weight_dev, float eps, float *out_dev, g4_stream stream);

/* rope_neox (ops.rs:134-162) in place on n_tokens x n_heads heads of
 * head_dim floats (rope_heads, model.rs:295-304); token i sits at position
 * pos0 + i.  Angles follow the reference's repeated f32 multiplication by
 * base^(-2/n_rot); freq_factors_dev (n_rot/2 floats, may be NULL) divides
 * them (global layers' rope_freqs). */
int g4_rope_neox_rows(g4_ctx *ctx, float *x_dev, int64_t n_tokens, int n_heads, int head_dim,
                      int n_rot, int64_t pos0, float base, const float *freq_factors_dev,
                      int64_t n_factors, g4_stream stream);

/* ------------------------------------- device-resident ContextMemory (KvCache) */
/* context_memory.rs:11-86 with device rows: n_layers layers, layer l holding
 * up to capacity rows of widths[l] floats (0 = layer keeps no cache). */
int g4_kv_create(g4_ctx *ctx, int n_layers, const int64_t *widths_host, int64_t capacity,
                 g4_kv_cache **cache);
int g4_kv_destroy(g4_kv_cache *cache);
/* append (context_memory.rs:44-51): copies one row of k and v (device). */
int g4_kv_append(g4_kv_cache *cache, int layer, const float *k_dev, const float *v_dev,
                 g4_stream stream);
/* append of n consecutive rows (a prompt chunk's K/V). */
int g4_kv_append_rows(g4_kv_cache *cache, int layer, const float *k_dev, const float *v_dev,
                      int64_t n, g4_stream stream);
/* view (context_memory.rs:53-69): the first len rows, or MissingLayer /
 * ContextTooLong with the reference's numbers.  On a ring layer (below) that
 * has wrapped, G4_ERR_COMPUTE: its first rows are gone. */
int g4_kv_view(const g4_kv_cache *cache, int layer, int64_t len, const float **k_dev,
               const float **v_dev, int64_t *row_stride);
/* The rows of positions [begin, end) as one run of rows (k_dev = position
 * begin's row, row_stride floats apart): the outcomes of view(layer, end),
 * and on a ring layer G4_ERR_COMPUTE when the range starts before the last
 * ring_rows positions.  The layer drivers view a window this way. */
int g4_kv_view_rows(const g4_kv_cache *cache, int layer, int64_t begin, int64_t end,
                    const float **k_dev, const float **v_dev, int64_t *row_stride);
/* g4_kv_create with sliding-window rings (no counterpart in the reference,
 * whose sliding owners keep their whole history, context_memory.rs:11-86):
 * layer l with 0 < ring_rows[l] < capacity keeps only its last ring_rows[l]
 * positions, in 2 * ring_rows[l] rows of storage (every position is stored
 * twice, at p % R and p % R + R, so that any R consecutive positions are one
 * run of rows).  Positions still count up to capacity (ContextTooLong as
 * before); the layer drivers read a ring layer exactly as a whole-history
 * one.  A prefill chunk of n tokens on a layer with window W needs
 * ring_rows >= W + n - 1.  ring_rows_host may be NULL (no rings). */
int g4_kv_create_ring(g4_ctx *ctx, int n_layers, const int64_t *widths_host, int64_t capacity,
                      const int64_t *ring_rows_host, g4_kv_cache **cache);
int64_t g4_kv_len(const g4_kv_cache *cache, int layer);
void g4_kv_clear(g4_kv_cache *cache); /* context_memory.rs:82-84 */

/* --------------------------------------------------- layer attention driver */
/* The Gemma4HyperParams fields attention reads (crates/llm-gemma4/src/idea/mod.rs:15-34). */
typedef struct {
    int n_layers, n_heads, n_kv_heads, head_dim_local, head_dim_global;
    int64_t sliding_window;
    int shared_kv_layers;
    float local_rope_base, global_rope_base, rms_norm_eps;
} g4_hparams;

/* The attention segment of Gemma4CpuModel::layer (model.rs:386-411) from the
 * projected q/k/v on, on the device: norm_heads(q, attn_q_norm), RoPE(q); for
 * owner layers norm_heads(k, attn_k_norm), norm_heads(v, none), RoPE(k),
 * append; view(kv_source_layer, pos+1); window range; attend(scale 1.0).
 * q_dev [n_heads*head_dim] and k_dev/v_dev [n_kv_heads*head_dim] (k/v
 * ignored on shared layers): with head_dim 256 or 512 and 8 query heads per
 * KV head the step is g4_decode_step_fused, which prepares them inside the
 * attention kernel and leaves them as given; other shapes run the
 * preparation first, in place.  rope_freqs_dev ([head_dim_global/2]) is used
 * on global layers.  source, kv_begin, kv_end (host, may be NULL) receive
 * the attended set. */
/* One decode step of a layer with its input preparation fused into the
 * attention kernel (no counterpart in the reference, whose steps are
 * separate, model.rs:394-410): the kernel applies norm_heads(q, q_norm_w) and
 * RoPE at `position` (rope_base, freq_factors_dev or NULL) to q_dev
 * [n_heads*head_dim]; with k_dev, also norm_heads(k, k_norm_w) + RoPE and
 * norm_heads(v, none) to k_dev/v_dev [n_kv_heads*head_dim], writes them to
 * k_row_dev/v_row_dev (the cache row of `position`) and attends them as the
 * last of the n_rows rows of k_cache_dev/v_cache_dev, which it does not
 * read.  Without k_dev (a KV-shared layer) all n_rows rows are read.
 * q/k/v are not modified; nothing moves on the host, so a captured graph can
 * replay it.  head_dim 256 or 512 with 8 query heads per KV head, else
 * G4_ERR_COMPUTE. */
int g4_decode_step_fused(g4_ctx *ctx, const float *q_dev, const float *k_dev, const float *v_dev,
                         const float *q_norm_w_dev, const float *k_norm_w_dev, float eps, float rope_base,
                         const float *freq_factors_dev, int64_t position, const float *k_cache_dev,
                         const float *v_cache_dev, int64_t row_stride, int64_t n_rows, float *k_row_dev,
                         float *v_row_dev, int n_heads, int n_kv_heads, int head_dim, float scale,
                         float *out_dev, g4_stream stream);
int g4_layer_attention(g4_ctx *ctx, g4_kv_cache *cache, const g4_hparams *hp, int layer,
                       int64_t position, float *q_dev, float *k_dev, float *v_dev,
                       const float *q_norm_w_dev, const float *k_norm_w_dev,
                       const float *rope_freqs_dev, float *out_dev, int *source,
                       int64_t *kv_begin, int64_t *kv_end, g4_stream stream);

/* The attention inputs of a layer step in one launch (model.rs:394-406):
 * for token t of n_tokens, at position pos0 + t, norm_heads(q, q_norm_w)
 * then rope_heads on q_dev [n_tokens][n_heads*head_dim]; when k_dev is not
 * NULL also norm_heads(k, k_norm_w), norm_heads(v, none) and rope_heads on
 * k, with k_dev/v_dev [n_tokens][n_kv_heads*head_dim].  Results are written
 * in place and, when k_rows_dev/v_rows_dev are given, also to the cache rows
 * k_rows_dev + t*row_stride (the append of model.rs:405).  RoPE rotates all
 * head_dim dims with base rope_base; freq_factors_dev ([head_dim/2], may be
 * NULL) divides the angles.  Norm weights may be NULL (no weight).  Same
 * arithmetic as g4_rms_norm_rows followed by g4_rope_neox_rows. */
int g4_prepare_qkv(g4_ctx *ctx, float *q_dev, float *k_dev, float *v_dev, int64_t n_tokens,
                   int64_t pos0, int n_heads, int n_kv_heads, int head_dim,
                   const float *q_norm_w_dev, const float *k_norm_w_dev, float eps,
                   float rope_base, const float *freq_factors_dev, float *k_rows_dev,
                   float *v_rows_dev, int64_t row_stride, g4_stream stream);

/* Whole-layer prefill: the attention segment of Gemma4CpuModel::layer
 * (model.rs:386-411) for the n_tokens prompt positions pos0, pos0+1, ... in
 * one call.  Run over the layers in ascending order, it gives what the
 * reference's token-at-a-time prompt loop (crates/llm-idea/src/transformer.rs:40-53,
 * crates/llm-gemma4/src/impl_/generate.rs:37-41) computes: query i attends the
 * rows a decode at position pos0+i would.  q_dev [n_tokens][n_heads*d] and,
 * on owner layers, k_dev/v_dev [n_tokens][n_kv_heads*d] are prepared in place
 * (as g4_prepare_qkv) and k/v appended; out_dev [n_tokens][n_heads*d].  An
 * owner layer's cache must already hold pos0 rows (else ContextTooLong, as
 * the first token's view would fail); a shared layer's source must hold
 * pos0 + n_tokens rows.  The reference has no batched prefill; this is the
 * driver its prompt loop would call. */
int g4_layer_prefill(g4_ctx *ctx, g4_kv_cache *cache, const g4_hparams *hp, int layer,
                     int64_t pos0, int64_t n_tokens, float *q_dev, float *k_dev, float *v_dev,
                     const float *q_norm_w_dev, const float *k_norm_w_dev,
                     const float *rope_freqs_dev, float *out_dev, int *source,
                     g4_stream stream);

/* ----------------------------------------------------------- policies */
/* layer_attention_kind (idea/mod.rs:148-156): 1 global, 0 local. */
int g4_layer_is_global(int n_layers, int layer);
/* kv_source_layer (crates/llm-gemma4/src/eng/mod.rs:71-90); KvShareError ->
 * G4_ERR_COMPUTE with its Display text, as model.rs:398 maps it. */
int g4_kv_source_layer(int n_layers, int shared_kv_layers, int layer, int *source);
/* windowed_len (eng/mod.rs:10-12). */
void g4_windowed_len(int64_t seq_len, int64_t window, int64_t *begin, int64_t *end);
/* proportional_rope_freq_factors (idea/mod.rs:162-165), out[head_dim/2] host. */
void g4_proportional_rope_freq_factors(int head_dim, float p, float *out_host);

/* -------------- mat-vecs over GGUF weight formats (crates/llm-backend-cpu/src/matvec.rs) */
/* Weights are row-major [rows][cols] in their GGUF storage: Q8_0 rows of
 * cols/32 blocks of 34 bytes (f16 scale, 32 int8), BF16 or f32 values.
 * Results are bit-identical to the reference's (same per-block integer dots,
 * same f32 products, sums in the reference's order); only tanh in GELU and
 * the soft-cap comes from the device libm.  Shape errors carry the
 * reference's messages ("Q8_0 weight has N elements, expected R rows of L"). */

/* quantize_q8_0 (matvec.rs:35-53): x_dev [n], n a multiple of 32 ->
 * scales_dev [n/32] (each the f16 rounding of max|x|/127, as f32) and
 * quants_dev [n]. */
int g4_quantize_q8_0(g4_ctx *ctx, const float *x_dev, int64_t n, float *scales_dev,
                     int8_t *quants_dev, g4_stream stream);
/* matvec_q8_0 (matvec.rs:55-62): out_dev[rows] = W @ x for a Q8_0 activation
 * (x_scales_dev [cols/32], x_quants_dev [cols]); w_bytes = rows*cols/32*34. */
int g4_matvec_q8_0(g4_ctx *ctx, const uint8_t *w_dev, int64_t w_bytes, int64_t rows, int64_t cols,
                   const float *x_scales_dev, const int8_t *x_quants_dev, float *out_dev,
                   g4_stream stream);
/* matvec_q8_0_then(.., softcap, cap) (matvec.rs:64-81, model.rs:447):
 * cap * tanh(logit / cap) on every output -- the final logits. */
int g4_matvec_q8_0_softcap(g4_ctx *ctx, const uint8_t *w_dev, int64_t w_bytes, int64_t rows,
                           int64_t cols, const float *x_scales_dev, const int8_t *x_quants_dev,
                           float cap, float *out_dev, g4_stream stream);
/* geglu_q8_0 (matvec.rs:83-102): gelu(gate_row . x) * (up_row . x); gelu is
 * gelu_tanh, or gelu_tanh_fp16_table when fp16_gelu (ops.rs:85-103). */
int g4_geglu_q8_0(g4_ctx *ctx, const uint8_t *gate_dev, const uint8_t *up_dev, int64_t w_bytes,
                  int64_t rows, int64_t cols, const float *x_scales_dev,
                  const int8_t *x_quants_dev, int fp16_gelu, float *out_dev, g4_stream stream);
/* The model-level calls with the activation quantization folded in (one
 * launch; the same results as g4_quantize_q8_0 followed by the call above):
 * `project` with quantized activations (model.rs:211-212), the GELU-gated
 * FFN input (model.rs:236-237) and the soft-capped logits (model.rs:447).
 * x_dev [cols] f32. */
int g4_project_q8_0(g4_ctx *ctx, const uint8_t *w_dev, int64_t w_bytes, int64_t rows, int64_t cols,
                    const float *x_dev, float *out_dev, g4_stream stream);
int g4_gated_ffn_q8_0(g4_ctx *ctx, const uint8_t *gate_dev, const uint8_t *up_dev, int64_t w_bytes,
                      int64_t rows, int64_t cols, const float *x_dev, int fp16_gelu, float *out_dev,
                      g4_stream stream);
int g4_logits_q8_0(g4_ctx *ctx, const uint8_t *w_dev, int64_t w_bytes, int64_t rows, int64_t cols,
                   const float *x_dev, float cap, float *out_dev, g4_stream stream);
/* matvec_q8_0_f32 / matvec_q8_0_f64_sums (matvec.rs:104-122): an f32
 * activation against dequantized blocks; f64_sums takes every sum in f64. */
int g4_matvec_q8_0_f32(g4_ctx *ctx, const uint8_t *w_dev, int64_t w_bytes, int64_t rows, int64_t cols,
                       const float *x_dev, int f64_sums, float *out_dev, g4_stream stream);
/* matvec_bf16 (matvec.rs:124-130): x rounded to bf16 first, as ggml does. */
int g4_matvec_bf16(g4_ctx *ctx, const uint16_t *w_dev, int64_t w_len, int64_t rows, int64_t cols,
                   const float *x_dev, float *out_dev, g4_stream stream);
/* matvec_f32 (matvec.rs:132-136). */
int g4_matvec_f32(g4_ctx *ctx, const float *w_dev, int64_t w_len, int64_t rows, int64_t cols,
                  const float *x_dev, float *out_dev, g4_stream stream);

/* ------------------------------------- ComputePort (crates/llm-eng/src/compute.rs:3-29) */
/* HipPort: the trait's method set on device buffers, with CpuPort's
 * semantics (crates/llm-backend-cpu/src/port.rs:11-51). */
int g4_port_matmul(g4_ctx *ctx, const float *a_dev, const float *b_dev, int64_t m, int64_t n,
                   int64_t k, float *out_dev, g4_stream stream);           /* ops.rs:9-39 */
int g4_port_rms_norm(g4_ctx *ctx, const float *x_dev, const float *weight_dev, int64_t n,
                     float eps, float *out_dev, g4_stream stream);         /* ops.rs:58-60 */
int g4_port_softmax(g4_ctx *ctx, const float *x_dev, int64_t n, float *out_dev,
                    g4_stream stream);                                      /* ops.rs:105-127 */
int g4_port_rope(g4_ctx *ctx, float *x_dev, int64_t len, int64_t pos, float theta,
                 int64_t dims, g4_stream stream);                           /* ops.rs:164-166 */
int g4_port_add(g4_ctx *ctx, const float *a_dev, const float *b_dev, int64_t n, float *out_dev,
                g4_stream stream);                                          /* ops.rs:168-178 */

#ifdef __cplusplus
}
#endif
#endif /* G4ATTN_H */
