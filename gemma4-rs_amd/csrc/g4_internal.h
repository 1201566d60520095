// Internal declarations shared by the backend's translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/g4attn.h"

namespace g4 {

// Error state of the calling thread, read back through g4_last_error().
int set_error(int code, const std::string &message, uint64_t a = 0, uint64_t b = 0);
void clear_error();

// hipError_t -> EngError::Compute("hip: ...").
int hip_failed(hipError_t e, const char *what);

#define G4_HIP(call)                                                   \
    do {                                                               \
        hipError_t e_ = (call);                                        \
        if (e_ != hipSuccess) return ::g4::hip_failed(e_, #call);      \
    } while (0)

// Status bits the kernels raise in the context's device status word.
enum : unsigned {
    kStatusNonFinite = 1u,   // softmax input not finite (model.rs:362-364)
    kStatusRangeTooLong = 2u // a ragged range exceeded max_kv_len
};

struct Workspace {
    void *ptr = nullptr;
    size_t bytes = 0;
};

}  // namespace g4

struct g4_ctx {
    int device = 0;
    unsigned *status_dev = nullptr;  // kStatus* bits, cleared by g4_check_status
    g4::Workspace ws;                // split-K partials of the decode kernels
    int64_t decode_chunk = 0;        // 0 = automatic
    int prefill_exact = 0;           // 1: prefill uses f32 MFMAs only (no split-f16 products)
    int num_cus = 256;
    int64_t *zero_rows = nullptr;    // device zeros: default row offsets of a batch
    int64_t zero_rows_len = 0;
    void *prefill_plan = nullptr;    // work-unit table of the last prefill shape
    void *scratch = nullptr;         // this device's static decode scratch (g4_attend_decode_noalloc)
    size_t scratch_bytes = 0;
};

namespace g4 {

// Grows the context's workspace to at least `bytes` (stream-ordered users
// must not be in flight on another stream when it grows).
int ensure_workspace(g4_ctx *ctx, size_t bytes, hipStream_t stream);
// Makes ctx->zero_rows hold at least n zero int64 values.
int ensure_zero_rows(g4_ctx *ctx, int64_t n);

// Launchers implemented in the .hip files.
struct DecodeArgs {
    int B;
    const float *q;
    const float *k;
    const float *v;
    int64_t row_stride;
    const int64_t *seq_row0;  // device or null
    const int64_t *kv_begin;  // device or null -> kv_begin0 for every sequence
    const int64_t *kv_end;    // device or null -> kv_end0
    int64_t kv_begin0, kv_end0;
    int64_t max_kv_len;
    // Prefill form: when `prefill_window >= 0`, sequence s is query s at
    // position pos0 + s, with range [(p+1-window)+ or 0, p+1).
    int64_t pos0;
    int64_t prefill_window;  // -1: not prefill; 0: global; >0: sliding window
    int64_t kv_origin;       // prefill form: the position of row 0 of k/v
    int n_heads, n_kv_heads, head_dim;
    float scale;
    float *out;
    // When set, the split partials go here instead of the context's
    // workspace (nothing is allocated); a shape that needs more than
    // scratch_bytes is refused.  Single-sequence decodes only.
    void *scratch;
    size_t scratch_bytes;
};
int launch_decode(g4_ctx *ctx, const DecodeArgs &a, hipStream_t stream);
// The device address (on the current device) and size of the static scratch
// array that g4_attend_decode_noalloc uses.
int decode_scratch_address(void **ptr, size_t *bytes);

// A layer's decode step with its input preparation fused in (the layer
// driver's form): the decode kernel prepares q itself (rms_norm with q_w,
// NEOX RoPE at `position`) and, on owner layers, the new row's k and v,
// which it appends at k_row/v_row and attends as the range's last key.  q, k
// and v are read, not modified.  The DecodeArgs are a single range whose
// last row is `position`; on an owner layer that row is not read from the
// cache.
constexpr int kPrepMaxAngles = 256;  // head_dim 512
struct LayerPrepArgs {
    const float *q;                  // [n_heads][head_dim]
    const float *k, *v;              // [n_kv_heads][head_dim]; k == nullptr on a KV-shared layer
    const float *q_w, *k_w, *factors;
    float eps;
    int64_t position;
    float *k_row, *v_row;            // owner layers: the cache row of `position`
    // rope_neox's angles at `position`, theta_i = position * theta_scale^i by
    // the reference's sequential recurrence, computed on the host (f32
    // multiplication rounds the same there) so that no workgroup spends the
    // 256 dependent steps; head_dim/2 of them are used.
    float angles[kPrepMaxAngles];
};
bool layer_decode_fusable(const DecodeArgs &a);
int launch_layer_decode(g4_ctx *ctx, const DecodeArgs &a, const LayerPrepArgs &lp, hipStream_t stream);

struct PrefillArgs {
    const float *q;
    const float *k;
    const float *v;
    int64_t row_stride;
    int64_t pos0, N, window;
    int64_t kv_origin;  // the position of row 0 of k/v (rows before it are never read)
    int n_heads, n_kv_heads, head_dim;
    float scale;
    float *out;
};
int launch_prefill(g4_ctx *ctx, const PrefillArgs &a, hipStream_t stream);
void release_prefill_plan(g4_ctx *ctx);
// The prefill kernel's work schedule for a shape (host only).
int describe_prefill_schedule(int64_t pos0, int64_t N, int64_t window, int head_dim, int n_kv_heads, int num_cus,
                              int32_t *units4, int64_t units_cap, int32_t *bin_start, int64_t bins_cap,
                              int32_t *counts);

int launch_rms_norm_rows(const float *x, int64_t n_rows, int64_t width, const float *w, float eps,
                         float *out, hipStream_t stream);
int launch_rope_rows(float *x, int64_t n_tokens, int n_heads, int head_dim, int n_rot,
                     int64_t pos0, float theta_scale, const float *factors, hipStream_t stream);
// Fused norm + RoPE + append of one layer step's q/k/v for n_tokens tokens
// (token t at position pos0 + t).  q: [n_tokens][n_heads][head_dim]; k, v:
// [n_tokens][n_kv_heads][head_dim] or k == nullptr (q only); k_rows/v_rows:
// the cache rows of token 0 (row_stride floats apart) or nullptr.
struct PrepareArgs {
    float *q;
    float *k;
    float *v;
    float *k_rows;
    float *v_rows;
    int64_t row_stride;
    const float *q_w;
    const float *k_w;
    const float *factors;  // [head_dim/2] RoPE divisors or nullptr
    int64_t n_tokens, pos0;
    int n_heads, n_kv_heads, head_dim;
    float eps, theta_scale;
};
int launch_prepare_qkv(const PrepareArgs &a, hipStream_t stream);
int launch_matmul(const float *a, const float *b, int64_t m, int64_t n, int64_t k, float *out,
                  hipStream_t stream);

// Mat-vecs over GGUF weight formats (g4_matvec.hip).
enum class MatvecKind { Q8, Q8Softcap, Q8Geglu, Q8GegluFp16, Q8F32, Q8F64, Bf16, F32 };
struct MatvecArgs {
    MatvecKind kind;
    const unsigned char *w;   // Q8_0 bytes, bf16 or f32 values, row-major [rows][cols]
    const unsigned char *w2;  // the up matrix of the Geglu kinds
    int64_t rows, cols;
    const float *xs;          // Q8_0 activation: block scales [cols/32]
    const signed char *xq;    // Q8_0 activation: values [cols]
    const float *x;           // f32 activation [cols] (Q8F32, Q8F64, Bf16, F32; the Q8 kinds
                              // quantize it themselves when xs is null)
    float arg;                // soft-cap
    float *out;               // [rows]
};
int launch_quantize_q8_0(const float *x, int64_t n, float *scales, signed char *quants, hipStream_t stream);
int launch_matvec(g4_ctx *ctx, const MatvecArgs &a, hipStream_t stream);
int launch_softmax(const float *x, int64_t n, float *out, unsigned *status, hipStream_t stream);
int launch_add(const float *a, const float *b, int64_t n, float *out, hipStream_t stream);

}  // namespace g4
