// C ABI entry points: context, errors, attention calls, device KvCache, the
// layer attention driver, the engine's policies and the ComputePort methods.

#include <climits>
#include <math.h>
#include <new>
#include <string>
#include <vector>

#include "g4_internal.h"

namespace {

thread_local std::string t_msg;
thread_local uint64_t t_field_a = 0, t_field_b = 0;

hipStream_t as_stream(g4_stream s) { return reinterpret_cast<hipStream_t>(s); }

// Runs `body`, turning any escaping C++ exception into an error code.
template <class F>
int guarded(F &&body) {
    try {
        return body();
    } catch (const std::bad_alloc &) {
        return g4::set_error(G4_ERR_COMPUTE, "host allocation failed");
    } catch (...) {
        return g4::set_error(G4_ERR_COMPUTE, "unexpected internal error");
    }
}

int invalid(const char *what) { return g4::set_error(G4_ERR_COMPUTE, what); }

}  // namespace

namespace g4 {

int set_error(int code, const std::string &message, uint64_t a, uint64_t b) {
    t_msg = message;
    t_field_a = a;
    t_field_b = b;
    return code;
}

void clear_error() {
    t_msg.clear();
    t_field_a = t_field_b = 0;
}

int hip_failed(hipError_t e, const char *what) {
    return set_error(G4_ERR_COMPUTE, std::string("hip: ") + hipGetErrorString(e) + " (" + what + ")");
}

int ensure_workspace(g4_ctx *ctx, size_t bytes, hipStream_t stream) {
    (void)stream;
    if (ctx->ws.bytes >= bytes) return G4_OK;
    // Growth is rare (first use of a larger shape): drain all work that may
    // still read the old buffer before replacing it.
    G4_HIP(hipDeviceSynchronize());
    if (ctx->ws.ptr) G4_HIP(hipFree(ctx->ws.ptr));
    ctx->ws.ptr = nullptr;
    ctx->ws.bytes = 0;
    const size_t grown = bytes + bytes / 4;
    G4_HIP(hipMalloc(&ctx->ws.ptr, grown));
    ctx->ws.bytes = grown;
    return G4_OK;
}

int ensure_zero_rows(g4_ctx *ctx, int64_t n) {
    if (ctx->zero_rows_len >= n) return G4_OK;
    G4_HIP(hipDeviceSynchronize());
    if (ctx->zero_rows) G4_HIP(hipFree(ctx->zero_rows));
    ctx->zero_rows = nullptr;
    ctx->zero_rows_len = 0;
    const int64_t len = n < 1024 ? 1024 : n;
    G4_HIP(hipMalloc(&ctx->zero_rows, len * sizeof(int64_t)));
    G4_HIP(hipMemset(ctx->zero_rows, 0, len * sizeof(int64_t)));
    ctx->zero_rows_len = len;
    return G4_OK;
}

}  // namespace g4

// -------------------------------------------------------------- device KvCache
struct g4_kv_cache {
    g4_ctx *ctx = nullptr;
    int n_layers = 0;
    int64_t capacity = 0;
    std::vector<int64_t> width;
    std::vector<float *> k, v;
    std::vector<int64_t> rows;  // positions appended
    // Ring layers keep only their last ring[l] rows: position p at slots
    // p % R and p % R + R of 2R rows, so any R consecutive positions are
    // contiguous rows.  0: the whole history, position p at row p.
    std::vector<int64_t> ring;
    int known_layers = 0;  // layers.len() of the reference's Vec<Layer>
};

namespace {

// Row of position p (resident) in layer l's storage.
int64_t slot_of(const g4_kv_cache *c, int l, int64_t p) { return c->ring[l] > 0 ? p % c->ring[l] : p; }

// Copies m rows of positions p.. (m <= R) from contiguous device rows src_k /
// src_v into ring layer l: each position to its slot and its mirror.
int ring_store(g4_kv_cache *c, int l, const float *src_k, const float *src_v, int64_t p, int64_t m,
               hipStream_t stream) {
    const int64_t R = c->ring[l], w = c->width[l], s0 = p % R;
    const int64_t m1 = std::min(m, R - s0), m2 = m - m1;  // before and after the wrap
    const size_t rb = (size_t)w * sizeof(float);
    for (int64_t mirror = 0; mirror <= R; mirror += R) {
        G4_HIP(hipMemcpyAsync(c->k[l] + (s0 + mirror) * w, src_k, rb * m1, hipMemcpyDeviceToDevice, stream));
        G4_HIP(hipMemcpyAsync(c->v[l] + (s0 + mirror) * w, src_v, rb * m1, hipMemcpyDeviceToDevice, stream));
        if (m2 > 0) {
            G4_HIP(hipMemcpyAsync(c->k[l] + mirror * w, src_k + m1 * w, rb * m2, hipMemcpyDeviceToDevice, stream));
            G4_HIP(hipMemcpyAsync(c->v[l] + mirror * w, src_v + m1 * w, rb * m2, hipMemcpyDeviceToDevice, stream));
        }
    }
    return G4_OK;
}

// After n rows were written at slots [s, s + n) of ring layer l (n <= R,
// so s + n <= 2R), copies each to its other slot, s +- R.
int ring_mirror(g4_kv_cache *c, int l, int64_t s, int64_t n, hipStream_t stream) {
    const int64_t R = c->ring[l], w = c->width[l];
    const size_t rb = (size_t)w * sizeof(float);
    const int64_t a0 = s, a1 = std::min(s + n, R);   // below R: mirrors at +R
    const int64_t b0 = std::max(s, R), b1 = s + n;   // from R on: mirrors at -R
    for (float *base : {c->k[l], c->v[l]}) {
        if (a1 > a0)
            G4_HIP(hipMemcpyAsync(base + (a0 + R) * w, base + a0 * w, rb * (a1 - a0), hipMemcpyDeviceToDevice, stream));
        if (b1 > b0)
            G4_HIP(hipMemcpyAsync(base + (b0 - R) * w, base + b0 * w, rb * (b1 - b0), hipMemcpyDeviceToDevice, stream));
    }
    return G4_OK;
}

}  // namespace

extern "C" {

const char *g4_last_error(void) { return t_msg.c_str(); }

void g4_last_error_fields(uint64_t *a, uint64_t *b) {
    if (a) *a = t_field_a;
    if (b) *b = t_field_b;
}

int g4_init(int device, g4_ctx **out) {
    return guarded([&] {
        g4::clear_error();
        if (!out) return invalid("g4_init: null output pointer");
        *out = nullptr;
        G4_HIP(hipSetDevice(device));
        auto *ctx = new g4_ctx();
        ctx->device = device;
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0)
            ctx->num_cus = cus;
        hipError_t e = hipMalloc(&ctx->status_dev, sizeof(unsigned));
        if (e == hipSuccess) e = hipMemset(ctx->status_dev, 0, sizeof(unsigned));
        if (e != hipSuccess) {
            if (ctx->status_dev) (void)hipFree(ctx->status_dev);
            delete ctx;
            return g4::hip_failed(e, "g4_init");
        }
        // This device's copy of the static decode scratch (with the device
        // current): g4_attend_decode_noalloc passes this address, never the
        // array's host-side name.
        const int rc = g4::decode_scratch_address(&ctx->scratch, &ctx->scratch_bytes);
        if (rc != G4_OK) {
            (void)hipFree(ctx->status_dev);
            delete ctx;
            return rc;
        }
        *out = ctx;
        return (int)G4_OK;
    });
}

int g4_release(g4_ctx *ctx) {
    return guarded([&] {
        if (!ctx) return (int)G4_OK;
        G4_HIP(hipSetDevice(ctx->device));
        G4_HIP(hipDeviceSynchronize());
        if (ctx->ws.ptr) G4_HIP(hipFree(ctx->ws.ptr));
        if (ctx->zero_rows) G4_HIP(hipFree(ctx->zero_rows));
        g4::release_prefill_plan(ctx);
        if (ctx->status_dev) G4_HIP(hipFree(ctx->status_dev));
        delete ctx;
        return (int)G4_OK;
    });
}

// ------------------------------------------------------------ device memory
int g4_alloc(g4_ctx *ctx, size_t bytes, void **ptr) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx || !ptr) return invalid("g4_alloc: null argument");
        *ptr = nullptr;
        if (bytes == 0) return (int)G4_OK;
        G4_HIP(hipSetDevice(ctx->device));
        G4_HIP(hipMalloc(ptr, bytes));
        return (int)G4_OK;
    });
}

int g4_free(g4_ctx *ctx, void *ptr) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx) return invalid("g4_free: null context");
        if (!ptr) return (int)G4_OK;
        G4_HIP(hipSetDevice(ctx->device));
        G4_HIP(hipDeviceSynchronize());
        G4_HIP(hipFree(ptr));
        return (int)G4_OK;
    });
}

namespace {

int copy_sync(g4_ctx *ctx, void *dst, const void *src, size_t bytes, hipMemcpyKind kind, const char *name) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx) return invalid((std::string(name) + ": null context").c_str());
        if (bytes == 0) return (int)G4_OK;
        if (!dst || !src) return invalid((std::string(name) + ": null pointer").c_str());
        G4_HIP(hipSetDevice(ctx->device));
        G4_HIP(hipDeviceSynchronize());
        G4_HIP(hipMemcpy(dst, src, bytes, kind));
        return (int)G4_OK;
    });
}

}  // namespace

int g4_copy_to_device(g4_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return copy_sync(ctx, dst, src, bytes, hipMemcpyHostToDevice, "g4_copy_to_device");
}

int g4_copy_to_host(g4_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return copy_sync(ctx, dst, src, bytes, hipMemcpyDeviceToHost, "g4_copy_to_host");
}

int g4_copy_on_device(g4_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return copy_sync(ctx, dst, src, bytes, hipMemcpyDeviceToDevice, "g4_copy_on_device");
}

int g4_sync(g4_ctx *ctx, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx) return invalid("g4_sync: null context");
        G4_HIP(hipSetDevice(ctx->device));
        G4_HIP(hipStreamSynchronize(as_stream(stream)));
        return (int)G4_OK;
    });
}

int g4_activate(g4_ctx *ctx) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx) return invalid("g4_activate: null context");
        G4_HIP(hipSetDevice(ctx->device));
        return (int)G4_OK;
    });
}

int g4_check_status(g4_ctx *ctx, g4_stream stream) {
    return guarded([&] {
        if (!ctx) return invalid("g4_check_status: null context");
        G4_HIP(hipStreamSynchronize(as_stream(stream)));
        unsigned st = 0;
        G4_HIP(hipMemcpy(&st, ctx->status_dev, sizeof st, hipMemcpyDeviceToHost));
        if (st == 0) return (int)G4_OK;
        G4_HIP(hipMemset(ctx->status_dev, 0, sizeof(unsigned)));
        if (st & g4::kStatusNonFinite)
            return g4::set_error(G4_ERR_COMPUTE, "softmax input is not finite");
        return g4::set_error(G4_ERR_CONTEXT_TOO_LONG,
                             "a sequence's K/V range is longer than max_kv_len");
    });
}

int g4_set_decode_chunk(g4_ctx *ctx, int64_t keys) {
    if (!ctx) return invalid("g4_set_decode_chunk: null context");
    if (keys < 0) return invalid("g4_set_decode_chunk: negative key count");
    ctx->decode_chunk = keys;
    return G4_OK;
}

int g4_set_prefill_exact(g4_ctx *ctx, int exact) {
    if (!ctx) return invalid("g4_set_prefill_exact: null context");
    if (exact != 0 && exact != 1) return invalid("g4_set_prefill_exact: exact must be 0 or 1");
    ctx->prefill_exact = exact;
    return G4_OK;
}

// ------------------------------------------------------------------ attention
static int check_heads(int n_heads, int n_kv_heads, int head_dim) {
    if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0)
        return invalid("attention needs positive head counts and head width");
    if (n_kv_heads > n_heads) return invalid("more KV heads than query heads");
    return G4_OK;
}

namespace {

// g4_attend_decode, with the split partials in the context's workspace or,
// when scratch is set, in the static scratch (no allocation).
int attend_decode(g4_ctx *ctx, const float *q, const float *k_cache, const float *v_cache, int64_t row_stride,
                  int64_t kv_begin, int64_t kv_end, int n_heads, int n_kv_heads, int head_dim, float scale,
                  float *out, g4_stream stream, bool scratch) {
    if (!ctx) return invalid("g4_attend_decode: null context");
    int rc = check_heads(n_heads, n_kv_heads, head_dim);
    if (rc != G4_OK) return rc;
    if (row_stride < (int64_t)n_kv_heads * head_dim) return invalid("row_stride below the row width");
    if (kv_begin < 0 || kv_end <= kv_begin)
        return g4::set_error(G4_ERR_COMPUTE, "softmax input is not finite");
    g4::DecodeArgs a{};
    a.B = 1;
    a.q = q;
    a.k = k_cache;
    a.v = v_cache;
    a.row_stride = row_stride;
    a.kv_begin0 = kv_begin;
    a.kv_end0 = kv_end;
    a.max_kv_len = kv_end - kv_begin;
    a.prefill_window = -1;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.head_dim = head_dim;
    a.scale = scale;
    a.out = out;
    if (scratch) {
        a.scratch = ctx->scratch;
        a.scratch_bytes = ctx->scratch_bytes;
    }
    return g4::launch_decode(ctx, a, as_stream(stream));
}

}  // namespace

int g4_attend_decode(g4_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
                     int64_t row_stride, int64_t kv_begin, int64_t kv_end, int n_heads,
                     int n_kv_heads, int head_dim, float scale, float *out, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        return attend_decode(ctx, q, k_cache, v_cache, row_stride, kv_begin, kv_end, n_heads, n_kv_heads, head_dim,
                             scale, out, stream, false);
    });
}

int g4_attend_decode_noalloc(g4_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
                             int64_t row_stride, int64_t kv_begin, int64_t kv_end, int n_heads, int n_kv_heads,
                             int head_dim, float scale, float *out, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        return attend_decode(ctx, q, k_cache, v_cache, row_stride, kv_begin, kv_end, n_heads, n_kv_heads, head_dim,
                             scale, out, stream, true);
    });
}

int g4_attend_decode_batch(g4_ctx *ctx, int B, const float *q, const float *k_base,
                           const float *v_base, int64_t row_stride, const int64_t *seq_row0,
                           const int64_t *kv_begin, const int64_t *kv_end, int64_t max_kv_len,
                           int n_heads, int n_kv_heads, int head_dim, float scale, float *out,
                           g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx) return invalid("g4_attend_decode_batch: null context");
        if (B < 0) return invalid("negative batch size");
        if (B == 0) return (int)G4_OK;
        int rc = check_heads(n_heads, n_kv_heads, head_dim);
        if (rc != G4_OK) return rc;
        if (!kv_begin || !kv_end) return invalid("kv_begin and kv_end are required");
        if (max_kv_len <= 0) return invalid("max_kv_len must be positive");
        if (row_stride < (int64_t)n_kv_heads * head_dim) return invalid("row_stride below the row width");
        g4::DecodeArgs a{};
        a.B = B;
        a.q = q;
        a.k = k_base;
        a.v = v_base;
        a.row_stride = row_stride;
        a.seq_row0 = seq_row0;
        a.kv_begin = kv_begin;
        a.kv_end = kv_end;
        a.max_kv_len = max_kv_len;
        a.prefill_window = -1;
        a.n_heads = n_heads;
        a.n_kv_heads = n_kv_heads;
        a.head_dim = head_dim;
        a.scale = scale;
        a.out = out;
        return g4::launch_decode(ctx, a, as_stream(stream));
    });
}

namespace {

// g4_attend_prefill with the K/V rows starting at position kv_origin (the
// rows a ring or a windowed view hands over); kv_origin 0 is the public form.
int attend_prefill_rows(g4_ctx *ctx, const float *q, const float *k_cache, const float *v_cache, int64_t row_stride,
                        int64_t pos0, int64_t N, int64_t window, int64_t kv_origin, int n_heads, int n_kv_heads,
                        int head_dim, float scale, float *out, g4_stream stream) {
    if (!ctx) return invalid("g4_attend_prefill: null context");
    if (N < 0 || pos0 < 0 || window < 0) return invalid("prefill needs N, pos0, window >= 0");
    if (N == 0) return (int)G4_OK;
    int rc = check_heads(n_heads, n_kv_heads, head_dim);
    if (rc != G4_OK) return rc;
    if (row_stride < (int64_t)n_kv_heads * head_dim) return invalid("row_stride below the row width");
    const int64_t first_row = (window > 0 && pos0 + 1 > window) ? pos0 + 1 - window : 0;
    if (kv_origin < 0 || kv_origin > first_row) return invalid("prefill attends rows before the first row held");
    g4::PrefillArgs a{};
    a.q = q;
    a.k = k_cache;
    a.v = v_cache;
    a.row_stride = row_stride;
    a.pos0 = pos0;
    a.N = N;
    a.window = window;
    a.kv_origin = kv_origin;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.head_dim = head_dim;
    a.scale = scale;
    a.out = out;
    return g4::launch_prefill(ctx, a, as_stream(stream));
}

}  // namespace

int g4_attend_prefill(g4_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
                      int64_t row_stride, int64_t pos0, int64_t N, int64_t window, int n_heads,
                      int n_kv_heads, int head_dim, float scale, float *out, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        return attend_prefill_rows(ctx, q, k_cache, v_cache, row_stride, pos0, N, window, 0, n_heads, n_kv_heads,
                                   head_dim, scale, out, stream);
    });
}

int g4_prefill_schedule(int64_t pos0, int64_t N, int64_t window, int head_dim, int n_kv_heads, int num_cus,
                        int32_t *units, int64_t units_cap, int32_t *bin_start, int64_t bins_cap, int32_t *counts) {
    return guarded([&] {
        g4::clear_error();
        if (N <= 0 || pos0 < 0 || window < 0) return invalid("prefill schedule needs N > 0, pos0, window >= 0");
        if (head_dim != 256 && head_dim != 512) return invalid("prefill schedule: head_dim must be 256 or 512");
        if (n_kv_heads < 1 || num_cus < 1) return invalid("prefill schedule: n_kv_heads and num_cus must be positive");
        if (!units || !bin_start || !counts) return invalid("prefill schedule: null output array");
        return g4::describe_prefill_schedule(pos0, N, window, head_dim, n_kv_heads, num_cus, units, units_cap,
                                             bin_start, bins_cap, counts);
    });
}

int g4_attend(g4_ctx *ctx, const float *q_host, size_t q_len, const float *keys_host,
              const float *values_host, size_t T, size_t n_heads, size_t n_kv_heads, float scale,
              float *out_host) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx) return invalid("g4_attend: null context");
        if (n_heads == 0 || n_kv_heads == 0) return invalid("attention needs positive head counts");
        const size_t head_dim = q_len / n_heads;
        if (head_dim == 0) return invalid("q is shorter than n_heads");
        // model.rs:362-364: an empty context fails the softmax of every head,
        // and a q whose length is not n_heads * head_dim leaves the heads'
        // concatenation shorter than q; both return this error.
        if (T == 0 || q_len != n_heads * head_dim)
            return g4::set_error(G4_ERR_COMPUTE, "softmax input is not finite");
        const size_t width = n_kv_heads * head_dim;
        const size_t used_q = n_heads * head_dim;
        G4_HIP(hipSetDevice(ctx->device));
        float *dq = nullptr, *dk = nullptr, *dv = nullptr, *dout = nullptr;
        auto release = [&] {
            if (dq) (void)hipFree(dq);
            if (dk) (void)hipFree(dk);
            if (dv) (void)hipFree(dv);
            if (dout) (void)hipFree(dout);
        };
        hipError_t e = hipMalloc(&dq, used_q * sizeof(float));
        if (e == hipSuccess) e = hipMalloc(&dk, T * width * sizeof(float));
        if (e == hipSuccess) e = hipMalloc(&dv, T * width * sizeof(float));
        if (e == hipSuccess) e = hipMalloc(&dout, used_q * sizeof(float));
        if (e == hipSuccess) e = hipMemcpy(dq, q_host, used_q * sizeof(float), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(dk, keys_host, T * width * sizeof(float), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(dv, values_host, T * width * sizeof(float), hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            release();
            return g4::hip_failed(e, "g4_attend staging");
        }
        int rc = g4_attend_decode(ctx, dq, dk, dv, (int64_t)width, 0, (int64_t)T, (int)n_heads,
                                  (int)n_kv_heads, (int)head_dim, scale, dout, nullptr);
        if (rc == G4_OK) rc = g4_check_status(ctx, nullptr);
        if (rc == G4_OK) {
            e = hipMemcpy(out_host, dout, used_q * sizeof(float), hipMemcpyDeviceToHost);
            if (e != hipSuccess) rc = g4::hip_failed(e, "g4_attend result");
        }
        release();
        return rc;
    });
}

// ---------------------------------------------------------------- preparation
int g4_rms_norm_rows(g4_ctx *ctx, const float *x, int64_t n_rows, int64_t width,
                     const float *weight, float eps, float *out, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx) return invalid("g4_rms_norm_rows: null context");
        if (width <= 0 || eps < 0.0f || n_rows < 0)
            return g4::set_error(G4_ERR_COMPUTE, "invalid RMS norm inputs");
        return g4::launch_rms_norm_rows(x, n_rows, width, weight, eps, out, as_stream(stream));
    });
}

int g4_rope_neox_rows(g4_ctx *ctx, float *x, int64_t n_tokens, int n_heads, int head_dim,
                      int n_rot, int64_t pos0, float base, const float *freq_factors,
                      int64_t n_factors, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx) return invalid("g4_rope_neox_rows: null context");
        const int half = n_rot / 2;
        // ops.rs:142-149
        if (n_rot <= 0 || n_rot % 2 != 0 || n_rot > head_dim || base <= 0.0f ||
            (freq_factors && n_factors < half) || n_heads <= 0 || n_tokens < 0 || pos0 < 0)
            return g4::set_error(G4_ERR_COMPUTE, "invalid RoPE inputs");
        // The reference computes base.powf(-2.0 / n_rot) on the host's libm.
        const float theta_scale = powf(base, -2.0f / (float)n_rot);
        return g4::launch_rope_rows(x, n_tokens, n_heads, head_dim, n_rot, pos0, theta_scale,
                                    freq_factors, as_stream(stream));
    });
}

// ------------------------------------------------------------------ KvCache
int g4_kv_create_ring(g4_ctx *ctx, int n_layers, const int64_t *widths, int64_t capacity,
                      const int64_t *ring_rows, g4_kv_cache **out) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx || !out || !widths) return invalid("g4_kv_create: null argument");
        if (n_layers <= 0 || capacity <= 0) return invalid("g4_kv_create: empty cache shape");
        for (int l = 0; ring_rows && l < n_layers; ++l)
            if (ring_rows[l] < 0) return invalid("g4_kv_create: negative ring size");
        *out = nullptr;
        G4_HIP(hipSetDevice(ctx->device));
        auto *c = new g4_kv_cache();
        c->ctx = ctx;
        c->n_layers = n_layers;
        c->capacity = capacity;
        c->width.assign(widths, widths + n_layers);
        c->k.assign(n_layers, nullptr);
        c->v.assign(n_layers, nullptr);
        c->rows.assign(n_layers, 0);
        c->ring.assign(n_layers, 0);
        for (int l = 0; l < n_layers; ++l) {
            if (c->width[l] <= 0) continue;
            // A ring as long as the capacity saves nothing: keep the history.
            if (ring_rows && ring_rows[l] > 0 && ring_rows[l] < capacity) c->ring[l] = ring_rows[l];
            const int64_t stored = c->ring[l] > 0 ? 2 * c->ring[l] : capacity;
            const size_t bytes = (size_t)stored * c->width[l] * sizeof(float);
            hipError_t e = hipMalloc(&c->k[l], bytes);
            if (e == hipSuccess) e = hipMalloc(&c->v[l], bytes);
            if (e != hipSuccess) {
                g4_kv_destroy(c);
                return g4::hip_failed(e, "g4_kv_create");
            }
        }
        *out = c;
        return (int)G4_OK;
    });
}

int g4_kv_create(g4_ctx *ctx, int n_layers, const int64_t *widths, int64_t capacity,
                 g4_kv_cache **out) {
    return g4_kv_create_ring(ctx, n_layers, widths, capacity, nullptr, out);
}

int g4_kv_destroy(g4_kv_cache *c) {
    if (!c) return G4_OK;
    (void)hipDeviceSynchronize();
    for (size_t l = 0; l < c->k.size(); ++l) {
        if (c->k[l]) (void)hipFree(c->k[l]);
        if (c->v[l]) (void)hipFree(c->v[l]);
    }
    delete c;
    return G4_OK;
}

int g4_kv_append_rows(g4_kv_cache *c, int layer, const float *k, const float *v, int64_t n,
                      g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        if (!c) return invalid("g4_kv_append: null cache");
        if (layer < 0 || layer >= c->n_layers) return invalid("g4_kv_append: layer outside the cache");
        if (n < 0) return invalid("g4_kv_append: negative row count");
        if (c->width[layer] <= 0) return invalid("g4_kv_append: layer keeps no K/V");
        if (c->rows[layer] + n > c->capacity)
            return g4::set_error(G4_ERR_CONTEXT_TOO_LONG,
                                 "context length " + std::to_string(c->rows[layer] + n) +
                                     " exceeds configured max " + std::to_string(c->capacity),
                                 (uint64_t)(c->rows[layer] + n), (uint64_t)c->capacity);
        const int64_t w = c->width[layer];
        if (c->ring[layer] > 0) {
            // Only the last R of the n rows stay resident.
            const int64_t skip = std::max<int64_t>(0, n - c->ring[layer]);
            const int rc = ring_store(c, layer, k + skip * w, v + skip * w, c->rows[layer] + skip, n - skip,
                                      as_stream(stream));
            if (rc != G4_OK) return rc;
        } else {
            const size_t row_bytes = (size_t)w * sizeof(float);
            const size_t off = (size_t)c->rows[layer] * w;
            G4_HIP(hipMemcpyAsync(c->k[layer] + off, k, row_bytes * n, hipMemcpyDeviceToDevice, as_stream(stream)));
            G4_HIP(hipMemcpyAsync(c->v[layer] + off, v, row_bytes * n, hipMemcpyDeviceToDevice, as_stream(stream)));
        }
        c->rows[layer] += n;
        // context_memory.rs:44-47: appending to layer L makes layers 0..=L exist.
        if (layer + 1 > c->known_layers) c->known_layers = layer + 1;
        return (int)G4_OK;
    });
}

int g4_kv_append(g4_kv_cache *c, int layer, const float *k, const float *v, g4_stream stream) {
    return g4_kv_append_rows(c, layer, k, v, 1, stream);
}

namespace {

// view(layer, len)'s outcomes (context_memory.rs:53-69): an error, or OK
// with *absent set when the layer does not exist and len is 0 (an empty view).
int view_check(const g4_kv_cache *c, int layer, int64_t len, bool *absent) {
    *absent = false;
    if (layer >= c->known_layers) {
        if (len == 0) {
            *absent = true;
            return G4_OK;
        }
        return g4::set_error(G4_ERR_MISSING_LAYER, "layer " + std::to_string(layer) + " has no cached K/V",
                             (uint64_t)layer);
    }
    const int64_t have = layer < c->n_layers ? c->rows[layer] : 0;
    if (len > have)
        return g4::set_error(G4_ERR_CONTEXT_TOO_LONG,
                             "context length " + std::to_string(len) + " exceeds configured max " +
                                 std::to_string(have),
                             (uint64_t)len, (uint64_t)have);
    return G4_OK;
}

}  // namespace

int g4_kv_view(const g4_kv_cache *c, int layer, int64_t len, const float **k, const float **v,
               int64_t *row_stride) {
    g4::clear_error();
    if (!c || !k || !v) return invalid("g4_kv_view: null argument");
    if (layer < 0 || len < 0) return invalid("g4_kv_view: negative layer or length");
    bool absent = false;
    const int rc = view_check(c, layer, len, &absent);
    if (rc != G4_OK) return rc;
    if (absent || layer >= c->n_layers) {  // an empty view of a layer that keeps nothing
        *k = *v = nullptr;
        if (row_stride) *row_stride = 0;
        return G4_OK;
    }
    // A ring layer's rows are in position order from row 0 only until it wraps.
    if (c->ring[layer] > 0 && c->rows[layer] > c->ring[layer] && len > 0)
        return g4::set_error(G4_ERR_COMPUTE, "layer " + std::to_string(layer) + " keeps only its last " +
                                                 std::to_string(c->ring[layer]) +
                                                 " rows; view them with g4_kv_view_rows");
    *k = c->k[layer];
    *v = c->v[layer];
    if (row_stride) *row_stride = c->width[layer];
    return G4_OK;
}

int g4_kv_view_rows(const g4_kv_cache *c, int layer, int64_t begin, int64_t end, const float **k, const float **v,
                    int64_t *row_stride) {
    g4::clear_error();
    if (!c || !k || !v) return invalid("g4_kv_view_rows: null argument");
    if (layer < 0 || begin < 0 || end < begin) return invalid("g4_kv_view_rows: needs 0 <= begin <= end");
    bool absent = false;
    const int rc = view_check(c, layer, end, &absent);  // as view(layer, end)
    if (rc != G4_OK) return rc;
    if (absent || layer >= c->n_layers) {
        *k = *v = nullptr;
        if (row_stride) *row_stride = 0;
        return G4_OK;
    }
    const int64_t R = c->ring[layer];
    if (R > 0 && begin < end && begin < c->rows[layer] - R)
        return g4::set_error(G4_ERR_COMPUTE, "positions before " + std::to_string(c->rows[layer] - R) +
                                                 " have left layer " + std::to_string(layer) + "'s ring of " +
                                                 std::to_string(R) + " rows");
    const int64_t off = slot_of(c, layer, begin) * c->width[layer];
    *k = c->k[layer] + off;
    *v = c->v[layer] + off;
    if (row_stride) *row_stride = c->width[layer];
    return G4_OK;
}

int64_t g4_kv_len(const g4_kv_cache *c, int layer) {
    if (!c || layer < 0 || layer >= c->n_layers) return 0;
    return c->rows[layer];
}

void g4_kv_clear(g4_kv_cache *c) {
    if (!c) return;
    for (auto &r : c->rows) r = 0;
    c->known_layers = 0;
}

// ------------------------------------------------------------------ policies
int g4_layer_is_global(int n_layers, int layer) {
    return (layer + 1 == n_layers || layer % 5 == 4) ? 1 : 0;
}

int g4_kv_source_layer(int n_layers, int shared_kv_layers, int layer, int *source) {
    g4::clear_error();
    if (!source) return invalid("g4_kv_source_layer: null output");
    if (layer < 0 || layer >= n_layers)
        return g4::set_error(G4_ERR_COMPUTE, "layer " + std::to_string(layer) +
                                                 " must be within n_layers " + std::to_string(n_layers));
    if (shared_kv_layers < 0 || shared_kv_layers >= n_layers)
        return g4::set_error(G4_ERR_COMPUTE, std::to_string(shared_kv_layers) +
                                                 " KV-shared layers leave no layer of " +
                                                 std::to_string(n_layers) + " to own a cache");
    const int first_shared = n_layers - shared_kv_layers;
    if (layer < first_shared) {
        *source = layer;
        return G4_OK;
    }
    const int kind = g4_layer_is_global(n_layers, layer);
    for (int e = first_shared - 1; e >= 0; --e) {
        if (g4_layer_is_global(n_layers, e) == kind) {
            *source = e;
            return G4_OK;
        }
    }
    return g4::set_error(G4_ERR_COMPUTE, "KV-shared layer " + std::to_string(layer) +
                                             " has no earlier layer of the same attention kind");
}

void g4_windowed_len(int64_t seq_len, int64_t window, int64_t *begin, int64_t *end) {
    if (begin) *begin = seq_len > window ? seq_len - window : 0;
    if (end) *end = seq_len;
}

void g4_proportional_rope_freq_factors(int head_dim, float p, float *out) {
    if (!out || head_dim <= 0) return;
    const float r = (float)head_dim * p / 2.0f;
    const int64_t rotated = r > 0.0f ? (int64_t)r : 0;
    for (int pair = 0; pair < head_dim / 2; ++pair) out[pair] = pair < rotated ? 1.0f : 1e30f;
}

// -------------------------------------------------- fused input preparation
namespace {

int context_too_long(int64_t got, int64_t max) {
    return g4::set_error(G4_ERR_CONTEXT_TOO_LONG,
                         "context length " + std::to_string(got) + " exceeds configured max " + std::to_string(max),
                         (uint64_t)got, (uint64_t)max);
}

// The preparation's argument checks (model.rs:394-406), with the
// reference's messages for its own failures.
int prepare_checks(g4_ctx *ctx, const float *q, const float *k, const float *v, int64_t n_tokens, int64_t pos0,
                   int n_heads, int n_kv_heads, int head_dim, float eps, float base, const float *k_rows,
                   const float *v_rows, int64_t row_stride) {
    if (!ctx || !q) return invalid("g4_prepare_qkv: null argument");
    if (n_tokens < 0 || pos0 < 0) return invalid("g4_prepare_qkv: negative token count or position");
    if (n_heads <= 0 || head_dim <= 0 || (k && (n_kv_heads <= 0 || !v)))
        return invalid("g4_prepare_qkv: needs positive head counts and head width");
    if ((k_rows || v_rows) && (!k || !k_rows || !v_rows || row_stride < (int64_t)n_kv_heads * head_dim))
        return invalid("g4_prepare_qkv: cache rows need k, v and a row_stride of at least the row width");
    // ops.rs:46-48
    if (eps < 0.0f) return g4::set_error(G4_ERR_COMPUTE, "invalid RMS norm inputs");
    // ops.rs:142-149 with n_rot = head_dim (rope_heads, model.rs:301)
    if (head_dim % 2 != 0 || base <= 0.0f) return g4::set_error(G4_ERR_COMPUTE, "invalid RoPE inputs");
    return G4_OK;
}

// rope_neox's theta_scale, base.powf(-2.0 / n_rot), on the host's libm (ops.rs:151).
float theta_scale_of(float base, int head_dim) { return powf(base, -2.0f / (float)head_dim); }

// Validates and launches the fused preparation (model.rs:394-406).
int prepare(g4_ctx *ctx, float *q, float *k, float *v, int64_t n_tokens, int64_t pos0, int n_heads,
            int n_kv_heads, int head_dim, const float *q_w, const float *k_w, float eps, float base,
            const float *factors, float *k_rows, float *v_rows, int64_t row_stride, hipStream_t stream) {
    const int rc = prepare_checks(ctx, q, k, v, n_tokens, pos0, n_heads, n_kv_heads, head_dim, eps, base, k_rows,
                                  v_rows, row_stride);
    if (rc != G4_OK) return rc;
    g4::PrepareArgs a{};
    a.q = q;
    a.k = k;
    a.v = k ? v : nullptr;
    a.k_rows = k_rows;
    a.v_rows = v_rows;
    a.row_stride = row_stride;
    a.q_w = q_w;
    a.k_w = k_w;
    a.factors = factors;
    a.n_tokens = n_tokens;
    a.pos0 = pos0;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.head_dim = head_dim;
    a.eps = eps;
    a.theta_scale = theta_scale_of(base, head_dim);
    return g4::launch_prepare_qkv(a, stream);
}

// The layer's attention set-up shared by the decode and prefill drivers:
// kind, head width, RoPE base/divisors and the K/V source layer.
struct LayerPlan {
    bool global;
    int head_dim;
    float base;
    const float *factors;
    int source;
};

int plan_layer(const g4_hparams *hp, int layer, const float *rope_freqs, LayerPlan &pl) {
    pl.global = g4_layer_is_global(hp->n_layers, layer) != 0;
    pl.head_dim = pl.global ? hp->head_dim_global : hp->head_dim_local;
    pl.base = pl.global ? hp->global_rope_base : hp->local_rope_base;
    pl.factors = pl.global ? rope_freqs : nullptr;
    // model.rs:398
    return g4_kv_source_layer(hp->n_layers, hp->shared_kv_layers, layer, &pl.source);
}

// Reserves rows [rows, rows + n) of an owner layer's cache for a fused
// append; the row count moves only after the launch succeeded.
// In a ring layer the n rows go to slots [s, s + n) with s = position % R
// (contiguous: n <= R), and commit_rows copies them to their mirror slots.
int owner_rows(g4_kv_cache *c, int layer, int64_t row_width, int64_t n, float **k_rows, float **v_rows) {
    if (layer >= c->n_layers || c->width[layer] <= 0) return invalid("g4_kv_append: layer keeps no K/V");
    if (c->width[layer] != row_width)
        return invalid("g4_layer_attention: the layer's cache width differs from n_kv_heads*head_dim");
    if (c->rows[layer] + n > c->capacity) return context_too_long(c->rows[layer] + n, c->capacity);
    if (c->ring[layer] > 0 && n > c->ring[layer])
        return g4::set_error(G4_ERR_COMPUTE, std::to_string(n) + " tokens do not fit layer " + std::to_string(layer) +
                                                 "'s ring of " + std::to_string(c->ring[layer]) + " rows");
    const int64_t slot = slot_of(c, layer, c->rows[layer]);
    *k_rows = c->k[layer] + slot * row_width;
    *v_rows = c->v[layer] + slot * row_width;
    return G4_OK;
}

// The row count after an append of n rows.
void count_rows(g4_kv_cache *c, int layer, int64_t n) {
    c->rows[layer] += n;
    // context_memory.rs:44-47: appending to layer L makes layers 0..=L exist.
    if (layer + 1 > c->known_layers) c->known_layers = layer + 1;
}

// In a ring layer, the mirror copies of positions [p, p + n), written at
// their primary slots (after the launch that wrote them, on its stream).
int mirror_rows(g4_kv_cache *c, int layer, int64_t p, int64_t n, hipStream_t stream) {
    return c->ring[layer] > 0 ? ring_mirror(c, layer, slot_of(c, layer, p), n, stream) : (int)G4_OK;
}

int commit_rows(g4_kv_cache *c, int layer, int64_t n, hipStream_t stream) {
    const int rc = mirror_rows(c, layer, c->rows[layer], n, stream);
    if (rc != G4_OK) return rc;
    count_rows(c, layer, n);
    return G4_OK;
}

}  // namespace

int g4_prepare_qkv(g4_ctx *ctx, float *q, float *k, float *v, int64_t n_tokens, int64_t pos0, int n_heads,
                   int n_kv_heads, int head_dim, const float *q_norm_w, const float *k_norm_w, float eps,
                   float rope_base, const float *freq_factors, float *k_rows, float *v_rows, int64_t row_stride,
                   g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        return prepare(ctx, q, k, v, n_tokens, pos0, n_heads, n_kv_heads, head_dim, q_norm_w, k_norm_w, eps,
                       rope_base, freq_factors, k_rows, v_rows, row_stride, as_stream(stream));
    });
}

// --------------------------------------------------------- layer attention
namespace {

// The fused decode step over rows [0, n_rows) of (keys, values), whose last
// row is `position`; with k, that row is prepared and written to
// (k_row, v_row) rather than read.  Unsupported shapes: G4_ERR_COMPUTE.
int decode_step_fused(g4_ctx *ctx, const float *q, const float *k, const float *v, const float *q_w, const float *k_w,
                      float eps, float base, const float *factors, int64_t position, const float *keys,
                      const float *values, int64_t row_stride, int64_t n_rows, float *k_row, float *v_row,
                      int n_heads, int n_kv_heads, int head_dim, float scale, float *out, hipStream_t stream) {
    int rc = prepare_checks(ctx, q, k, v, 1, position, n_heads, n_kv_heads, head_dim, eps, base, k_row, v_row,
                            row_stride);
    if (rc != G4_OK) return rc;
    if (k && (!k_row || !v_row)) return invalid("fused decode step: the new row needs its cache row");
    if (!keys || !values || !out) return invalid("fused decode step: null argument");
    if (n_rows <= 0 || n_rows > position + 1) return invalid("fused decode step: needs 0 < n_rows <= position + 1");
    g4::DecodeArgs da{};
    da.B = 1;
    da.k = keys;
    da.v = values;
    da.row_stride = row_stride;
    da.kv_begin0 = 0;
    da.kv_end0 = n_rows;
    da.max_kv_len = n_rows;
    da.prefill_window = -1;
    da.n_heads = n_heads;
    da.n_kv_heads = n_kv_heads;
    da.head_dim = head_dim;
    da.scale = scale;
    da.out = out;
    if (!g4::layer_decode_fusable(da))
        return g4::set_error(G4_ERR_COMPUTE, "fused decode step: needs head_dim 256 or 512 and 8 query heads per KV head");
    g4::LayerPrepArgs lp{};
    lp.q = q;
    lp.k = k;
    lp.v = k ? v : nullptr;
    lp.q_w = q_w;
    lp.k_w = k_w;
    lp.factors = factors;
    lp.eps = eps;
    lp.position = position;
    // rope_neox's angle recurrence (ops.rs:151-160), as the preparation kernels run it.
    const float theta_scale = theta_scale_of(base, head_dim);
    float th = (float)position;
    for (int i = 0; i < head_dim / 2; ++i) {
        lp.angles[i] = th;
        th = th * theta_scale;
    }
    lp.k_row = k_row;
    lp.v_row = v_row;
    return g4::launch_layer_decode(ctx, da, lp, stream);
}

}  // namespace

int g4_decode_step_fused(g4_ctx *ctx, const float *q, const float *k, const float *v, const float *q_norm_w,
                         const float *k_norm_w, float eps, float rope_base, const float *freq_factors,
                         int64_t position, const float *k_cache, const float *v_cache, int64_t row_stride,
                         int64_t n_rows, float *k_row, float *v_row, int n_heads, int n_kv_heads, int head_dim,
                         float scale, float *out, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        return decode_step_fused(ctx, q, k, v, q_norm_w, k_norm_w, eps, rope_base, freq_factors, position, k_cache,
                                 v_cache, row_stride, n_rows, k_row, v_row, n_heads, n_kv_heads, head_dim, scale, out,
                                 as_stream(stream));
    });
}

int g4_layer_attention(g4_ctx *ctx, g4_kv_cache *cache, const g4_hparams *hp, int layer,
                       int64_t position, float *q, float *k, float *v, const float *q_norm_w,
                       const float *k_norm_w, const float *rope_freqs, float *out, int *source_out,
                       int64_t *begin_out, int64_t *end_out, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx || !cache || !hp) return invalid("g4_layer_attention: null argument");
        if (layer < 0 || layer >= hp->n_layers) return invalid("g4_layer_attention: layer outside n_layers");
        if (position < 0) return invalid("g4_layer_attention: negative position");
        LayerPlan pl;
        int rc = plan_layer(hp, layer, rope_freqs, pl);
        if (rc != G4_OK) return rc;
        const int head_dim = pl.head_dim;
        const int64_t row_width = (int64_t)hp->n_kv_heads * head_dim;
        const bool owner = pl.source == layer;
        // model.rs:407-408: view(source, position + 1), then the window's rows.
        int64_t begin = 0, end = position + 1;
        if (!pl.global) g4_windowed_len(position + 1, hp->sliding_window, &begin, &end);
        if (source_out) *source_out = pl.source;
        if (begin_out) *begin_out = begin;
        if (end_out) *end_out = end;
        g4::DecodeArgs da{};  // the fused step's shape, for the eligibility test
        da.B = 1;
        da.row_stride = row_width;
        da.kv_end0 = end - begin;
        da.prefill_window = -1;
        da.n_heads = hp->n_heads;
        da.n_kv_heads = hp->n_kv_heads;
        da.head_dim = head_dim;
        float *k_rows = nullptr, *v_rows = nullptr;
        // The append pushes the new row after the cached ones (row
        // rows_before, context_memory.rs:44-51) and the view takes the first
        // position + 1 rows: the new row is the view's last one only when
        // rows_before == position.  Otherwise (a cache longer or shorter than
        // the position) the two-step path below appends and views as the
        // reference does.
        const int64_t rows_before = layer < cache->n_layers ? cache->rows[layer] : 0;
        if (g4::layer_decode_fusable(da) && (!owner || rows_before == position)) {
            // One launch (plus the split merge): the decode kernel prepares q
            // and, on an owner layer, the new row, which it appends and
            // attends (model.rs:394-410).  q, k and v are left as given.
            rc = prepare_checks(ctx, q, owner ? k : nullptr, v, 1, position, hp->n_heads, hp->n_kv_heads, head_dim,
                                hp->rms_norm_eps, pl.base, nullptr, nullptr, row_width);
            if (rc != G4_OK) return rc;
            // The appended row is counted before the launch: the window's
            // view includes it.
            const int known_before = cache->known_layers;
            if (owner) {
                rc = owner_rows(cache, layer, row_width, 1, &k_rows, &v_rows);
                if (rc != G4_OK) return rc;
                count_rows(cache, layer, 1);
            }
            const float *keys = nullptr, *values = nullptr;
            int64_t stride = 0;
            rc = g4_kv_view_rows(cache, pl.source, begin, end, &keys, &values, &stride);
            if (rc == G4_OK && stride != row_width)
                rc = invalid("g4_layer_attention: source layer's row width differs from this layer's");
            if (rc != G4_OK) {
                // The reference appends, then fails at the view (model.rs:405-407):
                // the row is written and stays counted.
                if (owner) {
                    const int saved = rc;
                    const std::string msg = g4_last_error();
                    uint64_t fa = 0, fb = 0;
                    g4_last_error_fields(&fa, &fb);
                    rc = prepare(ctx, q, k, v, 1, position, hp->n_heads, hp->n_kv_heads, head_dim, q_norm_w, k_norm_w,
                                 hp->rms_norm_eps, pl.base, pl.factors, k_rows, v_rows, row_width, as_stream(stream));
                    if (rc == G4_OK) rc = mirror_rows(cache, layer, rows_before, 1, as_stream(stream));
                    if (rc != G4_OK) return rc;
                    return g4::set_error(saved, msg, fa, fb);
                }
                return rc;
            }
            // model.rs:409-410: q and k are RMS-normalised, so the scale is 1.0.
            rc = decode_step_fused(ctx, q, owner ? k : nullptr, v, q_norm_w, k_norm_w, hp->rms_norm_eps, pl.base,
                                   pl.factors, position, keys, values, stride, end - begin, k_rows, v_rows,
                                   hp->n_heads, hp->n_kv_heads, head_dim, 1.0f, out, as_stream(stream));
            if (rc != G4_OK) {  // a launch failure: the row was not written
                if (owner) {
                    cache->rows[layer] = rows_before;
                    cache->known_layers = known_before;
                }
                return rc;
            }
            return owner ? mirror_rows(cache, layer, rows_before, 1, as_stream(stream)) : (int)G4_OK;
        }
        // Other shapes: model.rs:394-406 in one preparation launch (q norm +
        // RoPE; on owner layers k/v norm, k RoPE and the append), then the
        // decode over the view.
        if (owner) {
            rc = owner_rows(cache, layer, row_width, 1, &k_rows, &v_rows);
            if (rc != G4_OK) return rc;
        }
        rc = prepare(ctx, q, owner ? k : nullptr, v, 1, position, hp->n_heads, hp->n_kv_heads, head_dim, q_norm_w,
                     k_norm_w, hp->rms_norm_eps, pl.base, pl.factors, k_rows, v_rows, row_width, as_stream(stream));
        if (rc != G4_OK) return rc;
        if (owner) {
            rc = commit_rows(cache, layer, 1, as_stream(stream));
            if (rc != G4_OK) return rc;
        }
        const float *keys = nullptr, *values = nullptr;
        int64_t stride = 0;
        rc = g4_kv_view_rows(cache, pl.source, begin, end, &keys, &values, &stride);
        if (rc != G4_OK) return rc;
        if (stride != row_width)
            return invalid("g4_layer_attention: source layer's row width differs from this layer's");
        return g4_attend_decode(ctx, q, keys, values, stride, 0, end - begin, hp->n_heads,
                                hp->n_kv_heads, head_dim, 1.0f, out, stream);
    });
}

int g4_layer_prefill(g4_ctx *ctx, g4_kv_cache *cache, const g4_hparams *hp, int layer, int64_t pos0,
                     int64_t n_tokens, float *q, float *k, float *v, const float *q_norm_w,
                     const float *k_norm_w, const float *rope_freqs, float *out, int *source_out,
                     g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx || !cache || !hp) return invalid("g4_layer_prefill: null argument");
        if (layer < 0 || layer >= hp->n_layers) return invalid("g4_layer_prefill: layer outside n_layers");
        if (pos0 < 0 || n_tokens < 0) return invalid("g4_layer_prefill: negative position or token count");
        LayerPlan pl;
        int rc = plan_layer(hp, layer, rope_freqs, pl);
        if (rc != G4_OK) return rc;
        if (source_out) *source_out = pl.source;
        if (n_tokens == 0) return (int)G4_OK;
        // LocalWindowPolicy with no window attends nothing (eng/mod.rs:10-12).
        if (!pl.global && hp->sliding_window <= 0)
            return g4::set_error(G4_ERR_COMPUTE, "softmax input is not finite");
        const int head_dim = pl.head_dim;
        const int64_t row_width = (int64_t)hp->n_kv_heads * head_dim;
        const bool owner = pl.source == layer;
        float *k_rows = nullptr, *v_rows = nullptr;
        if (owner) {
            // Token pos0 appends its row, then views pos0 + 1 rows
            // (model.rs:405-407): a cache shorter than pos0 fails there.
            const int64_t have = layer < cache->n_layers ? cache->rows[layer] : 0;
            if (have < pos0) return context_too_long(pos0 + 1, have + 1);
            rc = owner_rows(cache, layer, row_width, n_tokens, &k_rows, &v_rows);
            if (rc != G4_OK) return rc;
        }
        rc = prepare(ctx, q, owner ? k : nullptr, v, n_tokens, pos0, hp->n_heads, hp->n_kv_heads, head_dim,
                     q_norm_w, k_norm_w, hp->rms_norm_eps, pl.base, pl.factors, k_rows, v_rows, row_width,
                     as_stream(stream));
        if (rc != G4_OK) return rc;
        if (owner) {
            rc = commit_rows(cache, layer, n_tokens, as_stream(stream));
            if (rc != G4_OK) return rc;
        }
        // The last token's view bounds every earlier one's; the chunk reads
        // rows from its first query's window start on.
        const int64_t lo = (!pl.global && pos0 + 1 > hp->sliding_window) ? pos0 + 1 - hp->sliding_window : 0;
        const float *keys = nullptr, *values = nullptr;
        int64_t stride = 0;
        rc = g4_kv_view_rows(cache, pl.source, lo, pos0 + n_tokens, &keys, &values, &stride);
        if (rc != G4_OK) return rc;
        if (stride != row_width)
            return invalid("g4_layer_prefill: source layer's row width differs from this layer's");
        // Query i attends the rows a decode at position pos0 + i would
        // (model.rs:407-410, eng/mod.rs:10-36), scale 1.0.
        return attend_prefill_rows(ctx, q, keys, values, stride, pos0, n_tokens, pl.global ? 0 : hp->sliding_window,
                                   lo, hp->n_heads, hp->n_kv_heads, head_dim, 1.0f, out, stream);
    });
}

// ------------------------------------------------------------------ mat-vecs
namespace {

// matvec.rs:206-214 (check_shape) with the reference's message.
int check_weight_shape(const char *kind, int64_t len, int64_t rows, int64_t row_len) {
    if (len >= 0 && rows >= 0 && row_len >= 0 && (row_len == 0 || rows <= INT64_MAX / row_len) &&
        rows * row_len == len)
        return G4_OK;
    return g4::set_error(G4_ERR_COMPUTE, std::string(kind) + " weight has " + std::to_string(len) +
                                             " elements, expected " + std::to_string(rows) + " rows of " +
                                             std::to_string(row_len));
}

int q8_cols_error(const char *what, int64_t cols) {
    return g4::set_error(G4_ERR_COMPUTE, std::string("Q8_0 ") + what + " " + std::to_string(cols) +
                                             " is not a multiple of 32");
}

// The Q8_0-activation forms: matvec, softcap, geglu; with x (and no xs/xq)
// the activation is quantized as part of the call.
int q8_matvec(g4_ctx *ctx, g4::MatvecKind kind, const uint8_t *w, const uint8_t *w2, int64_t w_bytes, int64_t rows,
              int64_t cols, const float *xs, const int8_t *xq, float arg, float *out, g4_stream stream,
              const float *x = nullptr) {
    if (!ctx) return invalid("mat-vec: null context");
    if (cols < 0 || cols % 32 != 0) return q8_cols_error("activation length", cols);
    const int rc = check_weight_shape("Q8_0", w_bytes, rows, cols / 32 * 34);
    if (rc != G4_OK) return rc;
    g4::MatvecArgs a{};
    a.kind = kind;
    a.w = w;
    a.w2 = w2;
    a.rows = rows;
    a.cols = cols;
    a.xs = xs;
    a.xq = (const signed char *)xq;
    a.x = x;
    a.arg = arg;
    a.out = out;
    return g4::launch_matvec(ctx, a, as_stream(stream));
}

}  // namespace

int g4_project_q8_0(g4_ctx *ctx, const uint8_t *w, int64_t w_bytes, int64_t rows, int64_t cols, const float *x,
                    float *out, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        return q8_matvec(ctx, g4::MatvecKind::Q8, w, nullptr, w_bytes, rows, cols, nullptr, nullptr, 0.0f, out,
                         stream, x);
    });
}

int g4_gated_ffn_q8_0(g4_ctx *ctx, const uint8_t *gate, const uint8_t *up, int64_t w_bytes, int64_t rows,
                      int64_t cols, const float *x, int fp16_gelu, float *out, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        return q8_matvec(ctx, fp16_gelu ? g4::MatvecKind::Q8GegluFp16 : g4::MatvecKind::Q8Geglu, gate, up, w_bytes,
                         rows, cols, nullptr, nullptr, 0.0f, out, stream, x);
    });
}

int g4_logits_q8_0(g4_ctx *ctx, const uint8_t *w, int64_t w_bytes, int64_t rows, int64_t cols, const float *x,
                   float cap, float *out, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        return q8_matvec(ctx, g4::MatvecKind::Q8Softcap, w, nullptr, w_bytes, rows, cols, nullptr, nullptr, cap,
                         out, stream, x);
    });
}

int g4_quantize_q8_0(g4_ctx *ctx, const float *x, int64_t n, float *scales, int8_t *quants, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx) return invalid("g4_quantize_q8_0: null context");
        // matvec.rs:36-42
        if (n < 0 || n % 32 != 0) return q8_cols_error("activation length", n);
        return g4::launch_quantize_q8_0(x, n, scales, (signed char *)quants, as_stream(stream));
    });
}

int g4_matvec_q8_0(g4_ctx *ctx, const uint8_t *w, int64_t w_bytes, int64_t rows, int64_t cols,
                   const float *x_scales, const int8_t *x_quants, float *out, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        return q8_matvec(ctx, g4::MatvecKind::Q8, w, nullptr, w_bytes, rows, cols, x_scales, x_quants, 0.0f, out,
                         stream);
    });
}

int g4_matvec_q8_0_softcap(g4_ctx *ctx, const uint8_t *w, int64_t w_bytes, int64_t rows, int64_t cols,
                           const float *x_scales, const int8_t *x_quants, float cap, float *out, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        return q8_matvec(ctx, g4::MatvecKind::Q8Softcap, w, nullptr, w_bytes, rows, cols, x_scales, x_quants, cap,
                         out, stream);
    });
}

int g4_geglu_q8_0(g4_ctx *ctx, const uint8_t *gate, const uint8_t *up, int64_t w_bytes, int64_t rows, int64_t cols,
                  const float *x_scales, const int8_t *x_quants, int fp16_gelu, float *out, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        return q8_matvec(ctx, fp16_gelu ? g4::MatvecKind::Q8GegluFp16 : g4::MatvecKind::Q8Geglu, gate, up, w_bytes,
                         rows, cols, x_scales, x_quants, 0.0f, out, stream);
    });
}

int g4_matvec_q8_0_f32(g4_ctx *ctx, const uint8_t *w, int64_t w_bytes, int64_t rows, int64_t cols, const float *x,
                       int f64_sums, float *out, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx) return invalid("g4_matvec_q8_0_f32: null context");
        // matvec.rs:186-190
        if (cols < 0 || cols % 32 != 0) return q8_cols_error("row length", cols);
        const int rc = check_weight_shape("Q8_0", w_bytes, rows, cols / 32 * 34);
        if (rc != G4_OK) return rc;
        g4::MatvecArgs a{};
        a.kind = f64_sums ? g4::MatvecKind::Q8F64 : g4::MatvecKind::Q8F32;
        a.w = w;
        a.rows = rows;
        a.cols = cols;
        a.x = x;
        a.out = out;
        return g4::launch_matvec(ctx, a, as_stream(stream));
    });
}

int g4_matvec_bf16(g4_ctx *ctx, const uint16_t *w, int64_t w_len, int64_t rows, int64_t cols, const float *x,
                   float *out, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx) return invalid("g4_matvec_bf16: null context");
        const int rc = check_weight_shape("BF16", w_len, rows, cols);
        if (rc != G4_OK) return rc;
        g4::MatvecArgs a{};
        a.kind = g4::MatvecKind::Bf16;
        a.w = (const unsigned char *)w;
        a.rows = rows;
        a.cols = cols;
        a.x = x;
        a.out = out;
        return g4::launch_matvec(ctx, a, as_stream(stream));
    });
}

int g4_matvec_f32(g4_ctx *ctx, const float *w, int64_t w_len, int64_t rows, int64_t cols, const float *x, float *out,
                  g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx) return invalid("g4_matvec_f32: null context");
        const int rc = check_weight_shape("f32", w_len, rows, cols);
        if (rc != G4_OK) return rc;
        g4::MatvecArgs a{};
        a.kind = g4::MatvecKind::F32;
        a.w = (const unsigned char *)w;
        a.rows = rows;
        a.cols = cols;
        a.x = x;
        a.out = out;
        return g4::launch_matvec(ctx, a, as_stream(stream));
    });
}

// ------------------------------------------------------------- ComputePort
int g4_port_matmul(g4_ctx *ctx, const float *a, const float *b, int64_t m, int64_t n, int64_t k,
                   float *out, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx) return invalid("g4_port_matmul: null context");
        if (m < 0 || n < 0 || k < 0) return g4::set_error(G4_ERR_COMPUTE, "matmul dimensions overflow");
        return g4::launch_matmul(a, b, m, n, k, out, as_stream(stream));
    });
}

int g4_port_rms_norm(g4_ctx *ctx, const float *x, const float *weight, int64_t n, float eps,
                     float *out, g4_stream stream) {
    return g4_rms_norm_rows(ctx, x, 1, n, weight, eps, out, stream);
}

int g4_port_softmax(g4_ctx *ctx, const float *x, int64_t n, float *out, g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx) return invalid("g4_port_softmax: null context");
        if (n <= 0) return g4::set_error(G4_ERR_COMPUTE, "softmax requires a non-empty buffer");
        int rc = g4::launch_softmax(x, n, out, ctx->status_dev, as_stream(stream));
        if (rc != G4_OK) return rc;
        // ComputePort::softmax returns its error directly, so this call waits.
        return g4_check_status(ctx, stream);
    });
}

int g4_port_rope(g4_ctx *ctx, float *x, int64_t len, int64_t pos, float theta, int64_t dims,
                 g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx) return invalid("g4_port_rope: null context");
        if (dims <= 0 || dims % 2 != 0 || dims > len || theta <= 0.0f || pos < 0)
            return g4::set_error(G4_ERR_COMPUTE, "invalid RoPE inputs");
        if (dims > INT32_MAX - 1) return invalid("g4_port_rope: dims above 2^31 - 2 are not supported");
        // One row: values past dims are left alone, so the row is dims wide.
        return g4_rope_neox_rows(ctx, x, 1, 1, (int)dims, (int)dims, pos, theta, nullptr, 0, stream);
    });
}

int g4_port_add(g4_ctx *ctx, const float *a, const float *b, int64_t n, float *out,
                g4_stream stream) {
    return guarded([&] {
        g4::clear_error();
        if (!ctx) return invalid("g4_port_add: null context");
        if (n < 0) return g4::set_error(G4_ERR_COMPUTE, "add buffer lengths differ");
        return g4::launch_add(a, b, n, out, as_stream(stream));
    });
}

}  // extern "C"
