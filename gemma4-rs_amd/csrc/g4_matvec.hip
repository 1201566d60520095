// Mat-vecs over the GGUF weight formats the engine keeps (Q8_0, BF16, F32)
// and the activations fused into them (Gemma's GELU-gated FFN input, the
// logit soft-cap): crates/llm-backend-cpu/src/matvec.rs, ops.rs:79-103.
//
// Every kernel reproduces the reference's arithmetic exactly: the integer
// block dots are exact in any order, and every floating-point sum is taken
// in the reference's order -- a row's block products (Q8_0) or element
// products (BF16, F32, dequantized Q8_0) added one after another from -0.0,
// as Rust's `Iterator::sum` does.  Only tanh inside GELU and the soft-cap
// comes from the device's libm.
//
// Q8_0 with quantized activations (the engine's default numerics) is the
// HBM-bound hot path: a wavefront takes a run of rows, streams their bytes
// into LDS with 16-byte direct-to-LDS loads (rows of 34-byte blocks are
// 16-byte aligned when cols is a multiple of 256), and lane b then takes
// block b: its f16 scale and 32 int8 values against the activation's block b
// (held in the lane's registers for the whole kernel), 8 v_dot4 steps.  The
// block products go to a table in LDS that lane r then sums for row r in
// block order, so the run's sequential sums proceed side by side.  The
// other formats, which the engine uses only for small tensors or for its
// comparison numerics, give each lane one row and sum sequentially.

#include <algorithm>
#include <type_traits>

#include "g4_internal.h"

namespace g4 {
namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kQ8Values = 32;  // values per Q8_0 block
constexpr int kQ8Bytes = 34;   // f16 scale + 32 int8
// Buffer resource (V#) word 3 for raw buffers on gfx950.
constexpr int kBufferWord3 = 0x00020000;
constexpr int kVmcntZero = 0x0F70;  // s_waitcnt vmcnt(0), other counters untouched

// Cache-policy operand of a buffer load: NT, non-temporal.  Large matrices
// stream their weights with it (output head 84.6 -> 78.9 us); small ones,
// which stay latency-bound, were 0.6 us slower with it.
constexpr int kNonTemporal = 2;

// One 16-byte load per active lane from `rsrc` at byte offset voff, written
// straight to LDS at lds + 16 * lane (lds is the same for the whole
// wavefront); AUX is the cache policy.
template <int AUX>
__device__ inline void load_to_lds(__amdgpu_buffer_rsrc_t rsrc, u32x4 *lds, uint32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)lds, 16, voff, 0, 0, AUX);
#endif
}

__device__ inline float half_bits_to_float(unsigned bits) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(bits & 0xffffu));
}

// f16 rounding of an f32 value (half::f16::from_f32).  The empty asm makes
// x opaque: otherwise the compiler fuses a product that feeds the conversion
// into one mixed-precision fma (v_fma_mixlo_f16 a, b, 0), which rounds the
// exact product to f16 once -- where the reference rounds it to f32 first --
// and turns a -0 product into +0.
__device__ inline float round_to_half(float x) {
    asm volatile("" : "+v"(x));
    return (float)(_Float16)x;
}

// Rust's `f32 as i8`: saturating, NaN -> 0.
__device__ inline int saturate_i8(float v) {
    if (v != v) return 0;
    return (int)fminf(fmaxf(v, -128.0f), 127.0f);
}

// ops.rs:85-89, evaluated left to right as rustc does (no contraction).
__device__ inline float gelu_tanh(float x) {
#pragma clang fp contract(off)
    return 0.5f * x * (1.0f + tanhf(0.7978846f * x * (1.0f + 0.044715f * x * x)));
}

// ops.rs:95-103
__device__ inline float gelu_tanh_fp16_table(float x) {
    if (x <= -10.0f) return 0.0f;
    if (x >= 10.0f) return x;
    return round_to_half(gelu_tanh(round_to_half(x)));
}

// quantize_q8_0 (matvec.rs:35-53): 32 lanes per block; max |x| over the
// block (NaN ignored, as f32::max does), scale = max/127 kept as its f16
// rounding, values x * (1/scale) rounded half to even and saturated.
__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float *x, int64_t n, float *scales,
                                                            signed char *quants) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const float v = i < n ? x[i] : 0.0f;
    float m = fmaxf(0.0f, fabsf(v));
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 32));
    const float scale = m / 127.0f;
    const float inverse = scale == 0.0f ? 0.0f : 1.0f / scale;
    if (i >= n) return;
    if ((i & 31) == 0) scales[i >> 5] = round_to_half(scale);
    quants[i] = (signed char)saturate_i8(rintf(v * inverse));
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// One block of 32 activation values (block b of x, 16-byte aligned).
__device__ inline void load_block(const float *x, int b, f32x4 (&v)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = ((const f32x4 *)(x + kQ8Values * b))[j];
}

// One lane's quantize_q8_0 of a loaded block: the same arithmetic as
// quantize_q8_0_kernel, the 32 values packed 4 to a dword.
__device__ inline float quantize_values(const f32x4 (&v)[8], int (&q)[8]) {
#pragma clang fp contract(off)
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int k = 0; k < 4; ++k) m = fmaxf(m, fabsf(v[j][k]));
    const float scale = m / 127.0f;
    const float inverse = scale == 0.0f ? 0.0f : 1.0f / scale;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        unsigned packed = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) packed |= ((unsigned)saturate_i8(rintf(v[j][k] * inverse)) & 0xffu) << (8 * k);
        q[j] = (int)packed;
    }
    return round_to_half(scale);
}

__device__ inline float quantize_block(const float *x, int b, int (&q)[8]) {
    f32x4 v[8];
    load_block(x, b, v);
    return quantize_values(v, q);
}

// Epilogues of the Q8_0 row kernel.
enum Epilogue : int { kPlain = 0, kSoftcap = 1, kGeglu = 2, kGegluFp16 = 3 };

// W @ x for Q8_0 rows against a Q8_0 activation (matvec.rs:55-102).  A
// workgroup is one wavefront and takes `rb` consecutive rows (rb <= 64), staged into
// LDS `g` rows at a time with direct-to-LDS 16-byte loads.  For each staged
// row, lane b computes block b's product (NS = blocks per lane: b = lane +
// 64 s) into a row-major product table in LDS; once all rows are done, lane
// r sums row r's products in block order -- up to 64 independent sequential
// sums at once, each exactly the reference's.  kGeglu* read a second matrix
// (up) beside the first (gate).  Large matrices stage one row at a time in
// small workgroups, so that many are resident per CU (measured faster than
// double-buffering fewer of them); small ones stage all their rows at once.
template <int EPI, int NS, bool STREAM>
__global__ __launch_bounds__(64) void matvec_q8_0_kernel(const unsigned char *__restrict__ w,
                                                         const unsigned char *__restrict__ w2, int64_t rows,
                                                         int nb, const float *__restrict__ xs,
                                                         const int *__restrict__ xq, const float *__restrict__ xf,
                                                         float arg, int g, int rb, float *__restrict__ out) {
#pragma clang fp contract(off)
    extern __shared__ u32x4 lds[];
    constexpr int NM = EPI >= kGeglu ? 2 : 1;  // matrices read
    const int lane = threadIdx.x;
    const int row_len = nb * kQ8Bytes;  // bytes, a multiple of 16
    const int chunks = row_len >> 4;    // 16-byte chunks per row
    const int pstride = nb + 1;         // product table row stride (odd: no bank conflicts)
    u32x4 *stage = lds;                                  // [g][NM][chunks]
    float *prod = (float *)(lds + (size_t)g * NM * chunks);  // [NM][rb][pstride]

    const int64_t row0 = (int64_t)blockIdx.x * rb;
    const int n_rows = (int)min((int64_t)rb, rows - row0);  // >= 1: the grid covers the rows exactly
    // Stage rows r0 .. r0 + min(g, n_rows - r0) - 1 of each matrix.
    auto stage_rows = [&](int r0) {
        const int nr = min(g, n_rows - r0);
        for (int r = 0; r < nr; ++r)
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                    (void *)((m == 0 ? w : w2) + (row0 + r0 + r) * row_len), 0, row_len, kBufferWord3);
                u32x4 *dst = stage + (r * NM + m) * chunks;
                for (int k = 0; k * 64 < chunks; ++k)
                    if (k * 64 + lane < chunks)
                        load_to_lds<STREAM ? kNonTemporal : 0>(rs, dst + 64 * k, (uint32_t)(k * 64 + lane) * 16u);
            }
    };
    // The first rows' loads are in flight while the activation is read (and
    // quantized, when it comes as f32).  Small matrices quantize the f32
    // activation here: its loads go first, since load counters complete in
    // issue order and the quantization would otherwise wait for the rows
    // (q projection 4096 x 1536: 8.05 -> 7.52 us).  Large ones read a
    // quantized activation after their rows (the order measured faster).
    f32x4 xv[STREAM ? 1 : NS][8];
    if constexpr (!STREAM) {
        if (xf) {
#pragma unroll
            for (int s = 0; s < NS; ++s) load_block(xf, min(lane + 64 * s, nb - 1), xv[s]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    stage_rows(0);
    if constexpr (!STREAM) __builtin_amdgcn_sched_barrier(0);

    // This lane's activation blocks: 8 packed int8 dwords and the scale.
    int xqr[NS][8];
    float xsr[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const int b = lane + 64 * s;
#pragma unroll
        for (int j = 0; j < 8; ++j) xqr[s][j] = 0;
        xsr[s] = 0.0f;
        if (b < nb) {
            if (xf) {  // quantize_q8_0 of the f32 activation, here
                if constexpr (STREAM)
                    xsr[s] = quantize_block(xf, b, xqr[s]);
                else
                    xsr[s] = quantize_values(xv[s], xqr[s]);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) xqr[s][j] = xq[b * 8 + j];
                xsr[s] = xs[b];
            }
        }
    }

    for (int r0 = 0; r0 < n_rows; r0 += g) {
        const int nr = min(g, n_rows - r0);
        if (r0 > 0) stage_rows(r0);
        __builtin_amdgcn_s_waitcnt(kVmcntZero);
        __syncthreads();
        for (int r = 0; r < nr; ++r)
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const unsigned *rw = (const unsigned *)(stage + (r * NM + m) * chunks);
                float *pr = prod + ((size_t)m * rb + r0 + r) * pstride;
#pragma unroll
                for (int s = 0; s < NS; ++s) {
                    const int b = lane + 64 * s;
                    if (b < nb) {
                        // Block b starts at byte 34b: dword 17(b/2), offset 0
                        // (even b: scale in the low half, values from byte 2)
                        // or dword 17(b/2) + 8, offset 2 (odd b: scale in the
                        // high half, values dword-aligned after it).
                        const unsigned *d = rw + 17 * (b >> 1) + ((b & 1) ? 8 : 0);
                        unsigned raw[9];
#pragma unroll
                        for (int j = 0; j < 9; ++j) raw[j] = d[j];
                        int dot = 0;
                        float ws;
                        if (b & 1) {
                            ws = half_bits_to_float(raw[0] >> 16);
#pragma unroll
                            for (int j = 0; j < 8; ++j) dot = __builtin_amdgcn_sdot4((int)raw[j + 1], xqr[s][j], dot, false);
                        } else {
                            ws = half_bits_to_float(raw[0]);
#pragma unroll
                            for (int j = 0; j < 8; ++j)
                                dot = __builtin_amdgcn_sdot4((int)__builtin_amdgcn_alignbyte(raw[j + 1], raw[j], 2),
                                                             xqr[s][j], dot, false);
                        }
                        // matvec.rs:148: `dot as f32 * (w_scale * x_scale)`
                        pr[b] = (float)dot * (ws * xsr[s]);
                    }
                }
            }
        __syncthreads();  // the stage is refilled next; the products are complete
    }
    if (lane >= n_rows) return;
    // Lane r: row r's block products summed in block order.
    float acc[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const float *pr = prod + ((size_t)m * rb + lane) * pstride;
        float sum = -0.0f;
        for (int b = 0; b < nb; ++b) sum += pr[b];
        acc[m] = sum;
    }
    float v = acc[0];
    if constexpr (EPI == kSoftcap) v = tanhf(v * (1.0f / arg)) * arg;  // ops.rs:79-81
    if constexpr (EPI == kGeglu) v = gelu_tanh(acc[0]) * acc[NM - 1];
    if constexpr (EPI == kGegluFp16) v = gelu_tanh_fp16_table(acc[0]) * acc[NM - 1];
    out[row0 + lane] = v;
}

// Reads the 34-byte Q8_0 block at byte `off` of a row (2-byte aligned):
// its f16 scale and the 32 values packed 4 to a dword.
__device__ inline float load_q8_block(const unsigned short *row16, int64_t off, unsigned (&q)[8]) {
    const unsigned short *p = row16 + off / 2;
    const float scale = half_bits_to_float(p[0]);
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = (unsigned)p[1 + 2 * j] | ((unsigned)p[2 + 2 * j] << 16);
    return scale;
}

// Q8_0 against a Q8_0 activation, one lane per row (any cols multiple of 32):
// the same block products and order as matvec_q8_0_kernel.
template <int EPI>
__global__ __launch_bounds__(256) void matvec_q8_0_rowwise_kernel(const unsigned char *__restrict__ w,
                                                                  const unsigned char *__restrict__ w2,
                                                                  int64_t rows, int nb, const float *__restrict__ xs,
                                                                  const int *__restrict__ xq, float arg,
                                                                  float *__restrict__ out) {
#pragma clang fp contract(off)
    const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (row >= rows) return;
    constexpr int NM = EPI >= kGeglu ? 2 : 1;
    const int64_t row_len = (int64_t)nb * kQ8Bytes;
    float acc[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const unsigned short *r16 = (const unsigned short *)((m == 0 ? w : w2) + row * row_len);
        float sum = -0.0f;
        for (int b = 0; b < nb; ++b) {
            unsigned q[8];
            const float ws = load_q8_block(r16, (int64_t)b * kQ8Bytes, q);
            int dot = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) dot = __builtin_amdgcn_sdot4((int)q[j], xq[b * 8 + j], dot, false);
            sum += (float)dot * (ws * xs[b]);
        }
        acc[m] = sum;
    }
    float v = acc[0];
    if constexpr (EPI == kSoftcap) v = tanhf(v * (1.0f / arg)) * arg;
    if constexpr (EPI == kGeglu) v = gelu_tanh(acc[0]) * acc[NM - 1];
    if constexpr (EPI == kGegluFp16) v = gelu_tanh_fp16_table(acc[0]) * acc[NM - 1];
    out[row] = v;
}

// matvec_q8_0_f32 / matvec_q8_0_f64_sums (matvec.rs:104-122, 153-176): f32
// activations against dequantized blocks, one lane per row.  Per block the
// 32 products summed in order, times the scale; the blocks summed in order
// (F64: every sum in f64, one rounding at the end).
template <bool F64>
__global__ __launch_bounds__(256) void matvec_q8_0_f32_kernel(const unsigned char *__restrict__ w, int64_t rows,
                                                              int nb, const float *__restrict__ x,
                                                              float *__restrict__ out) {
#pragma clang fp contract(off)
    const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (row >= rows) return;
    const unsigned short *r16 = (const unsigned short *)(w + row * (int64_t)nb * kQ8Bytes);
    using T = typename std::conditional<F64, double, float>::type;
    T sum = (T)-0.0;
    for (int b = 0; b < nb; ++b) {
        unsigned q[8];
        const float scale = load_q8_block(r16, (int64_t)b * kQ8Bytes, q);
        T dot = (T)-0.0;
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int v = (int)(signed char)(q[j] >> (8 * k));
                dot += (T)v * (T)x[b * kQ8Values + 4 * j + k];
            }
        sum += dot * (T)scale;
    }
    out[row] = (float)sum;
}

// matvec.rs:196-204 (f32_to_bf16) and 192-194.
__device__ inline float round_to_bf16(float value) {
    const unsigned bits = __float_as_uint(value);
    unsigned h;
    if (value != value)
        h = (bits >> 16) | 64u;
    else
        h = (bits + (0x7fffu + ((bits >> 16) & 1u))) >> 16;
    return __uint_as_float(h << 16);
}

// matvec_bf16 (matvec.rs:124-130, 178-180): x rounded to bf16, one lane per
// row, one sequential f32 sum over the row.
__global__ __launch_bounds__(256) void matvec_bf16_kernel(const unsigned short *__restrict__ w, int64_t rows,
                                                          int64_t cols, const float *__restrict__ x,
                                                          float *__restrict__ out) {
#pragma clang fp contract(off)
    const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (row >= rows) return;
    const unsigned short *r = w + row * cols;
    float sum = -0.0f;
    for (int64_t i = 0; i < cols; ++i) sum += __uint_as_float((unsigned)r[i] << 16) * round_to_bf16(x[i]);
    out[row] = sum;
}

// matvec_f32 (matvec.rs:132-136, 182-184): one lane per row, sequential sum.
__global__ __launch_bounds__(256) void matvec_f32_kernel(const float *__restrict__ w, int64_t rows, int64_t cols,
                                                         const float *__restrict__ x, float *__restrict__ out) {
#pragma clang fp contract(off)
    const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (row >= rows) return;
    const float *r = w + row * cols;
    float sum = -0.0f;
    for (int64_t i = 0; i < cols; ++i) sum += r[i] * x[i];
    out[row] = sum;
}

template <int EPI, int NS, bool STREAM>
int launch_q8_rows(const MatvecArgs &a, int g, int rb, hipStream_t stream) {
    constexpr int NM = EPI >= kGeglu ? 2 : 1;
    const int nb = (int)(a.cols / kQ8Values);
    const size_t lds = (size_t)g * NM * (nb * kQ8Bytes) + (size_t)NM * rb * (nb + 1) * sizeof(float);
    const int64_t groups = (a.rows + rb - 1) / rb;
    hipLaunchKernelGGL((matvec_q8_0_kernel<EPI, NS, STREAM>), dim3((unsigned)groups), dim3(64), lds, stream, a.w, a.w2,
                       a.rows, nb, a.xs, (const int *)a.xq, a.xs ? nullptr : a.x, a.arg, g, rb, a.out);
    G4_HIP(hipGetLastError());
    return G4_OK;
}

template <int EPI>
int launch_q8(g4_ctx *ctx, MatvecArgs a, hipStream_t stream) {
    constexpr int NM = EPI >= kGeglu ? 2 : 1;
    const int num_cus = ctx->num_cus;
    const int64_t nb = a.cols / kQ8Values;
    // Rows start 16-byte aligned when cols is a multiple of 256 and the
    // matrices are (GGUF aligns tensor data to 32 bytes).
    const bool aligned = ((uintptr_t)a.w % 16 == 0) && (NM == 1 || (uintptr_t)a.w2 % 16 == 0) &&
                         (a.xs || (uintptr_t)a.x % 16 == 0);
    // An empty row (cols == 0) takes the row-wise kernel, which reads no
    // block: the staged kernel loads the activation's blocks before it tests
    // them against the block count.
    const bool fast = a.cols % 256 == 0 && nb > 0 && nb <= 256 && aligned;
    // Rows per workgroup: up to 16, the product table under 16 KB.
    const int64_t rb_max = std::min<int64_t>(16, std::max<int64_t>(1, 16384 / (NM * (nb + 1) * 4)));
    const bool large = a.rows >= rb_max * 8 * num_cus;
    if (!a.xs && (!fast || large)) {
        // An f32 activation for a kernel that reads a quantized one, or a
        // matrix large enough that its many workgroups would each quantize
        // it again: quantize_q8_0 into the context's workspace first.
        const size_t sbytes = ((size_t)nb * sizeof(float) + 255) / 256 * 256;
        const int rc = ensure_workspace(ctx, sbytes + (size_t)a.cols, stream);
        if (rc != G4_OK) return rc;
        a.xs = (const float *)ctx->ws.ptr;
        a.xq = (const signed char *)ctx->ws.ptr + sbytes;
        const int rq = launch_quantize_q8_0(a.x, a.cols, (float *)a.xs, (signed char *)a.xq, stream);
        if (rq != G4_OK) return rq;
    }
    if (fast) {
        // Large matrices: 8 rows per workgroup, staged two at a time, so
        // that the workgroups are small and many are resident per CU, each
        // with two rows in flight.  Output head (262,144 x 1536, quantize
        // included): 75.5 us with 16 rows staged one at a time, 71.5 with
        // 8 (or 4) staged two at a time, 87 with 8 staged eight at a time,
        // 97-142 with 64 rows per workgroup.  Small ones: a workgroup's rows
        // all in flight at once, and about eight workgroups per CU.
        int64_t rb, g;
        if (large) {
            rb = std::min<int64_t>(8, rb_max);
            g = std::min<int64_t>(2, rb);
        } else {
            rb = std::max<int64_t>(1, std::min<int64_t>(rb_max, a.rows / (8LL * num_cus)));
            g = rb;
        }
        const int ns = (int)((nb + 63) / 64);
        if (large) {
            switch (ns) {
            case 1: return launch_q8_rows<EPI, 1, true>(a, (int)g, (int)rb, stream);
            case 2: return launch_q8_rows<EPI, 2, true>(a, (int)g, (int)rb, stream);
            case 3: return launch_q8_rows<EPI, 3, true>(a, (int)g, (int)rb, stream);
            default: return launch_q8_rows<EPI, 4, true>(a, (int)g, (int)rb, stream);
            }
        }
        switch (ns) {
        case 1: return launch_q8_rows<EPI, 1, false>(a, (int)g, (int)rb, stream);
        case 2: return launch_q8_rows<EPI, 2, false>(a, (int)g, (int)rb, stream);
        case 3: return launch_q8_rows<EPI, 3, false>(a, (int)g, (int)rb, stream);
        default: return launch_q8_rows<EPI, 4, false>(a, (int)g, (int)rb, stream);
        }
    }
    hipLaunchKernelGGL((matvec_q8_0_rowwise_kernel<EPI>), dim3((unsigned)((a.rows + 255) / 256)), dim3(256), 0,
                       stream, a.w, a.w2, a.rows, (int)nb, a.xs, (const int *)a.xq, a.arg, a.out);
    G4_HIP(hipGetLastError());
    return G4_OK;
}

}  // namespace

int launch_quantize_q8_0(const float *x, int64_t n, float *scales, signed char *quants, hipStream_t stream) {
    if (n <= 0) return G4_OK;
    hipLaunchKernelGGL(quantize_q8_0_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, x, n, scales,
                       quants);
    G4_HIP(hipGetLastError());
    return G4_OK;
}

int launch_matvec(g4_ctx *ctx, const MatvecArgs &a, hipStream_t stream) {
    if (a.rows <= 0) return G4_OK;
    const unsigned grid = (unsigned)((a.rows + 255) / 256);
    switch (a.kind) {
    case MatvecKind::Q8: return launch_q8<kPlain>(ctx, a, stream);
    case MatvecKind::Q8Softcap: return launch_q8<kSoftcap>(ctx, a, stream);
    case MatvecKind::Q8Geglu: return launch_q8<kGeglu>(ctx, a, stream);
    case MatvecKind::Q8GegluFp16: return launch_q8<kGegluFp16>(ctx, a, stream);
    case MatvecKind::Q8F32:
        hipLaunchKernelGGL(matvec_q8_0_f32_kernel<false>, dim3(grid), dim3(256), 0, stream, a.w, a.rows,
                           (int)(a.cols / kQ8Values), a.x, a.out);
        break;
    case MatvecKind::Q8F64:
        hipLaunchKernelGGL(matvec_q8_0_f32_kernel<true>, dim3(grid), dim3(256), 0, stream, a.w, a.rows,
                           (int)(a.cols / kQ8Values), a.x, a.out);
        break;
    case MatvecKind::Bf16:
        hipLaunchKernelGGL(matvec_bf16_kernel, dim3(grid), dim3(256), 0, stream, (const unsigned short *)a.w, a.rows,
                           a.cols, a.x, a.out);
        break;
    case MatvecKind::F32:
        hipLaunchKernelGGL(matvec_f32_kernel, dim3(grid), dim3(256), 0, stream, (const float *)a.w, a.rows, a.cols,
                           a.x, a.out);
        break;
    }
    G4_HIP(hipGetLastError());
    return G4_OK;
}

}  // namespace g4
