// Attention input preparation (per-head RMS norm, NEOX RoPE) and the
// ComputePort method set on the device.  Citations: crates/llm-backend-cpu/src/ops.rs.

#include <algorithm>

#include "g4_internal.h"
#include "g4_prep.h"

namespace g4 {
namespace {

// rms_norm (ops.rs:45-56) on rows of `width` floats, one wavefront per row.
// The mean of squares is accumulated in f64 from f32-rounded squares, as the
// reference does; the f64 tree sum differs from the sequential one only in
// bits far below the f32 rounding of the mean.
__global__ __launch_bounds__(256) void rms_norm_rows_kernel(const float *x, int64_t n_rows,
                                                            int64_t width, const float *w,
                                                            float eps, float *out) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n_rows) return;
    const float *xr = x + row * width;
    double sum = 0.0;
    for (int64_t i = lane; i < width; i += 64) {
        const float v = xr[i];
        const float sq = v * v;
        sum += (double)sq;
    }
    sum = wave_sum_f64(sum);
    const float mean = (float)(sum / (double)width);
    // 1 / sqrt(mean + eps) with the f32 rounding of each step: sqrt and the
    // division are done in f64 and rounded once to f32, which for these two
    // operations equals the correctly rounded f32 result (53 >= 2*24 + 2).
    const float root = (float)sqrt((double)(mean + eps));
    const float scale = (float)(1.0 / (double)root);
    float *orow = out + row * width;
    for (int64_t i = lane; i < width; i += 64) {
        const float v = xr[i] * scale;
        orow[i] = w ? v * w[i] : v;
    }
}

// rope_neox (ops.rs:134-162) on every head of one token per workgroup.  The
// angle of pair i is theta_i / factor_i with theta_0 = position and
// theta_{i+1} = theta_i * theta_scale in f32 -- a sequential recurrence, so
// one lane builds the table and the workgroup applies it.  The table goes
// through LDS kRopeChunk pairs at a time (the recurrence carried from one
// chunk to the next), so any rotation width fits.
constexpr int kRopeChunk = 4096;

__global__ __launch_bounds__(256) void rope_rows_kernel(float *x, int n_heads, int head_dim,
                                                        int n_rot, int64_t pos0,
                                                        float theta_scale,
                                                        const float *factors) {
#pragma clang fp contract(off)
    __shared__ float theta[kRopeChunk];
    __shared__ float carry;
    const int half = n_rot / 2;
    const int64_t token = blockIdx.x;
    float *xt = x + token * (int64_t)n_heads * head_dim;
    if (threadIdx.x == 0) carry = (float)(pos0 + token);
    for (int c0 = 0; c0 < half; c0 += kRopeChunk) {
        const int len = min(kRopeChunk, half - c0);
        __syncthreads();  // the previous chunk's readers are done with theta
        if (threadIdx.x == 0) {
            float t = carry;
            for (int i = 0; i < len; ++i) {
                theta[i] = t;
                t = t * theta_scale;
            }
            carry = t;
        }
        __syncthreads();
        for (int64_t e = threadIdx.x; e < (int64_t)n_heads * len; e += blockDim.x) {
            const int h = (int)(e / len), j = (int)(e % len), i = c0 + j;
            const float factor = factors ? factors[i] : 1.0f;
            const float angle = theta[j] / factor;
            float sn, cs;
            sincosf(angle, &sn, &cs);
            float *xh = xt + (int64_t)h * head_dim;
            const float a = xh[i], b = xh[i + half];
            xh[i] = a * cs - b * sn;
            xh[i + half] = a * sn + b * cs;
        }
    }
}

// The attention inputs of one layer step, fused (model.rs:394-406): for each
// token t at position pos0 + t, every q head gets norm_heads(attn_q_norm)
// then rope_heads; on owner layers every k head gets norm_heads(attn_k_norm)
// then rope_heads and every v head norm_heads(None).  Results go back in
// place and, when cache rows are given, to row t of the K and V caches (the
// `append` of model.rs:405).  One workgroup per token: the angle table of
// the token's position is built once in LDS and serves its q and k heads;
// each wavefront normalises one head at a time, stages it in LDS, then
// rotates its NEOX pairs.  The arithmetic is that of rms_norm_rows_kernel
// and rope_rows_kernel, operation for operation.  This form serves any head
// width up to 1024; prepare_heads_kernel below serves the common ones.
constexpr int kPrepWaves = 4;
constexpr int kPrepMaxDim = 1024;

__global__ __launch_bounds__(64 * kPrepWaves) void prepare_qkv_kernel(PrepareArgs a) {
#pragma clang fp contract(off)
    __shared__ float theta[kPrepMaxDim / 2];
    __shared__ float stage[kPrepWaves][kPrepMaxDim];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int d = a.head_dim, half = d / 2;
    const int64_t t = blockIdx.x;
    if (threadIdx.x == 0) {
        float th = (float)(a.pos0 + t);
        for (int i = 0; i < half; ++i) {
            theta[i] = th;
            th = th * a.theta_scale;
        }
    }
    __syncthreads();
    const int n_k = a.k ? a.n_kv_heads : 0;
    const int rows = a.n_heads + 2 * n_k;
    for (int r0 = 0; r0 < rows; r0 += kPrepWaves) {
        const int r = r0 + wave;
        const bool active = r < rows;
        // Row r: q heads, then k heads, then v heads.
        float *x = nullptr, *cache = nullptr;
        const float *w = nullptr;
        bool rope = true;
        if (r < a.n_heads) {
            x = a.q + (t * a.n_heads + r) * (int64_t)d;
            w = a.q_w;
        } else if (r < a.n_heads + n_k) {
            const int h = r - a.n_heads;
            x = a.k + (t * a.n_kv_heads + h) * (int64_t)d;
            w = a.k_w;
            if (a.k_rows) cache = a.k_rows + t * a.row_stride + (int64_t)h * d;
        } else if (active) {
            const int h = r - a.n_heads - n_k;
            x = a.v + (t * a.n_kv_heads + h) * (int64_t)d;
            rope = false;
            if (a.v_rows) cache = a.v_rows + t * a.row_stride + (int64_t)h * d;
        }
        float scale = 0.0f;
        if (active) {
            double sum = 0.0;
            for (int i = lane; i < d; i += 64) {
                const float xv = x[i];
                const float sq = xv * xv;
                sum += (double)sq;
            }
            sum = wave_sum_f64(sum);
            const float mean = (float)(sum / (double)d);
            const float root = (float)sqrt((double)(mean + a.eps));
            scale = (float)(1.0 / (double)root);
            for (int i = lane; i < d; i += 64) {
                float y = x[i] * scale;
                if (w) y = y * w[i];
                if (rope) {
                    stage[wave][i] = y;
                } else {
                    x[i] = y;
                    if (cache) cache[i] = y;
                }
            }
        }
        __syncthreads();
        if (active && rope) {
            for (int i = lane; i < half; i += 64) {
                const float factor = a.factors ? a.factors[i] : 1.0f;
                const float angle = theta[i] / factor;
                float sn, cs;
                sincosf(angle, &sn, &cs);
                const float p = stage[wave][i], q = stage[wave][i + half];
                const float lo = p * cs - q * sn;
                const float hi = p * sn + q * cs;
                x[i] = lo;
                x[i + half] = hi;
                if (cache) {
                    cache[i] = lo;
                    cache[i + half] = hi;
                }
            }
        }
        __syncthreads();
    }
}

// The same preparation for head widths D that are multiples of 128: lane l
// holds elements l + 64m of its head in registers, so NEOX partners (i,
// i + D/2) sit in the same lane and a head needs one load, one reduction and
// one store.  One wavefront per head row (up to 16 per workgroup, grid.y
// covers more), all of a token's rows loaded at once; wave 0 builds the
// angle table (the reference's sequential recurrence) while the loads are
// in flight.
constexpr int kPrepMaxRowsPerGroup = 16;

template <int D>
__global__ __launch_bounds__(64 * kPrepMaxRowsPerGroup) void prepare_heads_kernel(PrepareArgs a) {
#pragma clang fp contract(off)
    constexpr int HALF = D / 2;
    __shared__ float theta[HALF];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t t = blockIdx.x;
    const int n_k = a.k ? a.n_kv_heads : 0;
    const int rows = a.n_heads + 2 * n_k;
    const int r = blockIdx.y * kPrepMaxRowsPerGroup + wave;
    const bool active = r < rows;
    float *x = nullptr, *cache = nullptr;
    const float *w = nullptr;
    bool rope = true;
    if (r < a.n_heads) {
        x = a.q + (t * a.n_heads + r) * (int64_t)D;
        w = a.q_w;
    } else if (r < a.n_heads + n_k) {
        const int h = r - a.n_heads;
        x = a.k + (t * a.n_kv_heads + h) * (int64_t)D;
        w = a.k_w;
        if (a.k_rows) cache = a.k_rows + t * a.row_stride + (int64_t)h * D;
    } else if (active) {
        const int h = r - a.n_heads - n_k;
        x = a.v + (t * a.n_kv_heads + h) * (int64_t)D;
        w = nullptr;
        rope = false;
        if (a.v_rows) cache = a.v_rows + t * a.row_stride + (int64_t)h * D;
    }
    // The RoPE table (sine and cosine of each pair's angle) is built once per
    // workgroup and shared by its q and k heads; the divisors are loaded with
    // the rows.
    __shared__ float rcs[HALF], rsn[HALF];
    constexpr int TPT = HALF / 64 > 0 ? HALF / 64 : 1;  // table entries per thread, at most
    float fac[TPT];
#pragma unroll
    for (int k = 0; k < TPT; ++k) {
        const int i = threadIdx.x + k * blockDim.x;
        fac[k] = (i < HALF && a.factors) ? a.factors[i] : 1.0f;
    }
    PrepRow<D> row;
    if (active) prep_load<D>(row, lane, x, w);
    if (threadIdx.x == 0) {
        // The sequential chain is the workgroup's critical path: its wave
        // issues ahead of the others on its SIMD meanwhile (2048-token
        // chunk: 13.6 -> 13.1 us at d=256, 20.3 -> 19.7 us at d=512).
        __builtin_amdgcn_s_setprio(3);
        prep_angles(theta, HALF, a.pos0 + t, a.theta_scale);
        __builtin_amdgcn_s_setprio(0);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < TPT; ++k) {
        const int i = threadIdx.x + k * blockDim.x;
        if (i < HALF) prep_rope_table(rcs, rsn, i, theta[i], fac[k]);
    }
    if (active) prep_norm<D>(row, w != nullptr, a.eps);
    __syncthreads();
    if (!active) return;
    if (rope) prep_rope_tab<D>(row, lane, rcs, rsn);
    prep_store<D>(row, lane, x);
    if (cache) prep_store<D>(row, lane, cache);
}

// matmul_f32 (ops.rs:9-39): row-major [m,k] x [k,n], sequential inner sum of
// rounded products, as the reference's triple loop.
__global__ void matmul_kernel(const float *a, const float *b, int64_t m, int64_t n, int64_t k,
                              float *out) {
#pragma clang fp contract(off)
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= m * n) return;
    const int64_t row = idx / n, col = idx % n;
    float acc = 0.0f;
    for (int64_t i = 0; i < k; ++i) acc += a[row * k + i] * b[i * n + col];
    out[idx] = acc;
}

// Total order of f32::total_cmp as a signed key.
__device__ inline int total_key(float x) {
    int bits = __float_as_int(x);
    return bits ^ (int)(((unsigned)(bits >> 31)) >> 1);
}

// softmax_f32 (ops.rs:105-127) of one vector in one workgroup.
__global__ __launch_bounds__(256) void softmax_kernel(const float *x, int64_t n, float *out,
                                                      unsigned *status) {
    __shared__ int kmax[256];
    __shared__ float red[256];
    const int tid = threadIdx.x;
    int best = INT_MIN;
    for (int64_t i = tid; i < n; i += 256) best = max(best, total_key(x[i]));
    kmax[tid] = best;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if (tid < off) kmax[tid] = max(kmax[tid], kmax[tid + off]);
        __syncthreads();
    }
    const int kb = kmax[0];
    const float mx = __int_as_float(kb ^ (int)(((unsigned)(kb >> 31)) >> 1));
    float s = 0.0f;
    for (int64_t i = tid; i < n; i += 256) {
        const float e = expf(x[i] - mx);
        out[i] = e;
        s += e;
    }
    red[tid] = s;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if (tid < off) red[tid] = red[tid] + red[tid + off];
        __syncthreads();
    }
    const float sum = red[0];
    if (!isfinite(sum) || sum == 0.0f) {
        if (tid == 0) atomicOr(status, kStatusNonFinite);
        return;
    }
    for (int64_t i = tid; i < n; i += 256) out[i] = out[i] / sum;
}

__global__ void add_kernel(const float *a, const float *b, int64_t n, float *out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

}  // namespace

int launch_rms_norm_rows(const float *x, int64_t n_rows, int64_t width, const float *w, float eps,
                         float *out, hipStream_t stream) {
    if (n_rows <= 0) return G4_OK;
    hipLaunchKernelGGL(rms_norm_rows_kernel, dim3((unsigned)((n_rows + 3) / 4)), dim3(256), 0,
                       stream, x, n_rows, width, w, eps, out);
    G4_HIP(hipGetLastError());
    return G4_OK;
}

int launch_rope_rows(float *x, int64_t n_tokens, int n_heads, int head_dim, int n_rot,
                     int64_t pos0, float theta_scale, const float *factors, hipStream_t stream) {
    if (n_tokens <= 0) return G4_OK;
    hipLaunchKernelGGL(rope_rows_kernel, dim3((unsigned)n_tokens), dim3(256), 0, stream, x, n_heads,
                       head_dim, n_rot, pos0, theta_scale, factors);
    G4_HIP(hipGetLastError());
    return G4_OK;
}

int launch_prepare_qkv(const PrepareArgs &a, hipStream_t stream) {
    if (a.n_tokens <= 0) return G4_OK;
    if (a.head_dim > kPrepMaxDim)
        return set_error(G4_ERR_COMPUTE, "head_dim above 1024 is not supported");
    const int rows = a.n_heads + (a.k ? 2 * a.n_kv_heads : 0);
    const dim3 fgrid((unsigned)a.n_tokens, (unsigned)((rows + kPrepMaxRowsPerGroup - 1) / kPrepMaxRowsPerGroup));
    const dim3 fblock(64 * (unsigned)std::min(rows, kPrepMaxRowsPerGroup));
    switch (a.head_dim) {
    case 128: hipLaunchKernelGGL(prepare_heads_kernel<128>, fgrid, fblock, 0, stream, a); break;
    case 256: hipLaunchKernelGGL(prepare_heads_kernel<256>, fgrid, fblock, 0, stream, a); break;
    case 512: hipLaunchKernelGGL(prepare_heads_kernel<512>, fgrid, fblock, 0, stream, a); break;
    case 1024: hipLaunchKernelGGL(prepare_heads_kernel<1024>, fgrid, fblock, 0, stream, a); break;
    default:
        hipLaunchKernelGGL(prepare_qkv_kernel, dim3((unsigned)a.n_tokens), dim3(64 * kPrepWaves), 0, stream, a);
    }
    G4_HIP(hipGetLastError());
    return G4_OK;
}

int launch_matmul(const float *a, const float *b, int64_t m, int64_t n, int64_t k, float *out,
                  hipStream_t stream) {
    const int64_t total = m * n;
    if (total <= 0) return G4_OK;
    hipLaunchKernelGGL(matmul_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                       a, b, m, n, k, out);
    G4_HIP(hipGetLastError());
    return G4_OK;
}

int launch_softmax(const float *x, int64_t n, float *out, unsigned *status, hipStream_t stream) {
    hipLaunchKernelGGL(softmax_kernel, dim3(1), dim3(256), 0, stream, x, n, out, status);
    G4_HIP(hipGetLastError());
    return G4_OK;
}

int launch_add(const float *a, const float *b, int64_t n, float *out, hipStream_t stream) {
    if (n <= 0) return G4_OK;
    hipLaunchKernelGGL(add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a, b,
                       n, out);
    G4_HIP(hipGetLastError());
    return G4_OK;
}

}  // namespace g4
