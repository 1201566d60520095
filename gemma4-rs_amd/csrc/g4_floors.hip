// Reference kernels for the floors the attention kernels are measured
// against (benchmark support, built as libg4floors.so; the attention
// library does not use them):
//  - an empty kernel: what a launch costs with no work in it;
//  - a streaming read: what HBM delivers to a kernel that only reads, with
//    the same 16-byte non-temporal loads the decode kernels use for V;
//  - a matrix-pipe rate: back-to-back v_mfma_f32_16x16x32_f16 (the split
//    prefill's instruction) and v_mfma_f32_16x16x4f32 on two independent
//    accumulators per wave, as many waves per SIMD as asked.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

__global__ void empty_kernel() {}

// Workgroup b sums its contiguous share of x's n4 16-byte vectors, four
// loads per thread in flight, and writes the sum to sink[b] (so that the
// loads are not removed).
__global__ __launch_bounds__(256) void read_kernel(const f32x4 *__restrict__ x, int64_t n4, float *sink) {
    const int64_t per = (n4 + gridDim.x - 1) / gridDim.x;
    const int64_t lo = (int64_t)blockIdx.x * per;
    const int64_t hi = lo + per < n4 ? lo + per : n4;
    float acc = 0.0f;
    for (int64_t i = lo + threadIdx.x; i < hi; i += 4 * 256) {
        f32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t j = i + (int64_t)u * 256;
            v[u] = j < hi ? __builtin_nontemporal_load(x + j) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) acc += (v[u][0] + v[u][1]) + (v[u][2] + v[u][3]);
    }
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    __shared__ float part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = (part[0] + part[1]) + (part[2] + part[3]);
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Each wave runs `iters` rounds of two independent MFMAs; lane l writes one
// float to sink[block * 256 + l] (so that the MFMAs are not removed).
template <bool F16>
__global__ __launch_bounds__(256) void mfma_kernel(float *sink, int iters) {
    const int l = threadIdx.x;
    f16x8 a, b;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        a[j] = (_Float16)(l * 0.001f + j);
        b[j] = (_Float16)(j * 0.5f);
    }
    const float fa = l * 0.001f, fb = 0.5f;
    f32x4 c0 = {0.0f, 0.0f, 0.0f, 0.0f}, c1 = c0;
    for (int it = 0; it < iters; ++it) {
        if constexpr (F16) {
            c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c1, 0, 0, 0);
        } else {
            c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(fa, fb, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(fb, fa, c1, 0, 0, 0);
        }
    }
    const f32x4 s = c0 + c1;
    sink[blockIdx.x * 256 + l] = (s[0] + s[1]) + (s[2] + s[3]);
}

}  // namespace

extern "C" {

// One launch of an empty kernel of grid x threads workgroups on stream.
int g4f_empty(int grid, int threads, void *stream) {
    if (grid <= 0 || threads <= 0 || threads > 1024) return 1;
    hipLaunchKernelGGL(empty_kernel, dim3((unsigned)grid), dim3((unsigned)threads), 0, (hipStream_t)stream);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// One streaming read of `bytes` (a multiple of 16) at x by grid workgroups
// of 256 threads; sink holds grid floats.
int g4f_read(const void *x, int64_t bytes, float *sink, int grid, void *stream) {
    if (!x || !sink || bytes < 0 || bytes % 16 != 0 || grid <= 0) return 1;
    hipLaunchKernelGGL(read_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, (const f32x4 *)x,
                       bytes / 16, sink);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// One launch of 2 * iters MFMAs per wave on grid workgroups of four waves
// (grid = 256 * waves per SIMD on MI355X's 1024 SIMDs); f16 selects
// v_mfma_f32_16x16x32_f16, else v_mfma_f32_16x16x4f32.  sink holds grid * 256
// floats.
int g4f_mfma(int f16, int grid, int iters, float *sink, void *stream) {
    if (!sink || grid <= 0 || iters <= 0) return 1;
    if (f16)
        hipLaunchKernelGGL(mfma_kernel<true>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, sink, iters);
    else
        hipLaunchKernelGGL(mfma_kernel<false>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, sink, iters);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

}  // extern "C"
