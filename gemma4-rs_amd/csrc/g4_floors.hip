// Reference kernels for the floors the attention kernels are measured
// against (benchmark support, built as libg4floors.so; the attention
// library does not use them):
//  - an empty kernel: what a launch costs with no work in it;
//  - a streaming read: what HBM delivers to a kernel that only reads, with
//    the same 16-byte non-temporal loads the decode kernels use for V.
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

}  // extern "C"
