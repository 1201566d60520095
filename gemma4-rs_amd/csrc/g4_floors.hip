// Reference kernels for the floors the attention kernels are measured
// against (benchmark support, built as libg4floors.so; the attention
// library does not use them):
//  - an empty kernel: what a launch costs with no work in it;
//  - a streaming read: what HBM delivers to a kernel that only reads, with
//    the same 16-byte non-temporal loads the decode kernels use for V;
//  - a matrix-pipe rate: back-to-back v_mfma_f32_16x16x32_f16 (the split
//    prefill's instruction) and v_mfma_f32_16x16x4f32 on two independent
//    accumulators per wave, as many waves per SIMD as asked;
//  - the matrix pipe fed from LDS: one 16-byte operand per lane read from
//    LDS per one or two MFMAs (16x16x32 or 32x32x16 f16), which bounds what
//    a kernel streaming its operands through LDS can keep busy;
//  - MFMA / VALU overlap: how much independent f32 FMA work runs beside the
//    16x16x32 f16 MFMAs, from another wave of the same SIMD or from the same
//    wave between its MFMAs.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

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

typedef float f32x16 __attribute__((ext_vector_type(16)));

// Matrix pipe fed from LDS: each wave reads one 16-byte A operand per lane
// (ds_read_b128, the wave's 1 KiB contiguous, so bank-conflict free) from a
// 32 KiB LDS array and feeds it to MPR MFMAs on four independent
// accumulators; MPR = 0 keeps one operand in registers (the pipe alone).
// BIG selects v_mfma_f32_32x32x16_f16 (32 cycles of matrix work per 1 KiB
// operand) over v_mfma_f32_16x16x32_f16 (16).  Eight operands per round.
template <bool BIG, int MPR>
__global__ __launch_bounds__(256) void lds_mfma_kernel(float *sink, int iters) {
    __shared__ f32x4 buf[2048];
    for (int i = threadIdx.x; i < 2048; i += 256) buf[i] = f32x4{i * 1e-3f, 1.0f, 0.5f, 0.25f};
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    f16x8 b;
#pragma unroll
    for (int j = 0; j < 8; ++j) b[j] = (_Float16)(j * 0.5f);
    f16x8 a0 = __builtin_bit_cast(f16x8, buf[lane]);
    typedef typename std::conditional<BIG, f32x16, f32x4>::type acc_t;
    acc_t c[4] = {};
    const int off = wave * 64 + lane;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const f16x8 a = MPR == 0 ? a0 : __builtin_bit_cast(f16x8, buf[(off + (u + 8 * it) * 256) & 2047]);
#pragma unroll
            for (int m = 0; m < (MPR == 0 ? 1 : MPR); ++m) {
                acc_t &cc = c[(u * (MPR == 0 ? 1 : MPR) + m) & 3];
                if constexpr (BIG)
                    cc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, cc, 0, 0, 0);
                else
                    cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, cc, 0, 0, 0);
            }
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int j = 0; j < (BIG ? 16 : 4); ++j) s += c[k][j];
    sink[blockIdx.x * 256 + threadIdx.x] = s;
}

// MFMA / VALU overlap on workgroups of eight waves (waves w and w + 4 share
// a SIMD), one workgroup per CU (the LDS array reserves most of a CU's LDS).
// A wave of MFMAs runs `iters` rounds of four independent MFMAs; a wave of
// FMAs `iters` rounds of sixteen FMAs on eight independent chains (nominally
// as many VALU cycles as the MFMAs' 64 matrix cycles); an interleaving wave
// K FMAs after each of its MFMAs.  MODE: 0 every wave MFMAs; 1 waves 0-3
// MFMAs, the rest idle; 2 waves 4-7 FMAs, the rest idle; 3 waves 0-3 MFMAs
// and waves 4-7 FMAs; 4 waves 0-3 interleave, the rest idle; 5 every wave
// interleaves.
template <int MODE, int K>
__global__ __launch_bounds__(512) void mix_kernel(float *sink, int iters, float fa, float fb) {
    __shared__ float pad[24 * 1024];
    const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
    if (threadIdx.x == 0) pad[0] = fa;
    f16x8 a, b;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        a[j] = (_Float16)(l * 0.001f + j);
        b[j] = (_Float16)(j * 0.5f);
    }
    f32x4 c0 = {0.0f, 0.0f, 0.0f, 0.0f}, c1 = c0, c2 = c0, c3 = c0;
    float x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = l * 0.01f + i;
    const bool first = wave < 4;
    const bool mfma = MODE == 0 || ((MODE == 1 || MODE == 3) && first);
    const bool fma = (MODE == 2 || MODE == 3) && !first;
    const bool mixed = MODE == 5 || (MODE == 4 && first);
    if (mfma) {
        for (int it = 0; it < iters; ++it) {
            c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c3, 0, 0, 0);
        }
    }
    if (fma) {
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int i = 0; i < 8; ++i) x[i] = __builtin_fmaf(x[i], fa, fb);
        }
    }
    if (mixed) {
        for (int it = 0; it < iters; ++it) {
            c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c0, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < K; ++i) x[i & 7] = __builtin_fmaf(x[i & 7], fa, fb);
            c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c1, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < K; ++i) x[(i + 2) & 7] = __builtin_fmaf(x[(i + 2) & 7], fa, fb);
            c2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c2, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < K; ++i) x[(i + 4) & 7] = __builtin_fmaf(x[(i + 4) & 7], fa, fb);
            c3 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c3, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < K; ++i) x[(i + 6) & 7] = __builtin_fmaf(x[(i + 6) & 7], fa, fb);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, K, 0);  // VALU
            }
        }
    }
    const f32x4 s = (c0 + c1) + (c2 + c3);
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) t += x[i];
    __syncthreads();
    sink[blockIdx.x * 512 + threadIdx.x] = (s[0] + s[1]) + (s[2] + s[3]) + t + pad[l];
}

template <int MODE, int K>
void launch_mix(int grid, int iters, float *sink, hipStream_t st) {
    hipLaunchKernelGGL((mix_kernel<MODE, K>), dim3((unsigned)grid), dim3(512), 0, st, sink, iters, 1.0001f, 0.5f);
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

// One launch of the LDS-fed matrix-pipe kernel: mode 0..5 = (16x16x32,
// MPR 0), (16x16x32, 1), (16x16x32, 2), (32x32x16, 0), (32x32x16, 1),
// (32x32x16, 2); grid workgroups of four waves, 8 * iters operand rounds
// per wave (8 * iters * max(MPR, 1) MFMAs).  sink holds grid * 256 floats.
int g4f_lds_mfma(int mode, int grid, int iters, float *sink, void *stream) {
    if (!sink || grid <= 0 || iters <= 0 || mode < 0 || mode > 5) return 1;
    hipStream_t st = (hipStream_t)stream;
    const dim3 g((unsigned)grid), b(256);
    switch (mode) {
        case 0: hipLaunchKernelGGL((lds_mfma_kernel<false, 0>), g, b, 0, st, sink, iters); break;
        case 1: hipLaunchKernelGGL((lds_mfma_kernel<false, 1>), g, b, 0, st, sink, iters); break;
        case 2: hipLaunchKernelGGL((lds_mfma_kernel<false, 2>), g, b, 0, st, sink, iters); break;
        case 3: hipLaunchKernelGGL((lds_mfma_kernel<true, 0>), g, b, 0, st, sink, iters); break;
        case 4: hipLaunchKernelGGL((lds_mfma_kernel<true, 1>), g, b, 0, st, sink, iters); break;
        default: hipLaunchKernelGGL((lds_mfma_kernel<true, 2>), g, b, 0, st, sink, iters); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// One launch of the MFMA / VALU overlap kernel in `mode` (0..5, see
// mix_kernel) with k (1, 2 or 4) FMAs per MFMA for the interleaving modes;
// grid workgroups of eight waves, one per CU.  sink holds grid * 512 floats.
int g4f_mix(int mode, int k, int grid, int iters, float *sink, void *stream) {
    if (!sink || grid <= 0 || iters <= 0 || mode < 0 || mode > 5 || (k != 1 && k != 2 && k != 4)) return 1;
    hipStream_t st = (hipStream_t)stream;
    switch (mode) {
        case 0: launch_mix<0, 1>(grid, iters, sink, st); break;
        case 1: launch_mix<1, 1>(grid, iters, sink, st); break;
        case 2: launch_mix<2, 1>(grid, iters, sink, st); break;
        case 3: launch_mix<3, 1>(grid, iters, sink, st); break;
        case 4:
            if (k == 1) launch_mix<4, 1>(grid, iters, sink, st);
            else if (k == 2) launch_mix<4, 2>(grid, iters, sink, st);
            else launch_mix<4, 4>(grid, iters, sink, st);
            break;
        default:
            if (k == 1) launch_mix<5, 1>(grid, iters, sink, st);
            else if (k == 2) launch_mix<5, 2>(grid, iters, sink, st);
            else launch_mix<5, 4>(grid, iters, sink, st);
            break;
    }
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

}  // extern "C"
