// One head row's attention input preparation by one wavefront: rms_norm
// with an optional weight, then NEOX RoPE (crates/llm-backend-cpu/src/ops.rs:
// 45-56, 134-162; norm_heads / rope_heads, crates/llm-gemma4/src/impl_/
// model.rs:283-304).  Lane l holds elements l + 64m (m < D/64) of the row, so
// NEOX partners i and i + D/2 sit in the same lane.  The standalone
// preparation kernel and the decode kernel's fused prologue both use these,
// so they produce the same bits.
#ifndef G4_PREP_H
#define G4_PREP_H

#include <hip/hip_runtime.h>

namespace g4 {

template <int D>
struct PrepRow {
    static constexpr int E = D / 64;   // elements per lane
    static constexpr int PE = E / 2;   // NEOX pairs per lane
    static constexpr int HALF = D / 2;
    float x[E], w[E], f[PE], a[PE];  // row, weight, RoPE divisors, angles theta_i
};

// The angles theta_i = pos * theta_scale^i of rope_neox, by the reference's
// sequential recurrence (one thread; theta[HALF] in LDS).
__device__ inline void prep_angles(float *theta, int half, int64_t pos, float theta_scale) {
#pragma clang fp contract(off)
    float th = (float)pos;
    for (int i = 0; i < half; ++i) {
        theta[i] = th;
        th = th * theta_scale;
    }
}

// Loads row x, its weight w (or none) and the RoPE divisors (or 1).
template <int D>
__device__ __forceinline__ void prep_load(PrepRow<D> &r, int lane, const float *x, const float *w,
                                          const float *factors, bool rope) {
#pragma unroll
    for (int m = 0; m < PrepRow<D>::E; ++m) r.x[m] = x[lane + 64 * m];
    if (w) {
#pragma unroll
        for (int m = 0; m < PrepRow<D>::E; ++m) r.w[m] = w[lane + 64 * m];
    }
    if (rope) {
#pragma unroll
        for (int m = 0; m < PrepRow<D>::PE; ++m) r.f[m] = factors ? factors[lane + 64 * m] : 1.0f;
    }
}

// This lane's angles theta_{lane + 64m} from a table of D/2 (built by
// prep_angles, or by the same recurrence on the host).
template <int D>
__device__ __forceinline__ void prep_load_angles(PrepRow<D> &r, int lane, const float *theta) {
#pragma unroll
    for (int m = 0; m < PrepRow<D>::PE; ++m) r.a[m] = theta[lane + 64 * m];
}

// rms_norm (f64 mean of squares, ops.rs:45-56) times the weight, then RoPE
// with the loaded angles, in the row's registers.
template <int D>
__device__ __forceinline__ void prep_compute(PrepRow<D> &r, bool has_w, bool rope, float eps) {
#pragma clang fp contract(off)
    constexpr int E = PrepRow<D>::E, PE = PrepRow<D>::PE;
    double sum = 0.0;
#pragma unroll
    for (int m = 0; m < E; ++m) {
        const float sq = r.x[m] * r.x[m];
        sum += (double)sq;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    const float mean = (float)(sum / (double)D);
    const float root = (float)sqrt((double)(mean + eps));
    const float scale = (float)(1.0 / (double)root);
#pragma unroll
    for (int m = 0; m < E; ++m) {
        r.x[m] = r.x[m] * scale;
        if (has_w) r.x[m] = r.x[m] * r.w[m];
    }
    if (rope) {
#pragma unroll
        for (int m = 0; m < PE; ++m) {
            const float angle = r.a[m] / r.f[m];
            float sn, cs;
            sincosf(angle, &sn, &cs);
            const float p = r.x[m], q = r.x[m + PE];
            r.x[m] = p * cs - q * sn;
            r.x[m + PE] = p * sn + q * cs;
        }
    }
}

template <int D>
__device__ __forceinline__ void prep_store(const PrepRow<D> &r, int lane, float *dst) {
#pragma unroll
    for (int m = 0; m < PrepRow<D>::E; ++m) dst[lane + 64 * m] = r.x[m];
}

}  // namespace g4

#endif
