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

#include <type_traits>

namespace g4 {

// Sum over the 64 lanes of a wavefront, in f64, the same bits in every lane:
// a butterfly whose partners are lane ^ 1, ^ 2 (DPP quad_perm), ^ 7 (DPP
// row_half_mirror), ^ 8 (DPP row_ror:8), ^ 16 and ^ 32 (permlane swaps); the
// six masks span the six lane bits.  Both partners of an exchange add the
// same two values (f64 addition is commutative), so every lane ends with
// the same sum.  Sums of f32 squares of one row are exact in f64 unless the
// squares span more than about 2^20, so the order does not change them.
__device__ __forceinline__ double wave_sum_f64(double v) {
    auto dpp = [](double x, auto ctrl) {
        const unsigned long long b = __double_as_longlong(x);
        const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)b, decltype(ctrl)::value, 0xF, 0xF, false);
        const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), decltype(ctrl)::value, 0xF, 0xF, false);
        return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
    };
    v += dpp(v, std::integral_constant<int, 0xB1>{});   // lane ^ 1
    v += dpp(v, std::integral_constant<int, 0x4E>{});   // lane ^ 2
    v += dpp(v, std::integral_constant<int, 0x141>{});  // lane ^ 7 within 8
    v += dpp(v, std::integral_constant<int, 0x128>{});  // lane ^ 8 within 16
    {
        const unsigned long long b = __double_as_longlong(v);
        const auto lo = __builtin_amdgcn_permlane16_swap((unsigned)b, (unsigned)b, false, false);
        const auto hi = __builtin_amdgcn_permlane16_swap((unsigned)(b >> 32), (unsigned)(b >> 32), false, false);
        v = __longlong_as_double((long long)(((unsigned long long)hi[0] << 32) | lo[0])) +
            __longlong_as_double((long long)(((unsigned long long)hi[1] << 32) | lo[1]));
    }
    {
        const unsigned long long b = __double_as_longlong(v);
        const auto lo = __builtin_amdgcn_permlane32_swap((unsigned)b, (unsigned)b, false, false);
        const auto hi = __builtin_amdgcn_permlane32_swap((unsigned)(b >> 32), (unsigned)(b >> 32), false, false);
        v = __longlong_as_double((long long)(((unsigned long long)hi[0] << 32) | lo[0])) +
            __longlong_as_double((long long)(((unsigned long long)hi[1] << 32) | lo[1]));
    }
    return v;
}

template <int D>
struct PrepRow {
    static constexpr int E = D / 64;   // elements per lane
    static constexpr int PE = E / 2;   // NEOX pairs per lane
    static constexpr int HALF = D / 2;
    float x[E], w[E];  // row, weight
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

// Loads row x and its weight w (or none).
template <int D>
__device__ __forceinline__ void prep_load(PrepRow<D> &r, int lane, const float *x, const float *w) {
#pragma unroll
    for (int m = 0; m < PrepRow<D>::E; ++m) r.x[m] = x[lane + 64 * m];
    if (w) {
#pragma unroll
        for (int m = 0; m < PrepRow<D>::E; ++m) r.w[m] = w[lane + 64 * m];
    }
}

// rms_norm (f64 mean of squares, ops.rs:45-56) times the weight, in the
// row's registers.
template <int D>
__device__ __forceinline__ void prep_norm(PrepRow<D> &r, bool has_w, float eps) {
#pragma clang fp contract(off)
    constexpr int E = PrepRow<D>::E;
    double sum = 0.0;
#pragma unroll
    for (int m = 0; m < E; ++m) {
        const float sq = r.x[m] * r.x[m];
        sum += (double)sq;
    }
    sum = wave_sum_f64(sum);
    const float mean = (float)(sum / (double)D);
    const float root = (float)sqrt((double)(mean + eps));
    const float scale = (float)(1.0 / (double)root);
#pragma unroll
    for (int m = 0; m < E; ++m) {
        r.x[m] = r.x[m] * scale;
        if (has_w) r.x[m] = r.x[m] * r.w[m];
    }
}

// Entry i of a token's RoPE table: the sine and cosine of pair i's angle
// theta_i / f_i (rope_neox, ops.rs:134-162), computed once per workgroup
// and shared by all of the token's heads.
__device__ __forceinline__ void prep_rope_table(float *cs, float *sn, int i, float theta, float factor) {
#pragma clang fp contract(off)
    sincosf(theta / factor, &sn[i], &cs[i]);
}

// The NEOX rotation of the row's pairs (i, i + D/2) by the table's angles.
template <int D>
__device__ __forceinline__ void prep_rope_tab(PrepRow<D> &r, int lane, const float *cs, const float *sn) {
#pragma clang fp contract(off)
    constexpr int PE = PrepRow<D>::PE;
#pragma unroll
    for (int m = 0; m < PE; ++m) {
        const float c = cs[lane + 64 * m], s = sn[lane + 64 * m];
        const float a = r.x[m], b = r.x[m + PE];
        r.x[m] = a * c - b * s;
        r.x[m + PE] = a * s + b * c;
    }
}

template <int D>
__device__ __forceinline__ void prep_store(const PrepRow<D> &r, int lane, float *dst) {
#pragma unroll
    for (int m = 0; m < PrepRow<D>::E; ++m) dst[lane + 64 * m] = r.x[m];
}

}  // namespace g4

#endif
