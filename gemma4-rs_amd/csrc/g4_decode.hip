// Decode attention for Gemma 4's grouped-query layers on gfx950.
//
// One query position attends rows [begin, end) of a K/V cache whose rows are
// n_kv_heads*D f32 (the reference's `attend`, crates/llm-gemma4/src/impl_/model.rs:326-366).
// The G = n_heads/n_kv_heads query heads of a KV head (8 for Gemma 4 E2B)
// share every K/V byte, so the kernel streams each KV row from HBM once and
// applies it to all G heads with f32 MFMA:
//
//   S^T[16 keys x 16 cols] = K[16 keys x 4 dims] . Q^T[4 dims x 16 cols]   (v_mfma_f32_16x16x4f32)
//   O^T[16 dims x 16 cols] += V^T[16 dims x 4 keys] . P^T[4 keys x 16 cols]
//
// Columns are query heads (G <= 16; unused columns carry q = 0).  Computing
// S^T rather than S leaves each lane (g = lane/16, c = lane%16) holding the
// scores of keys 4g..4g+3 for head c -- exactly the B operand the P.V MFMA
// needs for k-step r = keys {4g + r}, so P never moves between lanes.
//
// A workgroup is 4 wavefronts that split the head dimension: wave w owns dims
// [w*D/4, (w+1)*D/4) of K, V, q and the output.  Each wave computes a partial
// S^T over its dims; the four partials are summed through LDS (fixed order, so
// every wave sees bit-identical scores and softmax state), then each wave
// accumulates P.V for its own dims.  Work is split over keys (split-K): a
// workgroup handles `chunk` consecutive keys of one (sequence, KV head) and
// leaves an online-softmax partial (m, l, O) that a second kernel merges.
//
// Softmax semantics follow softmax_f32 (crates/llm-backend-cpu/src/ops.rs:105-127):
// p = exp(s - max) / sum with scale applied to the dot product first
// (model.rs:334); a NaN or +inf score, or a row whose scores are all -inf,
// makes the call fail ("softmax input is not finite", model.rs:362-364).

#include "g4_internal.h"

namespace g4 {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxSplits = 1024;  // per (sequence, KV head); bounds the merge's LDS table

struct DecodeK {
    const float *q;
    const float *k;
    const float *v;
    int64_t row_stride;
    const int64_t *seq_row0;
    const int64_t *kv_begin;
    const int64_t *kv_end;
    int64_t kv_begin0, kv_end0, max_kv_len;
    int64_t pos0, prefill_window;
    int n_heads, n_kv_heads, group;
    float scale;
    int64_t chunk;
    int max_splits;
    float *out;
    float *part_o;   // [B][n_kv][max_splits][group][D]
    float2 *part_ml; // [B][n_kv][max_splits][group]  (running max, sum of exp)
    unsigned *status;
};

// Rows [begin, end) that sequence s attends, and where its cache starts.
__device__ inline void seq_range(const DecodeK &p, int s, int64_t &row0, int64_t &begin,
                                 int64_t &end) {
    if (p.prefill_window >= 0) {  // query s sits at position pos0 + s
        end = p.pos0 + s + 1;
        begin = (p.prefill_window > 0 && end > p.prefill_window) ? end - p.prefill_window : 0;
        row0 = 0;
    } else {
        row0 = p.seq_row0 ? p.seq_row0[s] : 0;
        begin = p.kv_begin ? p.kv_begin[s] : p.kv_begin0;
        end = p.kv_end ? p.kv_end[s] : p.kv_end0;
    }
}

__device__ inline int64_t num_splits(const DecodeK &p, int64_t len) {
    int64_t n = (len + p.chunk - 1) / p.chunk;
    return n < p.max_splits ? n : p.max_splits;
}

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// One workgroup = one (split, KV head, sequence).  D = head_dim (256 or 512).
template <int D>
__global__ __launch_bounds__(256) void decode_split_kernel(DecodeK p) {
    constexpr int DW = D / 4;   // dims owned by one wave
    constexpr int NU = DW / 32; // 32-dim K chunks per wave (8 MFMA k-steps each)
    constexpr int NV = DW / 64; // 64-dim V groups per wave (4 output tiles each)
    constexpr int NT = DW / 16; // 16-dim output tiles per wave
    static_assert(D % 256 == 0, "head_dim must be a multiple of 256");

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int split = blockIdx.x, kvh = blockIdx.y, s = blockIdx.z;

    int64_t row0, begin, end;
    seq_range(p, s, row0, begin, end);
    const int64_t len = end - begin;
    if (len <= 0 || len > p.max_kv_len) {
        if (split == 0 && kvh == 0 && threadIdx.x == 0)
            atomicOr(p.status, len <= 0 ? kStatusNonFinite : kStatusRangeTooLong);
        return;
    }
    const int64_t n_splits = num_splits(p, len);
    if (split >= n_splits) return;
    const int64_t k_lo = begin + split * p.chunk;
    const int64_t k_hi = (split + 1 == n_splits) ? end : k_lo + p.chunk;

    const int base = wave * DW;
    const bool col_valid = c < p.group;
    const int head = kvh * p.group + (col_valid ? c : 0);

    // Q^T as the B operand: lane (g, c) holds q[head c][base + 32u + 8g + j].
    float qreg[NU][8];
    {
        const float *qh = p.q + ((int64_t)s * p.n_heads + head) * D + base + 8 * g;
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            f32x4 a = *(const f32x4 *)(qh + 32 * u);
            f32x4 b = *(const f32x4 *)(qh + 32 * u + 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                qreg[u][j] = col_valid ? a[j] : 0.0f;
                qreg[u][4 + j] = col_valid ? b[j] : 0.0f;
            }
        }
    }

    const float *kcol = p.k + row0 * p.row_stride + (int64_t)kvh * D + base;
    const float *vcol = p.v + row0 * p.row_stride + (int64_t)kvh * D + base;

    __shared__ f32x4 sx[2][4][64];  // partial S^T exchange, double-buffered by iteration

    float m = -INFINITY, l = 0.0f;
    bool bad = false;
    f32x4 o[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) o[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    int it = 0;
    for (int64_t t0 = k_lo; t0 < k_hi; t0 += 16, ++it) {
        // K rows t0 + c (clamped into range; masked below), dims base+32u+8g..+7.
        const int64_t tk = (t0 + c < k_hi) ? t0 + c : k_hi - 1;
        const float *kp = kcol + tk * p.row_stride + 8 * g;
        f32x4 kv[NU][2];
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            kv[u][0] = *(const f32x4 *)(kp + 32 * u);
            kv[u][1] = *(const f32x4 *)(kp + 32 * u + 4);
        }
        // V rows t0 + 4g + r, dims base + 64U + 4c..+3.
        f32x4 vv[4][NV];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t tv = (t0 + 4 * g + r < k_hi) ? t0 + 4 * g + r : k_hi - 1;
            const float *vp = vcol + tv * p.row_stride + 4 * c;
#pragma unroll
            for (int U = 0; U < NV; ++U) vv[r][U] = *(const f32x4 *)(vp + 64 * U);
        }

        // Partial S^T over this wave's dims.
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[u][j >> 2][j & 3], qreg[u][j], acc, 0, 0, 0);

        const int buf = it & 1;
        sx[buf][wave][lane] = acc;
        __syncthreads();
        f32x4 sc = ((sx[buf][0][lane] + sx[buf][1][lane]) + sx[buf][2][lane]) + sx[buf][3][lane];

        // Scores of keys t0 + 4g + r for head c; mask the tail.
        float sv[4];
        float mt = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float x = sc[r] * p.scale;
            bad |= (x != x) || (x == INFINITY);
            sv[r] = (t0 + 4 * g + r < k_hi) ? x : -INFINITY;
            mt = fmaxf(mt, sv[r]);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float m_new = fmaxf(m, mt);
        float alpha, pr[4];
        if (m_new == -INFINITY) {  // every score so far is -inf: nothing accumulates
            alpha = 1.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) pr[r] = 0.0f;
        } else {
            alpha = exp2_fast((m - m_new) * kLog2e);
#pragma unroll
            for (int r = 0; r < 4; ++r) pr[r] = exp2_fast((sv[r] - m_new) * kLog2e);
        }
        l = l * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
        m = m_new;
#pragma unroll
        for (int i = 0; i < NT; ++i) o[i] *= alpha;

        // O^T += V^T . P^T, k-step r covers keys {t0 + 4g + r}.
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int U = 0; U < NV; ++U)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    o[4 * U + i] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[r][U][i], pr[r], o[4 * U + i], 0, 0, 0);
    }

    if (wave == 0 && __any(bad && col_valid) && lane == 0) atomicOr(p.status, kStatusNonFinite);

    // Sum of exp over the whole split for head c (lanes c, c+16, c+32, c+48).
    float lt = l + __shfl_xor(l, 16);
    lt = lt + __shfl_xor(lt, 32);

    if (n_splits == 1) {
        if (m == -INFINITY) {
            if (wave == 0 && lane == 0) atomicOr(p.status, kStatusNonFinite);
        }
        if (!col_valid) return;
        const float inv = 1.0f / lt;
        float *op = p.out + ((int64_t)s * p.n_heads + head) * D + base;
#pragma unroll
        for (int U = 0; U < NV; ++U)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) op[64 * U + 4 * (4 * g + r) + i] = o[4 * U + i][r] * inv;
        return;
    }
    if (!col_valid) return;
    const int64_t slot = ((int64_t)s * p.n_kv_heads + kvh) * p.max_splits + split;
    float *po = p.part_o + (slot * p.group + c) * D + base;
#pragma unroll
    for (int U = 0; U < NV; ++U)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) po[64 * U + 4 * (4 * g + r) + i] = o[4 * U + i][r];
    if (wave == 0 && g == 0) p.part_ml[slot * p.group + c] = float2{m, lt};
}

// Merges the split partials of one (sequence, head) for 64 dims:
// O = sum_j e^(m_j - M) O_j / sum_j e^(m_j - M) l_j.
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeK p, int D) {
    const int s = blockIdx.z, head = blockIdx.y;
    const int tid = threadIdx.x;
    int64_t row0, begin, end;
    seq_range(p, s, row0, begin, end);
    const int64_t len = end - begin;
    if (len <= 0 || len > p.max_kv_len) return;
    const int n = (int)num_splits(p, len);
    if (n <= 1) return;
    const int kvh = head / p.group, c = head % p.group;
    const int64_t slot0 = ((int64_t)s * p.n_kv_heads + kvh) * p.max_splits;

    __shared__ float w[kMaxSplits];
    __shared__ float red[256];
    __shared__ float part[4][64];

    float mx = -INFINITY;
    for (int j = tid; j < n; j += 256) mx = fmaxf(mx, p.part_ml[(slot0 + j) * p.group + c].x);
    red[tid] = mx;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if (tid < off) red[tid] = fmaxf(red[tid], red[tid + off]);
        __syncthreads();
    }
    const float M = red[0];
    __syncthreads();
    float lsum = 0.0f;
    for (int j = tid; j < n; j += 256) {
        float2 ml = p.part_ml[(slot0 + j) * p.group + c];
        float wj = (ml.x == -INFINITY) ? 0.0f : exp2_fast((ml.x - M) * kLog2e);
        w[j] = wj;
        lsum += wj * ml.y;
    }
    red[tid] = lsum;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if (tid < off) red[tid] = red[tid] + red[tid + off];
        __syncthreads();
    }
    const float L = red[0];
    if (M == -INFINITY && tid == 0 && blockIdx.x == 0) atomicOr(p.status, kStatusNonFinite);

    // 4 phases x 16 lanes x 4 dims: phase ph sums splits j = ph, ph+4, ...
    const int ph = tid >> 6, dl = tid & 63;
    const int d = blockIdx.x * 64 + dl;
    float acc = 0.0f;
    if (d < D) {
        for (int j = ph; j < n; j += 4) acc += w[j] * p.part_o[((slot0 + j) * p.group + c) * D + d];
    }
    part[ph][dl] = acc;
    __syncthreads();
    if (ph == 0 && d < D) {
        const float sum = ((part[0][dl] + part[1][dl]) + part[2][dl]) + part[3][dl];
        p.out[((int64_t)s * p.n_heads + head) * D + d] = sum / L;
    }
}

// Any shape the MFMA kernel does not cover (head_dim not a multiple of 256,
// more than 16 query heads per KV head): one workgroup per (head, sequence),
// 256 keys per step, online softmax in f32.
__global__ __launch_bounds__(256) void decode_generic_kernel(DecodeK p, int D) {
    const int head = blockIdx.x, s = blockIdx.y, tid = threadIdx.x;
    int64_t row0, begin, end;
    seq_range(p, s, row0, begin, end);
    const int64_t len = end - begin;
    if (len <= 0 || len > p.max_kv_len) {
        if (head == 0 && tid == 0) atomicOr(p.status, len <= 0 ? kStatusNonFinite : kStatusRangeTooLong);
        return;
    }
    const int kvh = head * p.n_kv_heads / p.n_heads;
    extern __shared__ float smem[];
    float *qs = smem;          // [D]
    float *ps = smem + D;      // [256]
    __shared__ float red[256];
    const float *qh = p.q + ((int64_t)s * p.n_heads + head) * D;
    for (int d = tid; d < D; d += 256) qs[d] = qh[d];
    const float *kb = p.k + row0 * p.row_stride + (int64_t)kvh * D;
    const float *vb = p.v + row0 * p.row_stride + (int64_t)kvh * D;
    constexpr int kMaxPer = 4;  // D <= 1024
    float o[kMaxPer] = {0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;
    bool bad = false;
    __syncthreads();
    for (int64_t t0 = begin; t0 < end; t0 += 256) {
        const int64_t t = t0 + tid;
        float x = -INFINITY;
        if (t < end) {
            const float *kr = kb + t * p.row_stride;
            float acc = 0.0f;
            for (int d = 0; d < D; ++d) acc = fmaf(qs[d], kr[d], acc);
            x = acc * p.scale;
            bad |= (x != x) || (x == INFINITY);
        }
        red[tid] = x;
        __syncthreads();
        for (int off = 128; off > 0; off >>= 1) {
            if (tid < off) red[tid] = fmaxf(red[tid], red[tid + off]);
            __syncthreads();
        }
        const float m_new = fmaxf(m, red[0]);
        __syncthreads();
        const float alpha = (m_new == -INFINITY) ? 1.0f : exp2_fast((m - m_new) * kLog2e);
        const float pt = (m_new == -INFINITY) ? 0.0f : exp2_fast((x - m_new) * kLog2e);
        ps[tid] = pt;
        red[tid] = pt;
        __syncthreads();
        for (int off = 128; off > 0; off >>= 1) {
            if (tid < off) red[tid] = red[tid] + red[tid + off];
            __syncthreads();
        }
        l = l * alpha + red[0];
        m = m_new;
        const int64_t nt = (end - t0 < 256) ? end - t0 : 256;
        for (int e = 0; e < kMaxPer; ++e) {
            const int d = tid + 256 * e;
            if (d >= D) break;
            float acc = o[e] * alpha;
            for (int64_t j = 0; j < nt; ++j) acc = fmaf(ps[j], vb[(t0 + j) * p.row_stride + d], acc);
            o[e] = acc;
        }
        __syncthreads();
    }
    if (__any(bad) && (tid & 63) == 0) atomicOr(p.status, kStatusNonFinite);
    if (m == -INFINITY && tid == 0) atomicOr(p.status, kStatusNonFinite);
    float *op = p.out + ((int64_t)s * p.n_heads + head) * D;
    for (int e = 0; e < kMaxPer; ++e) {
        const int d = tid + 256 * e;
        if (d < D) op[d] = o[e] / l;
    }
}

}  // namespace

int launch_decode(g4_ctx *ctx, const DecodeArgs &a, hipStream_t stream) {
    if (a.B <= 0) return G4_OK;
    const int D = a.head_dim;
    const int group = a.n_heads / a.n_kv_heads;
    DecodeK p{};
    p.q = a.q;
    p.k = a.k;
    p.v = a.v;
    p.row_stride = a.row_stride;
    p.seq_row0 = a.seq_row0;
    p.kv_begin = a.kv_begin;
    p.kv_end = a.kv_end;
    p.kv_begin0 = a.kv_begin0;
    p.kv_end0 = a.kv_end0;
    p.max_kv_len = a.max_kv_len;
    p.pos0 = a.pos0;
    p.prefill_window = a.prefill_window;
    p.n_heads = a.n_heads;
    p.n_kv_heads = a.n_kv_heads;
    p.group = group;
    p.scale = a.scale;
    p.out = a.out;
    p.status = ctx->status_dev;

    const bool mfma = (D == 256 || D == 512) && group <= 16 && a.n_heads % a.n_kv_heads == 0;
    if (!mfma) {
        if (D > 1024) return set_error(G4_ERR_COMPUTE, "head_dim above 1024 is not supported");
        p.chunk = a.max_kv_len > 0 ? a.max_kv_len : 1;
        p.max_splits = 1;
        hipLaunchKernelGGL(decode_generic_kernel, dim3(a.n_heads, a.B), dim3(256),
                           (size_t)(D + 256) * sizeof(float), stream, p, D);
        G4_HIP(hipGetLastError());
        return G4_OK;
    }

    // Split-K sizing: enough (sequence, KV head, split) work items to give
    // every CU a few workgroups, in multiples of the 16-key MFMA tile.
    const int64_t units = (int64_t)a.B * a.n_kv_heads;
    const int64_t max_len = a.max_kv_len > 0 ? a.max_kv_len : 1;
    int64_t chunk = ctx->decode_chunk;
    if (chunk <= 0) {
        const int64_t target = 4LL * ctx->num_cus;
        chunk = (max_len * units + target - 1) / target;
    }
    chunk = (chunk + 15) / 16 * 16;
    if (chunk < 16) chunk = 16;
    const int64_t min_chunk = (max_len + kMaxSplits - 1) / kMaxSplits;
    if (chunk < min_chunk) chunk = (min_chunk + 15) / 16 * 16;
    const int64_t max_splits = (max_len + chunk - 1) / chunk;
    p.chunk = chunk;
    p.max_splits = (int)max_splits;
    if (max_splits > 1) {
        const size_t slots = (size_t)units * max_splits * group;
        const size_t bytes = slots * D * sizeof(float) + slots * sizeof(float2) + 256;
        int rc = ensure_workspace(ctx, bytes, stream);
        if (rc != G4_OK) return rc;
        p.part_o = (float *)ctx->ws.ptr;
        size_t off = (slots * D * sizeof(float) + 255) / 256 * 256;
        p.part_ml = (float2 *)((char *)ctx->ws.ptr + off);
    }
    dim3 grid((unsigned)max_splits, (unsigned)a.n_kv_heads, (unsigned)a.B);
    if (D == 256)
        hipLaunchKernelGGL(decode_split_kernel<256>, grid, dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL(decode_split_kernel<512>, grid, dim3(256), 0, stream, p);
    G4_HIP(hipGetLastError());
    if (max_splits > 1) {
        hipLaunchKernelGGL(decode_merge_kernel, dim3((D + 63) / 64, a.n_heads, a.B), dim3(256), 0,
                           stream, p, D);
        G4_HIP(hipGetLastError());
    }
    return G4_OK;
}

}  // namespace g4
