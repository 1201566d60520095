// Chunked prefill: N queries of one sequence, query i at position pos0 + i,
// each attending exactly the rows a decode step at that position would
// (crates/llm-gemma4/src/impl_/generate.rs:37-41, eng/mod.rs:10-36): keys
// [0, p+1) on global layers, [(p+1-W)+, p+1) on sliding-window layers.
//
// MFMA tiling (f32, v_mfma_f32_16x16x4f32).  The 8 query heads that share a
// KV head are folded into the row dimension: a wavefront owns 16 rows (two
// positions x eight heads) and keeps their Q^T (B operand) and O^T
// accumulators in registers for the whole key range; a workgroup of four
// wavefronts covers eight positions and streams 16-key K/V tiles through
// double-buffered LDS, so every K/V byte fetched is used by 64 query rows.
// Per tile and wavefront:
//   S^T[16 keys x 16 rows] = K[16 keys x D] . Q^T[D x 16 rows]     (D/4 MFMAs)
//   mask (causal / window, per element), online softmax per row
//   O^T[D x 16 rows]      += V^T[D x 16 keys] . P^T[16 keys x 16 rows] (D/4 MFMAs)
// Computing S^T leaves lane (g, c) holding keys 4g..4g+3 of row c, which is
// the B-operand layout P^T needs, so P stays in registers.
//
// Two forms of the same tiling, chosen per work unit: split-f16 products
// (each f32 operand as an f16 hi + lo pair, v_mfma_f32_16x16x32_f16, K/V
// read from planes a prepass writes in operand order; see split_f16) for
// units whose inputs the split carries, and the f32 MFMA form above for the
// others.  Both leave the same partial layout, so one merge serves both.
//
// Work balance: the causal triangle gives the last position blocks many more
// tiles than the first, so a block's key range may be cut into units (at
// most kPrefillMaxUnitsDev per block), and the host assigns every unit to a
// workgroup (at most one per CU), which runs its units in turn; the
// schedule builder below explains the choice.  A block with one unit writes
// its output directly; otherwise each unit leaves an (m, l, O) partial and a
// merge kernel combines them in key order.

#include <algorithm>
#include <cmath>
#include <array>
#include <functional>
#include <queue>
#include <utility>
#include <vector>

#include "g4_internal.h"

namespace g4 {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
// s_waitcnt operand: vector memory count 0 (the LDS-bound tile loads have
// landed), export and LDS/scalar counts left at their maxima.
constexpr int kVmcntZero = 0x0F70;
constexpr int kRowsPerWave = 16;
constexpr int kWaves = 4;
constexpr int kPosPerWave = 2;                       // 16 rows = 2 positions x 8 heads
constexpr int kPosPerBlock = kWaves * kPosPerWave;   // 8
constexpr int kGroup = 8;                            // query heads per KV head
// Lazy-rescaling slack, 32 in log2 units: a weight p = e^(s - m) stays
// below 2^32, so l and O (sums of p and p*v over the keys) stay below
// 2^32 * keys * max|v| -- far from the f32 limit 2^128 -- and the final O/l
// is the same ratio whatever reference max m it was accumulated against.
// Normalised Gemma queries and keys give scores spread over tens of units,
// which a slack of 8 log2 units made rescale on most tiles.
constexpr float kRescaleSlack = 32.0f / 1.4426950408889634f;
constexpr int kPrefillMaxUnitsDev = 8;  // partial units per block (merge weight table)
// Buffer resource (V#) word 3 for raw 32-bit-element buffers on gfx9-class
// GPUs, gfx950 included.
constexpr int kBufferWord3 = 0x00020000;

// Split-f16 products.  An f32 value x is carried as two f16 values, hi =
// rn16(x) and lo = rn16((x - hi) * 2^11) (x - hi is exact in f32), so x =
// hi + lo * 2^-11 to within max(2^-22 |x|, 2^-36): the scaled lo keeps the
// residue of a small x out of the f16 subnormals (Ootomo & Yokota,
// "Recovering single precision accuracy from Tensor Cores while surpassing
// the FP32 theoretical peak performance", IJHPCA 2022, in its f16 form).  A
// score q.k is then hi.hi' + 2^-11 (hi.lo' + lo.hi') -- three
// v_mfma_f32_16x16x32_f16 into f32 accumulators, the two corrections in
// their own -- at 16x the f32 MFMA's products per instruction, so 3/16 of
// its matrix cycles; the dropped lo.lo' term is below 2^-22 |q_d k_d|.
// The f16 MFMAs keep subnormal operands and form products exactly.
//
// P.V splits V the same way without the scale (V's residue error, at most
// 2^-25 per element, is weighted by p/l <= 1) and carries the weights
// scaled by 2^kPScale instead: with the rescale slack below they stay under
// 2^15, and a weight's own floor is 2^-25 / 2^kPScale = 2^-32 of the row's
// reference weight, which keeps large |v| from amplifying it.
//
// hi stays finite for |x| < 2^15; a unit whose q rows or K/V tiles hold
// anything else (a larger value, NaN, inf) runs with f32 MFMAs instead,
// which also keeps the reference's non-finite semantics.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
constexpr float kSplitMax = 32768.0f;
constexpr float kLoScale = 2048.0f, kLoUnscale = 1.0f / 2048.0f;  // 2^11
// Weights p = 2^kPScale e^(s - m) with a slack of 8 log2 units stay below
// 2^15 (finite in f16).  Partials report m - kPScale ln 2, so that their
// (m, l, O) mean the same as the f32 form's.
constexpr int kPScale = 7;
constexpr float kRescaleSlackSplit = 8.0f / 1.4426950408889634f;
constexpr float kPScaleNat = 7.0f * 0.6931471805599453f;

__device__ inline f32x4 split_mfma(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// hi and lo halves of x, lo unscaled (V) or scaled by 2^11 (Q, K); `bad` is
// raised for a value the split does not carry.
template <bool SCALED>
__device__ inline void split_f16(float x, _Float16 &hi, _Float16 &lo, bool &bad) {
    bad |= !(__builtin_fabsf(x) < kSplitMax);  // NaN compares false
    hi = (_Float16)x;
    const float r = x - (float)hi;
    lo = (_Float16)(SCALED ? r * kLoScale : r);
}

struct PrefillUnit {
    int block;   // position block: positions pos0 + 8*block .. +7
    int t_lo;    // first 16-key tile
    int t_hi;    // one past the last tile
    int slot;    // partial slot, or -1 when the block has a single unit
};

struct PrefillBlockInfo {
    int first_slot;
    int n_units;
};

struct PrefillK {
    const float *q;
    const float *k;
    const float *v;
    int64_t row_stride;
    int64_t pos0, N, window;
    int64_t kv_origin;  // the position of row 0 of k/v
    int n_heads;
    float scale;
    float *out;
    const PrefillUnit *units;      // grouped by workgroup
    const int *bin_start;          // workgroup x runs units [bin_start[x], bin_start[x + 1])
    const PrefillBlockInfo *blocks;
    float *part_o;    // [slot][kv head][wave][D/16 tiles][64 lanes] f32x4
    float2 *part_ml;  // [slot][kv head][64 rows]
    int n_slots;
    unsigned *status;
    // Split-f16 planes of K and V (null: every unit uses f32 MFMAs):
    // [tile - t0][kv head][K block | V block], each block 16 keys x D dims
    // x (hi, lo) f16 in the MFMA operand order (prefill_split_kernel), and
    // two flags per (tile, kv head), K's and V's, set when the block's rows
    // hold a value the split does not carry.
    const _Float16 *planes;
    uint32_t plane_bytes;
    int64_t t0;
    const int *tile_flags;
};

// Conversion of the rows a prefill call attends, keys [row_lo, row_hi), into
// the split-f16 planes, one 16-key tile per (tile, kv head); rows of a tile
// outside the range are zeros.  Flags: [tile][kv head][K, V].
struct SplitK {
    const float *k;
    const float *v;
    int64_t row_stride;
    int64_t kv_origin;
    int64_t row_lo, row_hi;
    int64_t t0;
    _Float16 *planes;
    int *tile_flags;
};

// K block of a tile: for each 32-dim chunk u and part (hi, lo), 64 lanes x 8
// halves, lane 16g + c holding key c, dims 32u + 8g .. +7 -- the A operand of
// the score MFMA (S^T = K Q^T).  V block: for each O^T tile T (dims
// 64(T/4) + 4i + T%4, i < 16, the f32 path's accumulator order), 64 lanes x
// 8 halves, lane 16g + c holding dim 64(T/4) + 4c + T%4 of keys 4g .. 4g+3,
// hi parts then lo parts -- the A operand of O^T += V^T P^T, whose B operand
// is the lane's own four weights (keys 4g .. 4g+3, the score MFMA's output
// layout) twice.  Every block is one contiguous run of 16-byte lane slots,
// which the prefill kernel copies to LDS unchanged.
//
// Workgroup (tile, kv head, z): z = 0 writes the K block, z = 1 the V block,
// and its own flag.  A K thread makes the two slots (hi, lo) of one lane and
// chunk from two 16-byte loads; a V thread makes the four slots T = 4U .. 4U+3
// of one lane from four 16-byte loads (keys 4g .. 4g+3, dims 64U + 4c ..
// +3), so every load is issued before any conversion waits.
template <int D>
__global__ __launch_bounds__(256) void prefill_split_kernel(SplitK s) {
    constexpr int KIT = 2 * D / 256;  // K lane slots per thread: (D/32 chunks) x 64 lanes
    constexpr int VIT = D / 256;      // V lane groups per thread: (D/64) x 64 lanes
    static_assert(KIT >= 1 && VIT >= 1, "head width of at least 256");
    const int tid = threadIdx.x, kvh = blockIdx.y, n_kv = gridDim.y, tt = blockIdx.x;
    const int64_t key0 = 16 * (s.t0 + tt);
    _Float16 *kb = s.planes + ((int64_t)tt * n_kv + kvh) * (64 * D);
    _Float16 *vb = kb + 32 * D;
    auto row = [&](const float *base, int key) -> const float * {
        const int64_t pos = key0 + key;
        if (pos < s.row_lo || pos >= s.row_hi) return nullptr;
        return base + (pos - s.kv_origin) * s.row_stride + (int64_t)kvh * D;
    };
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    bool bad = false;
    if (blockIdx.z == 0) {
        f32x4 x[KIT][2];
#pragma unroll
        for (int e = 0; e < KIT; ++e) {
            const int it = tid + 256 * e, uu = it >> 6, g = (it >> 4) & 3, c = it & 15;
            const float *r = row(s.k, c);
            x[e][0] = r ? *(const f32x4 *)(r + 32 * uu + 8 * g) : zero;
            x[e][1] = r ? *(const f32x4 *)(r + 32 * uu + 8 * g + 4) : zero;
        }
#pragma unroll
        for (int e = 0; e < KIT; ++e) {
            const int it = tid + 256 * e, uu = it >> 6, lane = it & 63;
            f16x8 hi, lo;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                _Float16 h, l;
                split_f16<true>(x[e][j >> 2][j & 3], h, l, bad);
                hi[j] = h;
                lo[j] = l;
            }
            *(f16x8 *)(kb + ((uu * 2 + 0) * 64 + lane) * 8) = hi;
            *(f16x8 *)(kb + ((uu * 2 + 1) * 64 + lane) * 8) = lo;
        }
    } else {
        f32x4 x[VIT][4];
#pragma unroll
        for (int e = 0; e < VIT; ++e) {
            const int it = tid + 256 * e, U = it >> 6, g = (it >> 4) & 3, c = it & 15;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float *rp = row(s.v, 4 * g + r);
                x[e][r] = rp ? *(const f32x4 *)(rp + 64 * U + 4 * c) : zero;
            }
        }
#pragma unroll
        for (int e = 0; e < VIT; ++e) {
            const int it = tid + 256 * e, U = it >> 6, lane = it & 63;
#pragma unroll
            for (int i = 0; i < 4; ++i) {  // T = 4U + i: dim 64U + 4c + i
                f16x8 hl;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    _Float16 h, l;
                    split_f16<false>(x[e][r][i], h, l, bad);
                    hl[r] = h;
                    hl[4 + r] = l;
                }
                *(f16x8 *)(vb + ((4 * U + i) * 64 + lane) * 8) = hl;
            }
        }
    }
    // Zero rows (outside the range) never raise the flag.
    bad = __syncthreads_or(bad);
    if (tid == 0) s.tile_flags[((int64_t)tt * n_kv + kvh) * 2 + blockIdx.z] = bad ? 1 : 0;
}

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Reductions over the four 16-lane rows of a wavefront (lanes c, c+16,
// c+32, c+48), done with row swaps on the VALU and identical in every lane.
__device__ inline float rows_max(float v) {
    // NaN-propagating maximum: no operand canonicalisation (fmaxf needs it),
    // and a NaN only shows up for a row already flagged non-finite.
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float h = __builtin_elementwise_maximum(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(h), __float_as_uint(h), false, false);
    return __builtin_elementwise_maximum(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ inline float rows_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float h = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(h), __float_as_uint(h), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// s_waitcnt operand: LDS/scalar count 0 (this wave's ds_writes are done),
// vector memory and export counts left at their maxima.
constexpr int kLgkmcntZero = 0xC07F;

// Workgroup barrier after this wave's own LDS writes: they are complete
// (lgkm count 0) before the barrier, and the signal fences keep the compiler
// from moving LDS accesses across it.  Unlike __syncthreads(), whose fence
// also waits for the next tile's LDS-bound loads (they write LDS), those
// stay in flight; nothing read after this barrier is written by them.
__device__ inline void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(kLgkmcntZero);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// One 16-byte load per lane from `rsrc` at byte offset voff, written straight
// to LDS at lds + 16 * lane (lds is the same for the whole wavefront).
__device__ inline void load_to_lds(__amdgpu_buffer_rsrc_t rsrc, f32x4 *lds, uint32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)lds, 16, voff, 0, 0, 0);
#endif
}

// Workgroup geometry for head width D: 4 row groups of 16 rows, each owned by
// SPLIT wavefronts that divide the head dimension (DH = D / SPLIT dims each),
// so that one wavefront's Q^T and O^T fit the register file.
//
// At D = 512 the head does not fit one wavefront's registers (SPLIT = 2),
// and each SIMD runs the two waves of a row group.  At D = 256 a wavefront
// holds Q^T and O^T for the whole head (SPLIT = 1); to give each SIMD two
// waves there as well, a second group of four waves (KSPLIT = 2) takes the
// odd tiles of the same rows, keeping its own softmax state, and hands it to
// the first group at the end of the unit.  One workgroup per CU either way.
template <int D>
struct PrefillShape {
    static constexpr int SPLIT = D == 256 ? 1 : 2;
    static constexpr int KSPLIT = D == 256 ? 2 : 1;  // wave groups taking alternate tiles
    static constexpr int DH = D / SPLIT;
    static constexpr int RWAVES = kWaves * SPLIT;    // waves holding the result (the merge grid's z)
    static constexpr int WAVES = RWAVES * KSPLIT;
    static constexpr int THREADS = 64 * WAVES;
    static constexpr int TPS = KSPLIT;               // tiles per step, one per wave group
};

// One unit: the rows of position block u.block against its key tiles
// [u.t_lo, u.t_hi), leaving the block's output or the unit's partial.
// SPLIT16: products as split-f16 MFMAs from the planes; such a unit first
// checks that its q rows and tiles are carried exactly by the split, and
// returns false (having written nothing) when they are not, for the caller
// to run the f32 form.  The f32 form reads K/V rows directly and returns
// true.
// The kernel's LDS arrays (declared there, so that both forms of the unit
// share them).
struct PrefillLds {
    f32x4 *k0, *v0, *k1, *v1;
    f32x4 (*s0)[64], (*s1)[64];
    int *nf_tile;
    int *vote;  // one word per wavefront: the split form's go / no-go
};

template <int D, bool SPLIT16>
__device__ __forceinline__ bool prefill_unit(const PrefillK &p, const PrefillUnit u, const PrefillLds &L) {
    using S = PrefillShape<D>;
    constexpr int DH = S::DH;
    constexpr int NU = DH / 32;  // 32-dim K chunks per wave
    constexpr int NV = DH / 64;  // 64-dim V groups per wave
    constexpr int NT = DH / 16;  // O^T tiles per wave
    constexpr int TILE_F4 = 16 * D / 4;
    constexpr int PER_THREAD = TILE_F4 / S::THREADS;  // loads per thread per tile, of K and of V
    constexpr int TPS = S::TPS;

    const int tid = threadIdx.x;
    // The wavefront index is uniform; readfirstlane lets the compiler keep
    // it, and the tile tests derived from it, in scalar registers and
    // branch on them without exec masks.
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rg = wave % kWaves;                           // row group
    const int half = S::SPLIT == 2 ? wave / kWaves : 0;     // dim half
    const int kpar = S::KSPLIT == 2 ? wave / kWaves : 0;    // tile parity
    const int g = lane >> 4, c = lane & 15;
    const int kvh = blockIdx.y;

    const int64_t P0 = p.pos0 + (int64_t)kPosPerBlock * u.block;
    const int64_t last_pos = p.pos0 + p.N - 1;
    const int64_t pos = P0 + kPosPerWave * rg + (c >> 3);  // this lane's row position
    const bool row_valid = pos <= last_pos;
    const int head = kvh * kGroup + (c & 7);
    const int64_t win = p.window;
    const int d0 = half * DH;  // first dim of this wave

    f32x4 *const lds_k0 = L.k0, *const lds_v0 = L.v0, *const lds_k1 = L.k1, *const lds_v1 = L.v1;
    f32x4(*const lds_s0)[64] = L.s0;
    f32x4(*const lds_s1)[64] = L.s1;
    int *const nf_tile = L.nf_tile;
    // A flag of an earlier unit is cleared before this unit's first step
    // (the caller's barrier between units ordered that unit's last read).
    if (!SPLIT16 && tid < S::KSPLIT) nf_tile[tid] = 0;

    // K/V tiles go straight from memory to LDS (buffer_load ... lds: lane l
    // of a wavefront writes the 16 bytes it loads to LDS base + 16*l), so the
    // LDS layout is chosen by which address each lane loads: thread tid fills
    // float4 slot f = (e*WAVES + wave)*64 + lane of the tile, e < PER_THREAD.
    // K slots are swizzled -- ((u*4 + g)*2 + h)*16 + key holds dims
    // 32u + 8g + 4h .. +3 -- so the 16 lanes reading a quarter MFMA operand
    // read 256 contiguous bytes; V slots are row-major [key][D/4].  The
    // resources span the rows some query of this block attends, [block_lo,
    // last_pos]; every other row of a tile (before the window, past the
    // chunk) reads as zeros in hardware, so nothing it holds can reach the
    // output through a zero softmax weight (0 * NaN).  The tile's offset goes
    // into the per-lane offset, which the range check covers.
    const int stride = (int)p.row_stride;  // (pos0 + N) rows of it span < 2^31 bytes (checked by the launcher)
    const int64_t block_lo = (win > 0 && P0 + 1 > win) ? P0 + 1 - win : 0;
    const int n_rows = (int)(last_pos + 1 - block_lo);
    const int64_t first = (block_lo - p.kv_origin) * p.row_stride + (int64_t)kvh * D;  // row of key block_lo
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc((void *)(p.k + first), 0, (n_rows - 1) * stride * 4 + D * 4, kBufferWord3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc((void *)(p.v + first), 0, (n_rows - 1) * stride * 4 + D * 4, kBufferWord3);
    // Split form: one resource over all planes; a tile's K block of this KV
    // head is 64*D contiguous bytes (its V block follows), copied slot for
    // slot.
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc((void *)p.planes, 0, (int)p.plane_bytes, kBufferWord3);
    uint32_t koffs[PER_THREAD], voffs[PER_THREAD];
#pragma unroll
    for (int e = 0; e < PER_THREAD; ++e) {
        const int f = (e * S::WAVES + wave) * 64 + lane;
        if constexpr (SPLIT16) {
            koffs[e] = 16u * (uint32_t)f;
            voffs[e] = 16u * (uint32_t)f + 64u * D;
        } else {
            const int key = f & 15, rest = f >> 4;
            const int dim = 32 * (rest >> 3) + 8 * ((rest >> 1) & 3) + 4 * (rest & 1);
            koffs[e] = (uint32_t)(key * stride + dim) * 4u;
            voffs[e] = (uint32_t)((f / (D / 4)) * stride + 4 * (f % (D / 4))) * 4u;
        }
    }
    // Load i (of 2*PER_THREAD) of tile t: K slots for even i, V for odd.
    auto issue_part = [&](int t, int i, f32x4 *kb, f32x4 *vb) {
        const int e = i >> 1, slot = (e * S::WAVES + wave) * 64;
        if constexpr (SPLIT16) {
            const uint32_t toff = (uint32_t)(((t - p.t0) * (int64_t)gridDim.y + kvh) * (128LL * D));
            load_to_lds(prs, (i & 1) ? vb + slot : kb + slot, ((i & 1) ? voffs[e] : koffs[e]) + toff);
        } else {
            const uint32_t toff = (uint32_t)((16LL * t - block_lo) * stride * 4);  // wraps below block_lo: out of range
            if (i & 1)
                load_to_lds(vrs, vb + slot, voffs[e] + toff);
            else
                load_to_lds(krs, kb + slot, koffs[e] + toff);
        }
    };
    auto issue_tile = [&](int t, f32x4 *kb, f32x4 *vb) {
#pragma unroll
        for (int i = 0; i < 2 * PER_THREAD; ++i) issue_part(t, i, kb, vb);
    };

    // The split form loads its tile flags and q first, then issues its first
    // tiles before it knows whether it will use them: the flags and q land
    // while the tiles are in flight, and the check below waits for them
    // only (loads complete in order), not for the tiles.
    int flags = 0;
    if constexpr (SPLIT16) {
        for (int f = 2 * u.t_lo + tid; f < 2 * u.t_hi; f += S::THREADS)  // (tile, K | V) flags
            flags |= p.tile_flags[((int64_t)(f / 2 - p.t0) * gridDim.y + kvh) * 2 + (f & 1)];
    }
    // Q^T (B operand): lane (g, c) holds q[row c][d0 + 32u + 8g + j].
    float qreg[NU][8];
    {
        const int64_t qpos = row_valid ? pos : last_pos;
        const float *qr = p.q + ((qpos - p.pos0) * p.n_heads + head) * D + d0 + 8 * g;
#pragma unroll
        for (int uu = 0; uu < NU; ++uu) {
            const f32x4 a = *(const f32x4 *)(qr + 32 * uu);
            const f32x4 b = *(const f32x4 *)(qr + 32 * uu + 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                qreg[uu][j] = a[j];
                qreg[uu][4 + j] = b[j];
            }
        }
    }
    if constexpr (SPLIT16) {
        // K(0), V(0) and K(1): the split form's step loop reads K one step
        // ahead of V.
#pragma unroll
        for (int j = 0; j < TPS; ++j) {
            issue_tile(u.t_lo + j < u.t_hi ? u.t_lo + j : u.t_hi - 1, lds_k0 + j * TILE_F4, lds_v0 + j * TILE_F4);
            const int t1 = u.t_lo + TPS + j < u.t_hi ? u.t_lo + TPS + j : u.t_hi - 1;
#pragma unroll
            for (int e = 0; e < PER_THREAD; ++e) issue_part(t1, 2 * e, lds_k1 + j * TILE_F4, nullptr);
        }
    }
    // Split form: Q^T as hi and lo halves, in the same lanes.  The unit runs
    // in f32 instead when a q value or a tile flag says the split does not
    // carry its inputs exactly (the tiles issued above land first: the LDS
    // they write is the f32 form's too).
    f16x8 qh[SPLIT16 ? NU : 1], ql[SPLIT16 ? NU : 1];
    if constexpr (SPLIT16) {
        bool off = false;
#pragma unroll
        for (int uu = 0; uu < NU; ++uu)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                _Float16 h, lo;
                split_f16<true>(qreg[uu][j], h, lo, off);
                qh[uu][j] = h;
                ql[uu][j] = lo;
            }
        off |= flags != 0;
        // Workgroup vote through LDS behind an LDS-only barrier (a
        // __syncthreads would also wait for the tiles in flight).  The next
        // vote's writes follow this unit's later barriers, so no wave
        // overwrites a word another is still reading.
        const bool any = __any(off);  // every lane takes part in the ballot
        if (lane == 0) L.vote[wave] = any ? 1 : 0;
        lds_barrier();
        int v = 0;
#pragma unroll
        for (int w = 0; w < S::WAVES; ++w) v |= L.vote[w];
        if (v != 0) {
            __builtin_amdgcn_s_waitcnt(kVmcntZero);
            return false;
        }
    }

    f32x4 o[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) o[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;
    bool bad = false;
    const bool scaled = p.scale != 1.0f;  // Gemma's scale is 1: x * 1 == x, skip the multiply

    // Tiles t .. t+TPS-1 are read from (kb, vb) -- tile t+j at j*TILE_F4, by
    // the wave group of parity j -- while the next step's tiles load into
    // (kn, vn).
    // Tile tt is in the unit and every row of the block attends all of its
    // keys: 16 tt + 15 <= P0 and, with a window, 16 tt > P0 + 7 - W.  Those
    // tiles are [ex_lo, ex_hi], found once per unit in 64 bits so that the
    // per-step test is two 32-bit compares of tile indices.
    const int ex_hi = (int)((P0 + 1) / 16 - 1);
    const int64_t wlo = P0 + kPosPerBlock - 1 - win;
    const int ex_lo = (win > 0 && wlo >= 0) ? (int)(wlo / 16 + 1) : 0;
    auto exact = [&](int tt) { return tt < u.t_hi && tt >= ex_lo && tt <= ex_hi; };
    auto step = [&](int t, const f32x4 *kb, f32x4 *vb, f32x4 (*ls)[64], f32x4 *kn, f32x4 *vn) {
        // This step's tiles have landed (this wave's loads, then everyone's),
        // and every wave is done reading (kn, vn): fetch the next tiles into
        // them.  Past the unit's end the last tile is fetched again
        // (unread), keeping every step's loads unconditional.
        __builtin_amdgcn_s_waitcnt(kVmcntZero);
        __syncthreads();
        int tn[TPS];
#pragma unroll
        for (int j = 0; j < TPS; ++j) tn[j] = t + TPS + j < u.t_hi ? t + TPS + j : u.t_hi - 1;
        // This wave's tile; a group with no tile left in the unit computes a
        // stale one with every score masked (its weights are exactly 0).
        const int tw = t + kpar;
        const bool live = S::KSPLIT == 1 || tw < u.t_hi;  // one group: a step's tile is always live
        const f32x4 *kt = kb + kpar * TILE_F4;
        constexpr int NL = 2 * PER_THREAD * TPS;  // tile-part loads per step
        // Load i: tile i / (2 PER_THREAD) of the next step, part i % (2 PER_THREAD).
        auto load = [&](int i) {
            const int j = i / (2 * PER_THREAD);
            issue_part(tn[j], i % (2 * PER_THREAD), kn + j * TILE_F4, vn + j * TILE_F4);
        };
        // Partial S^T over this wave's DH dims: one accumulator per 32-dim
        // chunk (eight MFMAs of four products each), summed pairwise, so that
        // a score's f32 rounding grows with the log of the chunk count rather
        // than with the chunk count (with scores in the hundreds, two long
        // chains put the form's error at several times that of the
        // reference's own f32 loop).  A chunk's K operands are read from LDS
        // one chunk ahead, into the other of two register slots, so the MFMAs
        // of chunk uu run while chunk uu+1's reads are in flight (one slot
        // made every chunk wait for its own LDS read).  A group whose tile is
        // stale (the unit's last step with an odd tile count) only issues its
        // share of the next loads: its scores are all masked below.
        f32x4 acc[NU];
#pragma unroll
        for (int uu = 0; uu < NU; ++uu) acc[uu] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (live) {
            f32x4 kc[2][2];
            auto read_k = [&](int uu, f32x4(&dst)[2]) {
                const int ug = d0 / 32 + uu;
                dst[0] = kt[((ug * 4 + g) * 2 + 0) * 16 + c];
                dst[1] = kt[((ug * 4 + g) * 2 + 1) * 16 + c];
            };
            read_k(0, kc[0]);
#pragma unroll
            for (int uu = 0; uu < NU; ++uu) {
                if (uu + 1 < NU) read_k(uu + 1, kc[(uu + 1) & 1]);
                // The next tile's loads go out one or two per 8 MFMAs, so that
                // they issue while the matrix pipe works rather than queue up
                // behind each other at the top of the step.
                static_assert(NL % NU == 0 || NU % NL == 0, "loads spread over the chunks");
                if constexpr (NL >= NU) {
#pragma unroll
                    for (int i = uu * (NL / NU); i < (uu + 1) * (NL / NU); ++i) load(i);
                } else if (uu % (NU / NL) == 0) {
                    load(uu / (NU / NL));
                }
                const f32x4 k0 = kc[uu & 1][0], k1 = kc[uu & 1][1];
                f32x4 &a = acc[uu];
#pragma unroll
                for (int j = 0; j < 4; ++j) a = __builtin_amdgcn_mfma_f32_16x16x4f32(k0[j], qreg[uu][j], a, 0, 0, 0);
#pragma unroll
                for (int j = 0; j < 4; ++j) a = __builtin_amdgcn_mfma_f32_16x16x4f32(k1[j], qreg[uu][4 + j], a, 0, 0, 0);
            }
            // Scheduling: chunk 0's K reads, then per chunk the next chunk's K
            // reads, the next tile's loads (one or two per 8 MFMAs) and the
            // chunk's 8 MFMAs.
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
#pragma unroll
            for (int uu = 0; uu < NU; ++uu) {
                if (uu + 1 < NU) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);       // DS read
                __builtin_amdgcn_sched_group_barrier(0x010, NL >= NU ? NL / NU : 1, 0);  // VMEM
                __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);                        // MFMA
            }
        } else {
#pragma unroll
            for (int i = 0; i < NL; ++i) load(i);
        }
        static_assert((NU & (NU - 1)) == 0, "a power-of-two chunk count");
#pragma unroll
        for (int w = 1; w < NU; w *= 2)
#pragma unroll
            for (int uu = 0; uu + w < NU; uu += 2 * w) acc[uu] += acc[uu + w];
        f32x4 sc = acc[0];
        if constexpr (S::SPLIT == 2) {
            // Full scores = half 0 + half 1, added in that order by both waves.
            ls[wave][lane] = sc;
            lds_barrier();
            sc = ls[rg][lane] + ls[rg + kWaves][lane];
        }

        // Exact attended set per row: key <= pos and, with a window, key >
        // pos - W.  Tiles every row of the block sees whole skip the test.
        float sv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sv[r] = scaled ? sc[r] * p.scale : sc[r];
        const bool whole = exact(tw) || !live;  // a stale tile is masked whole below
        if (!live) {
#pragma unroll
            for (int r = 0; r < 4; ++r) sv[r] = -INFINITY;
        } else if (!whole) {
            const int64_t rel = pos - 16LL * tw;  // key - 16tw <= rel, and > rel - win
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int kr = 4 * g + r;
                if (!(kr <= rel && (win == 0 || kr > rel - win))) sv[r] = -INFINITY;
            }
        }
        // The lane's 4 scores (one row) by a NaN-propagating maximum
        // (v_maximum3_f32): NaN or +inf among them shows in mx, so one class
        // test flags the row.  For other scores mx is the plain maximum.
        const float mx = __builtin_elementwise_maximum(__builtin_elementwise_maximum(sv[0], sv[1]),
                                                       __builtin_elementwise_maximum(sv[2], sv[3]));
        bad |= __builtin_amdgcn_classf(mx, 0x203);  // signalling/quiet NaN, +inf
        const float mt = rows_max(mx);
        // Lazy rescaling: a row keeps its reference max m until a score
        // exceeds it by more than kRescaleSlack (p < 2^32 meanwhile, safe in
        // f32), so O is rescaled about once per row rather than every tile.
        if (__any(mt > m + kRescaleSlack)) {
            const float m_new = fmaxf(m, mt);
            const float alpha = (m_new == -INFINITY) ? 1.0f : exp2_fast((m - m_new) * kLog2e);
            l *= alpha;
            m = m_new;
#pragma unroll
            for (int i = 0; i < NT; ++i) o[i] *= alpha;
        }
        float pr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[r] = (m == -INFINITY) ? 0.0f : exp2_fast((sv[r] - m) * kLog2e);
        l += (pr[0] + pr[1]) + (pr[2] + pr[3]);

        // Edge tiles: some row of the block masks keys of the tile that
        // another row attends (or a wave group's tile is a stale one, every
        // key masked).  A masked key's weight is exactly 0, but 0 * NaN and
        // 0 * inf are NaN, and the reference multiplies only the rows a query
        // attends (model.rs:339-341).  So the group's V tile has its
        // non-finite values replaced by 0 in LDS before the product, and if
        // it held any, their p * v terms are added afterwards, from memory, to
        // the rows that attend them.  (Rows outside [block_lo, last_pos]
        // already read as 0.)  Steps with no edge tile skip all of this.
        bool fix = false;
        if (!exact(t) || (TPS == 2 && !exact(t + 1))) {  // uniform in the workgroup
            if (!(live && whole)) {
                constexpr int GL = 64 * S::RWAVES;  // lanes of the waves sharing this V tile
                f32x4 *vs = vb + kpar * TILE_F4;
                const int gl = tid - kpar * GL;
                bool found = false;
#pragma unroll
                for (int e = 0; e < TILE_F4 / GL; ++e) {
                    f32x4 x = vs[e * GL + gl];
                    bool bad4 = false;
#pragma unroll
                    for (int i = 0; i < 4; ++i) bad4 |= !__builtin_amdgcn_classf(x[i], 0x1F8);  // not -normal..+normal
                    if (bad4) {
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (!__builtin_amdgcn_classf(x[i], 0x1F8)) x[i] = 0.0f;
                        vs[e * GL + gl] = x;
                        found = true;
                    }
                }
                if (__any(found) && lane == 0) nf_tile[kpar] = tw + 1;
            }
            lds_barrier();  // the sanitized tile and the flag are visible to the group
            fix = !(live && whole) && nf_tile[kpar] == tw + 1;
        }

        // O^T += V^T . P^T over the tile's 16 keys (k-step r: keys 4g + r),
        // operand (r, U) read from LDS one step ahead as the K operands are.
        if (live) {
            constexpr int NPV = 4 * NV;
            f32x4 vc[2];
            auto read_v = [&](int idx, f32x4 &dst) {
                const int r = idx / NV, U = idx % NV;
                dst = vb[kpar * TILE_F4 + (4 * g + r) * (D / 4) + d0 / 4 + 16 * U + c];
            };
            read_v(0, vc[0]);
#pragma unroll
            for (int idx = 0; idx < NPV; ++idx) {
                if (idx + 1 < NPV) read_v(idx + 1, vc[(idx + 1) & 1]);
                const int r = idx / NV, U = idx % NV;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    o[4 * U + i] = __builtin_amdgcn_mfma_f32_16x16x4f32(vc[idx & 1][i], pr[r], o[4 * U + i], 0, 0, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
#pragma unroll
            for (int idx = 0; idx < NPV; ++idx) {
                if (idx + 1 < NPV) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);                      // MFMA
            }
        }

        if (fix) {
            // Key k = 4kq + r of the tile: its weight for this lane's row c is
            // pr[r] of lane (kq, c); it is attended iff k <= rel and (no
            // window or k > rel - W).  O^T tile 4U + i, row 4g + r2 of this
            // lane is dim d0 + 64U + 16g + 4r2 + i of row c.
            const int64_t rel = pos - 16LL * tw;
            for (int kq = 0; kq < 4; ++kq) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int k = 4 * kq + r;
                    const float pk = __shfl(pr[r], kq * 16 + c);
                    if (!(live && k <= rel && (win == 0 || k > rel - win))) continue;
                    const uint32_t roff = (uint32_t)(((16LL * tw + k - block_lo) * stride + d0 + 16 * g) * 4);
#pragma unroll
                    for (int U = 0; U < NV; ++U)
#pragma unroll
                        for (int r2 = 0; r2 < 4; ++r2) {
                            const f32x4 vv = __builtin_bit_cast(
                                f32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, roff + (64 * U + 4 * r2) * 4, 0, 0));
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                if (!__builtin_amdgcn_classf(vv[i], 0x1F8)) o[4 * U + i][r2] += pk * vv[i];
                            // One load at a time: this path is rare, and hoisting
                            // its loads would cost the hot loop registers.
                            __builtin_amdgcn_sched_barrier(0);
                        }
                }
            }
        }
    };
    if constexpr (SPLIT16) {
        // Software pipeline over steps s of TPS tiles: K(s) in k[s % 2], V(s)
        // in v[s % 2], K loaded one step ahead of V.  Iteration s, after the
        // step's one barrier: the first half of step s+1's score MFMAs (with
        // half of the next loads), and beside them step s's full scores (the
        // pair's partials, written at the end of iteration s-1), mask and
        // row maximum, which those MFMAs do not wait for; the lazy rescale;
        // the second half of the score MFMAs with step s's weights (VALU)
        // between them; P.V(s); last, step s+1's partial scores go to the
        // exchange slot that the next barrier publishes.  So the matrix pipe
        // starts right after the barrier instead of after the softmax's
        // dependent chain, and the two waves of a SIMD (the pair, at
        // D = 512) do not stop for a mid-step exchange.
        const int nsteps = (u.t_hi - u.t_lo + TPS - 1) / TPS;
        auto tile_at = [&](int st, int j) {
            const int tt = u.t_lo + TPS * st + j;
            return tt < u.t_hi ? tt : u.t_hi - 1;  // past the end: the last tile again (unread)
        };
        // Partial S^T of a step's tile for this wave's group over its dims,
        // from kt (that step's K buffer), one 32-dim chunk at a time; the
        // step's NL tile-part loads, load(i), are spread over the chunks.  A
        // stale tile (past the unit) is computed anyway, from the finite
        // values its buffer holds, and masked whole.
        constexpr int NL = 2 * PER_THREAD * TPS;  // tile-part loads per step
        static_assert(NL % NU == 0 || NU % NL == 0, "loads spread over the chunks");
        auto read_k = [&](const f32x4 *kt, int uu, f32x4(&dst)[2]) {
            const int ug = d0 / 32 + uu;
            dst[0] = kt[(ug * 2 + 0) * 64 + lane];
            dst[1] = kt[(ug * 2 + 1) * 64 + lane];
        };
        // Chunk uu: its three MFMAs into a0..a2 from the K operands in
        // kc[uu & 1], after chunk uu+1's operands are read into the other slot
        // and the chunk's share of the loads is issued.
        auto score_chunk = [&](const f32x4 *kt, int uu, f32x4(&kc)[2][2], f32x4 &a0, f32x4 &a1, f32x4 &a2,
                               auto &&load) {
            if (uu + 1 < NU) read_k(kt, uu + 1, kc[(uu + 1) & 1]);
            if constexpr (NL >= NU) {
#pragma unroll
                for (int i = uu * (NL / NU); i < (uu + 1) * (NL / NU); ++i) load(i);
            } else if (uu % (NU / NL) == 0) {
                load(uu / (NU / NL));
            }
            const f16x8 kh = __builtin_bit_cast(f16x8, kc[uu & 1][0]);
            const f16x8 kl = __builtin_bit_cast(f16x8, kc[uu & 1][1]);
            a0 = split_mfma(kh, qh[uu], a0);
            a1 = split_mfma(kh, ql[uu], a1);
            a2 = split_mfma(kl, qh[uu], a2);
        };
        // All chunks of one tile (the unit's first step).
        auto part_scores = [&](const f32x4 *kb_, auto &&load) -> f32x4 {
            const f32x4 *kt = kb_ + kpar * TILE_F4;
            f32x4 a0 = {0.0f, 0.0f, 0.0f, 0.0f}, a1 = a0, a2 = a0;
            f32x4 kc[2][2];
            read_k(kt, 0, kc[0]);
#pragma unroll
            for (int uu = 0; uu < NU; ++uu) score_chunk(kt, uu, kc, a0, a1, a2, load);
            return a0 + (a1 + a2) * kLoUnscale;
        };
        // K(0), V(0) and K(1) were issued at the unit's start.
        __builtin_amdgcn_s_waitcnt(kVmcntZero);
        __syncthreads();  // K(0), V(0), K(1) have landed
        f32x4 sc_next;    // D = 256: the wave's own scores of the next step
        {
            const f32x4 part = part_scores(lds_k0, [](int) {});
            if constexpr (S::SPLIT == 2)
                lds_s0[wave][lane] = part;
            else
                sc_next = part;
        }
        // Iteration st: kn1 holds K(st+1), kfree receives K(st+2), vcur holds
        // V(st), vnext receives V(st+1); xr holds step st's partials, xw
        // receives step st+1's.
        auto iter = [&](int st, const f32x4 *kn1, f32x4 *kfree, const f32x4 *vcur, f32x4 *vnext, f32x4(*xr)[64],
                        f32x4(*xw)[64]) {
            __builtin_amdgcn_s_waitcnt(kVmcntZero);
            __syncthreads();  // K(st+1), V(st) and step st's partials are in; k(st), v(st-1) are free
            auto load = [&](int i) {
                const int j = i / (2 * PER_THREAD), part = i % (2 * PER_THREAD);
                if (part & 1)
                    issue_part(tile_at(st + 1, j), part, nullptr, vnext + j * TILE_F4);
                else
                    issue_part(tile_at(st + 2, j), part, kfree + j * TILE_F4, nullptr);
            };
            // First half of step st+1's score MFMAs, with step st's full
            // scores, mask and row maximum found beside them (none of which
            // they depend on).
            const f32x4 *kt = kn1 + kpar * TILE_F4;
            f32x4 a0 = {0.0f, 0.0f, 0.0f, 0.0f}, a1 = a0, a2 = a0;
            f32x4 kc[2][2];
            read_k(kt, 0, kc[0]);
            f32x4 sc;
            if constexpr (S::SPLIT == 2)
                sc = xr[rg][lane] + xr[rg + kWaves][lane];  // half 0 + half 1, in that order
            else
                sc = sc_next;
            constexpr int H = NU / 2;
#pragma unroll
            for (int uu = 0; uu < H; ++uu) score_chunk(kt, uu, kc, a0, a1, a2, load);
            const int tw = u.t_lo + TPS * st + kpar;
            const bool live = S::KSPLIT == 1 || tw < u.t_hi;
            // Key 4g + r of the tile is kept iff the tile is live and every
            // row attends it whole, or key <= pos and, with a window,
            // key > pos - W (branch-free).
            const bool ex = exact(tw);
            const int64_t rel = pos - 16LL * tw;
            const int64_t rlo = rel - win;
            float sv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int kr = 4 * g + r;
                const bool keep = live & (ex | ((kr <= rel) & ((win == 0) | (kr > rlo))));
                sv[r] = keep ? sc[r] * p.scale : -INFINITY;  // x * 1 == x
            }
            const float mx = __builtin_elementwise_maximum(__builtin_elementwise_maximum(sv[0], sv[1]),
                                                           __builtin_elementwise_maximum(sv[2], sv[3]));
            bad |= __builtin_amdgcn_classf(mx, 0x203);  // signalling/quiet NaN, +inf
            const float mt = rows_max(mx);
            // Order: chunk 0's K reads (and the partials); per chunk the next
            // chunk's K reads, its share of the loads, its three MFMAs and
            // some of the VALU above.
            __builtin_amdgcn_sched_group_barrier(0x100, S::SPLIT == 2 ? 4 : 2, 0);  // DS read
#pragma unroll
            for (int uu = 0; uu < H; ++uu) {
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);                        // DS read
                __builtin_amdgcn_sched_group_barrier(0x010, NL >= NU ? NL / NU : 1, 0);  // VMEM
                __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);                        // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);                        // VALU
            }
            if (__any(mt > m + kRescaleSlackSplit)) {
                const float m_new = fmaxf(m, mt);
                const float alpha = (m_new == -INFINITY) ? 1.0f : exp2_fast((m - m_new) * kLog2e);
                l *= alpha;
                m = m_new;
#pragma unroll
                for (int i = 0; i < NT; ++i) o[i] *= alpha;
            }
            // Second half of the score MFMAs, with step st's weights.
#pragma unroll
            for (int uu = H; uu < NU; ++uu) score_chunk(kt, uu, kc, a0, a1, a2, load);
            const f32x4 part = a0 + (a1 + a2) * kLoUnscale;
            float pr[4];
#pragma unroll
            for (int r = 0; r < 4; ++r)
                pr[r] = (m == -INFINITY) ? 0.0f : exp2_fast((sv[r] - m) * kLog2e + (float)kPScale);
            l += (pr[0] + pr[1]) + (pr[2] + pr[3]);
            f16x8 ph, pl;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const _Float16 h = (_Float16)pr[r];
                const _Float16 lo = (_Float16)(pr[r] - (float)h);
                ph[r] = h;
                ph[4 + r] = h;
                pl[r] = lo;
                pl[4 + r] = lo;
            }
            // The same order for the second half, with the weights' VALU.
#pragma unroll
            for (int uu = H; uu < NU; ++uu) {
                if (uu + 1 < NU) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);       // DS read
                __builtin_amdgcn_sched_group_barrier(0x010, NL >= NU ? NL / NU : 1, 0);  // VMEM
                __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);                        // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);                        // VALU
            }
            // P.V is scheduled as a region of its own: scheduled together
            // with the score MFMAs, the first of the two unrolled iterations
            // read each V operand just before its MFMAs and waited for it.
            __builtin_amdgcn_sched_barrier(0);
            // P.V(st); a stale tile's weights are 0 and its V is finite.
            static_assert(NT % 2 == 0, "O^T tiles in pairs");
            const f32x4 *vt = vcur + kpar * TILE_F4 + (d0 / 16) * 64 + lane;
            f32x4 vc[2][2];
            vc[0][0] = vt[0];
            vc[0][1] = vt[64];
#pragma unroll
            for (int T = 0; T < NT; T += 2) {
                const int sl = (T / 2) & 1;
                if (T + 2 < NT) {
                    vc[sl ^ 1][0] = vt[(T + 2) * 64];
                    vc[sl ^ 1][1] = vt[(T + 3) * 64];
                }
                const f16x8 a0v = __builtin_bit_cast(f16x8, vc[sl][0]);
                const f16x8 a1v = __builtin_bit_cast(f16x8, vc[sl][1]);
                o[T] = split_mfma(a0v, ph, o[T]);
                o[T + 1] = split_mfma(a1v, ph, o[T + 1]);
                o[T] = split_mfma(a0v, pl, o[T]);
                o[T + 1] = split_mfma(a1v, pl, o[T + 1]);
            }
            if constexpr (S::SPLIT == 2)
                xw[wave][lane] = part;
            else
                sc_next = part;
            // P.V: two V reads per four MFMAs.
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
#pragma unroll
            for (int T = 0; T < NT; T += 2) {
                if (T + 2 < NT) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);                   // MFMA
            }
            __builtin_amdgcn_sched_barrier(0);  // the next iteration's barrier stays after this P.V
        };
        int st = 0;
        for (; st + 1 < nsteps; st += 2) {
            iter(st, lds_k1, lds_k0, lds_v0, lds_v1, lds_s0, lds_s1);
            iter(st + 1, lds_k0, lds_k1, lds_v1, lds_v0, lds_s1, lds_s0);
        }
        if (st < nsteps) iter(st, lds_k1, lds_k0, lds_v0, lds_v1, lds_s0, lds_s1);
    } else {
#pragma unroll
        for (int j = 0; j < TPS; ++j)
            issue_tile(u.t_lo + j < u.t_hi ? u.t_lo + j : u.t_hi - 1, lds_k0 + j * TILE_F4, lds_v0 + j * TILE_F4);
        int t = u.t_lo;
        for (; t + TPS < u.t_hi; t += 2 * TPS) {
            step(t, lds_k0, lds_v0, lds_s0, lds_k1, lds_v1);
            step(t + TPS, lds_k1, lds_v1, lds_s1, lds_k0, lds_v0);
        }
        if (t < u.t_hi) step(t, lds_k0, lds_v0, lds_s0, lds_k1, lds_v1);
    }

    if (__any(bad && row_valid) && lane == 0) atomicOr(p.status, kStatusNonFinite);
    __builtin_amdgcn_s_waitcnt(kVmcntZero);  // the last step's spare loads have landed
    if constexpr (S::KSPLIT == 2) {
        // The odd-tile group hands its (m, l, O) to the even-tile group of
        // the same rows, which combines them as two disjoint key sets.
        static_assert(kWaves * NT * 64 <= 2 * TPS * TILE_F4, "the hand-over fits two tile arrays");
        __syncthreads();  // every wave is done with the tile buffers (no tile load is in flight)
        f32x4 *xo = (rg < 2 ? lds_k0 : lds_v0) + (rg & 1) * (NT * 64);
        float2 *xm = (float2 *)lds_k1 + rg * 64;
        if (kpar == 1) {
#pragma unroll
            for (int i = 0; i < NT; ++i) xo[i * 64 + lane] = o[i];
            xm[lane] = float2{m, l};
        }
        __syncthreads();
        if (kpar == 0) {
            const float2 ml = xm[lane];
            const float mm = fmaxf(m, ml.x);
            const float a = (m == -INFINITY) ? 0.0f : exp2_fast((m - mm) * kLog2e);
            const float b = (ml.x == -INFINITY) ? 0.0f : exp2_fast((ml.x - mm) * kLog2e);
#pragma unroll
            for (int i = 0; i < NT; ++i) o[i] = a * o[i] + b * xo[i * 64 + lane];
            l = a * l + b * ml.y;
            m = mm;
        }
        __syncthreads();  // the hand-over buffers are free again
    }
    const float lt = rows_sum(l);
    const bool result = S::KSPLIT == 1 || wave < S::RWAVES;  // the waves holding the combined rows
    if (u.slot >= 0) {  // partial of a multi-unit block, in the accumulator layout
        const int64_t sl = (int64_t)u.slot * gridDim.y + kvh;
        f32x4 *po = (f32x4 *)(p.part_o + sl * (kWaves * kRowsPerWave * D));
        if (result) {
#pragma unroll
            for (int i = 0; i < NT; ++i) po[(wave * NT + i) * 64 + lane] = o[i];
            // The split form's weights carry 2^kPScale: fold it into m.
            const float mr = (SPLIT16 && m != -INFINITY) ? m - kPScaleNat : m;
            if (g == 0 && half == 0) p.part_ml[sl * (kWaves * kRowsPerWave) + rg * kRowsPerWave + c] = float2{mr, lt};
        }
        return true;
    }
    // Single unit: normalise and write row-major through LDS (coalesced).
    __syncthreads();  // every wave is done with the tile buffers (no tile load is in flight)
    // RWAVES/4 waves' rows per tile array.
    constexpr int WPA = S::RWAVES / 4;
    static_assert(WPA * kRowsPerWave * DH <= TPS * TILE_F4 * 4 && S::RWAVES % 4 == 0, "transpose fits the tile buffers");
    const int ta = (result ? wave : 0) / WPA;
    f32x4 *tb = ta == 0 ? lds_k0 : ta == 1 ? lds_v0 : ta == 2 ? lds_k1 : lds_v1;
    float *tr = (float *)tb + (wave % WPA) * (kRowsPerWave * DH);
    const float inv = 1.0f / lt;
    if (result) {
#pragma unroll
        for (int U = 0; U < NV; ++U)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) tr[c * DH + 64 * U + 4 * (4 * g + r) + i] = o[4 * U + i][r] * inv;
    }
    __syncthreads();
    if (!result) return true;
#pragma unroll
    for (int e = 0; e < kRowsPerWave * DH / 4 / 64; ++e) {
        const int f = lane + 64 * e;
        const int row = f / (DH / 4), c4 = f % (DH / 4);
        const int64_t rpos = P0 + kPosPerWave * rg + (row >> 3);
        if (rpos > last_pos) continue;
        float *orow = p.out + ((rpos - p.pos0) * p.n_heads + kvh * kGroup + (row & 7)) * D + d0;
        *(f32x4 *)(orow + 4 * c4) = *(const f32x4 *)(tr + row * DH + 4 * c4);
    }
    return true;
}

// A workgroup runs its units in turn (the host's schedule), each in the
// split-f16 form when the call has planes and the unit's inputs allow it,
// else with f32 MFMAs.
template <int D>
__global__ __launch_bounds__(PrefillShape<D>::THREADS, 1) void prefill_kernel(PrefillK p) {
    using S = PrefillShape<D>;
    constexpr int TILE_F4 = 16 * D / 4;
    // Double-buffered K and V tiles (TPS per buffer, tile j at j*TILE_F4) and
    // partial S^T of the D halves, each buffer its own array: the tiles being
    // loaded and the tiles being read are then distinct objects, so the
    // compiler need not wait for the former's loads before reading the
    // latter.  The epilogue reuses the four tile arrays.
    __shared__ f32x4 lds_k0[S::TPS * TILE_F4], lds_v0[S::TPS * TILE_F4], lds_k1[S::TPS * TILE_F4],
        lds_v1[S::TPS * TILE_F4];
    __shared__ f32x4 lds_s0[S::WAVES][64], lds_s1[S::WAVES][64];
    // Per wave group: 1 + the index of the last edge tile whose V held a
    // non-finite value (see the unit's step()); 0 = none.  Cleared here and
    // by each f32-form unit, so that leftover LDS contents never trigger a
    // fix-up pass; the unit's first barrier orders the clear before any
    // read.
    __shared__ int nf_tile[S::KSPLIT];
    __shared__ int vote[S::WAVES];
    if (threadIdx.x < S::KSPLIT) nf_tile[threadIdx.x] = 0;
    const PrefillLds L{lds_k0, lds_v0, lds_k1, lds_v1, lds_s0, lds_s1, nf_tile, vote};
    // Workgroups go to the 8 XCDs round-robin (workgroup w to XCD w % 8).
    // Bin b runs on XCD b / (bins / 8), so that consecutive bins -- the
    // schedule lists a sliding layer's blocks in position order -- share
    // one XCD's L2 and the window tiles they have in common.
    const int gx = gridDim.x;
    const int bin = gx % 8 == 0 ? (int)(blockIdx.x % 8) * (gx / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
    const int first = p.bin_start[bin], end = p.bin_start[bin + 1];
    for (int i = first; i < end; ++i) {
        // The previous unit's waves are done with the tile buffers (its
        // spare tile loads landed before its epilogue).
        if (i > first) __syncthreads();
        const PrefillUnit u = p.units[i];
        if (p.planes != nullptr && prefill_unit<D, true>(p, u, L)) continue;
        if (p.planes != nullptr) __syncthreads();  // the declined split form's tiles have landed
        prefill_unit<D, false>(p, u, L);
    }
}

// Combines the NU units of one position block (and KV head) in key order for
// the rows and dims of one producing wavefront (blockIdx.z), then writes
// them row-major through LDS.  The per-unit loads of an element are
// unrolled so that they are all in flight together; the unit count is a
// template argument (the kernel switches on the block's count), so each
// thread issues exactly its NU loads per element.
template <int D, int NU>
__device__ __forceinline__ void merge_units(const PrefillK &p, const PrefillBlockInfo &bi, float (*w)[kRowsPerWave],
                                            float *Linv, float *tr) {
    using S = PrefillShape<D>;
    constexpr int DH = S::DH;
    constexpr int NT = DH / 16;
    const int kvh = blockIdx.y, wave = blockIdx.z;
    const int rg = wave % kWaves, half = wave / kWaves;
    const int tid = threadIdx.x;
    // Every load first (one memory round trip): the wave's (m, l) per row and
    // unit, and this thread's partial vectors.
    constexpr int NE = NT * 64 / 256;  // vectors per thread
    static_assert(NT * 64 % 256 == 0, "whole vectors per thread");
    const int ml_row = rg * kRowsPerWave + (tid & (kRowsPerWave - 1));
    float2 ml[NU];
#pragma unroll
    for (int j = 0; j < NU; ++j) ml[j] = p.part_ml[((int64_t)(bi.first_slot + j) * gridDim.y + kvh) * 64 + ml_row];
    const int64_t slot_stride = (int64_t)gridDim.y * kWaves * kRowsPerWave * D / 4;  // f32x4
    const f32x4 *base = (const f32x4 *)p.part_o +
                        ((int64_t)bi.first_slot * gridDim.y + kvh) * (kWaves * kRowsPerWave * D / 4) +
                        (int64_t)wave * NT * 64;
    f32x4 v[NE][NU];
#pragma unroll
    for (int k = 0; k < NE; ++k)
#pragma unroll
        for (int j = 0; j < NU; ++j) v[k][j] = base[j * slot_stride + tid + 256 * k];
    __builtin_amdgcn_sched_barrier(0);  // no wait before every load above is issued
    if (tid < kRowsPerWave) {
        float M = -INFINITY;
#pragma unroll
        for (int j = 0; j < NU; ++j) M = fmaxf(M, ml[j].x);
        float L = 0.0f;
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            const float wj = ml[j].x == -INFINITY ? 0.0f : exp2_fast((ml[j].x - M) * kLog2e);
            L += wj * ml[j].y;
            w[j][tid] = wj;
        }
        Linv[tid] = 1.0f / L;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < NE; ++k) {
        const int e = tid + 256 * k;
        const int lane = e & 63, tile = e >> 6;
        const int g = lane >> 4, c = lane & 15;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < NU; ++j) acc += w[j][c] * v[k][j];
        const int U = tile >> 2, i = tile & 3;
        const float inv = Linv[c];
#pragma unroll
        for (int r = 0; r < 4; ++r) tr[c * DH + 64 * U + 4 * (4 * g + r) + i] = acc[r] * inv;
    }
    __syncthreads();
    const int64_t P0 = p.pos0 + (int64_t)kPosPerBlock * blockIdx.x;
    const int64_t last_pos = p.pos0 + p.N - 1;
    for (int f = tid; f < kRowsPerWave * DH / 4; f += 256) {
        const int row = f / (DH / 4), c4 = f % (DH / 4);
        const int64_t rpos = P0 + kPosPerWave * rg + (row >> 3);
        if (rpos <= last_pos) {
            float *orow = p.out + ((rpos - p.pos0) * p.n_heads + kvh * kGroup + (row & 7)) * D + half * DH;
            *(f32x4 *)(orow + 4 * c4) = *(const f32x4 *)(tr + row * DH + 4 * c4);
        }
    }
}

template <int D>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillK p) {
    __shared__ float w[kPrefillMaxUnitsDev][kRowsPerWave];
    __shared__ float Linv[kRowsPerWave];
    __shared__ float tr[kRowsPerWave * PrefillShape<D>::DH];
    const PrefillBlockInfo bi = p.blocks[blockIdx.x];
    static_assert(kPrefillMaxUnitsDev == 8, "one case per unit count");
    switch (bi.n_units) {  // uniform; 0 or 1 unit: nothing to merge
        case 2: merge_units<D, 2>(p, bi, w, Linv, tr); break;
        case 3: merge_units<D, 3>(p, bi, w, Linv, tr); break;
        case 4: merge_units<D, 4>(p, bi, w, Linv, tr); break;
        case 5: merge_units<D, 5>(p, bi, w, Linv, tr); break;
        case 6: merge_units<D, 6>(p, bi, w, Linv, tr); break;
        case 7: merge_units<D, 7>(p, bi, w, Linv, tr); break;
        case 8: merge_units<D, 8>(p, bi, w, Linv, tr); break;
        default: break;
    }
}

constexpr int kPrefillMaxUnits = kPrefillMaxUnitsDev;  // per position block

// A unit table in device memory, for one prefill shape.
struct PrefillPlan {
    int64_t pos0 = -1, N = -1, window = -1;
    int head_dim = 0, n_kv_heads = 0;
    int n_units = 0, n_bins = 0, n_blocks = 0, n_slots = 0;
    PrefillUnit *units = nullptr;
    int *bin_start = nullptr;
    PrefillBlockInfo *blocks = nullptr;
    uint64_t last_use = 0;
};

// The context's tables for the last few shapes (a layer-by-layer prompt
// alternates sliding and global shapes).  A cached table is never written
// again, so kernels still in flight on any stream keep reading a valid
// table; only evicting one waits for the device.
constexpr size_t kPrefillPlans = 8;
struct PrefillPlans {
    std::vector<PrefillPlan> plans;
    uint64_t tick = 0;
};

void free_plan(PrefillPlan &pl) {
    if (pl.units) (void)hipFree(pl.units);
    if (pl.bin_start) (void)hipFree(pl.bin_start);
    if (pl.blocks) (void)hipFree(pl.blocks);
    pl.units = nullptr;
    pl.bin_start = nullptr;
    pl.blocks = nullptr;
}

}  // namespace

// The tables live with the context (one per device; prefill calls on one
// context are issued from one host thread).
static PrefillPlans &plans_of(g4_ctx *ctx) {
    if (!ctx->prefill_plan) ctx->prefill_plan = new PrefillPlans();
    return *static_cast<PrefillPlans *>(ctx->prefill_plan);
}

void release_prefill_plan(g4_ctx *ctx) {
    if (!ctx->prefill_plan) return;
    auto *ps = static_cast<PrefillPlans *>(ctx->prefill_plan);
    for (auto &pl : ps->plans) free_plan(pl);
    delete ps;
    ctx->prefill_plan = nullptr;
}

// Work schedule of a prefill shape.  A unit is the tiles [t_lo, t_hi) of one
// position block; each workgroup runs a list of units (a bin) one after the
// other, and the grid is at most one workgroup per CU per KV head, so every
// bin starts at once and the host's assignment is the schedule: no
// workgroup waits for the hardware to hand it a CU, and the split of the
// key ranges is chosen knowing where each piece runs.
//
// Cost model, in tiles (one 16-key tile of 64 query rows): a unit costs its
// tiles plus kUnitCost (loading Q, filling the tile pipeline, writing O or
// the partial); blocks split into several units add a merge kernel of
// kMergeBase + kMergePerPartial per partial.  Measured on MI355X at
// d = 512: 4.9 us per tile, 9.1 us per unit (the fit over a 2048-token
// causal prompt's 480 units), merge 17 us for 384 partials.
constexpr double kUnitCost = 1.9;
constexpr double kMergePerPartial = 0.009;
constexpr int kMinUnitTiles = 4;  // a split leaves no piece shorter (unless the block is)

using Piece = std::array<int, 3>;  // block, t_lo, t_hi
using Bins = std::vector<std::vector<Piece>>;

static double merge_cost(int partials, int head_dim) {
    if (partials == 0) return 0.0;
    return (head_dim == 512 ? 0.6 : 1.2) + kMergePerPartial * partials;
}

// Makespan plus merge cost; nullopt-like -1 when a block has more pieces
// than the merge kernel combines.
static double schedule_cost(const Bins &bins, int n_blocks, int head_dim) {
    std::vector<int> pieces(n_blocks, 0);
    double makespan = 0.0;
    for (auto &bin : bins) {
        double load = 0.0;
        for (auto &pc : bin) {
            load += pc[2] - pc[1] + kUnitCost;
            ++pieces[pc[0]];
        }
        makespan = std::max(makespan, load);
    }
    int partials = 0;
    for (int n : pieces) {
        if (n > kPrefillMaxUnits) return -1.0;
        if (n > 1) partials += n;
    }
    return makespan + merge_cost(partials, head_dim);
}

// Fixed-length units (each block cut into ceil(tiles / ut) near-equal
// pieces) assigned heaviest first to the least loaded bin.
static Bins lpt_bins(const std::vector<std::pair<int, int>> &bt, int ut, int n_bins) {
    std::vector<Piece> units;
    for (int b = 0; b < (int)bt.size(); ++b) {
        const int t_lo = bt[b].first, tiles = bt[b].second - t_lo, nu = (tiles + ut - 1) / ut;
        for (int j = 0; j < nu; ++j) units.push_back({b, t_lo + j * tiles / nu, t_lo + (j + 1) * tiles / nu});
    }
    std::stable_sort(units.begin(), units.end(),
                     [](const Piece &x, const Piece &y) { return x[2] - x[1] > y[2] - y[1]; });
    Bins bins((size_t)n_bins);
    using Load = std::pair<double, int>;
    std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
    for (int i = 0; i < n_bins; ++i) heap.push({0.0, i});
    for (auto &u : units) {
        Load l = heap.top();
        heap.pop();
        bins[l.second].push_back(u);
        heap.push({l.first + (u[2] - u[1]) + kUnitCost, l.second});
    }
    return bins;
}

// Stream-K packing at capacity `cap`: blocks in the order largest,
// smallest, second largest, second smallest, ... fill the bins in turn; a
// block that does not fit is cut at the capacity and continues in the next
// bin.  False when more than n_bins bins are needed.
static bool stream_bins(const std::vector<std::pair<int, int>> &bt, double cap, int n_bins, Bins &bins) {
    std::vector<int> order(bt.size());
    for (size_t i = 0; i < order.size(); ++i) order[i] = (int)i;
    std::stable_sort(order.begin(), order.end(), [&](int x, int y) {
        return bt[x].second - bt[x].first > bt[y].second - bt[y].first;
    });
    std::vector<int> seq;
    for (int i = 0, j = (int)order.size() - 1; i <= j;) {
        seq.push_back(order[i++]);
        if (i <= j) seq.push_back(order[j--]);
    }
    bins.assign(1, {});
    double load = 0.0;
    for (int b : seq) {
        int lo = bt[b].first;
        const int hi = bt[b].second;
        while (lo < hi) {
            const int rem = hi - lo;
            const double room = cap - load - kUnitCost;
            const bool empty = bins.back().empty();
            // An empty bin takes any remainder up to a minimum piece whole.
            if (rem <= room || (empty && rem <= kMinUnitTiles)) {
                bins.back().push_back({b, lo, hi});
                load += rem + kUnitCost;
                break;
            }
            // The tiles that fit, leaving at least a minimum piece behind
            // (rem > kMinUnitTiles here when the bin is empty, so an empty
            // bin always takes at least one tile and every pass progresses).
            int take = std::max(0, (int)room);
            if (rem - take < kMinUnitTiles) take = rem - kMinUnitTiles;
            if (empty) take = std::max(take, 1);
            if (take >= kMinUnitTiles || (empty && take >= 1)) {
                bins.back().push_back({b, lo, lo + take});
                lo += take;
            }
            if (lo < hi) {
                if ((int)bins.size() == n_bins) return false;
                bins.push_back({});
                load = 0.0;
            }
        }
    }
    return true;
}

// The cheaper of the two schedules (by the cost model): fixed-length units
// placed by LPT (16 .. 128 tiles, or longer when a block needs it to stay
// within kPrefillMaxUnits units), or stream-K packing at the smallest
// feasible capacity or a little above.  Stream-K wins on causal prompts
// (every CU gets the same number of tiles, with about one split per CU);
// LPT wins where few long blocks each need many pieces.
static int build_schedule(const std::vector<std::pair<int, int>> &bt, int n_bins, int head_dim, Bins &best) {
    int max_tiles = 1;
    long long total = 0;
    for (auto &x : bt) {
        max_tiles = std::max(max_tiles, x.second - x.first);
        total += x.second - x.first;
    }
    double best_cost = -1.0;
    auto consider = [&](Bins &&bins) {
        const double cost = schedule_cost(bins, (int)bt.size(), head_dim);
        if (cost >= 0.0 && (best_cost < 0.0 || cost < best_cost)) {
            best_cost = cost;
            best = std::move(bins);
        }
    };
    const int ut_hi = std::max(128, ((max_tiles + kPrefillMaxUnits - 1) / kPrefillMaxUnits + 7) / 8 * 8);
    for (int ut = ut_hi; ut >= 16; ut -= 8) {
        if ((max_tiles + ut - 1) / ut > kPrefillMaxUnits) break;
        consider(lpt_bins(bt, ut, n_bins));
    }
    double lo = (double)total / n_bins + kUnitCost, hi = lo + max_tiles + 2 * kUnitCost;
    Bins bins;
    if (stream_bins(bt, hi, n_bins, bins)) {
        while (hi - lo > 0.25) {
            const double mid = 0.5 * (lo + hi);
            if (stream_bins(bt, mid, n_bins, bins))
                hi = mid;
            else
                lo = mid;
        }
        for (int k = 0; k < 12; ++k)
            if (stream_bins(bt, hi + 0.5 * k, n_bins, bins)) consider(std::move(bins));
    }
    return best_cost < 0.0 ? -1 : 0;
}

// The unit table, workgroup ranges and block table of a schedule; checks
// that every block's pieces tile its range exactly.
static int schedule_tables(const std::vector<std::pair<int, int>> &bt, Bins &bins, std::vector<PrefillUnit> &units,
                           std::vector<int> &bin_start, std::vector<PrefillBlockInfo> &blocks, int &n_slots) {
    const int n_blocks = (int)bt.size();
    bins.erase(std::remove_if(bins.begin(), bins.end(), [](const std::vector<Piece> &x) { return x.empty(); }),
               bins.end());
    std::stable_sort(bins.begin(), bins.end(), [](const std::vector<Piece> &x, const std::vector<Piece> &y) {
        int lx = 0, ly = 0;
        for (auto &pc : x) lx += pc[2] - pc[1];
        for (auto &pc : y) ly += pc[2] - pc[1];
        return lx > ly;
    });
    std::vector<std::vector<std::pair<int, int>>> of_block(n_blocks);  // (t_lo, unit index)
    units.clear();
    bin_start.assign(1, 0);
    for (auto &bin : bins) {
        for (auto &pc : bin) {
            of_block[pc[0]].push_back({pc[1], (int)units.size()});
            units.push_back({pc[0], pc[1], pc[2], -1});
        }
        bin_start.push_back((int)units.size());
    }
    blocks.assign(n_blocks, {0, 0});
    n_slots = 0;
    for (int b = 0; b < n_blocks; ++b) {
        auto &v = of_block[b];
        std::sort(v.begin(), v.end());
        int t = bt[b].first;
        for (auto &x : v) {
            const PrefillUnit &u = units[x.second];
            if (u.t_lo != t || u.t_hi <= u.t_lo) return set_error(G4_ERR_COMPUTE, "prefill schedule does not tile a block");
            t = u.t_hi;
        }
        if (t != bt[b].second || v.empty() || (int)v.size() > kPrefillMaxUnits)
            return set_error(G4_ERR_COMPUTE, "prefill schedule does not tile a block");
        blocks[b] = {v.size() > 1 ? n_slots : 0, (int)v.size()};
        if (v.size() > 1)
            for (auto &x : v) units[x.second].slot = n_slots++;
    }
    return G4_OK;
}

// [t_lo, t_hi) tiles of each position block of a prefill shape.
static std::vector<std::pair<int, int>> block_tile_ranges(int64_t pos0, int64_t N, int64_t window) {
    const int n_blocks = (int)((N + kPosPerBlock - 1) / kPosPerBlock);
    const int64_t last_pos = pos0 + N - 1;
    std::vector<std::pair<int, int>> bt(n_blocks);
    for (int b = 0; b < n_blocks; ++b) {
        const int64_t P0 = pos0 + (int64_t)kPosPerBlock * b;
        const int64_t P1 = std::min<int64_t>(P0 + kPosPerBlock - 1, last_pos);
        const int64_t k_lo = (window > 0 && P0 + 1 > window) ? P0 + 1 - window : 0;
        bt[b] = {(int)(k_lo / 16), (int)(P1 / 16 + 1)};
    }
    return bt;
}

static int bins_for(int num_cus, int n_kv_heads) { return std::max(1, num_cus / std::max(1, n_kv_heads)); }

// The schedule tables of a's shape: cached, or built and uploaded
// (synchronously: graph capture needs an earlier call with the same shape).
static int plan_for(g4_ctx *ctx, const PrefillArgs &a, const PrefillPlan **out) {
    PrefillPlans &ps = plans_of(ctx);
    ++ps.tick;
    for (auto &pl : ps.plans)
        if (pl.pos0 == a.pos0 && pl.N == a.N && pl.window == a.window && pl.head_dim == a.head_dim &&
            pl.n_kv_heads == a.n_kv_heads) {
            pl.last_use = ps.tick;
            *out = &pl;
            return G4_OK;
        }
    const std::vector<std::pair<int, int>> bt = block_tile_ranges(a.pos0, a.N, a.window);
    Bins bins;
    if (build_schedule(bt, bins_for(ctx->num_cus, a.n_kv_heads), a.head_dim, bins) != 0)
        return set_error(G4_ERR_COMPUTE, "prefill key range too long for one call");
    std::vector<PrefillUnit> units;
    std::vector<int> bin_start;
    std::vector<PrefillBlockInfo> blocks;
    int n_slots = 0;
    int rc = schedule_tables(bt, bins, units, bin_start, blocks, n_slots);
    if (rc != G4_OK) return rc;
    PrefillPlan pl;
    pl.pos0 = a.pos0;
    pl.N = a.N;
    pl.window = a.window;
    pl.head_dim = a.head_dim;
    pl.n_kv_heads = a.n_kv_heads;
    pl.n_units = (int)units.size();
    pl.n_bins = (int)bin_start.size() - 1;
    pl.n_blocks = (int)blocks.size();
    pl.n_slots = n_slots;
    pl.last_use = ps.tick;
    hipError_t e = hipMalloc(&pl.units, units.size() * sizeof(PrefillUnit));
    if (e == hipSuccess) e = hipMalloc(&pl.bin_start, bin_start.size() * sizeof(int));
    if (e == hipSuccess) e = hipMalloc(&pl.blocks, blocks.size() * sizeof(PrefillBlockInfo));
    if (e == hipSuccess)
        e = hipMemcpy(pl.units, units.data(), units.size() * sizeof(PrefillUnit), hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy(pl.bin_start, bin_start.data(), bin_start.size() * sizeof(int), hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy(pl.blocks, blocks.data(), blocks.size() * sizeof(PrefillBlockInfo), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        free_plan(pl);
        return hip_failed(e, "prefill unit table");
    }
    if (ps.plans.size() >= kPrefillPlans) {
        size_t lru = 0;
        for (size_t i = 1; i < ps.plans.size(); ++i)
            if (ps.plans[i].last_use < ps.plans[lru].last_use) lru = i;
        // Kernels on any stream may still read the evicted table.
        G4_HIP(hipDeviceSynchronize());
        free_plan(ps.plans[lru]);
        ps.plans[lru] = pl;
        *out = &ps.plans[lru];
    } else {
        ps.plans.push_back(pl);
        *out = &ps.plans.back();
    }
    return G4_OK;
}

int describe_prefill_schedule(int64_t pos0, int64_t N, int64_t window, int head_dim, int n_kv_heads, int num_cus,
                              int32_t *units4, int64_t units_cap, int32_t *bin_start_out, int64_t bins_cap,
                              int32_t *counts) {
    const std::vector<std::pair<int, int>> bt = block_tile_ranges(pos0, N, window);
    Bins bins;
    if (build_schedule(bt, bins_for(num_cus, n_kv_heads), head_dim, bins) != 0)
        return set_error(G4_ERR_COMPUTE, "prefill key range too long for one call");
    std::vector<PrefillUnit> units;
    std::vector<int> bin_start;
    std::vector<PrefillBlockInfo> blocks;
    int n_slots = 0;
    int rc = schedule_tables(bt, bins, units, bin_start, blocks, n_slots);
    if (rc != G4_OK) return rc;
    counts[0] = (int32_t)units.size();
    counts[1] = (int32_t)bin_start.size() - 1;
    counts[2] = n_slots;
    if ((int64_t)units.size() > units_cap || (int64_t)bin_start.size() > bins_cap)
        return set_error(G4_ERR_MSG, "prefill schedule: output arrays too small");
    for (size_t i = 0; i < units.size(); ++i) {
        units4[4 * i] = units[i].block;
        units4[4 * i + 1] = units[i].t_lo;
        units4[4 * i + 2] = units[i].t_hi;
        units4[4 * i + 3] = units[i].slot;
    }
    for (size_t i = 0; i < bin_start.size(); ++i) bin_start_out[i] = bin_start[i];
    return G4_OK;
}

int launch_prefill(g4_ctx *ctx, const PrefillArgs &a, hipStream_t stream) {
    const int group = a.n_heads / a.n_kv_heads;
    // The MFMA kernel addresses a block's rows with 32-bit byte offsets.
    const bool mfma = (a.head_dim == 256 || a.head_dim == 512) && group == kGroup &&
                      a.n_heads % a.n_kv_heads == 0 &&
                      (a.pos0 + a.N + 16 - a.kv_origin) * a.row_stride * (int64_t)sizeof(float) < (1LL << 31);
    if (!mfma) {
        // Any other shape: every query as an independent decode over its range.
        DecodeArgs d{};
        d.B = (int)a.N;
        d.q = a.q;
        d.k = a.k;
        d.v = a.v;
        d.row_stride = a.row_stride;
        d.pos0 = a.pos0;
        d.prefill_window = a.window;
        d.kv_origin = a.kv_origin;
        const int64_t last = a.pos0 + a.N;
        d.max_kv_len = (a.window > 0 && a.window < last) ? a.window : last;
        d.n_heads = a.n_heads;
        d.n_kv_heads = a.n_kv_heads;
        d.head_dim = a.head_dim;
        d.scale = a.scale;
        d.out = a.out;
        return launch_decode(ctx, d, stream);
    }
    const PrefillPlan *plp = nullptr;
    int rc = plan_for(ctx, a, &plp);
    if (rc != G4_OK) return rc;
    const PrefillPlan &pl = *plp;
    PrefillK p{};
    p.q = a.q;
    p.k = a.k;
    p.v = a.v;
    p.row_stride = a.row_stride;
    p.pos0 = a.pos0;
    p.N = a.N;
    p.window = a.window;
    p.kv_origin = a.kv_origin;
    p.n_heads = a.n_heads;
    p.scale = a.scale;
    p.out = a.out;
    p.units = pl.units;
    p.bin_start = pl.bin_start;
    p.blocks = pl.blocks;
    p.n_slots = pl.n_slots;
    p.status = ctx->status_dev;
    const int D = a.head_dim;
    // Workspace: the partials of split blocks, then the split-f16 planes of
    // the attended rows and their tile flags.
    auto up = [](size_t x) { return (x + 255) / 256 * 256; };
    const size_t per_slot = (size_t)a.n_kv_heads * kWaves * kRowsPerWave;
    const size_t obytes = up((size_t)pl.n_slots * per_slot * D * sizeof(float));
    const size_t mlbytes = up((size_t)pl.n_slots * per_slot * sizeof(float2));
    const int64_t row_lo = (a.window > 0 && a.pos0 + 1 > a.window) ? a.pos0 + 1 - a.window : 0;
    const int64_t row_hi = a.pos0 + a.N;
    const int64_t t0 = row_lo / 16, n_tiles = (row_hi - 1) / 16 + 1 - t0;
    const size_t plane_bytes = (size_t)n_tiles * a.n_kv_heads * 128 * D;
    // The split form: f16 products carry any |x| < 2^15 to f32 accuracy; the
    // planes are addressed with 32-bit offsets; a scale beyond 2^32 could
    // take scores near the f32 limit, where only the f32 form's rounding is
    // the reference's.
    const bool split = !ctx->prefill_exact && plane_bytes < (1ull << 31) && std::isfinite(a.scale) &&
                       std::fabs(a.scale) <= 4294967296.0f;
    const size_t bytes = obytes + mlbytes + (split ? up(plane_bytes) + up((size_t)n_tiles * a.n_kv_heads * 8) : 0);
    if (bytes > 0) {
        rc = ensure_workspace(ctx, bytes, stream);
        if (rc != G4_OK) return rc;
        char *w = (char *)ctx->ws.ptr;
        p.part_o = (float *)w;
        p.part_ml = (float2 *)(w + obytes);
        if (split) {
            p.planes = (const _Float16 *)(w + obytes + mlbytes);
            p.plane_bytes = (uint32_t)plane_bytes;
            p.t0 = t0;
            p.tile_flags = (const int *)(w + obytes + mlbytes + up(plane_bytes));
        }
    }
    if (split) {
        SplitK s{};
        s.k = a.k;
        s.v = a.v;
        s.row_stride = a.row_stride;
        s.kv_origin = a.kv_origin;
        s.row_lo = row_lo;
        s.row_hi = row_hi;
        s.t0 = t0;
        s.planes = (_Float16 *)p.planes;
        s.tile_flags = (int *)p.tile_flags;
        const dim3 sg((unsigned)n_tiles, (unsigned)a.n_kv_heads, 2);
        if (D == 256)
            hipLaunchKernelGGL(prefill_split_kernel<256>, sg, dim3(256), 0, stream, s);
        else
            hipLaunchKernelGGL(prefill_split_kernel<512>, sg, dim3(256), 0, stream, s);
        G4_HIP(hipGetLastError());
    }
    dim3 grid((unsigned)pl.n_bins, (unsigned)a.n_kv_heads);
    if (D == 256)
        hipLaunchKernelGGL(prefill_kernel<256>, grid, dim3(PrefillShape<256>::THREADS), 0, stream, p);
    else
        hipLaunchKernelGGL(prefill_kernel<512>, grid, dim3(PrefillShape<512>::THREADS), 0, stream, p);
    G4_HIP(hipGetLastError());
    if (pl.n_slots > 0) {
        // One merge workgroup per producing wavefront of a block.
        if (D == 256)
            hipLaunchKernelGGL(prefill_merge_kernel<256>,
                               dim3((unsigned)pl.n_blocks, (unsigned)a.n_kv_heads, (unsigned)PrefillShape<256>::RWAVES),
                               dim3(256), 0, stream, p);
        else
            hipLaunchKernelGGL(prefill_merge_kernel<512>,
                               dim3((unsigned)pl.n_blocks, (unsigned)a.n_kv_heads, (unsigned)PrefillShape<512>::RWAVES),
                               dim3(256), 0, stream, p);
        G4_HIP(hipGetLastError());
    }
    return G4_OK;
}

}  // namespace g4
