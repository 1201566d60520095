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
// A workgroup is 8 wavefronts that split the head dimension: wave w owns
// dims [DW*w, DW*w + DW) of K, V, q and the output, DW = D/8 (64 for the
// global layers' D = 512, 32 for the sliding layers' 256: two wavefronts per
// SIMD either way, so one wave's MFMA chain overlaps the other's softmax and
// LDS work).  Each wave computes a partial
// S^T over its dims; the partials are summed through LDS in a fixed order, so
// every wave sees bit-identical scores and softmax state, then each wave
// accumulates P.V for its own dims.  Work is split over keys (split-K): a
// workgroup handles a power-of-two run of keys of one (sequence, KV head),
// streaming 16-key tiles through a ring of register buffers (loads of the
// next tiles in flight while the current one is computed), and leaves an
// online-softmax partial (m, l, O) that a second kernel merges.
//
// Softmax semantics follow softmax_f32 (crates/llm-backend-cpu/src/ops.rs:105-127):
// p = exp(s - max) / sum with scale applied to the dot product first
// (model.rs:334); a NaN or +inf score, or a row whose scores are all -inf,
// makes the call fail ("softmax input is not finite", model.rs:362-364).

#include "g4_internal.h"
#include "g4_prep.h"

namespace g4 {
namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kDecodeBuffers = 4;  // K/V tiles held per wave: a pair computed, a pair in flight
constexpr int kMaxSplits = 512;  // per (sequence, KV head); bounds the split workspace
// Wavefronts per split workgroup (both head widths: two per SIMD).
constexpr int kDecodeWaves = 8;
// The online softmax keeps a reference maximum m and moves it only when a
// score exceeds it by more than this (natural-log units; p <= 2^8 meanwhile,
// safe in f32), so the accumulators are rescaled a few times per split, not
// per tile.
constexpr float kRescaleSlack = 8.0f / 1.4426950408889634f;

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
    int64_t kv_origin;  // prefill form: the position of row 0 of k/v
    int n_heads, n_kv_heads, group;
    float scale;
    int64_t chunk;    // keys per split: a multiple of 16
    int max_splits;
    float *out;
    float *part_o;   // per (sequence, KV head, split): D*G floats, accumulator layout
    float2 *part_ml; // [B][n_kv][max_splits][group]  (running max, sum of exp)
    unsigned *status;
    int n_seqs;      // B
    int *plan;       // streamed batches: pair prefix sums [B+1], then pairs per workgroup
};

// How a launch names each sequence's rows.  The form is a template parameter
// so that the kernels' prologues load their arguments without data-dependent
// branches (each dependent scalar load is a memory round trip).
enum Mode : int {
    kSingle = 0,  // one sequence: rows [kv_begin0, kv_end0)
    kBatch = 1,   // B sequences: rows [kv_begin[s], kv_end[s]) of a cache starting at row seq_row0[s]
    kPrefill = 2, // N queries of one sequence at positions pos0 + s (causal / windowed)
    kStream = 3   // kBatch rows through decode_stream_kernel (merge only)
};

// Rows [begin, end) that sequence s attends, and where its cache starts.
template <int MODE>
__device__ inline void seq_range(const DecodeK &p, int s, int64_t &row0, int64_t &begin,
                                 int64_t &end) {
    if constexpr (MODE == kPrefill) {
        end = p.pos0 + s + 1;
        begin = (p.prefill_window > 0 && end > p.prefill_window) ? end - p.prefill_window : 0;
        row0 = -p.kv_origin;  // key positions from kv_origin on are rows 0, 1, ...
    } else if constexpr (MODE == kBatch) {
        row0 = p.seq_row0[s];
        begin = p.kv_begin[s];
        end = p.kv_end[s];
    } else {
        row0 = 0;
        begin = p.kv_begin0;
        end = p.kv_end0;
    }
}

__device__ inline int64_t num_splits(const DecodeK &p, int64_t len) {
    const int64_t top = len + p.chunk - 1;
    const int64_t n = top < (1LL << 32) ? (int64_t)((uint32_t)top / (uint32_t)p.chunk) : top / p.chunk;
    return n < p.max_splits ? n : p.max_splits;
}

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Per-wave geometry for head dim D (256 or 512): DW dims per wave, KU
// 16-dim groups of S^T steps, TW O^T tiles of 16 rows (one dim per lane and
// tile of a V row).
template <int D>
struct DecodeShape {
    static constexpr int NW = kDecodeWaves;
    static constexpr int DW = D / NW;   // 32 or 64
    static constexpr int KU = DW / 16;  // 2 or 4
    static constexpr int TW = DW / 16;  // 2 or 4
};

template <int N> struct FloatVec;
template <> struct FloatVec<2> { typedef f32x2 type; };
template <> struct FloatVec<4> { typedef f32x4 type; };

// One 16-key tile of K and V in registers, in the MFMA operand layouts of
// lane (g, c) of a wave owning dims [base, base + DW):
//   k[u] = K[t0 + c][base + 16u + 4g .. +3]  (A of S^T = K.Q^T, steps 4u..4u+3;
//          the 4 lanes of a key read 64 contiguous bytes)
//   v[r] = V[t0 + 4g + r][base + TW*c .. +TW-1]  (A of O^T = V^T.P^T, one dim per O^T tile)
template <int D>
struct KvTile {
    f32x4 k[DecodeShape<D>::KU];
    typename FloatVec<DecodeShape<D>::TW>::type v[4];
};

// Split partials are stored in the accumulator layout, so every lane writes
// whole 16-byte vectors: for wave w, O^T tile i, lane group g and head c, the
// four rows r (dims w*DW + TW*(4g + r) + i) are one f32x4 at element
// ((w*TW + i)*4 + g)*G + c of the split's D*G/4 vectors.  Returns the dim of
// component 0; component r is TW*r further.
template <int D>
__device__ inline int partial_dim0(int e, int G) {
    constexpr int DW = DecodeShape<D>::DW, TW = DecodeShape<D>::TW;
    const int g = (e / G) & 3, wi = e / (4 * G);
    return (wi / TW) * DW + 4 * TW * g + wi % TW;
}

// Reductions over the four 16-lane rows of a wavefront (lanes c, c+16,
// c+32, c+48), done with row swaps on the VALU -- no LDS round trip -- and
// identical in every lane: rows (0,1) and (2,3) first, then the halves.
__device__ inline float rows_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float h = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(h), __float_as_uint(h), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ inline float rows_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float h = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(h), __float_as_uint(h), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Online-softmax combination of two partials (m, l, o) over disjoint key
// sets: the result is their union's (max, sum of exp, unnormalised output).
// Symmetric in its two arguments, bit for bit, so lanes that exchange
// partials agree.
__device__ inline void combine_partial(float &m, float &l, f32x4 &o, float m2, float l2, f32x4 o2) {
    const float mm = fmaxf(m, m2);
    const float a = (m == -INFINITY) ? 0.0f : exp2_fast((m - mm) * kLog2e);
    const float b = (m2 == -INFINITY) ? 0.0f : exp2_fast((m2 - mm) * kLog2e);
    l = a * l + b * l2;
    o = a * o + b * o2;
    m = mm;
}

// Folds a batch of split partials (m_j, l_j) / O_j into the running
// (m, l, o) of one stored vector; entries at or past n are ignored.
template <int NB>
__device__ inline void fold_batch(float &m, float &l, f32x4 &o, const float2 (&t)[NB], const f32x4 (&v)[NB],
                                  int j0, int jstep, int n) {
    float mb = m;
#pragma unroll
    for (int b = 0; b < NB; ++b)
        if (j0 + jstep * b < n) mb = fmaxf(mb, t[b].x);
    const float a = (m == -INFINITY) ? 0.0f : exp2_fast((m - mb) * kLog2e);
    l *= a;
    o *= a;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const bool use = j0 + jstep * b < n && t[b].x != -INFINITY;
        const float w = use ? exp2_fast((t[b].x - mb) * kLog2e) : 0.0f;
        l += w * t[b].y;
        o += w * v[b];
    }
    m = mb;
}

// Final output of stored vector e (head c = e % G) from its merged partial.
template <int D>
__device__ inline void write_merged(const DecodeK &p, int s, int kvh, int e, float m, float l, f32x4 o) {
    const int G = p.group, c = e % G;
    if (m == -INFINITY) {  // every score of this head was -inf
        atomicOr(p.status, kStatusNonFinite);
        return;
    }
    const float inv = 1.0f / l;
    float *op = p.out + ((int64_t)s * p.n_heads + kvh * G + c) * D + partial_dim0<D>(e, G);
#pragma unroll
    for (int r = 0; r < 4; ++r) op[DecodeShape<D>::TW * r] = o[r] * inv;
}

// Buffer resource (V#) word 3 for raw 32-bit-element buffers on gfx9-class
// GPUs, gfx950 included.
constexpr int kBufferWord3 = 0x00020000;
// Cache-policy operand of a buffer store: SC1, device scope -- the store is
// written through the XCD's L2 to the point of coherence.
constexpr int kDeviceScope = 16;
// Cache-policy operand of a buffer load: NT, non-temporal (streamed, not
// kept for reuse).
constexpr int kNonTemporal = 2;
// The cache policies of a decode's K and V loads, packed into one template
// argument: K's operand in the low byte, V's in the next.  A K load covers
// half of each 128-byte line it touches (4 lanes x 16 bytes of a key), the
// other half following in the next load; a V load covers whole lines.  With
// NT loads on K the first half's line is not kept for the second, while NT
// on V alone streams faster in every form measured (event-timed graph
// replays, against NT on both or on neither):
//   ragged batch, 32 global sequences (2 GB):    345 -> 318 us (6.4 TB/s)
//   one sequence, 4096 keys d=512 (HBM-cold):   10.1 -> 9.5 us
//   one sequence, 8192 keys d=512:              12.2 -> 11.0 us
//   ragged batch, 32 sliding windows of 512:    12.9 -> 12.5 us
// K keeps the default policy; NT on K was slower (351 us on the first).
// decode_stream_kernel reads K with whole-line loads through LDS instead
// (KLdsLane), NT like V: the first case then takes 304 us (6.7 TB/s).
constexpr int kv_policy(int k, int v) { return k | (v << 8); }
constexpr int kPolicyK(int aux) { return aux & 0xff; }
constexpr int kPolicyV(int aux) { return (aux >> 8) & 0xff; }
constexpr int kKvPolicy = kv_policy(0, kNonTemporal);

// A wavefront's view of one (sequence, KV head) decode: lane (g, c) =
// (lane/16, lane%16) of wave w, which owns head dims [base, base + DW).
// K and V are read through buffer resources spanning exactly the rows being
// attended: a load is the resource + a per-lane byte offset fixed for the
// call + the tile's offset (one add), and rows past the end read as zeros in
// hardware (their scores are masked, and zero V keeps 0 * V finite).
template <int D>
struct DecodeLane {
    using Shape = DecodeShape<D>;
    static constexpr int NW = Shape::NW, DW = Shape::DW, KU = Shape::KU, TW = Shape::TW;
    typedef typename FloatVec<TW>::type VRow;
    int lane, wave, g, c, base;
    uint32_t koff, voff[4], tile_bytes;

    __device__ __forceinline__ explicit DecodeLane(int stride) {
        lane = threadIdx.x & 63;
        // The wave index is uniform across a wavefront; saying so keeps the
        // buffer resources and tile offsets in scalar registers.
        wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        g = lane >> 4;
        c = lane & 15;
        base = wave * DW;
        tile_bytes = 64u * (uint32_t)stride;
        // Lane (g, c) reads K row c (dims 16u + 4g..+3) and V rows 4g + r
        // (dims TW*c..+TW-1) of a tile.  16 rows of stride fit 32 bits
        // (checked by the launcher).
        koff = (uint32_t)(c * stride + 4 * g) * 4u;
#pragma unroll
        for (int r = 0; r < 4; ++r) voff[r] = (uint32_t)((4 * g + r) * stride + TW * c) * 4u;
    }

    // Resource over n_keys rows starting at `first_row` (this wave's dims);
    // the rows span < 2^31 bytes (checked by the launcher).
    __device__ __forceinline__ __amdgpu_buffer_rsrc_t rows(const float *first_row, int n_keys, int stride) const {
        const int records = (n_keys - 1) * stride * 4 + DW * 4;
        return __builtin_amdgcn_make_buffer_rsrc((void *)(first_row + base), 0, records, kBufferWord3);
    }

    // The tile offset goes into the per-lane offset: the hardware range
    // check covers that offset (not the scalar one), so every row at or past
    // the end -- in the last tile, or a whole tile past it -- reads 0.
    template <int AUX>
    __device__ __forceinline__ void load_tile(__amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs, int tile,
                                              KvTile<D> &T) const {
        const uint32_t toff = (uint32_t)tile * tile_bytes;
#pragma unroll
        for (int u = 0; u < KU; ++u)
            T.k[u] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, koff + toff + 64u * u, 0, kPolicyK(AUX)));
        load_v<AUX>(vrs, toff, T);
    }

    // V of the tile at byte offset toff (a multiple of tile_bytes, or an
    // offset past the resource's range, which reads zeros).
    template <int AUX>
    __device__ __forceinline__ void load_v(__amdgpu_buffer_rsrc_t vrs, uint32_t toff, KvTile<D> &T) const {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if constexpr (TW == 4)
                T.v[r] = __builtin_bit_cast(VRow, __builtin_amdgcn_raw_buffer_load_b128(vrs, voff[r] + toff, 0, kPolicyV(AUX)));
            else
                T.v[r] = __builtin_bit_cast(VRow, __builtin_amdgcn_raw_buffer_load_b64(vrs, voff[r] + toff, 0, kPolicyV(AUX)));
        }
    }
};

// K through LDS (decode_stream_kernel).  A lane's K load above covers half
// of each 128-byte line it touches (the A operand puts one key in 16
// lanes' reach of 64 bytes), and that pattern streams at ~6.0 TB/s against
// ~7.0 for whole lines.  Here a tile's K slice of one wave (16 keys x DW
// dims, QPK 16-byte quads per key) arrives by KU LDS-DMA loads: load u
// takes, in lane L, quad (L % QPK) ^ sw(k) of key k = KPI*u + L / QPK --
// each load reads whole lines, non-temporally -- and writes LDS slot
// 64u + L.  The operand of lane (g, c), group u' (key c, quad 4u' + g) is
// then at slot 64(c / KPI) + QPK(c % KPI) + ((4u' + g) ^ sw(c)); the
// swizzle sw puts the keys that 8 or 16 lanes of a read name on distinct
// 16-byte bank groups.
template <int D>
struct KLdsLane {
    static constexpr int DW = DecodeShape<D>::DW, KU = DecodeShape<D>::KU;
    static constexpr int QPK = DW / 4;   // quads per key: 16 or 8
    static constexpr int KPI = 64 / QPK;  // keys per load: 4 or 8
    static_assert(KPI * KU == 16, "a tile's 16 keys in KU loads");
    __device__ __forceinline__ static int sw(int k) { return QPK == 16 ? k : ((k >> 1) ^ ((k & 1) << 2)); }
    uint32_t off[KU];  // byte offset of load u within a tile
    int rd[KU];        // slot of group u's operand

    __device__ __forceinline__ KLdsLane(const DecodeLane<D> &ln, int stride) {
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            const int k = KPI * u + ln.lane / QPK;
            off[u] = (uint32_t)(k * stride + 4 * ((ln.lane % QPK) ^ sw(k))) * 4u;
            rd[u] = 64 * (ln.c / KPI) + QPK * (ln.c % KPI) + ((4 * u + ln.g) ^ sw(ln.c));
        }
    }
};

struct NoHook {
    __device__ __forceinline__ void operator()() const {}
};

// Partial S^T of a pair, double-buffered: [buffer][tile][wave][lane].
template <int D>
using PairScores = f32x4[2][2][DecodeShape<D>::NW][64];

// Online-softmax state of one wave for one (sequence, KV head): Q^T as the
// B operand (lane (g, c) holds q[head c][base + 16u + 4g + j]), the
// reference maximum m and sum of exp l of head c, and this wave's O^T tiles.
template <int D>
struct DecodeAcc {
    using L = DecodeLane<D>;
    static constexpr int NW = L::NW, KU = L::KU, TW = L::TW;
    float qreg[KU][4];
    float m, l;
    f32x4 o[TW];
    bool bad;  // a NaN or +inf score was seen

    // q_row: head c's row, or for a padding column (c >= group) any real
    // head's.  MFMA output columns do not mix, a padding column's softmax
    // state only gates the shared rescale branch (its alpha is its own), and
    // its results and flags are never written, so the loaded row is used
    // as is: no select waits on the load before the K/V loads are issued.
    __device__ __forceinline__ void start(const L &ln, const float *q_row) {
        const float *qh = q_row + ln.base + 4 * ln.g;
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            const f32x4 a = *(const f32x4 *)(qh + 16 * u);
#pragma unroll
            for (int j = 0; j < 4; ++j) qreg[u][j] = a[j];
        }
        m = -INFINITY;
        l = 0.0f;
#pragma unroll
        for (int i = 0; i < TW; ++i) o[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    // One pair of tiles (32 keys) with `valid` of its keys in range: the two
    // score chains, the cross-wave sum, the softmax bookkeeping and the P.V
    // chains of a pair run together, so each fixed latency -- the barrier,
    // the LDS round trip, the softmax's dependent steps -- is paid once per
    // 32 keys.  NT = 1: only the first tile (a split of at most 16 keys).
    // after_exchange runs once every wave has passed the exchange barrier
    // (so this wave's reads of the pair's K operands have completed) and
    // this wave has issued its reads of the exchanged scores -- the last LDS
    // reads of the pair.
    template <int NT = 2, typename Hook = NoHook>
    __device__ __forceinline__ void pair(const L &ln, const KvTile<D> &P0, const KvTile<D> &P1, int valid,
                                         float scale, PairScores<D> &sx, int &buf,
                                         const Hook &after_exchange = Hook()) {
        const KvTile<D> *P[2] = {&P0, &P1};
        // Partial S^T of both tiles over this wave's dims (two MFMA chains).
        f32x4 acc[2] = {};
#pragma unroll
        for (int u = 0; u < KU; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(P[t]->k[u][j], qreg[u][j], acc[t], 0, 0, 0);

        // The tiles' S^T: the waves' partials summed in a fixed order, so
        // every wave holds the same bits (all reads issue before the first add).
#pragma unroll
        for (int t = 0; t < NT; ++t) sx[buf][t][ln.wave][ln.lane] = acc[t];
        __syncthreads();
        f32x4 sc[2];
        if constexpr (NT == 1) sc[1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            f32x4 v[NW];
#pragma unroll
            for (int w = 0; w < NW; ++w) v[w] = sx[buf][t][w][ln.lane];
            if constexpr (NW == 8)
                sc[t] = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
            else
                sc[t] = (v[0] + v[1]) + (v[2] + v[3]);
        }
        buf ^= 1;
        after_exchange();

        // Scores of keys 16t + 4g + r of the pair for head c; NaN or +inf
        // fails the call; keys past the end (a last pair) are masked.
        float sv[8];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sv[4 * t + r] = sc[t][r] * scale;
                if (t < NT) bad |= __builtin_amdgcn_classf(sv[4 * t + r], 0x203);  // signalling/quiet NaN, +inf
            }
        if (NT == 1 || valid < 32) {
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if (16 * (k >> 2) + 4 * ln.g + (k & 3) >= valid) sv[k] = -INFINITY;
        }
        const float mt = rows_max(fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                                        fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7]))));
        // Move the reference maximum only when a score outgrows it.
        const bool grow = mt > m + kRescaleSlack;
        if (__any(grow)) {
            const float m_new = grow ? mt : m;
            const float alpha = grow ? exp2_fast((m - m_new) * kLog2e) : 1.0f;
            l *= alpha;
#pragma unroll
            for (int i = 0; i < TW; ++i) o[i] *= alpha;
            m = m_new;
        }
        float pr[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) pr[k] = (m == -INFINITY) ? 0.0f : exp2_fast((sv[k] - m) * kLog2e);
        l += ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));

        // O^T += V^T . P^T: k-step (t, r) covers key 16t + 4g + r; O^T tile i
        // holds dims base + TW*c' + i for output row c'.
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int i = 0; i < TW; ++i)
                    o[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(P[t]->v[r][i], pr[4 * t + r], o[i], 0, 0, 0);
    }

    // One more key whose value row is held in LDS (vrow, D floats): sv is its
    // scaled score for head c (-inf for padding columns).
    __device__ __forceinline__ void fold_key(const L &ln, float sv, const float *vrow) {
        bad |= __builtin_amdgcn_classf(sv, 0x203);  // signalling/quiet NaN, +inf
        const bool grow = sv > m + kRescaleSlack;
        if (__any(grow)) {
            const float m_new = grow ? sv : m;
            const float alpha = grow ? exp2_fast((m - m_new) * kLog2e) : 1.0f;
            l *= alpha;
#pragma unroll
            for (int i = 0; i < TW; ++i) o[i] *= alpha;
            m = m_new;
        }
        const float pr = (sv == -INFINITY) ? 0.0f : exp2_fast((sv - m) * kLog2e);
        if (ln.g == 0) l += pr;  // l is summed over the four lane groups of a head
        // O^T tile i, component r of lane (g, c): dim base + TW*(4g + r) + i.
#pragma unroll
        for (int i = 0; i < TW; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[i][r] += pr * vrow[ln.base + TW * (4 * ln.g + r) + i];
    }

    // The attention output of head c (l summed over the lanes c, c+16, c+32,
    // c+48); out_row = the head's D floats.  A head whose scores were all
    // -inf fails the call.
    __device__ __forceinline__ void write_output(const L &ln, float *out_row, bool col_valid, unsigned *status) const {
        const float lt = rows_sum(l);
        if (ln.wave == 0 && __any(col_valid && m == -INFINITY) && ln.lane == 0) atomicOr(status, kStatusNonFinite);
        if (!col_valid) return;
        const float inv = 1.0f / lt;
        float *op = out_row + ln.base;
#pragma unroll
        for (int i = 0; i < TW; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) op[TW * (4 * ln.g + r) + i] = o[i][r] * inv;
    }

    // This wave's share of a split partial (see partial_dim0); `slot` is the
    // partial's index in units of G*D floats / G (m, l) pairs.  The stores
    // are written through to the point of coherence: the merge kernel reads
    // them from other XCDs, and the split kernel then ends with no dirty L2
    // lines of its own to write back (measured 0.6 us faster per decode at
    // 256 splits).
    __device__ __forceinline__ void write_partial(const L &ln, float *part_o, float2 *part_ml, int64_t slot, int G,
                                                  bool col_valid) const {
        const float lt = rows_sum(l);
        if (!col_valid) return;
        const __amdgpu_buffer_rsrc_t ro =
            __builtin_amdgcn_make_buffer_rsrc((void *)(part_o + slot * G * D), 0, G * D * 4, kBufferWord3);
#pragma unroll
        for (int i = 0; i < TW; ++i)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o[i]), ro,
                                                   (((ln.wave * TW + i) * 4 + ln.g) * G + ln.c) * 16, 0, kDeviceScope);
        if (ln.wave == 0 && ln.g == 0) {
            const __amdgpu_buffer_rsrc_t rm =
                __builtin_amdgcn_make_buffer_rsrc((void *)(part_ml + slot * G), 0, G * 8, kBufferWord3);
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f32x2{m, lt}), rm, ln.c * 8, 0,
                                                  kDeviceScope);
        }
    }
};

// Pairs q_first .. q_first + n_pairs - 1 of the rows behind (krs, vrs),
// which hold n_keys keys, into acc.  Pairs stream through NBUF/2 register
// slots, one pair in flight while one is computed; loads are issued
// unconditionally (clamped to the last pair), so the compiler's wait counts
// stay exact and never wait on a prefetch.  A pair's second tile past the
// end (odd tile count) reads zeros and is masked.  prime() issues the first
// pairs' loads and finish() computes every pair, so that a caller can do
// other work while the first tiles are in flight.  (A split of at most 16
// keys is a single tile, which callers load and compute themselves.)
template <int D, int NBUF, int AUX>
struct PairPipe {
    static constexpr int NPAIR = NBUF / 2;
    KvTile<D> T[NPAIR][2];

    __device__ __forceinline__ void load_pair(const DecodeLane<D> &ln, __amdgpu_buffer_rsrc_t krs,
                                              __amdgpu_buffer_rsrc_t vrs, int q_first, int n_pairs, int i,
                                              KvTile<D> (&P)[2]) const {
        const int q = q_first + (i < n_pairs ? i : n_pairs - 1);
        ln.template load_tile<AUX>(krs, vrs, 2 * q, P[0]);
        ln.template load_tile<AUX>(krs, vrs, 2 * q + 1, P[1]);
    }

    __device__ __forceinline__ void prime(const DecodeLane<D> &ln, __amdgpu_buffer_rsrc_t krs,
                                          __amdgpu_buffer_rsrc_t vrs, int q_first, int n_pairs) {
#pragma unroll
        for (int b = 0; b < NPAIR - 1; ++b) load_pair(ln, krs, vrs, q_first, n_pairs, b, T[b]);
    }

    __device__ __forceinline__ void finish(const DecodeLane<D> &ln, DecodeAcc<D> &acc, __amdgpu_buffer_rsrc_t krs,
                                           __amdgpu_buffer_rsrc_t vrs, int q_first, int n_pairs, int n_keys,
                                           float scale, PairScores<D> &sx, int &buf) {
        // Steady state: each step issues the loads of the pair NPAIR-1 ahead,
        // then computes the oldest buffered pair.
        int i0 = 0;
        for (; i0 + NPAIR - 1 < n_pairs; i0 += NPAIR) {
#pragma unroll
            for (int b = 0; b < NPAIR; ++b) {
                load_pair(ln, krs, vrs, q_first, n_pairs, i0 + b + NPAIR - 1, T[(b + NPAIR - 1) % NPAIR]);
                acc.pair(ln, T[b][0], T[b][1], n_keys - 32 * (q_first + i0 + b), scale, sx, buf);
            }
        }
        // Tail: the remaining (< NPAIR) pairs are already buffered in T[0..].
#pragma unroll
        for (int b = 0; b < NPAIR - 1; ++b)
            if (i0 + b < n_pairs) acc.pair(ln, T[b][0], T[b][1], n_keys - 32 * (q_first + i0 + b), scale, sx, buf);
    }
};

template <int D, int NBUF, int AUX>
__device__ __forceinline__ void run_pairs(const DecodeLane<D> &ln, DecodeAcc<D> &acc, __amdgpu_buffer_rsrc_t krs,
                                          __amdgpu_buffer_rsrc_t vrs, int q_first, int n_pairs, int n_keys,
                                          float scale, PairScores<D> &sx, int &buf) {
    PairPipe<D, NBUF, AUX> pp;
    if (n_keys - 32 * q_first <= 16) {  // a single tile: its second half is not computed
        // The scheduler issues the K loads ahead of the score chain and the V
        // loads after it, so the scores overlap the V transfer; issuing all
        // eight loads at once measured slower (4096 keys: 10.3 -> 11.2 us).
        ln.template load_tile<AUX>(krs, vrs, 2 * q_first, pp.T[0][0]);
        acc.template pair<1>(ln, pp.T[0][0], pp.T[0][0], n_keys - 32 * q_first, scale, sx, buf);
        return;
    }
    pp.prime(ln, krs, vrs, q_first, n_pairs);
    pp.finish(ln, acc, krs, vrs, q_first, n_pairs, n_keys, scale, sx, buf);
}

// One 16-byte load per lane from `rsrc` at byte offset voff (the range check
// covers it), written straight to LDS at lds + 16 * lane (lds is the same for
// the whole wavefront).
template <int POLICY>
__device__ __forceinline__ void load_to_lds(__amdgpu_buffer_rsrc_t rsrc, f32x4 *lds, uint32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)lds, 16, voff, 0, 0,
                                             POLICY);
#endif
}

// Tile offset of the loads past a run's last pair: beyond every resource's
// range (the stream kernel's ranges span < 2^31 bytes, and 2^31 plus a
// pair's tile and per-lane offsets, < 128 rows of stride, does not wrap), so
// they read zeros without touching memory while the loads themselves stay
// unconditional -- which keeps the compiler's wait counts exact.
constexpr uint32_t kPastEnd = 0x80000000u;

// run_pairs with K through LDS (KLdsLane; lk = this wave's two tile slices,
// [2 * KU][64] slots) and V through two register slots.  Pair i's V is
// fetched one pair ahead, at the top of pair i-1; its K once pair i-1's
// scores have been exchanged (after the last LDS read of pair i-1's K, and
// after the pair's other LDS reads, which the compiler would otherwise hold
// until the K transfer lands), so one LDS slice serves every pair.  Each
// pair waits for its K and V behind the next pair's V loads.
template <int D, int AUX>
__device__ __forceinline__ void run_pairs_ldsk(const DecodeLane<D> &ln, const KLdsLane<D> &kl, f32x4 (*lk)[64],
                                               DecodeAcc<D> &acc, __amdgpu_buffer_rsrc_t krs,
                                               __amdgpu_buffer_rsrc_t vrs, int q_first, int n_pairs, int n_keys,
                                               float scale, PairScores<D> &sx, int &buf) {
    constexpr int KU = DecodeShape<D>::KU;
    if (n_keys - 32 * q_first <= 16) {  // a single tile, through registers as run_pairs does
        KvTile<D> T;
        ln.template load_tile<AUX>(krs, vrs, 2 * q_first, T);
        acc.template pair<1>(ln, T, T, n_keys - 32 * q_first, scale, sx, buf);
        return;
    }
    auto pair_off = [&](int i) {  // byte offset of pair i of the run
        return i < n_pairs ? (uint32_t)(2 * (q_first + i)) * ln.tile_bytes : kPastEnd;
    };
    auto fetch_k = [&](uint32_t off) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < KU; ++u)
                load_to_lds<kPolicyV(AUX)>(krs, lk[t * KU + u], kl.off[u] + off + t * ln.tile_bytes);
    };
    auto fetch_v = [&](uint32_t off, KvTile<D>(&P)[2]) {
        ln.template load_v<AUX>(vrs, off, P[0]);
        ln.template load_v<AUX>(vrs, off + ln.tile_bytes, P[1]);
    };
    // Pair i from cur (its V), with the next pair's V into nxt.
    auto step = [&](int i, KvTile<D>(&cur)[2], KvTile<D>(&nxt)[2]) {
        const uint32_t next = pair_off(i + 1);
        fetch_v(next, nxt);
        // Pair i's K (LDS) and V have landed once at most the 8 V loads just
        // issued are outstanding (loads complete in order).
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const f32x4 *tile = lk[t * KU];  // the tile's 64 * KU slots
#pragma unroll
            for (int u = 0; u < KU; ++u) cur[t].k[u] = tile[kl.rd[u]];
        }
        acc.pair(ln, cur[0], cur[1], n_keys - 32 * (q_first + i), scale, sx, buf, [&] {
            __builtin_amdgcn_sched_barrier(0);
            fetch_k(next);
        });
    };
    // V before K, the order in which the steps issue them.
    KvTile<D> T[2][2];
    fetch_v(pair_off(0), T[0]);
    fetch_k(pair_off(0));
    for (int i = 0; i < n_pairs; i += 2) {
        step(i, T[0], T[1]);
        if (i + 1 < n_pairs) step(i + 1, T[1], T[0]);
    }
    // The run's last K transfer (past the end) writes this wave's slice;
    // let it land before the next run, or the workgroup's end, reuses it.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// One workgroup = one (split, KV head, sequence); NW wavefronts, each owning
// DW = D/NW of the head dims.
template <int D, int MODE, int NBUF, int AUX>
__global__ __launch_bounds__(64 * DecodeShape<D>::NW) void decode_split_kernel(DecodeK p) {
    const int split = blockIdx.x, kvh = blockIdx.y, s = blockIdx.z;
    const DecodeLane<D> ln((int)p.row_stride);

    int64_t row0, begin, end;
    seq_range<MODE>(p, s, row0, begin, end);
    const int64_t len = end - begin;
    if (MODE != kSingle && (len <= 0 || len > p.max_kv_len)) {  // kSingle: checked by the host
        if (split == 0 && kvh == 0 && threadIdx.x == 0)
            atomicOr(p.status, len <= 0 ? kStatusNonFinite : kStatusRangeTooLong);
        return;
    }
    // One sequence: the grid is exactly the split count, so no branch here
    // waits on a kernel argument before the K/V loads are issued.  Batches:
    // split s holds keys [begin + s chunk, min(end, begin + (s+1) chunk)),
    // no division on the way to the loads.
    const int64_t k_lo = begin + (int64_t)split * p.chunk;
    if (MODE != kSingle && k_lo >= end) return;
    const bool one_split = MODE == kSingle ? p.max_splits == 1 : len <= p.chunk;
    const int64_t k_hi = MODE == kSingle ? ((split + 1 == p.max_splits) ? end : k_lo + p.chunk)
                                         : (k_lo + p.chunk < end ? k_lo + p.chunk : end);
    const int n_keys = (int)(k_hi - k_lo);
    const int n_pairs = (n_keys + 31) >> 5;

    const int stride = (int)p.row_stride;
    const int64_t first = (row0 + k_lo) * p.row_stride + (int64_t)kvh * D;
    const __amdgpu_buffer_rsrc_t krs = ln.rows(p.k + first, n_keys, stride);
    const __amdgpu_buffer_rsrc_t vrs = ln.rows(p.v + first, n_keys, stride);

    const bool col_valid = ln.c < p.group;
    const int head = kvh * p.group + (col_valid ? ln.c : 0);
    DecodeAcc<D> acc;
    acc.bad = false;
    acc.start(ln, p.q + ((int64_t)s * p.n_heads + head) * D);
    __shared__ PairScores<D> sx;
    int buf = 0;
    run_pairs<D, NBUF, AUX>(ln, acc, krs, vrs, 0, n_pairs, n_keys, p.scale, sx, buf);

    if (ln.wave == 0 && __any(acc.bad && col_valid) && ln.lane == 0) atomicOr(p.status, kStatusNonFinite);
    if (one_split) {
        acc.write_output(ln, p.out + ((int64_t)s * p.n_heads + head) * D, col_valid, p.status);
        return;
    }
    const int64_t slot = ((int64_t)s * p.n_kv_heads + kvh) * p.max_splits + split;
    acc.write_partial(ln, p.part_o, p.part_ml, slot, p.group, col_valid);
}

// The layer driver's decode step with the input preparation fused in (see
// LayerPrepArgs): one sequence, one workgroup per split as
// decode_split_kernel, one query head per wavefront of the group.  A
// workgroup issues its first K/V loads, then, while they are in flight,
// prepares the group's q heads (and, in the last split of an owner layer,
// the new row's k and v, which it appends to the cache) with the arithmetic
// of the standalone preparation kernel; the new row, not in the cache when
// the loads were issued, is attended from LDS as the range's last key.
template <int D, int NBUF, int AUX>
__global__ __launch_bounds__(64 * DecodeShape<D>::NW) void decode_layer_kernel(DecodeK p, LayerPrepArgs lp) {
    constexpr int NW = DecodeShape<D>::NW;
    const int split = blockIdx.x, kvh = blockIdx.y;
    const DecodeLane<D> ln((int)p.row_stride);
    const int64_t begin = p.kv_begin0, end = p.kv_end0;
    const int64_t n_splits = p.max_splits;
    const bool last = split + 1 == n_splits;
    const bool fresh = lp.k != nullptr && last;  // this workgroup prepares and attends the new row
    const int64_t k_lo = begin + (int64_t)split * p.chunk;
    const int64_t k_hi = last ? end : k_lo + p.chunk;
    const int n_keys = (int)(k_hi - k_lo) - (fresh ? 1 : 0);  // keys read from the cache
    const int n_pairs = (n_keys + 31) >> 5;
    const bool single = n_keys <= 16;

    const int stride = (int)p.row_stride;
    const int64_t first = k_lo * p.row_stride + (int64_t)kvh * D;
    const int rows = n_keys > 0 ? n_keys : 1;  // with no key to read the resources go unused
    const __amdgpu_buffer_rsrc_t krs = ln.rows(p.k + first, rows, stride);
    const __amdgpu_buffer_rsrc_t vrs = ln.rows(p.v + first, rows, stride);
    // The preparation's loads first, then the K/V loads: memory counters
    // complete in issue order, so the preparation then waits only for its
    // own (small, mostly cached) rows and runs while the K/V tiles stream.
    // Wavefront w takes query head kvh*NW + w; in the fresh workgroup waves
    // 0 and 1 also take the new row's k and v.
    static_assert(D / 2 <= kPrepMaxAngles, "the angle table covers the head");
    __shared__ float qp[NW][D];
    __shared__ float kvn[2][D];
    __shared__ float sk[NW];
    const bool is_k = ln.wave == 0, prep_kv = fresh && ln.wave < 2;
    PrepRow<D> row, kv;
    prep_load<D>(row, ln.lane, lp.q + ((int64_t)kvh * NW + ln.wave) * D, lp.q_w);
    if (prep_kv) prep_load<D>(kv, ln.lane, (is_k ? lp.k : lp.v) + (int64_t)kvh * D, is_k ? lp.k_w : nullptr);
    // Thread i < D/2 builds entry i of the workgroup's RoPE table (shared by
    // the q heads and k); its angle and divisor load with the rows.
    static_assert(D / 2 <= 64 * NW, "one table entry per thread");
    const bool tab = (int)threadIdx.x < D / 2;
    const float th = tab ? lp.angles[threadIdx.x] : 0.0f;
    const float fac = (tab && lp.factors) ? lp.factors[threadIdx.x] : 1.0f;
    __builtin_amdgcn_sched_barrier(0);
    PairPipe<D, NBUF, AUX> pp;
    if (n_keys > 0) {
        if (single)
            ln.template load_tile<AUX>(krs, vrs, 0, pp.T[0][0]);
        else
            pp.prime(ln, krs, vrs, 0, n_pairs);
    }
    __builtin_amdgcn_sched_barrier(0);
    {
        __shared__ float rcs[D / 2], rsn[D / 2];
        if (tab) prep_rope_table(rcs, rsn, threadIdx.x, th, fac);
        prep_norm<D>(row, lp.q_w != nullptr, lp.eps);
        if (prep_kv) prep_norm<D>(kv, is_k && lp.k_w != nullptr, lp.eps);
        __syncthreads();  // the table
        prep_rope_tab<D>(row, ln.lane, rcs, rsn);
        prep_store<D>(row, ln.lane, qp[ln.wave]);
        if (prep_kv) {
            if (is_k) prep_rope_tab<D>(kv, ln.lane, rcs, rsn);
            prep_store<D>(kv, ln.lane, kvn[ln.wave]);
            prep_store<D>(kv, ln.lane, (is_k ? lp.k_row : lp.v_row) + (int64_t)kvh * D);  // the append
        }
        __syncthreads();
    }

    const bool col_valid = ln.c < p.group;
    const int hc = col_valid ? ln.c : 0;
    DecodeAcc<D> acc;
    acc.bad = false;
    acc.start(ln, qp[hc]);
    __shared__ PairScores<D> sx;
    int buf = 0;
    if (n_keys > 0) {
        if (single)
            acc.template pair<1>(ln, pp.T[0][0], pp.T[0][0], n_keys, p.scale, sx, buf);
        else
            pp.finish(ln, acc, krs, vrs, 0, n_pairs, n_keys, p.scale, sx, buf);
    }
    if (fresh) {
        // The new row's score: one head's dot product per wavefront.
        float dot = 0.0f;
#pragma unroll
        for (int m = 0; m < D / 64; ++m) dot += qp[ln.wave][ln.lane + 64 * m] * kvn[0][ln.lane + 64 * m];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) dot += __shfl_xor(dot, off);
        if (ln.lane == 0) sk[ln.wave] = dot;
        __syncthreads();
        acc.fold_key(ln, col_valid ? sk[hc] * p.scale : -INFINITY, kvn[1]);
    }

    if (ln.wave == 0 && __any(acc.bad && col_valid) && ln.lane == 0) atomicOr(p.status, kStatusNonFinite);
    if (n_splits == 1) {
        acc.write_output(ln, p.out + ((int64_t)kvh * p.group + hc) * D, col_valid, p.status);
        return;
    }
    const int64_t slot = (int64_t)kvh * p.max_splits + split;
    acc.write_partial(ln, p.part_o, p.part_ml, slot, p.group, col_valid);
}

// Ragged batches, streamed: the sequences' attended rows are cut into pairs
// of 16-key tiles (32 keys), numbered sequence after sequence, and each of a
// persistent grid of workgroups (one per CU) takes an equal run of pairs.  A
// workgroup streams its run across sequence boundaries -- the next pairs'
// loads are in flight while the current one is computed, whichever
// sequence they belong to -- so every CU streams HBM from start to end
// whatever the lengths.  A sequence that lies wholly inside one workgroup's
// run is finished there; the runs' first and last sequences may continue in
// the neighbouring workgroups and leave partials (slot 0: the run's first
// sequence, slot 1: its last) that decode_merge_kernel<kStream> combines.
constexpr int kStreamMaxSeqs = 1024;

// Pairs per sequence and their running sums in LDS (pref[s] = first pair of
// sequence s); invalid ranges count no pairs and raise the status.
__device__ inline int stream_plan(const DecodeK &p, int *pref, int64_t *first_row, int *seq_len, bool report) {
    const int B = p.n_seqs;
    for (int s = threadIdx.x; s < B; s += blockDim.x) {
        const int64_t b = p.kv_begin[s], e = p.kv_end[s], len = e - b;
        const bool ok = len > 0 && len <= p.max_kv_len;
        if (!ok && report) atomicOr(p.status, len <= 0 ? kStatusNonFinite : kStatusRangeTooLong);
        first_row[s] = p.seq_row0[s] + b;
        seq_len[s] = ok ? (int)len : 0;
        pref[s + 1] = ok ? (int)((len + 31) >> 5) : 0;
    }
    if (threadIdx.x == 0) pref[0] = 0;
    __syncthreads();
    if (threadIdx.x < 64) {  // inclusive scan of pref[1..B] by one wavefront
        const int lane = threadIdx.x, per = (B + 63) / 64;
        const int lo = 1 + lane * per, hi = min(lo + per, B + 1);
        int run = 0;
        for (int i = lo; i < hi; ++i) {
            run += pref[i];
            pref[i] = run;
        }
        int incl = run;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int t = __shfl_up(incl, off);
            if (lane >= off) incl += t;
        }
        const int excl = incl - run;
        for (int i = lo; i < hi; ++i) pref[i] += excl;
    }
    __syncthreads();
    return pref[B];
}

template <int D>
__global__ __launch_bounds__(64 * DecodeShape<D>::NW) void decode_stream_kernel(DecodeK p) {
    const int w = blockIdx.x, W = gridDim.x, kvh = blockIdx.y;
    const DecodeLane<D> ln((int)p.row_stride);
    const KLdsLane<D> kl(ln, (int)p.row_stride);
    const int B = p.n_seqs, G = p.group, stride = (int)p.row_stride;
    __shared__ int pref[kStreamMaxSeqs + 1];
    __shared__ int64_t first_row[kStreamMaxSeqs];
    __shared__ int seq_len[kStreamMaxSeqs];
    const int total = __builtin_amdgcn_readfirstlane(stream_plan(p, pref, first_row, seq_len, w == 0 && kvh == 0));
    // Values read back from LDS are the same in every lane; readfirstlane
    // keeps the cursors and buffer resources in scalar registers.
    auto pref_at = [&](int s) { return __builtin_amdgcn_readfirstlane(pref[s]); };
    auto len_at = [&](int s) { return __builtin_amdgcn_readfirstlane(seq_len[s]); };
    auto row_at = [&](int s) {
        const uint64_t r = (uint64_t)first_row[s];
        return (int64_t)(((uint64_t)__builtin_amdgcn_readfirstlane((unsigned)(r >> 32)) << 32) |
                         (unsigned)__builtin_amdgcn_readfirstlane((unsigned)r));
    };
    const int ppw = (total + W - 1) / W;
    if (w == 0 && kvh == 0) {
        for (int i = threadIdx.x; i <= B; i += blockDim.x) p.plan[i] = pref[i];
        if (threadIdx.x == 0) p.plan[B + 1] = ppw;
    }
    const int g0 = w * ppw, g1 = min(total, g0 + ppw);
    if (g0 >= g1) return;
    // Sequence holding pair g (the last s with pref[s] <= g; empty ones skipped).
    auto seq_of = [&](int g, int s) {
        while (pref_at(s + 1) <= g) ++s;
        return s;
    };

    __shared__ PairScores<D> sx;
    // Each wave's K slices of a pair (KLdsLane): 64 KiB at D = 512.
    __shared__ f32x4 lk[DecodeShape<D>::NW][2 * DecodeShape<D>::KU][64];
    int buf = 0;
    DecodeAcc<D> acc;
    acc.bad = false;
    const bool col_valid = ln.c < G;
    const int head = kvh * G + (col_valid ? ln.c : 0);
    // One segment per sequence the run touches: pairs [g, ge) of sequence cs.
    int cs = seq_of(g0, 0);
    for (int g = g0; g < g1;) {
        const int ga = pref_at(cs), gb = pref_at(cs + 1), ge = min(g1, gb), n_keys = len_at(cs);
        const int64_t first = row_at(cs) * p.row_stride + (int64_t)kvh * D;
        const __amdgpu_buffer_rsrc_t krs = ln.rows(p.k + first, n_keys, stride);
        const __amdgpu_buffer_rsrc_t vrs = ln.rows(p.v + first, n_keys, stride);
        acc.start(ln, p.q + ((int64_t)cs * p.n_heads + head) * D);
        run_pairs_ldsk<D, kKvPolicy>(ln, kl, lk[ln.wave], acc, krs, vrs, g - ga, ge - g, n_keys, p.scale, sx, buf);
        if (g == ga && ge == gb) {
            acc.write_output(ln, p.out + ((int64_t)cs * p.n_heads + head) * D, col_valid, p.status);
        } else {  // slot 0: the run's first sequence; 1: its last
            const int64_t slot = ((int64_t)(2 * w + (g == g0 ? 0 : 1))) * p.n_kv_heads + kvh;
            acc.write_partial(ln, p.part_o, p.part_ml, slot, G, col_valid);
        }
        g = ge;
        if (g < g1) cs = seq_of(g, cs);
    }
    if (ln.wave == 0 && __any(acc.bad && col_valid) && ln.lane == 0) atomicOr(p.status, kStatusNonFinite);
}

// Merges the split partials of one (sequence, KV head):
// Folds splits ph, ph + PH, ... < n of stored vector e into (m, l, o), NB
// splits per batch: every load of a batch is issued before any is used.
// Partial j sits at slot0 + j*jslot, plus first_extra for j = 0.
template <int D, int PH, int NB>
__device__ __forceinline__ void merge_fold(const DecodeK &p, int64_t slot0, int64_t jslot, int64_t first_extra,
                                           int ph, int e, int c, int n, int G, float &m, float &l, f32x4 &o) {
    auto slot = [&](int j) { return slot0 + j * jslot + (j == 0 ? first_extra : 0); };
    for (int j0 = ph; j0 < n; j0 += PH * NB) {
        float2 t[NB];
        f32x4 v[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) t[b] = p.part_ml[slot(min(j0 + PH * b, n - 1)) * G + c];
#pragma unroll
        for (int b = 0; b < NB; ++b) v[b] = ((const f32x4 *)(p.part_o + slot(min(j0 + PH * b, n - 1)) * G * D))[e];
        // No wait before every load above is issued: left alone, the
        // scheduler trickled the vector loads out between the folds.
        __builtin_amdgcn_sched_barrier(0);
        fold_batch(m, l, o, t, v, j0, PH, n);
    }
}

// O_c = sum_j e^(m_jc - M_c) O_jc / sum_j e^(m_jc - M_c) l_jc for each head c.
// A workgroup covers EPW stored vectors of one (sequence, KV head); its
// PH = 256/EPW thread phases each fold every PH-th split into a running
// partial in registers, then the phases are combined across lanes and waves
// in a fixed order (deterministic), and EPW lanes write the result.  The
// split count n is uniform in the workgroup: the batch size is the smallest
// that covers n in one memory round trip (up to 256 splits), so no lane
// reloads a split it does not use.
template <int MODE, int D, int EPW>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeK p) {
    constexpr int PH = 256 / EPW;
    static_assert(EPW == 8 || EPW == 16, "whole 128-byte rows per phase; at most 16 lanes write");
    const int s = blockIdx.z, kvh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int n = p.max_splits;
    // Partial j of this (sequence, KV head) is at slot0 + j*jslot, except for
    // streamed batches, whose first partial may sit in its workgroup's second
    // slot (first_extra).
    int64_t slot0 = ((int64_t)s * p.n_kv_heads + kvh) * p.max_splits, jslot = 1, first_extra = 0;
    if constexpr (MODE == kStream) {
        const int ga = p.plan[s], gb = p.plan[s + 1], ppw = p.plan[p.n_seqs + 1];
        if (gb <= ga) return;  // an invalid range: reported by the split kernel
        const int w1 = ga / ppw, w2 = (gb - 1) / ppw;
        if (w1 == w2) return;  // finished by its workgroup
        n = w2 - w1 + 1;
        slot0 = (int64_t)2 * w1 * p.n_kv_heads + kvh;
        jslot = 2 * p.n_kv_heads;
        first_extra = ga > w1 * ppw ? p.n_kv_heads : 0;
    } else if constexpr (MODE != kSingle) {
        int64_t row0, begin, end;
        seq_range<MODE>(p, s, row0, begin, end);
        const int64_t len = end - begin;
        if (len <= 0 || len > p.max_kv_len) return;
        n = (int)num_splits(p, len);
    }
    if (MODE != kSingle && n <= 1) return;  // kSingle: launched only with splits
    n = __builtin_amdgcn_readfirstlane(n);
    const int G = p.group;

    const int ph = tid / EPW, el = tid % EPW;
    const int e = blockIdx.x * EPW + el;  // stored vector index within a split
    const int c = e % G;

    float mt = -INFINITY, lt = 0.0f;
    f32x4 ot = {0.0f, 0.0f, 0.0f, 0.0f};
    if (n <= PH)
        merge_fold<D, PH, 1>(p, slot0, jslot, first_extra, ph, e, c, n, G, mt, lt, ot);
    else if (n <= 2 * PH)
        merge_fold<D, PH, 2>(p, slot0, jslot, first_extra, ph, e, c, n, G, mt, lt, ot);
    else if (n <= 4 * PH)
        merge_fold<D, PH, 4>(p, slot0, jslot, first_extra, ph, e, c, n, G, mt, lt, ot);
    else if (n <= 8 * PH || EPW == 8)
        merge_fold<D, PH, 8>(p, slot0, jslot, first_extra, ph, e, c, n, G, mt, lt, ot);
    else
        merge_fold<D, PH, 16>(p, slot0, jslot, first_extra, ph, e, c, n, G, mt, lt, ot);
    // The phases of wave w sit EPW lanes apart.
#pragma unroll
    for (int off = EPW; off <= 32; off <<= 1) {
        f32x4 o2;
#pragma unroll
        for (int r = 0; r < 4; ++r) o2[r] = __shfl_xor(ot[r], off);
        combine_partial(mt, lt, ot, __shfl_xor(mt, off), __shfl_xor(lt, off), o2);
    }
    __shared__ f32x4 red_o[4][EPW];
    __shared__ float2 red_ml[4][EPW];
    if (lane < EPW) {
        red_o[wave][el] = ot;
        red_ml[wave][el] = float2{mt, lt};
    }
    __syncthreads();
    if (tid >= EPW) return;
    float m = red_ml[0][el].x, l = red_ml[0][el].y;
    f32x4 o = red_o[0][el];
#pragma unroll
    for (int w = 1; w < 4; ++w) combine_partial(m, l, o, red_ml[w][el].x, red_ml[w][el].y, red_o[w][el]);
    write_merged<D>(p, s, kvh, e, m, l, o);
}

// Any shape the MFMA kernel does not cover (head_dim not a multiple of 256,
// more than 16 query heads per KV head): one workgroup per (head, sequence),
// 256 keys per step, online softmax in f32.
template <int MODE>
__global__ __launch_bounds__(256) void decode_generic_kernel(DecodeK p, int D) {
    const int head = blockIdx.x, s = blockIdx.y, tid = threadIdx.x;
    int64_t row0, begin, end;
    seq_range<MODE>(p, s, row0, begin, end);
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
    const float *kb = p.k + (int64_t)kvh * D;  // key t is row row0 + t
    const float *vb = p.v + (int64_t)kvh * D;
    constexpr int kMaxPer = 4;  // D <= 1024
    float o[kMaxPer] = {0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;
    bool bad = false;
    __syncthreads();
    for (int64_t t0 = begin; t0 < end; t0 += 256) {
        const int64_t t = t0 + tid;
        float x = -INFINITY;
        if (t < end) {
            const float *kr = kb + (row0 + t) * p.row_stride;
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
            for (int64_t j = 0; j < nt; ++j) acc = fmaf(ps[j], vb[(row0 + t0 + j) * p.row_stride + d], acc);
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

namespace {

// Ragged batch through decode_stream_kernel: one workgroup per CU per KV head
// (at least one), then the merge of the sequences that span workgroups.
int launch_stream(g4_ctx *ctx, const DecodeArgs &a, DecodeK p, hipStream_t stream) {
    const int D = a.head_dim, G = p.group;
    const int W = ctx->num_cus / a.n_kv_heads > 0 ? ctx->num_cus / a.n_kv_heads : 1;
    const size_t slots = (size_t)W * 2 * a.n_kv_heads;
    const size_t o_bytes = (slots * G * D * sizeof(float) + 255) / 256 * 256;
    const size_t ml_bytes = (slots * G * sizeof(float2) + 255) / 256 * 256;
    int rc = ensure_workspace(ctx, o_bytes + ml_bytes + (size_t)(a.B + 2) * sizeof(int), stream);
    if (rc != G4_OK) return rc;
    p.part_o = (float *)ctx->ws.ptr;
    p.part_ml = (float2 *)((char *)ctx->ws.ptr + o_bytes);
    p.plan = (int *)((char *)ctx->ws.ptr + o_bytes + ml_bytes);
    p.n_seqs = a.B;
    const dim3 grid((unsigned)W, (unsigned)a.n_kv_heads);
    if (D == 256)
        hipLaunchKernelGGL((decode_stream_kernel<256>), grid, dim3(64 * DecodeShape<256>::NW), 0, stream, p);
    else
        hipLaunchKernelGGL((decode_stream_kernel<512>), grid, dim3(64 * DecodeShape<512>::NW), 0, stream, p);
    G4_HIP(hipGetLastError());
    const dim3 mgrid(D * G / 64, a.n_kv_heads, a.B);
    if (D == 256)
        hipLaunchKernelGGL((decode_merge_kernel<kStream, 256, 16>), mgrid, dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL((decode_merge_kernel<kStream, 512, 16>), mgrid, dim3(256), 0, stream, p);
    G4_HIP(hipGetLastError());
    return G4_OK;
}

// lp: the fused layer step (one sequence), launched as decode_layer_kernel
// with the split kernel's sizing.
// The merge's workgroup width for n splits: one sequence above 64 splits
// takes 8 vectors per workgroup (twice the workgroups to share the bytes),
// otherwise 16 (fewer shuffle rounds).  Measured on one sequence: 32 splits
// at d=256 7.2 -> 6.2 us per step, 256 splits at d=512 10.3 -> 9.9 us.
template <int MODE, int D>
void launch_merge(const DecodeK &p, int64_t n, int group, int n_kv_heads, int B, hipStream_t stream) {
    if (MODE == kSingle && n > 64)
        hipLaunchKernelGGL((decode_merge_kernel<MODE, D, 8>), dim3(D * group / 32, n_kv_heads, B), dim3(256), 0,
                           stream, p);
    else
        hipLaunchKernelGGL((decode_merge_kernel<MODE, D, 16>), dim3(D * group / 64, n_kv_heads, B), dim3(256), 0,
                           stream, p);
}

template <int MODE>
int launch_mode(g4_ctx *ctx, const DecodeArgs &a, DecodeK p, hipStream_t stream,
                const LayerPrepArgs *lp = nullptr) {
    const int D = a.head_dim;
    const int group = p.group;
    const bool mfma = (D == 256 || D == 512) && group <= 16 && a.n_heads % a.n_kv_heads == 0 &&
                      a.row_stride <= (1LL << 25);  // 16 rows of stride fit 32-bit byte offsets
    if (!mfma) {
        if (D > 1024) return set_error(G4_ERR_COMPUTE, "head_dim above 1024 is not supported");
        p.chunk = 1LL << 40;  // one split
        p.max_splits = 1;
        hipLaunchKernelGGL(decode_generic_kernel<MODE>, dim3(a.n_heads, a.B), dim3(256),
                           (size_t)(D + 256) * sizeof(float), stream, p, D);
        G4_HIP(hipGetLastError());
        return G4_OK;
    }
    // Ragged batches stream unless a split size was set explicitly or the
    // batch is too small to give each CU a few 32-key pairs (then the split
    // grid's shorter prologue wins); the streamed kernel addresses a
    // sequence's rows with 32-bit byte offsets.
    if (MODE == kBatch && ctx->decode_chunk == 0 && a.B <= kStreamMaxSeqs &&
        (int64_t)a.B * a.max_kv_len >= 4 * 32 * (int64_t)ctx->num_cus &&
        (a.max_kv_len + 32) * a.row_stride * (int64_t)sizeof(float) < (1LL << 31))
        return launch_stream(ctx, a, p, stream);

    // Split-K sizing.  A split is a whole number (at least one) of 16-key
    // MFMA tiles.  One sequence: one workgroup per CU (the occupancy of the
    // split kernel), down to a single tile each -- a workgroup's time is
    // its MFMA and softmax work, so spreading the tiles over every CU wins
    // over fewer, longer splits.  Ragged batches: about eight per CU, at
    // least 64 keys, so that sequences of very different lengths still
    // balance over the CUs.  Contexts of up to two tiles run as one split
    // (no merge); longer ones split even when short: 64 keys took 6.8 us as
    // one workgroup, 5.7 us as four one-tile splits and the merge.
    const int64_t units = (int64_t)a.B * a.n_kv_heads;
    const int64_t max_len = a.max_kv_len > 0 ? a.max_kv_len : 1;
    int64_t chunk = ctx->decode_chunk;
    if (chunk <= 0) {
        const int64_t target = (MODE == kSingle ? 1LL : 8LL) * ctx->num_cus;
        chunk = (max_len * units + target - 1) / target;
        const int64_t floor_keys = MODE == kSingle ? 16 : 64;
        if (chunk < floor_keys) chunk = floor_keys;
        if (max_len <= 32) chunk = max_len;
    }
    const int64_t min_chunk = (max_len + kMaxSplits - 1) / kMaxSplits;
    if (chunk < min_chunk) chunk = min_chunk;
    // A split is a whole number of 16-key tiles.  Any multiple of 16, not
    // only powers of two: a context just past 256 x a power of two would
    // otherwise double the split size and leave half the CUs idle (one
    // sequence of 8300 keys at d=512: 130 splits of 64 keys, 15.5 us,
    // against 173 of 48).
    chunk = (chunk + 15) / 16 * 16;
    // The kernel addresses a split's rows with 32-bit byte offsets.
    const int64_t max_chunk = (1LL << 31) / (a.row_stride * (int64_t)sizeof(float)) / 2 / 16 * 16;
    if (chunk > max_chunk) chunk = max_chunk;
    if (chunk < min_chunk || max_chunk < 16)
        return set_error(G4_ERR_COMPUTE, "K/V range too large for the decode kernel's addressing");
    const int64_t max_splits = (max_len + chunk - 1) / chunk;
    p.chunk = chunk;
    p.max_splits = (int)max_splits;
    if (max_splits > 1) {
        const size_t slots = (size_t)units * max_splits * group;
        const size_t bytes = slots * D * sizeof(float) + slots * sizeof(float2) + 256;
        void *ws = a.scratch;
        if (ws) {
            if (bytes > a.scratch_bytes)
                return set_error(G4_ERR_COMPUTE, "g4_attend_decode_noalloc: this decode needs " + std::to_string(bytes) +
                                                     " bytes of split scratch, above the static " +
                                                     std::to_string(a.scratch_bytes));
        } else {
            int rc = ensure_workspace(ctx, bytes, stream);
            if (rc != G4_OK) return rc;
            ws = ctx->ws.ptr;
        }
        p.part_o = (float *)ws;
        size_t off = (slots * D * sizeof(float) + 255) / 256 * 256;
        p.part_ml = (float2 *)((char *)ws + off);
    }
    dim3 grid((unsigned)max_splits, (unsigned)a.n_kv_heads, (unsigned)a.B);
    if (MODE == kSingle && lp) {
        if (D == 256)
            hipLaunchKernelGGL((decode_layer_kernel<256, kDecodeBuffers, kKvPolicy>), grid,
                               dim3(64 * DecodeShape<256>::NW), 0, stream, p, *lp);
        else
            hipLaunchKernelGGL((decode_layer_kernel<512, kDecodeBuffers, kKvPolicy>), grid,
                               dim3(64 * DecodeShape<512>::NW), 0, stream, p, *lp);
    } else if (D == 256) {
        hipLaunchKernelGGL((decode_split_kernel<256, MODE, kDecodeBuffers, kKvPolicy>), grid,
                           dim3(64 * DecodeShape<256>::NW), 0, stream, p);
    } else {
        hipLaunchKernelGGL((decode_split_kernel<512, MODE, kDecodeBuffers, kKvPolicy>), grid,
                           dim3(64 * DecodeShape<512>::NW), 0, stream, p);
    }
    G4_HIP(hipGetLastError());
    if (max_splits > 1) {
        if (D == 256)
            launch_merge<MODE, 256>(p, max_splits, group, a.n_kv_heads, a.B, stream);
        else
            launch_merge<MODE, 512>(p, max_splits, group, a.n_kv_heads, a.B, stream);
        G4_HIP(hipGetLastError());
    }
    return G4_OK;
}

}  // namespace

// Split partials of g4_attend_decode_noalloc, for callers that cannot
// allocate.  One array per GPU, shared by every such call on it (calls that
// overlap on one GPU race).  8 MiB + 64 KiB holds the partials of any split
// plan with one KV head (at most kMaxSplits splits of 8 heads x 512 floats,
// plus their (m, l) pairs).  Nothing in it needs to start at zero: each split
// writes its partial before the merge reads it.
constexpr size_t kDecodeScratchBytes = (8u << 20) + (64u << 10);
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

int decode_scratch_address(void **ptr, size_t *bytes) {
    void *p = nullptr;
    G4_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return set_error(G4_ERR_COMPUTE, "hip: no device address for the decode scratch");
    *ptr = p;
    *bytes = kDecodeScratchBytes;
    return G4_OK;
}

int launch_decode(g4_ctx *ctx, const DecodeArgs &a, hipStream_t stream) {
    if (a.B <= 0) return G4_OK;
    if (a.scratch && (a.B != 1 || a.kv_begin || a.prefill_window >= 0))
        return set_error(G4_ERR_COMPUTE, "decode scratch: single-sequence decodes only");
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
    p.kv_origin = a.kv_origin;
    p.n_heads = a.n_heads;
    p.n_kv_heads = a.n_kv_heads;
    p.group = a.n_heads / a.n_kv_heads;
    p.scale = a.scale;
    p.out = a.out;
    p.status = ctx->status_dev;
    if (a.prefill_window >= 0) return launch_mode<kPrefill>(ctx, a, p, stream);
    if (a.kv_begin) {
        if (!p.seq_row0) {  // a zero row offset for every sequence
            int rc = ensure_zero_rows(ctx, a.B);
            if (rc != G4_OK) return rc;
            p.seq_row0 = ctx->zero_rows;
        }
        return launch_mode<kBatch>(ctx, a, p, stream);
    }
    return launch_mode<kSingle>(ctx, a, p, stream);
}

bool layer_decode_fusable(const DecodeArgs &a) {
    return a.B == 1 && !a.kv_begin && a.prefill_window < 0 && (a.head_dim == 256 || a.head_dim == 512) &&
           a.n_kv_heads > 0 && a.n_heads == kDecodeWaves * a.n_kv_heads && a.row_stride <= (1LL << 25) &&
           a.kv_end0 > a.kv_begin0;
}

int launch_layer_decode(g4_ctx *ctx, const DecodeArgs &a, const LayerPrepArgs &lp, hipStream_t stream) {
    if (!layer_decode_fusable(a)) return set_error(G4_ERR_COMPUTE, "fused layer decode: unsupported shape");
    DecodeK p{};
    p.q = lp.q;
    p.k = a.k;
    p.v = a.v;
    p.row_stride = a.row_stride;
    p.kv_begin0 = a.kv_begin0;
    p.kv_end0 = a.kv_end0;
    p.max_kv_len = a.max_kv_len;
    p.prefill_window = -1;
    p.n_heads = a.n_heads;
    p.n_kv_heads = a.n_kv_heads;
    p.group = a.n_heads / a.n_kv_heads;
    p.scale = a.scale;
    p.out = a.out;
    p.status = ctx->status_dev;
    return launch_mode<kSingle>(ctx, a, p, stream, &lp);
}

}  // namespace g4
