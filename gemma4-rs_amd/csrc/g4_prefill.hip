// Chunked prefill: N queries of one sequence, query i at position pos0 + i,
// each attending exactly the rows a decode step at that position would
// (crates/llm-gemma4/src/impl_/generate.rs:37-41, eng/mod.rs:10-36).

#include "g4_internal.h"

namespace g4 {

int launch_prefill(g4_ctx *ctx, const PrefillArgs &a, hipStream_t stream) {
    // Every query is an independent decode over its own causal/window range.
    DecodeArgs d{};
    d.B = (int)a.N;
    d.q = a.q;
    d.k = a.k;
    d.v = a.v;
    d.row_stride = a.row_stride;
    d.pos0 = a.pos0;
    d.prefill_window = a.window;
    const int64_t last = a.pos0 + a.N;
    d.max_kv_len = (a.window > 0 && a.window < last) ? a.window : last;
    d.n_heads = a.n_heads;
    d.n_kv_heads = a.n_kv_heads;
    d.head_dim = a.head_dim;
    d.scale = a.scale;
    d.out = a.out;
    return launch_decode(ctx, d, stream);
}

}  // namespace g4
