//! Raw declarations: every function of `include/g4attn.h`, the C ABI of
//! `libg4attn.so` -- the only library the crate binds (device memory
//! included: `g4_alloc`, `g4_copy_*`, `g4_free`).  Parameter names follow the
//! header (lower-cased); the types map `int` -> `c_int`, `int64_t` -> `i64`,
//! `size_t` -> `usize`, `g4_stream` -> `*mut c_void` (a `hipStream_t`, null
//! for the null stream).

use std::ffi::{c_char, c_int, c_void};

/// `g4_ctx`: one per device (split-K workspace, status word).
#[repr(C)]
pub struct G4Ctx {
    _opaque: [u8; 0],
}

/// `g4_kv_cache`: the device-resident `ContextMemory`.
#[repr(C)]
pub struct G4KvCache {
    _opaque: [u8; 0],
}

/// `g4_hparams`: the fields of `Gemma4HyperParams`
/// (crates/llm-gemma4/src/idea/mod.rs:15-34) the layer drivers read, with
/// `global_rope_base` = `global_p_rope.base`.
#[repr(C)]
#[derive(Clone, Copy, Debug, PartialEq)]
pub struct G4Hparams {
    pub n_layers: c_int,
    pub n_heads: c_int,
    pub n_kv_heads: c_int,
    pub head_dim_local: c_int,
    pub head_dim_global: c_int,
    pub sliding_window: i64,
    pub shared_kv_layers: c_int,
    pub local_rope_base: f32,
    pub global_rope_base: f32,
    pub rms_norm_eps: f32,
}

/// `g4_status`, one code per `EngError` variant (crates/llm-eng/src/error.rs:3-15).
pub const G4_OK: c_int = 0;
pub const G4_ERR_CONTEXT_TOO_LONG: c_int = 1;
pub const G4_ERR_MISSING_LAYER: c_int = 2;
pub const G4_ERR_MISSING_WEIGHT: c_int = 3;
pub const G4_ERR_COMPUTE: c_int = 4;
pub const G4_ERR_MSG: c_int = 5;

extern "C" {
    pub fn g4_last_error() -> *const c_char;
    pub fn g4_last_error_fields(a: *mut u64, b: *mut u64);
    pub fn g4_init(device: c_int, ctx: *mut *mut G4Ctx) -> c_int;
    pub fn g4_release(ctx: *mut G4Ctx) -> c_int;
    pub fn g4_check_status(ctx: *mut G4Ctx, stream: *mut c_void) -> c_int;
    pub fn g4_set_decode_chunk(ctx: *mut G4Ctx, keys: i64) -> c_int;
    pub fn g4_set_prefill_exact(ctx: *mut G4Ctx, exact: c_int) -> c_int;
    pub fn g4_alloc(ctx: *mut G4Ctx, bytes: usize, ptr_dev: *mut *mut c_void) -> c_int;
    pub fn g4_free(ctx: *mut G4Ctx, ptr_dev: *mut c_void) -> c_int;
    pub fn g4_copy_to_device(
        ctx: *mut G4Ctx,
        dst_dev: *mut c_void,
        src_host: *const c_void,
        bytes: usize,
    ) -> c_int;
    pub fn g4_copy_to_host(
        ctx: *mut G4Ctx,
        dst_host: *mut c_void,
        src_dev: *const c_void,
        bytes: usize,
    ) -> c_int;
    pub fn g4_copy_on_device(
        ctx: *mut G4Ctx,
        dst_dev: *mut c_void,
        src_dev: *const c_void,
        bytes: usize,
    ) -> c_int;
    pub fn g4_sync(ctx: *mut G4Ctx, stream: *mut c_void) -> c_int;
    pub fn g4_activate(ctx: *mut G4Ctx) -> c_int;
    pub fn g4_attend(
        ctx: *mut G4Ctx,
        q_host: *const f32,
        q_len: usize,
        keys_host: *const f32,
        values_host: *const f32,
        t: usize,
        n_heads: usize,
        n_kv_heads: usize,
        scale: f32,
        out_host: *mut f32,
    ) -> c_int;
    pub fn g4_attend_decode(
        ctx: *mut G4Ctx,
        q_dev: *const f32,
        k_cache_dev: *const f32,
        v_cache_dev: *const f32,
        row_stride: i64,
        kv_begin: i64,
        kv_end: i64,
        n_heads: c_int,
        n_kv_heads: c_int,
        head_dim: c_int,
        scale: f32,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_attend_decode_noalloc(
        ctx: *mut G4Ctx,
        q_dev: *const f32,
        k_cache_dev: *const f32,
        v_cache_dev: *const f32,
        row_stride: i64,
        kv_begin: i64,
        kv_end: i64,
        n_heads: c_int,
        n_kv_heads: c_int,
        head_dim: c_int,
        scale: f32,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_attend_decode_batch(
        ctx: *mut G4Ctx,
        b: c_int,
        q_dev: *const f32,
        k_base_dev: *const f32,
        v_base_dev: *const f32,
        row_stride: i64,
        seq_row0_dev: *const i64,
        kv_begin_dev: *const i64,
        kv_end_dev: *const i64,
        max_kv_len: i64,
        n_heads: c_int,
        n_kv_heads: c_int,
        head_dim: c_int,
        scale: f32,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_attend_prefill(
        ctx: *mut G4Ctx,
        q_dev: *const f32,
        k_cache_dev: *const f32,
        v_cache_dev: *const f32,
        row_stride: i64,
        pos0: i64,
        n: i64,
        window: i64,
        n_heads: c_int,
        n_kv_heads: c_int,
        head_dim: c_int,
        scale: f32,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_prefill_schedule(
        pos0: i64,
        n: i64,
        window: i64,
        head_dim: c_int,
        n_kv_heads: c_int,
        num_cus: c_int,
        units: *mut i32,
        units_cap: i64,
        bin_start: *mut i32,
        bins_cap: i64,
        counts: *mut i32,
    ) -> c_int;
    pub fn g4_rms_norm_rows(
        ctx: *mut G4Ctx,
        x_dev: *const f32,
        n_rows: i64,
        width: i64,
        weight_dev: *const f32,
        eps: f32,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_rope_neox_rows(
        ctx: *mut G4Ctx,
        x_dev: *mut f32,
        n_tokens: i64,
        n_heads: c_int,
        head_dim: c_int,
        n_rot: c_int,
        pos0: i64,
        base: f32,
        freq_factors_dev: *const f32,
        n_factors: i64,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_kv_create(
        ctx: *mut G4Ctx,
        n_layers: c_int,
        widths_host: *const i64,
        capacity: i64,
        cache: *mut *mut G4KvCache,
    ) -> c_int;
    pub fn g4_kv_destroy(cache: *mut G4KvCache) -> c_int;
    pub fn g4_kv_append(
        cache: *mut G4KvCache,
        layer: c_int,
        k_dev: *const f32,
        v_dev: *const f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_kv_append_rows(
        cache: *mut G4KvCache,
        layer: c_int,
        k_dev: *const f32,
        v_dev: *const f32,
        n: i64,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_kv_view(
        cache: *const G4KvCache,
        layer: c_int,
        len: i64,
        k_dev: *mut *const f32,
        v_dev: *mut *const f32,
        row_stride: *mut i64,
    ) -> c_int;
    pub fn g4_kv_view_rows(
        cache: *const G4KvCache,
        layer: c_int,
        begin: i64,
        end: i64,
        k_dev: *mut *const f32,
        v_dev: *mut *const f32,
        row_stride: *mut i64,
    ) -> c_int;
    pub fn g4_kv_create_ring(
        ctx: *mut G4Ctx,
        n_layers: c_int,
        widths_host: *const i64,
        capacity: i64,
        ring_rows_host: *const i64,
        cache: *mut *mut G4KvCache,
    ) -> c_int;
    pub fn g4_kv_len(cache: *const G4KvCache, layer: c_int) -> i64;
    pub fn g4_kv_clear(cache: *mut G4KvCache);
    pub fn g4_decode_step_fused(
        ctx: *mut G4Ctx,
        q_dev: *const f32,
        k_dev: *const f32,
        v_dev: *const f32,
        q_norm_w_dev: *const f32,
        k_norm_w_dev: *const f32,
        eps: f32,
        rope_base: f32,
        freq_factors_dev: *const f32,
        position: i64,
        k_cache_dev: *const f32,
        v_cache_dev: *const f32,
        row_stride: i64,
        n_rows: i64,
        k_row_dev: *mut f32,
        v_row_dev: *mut f32,
        n_heads: c_int,
        n_kv_heads: c_int,
        head_dim: c_int,
        scale: f32,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_layer_attention(
        ctx: *mut G4Ctx,
        cache: *mut G4KvCache,
        hp: *const G4Hparams,
        layer: c_int,
        position: i64,
        q_dev: *mut f32,
        k_dev: *mut f32,
        v_dev: *mut f32,
        q_norm_w_dev: *const f32,
        k_norm_w_dev: *const f32,
        rope_freqs_dev: *const f32,
        out_dev: *mut f32,
        source: *mut c_int,
        kv_begin: *mut i64,
        kv_end: *mut i64,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_prepare_qkv(
        ctx: *mut G4Ctx,
        q_dev: *mut f32,
        k_dev: *mut f32,
        v_dev: *mut f32,
        n_tokens: i64,
        pos0: i64,
        n_heads: c_int,
        n_kv_heads: c_int,
        head_dim: c_int,
        q_norm_w_dev: *const f32,
        k_norm_w_dev: *const f32,
        eps: f32,
        rope_base: f32,
        freq_factors_dev: *const f32,
        k_rows_dev: *mut f32,
        v_rows_dev: *mut f32,
        row_stride: i64,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_layer_prefill(
        ctx: *mut G4Ctx,
        cache: *mut G4KvCache,
        hp: *const G4Hparams,
        layer: c_int,
        pos0: i64,
        n_tokens: i64,
        q_dev: *mut f32,
        k_dev: *mut f32,
        v_dev: *mut f32,
        q_norm_w_dev: *const f32,
        k_norm_w_dev: *const f32,
        rope_freqs_dev: *const f32,
        out_dev: *mut f32,
        source: *mut c_int,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_layer_is_global(n_layers: c_int, layer: c_int) -> c_int;
    pub fn g4_kv_source_layer(
        n_layers: c_int,
        shared_kv_layers: c_int,
        layer: c_int,
        source: *mut c_int,
    ) -> c_int;
    pub fn g4_windowed_len(seq_len: i64, window: i64, begin: *mut i64, end: *mut i64);
    pub fn g4_proportional_rope_freq_factors(head_dim: c_int, p: f32, out_host: *mut f32);
    pub fn g4_quantize_q8_0(
        ctx: *mut G4Ctx,
        x_dev: *const f32,
        n: i64,
        scales_dev: *mut f32,
        quants_dev: *mut i8,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_matvec_q8_0(
        ctx: *mut G4Ctx,
        w_dev: *const u8,
        w_bytes: i64,
        rows: i64,
        cols: i64,
        x_scales_dev: *const f32,
        x_quants_dev: *const i8,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_matvec_q8_0_softcap(
        ctx: *mut G4Ctx,
        w_dev: *const u8,
        w_bytes: i64,
        rows: i64,
        cols: i64,
        x_scales_dev: *const f32,
        x_quants_dev: *const i8,
        cap: f32,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_geglu_q8_0(
        ctx: *mut G4Ctx,
        gate_dev: *const u8,
        up_dev: *const u8,
        w_bytes: i64,
        rows: i64,
        cols: i64,
        x_scales_dev: *const f32,
        x_quants_dev: *const i8,
        fp16_gelu: c_int,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_project_q8_0(
        ctx: *mut G4Ctx,
        w_dev: *const u8,
        w_bytes: i64,
        rows: i64,
        cols: i64,
        x_dev: *const f32,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_gated_ffn_q8_0(
        ctx: *mut G4Ctx,
        gate_dev: *const u8,
        up_dev: *const u8,
        w_bytes: i64,
        rows: i64,
        cols: i64,
        x_dev: *const f32,
        fp16_gelu: c_int,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_logits_q8_0(
        ctx: *mut G4Ctx,
        w_dev: *const u8,
        w_bytes: i64,
        rows: i64,
        cols: i64,
        x_dev: *const f32,
        cap: f32,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_matvec_q8_0_f32(
        ctx: *mut G4Ctx,
        w_dev: *const u8,
        w_bytes: i64,
        rows: i64,
        cols: i64,
        x_dev: *const f32,
        f64_sums: c_int,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_matvec_bf16(
        ctx: *mut G4Ctx,
        w_dev: *const u16,
        w_len: i64,
        rows: i64,
        cols: i64,
        x_dev: *const f32,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_matvec_f32(
        ctx: *mut G4Ctx,
        w_dev: *const f32,
        w_len: i64,
        rows: i64,
        cols: i64,
        x_dev: *const f32,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_port_matmul(
        ctx: *mut G4Ctx,
        a_dev: *const f32,
        b_dev: *const f32,
        m: i64,
        n: i64,
        k: i64,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_port_rms_norm(
        ctx: *mut G4Ctx,
        x_dev: *const f32,
        weight_dev: *const f32,
        n: i64,
        eps: f32,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_port_softmax(
        ctx: *mut G4Ctx,
        x_dev: *const f32,
        n: i64,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_port_rope(
        ctx: *mut G4Ctx,
        x_dev: *mut f32,
        len: i64,
        pos: i64,
        theta: f32,
        dims: i64,
        stream: *mut c_void,
    ) -> c_int;
    pub fn g4_port_add(
        ctx: *mut G4Ctx,
        a_dev: *const f32,
        b_dev: *const f32,
        n: i64,
        out_dev: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
}
