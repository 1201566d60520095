//! Attention on the port's device: the model's `attend`
//! (crates/llm-gemma4/src/impl_/model.rs:348-366) on host slices, and its
//! device forms over cache rows -- one decode step, a batch of ragged
//! sequences, and a chunked prefill -- plus the policies that pick the rows
//! (crates/llm-gemma4/src/eng/mod.rs, crates/llm-gemma4/src/idea/mod.rs).

use std::ffi::c_int;
use std::ops::Range;

use llm_eng::EngError;

use crate::device::{DevBuf, DeviceVec};
use crate::error::{check, compute_error, len_i64, to_c_int};
use crate::ffi;
use crate::kv::KvRows;
use crate::port::HipPort;

/// Heads and width of one attention call.
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub struct Heads {
    pub n_heads: usize,
    pub n_kv_heads: usize,
    pub head_dim: usize,
}

impl Heads {
    fn c(&self) -> Result<(c_int, c_int, c_int), EngError> {
        Ok((
            to_c_int(self.n_heads, "n_heads")?,
            to_c_int(self.n_kv_heads, "n_kv_heads")?,
            to_c_int(self.head_dim, "head_dim")?,
        ))
    }

    fn q_width(&self) -> Result<usize, EngError> {
        self.n_heads.checked_mul(self.head_dim).ok_or_else(|| compute_error("head count overflows"))
    }

    fn kv_width(&self) -> Result<usize, EngError> {
        self.n_kv_heads.checked_mul(self.head_dim).ok_or_else(|| compute_error("head count overflows"))
    }
}

fn need(what: &str, buf_len: usize, want: usize) -> Result<(), EngError> {
    if buf_len == want {
        Ok(())
    } else {
        Err(compute_error(format!("{what} holds {buf_len} floats, the call needs {want}")))
    }
}

impl HipPort {
    /// `attend` (model.rs:348-366): q [n_heads*head_dim] with head_dim =
    /// q.len() / n_heads over one key and one value row per position
    /// ([n_kv_heads*head_dim] each).  Same result and the same "softmax input
    /// is not finite" failure (an empty context, or a q that is not
    /// n_heads * head_dim long).  Synchronous; the rows cross PCIe each call.
    pub fn attend(
        &self,
        q: &[f32],
        keys: &[Vec<f32>],
        values: &[Vec<f32>],
        n_heads: usize,
        n_kv_heads: usize,
        scale: f32,
    ) -> Result<Vec<f32>, EngError> {
        let (k, v) = (keys.concat(), values.concat());
        // g4_attend reads keys.len() rows of n_kv_heads * head_dim floats once
        // its own checks pass (positive heads, head_dim > 0, a non-empty
        // context, q = n_heads * head_dim): the rows must be that wide.
        if n_heads > 0 && n_kv_heads > 0 && !keys.is_empty() {
            let head_dim = q.len() / n_heads;
            if head_dim > 0 && q.len() == n_heads * head_dim {
                let width = n_kv_heads.checked_mul(head_dim);
                let total = width.and_then(|w| w.checked_mul(keys.len()));
                if values.len() != keys.len() || total != Some(k.len()) || total != Some(v.len()) {
                    return Err(compute_error("keys and values need one row of n_kv_heads * head_dim per position"));
                }
            }
        }
        let mut out = vec![0.0f32; q.len()];
        let (pq, pk, pv, po) = (q.as_ptr(), k.as_ptr(), v.as_ptr(), out.as_mut_ptr());
        let (ql, t) = (q.len(), keys.len());
        // SAFETY: q, k, v and out are host buffers of the sizes checked above.
        self.context()
            .call(|ctx| unsafe { ffi::g4_attend(ctx, pq, ql, pk, pv, t, n_heads, n_kv_heads, scale, po) })?;
        Ok(out)
    }

    /// One decode step over every row of `rows` (a view or window of the
    /// cache): the device form of `attend(q, &keys[range], &values[range],
    /// ..)` (model.rs:407-410).  q and out [n_heads*head_dim].  Asynchronous:
    /// `synchronize` reports a non-finite softmax.
    pub fn attend_decode(
        &self,
        q: &DevBuf,
        rows: &KvRows<'_>,
        heads: Heads,
        scale: f32,
        out: &mut DevBuf,
    ) -> Result<(), EngError> {
        self.decode(q, rows, heads, scale, out, false)
    }

    /// `attend_decode` with its split partials in a fixed device array of the
    /// library: it allocates nothing, for callers that cannot (graph
    /// capture, serving loops).  No counterpart in the reference.
    ///
    /// # Safety
    ///
    /// Every call on one device shares that device's array, whatever the
    /// context or stream, and the work is queued asynchronously: the caller
    /// must order all `attend_decode_noalloc` calls on a device (one stream,
    /// or events between streams), including those of other `HipPort`s and
    /// of `on_stream` views.  Two calls whose work overlaps on the device
    /// corrupt each other's partials and return wrong outputs without an
    /// error.
    pub unsafe fn attend_decode_noalloc(
        &self,
        q: &DevBuf,
        rows: &KvRows<'_>,
        heads: Heads,
        scale: f32,
        out: &mut DevBuf,
    ) -> Result<(), EngError> {
        self.decode(q, rows, heads, scale, out, true)
    }

    fn decode(&self, q: &DevBuf, rows: &KvRows<'_>, heads: Heads, scale: f32, out: &mut DevBuf, noalloc: bool) -> Result<(), EngError> {
        let qw = heads.q_width()?;
        need("q", q.len(), qw)?;
        need("out", out.len(), qw)?;
        if !rows.is_empty() && rows.row_stride() < heads.kv_width()? {
            return Err(compute_error("cache rows are narrower than n_kv_heads * head_dim"));
        }
        let (nh, nkv, hd) = heads.c()?;
        let (stride, end) = (len_i64(rows.row_stride())?, len_i64(rows.len())?);
        let (pq, pk, pv, po, stream) = (q.as_ptr(), rows.k_ptr(), rows.v_ptr(), out.as_mut_ptr(), self.stream().as_raw());
        // SAFETY: q and out hold n_heads*head_dim floats; the rows come from a
        // live cache view of rows.len() rows of row_stride floats.
        self.context().call(|ctx| unsafe {
            if noalloc {
                ffi::g4_attend_decode_noalloc(ctx, pq, pk, pv, stride, 0, end, nh, nkv, hd, scale, po, stream)
            } else {
                ffi::g4_attend_decode(ctx, pq, pk, pv, stride, 0, end, nh, nkv, hd, scale, po, stream)
            }
        })
    }

    /// Chunked prefill: queries at positions pos0 .. pos0+n-1 (q and out
    /// [n][n_heads*head_dim]), query i attending exactly the rows a decode
    /// at pos0+i would -- all of [0, p+1) for `window` 0 (`GlobalPolicy`),
    /// the last `window` of them otherwise (`LocalWindowPolicy`).  `rows` is
    /// `view(layer, len)` with len >= pos0 + n.
    #[allow(clippy::too_many_arguments)]
    pub fn attend_prefill(
        &self,
        q: &DevBuf,
        rows: &KvRows<'_>,
        pos0: usize,
        n: usize,
        window: usize,
        heads: Heads,
        scale: f32,
        out: &mut DevBuf,
    ) -> Result<(), EngError> {
        let qw = heads.q_width()?.checked_mul(n).ok_or_else(|| compute_error("token count overflows"))?;
        need("q", q.len(), qw)?;
        need("out", out.len(), qw)?;
        if rows.first_position() != 0 || pos0.checked_add(n).map_or(true, |e| e > rows.len()) {
            return Err(compute_error("prefill needs the layer's rows from position 0 through pos0 + n - 1"));
        }
        if n > 0 && rows.row_stride() < heads.kv_width()? {
            return Err(compute_error("cache rows are narrower than n_kv_heads * head_dim"));
        }
        let (nh, nkv, hd) = heads.c()?;
        let (stride, p0, nn, w) = (len_i64(rows.row_stride())?, len_i64(pos0)?, len_i64(n)?, len_i64(window)?);
        let (pq, pk, pv, po, stream) = (q.as_ptr(), rows.k_ptr(), rows.v_ptr(), out.as_mut_ptr(), self.stream().as_raw());
        // SAFETY: q and out hold n rows of n_heads*head_dim floats; the view
        // holds rows 0 .. pos0+n of row_stride floats.
        self.context().call(|ctx| unsafe {
            ffi::g4_attend_prefill(ctx, pq, pk, pv, stride, p0, nn, w, nh, nkv, hd, scale, po, stream)
        })
    }

    /// B sequences of one decode step each, ragged: sequence b attends rows
    /// [kv_begin[b], kv_end[b]) of its block, which starts at row
    /// seq_row0[b] of k_base / v_base (rows of row_stride floats).  q and
    /// out [B][n_heads*head_dim].  `max_kv_len` bounds every range; a longer
    /// one is reported by `synchronize`.
    ///
    /// # Safety
    /// The index arrays live on the device, so they cannot be checked here:
    /// for every b, rows seq_row0[b] + kv_begin[b] .. seq_row0[b] + kv_end[b]
    /// must lie inside `k_base` and `v_base`, with 0 <= kv_begin[b] <= kv_end[b].
    #[allow(clippy::too_many_arguments)]
    pub unsafe fn attend_decode_batch(
        &self,
        q: &DevBuf,
        k_base: &DevBuf,
        v_base: &DevBuf,
        row_stride: usize,
        seq_row0: &DeviceVec<i64>,
        kv_begin: &DeviceVec<i64>,
        kv_end: &DeviceVec<i64>,
        max_kv_len: usize,
        heads: Heads,
        scale: f32,
        out: &mut DevBuf,
    ) -> Result<(), EngError> {
        let batch = seq_row0.len();
        if kv_begin.len() != batch || kv_end.len() != batch {
            return Err(compute_error("seq_row0, kv_begin and kv_end need one entry per sequence"));
        }
        let qw = heads.q_width()?.checked_mul(batch).ok_or_else(|| compute_error("batch overflows"))?;
        need("q", q.len(), qw)?;
        need("out", out.len(), qw)?;
        if row_stride < heads.kv_width()? {
            return Err(compute_error("cache rows are narrower than n_kv_heads * head_dim"));
        }
        let (nh, nkv, hd) = heads.c()?;
        let b = to_c_int(batch, "batch")?;
        let (stride, max_len) = (len_i64(row_stride)?, len_i64(max_kv_len)?);
        let (pq, pk, pv, po) = (q.as_ptr(), k_base.as_ptr(), v_base.as_ptr(), out.as_mut_ptr());
        let (r0, kb, ke, stream) = (seq_row0.as_ptr(), kv_begin.as_ptr(), kv_end.as_ptr(), self.stream().as_raw());
        // SAFETY: q and out hold B rows of n_heads*head_dim floats; the row
        // ranges are the caller's promise (above).
        self.context().call(|ctx| unsafe {
            ffi::g4_attend_decode_batch(ctx, b, pq, pk, pv, stride, r0, kb, ke, max_len, nh, nkv, hd, scale, po, stream)
        })
    }

    /// Keys per split of the decode kernels, rounded up to a multiple of 16
    /// (0: chosen per call).
    pub fn set_decode_chunk(&self, keys: usize) -> Result<(), EngError> {
        let keys = len_i64(keys)?;
        // SAFETY: ctx is live.
        self.context().call(|ctx| unsafe { ffi::g4_set_decode_chunk(ctx, keys) })
    }

    /// Prefill products: `true` = f32 MFMAs only; `false` (default) = split-f16
    /// MFMAs for every work unit whose inputs are finite and below 2^15.
    pub fn set_prefill_exact(&self, exact: bool) -> Result<(), EngError> {
        // SAFETY: ctx is live.
        self.context().call(|ctx| unsafe { ffi::g4_set_prefill_exact(ctx, exact as c_int) })
    }
}

/// `layer_attention_kind` (idea/mod.rs:148-156): true on global layers.
pub fn layer_is_global(n_layers: usize, layer: usize) -> Result<bool, EngError> {
    let (n, l) = (to_c_int(n_layers, "n_layers")?, to_c_int(layer, "layer")?);
    // SAFETY: a pure function of its arguments.
    Ok(unsafe { ffi::g4_layer_is_global(n, l) } != 0)
}

/// `kv_source_layer` (eng/mod.rs:71-90): the layer whose K/V `layer` reads,
/// with `KvShareError`'s text as `EngError::Compute` (model.rs:398).
pub fn kv_source_layer(n_layers: usize, shared_kv_layers: usize, layer: usize) -> Result<usize, EngError> {
    let (n, s, l) = (to_c_int(n_layers, "n_layers")?, to_c_int(shared_kv_layers, "shared_kv_layers")?, to_c_int(layer, "layer")?);
    let mut source: c_int = 0;
    // SAFETY: source is a valid out-pointer.
    check(unsafe { ffi::g4_kv_source_layer(n, s, l, &mut source) })?;
    Ok(source.max(0) as usize)
}

/// `windowed_len` (eng/mod.rs:10-12): `seq_len - window .. seq_len`,
/// saturating at 0.
pub fn windowed_len(seq_len: usize, window: usize) -> Result<Range<usize>, EngError> {
    let (s, w) = (len_i64(seq_len)?, len_i64(window)?);
    let (mut begin, mut end) = (0i64, 0i64);
    // SAFETY: both out-pointers are valid.
    unsafe { ffi::g4_windowed_len(s, w, &mut begin, &mut end) };
    Ok(begin.max(0) as usize..end.max(0) as usize)
}

/// `proportional_rope_freq_factors` (idea/mod.rs:162-165): the head_dim / 2
/// `rope_freqs` divisors of a global layer.
pub fn proportional_rope_freq_factors(head_dim: usize, p: f32) -> Result<Vec<f32>, EngError> {
    let d = to_c_int(head_dim, "head_dim")?;
    let mut out = vec![0.0f32; head_dim / 2];
    // SAFETY: out holds head_dim / 2 floats.
    unsafe { ffi::g4_proportional_rope_freq_factors(d, p, out.as_mut_ptr()) };
    Ok(out)
}
