//! `DeviceKvCache`: the `KvCache` of `ContextMemory`
//! (crates/llm-eng/src/context_memory.rs:11-86) with its rows in HBM, and the
//! layer drivers that run a layer's attention segment over it
//! (crates/llm-gemma4/src/impl_/model.rs:394-410).
//!
//! Layer `l` holds up to `capacity` rows of `widths[l]` floats
//! (`n_kv_heads * head_dim(l)` on the layers that own their K/V, 0 on the
//! layers that share an earlier layer's).  A ring layer keeps only its last
//! `ring_rows[l]` positions; windows over it read exactly as over the whole
//! history.

use std::ffi::c_int;
use std::marker::PhantomData;
use std::ptr;
use std::sync::Arc;

use llm_eng::EngError;

use crate::device::{Context, DevBuf};
use crate::error::{check, compute_error, len_i64, to_c_int};
use crate::ffi;
use crate::port::HipPort;

/// Rows of one layer as one run on the device: row r of the run at
/// `k + r * row_stride` (and the same in `v`).
#[derive(Clone, Copy, Debug)]
pub struct KvRows<'a> {
    k: *const f32,
    v: *const f32,
    row_stride: usize,
    first: usize,
    len: usize,
    _cache: PhantomData<&'a DeviceKvCache>,
}

impl<'a> KvRows<'a> {
    pub fn k_ptr(&self) -> *const f32 {
        self.k
    }

    pub fn v_ptr(&self) -> *const f32 {
        self.v
    }

    /// Floats from one row to the next.
    pub fn row_stride(&self) -> usize {
        self.row_stride
    }

    /// The position of the run's first row.
    pub fn first_position(&self) -> usize {
        self.first
    }

    pub fn len(&self) -> usize {
        self.len
    }

    pub fn is_empty(&self) -> bool {
        self.len == 0
    }
}

/// What a layer step attended: rows [kv_begin, kv_end) of layer `source`
/// (`kv_source_layer`, and the window of `LocalWindowPolicy` / `GlobalPolicy`).
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub struct Attended {
    pub source: usize,
    pub kv_begin: usize,
    pub kv_end: usize,
}

/// A layer's norm and RoPE weights on the device: `attn_q_norm`,
/// `attn_k_norm` (head_dim floats each) and, on global layers, `rope_freqs`
/// (head_dim / 2 divisors).  None means no weight (plain RMS norm, or
/// divisors of 1).
#[derive(Clone, Copy, Debug, Default)]
pub struct LayerWeights<'a> {
    pub q_norm: Option<&'a DevBuf>,
    pub k_norm: Option<&'a DevBuf>,
    pub rope_freqs: Option<&'a DevBuf>,
}

/// The device-resident `ContextMemory`.
pub struct DeviceKvCache {
    raw: *mut ffi::G4KvCache,
    ctx: Arc<Context>,
    widths: Vec<usize>,
}

// SAFETY: the cache is owned by the value; calls that change it take
// &mut self, and &self calls only read its host-side row counts.
unsafe impl Send for DeviceKvCache {}
unsafe impl Sync for DeviceKvCache {}

impl DeviceKvCache {
    /// `g4_kv_create`: every layer keeps its whole history.
    pub fn new(port: &HipPort, widths: &[usize], capacity: usize) -> Result<Self, EngError> {
        Self::create(port, widths, capacity, None)
    }

    /// `g4_kv_create_ring`: layer l keeps its last `ring_rows[l]` positions
    /// (0 = its whole history).  Sliding layers need at least
    /// `sliding_window + chunk - 1`, chunk being the longest prompt chunk
    /// given to `layer_prefill`.
    pub fn with_rings(port: &HipPort, widths: &[usize], capacity: usize, ring_rows: &[usize]) -> Result<Self, EngError> {
        if ring_rows.len() != widths.len() {
            return Err(EngError::Msg("ring_rows needs one entry per layer".to_owned()));
        }
        Self::create(port, widths, capacity, Some(ring_rows))
    }

    fn create(port: &HipPort, widths: &[usize], capacity: usize, rings: Option<&[usize]>) -> Result<Self, EngError> {
        let n_layers = to_c_int(widths.len(), "layer count")?;
        let w = widths.iter().map(|&x| len_i64(x)).collect::<Result<Vec<_>, _>>()?;
        let r = match rings {
            Some(rings) => Some(rings.iter().map(|&x| len_i64(x)).collect::<Result<Vec<_>, _>>()?),
            None => None,
        };
        let capacity = len_i64(capacity)?;
        let mut raw: *mut ffi::G4KvCache = ptr::null_mut();
        let out: *mut *mut ffi::G4KvCache = &mut raw;
        // SAFETY: w (and r) hold n_layers values; out is a valid out-pointer.
        port.context().call(|ctx| unsafe {
            match &r {
                Some(r) => ffi::g4_kv_create_ring(ctx, n_layers, w.as_ptr(), capacity, r.as_ptr(), out),
                None => ffi::g4_kv_create(ctx, n_layers, w.as_ptr(), capacity, out),
            }
        })?;
        Ok(Self { raw, ctx: Arc::clone(port.context()), widths: widths.to_vec() })
    }

    pub fn n_layers(&self) -> usize {
        self.widths.len()
    }

    /// Floats per row of `layer` (0: the layer keeps no K/V).
    pub fn width(&self, layer: usize) -> Option<usize> {
        self.widths.get(layer).copied()
    }

    /// Positions appended to `layer` so far.
    pub fn len(&self, layer: usize) -> usize {
        match c_int::try_from(layer) {
            // SAFETY: raw is live; the call only reads the row count.
            Ok(l) => unsafe { ffi::g4_kv_len(self.raw, l) }.max(0) as usize,
            Err(_) => 0,
        }
    }

    /// `append` (context_memory.rs:44-51): one row of k and v.
    pub fn append(&mut self, port: &HipPort, layer: usize, k: &DevBuf, v: &DevBuf) -> Result<(), EngError> {
        self.append_rows(port, layer, k, v, 1)
    }

    /// `n` rows of k and v ([n][width] each), as n appends.
    pub fn append_rows(&mut self, port: &HipPort, layer: usize, k: &DevBuf, v: &DevBuf, n: usize) -> Result<(), EngError> {
        if let Some(&w) = self.widths.get(layer) {
            let want = w.checked_mul(n);
            if w > 0 && (want != Some(k.len()) || want != Some(v.len())) {
                return Err(compute_error(format!("K/V rows of layer {layer} are {w} floats wide")));
            }
        }
        let layer = to_c_int(layer, "layer")?;
        let n = len_i64(n)?;
        let (raw, pk, pv, stream) = (self.raw, k.as_ptr(), v.as_ptr(), port.stream().as_raw());
        self.ctx.activate()?;
        // SAFETY: k and v hold n rows of the layer's width (checked above; the
        // call rejects a layer outside the cache or one keeping no K/V first).
        check(unsafe { ffi::g4_kv_append_rows(raw, layer, pk, pv, n, stream) })
    }

    /// `view(layer, len)` (context_memory.rs:53-69): the first `len` rows;
    /// `MissingLayer` / `ContextTooLong` as the reference reports them.
    pub fn view(&self, layer: usize, len: usize) -> Result<KvRows<'_>, EngError> {
        let l = to_c_int(layer, "layer")?;
        let n = len_i64(len)?;
        let (mut k, mut v, mut stride): (*const f32, *const f32, i64) = (ptr::null(), ptr::null(), 0);
        // SAFETY: raw is live; the out-pointers are valid.
        check(unsafe { ffi::g4_kv_view(self.raw, l, n, &mut k, &mut v, &mut stride) })?;
        Ok(KvRows { k, v, row_stride: stride.max(0) as usize, first: 0, len, _cache: PhantomData })
    }

    /// The rows of positions [begin, end) of `layer` as one run, for a whole
    /// history or a ring.
    pub fn view_rows(&self, layer: usize, begin: usize, end: usize) -> Result<KvRows<'_>, EngError> {
        let l = to_c_int(layer, "layer")?;
        let (b, e) = (len_i64(begin)?, len_i64(end)?);
        let (mut k, mut v, mut stride): (*const f32, *const f32, i64) = (ptr::null(), ptr::null(), 0);
        // SAFETY: raw is live; the out-pointers are valid.
        check(unsafe { ffi::g4_kv_view_rows(self.raw, l, b, e, &mut k, &mut v, &mut stride) })?;
        Ok(KvRows {
            k,
            v,
            row_stride: stride.max(0) as usize,
            first: begin,
            len: end.saturating_sub(begin),
            _cache: PhantomData,
        })
    }

    /// `clear` (context_memory.rs:82-84).
    pub fn clear(&mut self) {
        // SAFETY: raw is live.
        unsafe { ffi::g4_kv_clear(self.raw) };
    }

    /// The attention segment of `Gemma4CpuModel::layer` for one decode
    /// position (model.rs:394-410): norm and RoPE of q (and, on a layer that
    /// owns its K/V, of k and v, appended as row `position`), the view of the
    /// source layer, the window, and attention with scale 1.  q, k, v are the
    /// layer's projections ([n_heads*d], [n_kv_heads*d]); k and v may be
    /// None on a layer that shares an earlier layer's K/V.  They may be
    /// rewritten in place.  The result goes to `out` [n_heads*d].
    #[allow(clippy::too_many_arguments)]
    pub fn layer_attention(
        &mut self,
        port: &HipPort,
        hp: &ffi::G4Hparams,
        layer: usize,
        position: usize,
        q: &mut DevBuf,
        k: Option<&mut DevBuf>,
        v: Option<&mut DevBuf>,
        weights: &LayerWeights<'_>,
        out: &mut DevBuf,
    ) -> Result<Attended, EngError> {
        let shape = LayerShape::of(hp, layer)?;
        shape.check(1, q, k.as_deref(), v.as_deref(), weights, out)?;
        let l = to_c_int(layer, "layer")?;
        let position = len_i64(position)?;
        let (pk, pv) = (mut_ptr(k), mut_ptr(v));
        let (pq, po) = (q.as_mut_ptr(), out.as_mut_ptr());
        let (qn, kn, rf) = (opt_ptr(weights.q_norm), opt_ptr(weights.k_norm), opt_ptr(weights.rope_freqs));
        let (raw, stream) = (self.raw, port.stream().as_raw());
        let (mut source, mut begin, mut end): (c_int, i64, i64) = (0, 0, 0);
        let (ps, pb, pe): (*mut c_int, *mut i64, *mut i64) = (&mut source, &mut begin, &mut end);
        let php: *const ffi::G4Hparams = hp;
        // SAFETY: every buffer holds what the layer's shape needs (checked by
        // shape.check); raw, hp and the out-values are live for the call.
        port.context().call(|ctx| unsafe {
            ffi::g4_layer_attention(ctx, raw, php, l, position, pq, pk, pv, qn, kn, rf, po, ps, pb, pe, stream)
        })?;
        Ok(Attended { source: source.max(0) as usize, kv_begin: begin.max(0) as usize, kv_end: end.max(0) as usize })
    }

    /// The same segment for `n_tokens` prompt positions pos0, pos0+1, ... in
    /// one call; run over the layers in ascending order it gives what the
    /// token-at-a-time prompt loop computes (crates/llm-idea/src/transformer.rs:40-53).
    /// q [n_tokens][n_heads*d], k/v [n_tokens][n_kv_heads*d] (None on a
    /// shared layer), out [n_tokens][n_heads*d].  Returns the source layer.
    #[allow(clippy::too_many_arguments)]
    pub fn layer_prefill(
        &mut self,
        port: &HipPort,
        hp: &ffi::G4Hparams,
        layer: usize,
        pos0: usize,
        n_tokens: usize,
        q: &mut DevBuf,
        k: Option<&mut DevBuf>,
        v: Option<&mut DevBuf>,
        weights: &LayerWeights<'_>,
        out: &mut DevBuf,
    ) -> Result<usize, EngError> {
        let shape = LayerShape::of(hp, layer)?;
        shape.check(n_tokens, q, k.as_deref(), v.as_deref(), weights, out)?;
        let l = to_c_int(layer, "layer")?;
        let (pos0, n) = (len_i64(pos0)?, len_i64(n_tokens)?);
        let (pk, pv) = (mut_ptr(k), mut_ptr(v));
        let (pq, po) = (q.as_mut_ptr(), out.as_mut_ptr());
        let (qn, kn, rf) = (opt_ptr(weights.q_norm), opt_ptr(weights.k_norm), opt_ptr(weights.rope_freqs));
        let (raw, stream) = (self.raw, port.stream().as_raw());
        let mut source: c_int = 0;
        let ps: *mut c_int = &mut source;
        let php: *const ffi::G4Hparams = hp;
        // SAFETY: as in layer_attention, for n_tokens rows.
        port.context().call(|ctx| unsafe {
            ffi::g4_layer_prefill(ctx, raw, php, l, pos0, n, pq, pk, pv, qn, kn, rf, po, ps, stream)
        })?;
        Ok(source.max(0) as usize)
    }
}

impl Drop for DeviceKvCache {
    fn drop(&mut self) {
        // g4_kv_destroy waits for the device before freeing the rows.
        let _ = self.ctx.activate();
        // SAFETY: raw came from g4_kv_create* and is destroyed once; ctx
        // (which the cache refers to) is still alive.
        unsafe { ffi::g4_kv_destroy(self.raw) };
    }
}

fn opt_ptr(buf: Option<&DevBuf>) -> *const f32 {
    buf.map_or(ptr::null(), |b| b.as_ptr())
}

fn mut_ptr(buf: Option<&mut DevBuf>) -> *mut f32 {
    buf.map_or(ptr::null_mut(), |b| b.as_mut_ptr())
}

/// Widths of one layer's buffers, from the hyper-parameters and the
/// policies (`layer_attention_kind`, `kv_source_layer`).
struct LayerShape {
    head_dim: usize,
    q_width: usize,
    kv_width: usize,
    owner: bool,
    global: bool,
}

impl LayerShape {
    fn of(hp: &ffi::G4Hparams, layer: usize) -> Result<Self, EngError> {
        let count = |x: c_int, what: &str| {
            usize::try_from(x).ok().filter(|&x| x > 0).ok_or_else(|| EngError::Msg(format!("{what} must be positive")))
        };
        let n_layers = count(hp.n_layers, "n_layers")?;
        if layer >= n_layers {
            return Err(compute_error("g4_layer_attention: layer outside n_layers"));
        }
        let l = to_c_int(layer, "layer")?;
        // SAFETY: pure functions of their arguments.
        let global = unsafe { ffi::g4_layer_is_global(hp.n_layers, l) } != 0;
        let mut source: c_int = 0;
        check(unsafe { ffi::g4_kv_source_layer(hp.n_layers, hp.shared_kv_layers, l, &mut source) })?;
        let head_dim = count(if global { hp.head_dim_global } else { hp.head_dim_local }, "head_dim")?;
        let n_heads = count(hp.n_heads, "n_heads")?;
        let n_kv_heads = count(hp.n_kv_heads, "n_kv_heads")?;
        Ok(Self {
            head_dim,
            q_width: n_heads * head_dim,
            kv_width: n_kv_heads * head_dim,
            owner: source == l,
            global,
        })
    }

    /// Every buffer the C call reads or writes holds what it will touch.
    fn check(
        &self,
        n_tokens: usize,
        q: &DevBuf,
        k: Option<&DevBuf>,
        v: Option<&DevBuf>,
        weights: &LayerWeights<'_>,
        out: &DevBuf,
    ) -> Result<(), EngError> {
        let bad = |what: &str, want: usize, got: usize| {
            Err(compute_error(format!("{what} holds {got} floats, the layer needs {want}")))
        };
        let overflow = || compute_error("token count overflows");
        let q_len = self.q_width.checked_mul(n_tokens).ok_or_else(overflow)?;
        let kv_len = self.kv_width.checked_mul(n_tokens).ok_or_else(overflow)?;
        if q.len() != q_len {
            return bad("q", q_len, q.len());
        }
        if out.len() != q_len {
            return bad("out", q_len, out.len());
        }
        if self.owner {
            match (k, v) {
                (Some(k), Some(v)) => {
                    if k.len() != kv_len {
                        return bad("k", kv_len, k.len());
                    }
                    if v.len() != kv_len {
                        return bad("v", kv_len, v.len());
                    }
                }
                _ => return Err(compute_error("a layer that owns its K/V needs k and v")),
            }
        }
        for (name, w) in [("attn_q_norm", weights.q_norm), ("attn_k_norm", weights.k_norm)] {
            if let Some(w) = w {
                if w.len() != self.head_dim {
                    return bad(name, self.head_dim, w.len());
                }
            }
        }
        if let (true, Some(f)) = (self.global, weights.rope_freqs) {
            if f.len() < self.head_dim / 2 {
                return bad("rope_freqs", self.head_dim / 2, f.len());
            }
        }
        Ok(())
    }
}
