//! `HipPort`: `ComputePort` (crates/llm-eng/src/compute.rs:3-29) on device
//! buffers, in the place of `CpuPort` (crates/llm-backend-cpu/src/port.rs:8-51).
//!
//! The checks `CpuPort`'s ops make on buffer lengths are made here, before
//! anything is queued, with the same `EngError::Compute` texts
//! (crates/llm-backend-cpu/src/ops.rs:9-178); the checks on values (eps,
//! theta, dims, a non-finite softmax) are made by the C entry points, which
//! report the same texts.  `matmul`, `rms_norm`, `rope` and `add` queue their
//! kernel on the port's stream and return; `softmax` waits for its result,
//! because the trait returns its failure directly.

use std::sync::Arc;

use llm_eng::{compute::ComputePort, EngError};

use crate::device::{Context, DevBuf, Stream};
use crate::error::{compute_error, len_i64};
use crate::ffi;

/// A device, its context and the stream the port's work goes to.
#[derive(Clone, Debug)]
pub struct HipPort {
    ctx: Arc<Context>,
    stream: Stream,
}

impl HipPort {
    /// A port on `device` issuing its work to the null stream.
    pub fn new(device: i32) -> Result<Self, EngError> {
        Ok(Self { ctx: Arc::new(Context::new(device)?), stream: Stream::NULL })
    }

    /// The same context with its work on `stream`.  Calls through one
    /// context share its workspace: keep them on one stream at a time.
    pub fn on_stream(&self, stream: Stream) -> Self {
        Self { ctx: Arc::clone(&self.ctx), stream }
    }

    pub fn context(&self) -> &Arc<Context> {
        &self.ctx
    }

    pub fn stream(&self) -> Stream {
        self.stream
    }

    /// `F32Buf::from(values)` on the device (synchronous).
    pub fn upload(&self, values: &[f32]) -> Result<DevBuf, EngError> {
        DevBuf::from_slice(&self.ctx, values)
    }

    /// The buffer's values once the port's queued work is done.
    pub fn download(&self, buf: &DevBuf) -> Result<Vec<f32>, EngError> {
        let stream = self.stream.as_raw();
        // SAFETY: ctx is live; stream is null or valid (Stream::from_raw).
        self.ctx.call(|ctx| unsafe { ffi::g4_sync(ctx, stream) })?;
        buf.to_vec()
    }

    /// Waits for the port's stream and reports a softmax failure recorded
    /// by earlier attention calls (`g4_check_status`).
    pub fn synchronize(&self) -> Result<(), EngError> {
        let stream = self.stream.as_raw();
        // SAFETY: ctx is live; stream is null or valid (Stream::from_raw).
        self.ctx.call(|ctx| unsafe { ffi::g4_check_status(ctx, stream) })
    }

    /// An output buffer of `len` values on the port's device.
    pub(crate) fn alloc(&self, len: usize) -> Result<DevBuf, EngError> {
        DevBuf::uninit(&self.ctx, len)
    }
}

impl ComputePort for HipPort {
    type Buffer = DevBuf;

    /// `matmul_f32` (ops.rs:9-39): a [m][k] times b [k][n], inner sums in
    /// order of k.
    fn matmul(&self, a: &DevBuf, b: &DevBuf, m: usize, n: usize, k: usize) -> Result<DevBuf, EngError> {
        let overflow = || compute_error("matmul dimensions overflow");
        let a_len = m.checked_mul(k).ok_or_else(overflow)?;
        let b_len = k.checked_mul(n).ok_or_else(overflow)?;
        if a.len() != a_len || b.len() != b_len {
            return Err(compute_error("matmul buffer shape does not match dimensions"));
        }
        let out_len = m.checked_mul(n).ok_or_else(overflow)?;
        let (m, n, k) = (
            i64::try_from(m).map_err(|_| overflow())?,
            i64::try_from(n).map_err(|_| overflow())?,
            i64::try_from(k).map_err(|_| overflow())?,
        );
        let mut out = self.alloc(out_len)?;
        let (pa, pb, po, stream) = (a.as_ptr(), b.as_ptr(), out.as_mut_ptr(), self.stream.as_raw());
        // SAFETY: a, b and out hold m*k, k*n and m*n floats (checked above).
        self.ctx.call(|ctx| unsafe { ffi::g4_port_matmul(ctx, pa, pb, m, n, k, po, stream) })?;
        Ok(out)
    }

    /// `rms_norm_f32` (ops.rs:45-60): f64 mean of squares, times the weight.
    fn rms_norm(&self, x: &DevBuf, weight: &DevBuf, eps: f32) -> Result<DevBuf, EngError> {
        if x.is_empty() || eps < 0.0 || weight.len() != x.len() {
            return Err(compute_error("invalid RMS norm inputs"));
        }
        let n = len_i64(x.len())?;
        let mut out = self.alloc(x.len())?;
        let (px, pw, po, stream) = (x.as_ptr(), weight.as_ptr(), out.as_mut_ptr(), self.stream.as_raw());
        // SAFETY: x, weight and out hold n floats.
        self.ctx.call(|ctx| unsafe { ffi::g4_port_rms_norm(ctx, px, pw, n, eps, po, stream) })?;
        Ok(out)
    }

    /// `softmax_f32` (ops.rs:105-127).  Waits for the result: an empty buffer
    /// and a non-finite sum are this call's errors.
    fn softmax(&self, x: &DevBuf) -> Result<DevBuf, EngError> {
        let n = len_i64(x.len())?;
        let mut out = self.alloc(x.len())?;
        let (px, po, stream) = (x.as_ptr(), out.as_mut_ptr(), self.stream.as_raw());
        // SAFETY: x and out hold n floats; n == 0 is rejected before any access.
        self.ctx.call(|ctx| unsafe { ffi::g4_port_softmax(ctx, px, n, po, stream) })?;
        Ok(out)
    }

    /// `rope_f32` (ops.rs:164-166): NEOX rotation of the first `dims` values
    /// at `pos`, in place.  dims == 0, odd or above the length, and theta <= 0,
    /// fail with "invalid RoPE inputs".
    fn rope(&self, x: &mut DevBuf, pos: usize, theta: f32, dims: usize) -> Result<(), EngError> {
        let invalid = || compute_error("invalid RoPE inputs");
        let len = len_i64(x.len())?;
        // A dims beyond i64 is beyond the length; a position beyond i64 is
        // beyond any context.
        let dims = i64::try_from(dims).map_err(|_| invalid())?;
        let pos = i64::try_from(pos).map_err(|_| invalid())?;
        let (px, stream) = (x.as_mut_ptr(), self.stream.as_raw());
        // SAFETY: x holds len floats; the call touches the first dims <= len.
        self.ctx.call(|ctx| unsafe { ffi::g4_port_rope(ctx, px, len, pos, theta, dims, stream) })
    }

    /// `add_f32` (ops.rs:168-178).
    fn add(&self, a: &DevBuf, b: &DevBuf) -> Result<DevBuf, EngError> {
        if a.len() != b.len() {
            return Err(compute_error("add buffer lengths differ"));
        }
        let n = len_i64(a.len())?;
        let mut out = self.alloc(a.len())?;
        let (pa, pb, po, stream) = (a.as_ptr(), b.as_ptr(), out.as_mut_ptr(), self.stream.as_raw());
        // SAFETY: a, b and out hold n floats.
        self.ctx.call(|ctx| unsafe { ffi::g4_port_add(ctx, pa, pb, n, po, stream) })?;
        Ok(out)
    }
}
