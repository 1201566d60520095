//! Mat-vecs over GGUF weights kept in HBM in their file layout
//! (crates/llm-backend-cpu/src/matvec.rs): Q8_0 rows of cols/32 blocks of 34
//! bytes (f16 scale, 32 int8), BF16 or f32 values, [rows][cols].  As in the
//! reference, cols is the activation's length and the weight's size is
//! checked against rows x cols with its messages ("Q8_0 weight has N
//! elements, expected R rows of L").  Each call queues its kernel on the
//! port's stream.

use llm_eng::EngError;

use crate::device::{DevBuf, DeviceVec};
use crate::error::{compute_error, len_i64};
use crate::ffi;
use crate::port::HipPort;

/// A Q8_0 activation on the device (`Q8Activation`, matvec.rs:14-33): one
/// f32 scale per 32 values (the f16 rounding of max|x| / 127) and the int8
/// quants.
#[derive(Debug)]
pub struct DeviceQ8 {
    pub scales: DevBuf,
    pub quants: DeviceVec<i8>,
}

impl HipPort {
    /// `quantize_q8_0` (matvec.rs:35-53); x.len() a multiple of 32.
    pub fn quantize_q8_0(&self, x: &DevBuf) -> Result<DeviceQ8, EngError> {
        let n = len_i64(x.len())?;
        let mut scales = self.alloc(x.len() / 32)?;
        let mut quants = DeviceVec::<i8>::uninit(self.context(), x.len())?;
        let (px, ps, pq, stream) = (x.as_ptr(), scales.as_mut_ptr(), quants.as_mut_ptr(), self.stream().as_raw());
        // SAFETY: x holds n floats, scales n/32 and quants n (a length that is
        // not a multiple of 32 is rejected before any access).
        self.context().call(|ctx| unsafe { ffi::g4_quantize_q8_0(ctx, px, n, ps, pq, stream) })?;
        Ok(DeviceQ8 { scales, quants })
    }

    /// `matvec_q8_0` (matvec.rs:55-62): W x for a Q8_0 activation.
    pub fn matvec_q8_0(&self, weights: &DeviceVec<u8>, rows: usize, x: &DeviceQ8) -> Result<DevBuf, EngError> {
        self.q8_activation_call(weights, None, rows, x, Q8Op::Plain)
    }

    /// `matvec_q8_0_then(.., softcap, cap)` (matvec.rs:64-81, model.rs:447):
    /// cap * tanh(W x / cap), the final logits.
    pub fn matvec_q8_0_softcap(&self, weights: &DeviceVec<u8>, rows: usize, x: &DeviceQ8, cap: f32) -> Result<DevBuf, EngError> {
        self.q8_activation_call(weights, None, rows, x, Q8Op::Softcap(cap))
    }

    /// `geglu_q8_0` (matvec.rs:83-102): gelu(gate x) * (up x); `fp16_gelu`
    /// picks `gelu_tanh_fp16_table` (ops.rs:85-103).
    pub fn geglu_q8_0(
        &self,
        gate: &DeviceVec<u8>,
        up: &DeviceVec<u8>,
        rows: usize,
        x: &DeviceQ8,
        fp16_gelu: bool,
    ) -> Result<DevBuf, EngError> {
        if gate.len() != up.len() {
            return Err(compute_error("gate and up weights differ in size"));
        }
        self.q8_activation_call(gate, Some(up), rows, x, Q8Op::Geglu(fp16_gelu))
    }

    /// `project` with Q8_0 weights (model.rs:205-224): the activation's
    /// quantization and the mat-vec in one launch.
    pub fn project_q8_0(&self, weights: &DeviceVec<u8>, rows: usize, x: &DevBuf) -> Result<DevBuf, EngError> {
        self.q8_f32_call(weights, None, rows, x, Q8F32Op::Project)
    }

    /// `gated_ffn_input` (model.rs:229-243) with Q8_0 weights, quantization
    /// folded in.
    pub fn gated_ffn_q8_0(
        &self,
        gate: &DeviceVec<u8>,
        up: &DeviceVec<u8>,
        rows: usize,
        x: &DevBuf,
        fp16_gelu: bool,
    ) -> Result<DevBuf, EngError> {
        if gate.len() != up.len() {
            return Err(compute_error("gate and up weights differ in size"));
        }
        self.q8_f32_call(gate, Some(up), rows, x, Q8F32Op::GatedFfn(fp16_gelu))
    }

    /// The output head (model.rs:440-449): soft-capped logits, quantization
    /// folded in.
    pub fn logits_q8_0(&self, weights: &DeviceVec<u8>, rows: usize, x: &DevBuf, cap: f32) -> Result<DevBuf, EngError> {
        self.q8_f32_call(weights, None, rows, x, Q8F32Op::Logits(cap))
    }

    /// `matvec_q8_0_f32` / `matvec_q8_0_f64_sums` (matvec.rs:104-122): an f32
    /// activation against the dequantized blocks.
    pub fn matvec_q8_0_f32(&self, weights: &DeviceVec<u8>, rows: usize, x: &DevBuf, f64_sums: bool) -> Result<DevBuf, EngError> {
        self.q8_f32_call(weights, None, rows, x, Q8F32Op::F32(f64_sums))
    }

    /// `matvec_bf16` (matvec.rs:124-130): x rounded to bf16 first.
    pub fn matvec_bf16(&self, weights: &DeviceVec<u16>, rows: usize, x: &DevBuf) -> Result<DevBuf, EngError> {
        let (w_len, r, cols) = (len_i64(weights.len())?, len_i64(rows)?, len_i64(x.len())?);
        let mut out = self.alloc(rows)?;
        let (pw, px, po, stream) = (weights.as_ptr(), x.as_ptr(), out.as_mut_ptr(), self.stream().as_raw());
        // SAFETY: w_len = rows * cols is checked before any access; x holds
        // cols floats and out rows.
        self.context().call(|ctx| unsafe { ffi::g4_matvec_bf16(ctx, pw, w_len, r, cols, px, po, stream) })?;
        Ok(out)
    }

    /// `matvec_f32` (matvec.rs:132-136).
    pub fn matvec_f32(&self, weights: &DevBuf, rows: usize, x: &DevBuf) -> Result<DevBuf, EngError> {
        let (w_len, r, cols) = (len_i64(weights.len())?, len_i64(rows)?, len_i64(x.len())?);
        let mut out = self.alloc(rows)?;
        let (pw, px, po, stream) = (weights.as_ptr(), x.as_ptr(), out.as_mut_ptr(), self.stream().as_raw());
        // SAFETY: as matvec_bf16.
        self.context().call(|ctx| unsafe { ffi::g4_matvec_f32(ctx, pw, w_len, r, cols, px, po, stream) })?;
        Ok(out)
    }

    fn q8_activation_call(
        &self,
        w: &DeviceVec<u8>,
        w2: Option<&DeviceVec<u8>>,
        rows: usize,
        x: &DeviceQ8,
        op: Q8Op,
    ) -> Result<DevBuf, EngError> {
        if x.scales.len().checked_mul(32) != Some(x.quants.len()) {
            return Err(compute_error("a Q8_0 activation has one scale per 32 quants"));
        }
        let (w_bytes, r, cols) = (len_i64(w.len())?, len_i64(rows)?, len_i64(x.quants.len())?);
        let mut out = self.alloc(rows)?;
        let (pw, pw2) = (w.as_ptr(), w2.map_or(std::ptr::null(), |b| b.as_ptr()));
        let (ps, pq, po, stream) = (x.scales.as_ptr(), x.quants.as_ptr(), out.as_mut_ptr(), self.stream().as_raw());
        // SAFETY: the weights' byte counts are checked against rows x cols
        // before any access; the activation holds cols quants and cols/32
        // scales, out rows floats.
        self.context().call(|ctx| unsafe {
            match op {
                Q8Op::Plain => ffi::g4_matvec_q8_0(ctx, pw, w_bytes, r, cols, ps, pq, po, stream),
                Q8Op::Softcap(cap) => ffi::g4_matvec_q8_0_softcap(ctx, pw, w_bytes, r, cols, ps, pq, cap, po, stream),
                Q8Op::Geglu(fp16) => {
                    ffi::g4_geglu_q8_0(ctx, pw, pw2, w_bytes, r, cols, ps, pq, i32::from(fp16), po, stream)
                }
            }
        })?;
        Ok(out)
    }

    fn q8_f32_call(&self, w: &DeviceVec<u8>, w2: Option<&DeviceVec<u8>>, rows: usize, x: &DevBuf, op: Q8F32Op) -> Result<DevBuf, EngError> {
        let (w_bytes, r, cols) = (len_i64(w.len())?, len_i64(rows)?, len_i64(x.len())?);
        let mut out = self.alloc(rows)?;
        let (pw, pw2) = (w.as_ptr(), w2.map_or(std::ptr::null(), |b| b.as_ptr()));
        let (px, po, stream) = (x.as_ptr(), out.as_mut_ptr(), self.stream().as_raw());
        // SAFETY: as q8_activation_call, with x holding cols floats.
        self.context().call(|ctx| unsafe {
            match op {
                Q8F32Op::Project => ffi::g4_project_q8_0(ctx, pw, w_bytes, r, cols, px, po, stream),
                Q8F32Op::GatedFfn(fp16) => {
                    ffi::g4_gated_ffn_q8_0(ctx, pw, pw2, w_bytes, r, cols, px, i32::from(fp16), po, stream)
                }
                Q8F32Op::Logits(cap) => ffi::g4_logits_q8_0(ctx, pw, w_bytes, r, cols, px, cap, po, stream),
                Q8F32Op::F32(f64_sums) => {
                    ffi::g4_matvec_q8_0_f32(ctx, pw, w_bytes, r, cols, px, i32::from(f64_sums), po, stream)
                }
            }
        })?;
        Ok(out)
    }
}

#[derive(Clone, Copy)]
enum Q8Op {
    Plain,
    Softcap(f32),
    Geglu(bool),
}

#[derive(Clone, Copy)]
enum Q8F32Op {
    Project,
    GatedFfn(bool),
    Logits(f32),
    F32(bool),
}
