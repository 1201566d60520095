//! The per-device context, streams and device memory.

use std::ffi::{c_int, c_void};
use std::fmt;
use std::marker::PhantomData;
use std::mem::size_of;
use std::ptr;
use std::sync::{Arc, Mutex, PoisonError};

use llm_eng::EngError;

use crate::error::check;
use crate::ffi;

/// One `g4_ctx`: a device's split-K workspace and softmax status word.
/// Every call that passes the context holds its lock, so threads may share
/// it; the device work of those calls shares the workspace, so it must still
/// be ordered on one stream (or synchronized) by the caller.
pub struct Context {
    raw: Mutex<RawCtx>,
    device: i32,
}

struct RawCtx(*mut ffi::G4Ctx);

// SAFETY: the pointer is dereferenced only by the C side, under the mutex.
unsafe impl Send for RawCtx {}

impl Context {
    /// `g4_init(device)`.
    pub fn new(device: i32) -> Result<Self, EngError> {
        let mut raw: *mut ffi::G4Ctx = ptr::null_mut();
        // SAFETY: raw is a valid out-pointer.
        check(unsafe { ffi::g4_init(device, &mut raw) })?;
        Ok(Self { raw: Mutex::new(RawCtx(raw)), device })
    }

    pub fn device(&self) -> i32 {
        self.device
    }

    /// Makes the context's device the calling thread's current HIP device
    /// (`g4_activate`), for the device-pointer calls that run on it.
    pub fn activate(&self) -> Result<(), EngError> {
        // SAFETY: the context is live.
        self.call(|c| unsafe { ffi::g4_activate(c) })
    }

    /// Runs one C entry point with the raw context, under the lock, and
    /// maps its status.  (Entry points that allocate or copy make the
    /// context's device current themselves.)
    pub(crate) fn call(&self, f: impl FnOnce(*mut ffi::G4Ctx) -> c_int) -> Result<(), EngError> {
        let guard = self.raw.lock().unwrap_or_else(PoisonError::into_inner);
        check(f(guard.0))
    }
}

impl Drop for Context {
    fn drop(&mut self) {
        let raw = self.raw.get_mut().unwrap_or_else(PoisonError::into_inner).0;
        // SAFETY: raw came from g4_init and is released once.
        unsafe { ffi::g4_release(raw) };
    }
}

impl fmt::Debug for Context {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        f.debug_struct("Context").field("device", &self.device).finish()
    }
}

/// A `hipStream_t` owned by the caller; `Stream::NULL` is the null stream.
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub struct Stream(*mut c_void);

// SAFETY: a HIP stream handle may be used from any thread.
unsafe impl Send for Stream {}
unsafe impl Sync for Stream {}

impl Stream {
    pub const NULL: Stream = Stream(ptr::null_mut());

    /// # Safety
    /// `raw` is null or a valid `hipStream_t` of the context's device, and
    /// stays valid for as long as this value (or a port holding it) is used.
    pub unsafe fn from_raw(raw: *mut c_void) -> Self {
        Self(raw)
    }

    pub fn as_raw(self) -> *mut c_void {
        self.0
    }
}

impl Default for Stream {
    fn default() -> Self {
        Stream::NULL
    }
}

/// An owned device allocation of `len` values of `T` on a context's device
/// (`g4_alloc`, freed by `g4_free` on drop).  Zero-length buffers allocate
/// nothing.
pub struct DeviceVec<T: Copy> {
    ptr: *mut T,
    len: usize,
    ctx: Arc<Context>,
    _owns: PhantomData<T>,
}

/// The port's buffer: f32 values in HBM, the device image of `F32Buf`
/// (crates/llm-backend-cpu/src/buffer.rs:1-26).
pub type DevBuf = DeviceVec<f32>;

// SAFETY: the allocation is owned by the value; reads need &self and writes
// &mut self.
unsafe impl<T: Copy + Send> Send for DeviceVec<T> {}
unsafe impl<T: Copy + Sync> Sync for DeviceVec<T> {}

impl<T: Copy> DeviceVec<T> {
    /// `len` values whose contents are whatever the allocation held.
    pub fn uninit(ctx: &Arc<Context>, len: usize) -> Result<Self, EngError> {
        let bytes = len
            .checked_mul(size_of::<T>())
            .ok_or_else(|| EngError::Msg(format!("a device buffer of {len} values overflows usize")))?;
        let mut raw: *mut c_void = ptr::null_mut();
        let out: *mut *mut c_void = &mut raw;
        // SAFETY: out is a valid out-pointer.
        ctx.call(|c| unsafe { ffi::g4_alloc(c, bytes, out) })?;
        Ok(Self { ptr: raw.cast(), len, ctx: Arc::clone(ctx), _owns: PhantomData })
    }

    /// A device copy of `values` (synchronous).
    pub fn from_slice(ctx: &Arc<Context>, values: &[T]) -> Result<Self, EngError> {
        let mut buf = Self::uninit(ctx, values.len())?;
        buf.copy_from_slice(values)?;
        Ok(buf)
    }

    /// Overwrites the buffer with `values`, after the device's queued work.
    pub fn copy_from_slice(&mut self, values: &[T]) -> Result<(), EngError> {
        if values.len() != self.len {
            return Err(EngError::Msg(format!(
                "copy of {} values into a device buffer of {}",
                values.len(),
                self.len
            )));
        }
        let (dst, src, bytes) = (self.ptr.cast::<c_void>(), values.as_ptr().cast::<c_void>(), self.bytes());
        // SAFETY: source and destination both hold `bytes` bytes.
        self.ctx.call(|c| unsafe { ffi::g4_copy_to_device(c, dst, src, bytes) })
    }

    /// The values on the host, after the device's queued work.
    pub fn to_vec(&self) -> Result<Vec<T>, EngError> {
        let mut out = Vec::<T>::with_capacity(self.len);
        let (dst, src, bytes) = (out.as_mut_ptr().cast::<c_void>(), self.ptr.cast_const().cast::<c_void>(), self.bytes());
        // SAFETY: out has room for self.len values; the copy writes all of
        // them before set_len.
        self.ctx.call(|c| unsafe { ffi::g4_copy_to_host(c, dst, src, bytes) })?;
        unsafe { out.set_len(self.len) };
        Ok(out)
    }

    /// A second device buffer with the same values (synchronous).
    pub fn try_clone(&self) -> Result<Self, EngError> {
        let copy = Self::uninit(&self.ctx, self.len)?;
        let (dst, src, bytes) = (copy.ptr.cast::<c_void>(), self.ptr.cast_const().cast::<c_void>(), self.bytes());
        // SAFETY: both allocations hold `bytes` bytes.
        self.ctx.call(|c| unsafe { ffi::g4_copy_on_device(c, dst, src, bytes) })?;
        Ok(copy)
    }

    pub fn len(&self) -> usize {
        self.len
    }

    pub fn is_empty(&self) -> bool {
        self.len == 0
    }

    /// The device address (null when empty).
    pub fn as_ptr(&self) -> *const T {
        self.ptr
    }

    pub fn as_mut_ptr(&mut self) -> *mut T {
        self.ptr
    }

    /// The context the buffer was allocated on.
    pub fn context(&self) -> &Arc<Context> {
        &self.ctx
    }

    fn bytes(&self) -> usize {
        self.len * size_of::<T>()
    }
}

impl<T: Copy> Drop for DeviceVec<T> {
    fn drop(&mut self) {
        if !self.ptr.is_null() {
            let p = self.ptr.cast::<c_void>();
            // SAFETY: p came from g4_alloc on this context and is freed once;
            // g4_free waits for the device work that may still use it.
            let _ = self.ctx.call(|c| unsafe { ffi::g4_free(c, p) });
        }
    }
}

impl<T: Copy> fmt::Debug for DeviceVec<T> {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        f.debug_struct("DeviceVec").field("len", &self.len).field("ptr", &self.ptr).finish()
    }
}
