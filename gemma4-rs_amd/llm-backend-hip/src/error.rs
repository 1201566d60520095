//! Status codes of the C ABI -> `EngError` (crates/llm-eng/src/error.rs:3-15),
//! variant and payload as the CPU backend produces them.

use std::ffi::{c_int, CStr};

use llm_eng::EngError;

use crate::ffi;

/// `g4_status` -> `Result`.  `g4_last_error()` holds the failure's payload
/// text on the calling thread (the `Compute` / `Msg` message, or the full
/// text of the other variants); `g4_last_error_fields()` the numbers of
/// `ContextTooLong { got, max }` and `MissingLayer(layer)`.
pub fn check(code: c_int) -> Result<(), EngError> {
    if code == ffi::G4_OK {
        return Ok(());
    }
    // SAFETY: g4_last_error returns a NUL-terminated thread-local string that
    // lives until the next failing call on this thread; it is copied at once.
    let text = unsafe { CStr::from_ptr(ffi::g4_last_error()) }.to_string_lossy().into_owned();
    let (mut a, mut b) = (0u64, 0u64);
    // SAFETY: both pointers are valid for one u64 write.
    unsafe { ffi::g4_last_error_fields(&mut a, &mut b) };
    Err(match code {
        ffi::G4_ERR_CONTEXT_TOO_LONG => EngError::ContextTooLong { got: a as usize, max: b as usize },
        ffi::G4_ERR_MISSING_LAYER => EngError::MissingLayer(a as usize),
        ffi::G4_ERR_MISSING_WEIGHT => EngError::MissingWeight(text),
        ffi::G4_ERR_COMPUTE => EngError::Compute(text),
        _ => EngError::Msg(text),
    })
}

/// The CPU backend's `compute_error` (crates/llm-backend-cpu/src/ops.rs:5-7).
pub(crate) fn compute_error(message: impl Into<String>) -> EngError {
    EngError::Compute(message.into())
}

/// A host length as the ABI's `int64_t`; lengths of allocated buffers always fit.
pub(crate) fn len_i64(len: usize) -> Result<i64, EngError> {
    i64::try_from(len).map_err(|_| EngError::Msg(format!("length {len} exceeds the C ABI's int64_t")))
}

/// A head count or width as the ABI's `int`.
pub(crate) fn to_c_int(value: usize, what: &str) -> Result<c_int, EngError> {
    c_int::try_from(value).map_err(|_| EngError::Msg(format!("{what} {value} exceeds the C ABI's int")))
}
