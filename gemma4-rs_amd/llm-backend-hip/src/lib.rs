//! The MI355X (gfx950) backend of gemma4-rs, over `libg4attn.so` and the C
//! ABI of `include/g4attn.h`.
//!
//! - [`HipPort`]: `ComputePort` (crates/llm-eng/src/compute.rs:3-29) on
//!   device buffers, in the place of `CpuPort`
//!   (crates/llm-backend-cpu/src/port.rs:8-51), with its errors.
//! - Attention ([`attention`]): the model's `attend`
//!   (crates/llm-gemma4/src/impl_/model.rs:348-366) on host slices, and its
//!   device forms -- one decode step, ragged batches, chunked prefill.
//! - [`DeviceKvCache`]: `ContextMemory`'s `KvCache`
//!   (crates/llm-eng/src/context_memory.rs:11-86) in HBM, with the layer
//!   drivers that run a layer's whole attention segment
//!   (model.rs:394-410) in one call.
//! - Mat-vecs ([`matvec`]) over GGUF weight blobs uploaded once.
//!
//! Errors are `EngError` with the reference's variants and texts; the
//! status codes of the C side map back in [`error::check`].  Device memory
//! comes from the library too (`g4_alloc`, `g4_copy_*`, `g4_free`), so the
//! crate binds `libg4attn.so` alone.  Every declaration of `ffi` is checked
//! against the header by tests/test_rust_binding.py.

pub mod attention;
pub mod device;
pub mod error;
pub mod ffi;
pub mod kv;
pub mod matvec;
pub mod port;

pub use attention::{kv_source_layer, layer_is_global, proportional_rope_freq_factors, windowed_len, Heads};
pub use device::{Context, DevBuf, DeviceVec, Stream};
pub use ffi::G4Hparams;
pub use kv::{Attended, DeviceKvCache, KvRows, LayerWeights};
pub use matvec::DeviceQ8;
pub use port::HipPort;
