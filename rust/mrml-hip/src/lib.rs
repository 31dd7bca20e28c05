//! `mrml-hip`: the MI355X (gfx950) backend of MRML's decode hot path, as a
//! Rust crate over the C ABI of `libmrml_hip.so` (`include/mrml_hip.h`).
//!
//! [`HipDevice`] and [`HipBuffer`] mirror `CudaDevice` and `CudaBuffer`
//! (crates/mrml-tensor/src/cuda.rs:1243-1513, 1883-3111): the same method
//! names, argument order and meaning, so `model.rs` switches backends by
//! type name.  As there, an operator that fails to launch panics with the
//! library's message; allocation, copies and the lifecycle return
//! [`Result`].  Matrices live in the backend layouts written once by the
//! `upload_*` methods (the reference uploads raw GGUF blocks).
//!
//! Beyond the operator surface: [`Gemma2Model`] (the whole token step and the
//! chunked prefill, with the reference's penalised sampling on the device) and
//! [`GgufFile`] (the container reader).

pub mod ffi;

mod device;
mod gguf;
mod model;

pub use device::{DeviceInfo, HipArena, HipBuffer, HipDevice, HipGraph};
pub use gguf::{GgufFile, GgufTensor};
pub use model::{Gemma2Config, Gemma2Layer, Gemma2Model, Numerics, Sampler};

/// An error of the library: its status code and message.
#[derive(Clone, Debug)]
pub struct Error {
    pub status: i32,
    pub message: String,
}

impl std::fmt::Display for Error {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        write!(f, "mrml-hip status {}: {}", self.status, self.message)
    }
}

impl std::error::Error for Error {}

pub type Result<T> = std::result::Result<T, Error>;

pub(crate) fn load_error(message: String) -> Error {
    Error { status: ffi::MRML_HIP_E_NODEVICE, message }
}
