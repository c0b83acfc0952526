//! Safe layer over `nemotron-hip-sys`: the int8 per-row weight kind that
//! `nemotron-nn`'s `LinearProjection`, `MlpLayer` and `MoeLayer` route to the
//! MI355X (linear.rs:134-171, 283-342; mlp.rs:157-211; moe.rs:154-249).
//!
//! - [`Context`]: one GPU, the loaded gfx950 code object (shared, thread-safe).
//! - [`DeviceBuffer`]: owned device memory.
//! - [`HipError`]: the payload of the reference's error enums
//!   (`LinearError`, `GemmError`, `QuantizeError`, `MoeRoutingError`).
//! - [`Int8PerRowWeights`]: the `LinearWeights::Int8PerRow` variant and its
//!   `project_into` arm; [`Int8Mlp`] and [`Int8Moe`] the layer forms.
mod device;
mod error;
mod linear;
mod mlp;
mod moe;

pub use device::{Context, DeviceBuffer, Stream};
pub use error::HipError;
pub use linear::Int8PerRowWeights;
pub use mlp::Int8Mlp;
pub use moe::{DenseExpert, Int8Moe, MoeRouting};
pub use nemotron_hip_sys as sys;
