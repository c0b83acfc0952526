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
//! - [`Int4AffineWeights`]: the `LinearWeights::Int4Affine` arm
//!   (linear.rs:99-131, 316-321), projected on the device.
//! - [`kernels`]: the `nemotron-kernels` device wrappers `gemm`/`gemm_into`,
//!   `dequantize_int4` and `moe_route`.
//!
//! Every entry keeps the reference's host-fallback contract
//! (gemm.rs:290-310): outside the device envelope the library's host twin
//! computes the same result, so no shape the reference accepts fails here.
mod device;
mod error;
mod int4;
pub mod kernels;
mod linear;
mod mlp;
mod moe;

pub use device::{Context, DeviceBuffer, Stream};
pub use error::HipError;
pub use int4::Int4AffineWeights;
pub use kernels::{GemmShape, Int4Params};
pub use linear::Int8PerRowWeights;
pub use mlp::Int8Mlp;
pub use moe::{DenseExpert, Int8Moe, MoeRouting};
pub use nemotron_hip_sys as sys;
