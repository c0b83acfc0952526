//! The `nemotron-kernels` device wrappers that stay in the drop-in, over
//! device buffers (the reference's `GpuTensor` arguments), each with the
//! reference's host bridge when the shape is outside the device envelope
//! (gemm.rs:290-310):
//!
//! - [`gemm`] / [`gemm_into`]: `gemm` / `gemm_into` (gemm.rs:318-363), f32
//!   with f64 accumulation in k order on the device (bit-identical to
//!   `gemm_into_host`);
//! - [`dequantize_int4`]: `dequantize_int4` (quantize.rs:332-349), packed
//!   host bytes to device f32, any value count;
//! - [`moe_route`]: `moe_route` (moe_routing.rs:499-523), sigmoid top-k.
use std::sync::Arc;

use nemotron_hip_sys as sys;

use crate::device::{Context, DeviceBuffer, Stream};
use crate::error::{call, HipError};
use crate::moe::MoeRouting;

/// `GemmShape` (gemm.rs:28-66): `lhs` `[m][k]`, `rhs` `[k][n]`, out `[m][n]`.
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub struct GemmShape {
    pub m: usize,
    pub k: usize,
    pub n: usize,
}

fn download<T: Copy + Default>(b: &DeviceBuffer<T>) -> Result<Vec<T>, HipError> {
    let mut v = vec![T::default(); b.len()];
    b.copy_to_host(&mut v)?;
    Ok(v)
}

/// `gemm`: a new `[m][n]` device buffer (synchronous on `stream`).
pub fn gemm(
    ctx: &Arc<Context>,
    lhs: &DeviceBuffer<f32>,
    rhs: &DeviceBuffer<f32>,
    shape: GemmShape,
    stream: Option<&Stream>,
) -> Result<DeviceBuffer<f32>, HipError> {
    let len = shape
        .m
        .checked_mul(shape.n)
        .ok_or_else(|| HipError::InvalidShape(format!("{shape:?} overflows")))?;
    let mut out = DeviceBuffer::<f32>::new(ctx, len)?;
    gemm_into(ctx, lhs, rhs, shape, &mut out, stream)?;
    Ok(out)
}

/// `gemm_into`: writes the caller's `[m][n]` buffer; `out.len()` must be
/// `m * n` (LengthMismatch "output", gemm.rs:341-363).  The device GEMM covers
/// every shape `nh_supports_gemm_f32` admits; otherwise the operands are
/// copied to the host, `nh_gemm_f32_host` runs and the result is copied back.
pub fn gemm_into(
    ctx: &Arc<Context>,
    lhs: &DeviceBuffer<f32>,
    rhs: &DeviceBuffer<f32>,
    shape: GemmShape,
    out: &mut DeviceBuffer<f32>,
    stream: Option<&Stream>,
) -> Result<(), HipError> {
    let GemmShape { m, k, n } = shape;
    if unsafe { sys::nh_supports_gemm_f32(m, k, n) } != 0 {
        let r = call(|e| unsafe {
            sys::nh_gemm_f32(
                ctx.as_raw(),
                lhs.as_ptr(),
                lhs.len(),
                rhs.as_ptr(),
                rhs.len(),
                m,
                k,
                n,
                out.as_mut_ptr(),
                out.len(),
                Stream::raw_or_null(stream),
                e,
            )
        });
        match r {
            Err(HipError::Unsupported(_)) => {}
            r => {
                r?;
                return ctx.synchronize(stream);
            }
        }
    }
    ctx.synchronize(stream)?;
    let (a, b) = (download(lhs)?, download(rhs)?);
    let mut o = vec![0.0f32; out.len()];
    call(|e| unsafe {
        sys::nh_gemm_f32_host(a.as_ptr(), a.len(), b.as_ptr(), b.len(), m, k, n, o.as_mut_ptr(), o.len(), e)
    })?;
    out.copy_from_host(&o)
}

/// `Int4QuantizationParams` (quantize.rs:21-31): one scale and zero point.
#[derive(Clone, Copy, Debug, PartialEq)]
pub struct Int4Params {
    pub scale: f32,
    pub zero_point: u32,
}

/// `dequantize_int4`: `packed` host bytes (two codes per byte, low nibble
/// first) to `value_count` f32 values in device memory, unpacked and
/// dequantized on the device.  Errors as the reference: InvalidParams,
/// LengthMismatch "packed".
pub fn dequantize_int4(
    ctx: &Arc<Context>,
    packed: &[u8],
    value_count: usize,
    params: Int4Params,
    stream: Option<&Stream>,
) -> Result<DeviceBuffer<f32>, HipError> {
    let dev = DeviceBuffer::from_host(ctx, packed)?;
    let mut out = DeviceBuffer::<f32>::new(ctx, value_count)?;
    call(|e| unsafe {
        sys::nh_dequantize_int4(
            ctx.as_raw(),
            dev.as_ptr(),
            packed.len(),
            value_count,
            params.scale,
            params.zero_point,
            out.as_mut_ptr(),
            value_count,
            Stream::raw_or_null(stream),
            e,
        )
    })?;
    ctx.synchronize(stream)?;
    Ok(out)
}

/// `moe_route`: sigmoid scores of `scores` `[tokens][experts]`, the top-k
/// experts per token by (weight desc, expert asc) and their weights
/// (`routing` as MoeLayer uses it: `MoeRouting::REFERENCE`).  Indices are
/// i32 (usize in the reference).  Outside the device envelope (more than 1024
/// experts or top_k above 64) the host twin runs on a host copy.
pub fn moe_route(
    ctx: &Arc<Context>,
    scores: &DeviceBuffer<f32>,
    tokens: usize,
    experts: usize,
    top_k: usize,
    routing: MoeRouting,
    stream: Option<&Stream>,
) -> Result<(DeviceBuffer<i32>, DeviceBuffer<f32>), HipError> {
    if scores.len() != tokens.saturating_mul(experts) {
        return Err(HipError::LengthMismatch {
            argument: "scores",
            expected: tokens.saturating_mul(experts),
            actual: scores.len(),
        });
    }
    let routes = tokens * top_k;
    let mut idx = DeviceBuffer::<i32>::new(ctx, routes)?;
    let mut w = DeviceBuffer::<f32>::new(ctx, routes)?;
    let r = call(|e| unsafe {
        sys::nh_moe_route_sigmoid_topk(
            ctx.as_raw(),
            scores.as_ptr(),
            tokens,
            experts,
            top_k,
            routing.renormalize as core::ffi::c_int,
            routing.scaling,
            idx.as_mut_ptr(),
            w.as_mut_ptr(),
            Stream::raw_or_null(stream),
            e,
        )
    });
    match r {
        Err(HipError::Unsupported(_)) => {
            ctx.synchronize(stream)?;
            let s = download(scores)?;
            let (mut hi, mut hw) = (vec![0i32; routes], vec![0.0f32; routes]);
            call(|e| unsafe {
                sys::nh_moe_route_sigmoid_topk_host(
                    s.as_ptr(),
                    s.len(),
                    tokens,
                    experts,
                    top_k,
                    routing.renormalize as core::ffi::c_int,
                    routing.scaling,
                    hi.as_mut_ptr(),
                    routes,
                    hw.as_mut_ptr(),
                    routes,
                    e,
                )
            })?;
            idx.copy_from_host(&hi)?;
            w.copy_from_host(&hw)?;
        }
        r => {
            r?;
            ctx.synchronize(stream)?;
        }
    }
    Ok((idx, w))
}
