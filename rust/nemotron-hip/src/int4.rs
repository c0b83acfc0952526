//! The INT4 affine weight kind of `LinearProjection`
//! (`Int4LinearWeights`, linear.rs:99-131): the `[input_dim][output_dim]`
//! affine codes packed two per byte (low nibble first, quantize.rs:75-77)
//! with one scale and zero point.  The reference's `project_into` rejects
//! this arm (linear.rs:316-321); on the MI355X it projects: the codes stay
//! 4-bit on the device and the layer is the W8A8 linear with weights
//! `code - zero_point` and every row scale equal to `scale`
//! (`nh_linear_w4a8`), with the library's host twin on the packed layout
//! outside the device envelope.
use std::sync::{Arc, Mutex};

use nemotron_hip_sys as sys;

use crate::device::{Context, DeviceBuffer};
use crate::error::{call, HipError};
use crate::kernels::Int4Params;

pub struct Int4AffineWeights {
    ctx: Arc<Context>,
    input_dim: usize,
    output_dim: usize,
    params: Int4Params,
    packed: Vec<u8>,                 // the reference's layout, for the host twin
    tiled: DeviceBuffer<u8>,         // the device layout (nh_tile_weights_int4)
    bias: Option<Vec<f32>>,
    bias_dev: Option<DeviceBuffer<f32>>,
    workspace: Mutex<Option<DeviceBuffer<u8>>>,
}

impl Int4AffineWeights {
    /// `Int4LinearWeights::new` + validate (linear.rs:113-124): InvalidShape
    /// for a zero dimension, LengthMismatch "packed_weights", InvalidParams
    /// for the parameters (validate_int4_params, quantize.rs:180-186),
    /// LengthMismatch "bias".  The codes are repacked once into the tiled
    /// INT4 layout on the host and uploaded.
    pub fn new(
        ctx: &Arc<Context>,
        input_dim: usize,
        output_dim: usize,
        packed: &[u8],
        params: Int4Params,
        bias: Option<&[f32]>,
    ) -> Result<Self, HipError> {
        if input_dim == 0 || output_dim == 0 {
            return Err(HipError::InvalidShape(format!("input_dim={input_dim}, output_dim={output_dim}")));
        }
        let values = input_dim * output_dim;
        let want = unsafe { sys::nh_packed_int4_len(values) };
        if packed.len() != want {
            return Err(HipError::LengthMismatch { argument: "packed_weights", expected: want, actual: packed.len() });
        }
        if !params.scale.is_finite() || params.scale <= 0.0 || params.zero_point > 15 {
            return Err(HipError::InvalidParams(format!("scale={}, zero_point={}", params.scale, params.zero_point)));
        }
        if let Some(b) = bias {
            if b.len() != output_dim {
                return Err(HipError::LengthMismatch { argument: "bias", expected: output_dim, actual: b.len() });
            }
        }
        let tiled_len = unsafe { sys::nh_tiled_int4_weights_bytes(output_dim, input_dim) };
        let mut tiled = vec![0u8; tiled_len];
        call(|e| unsafe {
            sys::nh_tile_weights_int4_host(
                packed.as_ptr(),
                packed.len(),
                input_dim,
                output_dim,
                params.zero_point,
                tiled.as_mut_ptr(),
                tiled_len,
                e,
            )
        })?;
        Ok(Self {
            ctx: ctx.clone(),
            input_dim,
            output_dim,
            params,
            packed: packed.to_vec(),
            tiled: DeviceBuffer::from_host(ctx, &tiled)?,
            bias: bias.map(|b| b.to_vec()),
            bias_dev: bias.map(|b| DeviceBuffer::from_host(ctx, b)).transpose()?,
            workspace: Mutex::new(None),
        })
    }

    pub fn input_dim(&self) -> usize {
        self.input_dim
    }

    pub fn output_dim(&self) -> usize {
        self.output_dim
    }

    /// The `project_into` arm on host slices (`input` f32
    /// `[row_count][input_dim]`, `output` f32 `[row_count][output_dim]`), the
    /// reference's checks in its order; NonFiniteInput "input" for a NaN or
    /// infinity.  Synchronous.  Shapes the device does not cover run the host
    /// twin, bit-identical.
    pub fn project_into(&self, input: &[f32], row_count: usize, output: &mut [f32]) -> Result<(), HipError> {
        let (k, n) = (self.input_dim, self.output_dim);
        if row_count == 0 {
            return Err(HipError::InvalidRowCount(row_count));
        }
        if input.len() != row_count * k {
            return Err(HipError::LengthMismatch { argument: "input", expected: row_count * k, actual: input.len() });
        }
        if output.len() != row_count * n {
            return Err(HipError::LengthMismatch { argument: "output", expected: row_count * n, actual: output.len() });
        }
        let out_ptr = output.as_mut_ptr();
        let host = || {
            call(|e| unsafe {
                sys::nh_linear_w4a8_host(
                    input.as_ptr().cast(),
                    sys::nh_dtype::F32,
                    self.packed.as_ptr(),
                    self.packed.len(),
                    self.params.scale,
                    self.params.zero_point,
                    self.bias.as_ref().map_or(core::ptr::null(), |b| b.as_ptr()),
                    row_count,
                    n,
                    k,
                    out_ptr.cast(),
                    sys::nh_dtype::F32,
                    e,
                )
            })
        };
        // f32 rows take the expanded form on the device, which needs the W8A8
        // envelope (k % 16 == 0 and the dimension limits)
        if unsafe { sys::nh_supports_gemm_w8a8(row_count, n, k) } == 0 {
            return host();
        }
        let ctx = &self.ctx;
        let x = DeviceBuffer::from_host(ctx, input)?;
        let mut y = DeviceBuffer::<f32>::new(ctx, output.len())?;
        let mut word = DeviceBuffer::<u64>::zeroed(ctx, 1)?;
        let need = unsafe { sys::nh_linear_w4a8_workspace_size(row_count, n, k) };
        let mut guard = self.workspace.lock().unwrap_or_else(|p| p.into_inner());
        if guard.as_ref().map_or(true, |w| w.bytes() < need) {
            *guard = Some(DeviceBuffer::<u8>::new(ctx, need)?);
        }
        let ws = guard.as_mut().expect("workspace allocated above");
        let r = call(|e| unsafe {
            sys::nh_linear_w4a8(
                ctx.as_raw(),
                x.as_ptr().cast(),
                sys::nh_dtype::F32,
                self.tiled.as_ptr(),
                self.params.scale,
                self.params.zero_point,
                self.bias_dev.as_ref().map_or(core::ptr::null(), |b| b.as_ptr()),
                row_count,
                n,
                k,
                y.as_mut_ptr().cast(),
                sys::nh_dtype::F32,
                ws.as_mut_ptr().cast(),
                ws.bytes(),
                word.as_mut_ptr(),
                core::ptr::null_mut(),
                e,
            )
        });
        if let Err(HipError::Unsupported(_)) = r {
            drop(guard);
            return host();
        }
        r?;
        call(|e| unsafe { sys::nh_take_nonfinite(ctx.as_raw(), word.as_mut_ptr(), core::ptr::null_mut(), e) })?;
        y.copy_to_host(output)
    }
}
