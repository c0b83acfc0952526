//! `MlpLayer::forward_into` with two int8 per-row projections (mlp.rs:157-211):
//! h = ReLU^2(x W_up + b_up) in f32, then h W_down + b_down, each projection
//! quantizing its input per token on the device; one library call.  Outside
//! the device envelope the library's host twin runs (gemm.rs:290-310).
use std::sync::{Arc, Mutex};

use nemotron_hip_sys as sys;

use crate::device::{Context, DeviceBuffer};
use crate::error::{call, HipError};
use crate::linear::Int8PerRowWeights;

pub struct Int8Mlp {
    up: Int8PerRowWeights,
    down: Int8PerRowWeights,
    workspace: Mutex<Option<DeviceBuffer<u8>>>,
}

impl Int8Mlp {
    /// `up`: hidden -> intermediate, `down`: intermediate -> hidden, on one
    /// context (MlpLayer::new's ProjectionShapeMismatch checks, mlp.rs:103-120).
    pub fn new(up: Int8PerRowWeights, down: Int8PerRowWeights) -> Result<Self, HipError> {
        if up.output_dim() != down.input_dim() || down.output_dim() != up.input_dim() {
            return Err(HipError::InvalidShape(format!(
                "up_projection {}x{} and down_projection {}x{} do not form an MLP",
                up.input_dim(),
                up.output_dim(),
                down.input_dim(),
                down.output_dim()
            )));
        }
        if !Arc::ptr_eq(up.context(), down.context()) {
            return Err(HipError::InvalidParams("up and down projections live on different contexts".into()));
        }
        Ok(Self { up, down, workspace: Mutex::new(None) })
    }

    pub fn hidden_dim(&self) -> usize {
        self.up.input_dim()
    }

    pub fn intermediate_dim(&self) -> usize {
        self.up.output_dim()
    }

    pub(crate) fn up(&self) -> &Int8PerRowWeights {
        &self.up
    }

    pub(crate) fn down(&self) -> &Int8PerRowWeights {
        &self.down
    }

    /// Whether the device entry point runs `row_count` rows of this MLP.
    pub fn device_supports(&self, row_count: usize) -> bool {
        unsafe { sys::nh_supports_mlp_w8a8(row_count, self.hidden_dim(), self.intermediate_dim()) != 0 }
    }

    /// The host twin (`nh_mlp_w8a8_host`) on host slices, bit for bit the device result.
    fn forward_host(&self, input: &[f32], row_count: usize, output: &mut [f32]) -> Result<(), HipError> {
        let (h, i) = (self.hidden_dim(), self.intermediate_dim());
        self.up.with_host(|u| {
            self.down.with_host(|d| {
                call(|e| unsafe {
                    sys::nh_mlp_w8a8_host(
                        input.as_ptr().cast(),
                        sys::nh_dtype::F32,
                        u.codes.as_ptr(),
                        u.scales.as_ptr(),
                        u.bias_ptr(),
                        d.codes.as_ptr(),
                        d.scales.as_ptr(),
                        d.bias_ptr(),
                        row_count,
                        h,
                        i,
                        output.as_mut_ptr().cast(),
                        sys::nh_dtype::F32,
                        e,
                    )
                })
            })
        })
    }

    /// `input`, `output` f32 `[row_count][hidden]` host slices; the
    /// reference's checks in its order (InvalidRowCount, "input", "output").
    /// A non-finite value is NonFiniteInput with argument "input" (index into
    /// `input`) or "intermediate" (index into the `[row_count][intermediate]`
    /// ReLU^2 output).  Synchronous; outside the device envelope (or on an
    /// Unsupported device call) the host twin computes the same result.
    pub fn forward_into(&self, input: &[f32], row_count: usize, output: &mut [f32]) -> Result<(), HipError> {
        let (h, i) = (self.hidden_dim(), self.intermediate_dim());
        if row_count == 0 {
            return Err(HipError::InvalidRowCount(row_count));
        }
        if input.len() != row_count * h {
            return Err(HipError::LengthMismatch { argument: "input", expected: row_count * h, actual: input.len() });
        }
        if output.len() != row_count * h {
            return Err(HipError::LengthMismatch {
                argument: "output",
                expected: row_count * h,
                actual: output.len(),
            });
        }
        if !self.device_supports(row_count) {
            return self.forward_host(input, row_count, output);
        }
        let ctx: &Arc<Context> = self.up.context();
        let x = DeviceBuffer::from_host(ctx, input)?;
        let mut y = DeviceBuffer::<f32>::new(ctx, output.len())?;
        let mut word = DeviceBuffer::<u64>::zeroed(ctx, 1)?;
        let need = unsafe { sys::nh_mlp_w8a8_workspace_size(row_count, h, i) };
        let mut guard = self.workspace.lock().unwrap_or_else(|p| p.into_inner());
        if guard.as_ref().map_or(true, |w| w.bytes() < need) {
            *guard = Some(DeviceBuffer::<u8>::new(ctx, need)?);
        }
        let ws = guard.as_mut().expect("workspace allocated above");
        let r = call(|e| unsafe {
            sys::nh_mlp_w8a8(
                ctx.as_raw(),
                x.as_ptr().cast(),
                sys::nh_dtype::F32,
                self.up.codes_ptr(),
                self.up.scales_ptr(),
                self.up.bias_ptr(),
                self.down.codes_ptr(),
                self.down.scales_ptr(),
                self.down.bias_ptr(),
                row_count,
                h,
                i,
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
            return self.forward_host(input, row_count, output);
        }
        r?;
        call(|e| unsafe { sys::nh_take_nonfinite(ctx.as_raw(), word.as_mut_ptr(), core::ptr::null_mut(), e) })?;
        y.copy_to_host(output)
    }
}
