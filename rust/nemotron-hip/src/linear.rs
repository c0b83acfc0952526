//! The int8 per-row weight kind of `LinearProjection` (linear.rs:134-171,
//! 283-342): codes tiled on the device, one f32 scale per output, optional
//! bias; `project_into` quantizes each input row on the device (dynamic
//! per-token scales) and runs the W8A8 GEMV/GEMM with the bias fused.
//! Outside the device envelope (`nh_supports_linear_w8a8`, e.g. an input
//! width that is not a multiple of 16) it keeps the reference's
//! host-fallback contract (gemm.rs:290-310): the weights are copied to the
//! host once and the library's host twin computes the same result.
use core::ffi::c_void;
use std::fmt;
use std::sync::{Arc, Mutex};

use nemotron_hip_sys as sys;

use crate::device::{Context, DeviceBuffer, Stream};
use crate::error::{call, HipError};

struct Inner {
    ctx: Arc<Context>,
    input_dim: usize,
    output_dim: usize,
    codes: DeviceBuffer<i8>, // tiled [output_dim][input_dim]
    scales: DeviceBuffer<f32>,
    bias: Option<DeviceBuffer<f32>>,
    // per-token quantization workspace of the host-slice entry, grown on demand
    workspace: Mutex<Option<DeviceBuffer<u8>>>,
    // host copy of the tiled codes, scales and bias for the host twin, made on first use
    host: Mutex<Option<HostWeights>>,
}

/// The weights in host memory, in the device layout (tiled codes), for the
/// library's host twins.
pub(crate) struct HostWeights {
    pub(crate) codes: Vec<i8>,
    pub(crate) scales: Vec<f32>,
    pub(crate) bias: Option<Vec<f32>>,
}

impl HostWeights {
    pub(crate) fn bias_ptr(&self) -> *const f32 {
        self.bias.as_ref().map_or(core::ptr::null(), |b| b.as_ptr())
    }
}

/// `LinearWeights::Int8PerRow`: cloning shares the device copy, and two
/// values compare equal when they share it.
#[derive(Clone)]
pub struct Int8PerRowWeights {
    inner: Arc<Inner>,
}

impl Int8PerRowWeights {
    /// Quantizes the reference's dense f32 weights, stored row-major as
    /// `[input_dim][output_dim]` (linear.rs:324), to int8 codes with one
    /// scale per output (column), then tiles and uploads them.  Validation
    /// follows `LinearProjection::from_shape`: InvalidShape for a zero
    /// dimension, LengthMismatch "bias", then LengthMismatch "weights".
    pub fn quantize_dense(
        ctx: &Arc<Context>,
        input_dim: usize,
        output_dim: usize,
        weights: &[f32],
        bias: Option<&[f32]>,
    ) -> Result<Self, HipError> {
        check_dims(input_dim, output_dim, bias)?;
        let len = input_dim * output_dim;
        if weights.len() != len {
            return Err(HipError::LengthMismatch { argument: "weights", expected: len, actual: weights.len() });
        }
        // column n of [in][out] is output row n
        let mut rows = vec![0.0f32; len];
        for k in 0..input_dim {
            for n in 0..output_dim {
                rows[n * input_dim + k] = weights[k * output_dim + n];
            }
        }
        let mut codes = vec![0i8; len];
        let mut scales = vec![0.0f32; output_dim];
        call(|e| unsafe {
            sys::nh_quantize_rows_i8_host(
                rows.as_ptr().cast(),
                sys::nh_dtype::F32,
                output_dim,
                input_dim,
                codes.as_mut_ptr(),
                scales.as_mut_ptr(),
                e,
            )
        })?;
        Self::from_quantized(ctx, input_dim, output_dim, &codes, &scales, bias)
    }

    /// Already-quantized weights: `codes` row-major `[output_dim][input_dim]`
    /// (a checkpoint's I8 tensor), `scales` `[output_dim]`.
    pub fn from_quantized(
        ctx: &Arc<Context>,
        input_dim: usize,
        output_dim: usize,
        codes: &[i8],
        scales: &[f32],
        bias: Option<&[f32]>,
    ) -> Result<Self, HipError> {
        check_dims(input_dim, output_dim, bias)?;
        if codes.len() != input_dim * output_dim {
            return Err(HipError::LengthMismatch {
                argument: "codes",
                expected: input_dim * output_dim,
                actual: codes.len(),
            });
        }
        if scales.len() != output_dim {
            return Err(HipError::LengthMismatch { argument: "scales", expected: output_dim, actual: scales.len() });
        }
        let tiled_len = unsafe { sys::nh_tiled_weights_bytes(output_dim, input_dim) };
        let mut tiled = vec![0i8; tiled_len];
        call(|e| unsafe {
            sys::nh_tile_weights_i8_host(codes.as_ptr(), output_dim, input_dim, tiled.as_mut_ptr(), tiled_len, e)
        })?;
        Ok(Self::assemble(
            ctx,
            input_dim,
            output_dim,
            DeviceBuffer::from_host(ctx, &tiled)?,
            DeviceBuffer::from_host(ctx, scales)?,
            bias,
        )?)
    }

    /// An int8 layer stored in a safetensors file: `codes_name` I8
    /// `[output_dim][input_dim]`, `scales_name` F32 `[output_dim]`.
    pub fn from_safetensors(
        ctx: &Arc<Context>,
        path: &str,
        codes_name: &str,
        scales_name: &str,
        input_dim: usize,
        output_dim: usize,
        bias: Option<&[f32]>,
    ) -> Result<Self, HipError> {
        check_dims(input_dim, output_dim, bias)?;
        let cstr = |s: &str| std::ffi::CString::new(s).map_err(|_| HipError::Io("name holds a NUL byte".into()));
        let (path_c, codes_c, scales_c) = (cstr(path)?, cstr(codes_name)?, cstr(scales_name)?);
        let mut staging = DeviceBuffer::<i8>::new(ctx, input_dim * output_dim)?;
        let tiled_len = unsafe { sys::nh_tiled_weights_bytes(output_dim, input_dim) };
        let mut tiled = DeviceBuffer::<i8>::new(ctx, tiled_len)?;
        let mut scales = DeviceBuffer::<f32>::new(ctx, output_dim)?;
        call(|e| unsafe {
            sys::nh_load_linear_i8(
                ctx.as_raw(),
                path_c.as_ptr(),
                codes_c.as_ptr(),
                scales_c.as_ptr(),
                output_dim,
                input_dim,
                staging.as_mut_ptr().cast(),
                staging.bytes(),
                tiled.as_mut_ptr(),
                tiled_len,
                scales.as_mut_ptr(),
                e,
            )
        })?;
        drop(staging);
        Self::assemble(ctx, input_dim, output_dim, tiled, scales, bias)
    }

    fn assemble(
        ctx: &Arc<Context>,
        input_dim: usize,
        output_dim: usize,
        codes: DeviceBuffer<i8>,
        scales: DeviceBuffer<f32>,
        bias: Option<&[f32]>,
    ) -> Result<Self, HipError> {
        let bias = match bias {
            Some(b) => Some(DeviceBuffer::from_host(ctx, b)?),
            None => None,
        };
        Ok(Self {
            inner: Arc::new(Inner {
                ctx: ctx.clone(),
                input_dim,
                output_dim,
                codes,
                scales,
                bias,
                workspace: Mutex::new(None),
                host: Mutex::new(None),
            }),
        })
    }

    pub fn input_dim(&self) -> usize {
        self.inner.input_dim
    }

    pub fn output_dim(&self) -> usize {
        self.inner.output_dim
    }

    pub fn context(&self) -> &Arc<Context> {
        &self.inner.ctx
    }

    pub(crate) fn codes_ptr(&self) -> *const i8 {
        self.inner.codes.as_ptr()
    }

    pub(crate) fn scales_ptr(&self) -> *const f32 {
        self.inner.scales.as_ptr()
    }

    pub(crate) fn bias_ptr(&self) -> *const f32 {
        self.inner.bias.as_ref().map_or(core::ptr::null(), |b| b.as_ptr())
    }

    pub(crate) fn has_bias(&self) -> bool {
        self.inner.bias.is_some()
    }

    /// Runs `f` on the host copy of the weights (downloaded on first use:
    /// the host bridge of gemm.rs:301-310, once per layer instead of per call).
    pub(crate) fn with_host<R>(&self, f: impl FnOnce(&HostWeights) -> Result<R, HipError>) -> Result<R, HipError> {
        let mut guard = self.inner.host.lock().unwrap_or_else(|p| p.into_inner());
        if guard.is_none() {
            let mut codes = vec![0i8; self.inner.codes.len()];
            self.inner.codes.copy_to_host(&mut codes)?;
            let mut scales = vec![0.0f32; self.inner.scales.len()];
            self.inner.scales.copy_to_host(&mut scales)?;
            let bias = match self.inner.bias.as_ref() {
                Some(b) => {
                    let mut v = vec![0.0f32; b.len()];
                    b.copy_to_host(&mut v)?;
                    Some(v)
                }
                None => None,
            };
            *guard = Some(HostWeights { codes, scales, bias });
        }
        f(guard.as_ref().expect("host copy made above"))
    }

    /// Whether the device entry point runs `row_count` rows of this layer.
    pub fn device_supports(&self, row_count: usize) -> bool {
        unsafe { sys::nh_supports_linear_w8a8(row_count, self.inner.output_dim, self.inner.input_dim) != 0 }
    }

    /// The host twin (`nh_linear_w8a8_host`) on host slices: the same result
    /// as the device, bit for bit.
    fn project_host(&self, input: &[f32], row_count: usize, output: &mut [f32]) -> Result<(), HipError> {
        let (k, n) = (self.inner.input_dim, self.inner.output_dim);
        self.with_host(|w| {
            call(|e| unsafe {
                sys::nh_linear_w8a8_host(
                    input.as_ptr().cast(),
                    sys::nh_dtype::F32,
                    w.codes.as_ptr(),
                    w.scales.as_ptr(),
                    w.bias_ptr(),
                    row_count,
                    n,
                    k,
                    output.as_mut_ptr().cast(),
                    sys::nh_dtype::F32,
                    core::ptr::null_mut(),
                    core::ptr::null_mut(),
                    e,
                )
            })
        })
    }

    /// The `project_into` arm: `input` f32 `[row_count][input_dim]`, `output`
    /// f32 `[row_count][output_dim]` (host slices, as the reference's), with the
    /// reference's checks in its order (InvalidRowCount, LengthMismatch
    /// "input", LengthMismatch "output").  A NaN or infinity in `input` is
    /// NonFiniteInput { argument: "input", index, value }.  Synchronous.
    /// Shapes outside the device envelope, and a device call that reports
    /// Unsupported, take the host twin: the call never fails for a shape the
    /// reference accepts (gemm.rs:290-310).
    pub fn project_into(&self, input: &[f32], row_count: usize, output: &mut [f32]) -> Result<(), HipError> {
        let (k, n) = (self.inner.input_dim, self.inner.output_dim);
        if row_count == 0 {
            return Err(HipError::InvalidRowCount(row_count));
        }
        if input.len() != row_count * k {
            return Err(HipError::LengthMismatch { argument: "input", expected: row_count * k, actual: input.len() });
        }
        if output.len() != row_count * n {
            return Err(HipError::LengthMismatch {
                argument: "output",
                expected: row_count * n,
                actual: output.len(),
            });
        }
        if !self.device_supports(row_count) {
            return self.project_host(input, row_count, output);
        }
        let ctx = &self.inner.ctx;
        let x = DeviceBuffer::from_host(ctx, input)?;
        let mut y = DeviceBuffer::<f32>::new(ctx, output.len())?;
        let mut word = DeviceBuffer::<u64>::zeroed(ctx, 1)?;
        let mut guard = self.inner.workspace.lock().unwrap_or_else(|p| p.into_inner());
        let need = unsafe { sys::nh_linear_w8a8_workspace_size(row_count, k) };
        if guard.as_ref().map_or(true, |w| w.bytes() < need) {
            *guard = Some(DeviceBuffer::<u8>::new(ctx, need)?);
        }
        let ws = guard.as_mut().expect("workspace allocated above");
        match self.project_device(
            x.as_ptr().cast(),
            sys::nh_dtype::F32,
            row_count,
            y.as_mut_ptr().cast(),
            sys::nh_dtype::F32,
            ws.as_mut_ptr().cast(),
            ws.bytes(),
            word.as_mut_ptr(),
            None,
        ) {
            Err(HipError::Unsupported(_)) => {
                drop(guard);
                return self.project_host(input, row_count, output);
            }
            r => r?,
        }
        call(|e| unsafe { sys::nh_take_nonfinite(ctx.as_raw(), word.as_mut_ptr(), core::ptr::null_mut(), e) })?;
        y.copy_to_host(output)
    }

    /// The device-resident form: enqueues the quantized projection of the
    /// device rows `x` (f32 or bf16) into `out` on `stream` and returns;
    /// `workspace` holds `nh_linear_w8a8_workspace_size(row_count,
    /// input_dim)` bytes; `nonfinite` (optional) is the layer's non-finite
    /// word (read it with `nh_take_nonfinite`).
    #[allow(clippy::too_many_arguments)]
    pub fn project_device(
        &self,
        x: *const c_void,
        x_dtype: sys::nh_dtype,
        row_count: usize,
        out: *mut c_void,
        out_dtype: sys::nh_dtype,
        workspace: *mut c_void,
        workspace_bytes: usize,
        nonfinite: *mut u64,
        stream: Option<&Stream>,
    ) -> Result<(), HipError> {
        call(|e| unsafe {
            sys::nh_linear_w8a8(
                self.inner.ctx.as_raw(),
                x,
                x_dtype,
                self.codes_ptr(),
                self.scales_ptr(),
                self.bias_ptr(),
                row_count,
                self.inner.output_dim,
                self.inner.input_dim,
                out,
                out_dtype,
                workspace,
                workspace_bytes,
                core::ptr::null_mut(),
                core::ptr::null_mut(),
                nonfinite,
                Stream::raw_or_null(stream),
                e,
            )
        })
    }
}

fn check_dims(input_dim: usize, output_dim: usize, bias: Option<&[f32]>) -> Result<(), HipError> {
    if input_dim == 0 || output_dim == 0 {
        return Err(HipError::InvalidShape(format!("input_dim={input_dim}, output_dim={output_dim}")));
    }
    if let Some(b) = bias {
        if b.len() != output_dim {
            return Err(HipError::LengthMismatch { argument: "bias", expected: output_dim, actual: b.len() });
        }
    }
    Ok(())
}

impl PartialEq for Int8PerRowWeights {
    fn eq(&self, other: &Self) -> bool {
        Arc::ptr_eq(&self.inner, &other.inner)
    }
}

impl fmt::Debug for Int8PerRowWeights {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        f.debug_struct("Int8PerRowWeights")
            .field("input_dim", &self.inner.input_dim)
            .field("output_dim", &self.inner.output_dim)
            .field("bias", &self.inner.bias.is_some())
            .finish()
    }
}
