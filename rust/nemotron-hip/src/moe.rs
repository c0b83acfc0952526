//! `MoeLayer::forward_into` (moe.rs:154-249) with int8 per-row experts: the
//! dense f32 router on the device (bit-identical to router.project), sigmoid
//! top-k routing, the routed experts as two grouped GEMMs over an
//! expert-sorted permutation built on the device, the optional shared expert,
//! and the weighted combine in the reference's order; one library call.
use std::sync::{Arc, Mutex};

use nemotron_hip_sys as sys;

use crate::device::{Context, DeviceBuffer};
use crate::error::{call, HipError};
use crate::mlp::Int8Mlp;

/// Routing options.  `REFERENCE` is MoeLayer's moe_route_host: sigmoid
/// weights of the top-k experts as they are.
#[derive(Clone, Copy, Debug, PartialEq)]
pub struct MoeRouting {
    /// Divide the selected weights by their sum (route order).
    pub renormalize: bool,
    /// Multiply the (renormalized) weights by this factor.
    pub scaling: f32,
}

impl MoeRouting {
    pub const REFERENCE: Self = Self { renormalize: false, scaling: 1.0 };
}

pub struct Int8Moe {
    ctx: Arc<Context>,
    hidden: usize,
    inter: usize,
    experts: usize,
    top_k: usize,
    routing: MoeRouting,
    router_w: DeviceBuffer<f32>, // [hidden][experts]
    router_b: Option<DeviceBuffer<f32>>,
    w_up: DeviceBuffer<i8>, // experts x tiled [inter][hidden]
    s_up: DeviceBuffer<f32>,
    w_down: DeviceBuffer<i8>, // experts x tiled [hidden][inter]
    s_down: DeviceBuffer<f32>,
    shared: Option<Int8Mlp>,
    workspace: Mutex<Option<DeviceBuffer<u8>>>,
}

/// One expert's dense f32 weights as the reference's MlpLayer stores them:
/// `up` `[hidden][inter]`, `down` `[inter][hidden]` (row-major `[in][out]`).
pub struct DenseExpert<'a> {
    pub up: &'a [f32],
    pub down: &'a [f32],
}

fn quantize_tiled(in_dim: usize, out_dim: usize, w: &[f32], argument: &'static str) -> Result<(Vec<i8>, Vec<f32>), HipError> {
    if w.len() != in_dim * out_dim {
        return Err(HipError::LengthMismatch { argument, expected: in_dim * out_dim, actual: w.len() });
    }
    let mut rows = vec![0.0f32; w.len()];
    for k in 0..in_dim {
        for n in 0..out_dim {
            rows[n * in_dim + k] = w[k * out_dim + n];
        }
    }
    let mut codes = vec![0i8; w.len()];
    let mut scales = vec![0.0f32; out_dim];
    call(|e| unsafe {
        sys::nh_quantize_rows_i8_host(
            rows.as_ptr().cast(),
            sys::nh_dtype::F32,
            out_dim,
            in_dim,
            codes.as_mut_ptr(),
            scales.as_mut_ptr(),
            e,
        )
    })?;
    let tiled_len = unsafe { sys::nh_tiled_weights_bytes(out_dim, in_dim) };
    let mut tiled = vec![0i8; tiled_len];
    call(|e| unsafe { sys::nh_tile_weights_i8_host(codes.as_ptr(), out_dim, in_dim, tiled.as_mut_ptr(), tiled_len, e) })?;
    Ok((tiled, scales))
}

impl Int8Moe {
    /// Quantizes the experts (one scale per output row, per expert) and
    /// uploads them with the dense router (`router_w` `[hidden][experts]`,
    /// `router_b` `[experts]`).  Shape checks follow MoeLayer::new
    /// (moe.rs:69-106): InvalidShape for a zero dimension or top_k outside
    /// 1..=experts, LengthMismatch for a router or expert of the wrong size.
    #[allow(clippy::too_many_arguments)]
    pub fn quantize_dense(
        ctx: &Arc<Context>,
        hidden: usize,
        inter: usize,
        top_k: usize,
        routing: MoeRouting,
        router_w: &[f32],
        router_b: Option<&[f32]>,
        experts: &[DenseExpert<'_>],
        shared: Option<Int8Mlp>,
    ) -> Result<Self, HipError> {
        let e = experts.len();
        if hidden == 0 || inter == 0 || e == 0 || top_k == 0 || top_k > e {
            return Err(HipError::InvalidShape(format!(
                "hidden_dim={hidden}, intermediate_dim={inter}, expert_count={e}, top_k={top_k}"
            )));
        }
        if router_w.len() != hidden * e {
            return Err(HipError::LengthMismatch { argument: "router", expected: hidden * e, actual: router_w.len() });
        }
        if let Some(b) = router_b {
            if b.len() != e {
                return Err(HipError::LengthMismatch { argument: "router_bias", expected: e, actual: b.len() });
            }
        }
        if let Some(s) = shared.as_ref() {
            if s.hidden_dim() != hidden || !Arc::ptr_eq(s.up().context(), ctx) {
                return Err(HipError::InvalidShape("shared expert does not match the layer".into()));
            }
        }
        let (mut up, mut su, mut down, mut sd) = (Vec::new(), Vec::new(), Vec::new(), Vec::new());
        for ex in experts {
            let (t, s) = quantize_tiled(hidden, inter, ex.up, "expert_up")?;
            up.extend_from_slice(&t);
            su.extend_from_slice(&s);
            let (t, s) = quantize_tiled(inter, hidden, ex.down, "expert_down")?;
            down.extend_from_slice(&t);
            sd.extend_from_slice(&s);
        }
        Ok(Self {
            ctx: ctx.clone(),
            hidden,
            inter,
            experts: e,
            top_k,
            routing,
            router_w: DeviceBuffer::from_host(ctx, router_w)?,
            router_b: match router_b {
                Some(b) => Some(DeviceBuffer::from_host(ctx, b)?),
                None => None,
            },
            w_up: DeviceBuffer::from_host(ctx, &up)?,
            s_up: DeviceBuffer::from_host(ctx, &su)?,
            w_down: DeviceBuffer::from_host(ctx, &down)?,
            s_down: DeviceBuffer::from_host(ctx, &sd)?,
            shared,
            workspace: Mutex::new(None),
        })
    }

    /// `input`, `output` f32 `[row_count][hidden]`, the reference's checks in
    /// its order.  NonFiniteInput names "input" or "intermediate" (the
    /// `[routes][intermediate]` up output in expert-sorted slot order, or the
    /// shared expert's).  Synchronous.
    pub fn forward_into(&self, input: &[f32], row_count: usize, output: &mut [f32]) -> Result<(), HipError> {
        let h = self.hidden;
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
        let ctx = &self.ctx;
        let x = DeviceBuffer::from_host(ctx, input)?;
        let mut y = DeviceBuffer::<f32>::new(ctx, output.len())?;
        let mut word = DeviceBuffer::<u64>::zeroed(ctx, 1)?;
        let sh_inter = self.shared.as_ref().map_or(0, |s| s.intermediate_dim());
        let need = unsafe {
            sys::nh_moe_layer_w8a8_workspace_size(row_count, h, self.inter, self.experts, self.top_k, sh_inter)
        };
        let mut guard = self.workspace.lock().unwrap_or_else(|p| p.into_inner());
        if guard.as_ref().map_or(true, |w| w.bytes() < need) {
            *guard = Some(DeviceBuffer::<u8>::new(ctx, need)?);
        }
        let ws = guard.as_mut().expect("workspace allocated above");
        let null_i8 = core::ptr::null::<i8>();
        let null_f32 = core::ptr::null::<f32>();
        let (su_w, su_s, sd_w, sd_s) = match self.shared.as_ref() {
            Some(s) => (s.up().codes_ptr(), s.up().scales_ptr(), s.down().codes_ptr(), s.down().scales_ptr()),
            None => (null_i8, null_f32, null_i8, null_f32),
        };
        call(|e| unsafe {
            sys::nh_moe_layer_w8a8(
                ctx.as_raw(),
                x.as_ptr().cast(),
                sys::nh_dtype::F32,
                self.router_w.as_ptr(),
                self.router_b.as_ref().map_or(null_f32, |b| b.as_ptr()),
                row_count,
                h,
                self.inter,
                self.experts,
                self.top_k,
                self.routing.renormalize as core::ffi::c_int,
                self.routing.scaling,
                self.w_up.as_ptr(),
                self.s_up.as_ptr(),
                self.w_down.as_ptr(),
                self.s_down.as_ptr(),
                sh_inter,
                su_w,
                su_s,
                sd_w,
                sd_s,
                y.as_mut_ptr().cast(),
                sys::nh_dtype::F32,
                ws.as_mut_ptr().cast(),
                ws.bytes(),
                word.as_mut_ptr(),
                core::ptr::null_mut(),
                e,
            )
        })?;
        call(|e| unsafe { sys::nh_take_nonfinite(ctx.as_raw(), word.as_mut_ptr(), core::ptr::null_mut(), e) })?;
        y.copy_to_host(output)
    }
}
