//! `MoeLayer::forward_into` (moe.rs:154-249) with int8 per-row experts: the
//! dense f32 router on the device (bit-identical to router.project), sigmoid
//! top-k routing, the routed experts as two grouped GEMMs over an
//! expert-sorted permutation built on the device, the optional shared expert,
//! and the weighted combine in the reference's order; one library call.
//! Expert and shared-expert biases are the MlpLayer biases of the reference
//! (mlp.rs:79-96, 201-208).  Outside the device envelope the library's host
//! twin computes the same result (the host-fallback contract, gemm.rs:290-310).
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
    b_up: Option<DeviceBuffer<f32>>,   // [experts][inter] when any expert has an up bias
    b_down: Option<DeviceBuffer<f32>>, // [experts][hidden] when any expert has a down bias
    shared: Option<Int8Mlp>,
    shared_b_up: Option<DeviceBuffer<f32>>,
    shared_b_down: Option<DeviceBuffer<f32>>,
    workspace: Mutex<Option<DeviceBuffer<u8>>>,
}

/// One expert's dense f32 weights as the reference's MlpLayer stores them:
/// `up` `[hidden][inter]`, `down` `[inter][hidden]` (row-major `[in][out]`),
/// and its optional projection biases (`[inter]`, `[hidden]`).
pub struct DenseExpert<'a> {
    pub up: &'a [f32],
    pub down: &'a [f32],
    pub up_bias: Option<&'a [f32]>,
    pub down_bias: Option<&'a [f32]>,
}

/// The experts' biases gathered expert-major, zeros for an expert without
/// one (adding +0.0 leaves every value but -0.0 unchanged, and the combine
/// starts from +0.0, so the layer's output is the same); None when no expert
/// has one.
fn gather_biases(
    experts: &[DenseExpert<'_>],
    width: usize,
    pick: impl Fn(&DenseExpert<'_>) -> Option<&[f32]>,
    argument: &'static str,
) -> Result<Option<Vec<f32>>, HipError> {
    if experts.iter().all(|e| pick(e).is_none()) {
        return Ok(None);
    }
    let mut all = vec![0.0f32; experts.len() * width];
    for (i, e) in experts.iter().enumerate() {
        if let Some(b) = pick(e) {
            if b.len() != width {
                return Err(HipError::LengthMismatch { argument, expected: width, actual: b.len() });
            }
            all[i * width..(i + 1) * width].copy_from_slice(b);
        }
    }
    Ok(Some(all))
}

fn download(b: &DeviceBuffer<f32>) -> Result<Vec<f32>, HipError> {
    let mut v = vec![0.0f32; b.len()];
    b.copy_to_host(&mut v)?;
    Ok(v)
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
        let b_up = gather_biases(experts, inter, |e| e.up_bias, "expert_up_bias")?;
        let b_down = gather_biases(experts, hidden, |e| e.down_bias, "expert_down_bias")?;
        let upload = |v: Option<Vec<f32>>| -> Result<Option<DeviceBuffer<f32>>, HipError> {
            v.map(|v| DeviceBuffer::from_host(ctx, &v)).transpose()
        };
        // the shared expert's biases, as nh_moe_layer_w8a8 takes them
        let (shared_b_up, shared_b_down) = match shared.as_ref() {
            Some(s) => (
                if s.up().has_bias() { Some(s.up().with_host(|w| Ok(w.bias.clone().unwrap_or_default()))?) } else { None },
                if s.down().has_bias() { Some(s.down().with_host(|w| Ok(w.bias.clone().unwrap_or_default()))?) } else { None },
            ),
            None => (None, None),
        };
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
            b_up: upload(b_up)?,
            b_down: upload(b_down)?,
            shared,
            shared_b_up: upload(shared_b_up)?,
            shared_b_down: upload(shared_b_down)?,
            workspace: Mutex::new(None),
        })
    }

    fn biases(&self) -> sys::nh_moe_biases {
        let p = |b: &Option<DeviceBuffer<f32>>| b.as_ref().map_or(core::ptr::null(), |b| b.as_ptr());
        sys::nh_moe_biases {
            up: p(&self.b_up),
            down: p(&self.b_down),
            shared_up: p(&self.shared_b_up),
            shared_down: p(&self.shared_b_down),
        }
    }

    /// Whether the device entry point runs `row_count` rows of this layer.
    pub fn device_supports(&self, row_count: usize) -> bool {
        let sh_inter = self.shared.as_ref().map_or(0, |s| s.intermediate_dim());
        unsafe {
            sys::nh_supports_moe_layer_w8a8(row_count, self.hidden, self.inter, self.experts, self.top_k, sh_inter) != 0
        }
    }

    /// The host twin (`nh_moe_layer_w8a8_host`): every operand copied to the
    /// host (the bridge of gemm.rs:301-310), the same result bit for bit.
    fn forward_host(&self, input: &[f32], row_count: usize, output: &mut [f32]) -> Result<(), HipError> {
        let router_w = download(&self.router_w)?;
        let router_b = self.router_b.as_ref().map(download).transpose()?;
        let mut w_up = vec![0i8; self.w_up.len()];
        self.w_up.copy_to_host(&mut w_up)?;
        let mut w_down = vec![0i8; self.w_down.len()];
        self.w_down.copy_to_host(&mut w_down)?;
        let (s_up, s_down) = (download(&self.s_up)?, download(&self.s_down)?);
        let b: Vec<Option<Vec<f32>>> = [&self.b_up, &self.b_down, &self.shared_b_up, &self.shared_b_down]
            .iter()
            .map(|b| b.as_ref().map(download).transpose())
            .collect::<Result<_, _>>()?;
        let p = |v: &Option<Vec<f32>>| v.as_ref().map_or(core::ptr::null(), |v| v.as_ptr());
        let hb = sys::nh_moe_biases { up: p(&b[0]), down: p(&b[1]), shared_up: p(&b[2]), shared_down: p(&b[3]) };
        let sh_inter = self.shared.as_ref().map_or(0, |s| s.intermediate_dim());
        let out_ptr = output.as_mut_ptr();
        let run = |su_w: *const i8, su_s: *const f32, sd_w: *const i8, sd_s: *const f32| {
            call(|e| unsafe {
                sys::nh_moe_layer_w8a8_host(
                    input.as_ptr().cast(),
                    sys::nh_dtype::F32,
                    router_w.as_ptr(),
                    p(&router_b),
                    row_count,
                    self.hidden,
                    self.inter,
                    self.experts,
                    self.top_k,
                    self.routing.renormalize as core::ffi::c_int,
                    self.routing.scaling,
                    w_up.as_ptr(),
                    s_up.as_ptr(),
                    w_down.as_ptr(),
                    s_down.as_ptr(),
                    sh_inter,
                    su_w,
                    su_s,
                    sd_w,
                    sd_s,
                    &hb,
                    out_ptr.cast(),
                    sys::nh_dtype::F32,
                    e,
                )
            })
        };
        match self.shared.as_ref() {
            Some(s) => s.up().with_host(|u| {
                s.down().with_host(|d| run(u.codes.as_ptr(), u.scales.as_ptr(), d.codes.as_ptr(), d.scales.as_ptr()))
            }),
            None => run(core::ptr::null(), core::ptr::null(), core::ptr::null(), core::ptr::null()),
        }
    }

    /// `input`, `output` f32 `[row_count][hidden]`, the reference's checks in
    /// its order.  NonFiniteInput names "input", "shared_intermediate" (the
    /// shared expert's `[row_count][shared_inter]` ReLU^2 output, met first as
    /// in moe.rs:197-219) or "intermediate" (the `[routes][intermediate]` up
    /// output in expert-sorted slot order).  Synchronous; outside the device
    /// envelope (or on an Unsupported device call) the host twin runs.
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
        if !self.device_supports(row_count) {
            return self.forward_host(input, row_count, output);
        }
        let ctx = &self.ctx;
        let x = DeviceBuffer::from_host(ctx, input)?;
        let mut y = DeviceBuffer::<f32>::new(ctx, output.len())?;
        let mut word = DeviceBuffer::<u64>::zeroed(ctx, 1)?;
        let biases = self.biases();
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
        let r = call(|e| unsafe {
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
                &biases,
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
