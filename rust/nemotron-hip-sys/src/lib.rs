//! Raw bindings to `libnemotron_hip`, the MI355X (gfx950) int8 quantized-linear
//! path: one declaration per function of `include/nemotron_hip.h`, in its order,
//! with the same names, argument order and C types.  `nemotron-hip` is the safe
//! layer over it.
//!
//! Conventions of the C ABI (restated from the header):
//! - Device entry points take caller-owned device pointers and an explicit stream;
//!   they only enqueue work and validate every argument on the host before anything
//!   is launched.  `*_host` entry points run the library's CPU implementation.
//! - Lengths are element counts.  Every call returns an [`nh_status`]; the optional
//!   [`nh_error`] (may be null) carries the payload of the reference's error enums.
//! - int8 weights are tiled: a logical `[N][K]` code matrix is stored as
//!   `ceil(N/16) x ceil(K/64)` tiles of 1024 bytes, tile `(nt, kt)` at byte
//!   `(nt*KT + kt)*1024`, whose byte `16*(16*g + r) + b` holds
//!   `W[16*nt + r][64*kt + 16*g + b]` (zero outside the matrix).
//! - No function aborts the process.
#![allow(non_camel_case_types)]
#![no_std]

use core::ffi::{c_char, c_int, c_void};
use core::marker::{PhantomData, PhantomPinned};

/// Status of every call (the variants of QuantizeError, GemmError, MoeRoutingError,
/// LinearError and WeightError).  A transparent `int`: a value the library never
/// returns cannot make a Rust `match` undefined.
#[repr(transparent)]
#[derive(Clone, Copy, Debug, PartialEq, Eq, Hash)]
pub struct nh_status(pub c_int);

impl nh_status {
    pub const OK: Self = Self(0);
    /// `*Error::InvalidShape`
    pub const INVALID_SHAPE: Self = Self(1);
    /// `*Error::LengthMismatch { argument, expected, actual }`
    pub const LENGTH_MISMATCH: Self = Self(2);
    /// `QuantizeError::InvalidParams`
    pub const INVALID_PARAMS: Self = Self(3);
    /// `QuantizeError::NonFiniteInput { index, value }`
    pub const NON_FINITE_INPUT: Self = Self(4);
    /// `QuantizeError::Int4OutOfRange(u8)`
    pub const OUT_OF_RANGE: Self = Self(5);
    /// `LinearError::InvalidRowCount`
    pub const INVALID_ROW_COUNT: Self = Self(6);
    /// Shape outside the device envelope: the caller takes the `*_host` twin.
    pub const UNSUPPORTED: Self = Self(7);
    /// `*Error::DeviceError(String)`
    pub const DEVICE_ERROR: Self = Self(8);
    /// `WeightError::Io`
    pub const IO_ERROR: Self = Self(9);
    /// `WeightError::InvalidHeaderLength / InvalidHeaderJson / InvalidTensorHeader`
    pub const INVALID_HEADER: Self = Self(10);
    /// `WeightError::TensorNotFound`
    pub const TENSOR_NOT_FOUND: Self = Self(11);

    pub const fn is_ok(self) -> bool {
        self.0 == 0
    }
}

/// Element type of activations and outputs.
#[repr(transparent)]
#[derive(Clone, Copy, Debug, PartialEq, Eq, Hash)]
pub struct nh_dtype(pub c_int);

impl nh_dtype {
    pub const F32: Self = Self(0);
    pub const BF16: Self = Self(1);
}

/// Payload of a failed call.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct nh_error {
    /// Static NUL-terminated string naming the offending argument (or null).
    pub argument: *const c_char,
    pub expected: u64,
    pub actual: u64,
    /// `NonFiniteInput.index` (flat, row-major).
    pub index: u64,
    /// `NonFiniteInput.value`.
    pub value: f32,
    /// `Int4OutOfRange` payload.
    pub byte: u32,
    /// NUL-terminated human-readable detail (the `DeviceError` text).
    pub message: [c_char; 256],
}

impl Default for nh_error {
    fn default() -> Self {
        Self {
            argument: core::ptr::null(),
            expected: 0,
            actual: 0,
            index: 0,
            value: 0.0,
            byte: 0,
            message: [0; 256],
        }
    }
}

/// One tensor entry of a safetensors header.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct nh_tensor_info {
    /// The header's dtype string ("I8", "F32", "BF16", ...), NUL-terminated.
    pub dtype: [c_char; 16],
    pub ndim: u32,
    pub shape: [u64; 8],
    /// Absolute byte offset of the tensor's data in the file.
    pub data_begin: u64,
    /// `data_offsets` end - start.
    pub data_bytes: u64,
}

impl Default for nh_tensor_info {
    fn default() -> Self {
        Self { dtype: [0; 16], ndim: 0, shape: [0; 8], data_begin: 0, data_bytes: 0 }
    }
}

/// Optional biases of the int8 MoE layer's experts (each pointer may be null; a null
/// `*const nh_moe_biases` means none): the reference's routed experts and shared expert are
/// MlpLayers whose projections may carry biases (mlp.rs:79-96, moe.rs:60-65); an up bias is added
/// before ReLU^2, a down bias to the expert's own output, before the combine weight
/// (mlp.rs:201-208).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct nh_moe_biases {
    /// [experts][inter], expert-major like s_up.
    pub up: *const f32,
    /// [experts][hidden], like s_down.
    pub down: *const f32,
    /// [shared_inter].
    pub shared_up: *const f32,
    /// [hidden].
    pub shared_down: *const f32,
}

impl Default for nh_moe_biases {
    fn default() -> Self {
        Self {
            up: core::ptr::null(),
            down: core::ptr::null(),
            shared_up: core::ptr::null(),
            shared_down: core::ptr::null(),
        }
    }
}

/// Opaque device context (immutable once created; safe to share across threads).
#[repr(C)]
pub struct nh_context {
    _private: [u8; 0],
    _marker: PhantomData<(*mut u8, PhantomPinned)>,
}

/// `hipStream_t`; null is the device's null stream.
pub type nh_stream = *mut c_void;

// The C layouts (x86_64 / aarch64 LP64), checked at compile time.
const _: () = {
    use core::mem::{align_of, offset_of, size_of};
    assert!(size_of::<nh_status>() == 4 && size_of::<nh_dtype>() == 4);
    assert!(size_of::<nh_error>() == 296 && align_of::<nh_error>() == 8);
    assert!(offset_of!(nh_error, argument) == 0);
    assert!(offset_of!(nh_error, expected) == 8);
    assert!(offset_of!(nh_error, actual) == 16);
    assert!(offset_of!(nh_error, index) == 24);
    assert!(offset_of!(nh_error, value) == 32);
    assert!(offset_of!(nh_error, byte) == 36);
    assert!(offset_of!(nh_error, message) == 40);
    assert!(size_of::<nh_tensor_info>() == 104);
    assert!(offset_of!(nh_tensor_info, dtype) == 0);
    assert!(offset_of!(nh_tensor_info, ndim) == 16);
    assert!(offset_of!(nh_tensor_info, shape) == 24);
    assert!(offset_of!(nh_tensor_info, data_begin) == 88);
    assert!(offset_of!(nh_tensor_info, data_bytes) == 96);
    assert!(size_of::<nh_moe_biases>() == 32);
    assert!(offset_of!(nh_moe_biases, up) == 0);
    assert!(offset_of!(nh_moe_biases, down) == 8);
    assert!(offset_of!(nh_moe_biases, shared_up) == 16);
    assert!(offset_of!(nh_moe_biases, shared_down) == 24);
};

extern "C" {
    /// D0: device, context, buffers (GpuDevice / GpuTensor, device.rs:117-153, tensor.rs:259-446)
    pub fn nh_device_count() -> c_int;

    /// Loads the gfx950 code object (embedded in the library when path is NULL) with hipModuleLoadData
    /// and resolves every kernel once; the context is immutable afterwards and safe to share across
    /// threads (device.rs:33-42).
    pub fn nh_context_create(
        device: c_int,
        code_object_path: *const c_char,
        out: *mut *mut nh_context,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_context_destroy(ctx: *mut nh_context);

    pub fn nh_context_device(ctx: *const nh_context) -> c_int;

    pub fn nh_malloc(
        ctx: *mut nh_context,
        bytes: usize,
        ptr: *mut *mut c_void,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_free(ctx: *mut nh_context, ptr: *mut c_void, err: *mut nh_error) -> nh_status;

    pub fn nh_memcpy_htod(
        ctx: *mut nh_context,
        dst: *mut c_void,
        src: *const c_void,
        bytes: usize,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_memcpy_dtoh(
        ctx: *mut nh_context,
        dst: *mut c_void,
        src: *const c_void,
        bytes: usize,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_memset_d8(
        ctx: *mut nh_context,
        dst: *mut c_void,
        value: c_int,
        bytes: usize,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_stream_create(
        ctx: *mut nh_context,
        out: *mut nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_stream_destroy(
        ctx: *mut nh_context,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_stream_synchronize(
        ctx: *mut nh_context,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    /// Kernel registry (supported_*_kernels(), gemm.rs:80-82, quantize.rs:45-47, moe_routing.rs:71-73)
    pub fn nh_kernel_count() -> c_int;

    /// name of kernel i and its backend tag: 0 = host fallback, 1 = gfx950 device
    pub fn nh_kernel_name(i: c_int, backend: *mut c_int) -> *const c_char;

    /// Q0: affine INT4 (quantize.rs:49-204)
    ///
    /// Restates quantize.rs:49-51.
    pub fn nh_packed_int4_len(value_count: usize) -> usize;

    /// Restates quantize.rs:59-81.
    pub fn nh_pack_int4_host(
        values: *const u8,
        n: usize,
        packed: *mut u8,
        packed_len: usize,
        err: *mut nh_error,
    ) -> nh_status;

    /// Restates quantize.rs:89-120.
    pub fn nh_unpack_int4_host(
        packed: *const u8,
        packed_len: usize,
        value_count: usize,
        out: *mut u8,
        out_len: usize,
        err: *mut nh_error,
    ) -> nh_status;

    /// Restates quantize.rs:131-144.
    pub fn nh_quantize_int4_host(
        values: *const f32,
        n: usize,
        scale: f32,
        zero_point: u32,
        packed: *mut u8,
        packed_len: usize,
        err: *mut nh_error,
    ) -> nh_status;

    /// Restates quantize.rs:156-178.
    pub fn nh_dequantize_int4_host(
        packed: *const u8,
        packed_len: usize,
        value_count: usize,
        scale: f32,
        zero_point: u32,
        out: *mut f32,
        out_len: usize,
        err: *mut nh_error,
    ) -> nh_status;

    /// Q0d, replaces dequantize_int4 (quantize.rs:332-349): unpack + dequantize on the device from the
    /// packed bytes (any value_count, not only powers of two as :207-209).
    pub fn nh_dequantize_int4(
        ctx: *mut nh_context,
        packed: *const u8,
        packed_len: usize,
        value_count: usize,
        scale: f32,
        zero_point: u32,
        out: *mut f32,
        out_len: usize,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    /// Q1/Q2/Q3: symmetric int8, one f32 scale per row (new; numerics of quantize_scalar
    /// quantize.rs:188-200 with zero point 0)
    ///
    /// s[r] = max|x[r,:]| / 127 (RN); q = clamp(roundf(x / s), -127, 127); s == 0 -> codes 0.  Used for
    /// weights (Q1, offline) and per-token activations (Q2).  row_status (optional, [rows]) receives -1
    /// or the first non-finite column of the row; codes of such a row are unspecified.
    pub fn nh_quantize_rows_i8(
        ctx: *mut nh_context,
        x: *const c_void,
        dtype: nh_dtype,
        rows: usize,
        cols: usize,
        q: *mut i8,
        scales: *mut f32,
        row_status: *mut i32,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_quantize_rows_i8_host(
        x: *const c_void,
        dtype: nh_dtype,
        rows: usize,
        cols: usize,
        q: *mut i8,
        scales: *mut f32,
        err: *mut nh_error,
    ) -> nh_status;

    /// NonFiniteInput on the first bad element
    ///
    /// Q3: out = (float)q * s (dequantize_scalar, quantize.rs:202-204).
    pub fn nh_dequantize_i8(
        ctx: *mut nh_context,
        q: *const i8,
        scales: *const f32,
        rows: usize,
        cols: usize,
        out: *mut f32,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_dequantize_i8_host(
        q: *const i8,
        scales: *const f32,
        rows: usize,
        cols: usize,
        out: *mut f32,
        err: *mut nh_error,
    ) -> nh_status;

    /// Tiled int8 weight layout (see Conventions): bytes of the tiled form of an [n][k] matrix (0 for
    /// an invalid shape), and the conversion from row-major codes.  New: the reference has no int8
    /// weight format.
    pub fn nh_tiled_weights_bytes(n: usize, k: usize) -> usize;

    pub fn nh_tile_weights_i8(
        ctx: *mut nh_context,
        wq: *const i8,
        n: usize,
        k: usize,
        tiled: *mut i8,
        tiled_len: usize,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_tile_weights_i8_host(
        wq: *const i8,
        n: usize,
        k: usize,
        tiled: *mut i8,
        tiled_len: usize,
        err: *mut nh_error,
    ) -> nh_status;

    /// G0/G1/G2/G3: GEMM family (gemm.rs, linear.rs:283-342)
    ///
    /// G0: gemm_into_host restated (gemm.rs:91-147): f32 in, f64 accumulation.
    pub fn nh_gemm_f32_host(
        lhs: *const f32,
        lhs_len: usize,
        rhs: *const f32,
        rhs_len: usize,
        m: usize,
        k: usize,
        n: usize,
        out: *mut f32,
        out_len: usize,
        err: *mut nh_error,
    ) -> nh_status;

    /// G0d: the device GEMM of gemm / gemm_into (gemm.rs:318-363), f32 [m][k] x f32 [k][n] -> f32
    /// [m][n], accumulated in f64 with k ascending for every output: bit-identical to nh_gemm_f32_host.
    /// Same validation and error payloads as gemm_into; any alignment of m, k, n (the reference's
    /// cutile kernel needed tile multiples, gemm.rs:247-254, and bridged through the host otherwise).
    /// nh_supports_gemm_f32 is its envelope.
    pub fn nh_supports_gemm_f32(m: usize, k: usize, n: usize) -> c_int;

    pub fn nh_gemm_f32(
        ctx: *mut nh_context,
        lhs: *const f32,
        lhs_len: usize,
        rhs: *const f32,
        rhs_len: usize,
        m: usize,
        k: usize,
        n: usize,
        out: *mut f32,
        out_len: usize,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    /// Device envelope of the W8A8 GEMM family (supports_shape, gemm.rs:247-254).
    pub fn nh_supports_gemm_w8a8(m: usize, n: usize, k: usize) -> c_int;

    /// G1/G3: out[m,n] = ((float)sum_k xq[m,k]*wq[n,k] * sx[m]) * sw[n] (+ bias[n]) in f32 or bf16
    /// (RNE); wq tiled.  int32 accumulation is exact.  M <= 16 runs the HBM-bound GEMV, larger M the
    /// MFMA GEMM.
    pub fn nh_gemm_w8a8(
        ctx: *mut nh_context,
        xq: *const i8,
        sx: *const f32,
        wq: *const i8,
        sw: *const f32,
        bias: *const f32,
        m: usize,
        n: usize,
        k: usize,
        out: *mut c_void,
        out_dtype: nh_dtype,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    /// G3 with A also tiled: xq_tiled is nh_tile_weights_i8 of the row-major [m][k] codes
    /// (nh_tiled_weights_bytes(m, k) bytes), so every A load is one contiguous KiB as well; same result
    /// as nh_gemm_w8a8 on the row-major codes (the tiled-A GEMM is the faster one: the linear entry
    /// point uses it for m > 16).  No reference counterpart: G3 is new.
    pub fn nh_gemm_w8a8_ta(
        ctx: *mut nh_context,
        xq_tiled: *const i8,
        sx: *const f32,
        wq: *const i8,
        sw: *const f32,
        bias: *const f32,
        m: usize,
        n: usize,
        k: usize,
        out: *mut c_void,
        out_dtype: nh_dtype,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_gemm_w8a8_host(
        xq: *const i8,
        sx: *const f32,
        wq: *const i8,
        sw: *const f32,
        bias: *const f32,
        m: usize,
        n: usize,
        k: usize,
        out: *mut c_void,
        out_dtype: nh_dtype,
        err: *mut nh_error,
    ) -> nh_status;

    /// Non-finite inputs of the quantizing layers (the spec's Q2 error,
    /// QuantizeError::NonFiniteInput{index, value} in the style of quantize.rs:193-195).  Device
    /// launches cannot return it, so the layer entry points below take an optional device word
    /// `nonfinite` (uint64, zero before the first call, e.g. nh_memset_d8): a quantizer that meets a
    /// NaN or an infinity records the first one there (the layer's input ahead of its intermediate,
    /// then the lowest row-major index) and carries on; the codes of such a row, and the outputs that
    /// depend on them, are unspecified. nh_take_nonfinite synchronizes `stream`, returns
    /// NH_NON_FINITE_INPUT with err->argument "input" (index into x) or "intermediate" (index into the
    /// layer's f32 intermediate: the MLP's [m][inter] ReLU^2 output, the MoE's [routes][inter] up
    /// output in expert-sorted slot order), err->index and err->value, and clears the word; NH_OK when
    /// it is zero.  NULL skips the check at no cost.
    pub fn nh_take_nonfinite(
        ctx: *mut nh_context,
        nonfinite: *mut u64,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    /// Quantized linear layer, the drop-in for LinearProjection::project_into with int8 per-row weights
    /// (linear.rs:283-342): dynamic per-token quantization of x (f32 or bf16) then G1/G3 + bias.  For
    /// bf16 x with k <= 8192 and m <= 4 (m <= 8 when k % 512 == 0) the quantization is fused into the
    /// GEMV (one launch; the workspace is not touched); otherwise it runs as its own launch into a
    /// workspace of nh_linear_w8a8_workspace_size(m, k) bytes, 16-byte aligned (for m <= 16 it holds
    /// the codes in the GEMV's operand order).  Pass that workspace on every call.  xq_out/sx_out
    /// (optional) receive the quantized activations (row-major codes, scales).
    pub fn nh_linear_w8a8_workspace_size(m: usize, k: usize) -> usize;

    pub fn nh_linear_w8a8(
        ctx: *mut nh_context,
        x: *const c_void,
        x_dtype: nh_dtype,
        wq: *const i8,
        sw: *const f32,
        bias: *const f32,
        m: usize,
        n: usize,
        k: usize,
        out: *mut c_void,
        out_dtype: nh_dtype,
        workspace: *mut c_void,
        workspace_bytes: usize,
        xq_out: *mut i8,
        sx_out: *mut f32,
        nonfinite: *mut u64,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    /// Device envelope of nh_linear_w8a8 (supports_shape, gemm.rs:247-254): 1 when the device entry
    /// point runs the shape (k % 16 == 0, k <= 131072, every dimension and product below 2^31) with a
    /// 16-byte aligned wq (and workspace); otherwise it returns NH_UNSUPPORTED and the caller takes the
    /// host twin (the host-fallback contract, gemm.rs:290-310).
    pub fn nh_supports_linear_w8a8(m: usize, n: usize, k: usize) -> c_int;

    /// Host twin of nh_linear_w8a8 (LinearProjection::project_into with int8 per-row weights,
    /// linear.rs:283-342): the same arguments in host memory (wq tiled, as on the device), any shape,
    /// bit-identical outputs; no workspace.  A non-finite x returns NH_NON_FINITE_INPUT ("input",
    /// index, value) before any output is written.  xq_out/sx_out optional, as on the device.
    pub fn nh_linear_w8a8_host(
        x: *const c_void,
        x_dtype: nh_dtype,
        wq: *const i8,
        sw: *const f32,
        bias: *const f32,
        m: usize,
        n: usize,
        k: usize,
        out: *mut c_void,
        out_dtype: nh_dtype,
        xq_out: *mut i8,
        sx_out: *mut f32,
        err: *mut nh_error,
    ) -> nh_status;

    /// nh_linear_w8a8 without a workspace argument and without allocating, for callers that cannot call
    /// hipMalloc (code under HIP graph capture, tight serving loops, harnesses that forbid allocation).
    /// No counterpart in the reference.  The workspace is a static device array of 64 MiB (67108864
    /// bytes) per GPU, placed by the HIP runtime and held until the process ends; shapes whose
    /// nh_linear_w8a8_workspace_size(m, k) exceeds it return NH_UNSUPPORTED before anything is launched
    /// (m = 2048 fits k <= 32704, the 21504-wide MLP down projection included). Results are those of
    /// nh_linear_w8a8.  Every call on a GPU shares that GPU's array: calls that overlap on one GPU
    /// (concurrent streams or threads) race and must be serialized by the caller.
    pub fn nh_linear_w8a8_noalloc(
        ctx: *mut nh_context,
        x: *const c_void,
        x_dtype: nh_dtype,
        wq: *const i8,
        sw: *const f32,
        bias: *const f32,
        m: usize,
        n: usize,
        k: usize,
        out: *mut c_void,
        out_dtype: nh_dtype,
        xq_out: *mut i8,
        sx_out: *mut f32,
        nonfinite: *mut u64,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    /// L2: int8 MLP layer, the drop-in for MlpLayer::forward_into with int8 per-row weights
    /// (mlp.rs:157-211): h = ReLU^2(x W_up^T + b_up) in f32 (ReLU^2 after the bias, mlp.rs:205), then
    /// out = h W_down^T + b_down, each projection with per-token quantization of its input
    /// (nh_linear_w8a8). w_up is tiled [inter][hidden], w_down tiled [hidden][inter]; biases may be
    /// NULL.  Errors: INVALID_SHAPE for hidden or inter == 0 (MlpError:: InvalidShape),
    /// INVALID_ROW_COUNT for m == 0, LENGTH_MISMATCH "workspace" for a workspace smaller than
    /// nh_mlp_w8a8_workspace_size(m, hidden, inter) (16-byte aligned; it also holds h).
    pub fn nh_mlp_w8a8_workspace_size(m: usize, hidden: usize, inter: usize) -> usize;

    pub fn nh_mlp_w8a8(
        ctx: *mut nh_context,
        x: *const c_void,
        x_dtype: nh_dtype,
        w_up: *const i8,
        s_up: *const f32,
        b_up: *const f32,
        w_down: *const i8,
        s_down: *const f32,
        b_down: *const f32,
        m: usize,
        hidden: usize,
        inter: usize,
        out: *mut c_void,
        out_dtype: nh_dtype,
        workspace: *mut c_void,
        workspace_bytes: usize,
        nonfinite: *mut u64,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    /// Device envelope of nh_mlp_w8a8: both projections inside nh_supports_linear_w8a8 (16-byte
    /// aligned weights and workspace).
    pub fn nh_supports_mlp_w8a8(m: usize, hidden: usize, inter: usize) -> c_int;

    /// Host twin of nh_mlp_w8a8: same arguments in host memory, bit-identical outputs, no workspace;
    /// NH_NON_FINITE_INPUT "input" or "intermediate" (the f32 [m][inter] ReLU^2 output) as the device
    /// word reports them.
    pub fn nh_mlp_w8a8_host(
        x: *const c_void,
        x_dtype: nh_dtype,
        w_up: *const i8,
        s_up: *const f32,
        b_up: *const f32,
        w_down: *const i8,
        s_down: *const f32,
        b_down: *const f32,
        m: usize,
        hidden: usize,
        inter: usize,
        out: *mut c_void,
        out_dtype: nh_dtype,
        err: *mut nh_error,
    ) -> nh_status;

    /// G2: W8A32 dequant GEMV, y = x * ((float)q * s)^T: the value of materialize_dense +
    /// gemm_into_host (linear.rs:126-131).  The device sums each 16-code group in f32 and the groups in
    /// f64, then scales by s, so |y - exact| <= 16 u sum_k |x q s| + u |y| (u = 2^-24); the _host form
    /// keeps the reference's f64 arithmetic exactly.
    pub fn nh_gemv_w8a32(
        ctx: *mut nh_context,
        x: *const f32,
        wq: *const i8,
        sw: *const f32,
        m: usize,
        n: usize,
        k: usize,
        y: *mut f32,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_gemv_w8a32_host(
        x: *const f32,
        wq: *const i8,
        sw: *const f32,
        m: usize,
        n: usize,
        k: usize,
        y: *mut f32,
        err: *mut nh_error,
    ) -> nh_status;

    /// R1..R4: MoE routing, permutation, grouped GEMM, combine
    pub fn nh_sigmoid_f32_host(x: f32) -> f32;

    /// sigmoid_scalar, activations.rs:73-81
    ///
    /// R1: moe_route_into_host / moe_route (moe_routing.rs:118-141, :499-523): sigmoid scores, top-k by
    /// (weight desc, expert asc).  renormalize divides the selected weights by their sum (route order);
    /// scaling multiplies after. Indices are int32 (usize in the reference).
    pub fn nh_moe_route_sigmoid_topk(
        ctx: *mut nh_context,
        scores: *const f32,
        tokens: usize,
        experts: usize,
        top_k: usize,
        renormalize: c_int,
        scaling: f32,
        indices: *mut i32,
        weights: *mut f32,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_moe_route_sigmoid_topk_host(
        scores: *const f32,
        scores_len: usize,
        tokens: usize,
        experts: usize,
        top_k: usize,
        renormalize: c_int,
        scaling: f32,
        indices: *mut i32,
        indices_len: usize,
        weights: *mut f32,
        weights_len: usize,
        err: *mut nh_error,
    ) -> nh_status;

    /// R1s: moe_route_softmax_into_host (moe_routing.rs:143-166, :188-216).
    pub fn nh_moe_route_softmax_topk_host(
        scores: *const f32,
        scores_len: usize,
        tokens: usize,
        experts: usize,
        top_k: usize,
        indices: *mut i32,
        indices_len: usize,
        weights: *mut f32,
        weights_len: usize,
        err: *mut nh_error,
    ) -> nh_status;

    /// R2: counts -> offsets[E+1] (exclusive scan), perm (slot -> route, stable by route id inside an
    /// expert), pos (route -> slot).
    pub fn nh_moe_permute(
        ctx: *mut nh_context,
        indices: *const i32,
        tokens: usize,
        top_k: usize,
        experts: usize,
        offsets: *mut i32,
        perm: *mut i32,
        pos: *mut i32,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_moe_permute_host(
        indices: *const i32,
        tokens: usize,
        top_k: usize,
        experts: usize,
        offsets: *mut i32,
        perm: *mut i32,
        pos: *mut i32,
        err: *mut nh_error,
    ) -> nh_status;

    /// R3: grouped W8A8 GEMM over the expert segments of offsets (w = E tiled [n][k] matrices at a
    /// stride of nh_tiled_weights_bytes(n, k)).  gather != 0: the A row of slot i is token perm[i] /
    /// top_k (up projection); otherwise the A row is slot i (down projection).  out is f32 [routes][n];
    /// relu2 applies ReLU^2 after the epilogue (mlp.rs:205).
    pub fn nh_moe_grouped_gemm_w8a8(
        ctx: *mut nh_context,
        aq: *const i8,
        sa: *const f32,
        gather: c_int,
        top_k: usize,
        offsets: *const i32,
        perm: *const i32,
        routes: usize,
        a_rows: usize,
        experts: usize,
        w: *const i8,
        sw: *const f32,
        n: usize,
        k: usize,
        relu2: c_int,
        out: *mut f32,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_moe_grouped_gemm_w8a8_host(
        aq: *const i8,
        sa: *const f32,
        gather: c_int,
        top_k: usize,
        offsets: *const i32,
        perm: *const i32,
        routes: usize,
        a_rows: usize,
        experts: usize,
        w: *const i8,
        sw: *const f32,
        n: usize,
        k: usize,
        relu2: c_int,
        out: *mut f32,
        err: *mut nh_error,
    ) -> nh_status;

    /// R4: out[t] = sum_j w[t,j] * slot_out[pos[t*k+j]] in route order (f32), the combine of
    /// MoeLayer::forward_into (moe.rs:195, :221-244).
    pub fn nh_moe_combine(
        ctx: *mut nh_context,
        slot_out: *const f32,
        pos: *const i32,
        weights: *const f32,
        tokens: usize,
        top_k: usize,
        hidden: usize,
        out: *mut c_void,
        out_dtype: nh_dtype,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_moe_combine_host(
        slot_out: *const f32,
        pos: *const i32,
        weights: *const f32,
        tokens: usize,
        top_k: usize,
        hidden: usize,
        out: *mut c_void,
        out_dtype: nh_dtype,
        err: *mut nh_error,
    ) -> nh_status;

    /// R4 with the shared expert (moe.rs:197-219): out[t] = 0 + shared[t] + sum_j w[t,j] *
    /// slot_out[pos[t*k+j]], each add in that order in f32 (the reference zeroes the output, adds the
    /// shared expert's row, then the routes). shared is f32 [tokens][hidden] or NULL (then exactly
    /// nh_moe_combine).
    pub fn nh_moe_combine_shared(
        ctx: *mut nh_context,
        slot_out: *const f32,
        pos: *const i32,
        weights: *const f32,
        shared: *const f32,
        tokens: usize,
        top_k: usize,
        hidden: usize,
        out: *mut c_void,
        out_dtype: nh_dtype,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_moe_combine_shared_host(
        slot_out: *const f32,
        pos: *const i32,
        weights: *const f32,
        shared: *const f32,
        tokens: usize,
        top_k: usize,
        hidden: usize,
        out: *mut c_void,
        out_dtype: nh_dtype,
        err: *mut nh_error,
    ) -> nh_status;

    /// Whole int8 MoE layer on the device: Q2(x) -> R1 -> R2 -> up (R3, gather, ReLU^2) -> Q2 -> down
    /// (R3) -> R4.  Replaces MoeLayer::forward_into (moe.rs:154-249) for routed experts with int8
    /// per-row weights w_up = E tiled [inter][hidden] matrices, w_down = E tiled [hidden][inter]
    /// matrices, each expert at a stride of nh_tiled_weights_bytes of its shape.  The routing stages
    /// leave indices, weights, offsets, perm and pos in the workspace at the byte offsets reported by
    /// nh_moe_workspace_layout.
    pub fn nh_moe_forward_w8a8_workspace_size(
        tokens: usize,
        hidden: usize,
        inter: usize,
        experts: usize,
        top_k: usize,
    ) -> usize;

    /// byte offsets in the workspace of: [0] indices i32[T*k], [1] weights f32[T*k], [2] offsets
    /// i32[E+1], [3] perm i32[T*k], [4] pos i32[T*k].
    pub fn nh_moe_workspace_layout(
        tokens: usize,
        hidden: usize,
        inter: usize,
        experts: usize,
        top_k: usize,
        offsets_out: *mut usize,
    );

    pub fn nh_moe_forward_w8a8(
        ctx: *mut nh_context,
        x: *const c_void,
        x_dtype: nh_dtype,
        logits: *const f32,
        tokens: usize,
        hidden: usize,
        inter: usize,
        experts: usize,
        top_k: usize,
        renormalize: c_int,
        scaling: f32,
        w_up: *const i8,
        s_up: *const f32,
        w_down: *const i8,
        s_down: *const f32,
        biases: *const nh_moe_biases,
        out: *mut c_void,
        out_dtype: nh_dtype,
        workspace: *mut c_void,
        workspace_bytes: usize,
        nonfinite: *mut u64,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    /// The int8 MoE layer with its shared expert, MoeLayer::forward_into with shared_expert = Some(..)
    /// (moe.rs:197-219): the shared expert is an int8 MLP over every token (nh_mlp_w8a8 on x, f32, with
    /// biases->shared_up and ->shared_down: w_up_shared tiled [shared_inter][hidden], w_down_shared
    /// tiled [hidden][shared_inter]), added to each output row before the routed experts
    /// (nh_moe_combine_shared).  Non-finite values of its intermediate are reported as
    /// "shared_intermediate" (index into [tokens][shared_inter]), ahead of the routed experts'
    /// "intermediate", as the reference meets them.  Routing, experts and
    /// errors as nh_moe_forward_w8a8; INVALID_PARAMS for a NULL w_up_shared, INVALID_SHAPE for
    /// shared_inter == 0 or a missing shared operand.  The workspace
    /// (nh_moe_forward_shared_w8a8_workspace_size) starts with nh_moe_workspace_layout's fields.
    pub fn nh_moe_forward_shared_w8a8_workspace_size(
        tokens: usize,
        hidden: usize,
        inter: usize,
        experts: usize,
        top_k: usize,
        shared_inter: usize,
    ) -> usize;

    pub fn nh_moe_forward_shared_w8a8(
        ctx: *mut nh_context,
        x: *const c_void,
        x_dtype: nh_dtype,
        logits: *const f32,
        tokens: usize,
        hidden: usize,
        inter: usize,
        experts: usize,
        top_k: usize,
        renormalize: c_int,
        scaling: f32,
        w_up: *const i8,
        s_up: *const f32,
        w_down: *const i8,
        s_down: *const f32,
        shared_inter: usize,
        w_up_shared: *const i8,
        s_up_shared: *const f32,
        w_down_shared: *const i8,
        s_down_shared: *const f32,
        biases: *const nh_moe_biases,
        out: *mut c_void,
        out_dtype: nh_dtype,
        workspace: *mut c_void,
        workspace_bytes: usize,
        nonfinite: *mut u64,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    /// The whole MoeLayer::forward_into (moe.rs:154-249) from its input, router included: logits = x
    /// router_w (+ router_b), router_w f32 [hidden][experts] as the reference's dense router
    /// LinearProjection stores it (moe.rs:185-188, linear.rs:324), accumulated in f64 with k ascending
    /// and rounded to f32, then the bias added in f32 (gemm_into_host + project_into, bit-identical;
    /// bf16 x is widened exactly).  Then routing and experts as nh_moe_forward_w8a8, with the shared
    /// expert when shared_inter != 0 (its four operands as nh_moe_forward_shared_w8a8).  MoeLayer
    /// routes with moe_route_host: renormalize = 0, scaling = 1.  The workspace
    /// (nh_moe_layer_w8a8_workspace_size) starts with nh_moe_workspace_layout's fields.  Errors:
    /// INVALID_ROW_COUNT (tokens == 0), INVALID_SHAPE, INVALID_PARAMS (router_w NULL), LENGTH_MISMATCH
    /// "workspace".
    pub fn nh_moe_layer_w8a8_workspace_size(
        tokens: usize,
        hidden: usize,
        inter: usize,
        experts: usize,
        top_k: usize,
        shared_inter: usize,
    ) -> usize;

    pub fn nh_moe_layer_w8a8(
        ctx: *mut nh_context,
        x: *const c_void,
        x_dtype: nh_dtype,
        router_w: *const f32,
        router_b: *const f32,
        tokens: usize,
        hidden: usize,
        inter: usize,
        experts: usize,
        top_k: usize,
        renormalize: c_int,
        scaling: f32,
        w_up: *const i8,
        s_up: *const f32,
        w_down: *const i8,
        s_down: *const f32,
        shared_inter: usize,
        w_up_shared: *const i8,
        s_up_shared: *const f32,
        w_down_shared: *const i8,
        s_down_shared: *const f32,
        biases: *const nh_moe_biases,
        out: *mut c_void,
        out_dtype: nh_dtype,
        workspace: *mut c_void,
        workspace_bytes: usize,
        nonfinite: *mut u64,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    /// Host twin of nh_moe_layer_w8a8 (the library's CPU implementation, for the host-fallback
    /// contract, gemm.rs:290-310): the same arguments in host memory, the same result bit for bit
    /// (router logits in f64 with k ascending, sigmoid top-k, the experts' int8 MLPs in slot order, the
    /// combine), no workspace.  Non-finite values return NH_NON_FINITE_INPUT at once, in the device
    /// word's order: "input", then "shared_intermediate", then "intermediate" (index in expert-sorted
    /// slot order).
    pub fn nh_moe_layer_w8a8_host(
        x: *const c_void,
        x_dtype: nh_dtype,
        router_w: *const f32,
        router_b: *const f32,
        tokens: usize,
        hidden: usize,
        inter: usize,
        experts: usize,
        top_k: usize,
        renormalize: c_int,
        scaling: f32,
        w_up: *const i8,
        s_up: *const f32,
        w_down: *const i8,
        s_down: *const f32,
        shared_inter: usize,
        w_up_shared: *const i8,
        s_up_shared: *const f32,
        w_down_shared: *const i8,
        s_down_shared: *const f32,
        biases: *const nh_moe_biases,
        out: *mut c_void,
        out_dtype: nh_dtype,
        err: *mut nh_error,
    ) -> nh_status;

    /// Device envelope of nh_moe_layer_w8a8's shape (the router GEMM, routing and the experts): 1 when
    /// the device entry point runs it with 16-byte aligned weights and workspace, 0 when it returns
    /// NH_UNSUPPORTED (take the host twin).
    pub fn nh_supports_moe_layer_w8a8(
        tokens: usize,
        hidden: usize,
        inter: usize,
        experts: usize,
        top_k: usize,
        shared_inter: usize,
    ) -> c_int;

    /// INT4 affine weights on the device (W4A8). The reference's INT4 linear weights
    /// (Int4LinearWeights, linear.rs:99-131) are the [input_dim = K][output_dim = N] matrix of affine
    /// codes packed two per byte, low nibble first (quantize.rs:75-77), with one per-tensor scale and
    /// zero point; the reference materialises them as (code - zp) * scale (quantize.rs:202-204) and
    /// rejects projecting with them (linear.rs:316-321).  On the device the codes stay 4-bit: code - zp
    /// is exact in int8 (both 0..15), so the layer is the W8A8 linear with weights (code - zp) and
    /// every row scale equal to `scale`, bit-exact with it, at half the weight bytes.
    pub fn nh_tiled_int4_weights_bytes(n: usize, k: usize) -> usize;

    /// Offline repack of the reference's packed [k][n] codes into the tiled INT4 layout.  Errors:
    /// INVALID_SHAPE (k or n == 0), LENGTH_MISMATCH "packed_weights" (Int4LinearWeights::validate,
    /// linear.rs:113-121) or "tiled", INVALID_PARAMS (zero_point > 15).
    pub fn nh_tile_weights_int4(
        ctx: *mut nh_context,
        packed: *const u8,
        packed_len: usize,
        k: usize,
        n: usize,
        zero_point: u32,
        tiled: *mut u8,
        tiled_len: usize,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_tile_weights_int4_host(
        packed: *const u8,
        packed_len: usize,
        k: usize,
        n: usize,
        zero_point: u32,
        tiled: *mut u8,
        tiled_len: usize,
        err: *mut nh_error,
    ) -> nh_status;

    /// W4A8 linear over tiled INT4 weights: acc = sum_k xq * (code - zp) (int32, exact) on per-token Q2
    /// codes of x, y = ((float)acc * sx) * scale [+ bias]. Two device forms: * bf16 x with
    /// nh_supports_linear_w4a8(m, n, k) (m <= 16, k <= 8192, k % 16 == 0): the fused decode unit
    /// streams the 4-bit weights (groups of 4 rows, each streaming them once); workspace may be NULL; *
    /// otherwise (f32 x, prefill-sized m, longer K; k % 16 == 0 and the W8A8 GEMM envelope): the
    /// weights are expanded into int8 tiles of code - zp in the workspace
    /// (nh_linear_w4a8_workspace_size(m, n, k) bytes, 16-byte aligned; LENGTH_MISMATCH "workspace" when
    /// smaller) and nh_linear_w8a8's path runs on them with every row scale equal to `scale`. Both are
    /// bit-identical to the layer's definition.  Errors in the reference's order: INVALID_SHAPE,
    /// INVALID_PARAMS (validate_int4_params, quantize.rs:180-186), INVALID_ROW_COUNT.
    pub fn nh_supports_linear_w4a8(m: usize, n: usize, k: usize) -> c_int;

    pub fn nh_linear_w4a8_workspace_size(m: usize, n: usize, k: usize) -> usize;

    pub fn nh_linear_w4a8(
        ctx: *mut nh_context,
        x: *const c_void,
        x_dtype: nh_dtype,
        w4_tiled: *const u8,
        scale: f32,
        zero_point: u32,
        bias: *const f32,
        m: usize,
        n: usize,
        k: usize,
        out: *mut c_void,
        out_dtype: nh_dtype,
        workspace: *mut c_void,
        workspace_bytes: usize,
        nonfinite: *mut u64,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    /// The host twin on the reference's packed layout (f32 or bf16 x, any shape).
    pub fn nh_linear_w4a8_host(
        x: *const c_void,
        x_dtype: nh_dtype,
        packed: *const u8,
        packed_len: usize,
        scale: f32,
        zero_point: u32,
        bias: *const f32,
        m: usize,
        n: usize,
        k: usize,
        out: *mut c_void,
        out_dtype: nh_dtype,
        err: *mut nh_error,
    ) -> nh_status;

    pub fn nh_safetensors_tensor_info(
        path: *const c_char,
        name: *const c_char,
        info: *mut nh_tensor_info,
        err: *mut nh_error,
    ) -> nh_status;

    /// The tensor's raw bytes into dst (device memory of exactly data_bytes: LENGTH_MISMATCH "dst"
    /// otherwise); synchronous.
    pub fn nh_safetensors_read(
        ctx: *mut nh_context,
        path: *const c_char,
        name: *const c_char,
        dst: *mut c_void,
        dst_len: usize,
        err: *mut nh_error,
    ) -> nh_status;

    /// An int8 per-row linear layer from a file: codes_name I8 [n][k] (output rows) and scales_name F32
    /// [n], into the tiled layout (tiled_len = nh_tiled_weights_bytes(n, k)) and device scales, through
    /// a device staging buffer of at least n * k bytes; synchronous.  INVALID_SHAPE for a dtype or
    /// shape other than those.
    pub fn nh_load_linear_i8(
        ctx: *mut nh_context,
        path: *const c_char,
        codes_name: *const c_char,
        scales_name: *const c_char,
        n: usize,
        k: usize,
        staging: *mut c_void,
        staging_len: usize,
        tiled: *mut i8,
        tiled_len: usize,
        scales: *mut f32,
        err: *mut nh_error,
    ) -> nh_status;

    /// diagnostics. One read of `bytes` (a multiple of 16, < 2^31) from 16-byte aligned device memory,
    /// in the weight streams' load pattern (16-byte non-temporal loads, one contiguous KiB per wave
    /// instruction, 1024 workgroups of 256 threads): the HBM floor the bandwidth-bound kernels are
    /// compared with.  `sink` is 256 device ints, written only when the data's XOR is one magic value.
    /// No counterpart in the reference.
    pub fn nh_stream_read(
        ctx: *mut nh_context,
        src: *const c_void,
        bytes: usize,
        sink: *mut i32,
        stream: nh_stream,
        err: *mut nh_error,
    ) -> nh_status;

    /// The in-launch handoff of `nh_linear_w8a8` at up to 16 bf16 rows (the row quantizer's
    /// workgroups hand the codes to the GEMV's workgroups inside one launch, through a counter
    /// slot of the context): synchronizes the device, then counts the slots whose wait ran out of
    /// polls (`*timeouts`) and the slots not back at zero (`*busy`).  Both are 0 unless a handoff
    /// launch misbehaved.  No counterpart in the reference.
    pub fn nh_handoff_status(
        ctx: *mut nh_context,
        timeouts: *mut u32,
        busy: *mut u32,
        err: *mut nh_error,
    ) -> nh_status;

    /// synthetic inputs (build-defined seeded generator; the reference has no RNG): splitmix64 ->
    /// Box-Muller (f64) -> f32
    pub fn nh_fill_normal_f32_host(seed: u64, mean: f32, stddev: f32, out: *mut f32, n: usize);
}
