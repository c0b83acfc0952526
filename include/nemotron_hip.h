/*
 * nemotron_hip.h -- C ABI of the MI355X (gfx950) int8 quantized-linear path.
 *
 * Drop-in boundary for nemotron-rs's nemotron-kernels wrappers: a Rust FFI
 * crate (nemotron-hip-sys) binds these declarations 1:1 and the existing
 * wrapper signatures keep their host-fallback contract by calling the *_host
 * twin whenever an nh_supports_* predicate says the device envelope does not
 * cover a shape (gemm.rs:290-299 backend_for_shape pattern).
 *
 * Conventions
 *   - Device entry points take caller-owned DEVICE pointers and an explicit
 *     stream; they only enqueue work (no allocation, no synchronisation).
 *     Every argument is validated on the host BEFORE anything is launched,
 *     as the reference validates before upload (gemm.rs:323, quantize.rs:286).
 *   - *_host entry points take HOST pointers and run the library's own CPU
 *     implementation (the reference's *_host functions).
 *   - Lengths are element counts.  Status codes mirror the reference error
 *     enums; nh_error (optional, may be NULL) carries their payload.
 *   - int8 weights (the wq / w / w_up / w_down arguments of the W8A8 and
 *     W8A32 entry points) are TILED, with one f32 scale per output row N:
 *     a logical [N][K] matrix is stored as ceil(N/16) x KT tiles of 1024
 *     bytes, KT = ceil(K/64); tile (nt, kt) starts at byte (nt*KT + kt)*1024
 *     and its byte 16*(16*g + r) + b holds W[16*nt + r][64*kt + 16*g + b]
 *     (zero outside the matrix).  That is the lane order of the int8 MFMA
 *     operand, so every weight load reads one contiguous KiB.  Quantize the
 *     rows with nh_quantize_rows_i8, then tile them once, offline, with
 *     nh_tile_weights_i8 (size: nh_tiled_weights_bytes).  The reference
 *     stores f32 linear weights [K][N] (linear.rs:324); the quantized row n
 *     is column n of that matrix.  Activations stay row-major [M][K].
 *   - Functions never abort the process.
 */
#ifndef NEMOTRON_HIP_H
#define NEMOTRON_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error variants of QuantizeError (quantize.rs:211-225), GemmError
 * (gemm.rs:175-184), MoeRoutingError (moe_routing.rs:422-430) and LinearError
 * (linear.rs:369-385). */
typedef enum nh_status {
    NH_OK = 0,
    NH_INVALID_SHAPE = 1,     /* *Error::InvalidShape */
    NH_LENGTH_MISMATCH = 2,   /* *Error::LengthMismatch{argument, expected, actual} */
    NH_INVALID_PARAMS = 3,    /* QuantizeError::InvalidParams */
    NH_NON_FINITE_INPUT = 4,  /* QuantizeError::NonFiniteInput{index, value} */
    NH_OUT_OF_RANGE = 5,      /* QuantizeError::Int4OutOfRange(u8) */
    NH_INVALID_ROW_COUNT = 6, /* LinearError::InvalidRowCount */
    NH_UNSUPPORTED = 7,       /* shape outside the device envelope: use the *_host twin */
    NH_DEVICE_ERROR = 8,      /* *Error::DeviceError(String) */
    NH_IO_ERROR = 9,          /* WeightError::Io */
    NH_INVALID_HEADER = 10,   /* WeightError::InvalidHeaderLength / InvalidHeaderJson / InvalidTensorHeader */
    NH_TENSOR_NOT_FOUND = 11  /* WeightError::TensorNotFound */
} nh_status;

typedef struct nh_error {
    const char *argument; /* static string naming the offending argument */
    uint64_t expected;
    uint64_t actual;
    uint64_t index;       /* NonFiniteInput.index (flat, row-major) */
    float value;          /* NonFiniteInput.value */
    uint32_t byte;        /* Int4OutOfRange payload */
    char message[256];    /* human-readable detail (DeviceError text) */
} nh_error;

typedef enum nh_dtype { NH_F32 = 0, NH_BF16 = 1 } nh_dtype;

typedef struct nh_context nh_context;
typedef void *nh_stream; /* hipStream_t; NULL = the device's null stream */

/* ---- D0: device, context, buffers (GpuDevice / GpuTensor, device.rs:117-153,
 *      tensor.rs:259-446) ------------------------------------------------- */
int nh_device_count(void);
/* Loads the gfx950 code object (embedded in the library when path is NULL)
 * with hipModuleLoadData and resolves every kernel once; the context is
 * immutable afterwards and safe to share across threads (device.rs:33-42). */
nh_status nh_context_create(int device, const char *code_object_path, nh_context **out, nh_error *err);
void nh_context_destroy(nh_context *ctx);
int nh_context_device(const nh_context *ctx);
nh_status nh_malloc(nh_context *ctx, size_t bytes, void **ptr, nh_error *err);
nh_status nh_free(nh_context *ctx, void *ptr, nh_error *err);
nh_status nh_memcpy_htod(nh_context *ctx, void *dst, const void *src, size_t bytes, nh_error *err);
nh_status nh_memcpy_dtoh(nh_context *ctx, void *dst, const void *src, size_t bytes, nh_error *err);
nh_status nh_memset_d8(nh_context *ctx, void *dst, int value, size_t bytes, nh_error *err);
nh_status nh_stream_create(nh_context *ctx, nh_stream *out, nh_error *err);
nh_status nh_stream_destroy(nh_context *ctx, nh_stream stream, nh_error *err);
nh_status nh_stream_synchronize(nh_context *ctx, nh_stream stream, nh_error *err);

/* ---- Kernel registry (supported_*_kernels(), gemm.rs:80-82,
 *      quantize.rs:45-47, moe_routing.rs:71-73) --------------------------- */
int nh_kernel_count(void);
/* name of kernel i and its backend tag: 0 = host fallback, 1 = gfx950 device */
const char *nh_kernel_name(int i, int *backend);

/* ---- Q0: affine INT4 (quantize.rs:49-204) ----------------------------- */
size_t nh_packed_int4_len(size_t value_count);                                           /* :49-51 */
nh_status nh_pack_int4_host(const uint8_t *values, size_t n, uint8_t *packed, size_t packed_len,
                            nh_error *err);                                               /* :59-81 */
nh_status nh_unpack_int4_host(const uint8_t *packed, size_t packed_len, size_t value_count,
                              uint8_t *out, size_t out_len, nh_error *err);               /* :89-120 */
nh_status nh_quantize_int4_host(const float *values, size_t n, float scale, uint32_t zero_point,
                                uint8_t *packed, size_t packed_len, nh_error *err);       /* :131-144 */
nh_status nh_dequantize_int4_host(const uint8_t *packed, size_t packed_len, size_t value_count,
                                  float scale, uint32_t zero_point, float *out, size_t out_len,
                                  nh_error *err);                                         /* :156-178 */
/* Q0d, replaces dequantize_int4 (quantize.rs:332-349): unpack + dequantize
 * on the device from the packed bytes (any value_count, not only powers of
 * two as :207-209). */
nh_status nh_dequantize_int4(nh_context *ctx, const uint8_t *packed, size_t packed_len, size_t value_count,
                             float scale, uint32_t zero_point, float *out, size_t out_len, nh_stream stream,
                             nh_error *err);

/* ---- Q1/Q2/Q3: symmetric int8, one f32 scale per row (new; numerics of
 *      quantize_scalar quantize.rs:188-200 with zero point 0) ------------- */
/* s[r] = max|x[r,:]| / 127 (RN); q = clamp(roundf(x / s), -127, 127);
 * s == 0 -> codes 0.  Used for weights (Q1, offline) and per-token
 * activations (Q2).  row_status (optional, [rows]) receives -1 or the first
 * non-finite column of the row; codes of such a row are unspecified. */
nh_status nh_quantize_rows_i8(nh_context *ctx, const void *x, nh_dtype dtype, size_t rows, size_t cols,
                              int8_t *q, float *scales, int32_t *row_status, nh_stream stream, nh_error *err);
nh_status nh_quantize_rows_i8_host(const void *x, nh_dtype dtype, size_t rows, size_t cols, int8_t *q,
                                   float *scales, nh_error *err); /* NonFiniteInput on the first bad element */
/* Q3: out = (float)q * s (dequantize_scalar, quantize.rs:202-204). */
nh_status nh_dequantize_i8(nh_context *ctx, const int8_t *q, const float *scales, size_t rows, size_t cols,
                           float *out, nh_stream stream, nh_error *err);
nh_status nh_dequantize_i8_host(const int8_t *q, const float *scales, size_t rows, size_t cols, float *out,
                                nh_error *err);

/* Tiled int8 weight layout (see Conventions): bytes of the tiled form of
 * an [n][k] matrix (0 for an invalid shape), and the conversion from
 * row-major codes.  New: the reference has no int8 weight format. */
size_t nh_tiled_weights_bytes(size_t n, size_t k);
nh_status nh_tile_weights_i8(nh_context *ctx, const int8_t *wq, size_t n, size_t k, int8_t *tiled,
                             size_t tiled_len, nh_stream stream, nh_error *err);
nh_status nh_tile_weights_i8_host(const int8_t *wq, size_t n, size_t k, int8_t *tiled, size_t tiled_len,
                                  nh_error *err);

/* ---- G0/G1/G2/G3: GEMM family (gemm.rs, linear.rs:283-342) ------------- */
/* G0: gemm_into_host restated (gemm.rs:91-147): f32 in, f64 accumulation. */
nh_status nh_gemm_f32_host(const float *lhs, size_t lhs_len, const float *rhs, size_t rhs_len, size_t m,
                           size_t k, size_t n, float *out, size_t out_len, nh_error *err);
/* G0d: the device GEMM of gemm / gemm_into (gemm.rs:318-363), f32 [m][k] x
 * f32 [k][n] -> f32 [m][n], accumulated in f64 with k ascending for every
 * output: bit-identical to nh_gemm_f32_host.  Same validation and error
 * payloads as gemm_into; any alignment of m, k, n (the reference's cutile
 * kernel needed tile multiples, gemm.rs:247-254, and bridged through the
 * host otherwise).  nh_supports_gemm_f32 is its envelope. */
int nh_supports_gemm_f32(size_t m, size_t k, size_t n);
nh_status nh_gemm_f32(nh_context *ctx, const float *lhs, size_t lhs_len, const float *rhs, size_t rhs_len,
                      size_t m, size_t k, size_t n, float *out, size_t out_len, nh_stream stream, nh_error *err);
/* Device envelope of the W8A8 GEMM family (supports_shape, gemm.rs:247-254). */
int nh_supports_gemm_w8a8(size_t m, size_t n, size_t k);
/* G1/G3: out[m,n] = ((float)sum_k xq[m,k]*wq[n,k] * sx[m]) * sw[n] (+ bias[n])
 * in f32 or bf16 (RNE); wq tiled.  int32 accumulation is exact.  M <= 16
 * runs the HBM-bound GEMV, larger M the MFMA GEMM. */
nh_status nh_gemm_w8a8(nh_context *ctx, const int8_t *xq, const float *sx, const int8_t *wq, const float *sw,
                       const float *bias, size_t m, size_t n, size_t k, void *out, nh_dtype out_dtype,
                       nh_stream stream, nh_error *err);
/* G3 with A also tiled: xq_tiled is nh_tile_weights_i8 of the row-major
 * [m][k] codes (nh_tiled_weights_bytes(m, k) bytes), so every A load is one
 * contiguous KiB as well; same result as nh_gemm_w8a8 on the row-major
 * codes (the tiled-A GEMM is the faster one: the linear entry point uses it
 * for m > 16).  No reference counterpart: G3 is new. */
nh_status nh_gemm_w8a8_ta(nh_context *ctx, const int8_t *xq_tiled, const float *sx, const int8_t *wq,
                          const float *sw, const float *bias, size_t m, size_t n, size_t k, void *out,
                          nh_dtype out_dtype, nh_stream stream, nh_error *err);
nh_status nh_gemm_w8a8_host(const int8_t *xq, const float *sx, const int8_t *wq, const float *sw,
                            const float *bias, size_t m, size_t n, size_t k, void *out, nh_dtype out_dtype,
                            nh_error *err);
/* Non-finite inputs of the quantizing layers (the spec's Q2 error,
 * QuantizeError::NonFiniteInput{index, value} in the style of
 * quantize.rs:193-195).  Device launches cannot return it, so the layer entry
 * points below take an optional device word `nonfinite` (uint64, zero before
 * the first call, e.g. nh_memset_d8): a quantizer that meets a NaN or an
 * infinity records the first one there (the layer's input ahead of its
 * intermediate, then the lowest row-major index) and carries on; the codes of
 * such a row, and the outputs that depend on them, are unspecified.
 * nh_take_nonfinite synchronizes `stream`, returns NH_NON_FINITE_INPUT with
 * err->argument "input" (index into x), "shared_intermediate" (the MoE
 * shared expert's f32 [tokens][shared_inter] ReLU^2 output) or
 * "intermediate" (index into the layer's f32 intermediate: the MLP's
 * [m][inter] ReLU^2 output, the MoE's [routes][inter] up output in
 * expert-sorted slot order), err->index and err->value, and clears the word;
 * NH_OK when it is zero.  The word keeps the first value in that order of
 * stages, then the lowest index.  NULL skips the check at no cost. */
nh_status nh_take_nonfinite(nh_context *ctx, uint64_t *nonfinite, nh_stream stream, nh_error *err);

/* Quantized linear layer, the drop-in for LinearProjection::project_into
 * with int8 per-row weights (linear.rs:283-342): dynamic per-token
 * quantization of x (f32 or bf16) then G1/G3 + bias.  For bf16 x with
 * k <= 8192 and m <= 4 (m <= 8 when k % 512 == 0) the quantization is fused
 * into the GEMV (one launch; the workspace is not touched); other bf16 x
 * with m <= 16 and k <= 8192 is one launch whose quantizer workgroups hand
 * the codes to its GEMV workgroups through the workspace and a counter slot
 * of the context (kHandoffSlots = 256 slots taken in turn: at most 256 such
 * launches may be in flight at once on one context); otherwise the
 * quantization runs as its own launch into a workspace of
 * nh_linear_w8a8_workspace_size(m, k) bytes, 16-byte aligned (for m <= 16
 * it holds the codes in the GEMV's operand order).  Pass that workspace on
 * every call.  xq_out/sx_out (optional) receive the quantized activations
 * (row-major codes, scales). */
size_t nh_linear_w8a8_workspace_size(size_t m, size_t k);
nh_status nh_linear_w8a8(nh_context *ctx, const void *x, nh_dtype x_dtype, const int8_t *wq, const float *sw,
                         const float *bias, size_t m, size_t n, size_t k, void *out, nh_dtype out_dtype,
                         void *workspace, size_t workspace_bytes, int8_t *xq_out, float *sx_out,
                         uint64_t *nonfinite, nh_stream stream, nh_error *err);
/* Device envelope of nh_linear_w8a8 (supports_shape, gemm.rs:247-254): 1 when
 * the device entry point runs the shape (k % 16 == 0, k <= 131072, every
 * dimension and product below 2^31) with a 16-byte aligned wq (and
 * workspace); otherwise it returns NH_UNSUPPORTED and the caller takes the
 * host twin (the host-fallback contract, gemm.rs:290-310). */
int nh_supports_linear_w8a8(size_t m, size_t n, size_t k);
/* Host twin of nh_linear_w8a8 (LinearProjection::project_into with int8
 * per-row weights, linear.rs:283-342): the same arguments in host memory (wq
 * tiled, as on the device), any shape, bit-identical outputs; no workspace.
 * A non-finite x returns NH_NON_FINITE_INPUT ("input", index, value) before
 * any output is written.  xq_out/sx_out optional, as on the device. */
nh_status nh_linear_w8a8_host(const void *x, nh_dtype x_dtype, const int8_t *wq, const float *sw, const float *bias,
                              size_t m, size_t n, size_t k, void *out, nh_dtype out_dtype, int8_t *xq_out,
                              float *sx_out, nh_error *err);
/* nh_linear_w8a8 without a workspace argument and without allocating, for
 * callers that cannot call hipMalloc (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation).  No counterpart in the
 * reference.  The workspace is a static device array of 64 MiB (67108864
 * bytes) per GPU, placed by the HIP runtime and held until the process ends;
 * shapes whose nh_linear_w8a8_workspace_size(m, k) exceeds it return
 * NH_UNSUPPORTED before anything is launched (m = 2048 fits k <= 32704, the
 * 21504-wide MLP down projection included).
 * Results are those of nh_linear_w8a8.  Every call on a GPU shares that
 * GPU's array: calls that overlap on one GPU (concurrent streams or threads)
 * race and must be serialized by the caller. */
nh_status nh_linear_w8a8_noalloc(nh_context *ctx, const void *x, nh_dtype x_dtype, const int8_t *wq, const float *sw,
                                 const float *bias, size_t m, size_t n, size_t k, void *out, nh_dtype out_dtype,
                                 int8_t *xq_out, float *sx_out, uint64_t *nonfinite, nh_stream stream,
                                 nh_error *err);
/* L2: int8 MLP layer, the drop-in for MlpLayer::forward_into with int8
 * per-row weights (mlp.rs:157-211): h = ReLU^2(x W_up^T + b_up) in f32
 * (ReLU^2 after the bias, mlp.rs:205), then out = h W_down^T + b_down, each
 * projection with per-token quantization of its input (nh_linear_w8a8).
 * w_up is tiled [inter][hidden], w_down tiled [hidden][inter]; biases may
 * be NULL.  Errors: INVALID_SHAPE for hidden or inter == 0 (MlpError::
 * InvalidShape), INVALID_ROW_COUNT for m == 0, LENGTH_MISMATCH "workspace"
 * for a workspace smaller than nh_mlp_w8a8_workspace_size(m, hidden, inter)
 * (16-byte aligned; it also holds h). */
size_t nh_mlp_w8a8_workspace_size(size_t m, size_t hidden, size_t inter);
nh_status nh_mlp_w8a8(nh_context *ctx, const void *x, nh_dtype x_dtype, const int8_t *w_up, const float *s_up,
                      const float *b_up, const int8_t *w_down, const float *s_down, const float *b_down, size_t m,
                      size_t hidden, size_t inter, void *out, nh_dtype out_dtype, void *workspace,
                      size_t workspace_bytes, uint64_t *nonfinite, nh_stream stream, nh_error *err);
/* Device envelope of nh_mlp_w8a8: both projections inside
 * nh_supports_linear_w8a8 (16-byte aligned weights and workspace). */
int nh_supports_mlp_w8a8(size_t m, size_t hidden, size_t inter);
/* Host twin of nh_mlp_w8a8: same arguments in host memory, bit-identical
 * outputs, no workspace; NH_NON_FINITE_INPUT "input" or "intermediate" (the
 * f32 [m][inter] ReLU^2 output) as the device word reports them. */
nh_status nh_mlp_w8a8_host(const void *x, nh_dtype x_dtype, const int8_t *w_up, const float *s_up, const float *b_up,
                           const int8_t *w_down, const float *s_down, const float *b_down, size_t m, size_t hidden,
                           size_t inter, void *out, nh_dtype out_dtype, nh_error *err);
/* G2: W8A32 dequant GEMV, y = x * ((float)q * s)^T: the value of
 * materialize_dense + gemm_into_host (linear.rs:126-131).  The device sums
 * each 16-code group in f32 and the groups in f64, then scales by s, so
 * |y - exact| <= 16 u sum_k |x q s| + u |y| (u = 2^-24); the _host form keeps
 * the reference's f64 arithmetic exactly. */
nh_status nh_gemv_w8a32(nh_context *ctx, const float *x, const int8_t *wq, const float *sw, size_t m, size_t n,
                        size_t k, float *y, nh_stream stream, nh_error *err);
nh_status nh_gemv_w8a32_host(const float *x, const int8_t *wq, const float *sw, size_t m, size_t n, size_t k,
                             float *y, nh_error *err);

/* ---- R1..R4: MoE routing, permutation, grouped GEMM, combine ---------- */
float nh_sigmoid_f32_host(float x); /* sigmoid_scalar, activations.rs:73-81 */
/* R1: moe_route_into_host / moe_route (moe_routing.rs:118-141, :499-523):
 * sigmoid scores, top-k by (weight desc, expert asc).  renormalize divides
 * the selected weights by their sum (route order); scaling multiplies after.
 * Indices are int32 (usize in the reference). */
nh_status nh_moe_route_sigmoid_topk(nh_context *ctx, const float *scores, size_t tokens, size_t experts,
                                    size_t top_k, int renormalize, float scaling, int32_t *indices,
                                    float *weights, nh_stream stream, nh_error *err);
nh_status nh_moe_route_sigmoid_topk_host(const float *scores, size_t scores_len, size_t tokens, size_t experts,
                                         size_t top_k, int renormalize, float scaling, int32_t *indices,
                                         size_t indices_len, float *weights, size_t weights_len, nh_error *err);
/* R1s: moe_route_softmax_into_host (moe_routing.rs:143-166, :188-216). */
nh_status nh_moe_route_softmax_topk_host(const float *scores, size_t scores_len, size_t tokens, size_t experts,
                                         size_t top_k, int32_t *indices, size_t indices_len, float *weights,
                                         size_t weights_len, nh_error *err);
/* R2: counts -> offsets[E+1] (exclusive scan), perm (slot -> route, stable
 * by route id inside an expert), pos (route -> slot). */
nh_status nh_moe_permute(nh_context *ctx, const int32_t *indices, size_t tokens, size_t top_k, size_t experts,
                         int32_t *offsets, int32_t *perm, int32_t *pos, nh_stream stream, nh_error *err);
nh_status nh_moe_permute_host(const int32_t *indices, size_t tokens, size_t top_k, size_t experts,
                              int32_t *offsets, int32_t *perm, int32_t *pos, nh_error *err);
/* R3: grouped W8A8 GEMM over the expert segments of offsets (w = E tiled
 * [n][k] matrices at a stride of nh_tiled_weights_bytes(n, k)).  gather != 0:
 * the A row of slot i is token perm[i] / top_k (up projection); otherwise
 * the A row is slot i (down projection).  out is f32 [routes][n]; relu2
 * applies ReLU^2 after the epilogue (mlp.rs:205). */
nh_status nh_moe_grouped_gemm_w8a8(nh_context *ctx, const int8_t *aq, const float *sa, int gather,
                                   size_t top_k, const int32_t *offsets, const int32_t *perm, size_t routes,
                                   size_t a_rows, size_t experts, const int8_t *w, const float *sw, size_t n,
                                   size_t k, int relu2, float *out, nh_stream stream, nh_error *err);
nh_status nh_moe_grouped_gemm_w8a8_host(const int8_t *aq, const float *sa, int gather, size_t top_k,
                                        const int32_t *offsets, const int32_t *perm, size_t routes,
                                        size_t a_rows, size_t experts, const int8_t *w, const float *sw, size_t n,
                                        size_t k, int relu2, float *out, nh_error *err);
/* R4: out[t] = sum_j w[t,j] * slot_out[pos[t*k+j]] in route order (f32),
 * the combine of MoeLayer::forward_into (moe.rs:195, :221-244). */
nh_status nh_moe_combine(nh_context *ctx, const float *slot_out, const int32_t *pos, const float *weights,
                         size_t tokens, size_t top_k, size_t hidden, void *out, nh_dtype out_dtype,
                         nh_stream stream, nh_error *err);
nh_status nh_moe_combine_host(const float *slot_out, const int32_t *pos, const float *weights, size_t tokens,
                              size_t top_k, size_t hidden, void *out, nh_dtype out_dtype, nh_error *err);
/* R4 with the shared expert (moe.rs:197-219): out[t] = 0 + shared[t] +
 * sum_j w[t,j] * slot_out[pos[t*k+j]], each add in that order in f32 (the
 * reference zeroes the output, adds the shared expert's row, then the routes).
 * shared is f32 [tokens][hidden] or NULL (then exactly nh_moe_combine). */
nh_status nh_moe_combine_shared(nh_context *ctx, const float *slot_out, const int32_t *pos, const float *weights,
                                const float *shared, size_t tokens, size_t top_k, size_t hidden, void *out,
                                nh_dtype out_dtype, nh_stream stream, nh_error *err);
nh_status nh_moe_combine_shared_host(const float *slot_out, const int32_t *pos, const float *weights,
                                     const float *shared, size_t tokens, size_t top_k, size_t hidden, void *out,
                                     nh_dtype out_dtype, nh_error *err);
/* Optional biases of the int8 MoE layer's experts.  The reference's routed
 * experts and shared expert are MlpLayers whose projections may carry biases
 * (mlp.rs:79-96, moe.rs:60-65): an up bias is added before ReLU^2, a down
 * bias to the expert's own output, i.e. before the combine weight
 * (mlp.rs:201-208).  Each pointer may be NULL (no bias there); a NULL
 * nh_moe_biases* means no biases at all.  Shared-expert biases without a
 * shared expert are INVALID_PARAMS. */
typedef struct nh_moe_biases {
    const float *up;          /* [experts][inter], expert-major like s_up */
    const float *down;        /* [experts][hidden], like s_down */
    const float *shared_up;   /* [shared_inter] */
    const float *shared_down; /* [hidden] */
} nh_moe_biases;
/* Whole int8 MoE layer on the device: Q2(x) -> R1 -> R2 -> up (R3, gather,
 * + bias, ReLU^2) -> Q2 -> down (R3, + bias) -> R4.  Replaces MoeLayer::forward_into
 * (moe.rs:154-249) for routed experts with int8 per-row weights
 * w_up = E tiled [inter][hidden] matrices, w_down = E tiled [hidden][inter]
 * matrices, each expert at a stride of nh_tiled_weights_bytes of its shape.  The routing stages
 * leave indices, weights, offsets, perm and pos in the workspace at the byte
 * offsets reported by nh_moe_workspace_layout. */
size_t nh_moe_forward_w8a8_workspace_size(size_t tokens, size_t hidden, size_t inter, size_t experts,
                                          size_t top_k);
/* byte offsets in the workspace of: [0] indices i32[T*k], [1] weights
 * f32[T*k], [2] offsets i32[E+1], [3] perm i32[T*k], [4] pos i32[T*k]. */
void nh_moe_workspace_layout(size_t tokens, size_t hidden, size_t inter, size_t experts, size_t top_k,
                             size_t offsets_out[5]);
nh_status nh_moe_forward_w8a8(nh_context *ctx, const void *x, nh_dtype x_dtype, const float *logits,
                              size_t tokens, size_t hidden, size_t inter, size_t experts, size_t top_k,
                              int renormalize, float scaling, const int8_t *w_up, const float *s_up,
                              const int8_t *w_down, const float *s_down, const nh_moe_biases *biases, void *out,
                              nh_dtype out_dtype, void *workspace, size_t workspace_bytes, uint64_t *nonfinite,
                              nh_stream stream, nh_error *err);
/* The int8 MoE layer with its shared expert, MoeLayer::forward_into with
 * shared_expert = Some(..) (moe.rs:197-219): the shared expert is an int8
 * MLP over every token (nh_mlp_w8a8 on x, f32, with biases->shared_up and
 * ->shared_down: w_up_shared tiled [shared_inter][hidden], w_down_shared
 * tiled [hidden][shared_inter]), added to each output row before the routed
 * experts (nh_moe_combine_shared).  Non-finite values of its intermediate are
 * reported as "shared_intermediate" (index into [tokens][shared_inter]),
 * ahead of the routed experts' "intermediate", as the reference meets them.
 * Routing, experts and errors as nh_moe_forward_w8a8; INVALID_PARAMS for a
 * NULL w_up_shared, INVALID_SHAPE for shared_inter == 0 or a missing shared
 * operand.  The workspace (nh_moe_forward_shared_w8a8_workspace_size) starts
 * with nh_moe_workspace_layout's fields. */
size_t nh_moe_forward_shared_w8a8_workspace_size(size_t tokens, size_t hidden, size_t inter, size_t experts,
                                                 size_t top_k, size_t shared_inter);
nh_status nh_moe_forward_shared_w8a8(nh_context *ctx, const void *x, nh_dtype x_dtype, const float *logits,
                                     size_t tokens, size_t hidden, size_t inter, size_t experts, size_t top_k,
                                     int renormalize, float scaling, const int8_t *w_up, const float *s_up,
                                     const int8_t *w_down, const float *s_down, size_t shared_inter,
                                     const int8_t *w_up_shared, const float *s_up_shared,
                                     const int8_t *w_down_shared, const float *s_down_shared,
                                     const nh_moe_biases *biases, void *out, nh_dtype out_dtype, void *workspace,
                                     size_t workspace_bytes, uint64_t *nonfinite, nh_stream stream, nh_error *err);
/* The whole MoeLayer::forward_into (moe.rs:154-249) from its input, router
 * included: logits = x router_w (+ router_b), router_w f32 [hidden][experts]
 * as the reference's dense router LinearProjection stores it (moe.rs:185-188,
 * linear.rs:324), accumulated in f64 with k ascending and rounded to f32,
 * then the bias added in f32 (gemm_into_host + project_into, bit-identical;
 * bf16 x is widened exactly).  Then routing and experts as
 * nh_moe_forward_w8a8, with the shared expert when shared_inter != 0 (its
 * four operands as nh_moe_forward_shared_w8a8).  MoeLayer routes with
 * moe_route_host: renormalize = 0, scaling = 1.  The workspace
 * (nh_moe_layer_w8a8_workspace_size) starts with nh_moe_workspace_layout's
 * fields.  Errors: INVALID_ROW_COUNT (tokens == 0), INVALID_SHAPE,
 * INVALID_PARAMS (router_w NULL), LENGTH_MISMATCH "workspace". */
size_t nh_moe_layer_w8a8_workspace_size(size_t tokens, size_t hidden, size_t inter, size_t experts, size_t top_k,
                                        size_t shared_inter);
nh_status nh_moe_layer_w8a8(nh_context *ctx, const void *x, nh_dtype x_dtype, const float *router_w,
                            const float *router_b, size_t tokens, size_t hidden, size_t inter, size_t experts,
                            size_t top_k, int renormalize, float scaling, const int8_t *w_up, const float *s_up,
                            const int8_t *w_down, const float *s_down, size_t shared_inter,
                            const int8_t *w_up_shared, const float *s_up_shared, const int8_t *w_down_shared,
                            const float *s_down_shared, const nh_moe_biases *biases, void *out, nh_dtype out_dtype,
                            void *workspace, size_t workspace_bytes, uint64_t *nonfinite, nh_stream stream,
                            nh_error *err);
/* Host twin of nh_moe_layer_w8a8 (the library's CPU implementation, for the
 * host-fallback contract, gemm.rs:290-310): the same arguments in host
 * memory, the same result bit for bit (router logits in f64 with k
 * ascending, sigmoid top-k, the experts' int8 MLPs in slot order, the
 * combine), no workspace.  Non-finite values return NH_NON_FINITE_INPUT at
 * once, in the device word's order: "input", then "shared_intermediate",
 * then "intermediate" (index in expert-sorted slot order). */
nh_status nh_moe_layer_w8a8_host(const void *x, nh_dtype x_dtype, const float *router_w, const float *router_b,
                                 size_t tokens, size_t hidden, size_t inter, size_t experts, size_t top_k,
                                 int renormalize, float scaling, const int8_t *w_up, const float *s_up,
                                 const int8_t *w_down, const float *s_down, size_t shared_inter,
                                 const int8_t *w_up_shared, const float *s_up_shared, const int8_t *w_down_shared,
                                 const float *s_down_shared, const nh_moe_biases *biases, void *out,
                                 nh_dtype out_dtype, nh_error *err);
/* Device envelope of nh_moe_layer_w8a8's shape (the router GEMM, routing and
 * the experts): 1 when the device entry point runs it with 16-byte aligned
 * weights and workspace, 0 when it returns NH_UNSUPPORTED (take the host twin). */
int nh_supports_moe_layer_w8a8(size_t tokens, size_t hidden, size_t inter, size_t experts, size_t top_k,
                               size_t shared_inter);

/* ---- INT4 affine weights on the device (W4A8) ---------------------------
 * The reference's INT4 linear weights (Int4LinearWeights, linear.rs:99-131)
 * are the [input_dim = K][output_dim = N] matrix of affine codes packed two
 * per byte, low nibble first (quantize.rs:75-77), with one per-tensor scale
 * and zero point; the reference materialises them as (code - zp) * scale
 * (quantize.rs:202-204) and rejects projecting with them
 * (linear.rs:316-321).  On the device the codes stay 4-bit: code - zp is
 * exact in int8 (both 0..15), so the layer is the W8A8 linear with weights
 * (code - zp) and every row scale equal to `scale`, bit-exact with it, at half
 * the weight bytes. */
size_t nh_tiled_int4_weights_bytes(size_t n, size_t k);
/* Offline repack of the reference's packed [k][n] codes into the tiled INT4
 * layout.  Errors: INVALID_SHAPE (k or n == 0), LENGTH_MISMATCH
 * "packed_weights" (Int4LinearWeights::validate, linear.rs:113-121) or
 * "tiled", INVALID_PARAMS (zero_point > 15). */
nh_status nh_tile_weights_int4(nh_context *ctx, const uint8_t *packed, size_t packed_len, size_t k, size_t n,
                               uint32_t zero_point, uint8_t *tiled, size_t tiled_len, nh_stream stream,
                               nh_error *err);
nh_status nh_tile_weights_int4_host(const uint8_t *packed, size_t packed_len, size_t k, size_t n,
                                    uint32_t zero_point, uint8_t *tiled, size_t tiled_len, nh_error *err);
/* W4A8 linear over tiled INT4 weights: acc = sum_k xq * (code - zp) (int32,
 * exact) on per-token Q2 codes of x, y = ((float)acc * sx) * scale [+ bias].
 * Two device forms:
 *  * bf16 x with nh_supports_linear_w4a8(m, n, k) (m <= 16, k <= 8192,
 *    k % 16 == 0): the fused decode unit streams the 4-bit weights once (3..16
 *    rows with k % 512 == 0 and k <= 4096 in one launch, else groups of 4
 *    rows, each streaming them once); workspace may be NULL;
 *  * otherwise (f32 x, prefill-sized m, longer K; k % 16 == 0 and the W8A8
 *    GEMM envelope): the weights are expanded into int8 tiles of code - zp
 *    in the workspace (nh_linear_w4a8_workspace_size(m, n, k) bytes, 16-byte
 *    aligned; LENGTH_MISMATCH "workspace" when smaller) and nh_linear_w8a8's
 *    path runs on them with every row scale equal to `scale`.
 * Both are bit-identical to the layer's definition.  Errors in the
 * reference's order: INVALID_SHAPE, INVALID_PARAMS (validate_int4_params,
 * quantize.rs:180-186), INVALID_ROW_COUNT. */
int nh_supports_linear_w4a8(size_t m, size_t n, size_t k);
size_t nh_linear_w4a8_workspace_size(size_t m, size_t n, size_t k);
nh_status nh_linear_w4a8(nh_context *ctx, const void *x, nh_dtype x_dtype, const uint8_t *w4_tiled, float scale,
                         uint32_t zero_point, const float *bias, size_t m, size_t n, size_t k, void *out,
                         nh_dtype out_dtype, void *workspace, size_t workspace_bytes, uint64_t *nonfinite,
                         nh_stream stream, nh_error *err);
/* The host twin on the reference's packed layout (f32 or bf16 x, any shape). */
nh_status nh_linear_w4a8_host(const void *x, nh_dtype x_dtype, const uint8_t *packed, size_t packed_len,
                              float scale, uint32_t zero_point, const float *bias, size_t m, size_t n, size_t k,
                              void *out, nh_dtype out_dtype, nh_error *err);

/* ---- safetensors weights into device memory -----------------------------
 * One .safetensors file: the 8-byte little-endian header length, the JSON
 * header, the data section (WeightManifest::load_tensor and
 * read_safetensors_header, nemotron-model/src/weights.rs:161-267).  Every
 * tensor entry is validated as RawTensorHeader::from_value does
 * (weights.rs:276-358) before the lookup.  Errors: IO_ERROR (WeightError::Io),
 * INVALID_HEADER (InvalidHeaderLength: expected = file length, actual = the
 * header length; InvalidHeaderJson; InvalidTensorHeader with the reference's
 * reason text), TENSOR_NOT_FOUND ("tensor not found: <name>"). */
typedef struct nh_tensor_info {
    char dtype[16];      /* the header's dtype string: "I8", "F32", "BF16", "U8", ... */
    uint32_t ndim;
    uint64_t shape[8];
    uint64_t data_begin; /* absolute byte offset of the tensor's data in the file */
    uint64_t data_bytes; /* data_offsets end - start */
} nh_tensor_info;
nh_status nh_safetensors_tensor_info(const char *path, const char *name, nh_tensor_info *info, nh_error *err);
/* The tensor's raw bytes into dst (device memory of exactly data_bytes:
 * LENGTH_MISMATCH "dst" otherwise); synchronous. */
nh_status nh_safetensors_read(nh_context *ctx, const char *path, const char *name, void *dst, size_t dst_len,
                              nh_error *err);
/* An int8 per-row linear layer from a file: codes_name I8 [n][k] (output
 * rows) and scales_name F32 [n], into the tiled layout (tiled_len =
 * nh_tiled_weights_bytes(n, k)) and device scales, through a device staging
 * buffer of at least n * k bytes; synchronous.  INVALID_SHAPE for a dtype or
 * shape other than those. */
nh_status nh_load_linear_i8(nh_context *ctx, const char *path, const char *codes_name, const char *scales_name,
                            size_t n, size_t k, void *staging, size_t staging_len, int8_t *tiled, size_t tiled_len,
                            float *scales, nh_error *err);

/* ---- diagnostics ----------------------------------------------------------
 * One read of `bytes` (a multiple of 16, < 2^31) from 16-byte aligned device
 * memory, in the weight streams' load pattern (16-byte non-temporal loads,
 * one contiguous KiB per wave instruction, 1024 workgroups of 256 threads):
 * the HBM floor the bandwidth-bound kernels are compared with.  `sink` is
 * 256 device ints, written only when the data's XOR is one magic value.  No
 * counterpart in the reference. */
nh_status nh_stream_read(nh_context *ctx, const void *src, size_t bytes, int32_t *sink, nh_stream stream,
                         nh_error *err);

/* The in-launch handoff of nh_linear_w8a8 at up to 16 bf16 rows (the row
 * quantizer's workgroups hand the codes to the GEMV's workgroups inside one
 * launch, through a counter slot of the context): synchronizes the device,
 * then counts the slots whose wait ran out of polls (*timeouts) and the slots
 * not back at zero (*busy).  Both are 0 unless a handoff launch misbehaved.
 * No counterpart in the reference. */
nh_status nh_handoff_status(nh_context *ctx, uint32_t *timeouts, uint32_t *busy, nh_error *err);

/* ---- synthetic inputs (build-defined seeded generator; the reference has
 *      no RNG): splitmix64 -> Box-Muller (f64) -> f32 ------------------- */
void nh_fill_normal_f32_host(uint64_t seed, float mean, float stddev, float *out, size_t n);

#ifdef __cplusplus
}
#endif
#endif /* NEMOTRON_HIP_H */
