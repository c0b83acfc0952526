/*
 * nh_oracle.h -- CPU oracle for the int8 quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * (trungnt13/nemotron-cutile-rs) host algorithms on the path, plus the
 * spec-defined int8 functions that the reference does not have.  Only the
 * tests, the smoke check and the CPU-baseline leg of bench.py may load it;
 * the product library never links or calls it.
 *
 * Every function names the reference file:line it follows.  Functions that are
 * new (no reference implementation) say "spec" and name the invariants that
 * pin them in the tests.
 *
 * Status codes mirror the reference error enums:
 *   QuantizeError (nemotron-kernels/src/quantize.rs:211-225),
 *   GemmError (nemotron-kernels/src/gemm.rs:175-184),
 *   MoeRoutingError (nemotron-kernels/src/moe_routing.rs:422-430),
 *   LinearError (nemotron-nn/src/linear.rs:369-385).
 */
#ifndef NH_ORACLE_H
#define NH_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    OR_OK = 0,
    OR_INVALID_SHAPE = 1,
    OR_LENGTH_MISMATCH = 2,
    OR_INVALID_PARAMS = 3,
    OR_NON_FINITE_INPUT = 4,
    OR_OUT_OF_RANGE = 5,
    OR_INVALID_ROW_COUNT = 6,
};

typedef struct or_error {
    const char *argument; /* LengthMismatch.argument */
    uint64_t expected;    /* LengthMismatch.expected */
    uint64_t actual;      /* LengthMismatch.actual */
    uint64_t index;       /* NonFiniteInput.index */
    float value;          /* NonFiniteInput.value */
    uint32_t byte;        /* Int4OutOfRange(u8) */
} or_error;

/* ---- synthetic inputs (build-defined; the reference has no RNG) ---------- */
uint64_t or_splitmix64_next(uint64_t *state);
void or_fill_normal_f32(uint64_t seed, float mean, float stddev, float *out, size_t n);

/* ---- bf16 (round to nearest even) ---------------------------------------- */
uint16_t or_f32_to_bf16(float x);
float or_bf16_to_f32(uint16_t b);
void or_f32_to_bf16_array(const float *x, uint16_t *out, size_t n);

/* ---- Q0: affine INT4 (quantize.rs:49-204) --------------------------------- */
size_t or_packed_int4_len(size_t value_count);
int or_pack_int4(const uint8_t *values, size_t n, uint8_t *packed, size_t packed_len, or_error *err);
int or_unpack_int4(const uint8_t *packed, size_t packed_len, size_t value_count, uint8_t *out,
                   size_t out_len, or_error *err);
int or_quantize_int4(const float *values, size_t n, float scale, uint32_t zero_point, uint8_t *packed,
                     size_t packed_len, or_error *err);
int or_dequantize_int4(const uint8_t *packed, size_t packed_len, size_t value_count, float scale,
                       uint32_t zero_point, float *out, size_t out_len, or_error *err);

/* ---- Q1/Q2/Q3: symmetric int8, one scale per row (spec) ------------------- */
int or_quantize_rows_i8_f32(const float *x, size_t rows, size_t cols, int8_t *q, float *scales,
                            or_error *err);
int or_quantize_rows_i8_bf16(const uint16_t *x, size_t rows, size_t cols, int8_t *q, float *scales,
                             or_error *err);
void or_dequantize_i8(const int8_t *q, const float *scales, size_t rows, size_t cols, float *out);

/* ---- G0: reference f32 GEMM, f64 accumulation (gemm.rs:91-147,192-208) ---- */
int or_gemm_f32(const float *lhs, size_t lhs_len, const float *rhs, size_t rhs_len, size_t m, size_t k,
                size_t n, float *out, size_t out_len, or_error *err);
/* the same loop over output columns [col0, col1) only (multi-core timing) */
void or_gemm_f32_col_range(const float *lhs, const float *rhs, size_t m, size_t k, size_t n, size_t col0,
                           size_t col1, float *out);

/* ---- G1/G3: W8A8 (spec) --------------------------------------------------- */
void or_gemm_i8_i32(const int8_t *xq, const int8_t *wq, size_t m, size_t n, size_t k, int32_t *acc);
void or_epilogue_w8a8(const int32_t *acc, const float *sx, const float *sw, const float *bias, size_t m,
                      size_t n, int relu2, int out_bf16, void *out);
void or_linear_w8a8(const int8_t *xq, const float *sx, const int8_t *wq, const float *sw,
                    const float *bias, size_t m, size_t n, size_t k, int out_bf16, void *out);

/* ---- G2: W8A32 dequant GEMV = G0 on the materialised weights ------------- */
void or_gemv_w8a32(const float *x, const int8_t *wq, const float *sw, size_t m, size_t n, size_t k,
                   float *y);

/* ---- scalar activations (activations.rs:68-81) ---------------------------- */
float or_sigmoid(float x);
float or_relu2(float x);

/* ---- R1/R1s: routing (moe_routing.rs:118-216) ----------------------------- */
int or_route_sigmoid_topk(const float *scores, size_t scores_len, size_t tokens, size_t experts,
                          size_t top_k, int renormalize, float scaling, int32_t *indices,
                          size_t indices_len, float *weights, size_t weights_len, or_error *err);
int or_route_softmax_topk(const float *scores, size_t scores_len, size_t tokens, size_t experts,
                          size_t top_k, int32_t *indices, size_t indices_len, float *weights,
                          size_t weights_len, or_error *err);

/* ---- R2/R3/R4: permutation, grouped GEMM, combine (spec) ------------------ */
void or_moe_permute(const int32_t *indices, size_t tokens, size_t top_k, size_t experts,
                    int32_t *offsets, int32_t *perm, int32_t *pos);
void or_moe_grouped_w8a8(const int8_t *aq, const float *sa, int gather_tokens, size_t top_k,
                         const int32_t *offsets, const int32_t *perm, size_t experts, const int8_t *w,
                         const float *sw, const float *bias, size_t n, size_t k, int relu2, float *out);
void or_moe_combine(const float *slot_out, const int32_t *pos, const float *weights, size_t tokens,
                    size_t top_k, size_t hidden, int out_bf16, void *out);
int or_moe_forward_w8a8(const uint16_t *x_bf16, const float *logits, size_t tokens, size_t hidden,
                        size_t inter, size_t experts, size_t top_k, int renormalize, float scaling,
                        const int8_t *w_up, const float *s_up, const int8_t *w_down,
                        const float *s_down, uint16_t *out_bf16, int32_t *idx_out, float *w_out,
                        int32_t *offsets_out, int32_t *perm_out, int32_t *pos_out);
void or_moe_combine_shared(const float *slot_out, const int32_t *pos, const float *weights, const float *shared,
                           size_t tokens, size_t top_k, size_t hidden, int out_bf16, void *out);
int or_mlp_w8a8(const uint16_t *x_bf16, size_t rows, size_t hidden, size_t inter, const int8_t *w_up,
                const float *s_up, const float *b_up, const int8_t *w_down, const float *s_down,
                const float *b_down, float *out);
int or_moe_forward_shared_w8a8(const uint16_t *x_bf16, const float *logits, size_t tokens, size_t hidden,
                               size_t inter, size_t experts, size_t top_k, int renormalize, float scaling,
                               const int8_t *w_up, const float *s_up, const int8_t *w_down,
                               const float *s_down, size_t inter_sh, const int8_t *w_up_sh,
                               const float *s_up_sh, const int8_t *w_down_sh, const float *s_down_sh,
                               const float *const *biases, uint16_t *out_bf16, int32_t *idx_out, float *w_out,
                               int32_t *offsets_out, int32_t *perm_out, int32_t *pos_out);

/* ---- W4A8: the reference's INT4 linear weights with int8 activations ---- */
int or_linear_w4a8(const uint16_t *x_bf16, size_t m, size_t k, const uint8_t *packed, size_t n, float scale,
                   uint32_t zp, const float *bias, int out_bf16, void *out);

/* ---- L1/L2 and the reference MoE layer (linear.rs, mlp.rs, moe.rs) ------- */
int or_linear_project(const float *input, size_t input_len, size_t rows, const float *weights,
                      size_t in_dim, size_t out_dim, const float *bias, float *out, size_t out_len,
                      or_error *err);
int or_mlp_forward(const float *input, size_t rows, size_t hidden, size_t inter, const float *w_up,
                   const float *b_up, const float *w_down, const float *b_down, float *out);
int or_moe_forward_dense(const float *input, size_t rows, size_t hidden, size_t experts, size_t top_k,
                         const float *router_w, const float *router_b, size_t inter,
                         const float *const *w_up, const float *const *w_down, const float *const *b_up,
                         const float *const *b_down, size_t shared_inter, const float *shared_up,
                         const float *shared_down, const float *shared_b_up, const float *shared_b_down,
                         float *out);

#ifdef __cplusplus
}
#endif
#endif
