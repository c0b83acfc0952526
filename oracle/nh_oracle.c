/*
 * nh_oracle.c -- CPU oracle (test infrastructure only; see nh_oracle.h).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no -ffast-math) so that
 * every f32/f64 operation is rounded exactly where the reference's Rust code
 * rounds it (Rust never contracts a*b+c into an FMA).
 *
 * Rounding conventions restated from the reference:
 *   - Rust f32::round = round half away from zero = C roundf
 *     (nemotron-kernels/src/quantize.rs:198).
 *   - Rust f32::exp resolves to the platform libm expf on linux-gnu, so the
 *     oracle calls glibc expf (nemotron-kernels/src/activations.rs:73-81).
 *   - Rust f32::max(NaN, y) = y = C fmaxf (activations.rs:68-71).
 *   - f32::total_cmp orders by the sign-magnitude-flipped bit pattern
 *     (nemotron-kernels/src/moe_routing.rs:176-180).
 */
#include "nh_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static void set_mismatch(or_error *err, const char *argument, uint64_t expected, uint64_t actual) {
    if (err) {
        err->argument = argument;
        err->expected = expected;
        err->actual = actual;
    }
}

/* ------------------------------------------------------------------------ */
/* Synthetic inputs: splitmix64 -> two 53-bit uniforms in (0,1) -> Box-Muller
 * in f64 -> mean + std*z rounded to f32.  Pairs (cos, sin) fill consecutive
 * elements.  Build-defined (the reference has no RNG). */
uint64_t or_splitmix64_next(uint64_t *state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static double uniform53(uint64_t *state) {
    double u;
    do {
        u = (double)(or_splitmix64_next(state) >> 11) * 0x1.0p-53;
    } while (u == 0.0);
    return u;
}

void or_fill_normal_f32(uint64_t seed, float mean, float stddev, float *out, size_t n) {
    uint64_t state = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        double u1 = uniform53(&state);
        double u2 = uniform53(&state);
        double r = sqrt(-2.0 * log(u1));
        double t = two_pi * u2;
        double z0 = r * cos(t);
        double z1 = r * sin(t);
        out[i] = (float)((double)mean + (double)stddev * z0);
        if (i + 1 < n) out[i + 1] = (float)((double)mean + (double)stddev * z1);
    }
}

/* ------------------------------------------------------------------------ */
uint16_t or_f32_to_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float or_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void or_f32_to_bf16_array(const float *x, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = or_f32_to_bf16(x[i]);
}

/* ------------------------------------------------------------------------ */
/* Q0: affine INT4.  quantize.rs:49-51 (packed_int4_len). */
size_t or_packed_int4_len(size_t value_count) { return value_count / 2 + (value_count % 2); }

/* quantize.rs:59-81 (pack_int4_into_host): length check, zero fill, low
 * nibble first; the first code > 15 aborts with Int4OutOfRange. */
int or_pack_int4(const uint8_t *values, size_t n, uint8_t *packed, size_t packed_len, or_error *err) {
    size_t expected = or_packed_int4_len(n);
    if (packed_len != expected) {
        set_mismatch(err, "packed", expected, packed_len);
        return OR_LENGTH_MISMATCH;
    }
    memset(packed, 0, packed_len);
    for (size_t i = 0; i < n; ++i) {
        uint8_t v = values[i];
        if (v > 0x0F) {
            if (err) err->byte = v;
            return OR_OUT_OF_RANGE;
        }
        packed[i / 2] |= (i % 2 == 0) ? v : (uint8_t)(v << 4);
    }
    return OR_OK;
}

/* quantize.rs:89-120 (unpack_int4_into_host): packed length checked first,
 * then output length. */
int or_unpack_int4(const uint8_t *packed, size_t packed_len, size_t value_count, uint8_t *out,
                   size_t out_len, or_error *err) {
    size_t expected = or_packed_int4_len(value_count);
    if (packed_len != expected) {
        set_mismatch(err, "packed", expected, packed_len);
        return OR_LENGTH_MISMATCH;
    }
    if (out_len != value_count) {
        set_mismatch(err, "output", value_count, out_len);
        return OR_LENGTH_MISMATCH;
    }
    for (size_t i = 0; i < value_count; ++i) {
        uint8_t byte = packed[i / 2];
        out[i] = (i % 2 == 0) ? (byte & 0x0F) : ((byte >> 4) & 0x0F);
    }
    return OR_OK;
}

/* quantize.rs:180-186 (validate_int4_params). */
static int validate_int4_params(float scale, uint32_t zero_point) {
    if (!isfinite(scale) || scale <= 0.0f || zero_point > 0x0F) return OR_INVALID_PARAMS;
    return OR_OK;
}

/* quantize.rs:131-144 + :188-200: params validated, then every value is
 * quantized (first non-finite aborts) BEFORE the packed length is checked by
 * the pack step. */
int or_quantize_int4(const float *values, size_t n, float scale, uint32_t zero_point, uint8_t *packed,
                     size_t packed_len, or_error *err) {
    int st = validate_int4_params(scale, zero_point);
    if (st) return st;
    uint8_t *codes = (uint8_t *)malloc(n ? n : 1);
    for (size_t i = 0; i < n; ++i) {
        float v = values[i];
        if (!isfinite(v)) {
            if (err) {
                err->index = i;
                err->value = v;
            }
            free(codes);
            return OR_NON_FINITE_INPUT;
        }
        float scaled = v / scale + (float)zero_point;
        float q = roundf(scaled);
        if (q < 0.0f) q = 0.0f;
        if (q > 15.0f) q = 15.0f;
        codes[i] = (uint8_t)q;
    }
    st = or_pack_int4(codes, n, packed, packed_len, err);
    free(codes);
    return st;
}

/* quantize.rs:156-178 + :202-204: params, output length, unpack (packed
 * length), then (code - zp) * scale in f32. */
int or_dequantize_int4(const uint8_t *packed, size_t packed_len, size_t value_count, float scale,
                       uint32_t zero_point, float *out, size_t out_len, or_error *err) {
    int st = validate_int4_params(scale, zero_point);
    if (st) return st;
    if (out_len != value_count) {
        set_mismatch(err, "output", value_count, out_len);
        return OR_LENGTH_MISMATCH;
    }
    uint8_t *codes = (uint8_t *)malloc(value_count ? value_count : 1);
    st = or_unpack_int4(packed, packed_len, value_count, codes, value_count, err);
    if (st == OR_OK) {
        for (size_t i = 0; i < value_count; ++i)
            out[i] = ((float)codes[i] - (float)zero_point) * scale;
    }
    free(codes);
    return st;
}

/* ------------------------------------------------------------------------ */
/* Q1/Q2 (spec; rounding and division style of quantize.rs:197-198 with
 * zero_point 0 and a symmetric clamp):
 *   amax = max_k |x[r,k]|;  s = amax / 127.0f (one RN division);
 *   s == 0  ->  every code 0 (covers an all-zero row and an underflowed s);
 *   else q = clamp(roundf(x / s), -127, 127).
 * The first non-finite element in row-major order is reported as
 * NonFiniteInput{index, value} before anything is written. */
static int8_t quantize_one_i8(float v, float s) {
    if (s == 0.0f) return 0;
    float q = roundf(v / s);
    if (q > 127.0f) q = 127.0f;
    if (q < -127.0f) q = -127.0f;
    return (int8_t)q;
}

static int quantize_rows_core(const float *x, size_t rows, size_t cols, int8_t *q, float *scales,
                              or_error *err) {
    for (size_t i = 0; i < rows * cols; ++i) {
        if (!isfinite(x[i])) {
            if (err) {
                err->index = i;
                err->value = x[i];
            }
            return OR_NON_FINITE_INPUT;
        }
    }
    for (size_t r = 0; r < rows; ++r) {
        const float *row = x + r * cols;
        float amax = 0.0f;
        for (size_t c = 0; c < cols; ++c) {
            float a = fabsf(row[c]);
            if (a > amax) amax = a;
        }
        float s = amax / 127.0f;
        scales[r] = s;
        for (size_t c = 0; c < cols; ++c) q[r * cols + c] = quantize_one_i8(row[c], s);
    }
    return OR_OK;
}

int or_quantize_rows_i8_f32(const float *x, size_t rows, size_t cols, int8_t *q, float *scales,
                            or_error *err) {
    return quantize_rows_core(x, rows, cols, q, scales, err);
}

int or_quantize_rows_i8_bf16(const uint16_t *x, size_t rows, size_t cols, int8_t *q, float *scales,
                             or_error *err) {
    size_t n = rows * cols;
    float *wide = (float *)malloc((n ? n : 1) * sizeof(float));
    for (size_t i = 0; i < n; ++i) wide[i] = or_bf16_to_f32(x[i]);
    int st = quantize_rows_core(wide, rows, cols, q, scales, err);
    free(wide);
    return st;
}

/* Q3: x' = (float)q * s  (dequantize_scalar, quantize.rs:202-204, zp = 0). */
void or_dequantize_i8(const int8_t *q, const float *scales, size_t rows, size_t cols, float *out) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) out[r * cols + c] = (float)q[r * cols + c] * scales[r];
}

/* ------------------------------------------------------------------------ */
/* G0: gemm.rs:192-208 (checked_shape_lengths), :114-147 (validate_shape),
 * :99-109 (row, col, depth ascending; f64 accumulator; one f32 rounding). */
int or_gemm_f32(const float *lhs, size_t lhs_len, const float *rhs, size_t rhs_len, size_t m, size_t k,
                size_t n, float *out, size_t out_len, or_error *err) {
    size_t ll, rl, ol;
    if (m == 0 || k == 0 || n == 0) return OR_INVALID_SHAPE;
    if (__builtin_mul_overflow(m, k, &ll) || __builtin_mul_overflow(k, n, &rl) ||
        __builtin_mul_overflow(m, n, &ol))
        return OR_INVALID_SHAPE;
    if (lhs_len != ll) {
        set_mismatch(err, "lhs", ll, lhs_len);
        return OR_LENGTH_MISMATCH;
    }
    if (rhs_len != rl) {
        set_mismatch(err, "rhs", rl, rhs_len);
        return OR_LENGTH_MISMATCH;
    }
    if (out_len != ol) {
        set_mismatch(err, "output", ol, out_len);
        return OR_LENGTH_MISMATCH;
    }
    for (size_t row = 0; row < m; ++row) {
        for (size_t col = 0; col < n; ++col) {
            double acc = 0.0;
            for (size_t d = 0; d < k; ++d) acc += (double)lhs[row * k + d] * (double)rhs[d * n + col];
            out[row * n + col] = (float)acc;
        }
    }
    return OR_OK;
}

/* gemm_into_host's loop (gemm.rs:99-109) restricted to the output columns
 * [col0, col1) of the same [m][n] output, on the whole [k][n] rhs (row stride
 * n): the per-output arithmetic is identical, so disjoint column ranges run on
 * several threads write exactly or_gemm_f32's output, on the reference's one
 * shared matrix.  Used only to time the host path on several cores. */
void or_gemm_f32_col_range(const float *lhs, const float *rhs, size_t m, size_t k, size_t n, size_t col0,
                           size_t col1, float *out) {
    for (size_t row = 0; row < m; ++row) {
        for (size_t col = col0; col < col1 && col < n; ++col) {
            double acc = 0.0;
            for (size_t d = 0; d < k; ++d) acc += (double)lhs[row * k + d] * (double)rhs[d * n + col];
            out[row * n + col] = (float)acc;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* G1/G3 (spec): acc[m,n] = sum_k xq[m,k] * wq[n,k] exactly in int32
 * (|acc| <= K * 127^2 < 2^31 for K <= 133,152). */
void or_gemm_i8_i32(const int8_t *xq, const int8_t *wq, size_t m, size_t n, size_t k, int32_t *acc) {
    for (size_t r = 0; r < m; ++r) {
        const int8_t *a = xq + r * k;
        for (size_t c = 0; c < n; ++c) {
            const int8_t *b = wq + c * k;
            int32_t s = 0;
            for (size_t d = 0; d < k; ++d) s += (int32_t)a[d] * (int32_t)b[d];
            acc[r * n + c] = s;
        }
    }
}

static float epilogue_value(int32_t acc, float sx, float sw, const float *bias, size_t col, int relu2) {
    float y = ((float)acc * sx) * sw;
    if (bias) y = y + bias[col]; /* bias after the GEMM, as linear.rs:333-339 */
    if (relu2) y = or_relu2(y); /* mlp.rs:205 applies ReLU^2 to the biased up output */
    return y;
}

/* Epilogue (spec): y = ((float)acc * sx[m]) * sw[n]  (two RN multiplies, no
 * FMA) [+ bias[n]] [relu2] -> f32 or bf16 (RNE). */
void or_epilogue_w8a8(const int32_t *acc, const float *sx, const float *sw, const float *bias, size_t m,
                      size_t n, int relu2, int out_bf16, void *out) {
    for (size_t r = 0; r < m; ++r) {
        for (size_t c = 0; c < n; ++c) {
            float y = epilogue_value(acc[r * n + c], sx[r], sw[c], bias, c, relu2);
            if (out_bf16)
                ((uint16_t *)out)[r * n + c] = or_f32_to_bf16(y);
            else
                ((float *)out)[r * n + c] = y;
        }
    }
}

void or_linear_w8a8(const int8_t *xq, const float *sx, const int8_t *wq, const float *sw,
                    const float *bias, size_t m, size_t n, size_t k, int out_bf16, void *out) {
    int32_t *acc = (int32_t *)malloc((m * n + 1) * sizeof(int32_t));
    or_gemm_i8_i32(xq, wq, m, n, k, acc);
    or_epilogue_w8a8(acc, sx, sw, bias, m, n, 0, out_bf16, out);
    free(acc);
}

/* G2: W8A32 dequant GEMV.  The reference path for quantized weights is
 * materialise-then-GEMM (linear.rs:126-131 materialize_dense, then
 * gemm_into_host gemm.rs:99-109): W'[k][n] = (float)q[n][k] * s[n] in f32,
 * then an f64 accumulation over k ascending and one rounding to f32. */
void or_gemv_w8a32(const float *x, const int8_t *wq, const float *sw, size_t m, size_t n, size_t k,
                   float *y) {
    for (size_t r = 0; r < m; ++r) {
        for (size_t c = 0; c < n; ++c) {
            double acc = 0.0;
            for (size_t d = 0; d < k; ++d) {
                float wv = (float)wq[c * k + d] * sw[c];
                acc += (double)x[r * k + d] * (double)wv;
            }
            y[r * n + c] = (float)acc;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* activations.rs:73-81: numerically stable sigmoid with libm expf. */
float or_sigmoid(float x) {
    if (x >= 0.0f) {
        float z = expf(-x);
        return 1.0f / (1.0f + z);
    }
    float z = expf(x);
    return z / (1.0f + z);
}

/* activations.rs:68-71 */
float or_relu2(float x) {
    float r = fmaxf(x, 0.0f);
    return r * r;
}

/* f32::total_cmp key: flip the magnitude bits of negatives. */
static int32_t total_cmp_key(float v) {
    int32_t b;
    memcpy(&b, &v, 4);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

/* moe_routing.rs:218-267 (validate_route, validate_route_outputs,
 * validate_shape). */
static int validate_route(size_t scores_len, size_t tokens, size_t experts, size_t top_k,
                          size_t indices_len, size_t weights_len, or_error *err) {
    if (experts == 0 || top_k == 0 || top_k > experts) return OR_INVALID_SHAPE;
    if (scores_len != tokens * experts) {
        set_mismatch(err, "scores", tokens * experts, scores_len);
        return OR_LENGTH_MISMATCH;
    }
    if (indices_len != tokens * top_k) {
        set_mismatch(err, "indices", tokens * top_k, indices_len);
        return OR_LENGTH_MISMATCH;
    }
    if (weights_len != tokens * top_k) {
        set_mismatch(err, "weights", tokens * top_k, weights_len);
        return OR_LENGTH_MISMATCH;
    }
    return OR_OK;
}

/* Order of moe_routing.rs:176-180 and :201-205: weight descending by
 * total_cmp, ties to the lower expert index.  Selecting the best remaining
 * entry top_k times yields the same prefix as the reference's full sort. */
static void select_ranked(const float *w, size_t experts, size_t top_k, int32_t *idx, float *out_w,
                          unsigned char *taken) {
    memset(taken, 0, experts);
    for (size_t j = 0; j < top_k; ++j) {
        size_t best = experts;
        int32_t best_key = 0;
        for (size_t e = 0; e < experts; ++e) {
            if (taken[e]) continue;
            int32_t key = total_cmp_key(w[e]);
            if (best == experts || key > best_key) {
                best = e;
                best_key = key;
            }
        }
        taken[best] = 1;
        idx[j] = (int32_t)best;
        out_w[j] = w[best];
    }
}

/* R1: moe_routing.rs:118-141 + :168-186 (sigmoid scores, top-k, raw sigmoid
 * weights).  renormalize/scaling are spec additions (north_star asks for
 * renormalised weights; the reference's select_top_k does not renormalise):
 * total = sum of the selected weights in route order (f32), w /= total, then
 * w *= scaling when scaling != 1. */
int or_route_sigmoid_topk(const float *scores, size_t scores_len, size_t tokens, size_t experts,
                          size_t top_k, int renormalize, float scaling, int32_t *indices,
                          size_t indices_len, float *weights, size_t weights_len, or_error *err) {
    int st = validate_route(scores_len, tokens, experts, top_k, indices_len, weights_len, err);
    if (st) return st;
    float *sig = (float *)malloc(experts * sizeof(float));
    unsigned char *taken = (unsigned char *)malloc(experts);
    for (size_t t = 0; t < tokens; ++t) {
        for (size_t e = 0; e < experts; ++e) sig[e] = or_sigmoid(scores[t * experts + e]);
        int32_t *idx = indices + t * top_k;
        float *w = weights + t * top_k;
        select_ranked(sig, experts, top_k, idx, w, taken);
        if (renormalize) {
            float total = 0.0f;
            for (size_t j = 0; j < top_k; ++j) total = total + w[j];
            for (size_t j = 0; j < top_k; ++j) w[j] = w[j] / total;
        }
        if (scaling != 1.0f)
            for (size_t j = 0; j < top_k; ++j) w[j] = w[j] * scaling;
    }
    free(sig);
    free(taken);
    return OR_OK;
}

/* R1s: moe_routing.rs:143-166 + :188-216. */
int or_route_softmax_topk(const float *scores, size_t scores_len, size_t tokens, size_t experts,
                          size_t top_k, int32_t *indices, size_t indices_len, float *weights,
                          size_t weights_len, or_error *err) {
    int st = validate_route(scores_len, tokens, experts, top_k, indices_len, weights_len, err);
    if (st) return st;
    float *p = (float *)malloc(experts * sizeof(float));
    unsigned char *taken = (unsigned char *)malloc(experts);
    for (size_t t = 0; t < tokens; ++t) {
        const float *row = scores + t * experts;
        float mx = -INFINITY;
        for (size_t e = 0; e < experts; ++e) mx = fmaxf(mx, row[e]);
        float total = 0.0f;
        for (size_t e = 0; e < experts; ++e) {
            p[e] = expf(row[e] - mx);
            total = total + p[e];
        }
        for (size_t e = 0; e < experts; ++e) p[e] = p[e] / total;
        int32_t *idx = indices + t * top_k;
        float *w = weights + t * top_k;
        select_ranked(p, experts, top_k, idx, w, taken);
        float selected = 0.0f;
        for (size_t j = 0; j < top_k; ++j) selected = selected + w[j];
        for (size_t j = 0; j < top_k; ++j) w[j] = w[j] / selected;
    }
    free(p);
    free(taken);
    return OR_OK;
}

/* ------------------------------------------------------------------------ */
/* R2 (spec): flat route r = t*top_k + j with expert e_r;
 * offsets = exclusive scan of the per-expert counts (length experts+1);
 * perm lists routes grouped by expert, ascending r inside each group
 * (stable); pos is the inverse (pos[perm[i]] = i). */
void or_moe_permute(const int32_t *indices, size_t tokens, size_t top_k, size_t experts,
                    int32_t *offsets, int32_t *perm, int32_t *pos) {
    size_t routes = tokens * top_k;
    int32_t *fill = (int32_t *)calloc(experts + 1, sizeof(int32_t));
    memset(offsets, 0, (experts + 1) * sizeof(int32_t));
    for (size_t r = 0; r < routes; ++r) offsets[indices[r] + 1] += 1;
    for (size_t e = 0; e < experts; ++e) offsets[e + 1] += offsets[e];
    for (size_t r = 0; r < routes; ++r) {
        int32_t e = indices[r];
        int32_t slot = offsets[e] + fill[e]++;
        perm[slot] = (int32_t)r;
        pos[r] = slot;
    }
    free(fill);
}

/* R3 (spec): per expert e, rows in slots [offsets[e], offsets[e+1]).
 * gather_tokens: the A row of slot i is token perm[i] / top_k (the up
 * projection reads token rows); otherwise A row = slot (the down projection
 * reads the requantised slot rows).  Epilogue as G1 with the expert's bias
 * row (bias [E][n] or NULL: the expert MlpLayer's projection bias,
 * mlp.rs:201-208), then ReLU^2 for the up projection (mlp.rs:205). */
void or_moe_grouped_w8a8(const int8_t *aq, const float *sa, int gather_tokens, size_t top_k,
                         const int32_t *offsets, const int32_t *perm, size_t experts, const int8_t *w,
                         const float *sw, const float *bias, size_t n, size_t k, int relu2, float *out) {
    for (size_t e = 0; e < experts; ++e) {
        const int8_t *we = w + e * n * k;
        const float *se = sw + e * n;
        const float *be = bias ? bias + e * n : NULL;
        for (int32_t slot = offsets[e]; slot < offsets[e + 1]; ++slot) {
            size_t row = gather_tokens ? (size_t)perm[slot] / top_k : (size_t)slot;
            const int8_t *a = aq + row * k;
            for (size_t c = 0; c < n; ++c) {
                const int8_t *b = we + c * k;
                int32_t acc = 0;
                for (size_t d = 0; d < k; ++d) acc += (int32_t)a[d] * (int32_t)b[d];
                out[(size_t)slot * n + c] = epilogue_value(acc, sa[row], se[c], be, c, relu2);
            }
        }
    }
}

/* R4: combine semantics of moe.rs:195 and :221-244 (output zeroed, then
 * value += weight * expert_value in route order, f32), reading each route's
 * expert row from its slot. */
void or_moe_combine(const float *slot_out, const int32_t *pos, const float *weights, size_t tokens,
                    size_t top_k, size_t hidden, int out_bf16, void *out) {
    or_moe_combine_shared(slot_out, pos, weights, NULL, tokens, top_k, hidden, out_bf16, out);
}

/* moe.rs:195-244: the output row starts at 0.0, the shared expert's row is
 * added (moe.rs:212-219), then each route's weighted output in route order. */
void or_moe_combine_shared(const float *slot_out, const int32_t *pos, const float *weights, const float *shared,
                           size_t tokens, size_t top_k, size_t hidden, int out_bf16, void *out) {
    for (size_t t = 0; t < tokens; ++t) {
        for (size_t h = 0; h < hidden; ++h) {
            float v = 0.0f;
            if (shared) v = v + shared[t * hidden + h];
            for (size_t j = 0; j < top_k; ++j) {
                size_t r = t * top_k + j;
                if (pos[r] < 0 || (size_t)pos[r] >= tokens * top_k) continue; /* not placed (pos -1) */
                v = v + weights[r] * slot_out[(size_t)pos[r] * hidden + h];
            }
            if (out_bf16)
                ((uint16_t *)out)[t * hidden + h] = or_f32_to_bf16(v);
            else
                ((float *)out)[t * hidden + h] = v;
        }
    }
}

/* int8 MLP of bf16 rows (spec composition, L2 with int8 weights and
 * optional biases, mlp.rs:201-208): Q2(x) -> W8A8 up + b_up, ReLU^2 (f32) ->
 * Q2 -> W8A8 down + b_down (f32). */
int or_mlp_w8a8(const uint16_t *x_bf16, size_t rows, size_t hidden, size_t inter, const int8_t *w_up,
                const float *s_up, const float *b_up, const int8_t *w_down, const float *s_down,
                const float *b_down, float *out) {
    int8_t *xq = (int8_t *)malloc(rows * hidden + 1);
    float *sx = (float *)malloc((rows + 1) * sizeof(float));
    int32_t *acc = (int32_t *)malloc((rows * (inter > hidden ? inter : hidden) + 1) * sizeof(int32_t));
    float *h = (float *)malloc((rows * inter + 1) * sizeof(float));
    int8_t *hq = (int8_t *)malloc(rows * inter + 1);
    float *sh = (float *)malloc((rows + 1) * sizeof(float));
    or_error err;
    int st = or_quantize_rows_i8_bf16(x_bf16, rows, hidden, xq, sx, &err);
    if (st == OR_OK) {
        or_gemm_i8_i32(xq, w_up, rows, inter, hidden, acc);
        or_epilogue_w8a8(acc, sx, s_up, b_up, rows, inter, 1, 0, h);
        st = or_quantize_rows_i8_f32(h, rows, inter, hq, sh, &err);
    }
    if (st == OR_OK) {
        or_gemm_i8_i32(hq, w_down, rows, hidden, inter, acc);
        or_epilogue_w8a8(acc, sh, s_down, b_down, rows, hidden, 0, 0, out);
    }
    free(xq);
    free(sx);
    free(acc);
    free(h);
    free(hq);
    free(sh);
    return st;
}

/* Full int8 MoE pipeline (spec composition of Q2, R1, R2, R3, R4):
 * x(bf16) -> Q2 -> route -> permute -> up (gather, ReLU^2, f32) -> Q2 ->
 * down (f32 per slot) -> combine -> bf16. */
int or_moe_forward_w8a8(const uint16_t *x_bf16, const float *logits, size_t tokens, size_t hidden,
                        size_t inter, size_t experts, size_t top_k, int renormalize, float scaling,
                        const int8_t *w_up, const float *s_up, const int8_t *w_down,
                        const float *s_down, uint16_t *out_bf16, int32_t *idx_out, float *w_out,
                        int32_t *offsets_out, int32_t *perm_out, int32_t *pos_out) {
    return or_moe_forward_shared_w8a8(x_bf16, logits, tokens, hidden, inter, experts, top_k, renormalize, scaling,
                                      w_up, s_up, w_down, s_down, 0, NULL, NULL, NULL, NULL, NULL, out_bf16,
                                      idx_out, w_out, offsets_out, perm_out, pos_out);
}

/* The same with a shared expert (w_up_sh not NULL): or_mlp_w8a8 of x, added
 * by the combine ahead of the routes (moe.rs:197-219).  biases (NULL, or 4
 * pointers each NULL or not): the routed experts' up [E][inter] and down
 * [E][hidden] biases, the shared expert's up [inter_sh] and down [hidden]. */
int or_moe_forward_shared_w8a8(const uint16_t *x_bf16, const float *logits, size_t tokens, size_t hidden,
                               size_t inter, size_t experts, size_t top_k, int renormalize, float scaling,
                               const int8_t *w_up, const float *s_up, const int8_t *w_down,
                               const float *s_down, size_t inter_sh, const int8_t *w_up_sh,
                               const float *s_up_sh, const int8_t *w_down_sh, const float *s_down_sh,
                               const float *const *biases, uint16_t *out_bf16, int32_t *idx_out, float *w_out,
                               int32_t *offsets_out, int32_t *perm_out, int32_t *pos_out) {
    const float *b_up = biases ? biases[0] : NULL, *b_down = biases ? biases[1] : NULL;
    const float *b_up_sh = biases ? biases[2] : NULL, *b_down_sh = biases ? biases[3] : NULL;
    size_t routes = tokens * top_k;
    int8_t *xq = (int8_t *)malloc(tokens * hidden + 1);
    float *sx = (float *)malloc((tokens + 1) * sizeof(float));
    float *h = (float *)malloc((routes * inter + 1) * sizeof(float));
    int8_t *hq = (int8_t *)malloc(routes * inter + 1);
    float *sh = (float *)malloc((routes + 1) * sizeof(float));
    float *d = (float *)malloc((routes * hidden + 1) * sizeof(float));
    or_error err;
    int st = or_quantize_rows_i8_bf16(x_bf16, tokens, hidden, xq, sx, &err);
    if (st == OR_OK)
        st = or_route_sigmoid_topk(logits, tokens * experts, tokens, experts, top_k, renormalize, scaling,
                                   idx_out, routes, w_out, routes, &err);
    if (st == OR_OK) {
        or_moe_permute(idx_out, tokens, top_k, experts, offsets_out, perm_out, pos_out);
        or_moe_grouped_w8a8(xq, sx, 1, top_k, offsets_out, perm_out, experts, w_up, s_up, b_up, inter, hidden,
                            1, h);
        st = or_quantize_rows_i8_f32(h, routes, inter, hq, sh, &err);
    }
    float *shared = NULL;
    if (st == OR_OK && w_up_sh) {
        shared = (float *)malloc((tokens * hidden + 1) * sizeof(float));
        st = or_mlp_w8a8(x_bf16, tokens, hidden, inter_sh, w_up_sh, s_up_sh, b_up_sh, w_down_sh, s_down_sh,
                         b_down_sh, shared);
    }
    if (st == OR_OK) {
        or_moe_grouped_w8a8(hq, sh, 0, top_k, offsets_out, perm_out, experts, w_down, s_down, b_down, hidden,
                            inter, 0, d);
        or_moe_combine_shared(d, pos_out, w_out, shared, tokens, top_k, hidden, 1, out_bf16);
    }
    free(shared);
    free(xq);
    free(sx);
    free(h);
    free(hq);
    free(sh);
    free(d);
    return st;
}

/* W4A8 linear: the reference's INT4 linear weights
 * (packed [K][N] affine codes, low nibble first, quantize.rs:75-77; one scale
 * and zero point, linear.rs:99-131) with per-token Q2 of bf16 x:
 * acc[m][n] = sum_k xq[m][k] * (code[k][n] - zp), exact in int32, then the
 * W8A8 epilogue with sw[n] = scale. */
int or_linear_w4a8(const uint16_t *x_bf16, size_t m, size_t k, const uint8_t *packed, size_t n, float scale,
                   uint32_t zp, const float *bias, int out_bf16, void *out) {
    int8_t *xq = (int8_t *)malloc(m * k + 1);
    float *sx = (float *)malloc((m + 1) * sizeof(float));
    int8_t *w = (int8_t *)malloc(n * k + 1); /* [N][K] = code - zp, transposed from [K][N] */
    int32_t *acc = (int32_t *)malloc((m * n + 1) * sizeof(int32_t));
    float *sw = (float *)malloc((n + 1) * sizeof(float));
    or_error err;
    int st = or_quantize_rows_i8_bf16(x_bf16, m, k, xq, sx, &err);
    if (st == OR_OK) {
        for (size_t kk = 0; kk < k; ++kk)
            for (size_t c = 0; c < n; ++c) {
                size_t i = kk * n + c;
                int code = (packed[i / 2] >> (4 * (i % 2))) & 15;
                w[c * k + kk] = (int8_t)(code - (int)zp);
            }
        for (size_t c = 0; c < n; ++c) sw[c] = scale;
        or_gemm_i8_i32(xq, w, m, n, k, acc);
        or_epilogue_w8a8(acc, sx, sw, bias, m, n, 0, out_bf16, out);
    }
    free(xq);
    free(sx);
    free(w);
    free(acc);
    free(sw);
    return st;
}

/* ------------------------------------------------------------------------ */
/* L1: linear.rs:283-342 (project_into): row_count, input and output lengths
 * are checked, weights are [in_dim, out_dim] row-major (linear.rs:324), then
 * gemm_into_host and a per-row bias add. */
int or_linear_project(const float *input, size_t input_len, size_t rows, const float *weights,
                      size_t in_dim, size_t out_dim, const float *bias, float *out, size_t out_len,
                      or_error *err) {
    if (in_dim == 0 || out_dim == 0) return OR_INVALID_SHAPE; /* linear.rs:361-367 */
    if (rows == 0) return OR_INVALID_ROW_COUNT;
    if (input_len != rows * in_dim) {
        set_mismatch(err, "input", rows * in_dim, input_len);
        return OR_LENGTH_MISMATCH;
    }
    if (out_len != rows * out_dim) {
        set_mismatch(err, "output", rows * out_dim, out_len);
        return OR_LENGTH_MISMATCH;
    }
    int st = or_gemm_f32(input, input_len, weights, in_dim * out_dim, rows, in_dim, out_dim, out, out_len, err);
    if (st) return st;
    if (bias)
        for (size_t r = 0; r < rows; ++r)
            for (size_t c = 0; c < out_dim; ++c) out[r * out_dim + c] = out[r * out_dim + c] + bias[c];
    return OR_OK;
}

/* L2: mlp.rs:157-211: up projection (+bias), ReLU^2 in place, down
 * projection (+bias). */
int or_mlp_forward(const float *input, size_t rows, size_t hidden, size_t inter, const float *w_up,
                   const float *b_up, const float *w_down, const float *b_down, float *out) {
    float *act = (float *)malloc((rows * inter + 1) * sizeof(float));
    or_error err;
    int st = or_linear_project(input, rows * hidden, rows, w_up, hidden, inter, b_up, act, rows * inter, &err);
    if (st == OR_OK) {
        for (size_t i = 0; i < rows * inter; ++i) act[i] = or_relu2(act[i]);
        st = or_linear_project(act, rows * inter, rows, w_down, inter, hidden, b_down, out, rows * hidden, &err);
    }
    free(act);
    return st;
}

/* Reference MoE layer, moe.rs:154-249: router projection (+bias), sigmoid
 * top-k without renormalisation, output zeroed, optional shared expert added
 * first, then for every route value += weight * expert(all rows)[token]; an
 * expert's MLP runs over ALL rows the first time it is selected (:226-233).
 * Expert e's MlpLayer biases are b_up[e] / b_down[e] (b_up or b_down NULL, or
 * an entry NULL: no bias), the shared expert's shared_b_up / shared_b_down
 * (mlp.rs:79-96, 201-208). */
int or_moe_forward_dense(const float *input, size_t rows, size_t hidden, size_t experts, size_t top_k,
                         const float *router_w, const float *router_b, size_t inter,
                         const float *const *w_up, const float *const *w_down, const float *const *b_up,
                         const float *const *b_down, size_t shared_inter, const float *shared_up,
                         const float *shared_down, const float *shared_b_up, const float *shared_b_down,
                         float *out) {
    if (rows == 0) return OR_INVALID_ROW_COUNT;
    size_t routes = rows * top_k;
    float *scores = (float *)malloc(rows * experts * sizeof(float));
    int32_t *idx = (int32_t *)malloc(routes * sizeof(int32_t));
    float *w = (float *)malloc(routes * sizeof(float));
    float **expert_out = (float **)calloc(experts, sizeof(float *));
    float *shared = NULL;
    or_error err;
    int st = or_linear_project(input, rows * hidden, rows, router_w, hidden, experts, router_b, scores,
                               rows * experts, &err);
    if (st == OR_OK)
        st = or_route_sigmoid_topk(scores, rows * experts, rows, experts, top_k, 0, 1.0f, idx, routes, w,
                                   routes, &err);
    if (st == OR_OK) {
        for (size_t i = 0; i < rows * hidden; ++i) out[i] = 0.0f;
        if (shared_up) {
            shared = (float *)malloc(rows * hidden * sizeof(float));
            st = or_mlp_forward(input, rows, hidden, shared_inter, shared_up, shared_b_up, shared_down,
                                shared_b_down, shared);
        }
    }
    for (size_t t = 0; st == OR_OK && t < rows; ++t) {
        float *orow = out + t * hidden;
        if (shared)
            for (size_t h = 0; h < hidden; ++h) orow[h] = orow[h] + shared[t * hidden + h];
        for (size_t j = 0; j < top_k && st == OR_OK; ++j) {
            int32_t e = idx[t * top_k + j];
            float wt = w[t * top_k + j];
            if (!expert_out[e]) {
                expert_out[e] = (float *)malloc(rows * hidden * sizeof(float));
                st = or_mlp_forward(input, rows, hidden, inter, w_up[e], b_up ? b_up[e] : NULL, w_down[e],
                                    b_down ? b_down[e] : NULL, expert_out[e]);
            }
            for (size_t h = 0; h < hidden; ++h) orow[h] = orow[h] + wt * expert_out[e][t * hidden + h];
        }
    }
    for (size_t e = 0; e < experts; ++e) free(expert_out[e]);
    free(expert_out);
    free(shared);
    free(scores);
    free(idx);
    free(w);
    return st;
}
