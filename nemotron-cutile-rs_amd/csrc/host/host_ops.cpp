// Host twins: the library's CPU implementation of every op, used by callers
// outside the device envelope (the reference's host-fallback contract,
// gemm.rs:290-310).  They share nh_numerics.h with the kernels, so a twin and
// its kernel round identically.  Built with -ffp-contract=off.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "../kernels/nh_numerics.h"
#include "../runtime/nh_runtime.h"

using namespace nh;

namespace {

bool int4_params_ok(float scale, uint32_t zp) { return std::isfinite(scale) && scale > 0.0f && zp <= 0x0F; }

float load_f32(const void* x, size_t i, nh_dtype d) {
    return d == NH_BF16 ? bf16_to_f32(((const uint16_t*)x)[i]) : ((const float*)x)[i];
}

void store_f32(void* out, size_t i, float v, nh_dtype d) {
    if (d == NH_BF16)
        ((uint16_t*)out)[i] = f32_to_bf16(v);
    else
        ((float*)out)[i] = v;
}

nh_status route_shape(size_t scores_len, size_t tokens, size_t experts, size_t top_k, size_t indices_len,
                      size_t weights_len, nh_error* err) {
    if (experts == 0 || top_k == 0 || top_k > experts)
        return set_error(err, NH_INVALID_SHAPE, "invalid routing shape tokens=%zu experts=%zu top_k=%zu", tokens,
                         experts, top_k);
    size_t sl, rl;
    if (!mul_ok(tokens, experts, &sl) || !mul_ok(tokens, top_k, &rl))
        return set_error(err, NH_INVALID_SHAPE, "routing shape overflows");
    if (scores_len != sl) return mismatch(err, "scores", sl, scores_len);
    if (indices_len != rl) return mismatch(err, "indices", rl, indices_len);
    if (weights_len != rl) return mismatch(err, "weights", rl, weights_len);
    return NH_OK;
}

// Top-k of one token's weights by (total_cmp desc, expert asc).
void top_k_of(const std::vector<float>& w, size_t top_k, int32_t* idx, float* out) {
    std::vector<int32_t> order(w.size());
    for (size_t e = 0; e < w.size(); ++e) order[e] = (int32_t)e;
    std::partial_sort(order.begin(), order.begin() + top_k, order.end(), [&](int32_t a, int32_t b) {
        const int32_t ka = total_cmp_key(w[a]), kb = total_cmp_key(w[b]);
        return ka != kb ? ka > kb : a < b;
    });
    for (size_t j = 0; j < top_k; ++j) {
        idx[j] = order[j];
        out[j] = w[order[j]];
    }
}

}  // namespace

extern "C" {

size_t nh_packed_int4_len(size_t value_count) { return value_count / 2 + value_count % 2; }

nh_status nh_pack_int4_host(const uint8_t* values, size_t n, uint8_t* packed, size_t packed_len, nh_error* err) {
    clear_error(err);
    if (packed_len != nh_packed_int4_len(n)) return mismatch(err, "packed", nh_packed_int4_len(n), packed_len);
    if (packed_len) std::memset(packed, 0, packed_len);
    for (size_t i = 0; i < n; ++i) {
        if (values[i] > 0x0F) {
            if (err) err->byte = values[i];
            return set_error(err, NH_OUT_OF_RANGE, "INT4 value %u out of range", (unsigned)values[i]);
        }
        packed[i >> 1] |= (i & 1) ? (uint8_t)(values[i] << 4) : values[i];
    }
    return NH_OK;
}

nh_status nh_unpack_int4_host(const uint8_t* packed, size_t packed_len, size_t value_count, uint8_t* out,
                              size_t out_len, nh_error* err) {
    clear_error(err);
    if (packed_len != nh_packed_int4_len(value_count))
        return mismatch(err, "packed", nh_packed_int4_len(value_count), packed_len);
    if (out_len != value_count) return mismatch(err, "output", value_count, out_len);
    for (size_t i = 0; i < value_count; ++i) out[i] = (i & 1) ? (packed[i >> 1] >> 4) & 0x0F : packed[i >> 1] & 0x0F;
    return NH_OK;
}

nh_status nh_quantize_int4_host(const float* values, size_t n, float scale, uint32_t zero_point, uint8_t* packed,
                                size_t packed_len, nh_error* err) {
    clear_error(err);
    if (!int4_params_ok(scale, zero_point)) return set_error(err, NH_INVALID_PARAMS, "invalid INT4 params");
    std::vector<uint8_t> codes(n);
    for (size_t i = 0; i < n; ++i) {
        const float v = values[i];
        if (!std::isfinite(v)) {
            if (err) {
                err->index = i;
                err->value = v;
            }
            return set_error(err, NH_NON_FINITE_INPUT, "non-finite input at %zu", i);
        }
        float q = std::round(v / scale + (float)zero_point);
        q = std::min(std::max(q, 0.0f), 15.0f);
        codes[i] = (uint8_t)q;
    }
    return nh_pack_int4_host(codes.data(), n, packed, packed_len, err);
}

nh_status nh_dequantize_int4_host(const uint8_t* packed, size_t packed_len, size_t value_count, float scale,
                                  uint32_t zero_point, float* out, size_t out_len, nh_error* err) {
    clear_error(err);
    if (!int4_params_ok(scale, zero_point)) return set_error(err, NH_INVALID_PARAMS, "invalid INT4 params");
    if (out_len != value_count) return mismatch(err, "output", value_count, out_len);
    std::vector<uint8_t> codes(value_count);
    nh_status st = nh_unpack_int4_host(packed, packed_len, value_count, codes.data(), value_count, err);
    if (st) return st;
    for (size_t i = 0; i < value_count; ++i) out[i] = ((float)codes[i] - (float)zero_point) * scale;
    return NH_OK;
}

nh_status nh_quantize_rows_i8_host(const void* x, nh_dtype dtype, size_t rows, size_t cols, int8_t* q,
                                   float* scales, nh_error* err) {
    clear_error(err);
    if (dtype != NH_F32 && dtype != NH_BF16) return set_error(err, NH_INVALID_PARAMS, "unknown dtype");
    size_t total;
    if (!mul_ok(rows, cols, &total)) return set_error(err, NH_INVALID_SHAPE, "rows*cols overflows");
    for (size_t i = 0; i < total; ++i) {
        const float v = load_f32(x, i, dtype);
        if (!std::isfinite(v)) {
            if (err) {
                err->index = i;
                err->value = v;
            }
            return set_error(err, NH_NON_FINITE_INPUT, "non-finite input at %zu", i);
        }
    }
    for (size_t r = 0; r < rows; ++r) {
        float amax = 0.0f;
        for (size_t c = 0; c < cols; ++c) amax = std::max(amax, std::fabs(load_f32(x, r * cols + c, dtype)));
        const float s = scale_from_amax(amax);
        scales[r] = s;
        const float rcp = s > 0.0f ? 1.0f / s : 0.0f;
        for (size_t c = 0; c < cols; ++c) q[r * cols + c] = (int8_t)quantize_i8_fast(load_f32(x, r * cols + c, dtype), s, rcp);
    }
    return NH_OK;
}

nh_status nh_dequantize_i8_host(const int8_t* q, const float* scales, size_t rows, size_t cols, float* out,
                                nh_error* err) {
    clear_error(err);
    size_t total;
    if (!mul_ok(rows, cols, &total)) return set_error(err, NH_INVALID_SHAPE, "rows*cols overflows");
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) out[r * cols + c] = (float)q[r * cols + c] * scales[r];
    return NH_OK;
}

nh_status nh_gemm_f32_host(const float* lhs, size_t lhs_len, const float* rhs, size_t rhs_len, size_t m, size_t k,
                           size_t n, float* out, size_t out_len, nh_error* err) {
    clear_error(err);
    size_t ll, rl, ol;
    if (m == 0 || k == 0 || n == 0 || !mul_ok(m, k, &ll) || !mul_ok(k, n, &rl) || !mul_ok(m, n, &ol))
        return set_error(err, NH_INVALID_SHAPE, "invalid GEMM shape m=%zu k=%zu n=%zu", m, k, n);
    if (lhs_len != ll) return mismatch(err, "lhs", ll, lhs_len);
    if (rhs_len != rl) return mismatch(err, "rhs", rl, rhs_len);
    if (out_len != ol) return mismatch(err, "output", ol, out_len);
    for (size_t r = 0; r < m; ++r)
        for (size_t c = 0; c < n; ++c) {
            double acc = 0.0;
            for (size_t d = 0; d < k; ++d) acc += (double)lhs[r * k + d] * (double)rhs[d * n + c];
            out[r * n + c] = (float)acc;
        }
    return NH_OK;
}

// Row c of a tiled [n][k] int8 matrix, gathered into row[0..k).
static void untile_row(const int8_t* w, size_t c, size_t k, int8_t* row) {
    const uint64_t kt = tiled_k_tiles(k);
    for (size_t d = 0; d < k; d += 16) {
        const int8_t* src = w + tiled_offset(c, d, kt);
        for (size_t b = 0; b < 16 && d + b < k; ++b) row[d + b] = src[b];
    }
}

nh_status nh_tile_weights_i8_host(const int8_t* wq, size_t n, size_t k, int8_t* tiled, size_t tiled_len,
                                  nh_error* err) {
    clear_error(err);
    if (n == 0 || k == 0 || n > (1ull << 40) || k > (1ull << 40))
        return set_error(err, NH_INVALID_SHAPE, "invalid weight shape n=%zu k=%zu", n, k);
    const size_t need = (size_t)tiled_bytes(n, k);
    if (tiled_len != need) return mismatch(err, "tiled", need, tiled_len);
    std::memset(tiled, 0, need);
    const uint64_t kt = tiled_k_tiles(k);
    for (size_t c = 0; c < n; ++c)
        for (size_t d = 0; d < k; ++d) tiled[tiled_offset(c, d, kt)] = wq[c * k + d];
    return NH_OK;
}

nh_status nh_gemm_w8a8_host(const int8_t* xq, const float* sx, const int8_t* wq, const float* sw, const float* bias,
                            size_t m, size_t n, size_t k, void* out, nh_dtype out_dtype, nh_error* err) {
    clear_error(err);
    size_t t;
    if (m == 0 || n == 0 || k == 0 || !mul_ok(m, k, &t) || !mul_ok(n, k, &t) || !mul_ok(m, n, &t))
        return set_error(err, NH_INVALID_SHAPE, "invalid GEMM shape");
    if (out_dtype != NH_F32 && out_dtype != NH_BF16) return set_error(err, NH_INVALID_PARAMS, "unknown dtype");
    std::vector<int8_t> row(k);
    for (size_t c = 0; c < n; ++c) {
        untile_row(wq, c, k, row.data());
        for (size_t r = 0; r < m; ++r) {
            int32_t acc = 0;
            for (size_t d = 0; d < k; ++d) acc += (int32_t)xq[r * k + d] * (int32_t)row[d];
            float y = epilogue_w8a8(acc, sx[r], sw[c]);
            if (bias) y = y + bias[c];
            store_f32(out, r * n + c, y, out_dtype);
        }
    }
    return NH_OK;
}

// INT4 [K][N] packed codes -> tiled INT4 (nh_numerics.h), same bytes as the
// device repack.
nh_status nh_tile_weights_int4_host(const uint8_t* packed, size_t packed_len, size_t k, size_t n, uint32_t zero_point,
                                    uint8_t* tiled, size_t tiled_len, nh_error* err) {
    clear_error(err);
    size_t kn;
    if (k == 0 || n == 0 || !mul_ok(k, n, &kn)) return set_error(err, NH_INVALID_SHAPE, "invalid INT4 weight shape");
    if (packed_len != nh_packed_int4_len(kn)) return mismatch(err, "packed_weights", nh_packed_int4_len(kn), packed_len);
    if (zero_point > 0x0F) return set_error(err, NH_INVALID_PARAMS, "zero_point %u > 15", zero_point);
    const size_t need = (size_t)tiled_int4_bytes(n, k);
    if (tiled_len != need) return mismatch(err, "tiled", need, tiled_len);
    const size_t kt = (size_t)tiled_k_tiles(k), lanes = need / 8;
    for (size_t c = 0; c < lanes; ++c) {
        const size_t t = c >> 6, lane = c & 63;
        const size_t row = (t / kt) * 16 + (lane & 15), k0 = (t % kt) * 64 + (lane >> 4) * 16;
        uint8_t* dst = tiled + c * 8;
        std::memset(dst, 0, 8);
        for (size_t j = 0; j < 16; ++j) {
            uint32_t code = zero_point;
            if (row < n && k0 + j < k) {
                const size_t i = (k0 + j) * n + row;
                code = (packed[i >> 1] >> ((i & 1) * 4)) & 15u;
            }
            dst[j >> 1] |= (uint8_t)(code << ((j & 1) * 4));
        }
    }
    return NH_OK;
}

// W4A8 linear on the reference's packed [K][N] INT4 weights: per-token Q2 of
// x, acc = sum_k xq * (code - zero_point) exactly in int32, y = ((float)acc *
// sx) * scale [+ bias].
nh_status nh_linear_w4a8_host(const void* x, nh_dtype x_dtype, const uint8_t* packed, size_t packed_len, float scale,
                              uint32_t zero_point, const float* bias, size_t m, size_t n, size_t k, void* out,
                              nh_dtype out_dtype, nh_error* err) {
    clear_error(err);
    size_t kn, mk;
    if (k == 0 || n == 0 || !mul_ok(k, n, &kn)) return set_error(err, NH_INVALID_SHAPE, "invalid linear shape");
    if (packed_len != nh_packed_int4_len(kn)) return mismatch(err, "packed_weights", nh_packed_int4_len(kn), packed_len);
    if (!int4_params_ok(scale, zero_point))
        return set_error(err, NH_INVALID_PARAMS, "invalid INT4 params scale=%g zero_point=%u", (double)scale, zero_point);
    if (m == 0) return set_error(err, NH_INVALID_ROW_COUNT, "row_count must be non-zero, got 0");
    if (out_dtype != NH_F32 && out_dtype != NH_BF16) return set_error(err, NH_INVALID_PARAMS, "unknown dtype");
    if (!mul_ok(m, k, &mk)) return set_error(err, NH_INVALID_SHAPE, "m*k overflows");
    std::vector<int8_t> xq(mk);
    std::vector<float> sx(m);
    nh_status st = nh_quantize_rows_i8_host(x, x_dtype, m, k, xq.data(), sx.data(), err);
    if (st) return st;
    std::vector<int8_t> col(k);
    for (size_t c = 0; c < n; ++c) {
        for (size_t d = 0; d < k; ++d) {
            const size_t i = d * n + c;
            col[d] = (int8_t)((int)((packed[i >> 1] >> ((i & 1) * 4)) & 15u) - (int)zero_point);
        }
        for (size_t r = 0; r < m; ++r) {
            int32_t acc = 0;
            for (size_t d = 0; d < k; ++d) acc += (int32_t)xq[r * k + d] * (int32_t)col[d];
            float y = epilogue_w8a8(acc, sx[r], scale);
            if (bias) y = y + bias[c];
            store_f32(out, r * n + c, y, out_dtype);
        }
    }
    return NH_OK;
}

nh_status nh_gemv_w8a32_host(const float* x, const int8_t* wq, const float* sw, size_t m, size_t n, size_t k,
                             float* y, nh_error* err) {
    clear_error(err);
    size_t t;
    if (m == 0 || n == 0 || k == 0 || !mul_ok(m, k, &t) || !mul_ok(n, k, &t))
        return set_error(err, NH_INVALID_SHAPE, "invalid GEMV shape");
    std::vector<int8_t> row(k);
    for (size_t c = 0; c < n; ++c) {
        untile_row(wq, c, k, row.data());
        for (size_t r = 0; r < m; ++r) {
            double acc = 0.0;
            for (size_t d = 0; d < k; ++d) acc += (double)x[r * k + d] * (double)((float)row[d] * sw[c]);
            y[r * n + c] = (float)acc;
        }
    }
    return NH_OK;
}

float nh_sigmoid_f32_host(float x) { return sigmoid_f32(x); }

nh_status nh_moe_route_sigmoid_topk_host(const float* scores, size_t scores_len, size_t tokens, size_t experts,
                                         size_t top_k, int renormalize, float scaling, int32_t* indices,
                                         size_t indices_len, float* weights, size_t weights_len, nh_error* err) {
    clear_error(err);
    nh_status st = route_shape(scores_len, tokens, experts, top_k, indices_len, weights_len, err);
    if (st) return st;
    std::vector<float> w(experts);
    for (size_t t = 0; t < tokens; ++t) {
        for (size_t e = 0; e < experts; ++e) w[e] = sigmoid_f32(scores[t * experts + e]);
        int32_t* idx = indices + t * top_k;
        float* out = weights + t * top_k;
        top_k_of(w, top_k, idx, out);
        if (renormalize) {
            float total = 0.0f;
            for (size_t j = 0; j < top_k; ++j) total = total + out[j];
            for (size_t j = 0; j < top_k; ++j) out[j] = out[j] / total;
        }
        if (scaling != 1.0f)
            for (size_t j = 0; j < top_k; ++j) out[j] = out[j] * scaling;
    }
    return NH_OK;
}

nh_status nh_moe_route_softmax_topk_host(const float* scores, size_t scores_len, size_t tokens, size_t experts,
                                         size_t top_k, int32_t* indices, size_t indices_len, float* weights,
                                         size_t weights_len, nh_error* err) {
    clear_error(err);
    nh_status st = route_shape(scores_len, tokens, experts, top_k, indices_len, weights_len, err);
    if (st) return st;
    std::vector<float> p(experts);
    for (size_t t = 0; t < tokens; ++t) {
        const float* row = scores + t * experts;
        float mx = -INFINITY;
        for (size_t e = 0; e < experts; ++e) mx = std::fmax(mx, row[e]);
        float total = 0.0f;
        for (size_t e = 0; e < experts; ++e) {
            p[e] = expf_rn(row[e] - mx);
            total = total + p[e];
        }
        for (size_t e = 0; e < experts; ++e) p[e] = p[e] / total;
        int32_t* idx = indices + t * top_k;
        float* out = weights + t * top_k;
        top_k_of(p, top_k, idx, out);
        float sel = 0.0f;
        for (size_t j = 0; j < top_k; ++j) sel = sel + out[j];
        for (size_t j = 0; j < top_k; ++j) out[j] = out[j] / sel;
    }
    return NH_OK;
}

nh_status nh_moe_permute_host(const int32_t* indices, size_t tokens, size_t top_k, size_t experts, int32_t* offsets,
                              int32_t* perm, int32_t* pos, nh_error* err) {
    clear_error(err);
    if (experts == 0 || top_k == 0) return set_error(err, NH_INVALID_SHAPE, "experts and top_k must be non-zero");
    const size_t routes = tokens * top_k;
    std::vector<int32_t> count(experts, 0);
    for (size_t r = 0; r < routes; ++r) {
        if (indices[r] < 0 || (size_t)indices[r] >= experts)
            return set_error(err, NH_OUT_OF_RANGE, "route %zu names expert %d of %zu", r, indices[r], experts);
        ++count[indices[r]];
    }
    offsets[0] = 0;
    for (size_t e = 0; e < experts; ++e) offsets[e + 1] = offsets[e] + count[e];
    std::vector<int32_t> next(offsets, offsets + experts);
    for (size_t r = 0; r < routes; ++r) {
        const int32_t slot = next[indices[r]]++;
        perm[slot] = (int32_t)r;
        pos[r] = slot;
    }
    return NH_OK;
}

}  // extern "C"

namespace {

// R3 on the host, with an optional per-expert bias [E][n] added before
// ReLU^2 (the experts' MlpLayer biases, mlp.rs:201-205).
void grouped_host(const int8_t* aq, const float* sa, int gather, size_t top_k, const int32_t* offsets,
                  const int32_t* perm, size_t experts, const int8_t* w, const float* sw, const float* bias, size_t n,
                  size_t k, int relu2_flag, float* out) {
    std::vector<int8_t> wrow(k);
    for (size_t e = 0; e < experts; ++e) {
        const int8_t* we = w + e * (size_t)tiled_bytes(n, k);
        for (size_t c = 0; c < n; ++c) {
            untile_row(we, c, k, wrow.data());
            for (int32_t slot = offsets[e]; slot < offsets[e + 1]; ++slot) {
                const size_t row = gather ? (size_t)perm[slot] / top_k : (size_t)slot;
                const int8_t* a = aq + row * k;
                int32_t acc = 0;
                for (size_t d = 0; d < k; ++d) acc += (int32_t)a[d] * (int32_t)wrow[d];
                float y = epilogue_w8a8(acc, sa[row], sw[e * n + c]);
                if (bias) y = y + bias[e * n + c];
                if (relu2_flag) y = relu2(y);
                out[(size_t)slot * n + c] = y;
            }
        }
    }
}

// Q2 of x then G1/G3 + bias [+ ReLU^2] into out (the order of
// LinearProjection::project_into, linear.rs:325-339, then mlp.rs:205).  A
// non-finite x is NonFiniteInput with argument `what`.
nh_status linear_host(const void* x, nh_dtype x_dtype, const int8_t* wq, const float* sw, const float* bias,
                      size_t m, size_t n, size_t k, int relu2_flag, void* out, nh_dtype out_dtype, int8_t* xq_out,
                      float* sx_out, const char* what, nh_error* err) {
    std::vector<int8_t> xq(m * k);
    std::vector<float> sx(m);
    nh_status st = nh_quantize_rows_i8_host(x, x_dtype, m, k, xq.data(), sx.data(), err);
    if (st) {
        if (err && st == NH_NON_FINITE_INPUT) err->argument = what;
        return st;
    }
    std::vector<int8_t> row(k);
    for (size_t c = 0; c < n; ++c) {
        untile_row(wq, c, k, row.data());
        for (size_t r = 0; r < m; ++r) {
            int32_t acc = 0;
            for (size_t d = 0; d < k; ++d) acc += (int32_t)xq[r * k + d] * (int32_t)row[d];
            float y = epilogue_w8a8(acc, sx[r], sw[c]);
            if (bias) y = y + bias[c];
            if (relu2_flag) y = relu2(y);
            store_f32(out, r * n + c, y, out_dtype);
        }
    }
    if (xq_out) std::memcpy(xq_out, xq.data(), m * k);
    if (sx_out) std::memcpy(sx_out, sx.data(), m * sizeof(float));
    return NH_OK;
}

// The MLP (mlp.rs:157-211) on the host: h = ReLU^2(x W_up^T + b_up) in f32,
// then h quantized per row (its non-finite values reported as `h_what`) and
// projected down (+ b_down).
nh_status mlp_host(const void* x, nh_dtype x_dtype, const int8_t* w_up, const float* s_up, const float* b_up,
                   const int8_t* w_down, const float* s_down, const float* b_down, size_t m, size_t hidden,
                   size_t inter, void* out, nh_dtype out_dtype, const char* h_what, nh_error* err) {
    std::vector<float> h(m * inter);
    nh_status st = linear_host(x, x_dtype, w_up, s_up, b_up, m, inter, hidden, 1, h.data(), NH_F32, nullptr, nullptr,
                               "input", err);
    if (st) return st;
    return linear_host(h.data(), NH_F32, w_down, s_down, b_down, m, hidden, inter, 0, out, out_dtype, nullptr, nullptr,
                       h_what, err);
}

bool dims_ok(size_t a, size_t b, size_t c) {
    size_t t;
    return a && b && c && mul_ok(a, b, &t) && mul_ok(b, c, &t) && mul_ok(a, c, &t);
}

}  // namespace

extern "C" {

nh_status nh_moe_grouped_gemm_w8a8_host(const int8_t* aq, const float* sa, int gather, size_t top_k,
                                        const int32_t* offsets, const int32_t* perm, size_t routes, size_t a_rows,
                                        size_t experts, const int8_t* w, const float* sw, size_t n, size_t k,
                                        int relu2_flag, float* out, nh_error* err) {
    clear_error(err);
    (void)routes;
    (void)a_rows;
    if (experts == 0 || top_k == 0 || n == 0 || k == 0) return set_error(err, NH_INVALID_SHAPE, "invalid shape");
    grouped_host(aq, sa, gather, top_k, offsets, perm, experts, w, sw, nullptr, n, k, relu2_flag, out);
    return NH_OK;
}

int nh_supports_linear_w8a8(size_t m, size_t n, size_t k) { return dims_ok(m, n, k) && nh_supports_gemm_w8a8(m, n, k); }

int nh_supports_mlp_w8a8(size_t m, size_t hidden, size_t inter) {
    return nh_supports_linear_w8a8(m, inter, hidden) && nh_supports_linear_w8a8(m, hidden, inter);
}

nh_status nh_linear_w8a8_host(const void* x, nh_dtype x_dtype, const int8_t* wq, const float* sw, const float* bias,
                              size_t m, size_t n, size_t k, void* out, nh_dtype out_dtype, int8_t* xq_out,
                              float* sx_out, nh_error* err) {
    clear_error(err);
    // project_into's order (linear.rs:290-311): the layer's shape, then the rows
    if (n == 0 || k == 0) return set_error(err, NH_INVALID_SHAPE, "invalid linear shape k=%zu n=%zu", k, n);
    if (m == 0) return set_error(err, NH_INVALID_ROW_COUNT, "row_count must be non-zero, got 0");
    if ((x_dtype != NH_F32 && x_dtype != NH_BF16) || (out_dtype != NH_F32 && out_dtype != NH_BF16))
        return set_error(err, NH_INVALID_PARAMS, "unknown dtype");
    if (!dims_ok(m, n, k)) return set_error(err, NH_INVALID_SHAPE, "linear shape m=%zu n=%zu k=%zu overflows", m, n, k);
    return linear_host(x, x_dtype, wq, sw, bias, m, n, k, 0, out, out_dtype, xq_out, sx_out, "input", err);
}

nh_status nh_mlp_w8a8_host(const void* x, nh_dtype x_dtype, const int8_t* w_up, const float* s_up, const float* b_up,
                           const int8_t* w_down, const float* s_down, const float* b_down, size_t m, size_t hidden,
                           size_t inter, void* out, nh_dtype out_dtype, nh_error* err) {
    clear_error(err);
    if (hidden == 0 || inter == 0)
        return set_error(err, NH_INVALID_SHAPE, "mlp shape must be non-zero, got hidden_dim=%zu, intermediate_dim=%zu",
                         hidden, inter);
    if (m == 0) return set_error(err, NH_INVALID_ROW_COUNT, "row_count must be non-zero, got 0");
    if ((x_dtype != NH_F32 && x_dtype != NH_BF16) || (out_dtype != NH_F32 && out_dtype != NH_BF16))
        return set_error(err, NH_INVALID_PARAMS, "unknown dtype");
    if (!dims_ok(m, inter, hidden)) return set_error(err, NH_INVALID_SHAPE, "mlp shape overflows");
    return mlp_host(x, x_dtype, w_up, s_up, b_up, w_down, s_down, b_down, m, hidden, inter, out, out_dtype,
                    "intermediate", err);
}

int nh_supports_moe_layer_w8a8(size_t tokens, size_t hidden, size_t inter, size_t experts, size_t top_k,
                               size_t shared_inter) {
    size_t routes, t;
    if (!tokens || !hidden || !inter || !experts || !top_k || top_k > experts) return 0;
    if (!mul_ok(tokens, top_k, &routes) || routes >= (1ull << 31) || !mul_ok(tokens, hidden, &t)) return 0;
    // the router GEMM, the routing and the permutation
    if (!nh_supports_gemm_f32(tokens, hidden, experts) || experts > 1024 || top_k > 64 || tokens > 0x7fffffff / 4)
        return 0;
    // the expert GEMMs (the grouped kernel's envelope covers the fused pair)
    if (!nh_supports_gemm_w8a8(routes, inter, hidden) || !nh_supports_gemm_w8a8(routes, hidden, inter)) return 0;
    if (hidden > 8192 || inter > 8192 || routes * hidden >= (1ull << 31) || routes * inter >= (1ull << 31)) return 0;
    return shared_inter == 0 || nh_supports_mlp_w8a8(tokens, hidden, shared_inter);
}

nh_status nh_moe_layer_w8a8_host(const void* x, nh_dtype x_dtype, const float* router_w, const float* router_b,
                                 size_t tokens, size_t hidden, size_t inter, size_t experts, size_t top_k,
                                 int renormalize, float scaling, const int8_t* w_up, const float* s_up,
                                 const int8_t* w_down, const float* s_down, size_t shared_inter,
                                 const int8_t* w_up_shared, const float* s_up_shared, const int8_t* w_down_shared,
                                 const float* s_down_shared, const nh_moe_biases* biases, void* out,
                                 nh_dtype out_dtype, nh_error* err) {
    clear_error(err);
    // the device entry point's checks, in its order
    if (tokens == 0) return set_error(err, NH_INVALID_ROW_COUNT, "row_count must be non-zero, got 0");
    if (hidden == 0 || experts == 0 || top_k == 0 || top_k > experts || inter == 0)
        return set_error(err, NH_INVALID_SHAPE, "invalid MoE shape");
    if (!router_w) return set_error(err, NH_INVALID_PARAMS, "router_w must not be null");
    if ((shared_inter != 0) != (w_up_shared != nullptr))
        return set_error(err, NH_INVALID_SHAPE, "shared_inter and w_up_shared must be given together");
    if ((x_dtype != NH_F32 && x_dtype != NH_BF16) || (out_dtype != NH_F32 && out_dtype != NH_BF16))
        return set_error(err, NH_INVALID_PARAMS, "unknown dtype");
    const bool has_shared = w_up_shared != nullptr;
    if (has_shared && (!s_up_shared || !w_down_shared || !s_down_shared))
        return set_error(err, NH_INVALID_SHAPE, "shared expert needs intermediate_dim > 0 and all four operands");
    const nh_moe_biases nob{nullptr, nullptr, nullptr, nullptr};
    const nh_moe_biases& b = biases ? *biases : nob;
    if (!has_shared && (b.shared_up || b.shared_down))
        return set_error(err, NH_INVALID_PARAMS, "shared expert biases given without a shared expert");
    size_t routes;
    if (!mul_ok(tokens, top_k, &routes) || !dims_ok(tokens, hidden, experts) || !dims_ok(routes, inter, hidden) ||
        routes >= (1ull << 31))
        return set_error(err, NH_INVALID_SHAPE, "MoE shape overflows");
    // Q2 of every token (the routed experts' A rows); a non-finite x is the
    // layer's input error, ahead of everything else
    std::vector<int8_t> xq(tokens * hidden);
    std::vector<float> sx(tokens);
    nh_status st = nh_quantize_rows_i8_host(x, x_dtype, tokens, hidden, xq.data(), sx.data(), err);
    if (st) {
        if (err && st == NH_NON_FINITE_INPUT) err->argument = "input";
        return st;
    }
    // router.project (moe.rs:185-188): gemm_into_host (f64, k ascending), then the bias in f32
    std::vector<float> logits(tokens * experts);
    for (size_t t = 0; t < tokens; ++t)
        for (size_t e = 0; e < experts; ++e) {
            double acc = 0.0;
            for (size_t d = 0; d < hidden; ++d)
                acc += (double)load_f32(x, t * hidden + d, x_dtype) * (double)router_w[d * experts + e];
            float v = (float)acc;
            if (router_b) v = v + router_b[e];
            logits[t * experts + e] = v;
        }
    std::vector<int32_t> idx(routes), offsets(experts + 1), perm(routes), pos(routes);
    std::vector<float> wts(routes);
    if ((st = nh_moe_route_sigmoid_topk_host(logits.data(), logits.size(), tokens, experts, top_k, renormalize,
                                             scaling, idx.data(), routes, wts.data(), routes, err)))
        return st;
    if ((st = nh_moe_permute_host(idx.data(), tokens, top_k, experts, offsets.data(), perm.data(), pos.data(), err)))
        return st;
    // the shared expert first (moe.rs:197-219): its intermediate is met before the routed experts'
    std::vector<float> shared;
    if (has_shared) {
        shared.resize(tokens * hidden);
        if ((st = mlp_host(x, x_dtype, w_up_shared, s_up_shared, b.shared_up, w_down_shared, s_down_shared,
                           b.shared_down, tokens, hidden, shared_inter, shared.data(), NH_F32, "shared_intermediate",
                           err)))
            return st;
    }
    // up (+ bias, ReLU^2) per slot, h quantized per row (the layer's intermediate), down (+ bias)
    std::vector<float> h(routes * inter), d(routes * hidden);
    grouped_host(xq.data(), sx.data(), 1, top_k, offsets.data(), perm.data(), experts, w_up, s_up, b.up, inter, hidden,
                 1, h.data());
    std::vector<int8_t> hq(routes * inter);
    std::vector<float> sh(routes);
    if ((st = nh_quantize_rows_i8_host(h.data(), NH_F32, routes, inter, hq.data(), sh.data(), err))) {
        if (err && st == NH_NON_FINITE_INPUT) err->argument = "intermediate";
        return st;
    }
    grouped_host(hq.data(), sh.data(), 0, top_k, offsets.data(), perm.data(), experts, w_down, s_down, b.down, hidden,
                 inter, 0, d.data());
    return nh_moe_combine_shared_host(d.data(), pos.data(), wts.data(), has_shared ? shared.data() : nullptr, tokens,
                                      top_k, hidden, out, out_dtype, err);
}

nh_status nh_moe_combine_host(const float* slot_out, const int32_t* pos, const float* weights, size_t tokens,
                              size_t top_k, size_t hidden, void* out, nh_dtype out_dtype, nh_error* err) {
    return nh_moe_combine_shared_host(slot_out, pos, weights, nullptr, tokens, top_k, hidden, out, out_dtype, err);
}

nh_status nh_moe_combine_shared_host(const float* slot_out, const int32_t* pos, const float* weights,
                                     const float* shared, size_t tokens, size_t top_k, size_t hidden, void* out,
                                     nh_dtype out_dtype, nh_error* err) {
    clear_error(err);
    if (out_dtype != NH_F32 && out_dtype != NH_BF16) return set_error(err, NH_INVALID_PARAMS, "unknown dtype");
    for (size_t t = 0; t < tokens; ++t)
        for (size_t h = 0; h < hidden; ++h) {
            float v = 0.0f;
            if (shared) v = v + shared[t * hidden + h];  // the shared expert first (moe.rs:212-219)
            for (size_t j = 0; j < top_k; ++j) {
                const size_t r = t * top_k + j;
                if (pos[r] < 0 || (size_t)pos[r] >= tokens * top_k) continue;  // not placed: adds nothing
                const float p = weights[r] * slot_out[(size_t)pos[r] * hidden + h];
                v = v + p;
            }
            store_f32(out, t * hidden + h, v, out_dtype);
        }
    return NH_OK;
}

// splitmix64 -> two 53-bit uniforms in (0, 1) -> Box-Muller in f64 ->
// mean + std * z rounded to f32; (cos, sin) fill consecutive elements.
void nh_fill_normal_f32_host(uint64_t seed, float mean, float stddev, float* out, size_t n) {
    uint64_t state = seed;
    auto next = [&state]() {
        uint64_t z = (state += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    };
    auto uniform = [&]() {
        double u;
        do u = (double)(next() >> 11) * 0x1.0p-53;
        while (u == 0.0);
        return u;
    };
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        const double u1 = uniform(), u2 = uniform();
        const double r = std::sqrt(-2.0 * std::log(u1));
        const double t = two_pi * u2;
        out[i] = (float)((double)mean + (double)stddev * (r * std::cos(t)));
        if (i + 1 < n) out[i + 1] = (float)((double)mean + (double)stddev * (r * std::sin(t)));
    }
}

}  // extern "C"
