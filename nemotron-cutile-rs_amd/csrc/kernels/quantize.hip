// Q1/Q2/Q3 and Q0d kernels: symmetric int8 row quantization, int8
// dequantization, affine INT4 dequantization.  HBM-bound elementwise work:
// one workgroup per row for the row quantizer (two passes over a row that
// stays in L2), grid-stride loops for the dequantizers.
#include "nh_device.h"

using namespace nh;

// One workgroup per row: pass 1 = absmax + first non-finite column, pass 2 =
// codes (quantize_i8_fast: bit-identical to the division, without it).  Rows of the decode/MoE/weight shapes are 1.8-21.5 K elements, so the
// second pass hits L2.
extern "C" __global__ __launch_bounds__(256) void nh_quantize_rows_i8_kernel(QuantizeRowsArgs a) {
    __shared__ float redf[4];
    __shared__ int redi[4];
    const int64_t row = blockIdx.x;
    if (row >= a.rows) return;
    const int64_t cols = a.cols;
    const int64_t base = row * cols;
    float amax = 0.0f;
    int bad = 0x7fffffff;
    if (a.x_dtype == DT_BF16) {
        const uint16_t* x = (const uint16_t*)a.x + base;
        for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
            float v = bf16_to_f32(x[c]);
            if (!is_finite_f32(v)) bad = min(bad, (int)c);
            else amax = fmaxf(amax, fabsf(v));
        }
    } else {
        const float* x = (const float*)a.x + base;
        for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
            float v = x[c];
            if (!is_finite_f32(v)) bad = min(bad, (int)c);
            else amax = fmaxf(amax, fabsf(v));
        }
    }
    amax = block_max(amax, redf);
    bad = block_min_i32(bad, redi);
    const float s = scale_from_amax(amax);
    if (threadIdx.x == 0) {
        a.scales[row] = s;
        if (a.row_status) a.row_status[row] = bad == 0x7fffffff ? -1 : bad;
    }
    int8_t* q = a.q + base;
    const float r = s > 0.0f ? 1.0f / s : 0.0f;
    if (a.x_dtype == DT_BF16) {
        const uint16_t* x = (const uint16_t*)a.x + base;
        for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) q[c] = (int8_t)quantize_i8_fast(bf16_to_f32(x[c]), s, r);
    } else {
        const float* x = (const float*)a.x + base;
        for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) q[c] = (int8_t)quantize_i8_fast(x[c], s, r);
    }
}

// Row-major int8 [rows][cols] -> the tiled layout (nh_numerics.h): thread c
// writes 16-byte chunk c of the tiled buffer (lane c % 64 of tile c / 64),
// zeros outside the matrix.
extern "C" __global__ __launch_bounds__(256) void nh_tile_weights_kernel(TileWeightsArgs a) {
    for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < a.chunks;
         c += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = c >> 6;
        const int lane = (int)(c & 63);
        const int64_t row = (t / a.kt) * 16 + (lane & 15);
        const int64_t k0 = (t % a.kt) * 64 + (lane >> 4) * 16;
        v4i v = {0, 0, 0, 0};
        if (row < a.rows && k0 < a.cols) {
            const int8_t* src = a.w + row * a.cols + k0;
            if (k0 + 16 <= a.cols && ((uintptr_t)src & 15) == 0) {
                v = *(const v4i*)src;
            } else {
                uint8_t bytes[16];
                for (int b = 0; b < 16; ++b) bytes[b] = k0 + b < a.cols ? (uint8_t)src[b] : 0;
                for (int j = 0; j < 4; ++j)
                    v[j] = (int)(bytes[4 * j] | (bytes[4 * j + 1] << 8) | (bytes[4 * j + 2] << 16) |
                                 ((uint32_t)bytes[4 * j + 3] << 24));
            }
        }
        *(v4i*)(a.tiled + c * 16) = v;
    }
}

extern "C" __global__ __launch_bounds__(256) void nh_dequantize_i8_kernel(DequantizeI8Args a) {
    const int64_t total = a.rows * a.cols;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / a.cols;
        a.out[i] = (float)a.q[i] * a.scales[r];
    }
}

// (code - zero_point) * scale straight from the packed nibbles (low nibble
// first, quantize.rs:75-77 and :110-116); the reference unpacked on the host
// and uploaded one f32 per code (quantize.rs:294-301).
extern "C" __global__ __launch_bounds__(256) void nh_dequantize_int4_kernel(DequantizeInt4Args a) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.value_count;
         i += (int64_t)gridDim.x * blockDim.x) {
        const uint8_t byte = a.packed[i >> 1];
        const uint32_t code = (i & 1) ? ((byte >> 4) & 0x0F) : (byte & 0x0F);
        a.out[i] = ((float)code - a.zero_point) * a.scale;
    }
}
