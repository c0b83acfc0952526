// Q1/Q2/Q3 and Q0d kernels: symmetric int8 row quantization, int8
// dequantization, affine INT4 dequantization.  HBM-bound elementwise work:
// one workgroup per row for the row quantizer (two passes over a row that
// stays in L2), grid-stride loops for the dequantizers.
#include "nh_device.h"

using namespace nh;

// One workgroup per row: pass 1 = absmax + first non-finite column, pass 2 =
// codes.  Rows of the decode/MoE/weight shapes are 1.8-21.5 K elements, so the
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
    if (a.x_dtype == DT_BF16) {
        const uint16_t* x = (const uint16_t*)a.x + base;
        for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) q[c] = quantize_i8(bf16_to_f32(x[c]), s);
    } else {
        const float* x = (const float*)a.x + base;
        for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) q[c] = quantize_i8(x[c], s);
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
