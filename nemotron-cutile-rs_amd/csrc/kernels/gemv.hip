// G1 / decode unit / G2: the M <= 16 GEMV family.  These kernels stream the
// int8 weight matrix from HBM exactly once, so they are HBM-bound: the design
// goal is bytes in flight from the first cycle to the last.
//
// Weights are in the tiled layout (nh_numerics.h): the KT = ceil(K/64) tiles
// of one 16-row N tile are KT contiguous KiB, and one 64-lane 16-byte load of
// a tile is the B operand of one v_mfma_i32_16x16x64_i8 K step, so every
// weight load instruction reads one contiguous KiB.  A workgroup owns one
// 16-row N tile; wave w of W owns K tiles w, w + W, w + 2W, ...  Each wave
// issues the loads of a whole 16-tile slab (16 KiB) before doing anything
// else, with the non-temporal policy (the weights are read once), so the
// activation prologue and the MFMAs run while the slab is in flight.  The
// waves' int32 partial tiles are summed through LDS and wave 0 applies the
// epilogue y = ((float)acc * sx[m]) * sw[n] [+ bias[n]].
//
// MFMA operand convention (16x16x64, int8): lane l supplies row (l % 16) of
// its operand and bytes [16*(l/16), +16) of the 64-byte K step; the same
// convention for A and B makes the dot product independent of how the
// hardware orders K inside a lane.  Result: lane l holds
// D[m = 4*(l/16) + r][n = l % 16] in register r.
//
// Tiles past KT (when W does not divide KT) read zeros from the buffer
// resource and meet zero activation codes.
#include "nh_device.h"

using namespace nh;

namespace {

constexpr int kSlab = 16;                // K tiles per wave in flight at once
// The decode unit issues the first kSlabHead tiles of its slab, quantizes the
// activations while they stream (the activation loads went first, so they
// return first), then issues the rest: the quantizer's VALU work no longer
// waits for the whole slab to have been issued (measured 0.1-0.2 us faster).
constexpr int kSlabHead = 4;

// The KT KiB of 16-row N tile `tile`.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_tile_rsrc(const int8_t* wq, int tile, int kt) {
    return make_rsrc(wq + (int64_t)tile * kt * 1024, (uint32_t)kt * 1024u);
}

// Loads of one slab: K tiles first, first + stride, ... (16 of them).
__device__ __forceinline__ void load_slab(v4i (&b)[kSlab], __amdgpu_buffer_rsrc_t r, int first, int stride,
                                          int lane) {
#pragma unroll
    for (int s = 0; s < kSlab; ++s) b[s] = buffer_load16_stream(r, (first + s * stride) * 1024 + lane * 16);
}

// Sum the waves' partial tiles into wave 0 (which returns true); `red`
// holds W * 64 v4i.
__device__ __forceinline__ bool reduce_waves(v4i& acc, v4i* red, int W) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (W > 1) {
        red[wave * 64 + lane] = acc;
        __syncthreads();
        if (wave == 0)
            for (int w = 1; w < W; ++w) acc += red[w * 64 + lane];
    }
    return wave == 0;
}

__device__ __forceinline__ void store_y(void* out, int out_dtype, int64_t i, int32_t acc, float sx, float swn,
                                        const float* bias, float bn) {
    float y = epilogue_w8a8(acc, sx, swn);
    if (bias) y = y + bn;
    store_out(out, i, y, out_dtype);
}

}  // namespace

// G1: quantized activations already in memory (xq [M][K] row-major, M <= 16);
// the A fragments come from L2 (xq is at most 16 x K bytes, shared by every
// workgroup).  Any K <= 131072: waves walk their K tiles slab by slab.
extern "C" __global__ __launch_bounds__(512) void nh_gemv_w8a8_kernel(GemvW8A8Args a) {
    __shared__ v4i red[8 * 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = a.waves;
    const int r16 = lane & 15, g = lane >> 4;
    const int M = a.M, N = a.N, K = a.K, kt = a.kt;
    const int tile = blockIdx.x;
    const __amdgpu_buffer_rsrc_t wr = row_tile_rsrc(a.wq, tile, kt);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.xq, (uint32_t)M * (uint32_t)K);
    // epilogue operands first, ahead of the weight stream
    const int n = tile * 16 + r16;
    const float swn = n < N ? a.sw[n] : 0.0f;
    const float bn = (a.bias && n < N) ? a.bias[n] : 0.0f;
    float sxl[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) sxl[r] = 4 * g + r < M ? a.sx[4 * g + r] : 0.0f;
    const int steps = (kt + W - 1) / W;
    v4i acc = {0, 0, 0, 0};
    for (int s0 = 0; s0 < steps; s0 += kSlab) {
        v4i x[kSlab], b[kSlab];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < kSlab; ++s) {  // activation fragments (L2) first
            const int k = (wave + (s0 + s) * W) * 64 + g * 16;
            x[s] = buffer_load16(xr, (r16 < M && k < K) ? r16 * K + k : kOutOfRange);
        }
        load_slab(b, wr, wave + s0 * W, W, lane);  // then the weight slab (HBM)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < kSlab; ++s) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x[s], b[s], acc, 0, 0, 0);
    }
    if (reduce_waves(acc, red, W) && n < N) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (4 * g + r < M) store_y(a.out, a.out_dtype, (int64_t)(4 * g + r) * N + n, acc[r], sxl[r], swn, a.bias, bn);
    }
}

// Decode unit, M <= MM <= 4, K <= 8192: per-token quantization of the bf16
// activation rows (Q2) fused in front of the GEMV.  Every workgroup quantizes
// the rows into LDS itself while its weight slab is in flight, so the unit is
// one launch and the int8 activations never round-trip through HBM.  The
// quantizer multiplies by the reciprocal scale (quantize8_bf16) with an exact
// tie decision for the rare value next to a rounding tie, so codes and scales
// are bit-identical to quantize_i8 in every workgroup; workgroup 0 also
// writes them out when asked.
template <int MM>
__device__ __forceinline__ void linear_decode(const LinearDecodeArgs& a, int8_t* xs) {
    __shared__ v4i red[8 * 64];
    __shared__ float redf[8][MM];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = a.waves;
    const int T = 64 * W;
    const int M = a.M, N = a.N, K = a.K, kt = a.kt;
    const int ldx = W * 1024 + 16;  // LDS row pitch: every K tile a wave can own (16 per wave)
    const int tile = blockIdx.x;

    // 1. this thread's two 16-byte chunks (8 bf16 values each: chunks t and
    //    t + T, 2 * T * 8 = W * 1024 values) of each row, the epilogue
    //    operands, then the head of the weight slab.  Loads complete in
    //    issue order, so the quantizer waits only for the activations.
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, (uint32_t)M * (uint32_t)K * 2u);
    v4i xv[MM][2];
    v4i b[kSlab];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            const int c = (threadIdx.x + v * T) * 8;
            xv[m][v] = buffer_load16(xrs, (m < M && c < K) ? (m * K + c) * 2 : kOutOfRange);
        }
    const int n = tile * 16 + (lane & 15);
    const float swn = n < N ? a.sw[n] : 0.0f;
    const float bn = (a.bias && n < N) ? a.bias[n] : 0.0f;
    const __amdgpu_buffer_rsrc_t wr = row_tile_rsrc(a.wq, tile, kt);
#pragma unroll
    for (int s = 0; s < kSlabHead; ++s) b[s] = buffer_load16_stream(wr, (wave + s * W) * 1024 + lane * 16);
    __builtin_amdgcn_sched_barrier(0);

    // 2. row absmax over the workgroup; every thread derives the scales
    float sx[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        float amax = 0.0f;
#pragma unroll
        for (int v = 0; v < 2; ++v)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t u = (uint32_t)xv[m][v][j];
                amax = fmaxf(amax, fmaxf(fabsf(f32_from_bits(u << 16)), fabsf(f32_from_bits(u & 0xffff0000u))));
            }
        amax = wave_max(amax);
        if (lane == 0) redf[wave][m] = amax;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        float r = redf[0][m];
        for (int i = 1; i < W; ++i) r = fmaxf(r, redf[i][m]);
        sx[m] = scale_from_amax(r);
    }
    // 3. codes into LDS (zeros past K and for rows >= M)
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        const float rcp = 1.0f / sx[m];
        const bool pow2 = scale_is_pow2(sx[m]);
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            const int c = (threadIdx.x + v * T) * 8;
            uint32_t code[2] = {0, 0};
            if (m < M && c < K) {
                quantize8_bf16(xv[m][v], sx[m], rcp, pow2, code);
                if (blockIdx.x == 0 && a.xq_out) *(uint2*)(a.xq_out + (int64_t)m * K + c) = make_uint2(code[0], code[1]);
            }
            *(uint2*)(xs + m * ldx + c) = make_uint2(code[0], code[1]);
        }
        if (blockIdx.x == 0 && threadIdx.x == 0 && a.sx_out && m < M) a.sx_out[m] = sx[m];
    }
    // the rest of the slab: its loads queue behind the head's while the MFMAs wait
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = kSlabHead; s < kSlab; ++s) b[s] = buffer_load16_stream(wr, (wave + s * W) * 1024 + lane * 16);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();

    // 4. MFMAs with A from LDS (lanes of rows >= MM read row 0: discarded outputs)
    const int8_t* xrow = xs + ((lane & 15) < MM ? (lane & 15) : 0) * ldx + (lane >> 4) * 16;
    v4i acc = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < kSlab; ++s)
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(*(const v4i*)(xrow + (wave + s * W) * 64), b[s], acc, 0, 0, 0);
    if (reduce_waves(acc, red, W) && n < N && (lane >> 4) == 0) {
#pragma unroll
        for (int r = 0; r < MM; ++r)
            if (r < M) store_y(a.out, a.out_dtype, (int64_t)r * N + n, acc[r], sx[r], swn, a.bias, bn);
    }
}

extern "C" __global__ __launch_bounds__(512) void nh_linear_decode_w8a8_m1_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t xs[];  // [MM][W * 1024 + 16] codes
    linear_decode<1>(a, xs);
}

extern "C" __global__ __launch_bounds__(512) void nh_linear_decode_w8a8_m2_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t xs[];
    linear_decode<2>(a, xs);
}

extern "C" __global__ __launch_bounds__(512) void nh_linear_decode_w8a8_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t xs[];
    linear_decode<4>(a, xs);
}

// G2: W8A32 dequant GEMV.  The reference's quantized-weight path materialises
// W' = (float)q * s in f32 and accumulates x * W' in f64 (linear.rs:126-131,
// gemm.rs:99-109); this kernel does the same arithmetic per element (f32
// multiply, exact f64 product, f64 sum) in a different summation order, so
// it agrees with that path to a few f64 ulps before the final f32 rounding.
// grid = (N tiles, ceil(M / 4)): a workgroup owns 16 weight rows and 4
// activation rows; lane (r, g) dequantizes 16 weights of row r per K tile
// and the f64 partial sums meet through shuffles and LDS.
extern "C" __global__ __launch_bounds__(512) void nh_gemv_w8a32_kernel(GemvW8A32Args a) {
    __shared__ double redd[8][4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = a.waves;
    const int r16 = lane & 15, g = lane >> 4;
    const int M = a.M, N = a.N, K = a.K, kt = a.kt;
    const int tile = blockIdx.x, m0 = blockIdx.y * 4;
    const __amdgpu_buffer_rsrc_t wr = row_tile_rsrc(a.wq, tile, kt);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)M * (uint32_t)K * 4u);
    const int n = tile * 16 + r16;
    const float s = n < N ? a.sw[n] : 0.0f;
    const int steps = (kt + W - 1) / W;
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (int s0 = 0; s0 < steps; s0 += kSlab) {
        v4i b[kSlab];
        __builtin_amdgcn_sched_barrier(0);
        load_slab(b, wr, wave + s0 * W, W, lane);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int st = 0; st < kSlab; ++st) {
            const int k = (wave + (s0 + st) * W) * 64 + g * 16;
            if (k >= K) continue;
            float wv[16];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) wv[4 * j + e] = (float)(int8_t)(b[st][j] >> (8 * e)) * s;
#pragma unroll
            for (int mm = 0; mm < 4; ++mm) {
                const int m = m0 + mm;
                if (m >= M) break;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const v4i xx = buffer_load16(xr, (m * K + k + 4 * q) * 4);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        // the f64 product of two f32 values is exact, so the fused
                        // form rounds exactly like the reference's acc += a * b
                        acc[mm] = __builtin_fma((double)f32_from_bits((uint32_t)xx[e]), (double)wv[4 * q + e], acc[mm]);
                }
            }
        }
    }
    // the 4 lanes of a row (g = 0..3), then the waves
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
        acc[mm] += __shfl_xor(acc[mm], 16, kWave);
        acc[mm] += __shfl_xor(acc[mm], 32, kWave);
        redd[wave][mm][lane] = acc[mm];
    }
    __syncthreads();
    if (wave == 0 && g == 0 && n < N) {
#pragma unroll
        for (int mm = 0; mm < 4; ++mm) {
            const int m = m0 + mm;
            if (m >= M) break;
            double t = redd[0][mm][lane];
            for (int w = 1; w < W; ++w) t += redd[w][mm][lane];
            a.y[(int64_t)m * N + n] = (float)t;
        }
    }
}
