// G1 / decode unit / G2: the M <= 16 GEMV family.  These kernels stream the
// int8 weight matrix from HBM exactly once, so they are HBM-bound: the design
// goal is bytes in flight, not arithmetic.
//
// Layout: W is [N][K] int8 (K contiguous), one f32 scale per output row.
// A workgroup owns one 16-row N tile; its ksplit waves split K, each wave
// streams its [16 x kslice] slab with 16-byte loads and feeds
// v_mfma_i32_16x16x64_i8 (A = activation rows, B = weight rows).  The int32
// partial tiles of the waves are summed through LDS and the epilogue
// y = ((float)acc * sx[m]) * sw[n] [+ bias[n]] is applied by wave 0.
//
// MFMA operand convention used throughout (16x16x64, int8):
//   lane l supplies row (l % 16) of its operand and bytes [16*(l/16), +16)
//   of the current 64-wide K step; the same convention for A and B makes the
//   dot product independent of how the hardware orders K inside a lane.
//   Result: lane l holds D[m = 4*(l/16) + r][n = l % 16] in register r.
#include "nh_device.h"

using namespace nh;

namespace {

constexpr int kChunk = 8;  // K steps (64 bytes each) per batch of loads

__device__ __forceinline__ v4i load16(const int8_t* p) { return *(const v4i*)p; }

// Sum the ksplit partial tiles held by the waves of this workgroup and write
// the epilogue for the 16 x 16 tile.  `red` holds blockDim/64 * 64 v4i.
__device__ __forceinline__ void reduce_and_store(v4i acc, v4i* red, int tile, int M, int N,
                                                 const float* sx, const float* sw, const float* bias,
                                                 void* out, int out_dtype) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (nw > 1) {
        red[wave * 64 + lane] = acc;
        __syncthreads();
        if (wave == 0) {
            for (int w = 1; w < nw; ++w) acc += red[w * 64 + lane];
        }
    }
    if (wave == 0) {
        const int n = tile * 16 + (lane & 15);
        if (n < N) {
            const float swn = sw[n];
            const float bn = bias ? bias[n] : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 4 * (lane >> 4) + r;
                if (m < M) {
                    float y = epilogue_w8a8(acc[r], sx[m], swn);
                    if (bias) y = y + bn;
                    store_out(out, (int64_t)m * N + n, y, out_dtype);
                }
            }
        }
    }
    if (nw > 1) __syncthreads();
}

}  // namespace

// G1: quantized activations already in HBM (xq, sx).
extern "C" __global__ __launch_bounds__(1024) void nh_gemv_w8a8_kernel(GemvW8A8Args a) {
    __shared__ v4i red[16 * 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int M = a.M, N = a.N, K = a.K;
    const int kbeg = wave * a.kslice;
    const int kend = min(K, kbeg + a.kslice);
    const bool mok = r16 < M;
    const int8_t* xrow = a.xq + (int64_t)(mok ? r16 : 0) * K;
    for (int tile = blockIdx.x; tile < a.ntiles; tile += gridDim.x) {
        const int n = tile * 16 + r16;
        const bool nok = n < N;
        const int8_t* wrow = a.wq + (int64_t)(nok ? n : 0) * K;
        v4i acc = {0, 0, 0, 0};
        for (int k0 = kbeg; k0 < kend; k0 += 64 * kChunk) {
            v4i b[kChunk], x[kChunk];
#pragma unroll
            for (int s = 0; s < kChunk; ++s) {
                const int k = k0 + s * 64 + g * 16;
                const bool kok = k < kend;
                b[s] = (nok && kok) ? load16(wrow + k) : v4i{0, 0, 0, 0};
                x[s] = (mok && kok) ? load16(xrow + k) : v4i{0, 0, 0, 0};
            }
#pragma unroll
            for (int s = 0; s < kChunk; ++s) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x[s], b[s], acc, 0, 0, 0);
        }
        reduce_and_store(acc, red, tile, M, N, a.sx, a.sw, a.bias, a.out, a.out_dtype);
    }
}

// Decode unit: per-token quantization of the M activation rows (Q2) fused in
// front of the GEMV.  Every workgroup quantizes the rows into LDS (the rows
// are M*K <= 64 KiB, read from L2), so no second launch and no round trip of
// the int8 activations through HBM.  Codes and scales are bit-identical in
// every workgroup; workgroup 0 also writes them out when asked.
extern "C" __global__ __launch_bounds__(1024) void nh_linear_decode_w8a8_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t xs[];  // [M][K + 16] codes, then M floats of scale
    __shared__ v4i red[16 * 64];
    __shared__ float redf[16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int M = a.M, N = a.N, K = a.K;
    const int ldx = K + 16;
    float* sxs = (float*)(xs + (int64_t)M * ldx);

    // ---- Q2 into LDS: one row at a time, whole workgroup per row ----------
    for (int m = 0; m < M; ++m) {
        float amax = 0.0f;
        for (int c = threadIdx.x; c < K; c += blockDim.x) {
            const float v = load_as_f32(a.x, (int64_t)m * K + c, a.x_dtype);
            amax = fmaxf(amax, fabsf(v));
        }
        amax = wave_max(amax);
        if (lane == 0) redf[wave] = amax;
        __syncthreads();
        float rm = redf[0];
        for (int i = 1; i < nw; ++i) rm = fmaxf(rm, redf[i]);
        const float s = scale_from_amax(rm);
        for (int c = threadIdx.x; c < K; c += blockDim.x) {
            const float v = load_as_f32(a.x, (int64_t)m * K + c, a.x_dtype);
            const int8_t q = quantize_i8(v, s);
            xs[m * ldx + c] = q;
            if (blockIdx.x == 0 && a.xq_out) a.xq_out[(int64_t)m * K + c] = q;
        }
        if (threadIdx.x == 0) {
            sxs[m] = s;
            if (blockIdx.x == 0 && a.sx_out) a.sx_out[m] = s;
        }
        __syncthreads();
    }

    // ---- GEMV with A from LDS ----------------------------------------------
    const int kbeg = wave * a.kslice;
    const int kend = min(K, kbeg + a.kslice);
    const bool mok = r16 < M;
    const int8_t* xrow = xs + (mok ? r16 : 0) * ldx;
    for (int tile = blockIdx.x; tile < a.ntiles; tile += gridDim.x) {
        const int n = tile * 16 + r16;
        const bool nok = n < N;
        const int8_t* wrow = a.wq + (int64_t)(nok ? n : 0) * K;
        v4i acc = {0, 0, 0, 0};
        for (int k0 = kbeg; k0 < kend; k0 += 64 * kChunk) {
            v4i b[kChunk];
#pragma unroll
            for (int s = 0; s < kChunk; ++s) {
                const int k = k0 + s * 64 + g * 16;
                b[s] = (nok && k < kend) ? load16(wrow + k) : v4i{0, 0, 0, 0};
            }
#pragma unroll
            for (int s = 0; s < kChunk; ++s) {
                const int k = k0 + s * 64 + g * 16;
                const v4i x = (mok && k < kend) ? *(const v4i*)(xrow + k) : v4i{0, 0, 0, 0};
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x, b[s], acc, 0, 0, 0);
            }
        }
        reduce_and_store(acc, red, tile, M, N, sxs, a.sw, a.bias, a.out, a.out_dtype);
    }
}

// G2: W8A32 dequant GEMV.  The reference's quantized-weight path materialises
// W' = (float)q * s in f32 and accumulates x * W' in f64 (linear.rs:126-131,
// gemm.rs:99-109); this kernel does the same arithmetic per element (f32
// multiply, exact f64 product, f64 sum) in a different summation order, so
// it agrees with that path to a few f64 ulps before the final f32 rounding.
// One wave per weight row; lanes split K in 16-byte chunks (1 KiB per wave
// per load, fully coalesced).
extern "C" __global__ __launch_bounds__(256) void nh_gemv_w8a32_kernel(GemvW8A32Args a) {
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int K = a.K, N = a.N, M = a.M;
    const int nbeg = gw * a.rows_per_wave;
    const int nend = min(N, nbeg + a.rows_per_wave);
    for (int n = nbeg; n < nend; ++n) {
        const int8_t* wrow = a.wq + (int64_t)n * K;
        const float s = a.sw[n];
        for (int m = 0; m < M; ++m) {
            const float* x = a.x + (int64_t)m * K;
            double acc = 0.0;
            for (int k = lane * 16; k < K; k += 64 * 16) {
                const v4i w4 = load16(wrow + k);
                const float4* xv = (const float4*)(x + k);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float4 xx = xv[j];
                    const int word = w4[j];
                    const float xs[4] = {xx.x, xx.y, xx.z, xx.w};
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const float wv = (float)(int8_t)(word >> (8 * b)) * s;
                        // the f64 product of two f32 values is exact, so the fused
                        // form rounds exactly like the reference's acc += a * b
                        acc = __builtin_fma((double)xs[b], (double)wv, acc);
                    }
                }
            }
            acc = wave_sum_f64(acc);
            if (lane == 0) a.y[(int64_t)m * N + n] = (float)acc;
        }
    }
}
