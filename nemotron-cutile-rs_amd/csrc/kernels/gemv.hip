// G1 / decode unit / G2: the M <= 16 GEMV family.  These kernels stream the
// int8 weight matrix from HBM exactly once, so they are HBM-bound: the design
// goal is bytes in flight from the first cycle to the last.
//
// Layout: W is [N][K] int8 (K contiguous), one f32 scale per output row.
// A workgroup owns one 16-row N tile; its waves split K into slices of up to
// 1 KiB.  Each wave issues the loads of its whole [16 x 1 KiB] weight slab
// (16 buffer loads of 16 B per lane through one address register, 16 KiB per
// wave) before doing anything else, so the activation prologue and the MFMAs
// run while the slab is in flight.  The int32 partial tiles of the waves are
// summed through LDS and the epilogue y = ((float)acc * sx[m]) * sw[n]
// [+ bias[n]] is applied by wave 0.
//
// MFMA operand convention used throughout (16x16x64, int8):
//   lane l supplies row (l % 16) of its operand and bytes [16*(l/16), +16)
//   of the current 64-wide K step; the same convention for A and B makes the
//   dot product independent of how the hardware orders K inside a lane.
//   Result: lane l holds D[m = 4*(l/16) + r][n = l % 16] in register r.
//
// Weight fragments are never masked: a K position past the wave's slice
// meets a zeroed activation fragment, and a row past N reads zeros from the
// buffer resource and only feeds output columns that are not stored.
#include "nh_device.h"

using namespace nh;

namespace {

constexpr int kSteps = 16;  // 64-byte K steps per wave slab: 1 KiB of K

// Buffer resource over the 16 weight rows of `tile` (rows past N read zeros).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const int8_t* wq, int tile, int N, int K) {
    const int rows = min(16, N - tile * 16);
    return make_rsrc(wq + (int64_t)tile * 16 * K, (uint32_t)rows * (uint32_t)K);
}

// The 16 loads of one slab: lane offset `off` (row r16, byte g*16 of the
// step) plus 64 * s.  Scheduling barriers around the call keep every load
// issued before the first wait (the default schedule sinks them two deep).
__device__ __forceinline__ void load_slab(v4i (&b)[kSteps], __amdgpu_buffer_rsrc_t r, int off) {
#pragma unroll
    for (int s = 0; s < kSteps; ++s) b[s] = buffer_load16(r, off + s * 64);
}

__device__ __forceinline__ v4i zero_unless(bool ok, v4i v) { return ok ? v : v4i{0, 0, 0, 0}; }

// Sum the partial tiles held by the waves of this workgroup and write the
// epilogue for the 16 x 16 tile.  `red` holds blockDim/64 * 64 v4i.
__device__ __forceinline__ void reduce_and_store(v4i acc, v4i* red, int tile, int M, int N, const float* sx,
                                                 const float* sw, const float* bias, void* out, int out_dtype) {
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
}

}  // namespace

// G1: quantized activations already in HBM (xq, sx); A fragments come from
// L2 (xq is at most 16 x K bytes and shared by every workgroup).
extern "C" __global__ __launch_bounds__(512) void nh_gemv_w8a8_kernel(GemvW8A8Args a) {
    __shared__ v4i red[8 * 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int M = a.M, N = a.N, K = a.K;
    const int tile = blockIdx.x;
    const int kbeg = wave * a.kslice;
    const int kend = min(K, kbeg + a.kslice);
    const __amdgpu_buffer_rsrc_t wr = tile_rsrc(a.wq, tile, N, K);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.xq, (uint32_t)M * (uint32_t)K);  // rows >= M read zeros
    const int lane_off = r16 * K + g * 16;
    v4i acc = {0, 0, 0, 0};
    for (int k0 = kbeg; k0 < kend; k0 += 64 * kSteps) {
        v4i b[kSteps], x[kSteps];
        __builtin_amdgcn_sched_barrier(0);
        load_slab(x, xr, lane_off + k0);  // activation fragments (L2) first
        load_slab(b, wr, lane_off + k0);  // then the weight slab (HBM)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const v4i xa = zero_unless(k0 + s * 64 + g * 16 < kend, x[s]);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, b[s], acc, 0, 0, 0);
        }
    }
    reduce_and_store(acc, red, tile, M, N, a.sx, a.sw, a.bias, a.out, a.out_dtype);
}

// Decode unit, M <= MM <= 4: per-token quantization of the bf16 activation
// rows (Q2) fused in front of the GEMV.  Every workgroup quantizes the rows
// into LDS itself while its weight slab is in flight, so the unit is one
// launch and the int8 activations never round-trip through HBM.  Codes and
// scales are bit-identical in every workgroup (quantize_i8_rcp is exactly
// quantize_i8); workgroup 0 also writes them out when asked.
template <int MM>
__device__ __forceinline__ void linear_decode(const LinearDecodeArgs& a, int8_t* xs) {
    __shared__ v4i red[8 * 64];
    __shared__ float redf[8][MM];
    __shared__ float srow[MM];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int M = a.M, N = a.N, K = a.K;
    const int ldx = K + 16;
    const int tile = blockIdx.x;
    const int kbeg = wave * a.kslice;
    const int kend = min(K, kbeg + a.kslice);
    const __amdgpu_buffer_rsrc_t wr = tile_rsrc(a.wq, tile, N, K);
    const int lane_off = r16 * K + g * 16;

    // 1. this thread's share of the M bf16 rows (8 values per 16-byte load,
    //    2 loads per row: K <= 16 * blockDim) goes into registers, then the
    //    weight slab goes in flight.  Loads complete in issue order, so the
    //    prologue waits only for the activations.
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, (uint32_t)M * (uint32_t)K * 2u);
    v4i xr[MM][2];
    v4i b[kSteps];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int v = 0; v < 2; ++v) xr[m][v] = buffer_load16(xrs, (m * K + (threadIdx.x + v * blockDim.x) * 8) * 2);
    load_slab(b, wr, lane_off + kbeg);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int v = 0; v < 2; ++v) xr[m][v] = zero_unless((int)((threadIdx.x + v * blockDim.x) * 8) < K, xr[m][v]);

    // 2. Q2 of the rows into LDS: row absmax, then codes
    float amax[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        amax[m] = 0.0f;
#pragma unroll
        for (int v = 0; v < 2; ++v)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t w = (uint32_t)xr[m][v][j];
                amax[m] = fmaxf(amax[m], fabsf(f32_from_bits(w << 16)));
                amax[m] = fmaxf(amax[m], fabsf(f32_from_bits(w & 0xffff0000u)));
            }
        const float wm = wave_max(amax[m]);
        if (lane == 0) redf[wave][m] = wm;
    }
    __syncthreads();
    if (threadIdx.x < M) {
        float r = redf[0][threadIdx.x];
        for (int i = 1; i < nw; ++i) r = fmaxf(r, redf[i][threadIdx.x]);
        const float s = scale_from_amax(r);
        srow[threadIdx.x] = s;
        if (blockIdx.x == 0 && a.sx_out) a.sx_out[threadIdx.x] = s;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        if (m < M) {
            const float s = srow[m];
            const float rcp = 1.0f / s;
#pragma unroll
            for (int v = 0; v < 2; ++v) {
                const int c = (threadIdx.x + v * blockDim.x) * 8;
                if (c < K) {
                    uint32_t code[2] = {0, 0};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t w = (uint32_t)xr[m][v][j];
                        const uint32_t q0 = (uint8_t)quantize_i8_rcp(f32_from_bits(w << 16), s, rcp);
                        const uint32_t q1 = (uint8_t)quantize_i8_rcp(f32_from_bits(w & 0xffff0000u), s, rcp);
                        code[j >> 1] |= (q0 | (q1 << 8)) << (16 * (j & 1));
                    }
                    *(uint2*)(xs + m * ldx + c) = make_uint2(code[0], code[1]);
                    if (blockIdx.x == 0 && a.xq_out)
                        *(uint2*)(a.xq_out + (int64_t)m * K + c) = make_uint2(code[0], code[1]);
                }
            }
        }
    }
    __syncthreads();

    // 3. MFMAs with A from LDS; further slabs only when a wave owns > 1 KiB of K
    const int8_t* xrow = xs + (r16 < M ? r16 : 0) * ldx;  // rows >= M feed discarded outputs
    v4i acc = {0, 0, 0, 0};
    if (kend - kbeg == 64 * kSteps) {  // one full slab (the common case): no K tail to mask
#pragma unroll
        for (int s = 0; s < kSteps; ++s)
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(*(const v4i*)(xrow + kbeg + s * 64 + g * 16), b[s], acc, 0,
                                                        0, 0);
        reduce_and_store(acc, red, tile, M, N, srow, a.sw, a.bias, a.out, a.out_dtype);
        return;
    }
    for (int k0 = kbeg; k0 < kend; k0 += 64 * kSteps) {
        if (k0 != kbeg) {
            __builtin_amdgcn_sched_barrier(0);
            load_slab(b, wr, lane_off + k0);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const int k = k0 + s * 64 + g * 16;
            const v4i x = zero_unless(k < kend, *(const v4i*)(xrow + (k < kend ? k : k0)));
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x, b[s], acc, 0, 0, 0);
        }
    }
    reduce_and_store(acc, red, tile, M, N, srow, a.sw, a.bias, a.out, a.out_dtype);
}

extern "C" __global__ __launch_bounds__(512) void nh_linear_decode_w8a8_m1_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t xs[];  // [M][K + 16] codes
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
                const v4i w4 = *(const v4i*)(wrow + k);
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
