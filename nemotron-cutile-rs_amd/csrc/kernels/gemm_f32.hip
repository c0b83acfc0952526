// G0d: the reference's device f32 GEMM (gemm.rs:318-363) restated for gfx950.
// out[m][n] = sum_k lhs[m][k] * rhs[k][n] with lhs [M][K] and rhs [K][N]
// row-major f32, accumulated in f64 with k ascending for every output, then
// rounded to f32: the arithmetic and order of gemm_into_host (gemm.rs:99-109).
// Each f32 x f32 product is exact in f64, so the fused multiply-add rounds
// exactly like the reference's `acc += lhs as f64 * rhs as f64`, and the
// device result equals the host path bit for bit (no tolerance needed).
//
// A workgroup of 256 threads owns a 64 x 64 output tile, each thread a 4 x 4
// block; K advances 16 at a time through LDS (A transposed to [k][m] so both
// operand reads are 16-byte vectors).  The last K step accumulates only the
// positions that exist, so every output sees exactly K fused multiply-adds.
//
// For the MoE router (moe.rs:185-188, a dense f32 LinearProjection) the lhs
// may be bf16 (widened exactly to f32 on load) and a bias may follow the
// rounding to f32, as project_into adds it (linear.rs:330-336).
#include "nh_device.h"

using namespace nh;

extern "C" __global__ __launch_bounds__(256) void nh_gemm_f32_kernel(GemmF32Args a) {
    __shared__ __align__(16) float As[16][64 + 4];
    __shared__ __align__(16) float Bs[16][64 + 4];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int64_t M = a.M, K = a.K, N = a.N;
    const int64_t m0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
    double acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;
    for (int64_t k0 = 0; k0 < K; k0 += 16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = threadIdx.x + 256 * i;
            const int r = idx >> 4, kk = idx & 15;
            const int64_t gm = m0 + r, gk = k0 + kk;
            float v = 0.0f;
            if (gm < M && gk < K)
                v = a.lhs_bf16 ? f32_from_bits((uint32_t)((const uint16_t*)a.lhs)[gm * K + gk] << 16)
                               : ((const float*)a.lhs)[gm * K + gk];
            As[kk][r] = v;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = threadIdx.x + 256 * i;
            const int kk = idx >> 6, c = idx & 63;
            const int64_t gk = k0 + kk, gn = n0 + c;
            Bs[kk][c] = (gk < K && gn < N) ? a.rhs[gk * N + gn] : 0.0f;
        }
        __syncthreads();
        const int kmax = (int)(K - k0 < 16 ? K - k0 : 16);
        for (int kk = 0; kk < kmax; ++kk) {
            const float4 av = *(const float4*)&As[kk][ty * 4];
            const float4 bv = *(const float4*)&Bs[kk][tx * 4];
            const double ad[4] = {av.x, av.y, av.z, av.w};
            const double bd[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fma(ad[i], bd[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t gm = m0 + ty * 4 + i;
        if (gm >= M) break;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t gn = n0 + tx * 4 + j;
            if (gn < N) a.out[gm * N + gn] = a.bias ? (float)acc[i][j] + a.bias[gn] : (float)acc[i][j];
        }
    }
}
