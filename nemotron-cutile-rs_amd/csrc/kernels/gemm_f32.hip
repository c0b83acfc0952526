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
    // operands widened to f64 once, as they are staged (each value is read by
    // 16 lanes), so the K loop is loads and fused multiply-adds only
    __shared__ __align__(16) double As[16][64 + 2];
    __shared__ __align__(16) double Bs[16][64 + 2];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int64_t M = a.M, K = a.K, N = a.N;
    const int64_t m0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
    double acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;
    // one K step's values of this thread, loaded a step ahead of their use
    float ra[4], rb[4];
    auto fetch = [&](int64_t k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = threadIdx.x + 256 * i;
            const int r = idx >> 4, kk = idx & 15;
            const int64_t gm = m0 + r, gk = k0 + kk;
            float v = 0.0f;
            if (gm < M && gk < K)
                v = a.lhs_bf16 ? f32_from_bits((uint32_t)((const uint16_t*)a.lhs)[gm * K + gk] << 16)
                               : ((const float*)a.lhs)[gm * K + gk];
            ra[i] = v;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = threadIdx.x + 256 * i;
            const int kk = idx >> 6, c = idx & 63;
            const int64_t gk = k0 + kk, gn = n0 + c;
            rb[i] = (gk < K && gn < N) ? a.rhs[gk * N + gn] : 0.0f;
        }
    };
    fetch(0);
    for (int64_t k0 = 0; k0 < K; k0 += 16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = threadIdx.x + 256 * i;
            As[idx & 15][idx >> 4] = (double)ra[i];
            Bs[idx >> 6][idx & 63] = (double)rb[i];
        }
        __syncthreads();
        if (k0 + 16 < K) fetch(k0 + 16);  // uniform
        const int kmax = (int)(K - k0 < 16 ? K - k0 : 16);
        for (int kk = 0; kk < kmax; ++kk) {
            const double2 a01 = *(const double2*)&As[kk][ty * 4], a23 = *(const double2*)&As[kk][ty * 4 + 2];
            const double2 b01 = *(const double2*)&Bs[kk][tx * 4], b23 = *(const double2*)&Bs[kk][tx * 4 + 2];
            const double ad[4] = {a01.x, a01.y, a23.x, a23.y};
            const double bd[4] = {b01.x, b01.y, b23.x, b23.y};
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

// The same product for outputs too few to fill the CUs with 64 x 64 tiles
// (the MoE router: 512 tokens x 128 experts are 16 such tiles): one output per
// lane, so every SIMD runs a wave of independent k-ordered chains.  A wave
// owns one lhs row and 64 consecutive columns, a workgroup four rows.
//
// Neither operand is widened to f64 once per use.  The rhs block of 64 k x 64
// columns is widened once per workgroup while it is staged and kept in LDS as
// f64 [column][k] (a lane reads two k of its column per 16-byte load).  The row's values are the same
// for the whole wave: lane j of every 16-lane row holds the f64 of column
// k0 + 16 b + j (b = 0..3, one widening per 16 k), and each fused multiply-add
// takes its lhs operand from a row broadcast (DPP row_newbcast) of lane j.
// The next block's rhs and lhs loads are in flight while the current one is
// consumed.  Same arithmetic and order as nh_gemm_f32_kernel: every output
// sees exactly K fused multiply-adds, k ascending.
namespace {

constexpr int kNarrowK = 64;

template <int J>
__device__ __forceinline__ double row_bcast(double v) {
    return __builtin_amdgcn_mov_dpp(v, 0x150 + J, 0xf, 0xf, true);  // row_newbcast:J
}

template <bool kBf16>
__device__ __forceinline__ float lhs_value(const void* row, int64_t k) {
    if constexpr (kBf16)
        return f32_from_bits((uint32_t)((const uint16_t*)row)[k] << 16);
    else
        return ((const float*)row)[k];
}

// Sixteen k of the block: lhs from lane J of the row, rhs from registers.
template <int J>
__device__ __forceinline__ void narrow_16(double& acc, double av, const double2* bv) {
    if constexpr (J < 16) {
        acc = __builtin_fma(row_bcast<J>(av), bv[J / 2].x, acc);
        acc = __builtin_fma(row_bcast<J + 1>(av), bv[J / 2].y, acc);
        narrow_16<J + 2>(acc, av, bv);
    }
}

template <bool kBf16>
__device__ __forceinline__ double narrow_chain(const GemmF32Args& a, const void* row, double (*Bt)[kNarrowK + 2],
                                               int lane, int wave, int64_t n, bool row_ok, bool col_ok) {
    const int64_t K = a.K, N = a.N;
    const int j = lane & 15;
    float rb[16], ra[4];
    // The rhs rows [k0, k0 + 64) as one buffer resource: rows past K and
    // columns past N read as zeros without a branch per load.  The launch
    // keeps N below 64 x (CU count), so 64 rows of offsets fit in 31 bits.
    auto fetch = [&](int64_t k0) {
        const int64_t rows = K - k0 < kNarrowK ? K - k0 : kNarrowK;
        const auto rs = make_rsrc(a.rhs + k0 * N, (uint32_t)(rows * N * 4));
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int kr = 4 * (wave + 4 * i) + r;
                const int off = col_ok ? (kr * (int)N + (int)n) * 4 : kOutOfRange;
                rb[4 * i + r] = f32_from_bits(__builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
            }
        if (row_ok && rows == kNarrowK) {  // uniform; a partial block reads its row per k
#pragma unroll
            for (int b = 0; b < 4; ++b) ra[b] = lhs_value<kBf16>(row, k0 + 16 * b + j);
        }
    };
    double acc = 0.0;
    fetch(0);
    for (int64_t k0 = 0; k0 < K; k0 += kNarrowK) {
        __syncthreads();  // the previous block's reads are done
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            double* dst = &Bt[lane][4 * (wave + 4 * i)];
            *(double2*)dst = make_double2((double)rb[4 * i], (double)rb[4 * i + 1]);
            *(double2*)(dst + 2) = make_double2((double)rb[4 * i + 2], (double)rb[4 * i + 3]);
        }
        double av[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) av[b] = (double)ra[b];
        __syncthreads();
        if (k0 + kNarrowK < K) fetch(k0 + kNarrowK);  // uniform
        if (!row_ok) continue;                          // uniform: the wave only stages
        const double* bt = Bt[lane];
        if (K - k0 >= kNarrowK) {
            double2 bv[32];  // the whole block's column: reads issued ahead of the chain
#pragma unroll
            for (int i = 0; i < 32; ++i) bv[i] = *(const double2*)(bt + 2 * i);
#pragma unroll
            for (int b = 0; b < 4; ++b) narrow_16<0>(acc, av[b], bv + 8 * b);
        } else {
            const int kmax = (int)(K - k0);
            for (int kk = 0; kk < kmax; ++kk)
                acc = __builtin_fma((double)lhs_value<kBf16>(row, k0 + kk), bt[kk], acc);
        }
    }
    return acc;
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void nh_gemm_f32_small_kernel(GemmF32Args a) {
    __shared__ __align__(16) double Bt[64][kNarrowK + 2];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t m = (int64_t)blockIdx.y * 4 + wave, n = (int64_t)blockIdx.x * 64 + lane;
    const bool row_ok = m < a.M, col_ok = n < a.N;
    double acc;
    if (a.lhs_bf16)
        acc = narrow_chain<true>(a, (const uint16_t*)a.lhs + (row_ok ? m : 0) * a.K, Bt, lane, wave, n, row_ok, col_ok);
    else
        acc = narrow_chain<false>(a, (const float*)a.lhs + (row_ok ? m : 0) * a.K, Bt, lane, wave, n, row_ok, col_ok);
    if (row_ok && col_ok) a.out[m * a.N + n] = a.bias ? (float)acc + a.bias[n] : (float)acc;
}
