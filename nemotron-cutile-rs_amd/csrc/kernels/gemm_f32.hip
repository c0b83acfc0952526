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
#include <type_traits>

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

// The same product on the f64 matrix cores, for outputs too few to fill the
// CUs with 64 x 64 tiles (the MoE router: 512 tokens x 128 experts are 16 such
// tiles).  v_mfma_f64_4x4x4f64 computes, for each of its 64 outputs, four
// fused multiply-adds in k order onto the accumulator: on the device every
// output equals the chain fma(a3, b3, fma(a2, b2, fma(a1, b1, fma(a0, b0,
// c)))) bit for bit (12,800 outputs of random-exponent operands; the reversed
// order matched 61% of them), so a chain of these MFMAs is the reference's
// f64 accumulation in k order.  Operand roles (read off one-hot probes): A
// lane 16 k + 4 b + i holds A[i][k] of block b, B lane 16 k + 4 b + j holds
// B[k][j] of block b, D lane 16 i + 4 b + j holds D[i][j] of block b: four
// 4 x 4 blocks per wave.
//
// A workgroup of 4 waves owns 16 x 16 outputs: wave w the rows 4w..4w+3 and,
// as its blocks b, the columns 4b..4b+3.  K advances in chunks of 128 through
// LDS (f32, widened as an operand is read; double buffered, the loads of the
// next two chunks in flight while the current one runs).  A chunk's operands
// are read into registers before its chain, so the LDS latency is paid once
// per chunk.  k past K, rows past M and columns past N are zeros: an added
// fma(0, 0, acc) leaves acc unchanged, as acc starts at +0.0 and a k-ordered
// sum of products that starts there is never -0.0.  One chain of 64 outputs
// per wave takes ~21 cycles per 4-k step (the MFMA's dependent latency; its
// issue rate is one per 16 cycles), against ~40 cycles per single k step for
// a lane-per-output FMA chain.
//
// Loads go through buffer resources over the whole operands (wave-uniform;
// the launch keeps both below 2^31 bytes), positions past the matrix sent out
// of range so they read zeros with no branch, and every fetch issues the same
// loads, so the waits before a chunk is staged count exactly the younger
// fetch's loads.  VEC (16-byte aligned operands, K a multiple of 8 for bf16 or
// 4 for f32, N a multiple of 4): 16-byte loads, 3 or 4 per thread and chunk;
// otherwise one load per value.
namespace {

template <bool BF16, bool VEC>
__device__ __forceinline__ void gemm_f32_mfma(const GemmF32Args& a) {
    constexpr int KC = 128;
    __shared__ float As[2][16][KC + 4];  // [row][k]; the pad puts the 16 rows of a read on distinct banks
    __shared__ float Bs[2][KC][16];      // [k][column]
    const int t = threadIdx.x, lane = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int64_t M = a.M, K = a.K, N = a.N;
    const int64_t tiles_n = (N + 15) / 16;
    const int64_t m0 = (int64_t)(blockIdx.x / tiles_n) * 16, n0 = (int64_t)(blockIdx.x % tiles_n) * 16;
    // staging roles: A row t / 16, k (t % 16) * 8 .. + 7; B k-rows t / 4 and
    // t / 4 + 64, columns (t % 4) * 4 .. + 3
    const int64_t am = m0 + (t >> 4), ak = (t & 15) * 8, bk = t >> 2, bn = n0 + (t & 3) * 4;
    constexpr uint32_t esz = BF16 ? 2u : 4u;
    const __amdgpu_buffer_rsrc_t rA = make_rsrc(a.lhs, (uint32_t)(M * K * esz));
    const __amdgpu_buffer_rsrc_t rB = make_rsrc(a.rhs, (uint32_t)(K * N * 4));
    const uint32_t oor = (uint32_t)kOutOfRange;
    float ra[2][8], rb[2][8];  // chunks c + 1 and c + 2 in flight
    auto fetch = [&](int64_t k0, float (&ra)[8], float (&rb)[8]) {
        const int64_t gk = k0 + ak;
        const uint32_t abase = (uint32_t)((am * K + gk) * esz);
        if constexpr (VEC && BF16) {
            const v4i v = buffer_load16(rA, am < M && gk < K ? abase : oor);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                ra[2 * e] = f32_from_bits((uint32_t)v[e] << 16);
                ra[2 * e + 1] = f32_from_bits((uint32_t)v[e] & 0xffff0000u);
            }
        } else if constexpr (VEC) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const v4i v = buffer_load16(rA, am < M && gk + 4 * h < K ? abase + 16u * h : oor);
#pragma unroll
                for (int e = 0; e < 4; ++e) ra[4 * h + e] = f32_from_bits((uint32_t)v[e]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t off = am < M && gk + e < K ? abase + esz * e : oor;
                ra[e] = BF16 ? f32_from_bits((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rA, off, 0, 0) << 16)
                             : f32_from_bits(__builtin_amdgcn_raw_buffer_load_b32(rA, off, 0, 0));
            }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t gkb = k0 + bk + 64 * h;
            const uint32_t bbase = (uint32_t)((gkb * N + bn) * 4);
            if constexpr (VEC) {
                const v4i v = buffer_load16(rB, gkb < K && bn < N ? bbase : oor);
#pragma unroll
                for (int e = 0; e < 4; ++e) rb[4 * h + e] = f32_from_bits((uint32_t)v[e]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    rb[4 * h + e] = f32_from_bits(
                        __builtin_amdgcn_raw_buffer_load_b32(rB, gkb < K && bn + e < N ? bbase + 4u * e : oor, 0, 0));
            }
        }
    };
    // MFMA operand roles of this lane
    const int rk = lane >> 4, arow = 4 * w + (lane & 3), bcol = 4 * ((lane >> 2) & 3) + (lane & 3);
    double acc = 0.0;
    // chunk at k0 from LDS buffer B (a constant, so the register sets are
    // not indexed at run time)
    auto chunk = [&](int64_t k0, auto bufc) {
        constexpr int B = decltype(bufc)::value;
#pragma unroll
        for (int e = 0; e < 8; ++e) As[B][t >> 4][ak + e] = ra[B][e];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) Bs[B][bk + 64 * h][(t & 3) * 4 + e] = rb[B][4 * h + e];
        __syncthreads();
        if (k0 + 2 * KC < K) fetch(k0 + 2 * KC, ra[B], rb[B]);  // uniform
        float av[KC / 4], bv[KC / 4];
#pragma unroll
        for (int st = 0; st < KC / 4; ++st) {
            av[st] = As[B][arow][4 * st + rk];
            bv[st] = Bs[B][4 * st + rk][bcol];
        }
        __builtin_amdgcn_sched_barrier(0);  // the reads go out ahead of the chain
#pragma unroll
        for (int st = 0; st < KC / 4; ++st)
            acc = __builtin_amdgcn_mfma_f64_4x4x4f64((double)av[st], (double)bv[st], acc, 0, 0, 0);
    };
    fetch(0, ra[0], rb[0]);
    if (KC < K) fetch(KC, ra[1], rb[1]);
    for (int64_t k0 = 0; k0 < K; k0 += 2 * KC) {
        chunk(k0, std::integral_constant<int, 0>{});
        if (k0 + KC < K) chunk(k0 + KC, std::integral_constant<int, 1>{});  // uniform
    }
    // D lane 16 i + 4 b + j: output (4w + i, 4b + j)
    const int64_t gm = m0 + 4 * w + (lane >> 4), gn = n0 + 4 * ((lane >> 2) & 3) + (lane & 3);
    if (gm < M && gn < N) a.out[gm * N + gn] = a.bias ? (float)acc + a.bias[gn] : (float)acc;
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void nh_gemm_f32_mfma_kernel(GemmF32Args a) {
    gemm_f32_mfma<false, true>(a);
}

extern "C" __global__ __launch_bounds__(256) void nh_gemm_f32_mfma_bf16_kernel(GemmF32Args a) {
    gemm_f32_mfma<true, true>(a);
}

// Any alignment, K and N: one load per value.
extern "C" __global__ __launch_bounds__(256) void nh_gemm_f32_mfma_any_kernel(GemmF32Args a) {
    if (a.lhs_bf16)
        gemm_f32_mfma<true, false>(a);
    else
        gemm_f32_mfma<false, false>(a);
}
