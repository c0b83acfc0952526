// G3: W8A8 GEMM for prefill-sized M on int8 MFMA (v_mfma_i32_32x32x32_i8).
// Weights (B) are in the tiled layout (nh_numerics.h); activations (A) are
// row-major [M][K].
//
// Workgroup = 256 threads = 4 waves in a 2 x 2 grid over a BM x BN output
// tile.  K advances in 128-byte steps; A (activations, [M][K]) and B (weights,
// [N][K]) tiles are staged through LDS with a 144-byte row pitch (9 x 16 B:
// eight consecutive rows read by a ds_read_b128 land in distinct banks) and
// double-buffered: the global loads of step t+1 are in flight while the MFMAs
// of step t run.  The fused epilogue applies the per-token and per-channel
// scales (+bias, +ReLU^2) and writes f32 or bf16.
//
// 32x32x32 int8 MFMA operand convention: lane l supplies row (l % 32) of its
// operand and bytes [16*(l/32), +16) of the current 32-byte K step (same
// convention for A and B).  Result: lane l, register r holds
// D[m = 8*(r/4) + 4*(l/32) + (r%4)][n = l % 32].
//
// blockIdx -> tile mapping is XCD-aware: workgroups are dealt round-robin to
// the 8 XCDs, so consecutive ids are re-packed to make each XCD own a
// contiguous range of tiles (column-major: neighbours share B columns and
// the A panel), which keeps both panels in that XCD's L2.
#include "nh_device.h"

using namespace nh;

namespace {

constexpr int kBK = 128;            // bytes of K per pipeline step
constexpr int kPitch = kBK + 16;    // LDS row pitch
constexpr int kThreads = 256;

template <int BM, int BN>
__device__ __forceinline__ void gemm_tile(const GemmW8A8Args& a, int8_t* smem) {
    constexpr int WM = BM / 2, WN = BN / 2;       // per-wave tile
    constexpr int TM = WM / 32, TN = WN / 32;     // 32x32 MFMA tiles per wave
    constexpr int CA = BM * kBK / 16 / kThreads;  // 16-byte chunks per thread (A)
    constexpr int CB = BN * kBK / 16 / kThreads;  // (B)
    constexpr int kStage = (BM + BN) * kPitch;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int M = a.M, N = a.N, K = a.K;

    // XCD-aware tile id
    const int nblk = a.tiles_m * a.tiles_n;
    int b = blockIdx.x;
    if ((nblk & 7) == 0) b = (b & 7) * (nblk >> 3) + (b >> 3);
    const int tm_idx = b % a.tiles_m, tn_idx = b / a.tiles_m;
    const int m0 = tm_idx * BM, n0 = tn_idx * BN;

    // global -> register staging
    v4i ga[CA], gb[CB];
    auto load_stage = [&](int k0) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int c = tid + i * kThreads;
            const int row = c >> 3, col = (c & 7) * 16;
            const int gm = m0 + row, gk = k0 + col;
            ga[i] = (gm < M && gk < K) ? *(const v4i*)(a.xq + (int64_t)gm * K + gk) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int c = tid + i * kThreads;
            const int row = c >> 3, col = (c & 7) * 16;
            const int gn = n0 + row, gk = k0 + col;
            gb[i] = (gn < N && gk < K) ? *(const v4i*)(a.wq + tiled_offset(gn, gk, a.kt)) : v4i{0, 0, 0, 0};
        }
    };
    auto store_stage = [&](int buf) {
        int8_t* sa = smem + buf * kStage;
        int8_t* sb = sa + BM * kPitch;
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int c = tid + i * kThreads;
            *(v4i*)(sa + (c >> 3) * kPitch + (c & 7) * 16) = ga[i];
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int c = tid + i * kThreads;
            *(v4i*)(sb + (c >> 3) * kPitch + (c & 7) * 16) = gb[i];
        }
    };

    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = v16i{};

    const int nk = (K + kBK - 1) / kBK;
    load_stage(0);
    store_stage(0);
    __syncthreads();
    const int fr = lane & 31, fk = (lane >> 5) * 16;
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load_stage((kt + 1) * kBK);
        const int8_t* sa = smem + buf * kStage + (wm * WM + fr) * kPitch + fk;
        const int8_t* sb = smem + buf * kStage + BM * kPitch + (wn * WN + fr) * kPitch + fk;
#pragma unroll
        for (int ks = 0; ks < kBK; ks += 32) {
            v4i af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) af[i] = *(const v4i*)(sa + i * 32 * kPitch + ks);
#pragma unroll
            for (int j = 0; j < TN; ++j) bf[j] = *(const v4i*)(sb + j * 32 * kPitch + ks);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store_stage(buf ^ 1);
        __syncthreads();
    }

    // fused epilogue
    const int quad = lane >> 5;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = n0 + wn * WN + j * 32 + (lane & 31);
        if (n >= N) continue;
        const float swn = a.sw[n];
        const float bn = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * quad + (r & 3);
                if (m < M) {
                    float y = epilogue_w8a8(acc[i][j][r], a.sx[m], swn);
                    if (a.bias) y = y + bn;
                    if (a.relu2) y = relu2(y);
                    store_out(a.out, (int64_t)m * N + n, y, a.out_dtype);
                }
            }
        }
    }
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void nh_gemm_w8a8_kernel(GemmW8A8Args a) {
    extern __shared__ __align__(16) int8_t smem[];
    gemm_tile<256, 128>(a, smem);
}

extern "C" __global__ __launch_bounds__(256) void nh_gemm_w8a8_128x128_kernel(GemmW8A8Args a) {
    extern __shared__ __align__(16) int8_t smem[];
    gemm_tile<128, 128>(a, smem);
}
