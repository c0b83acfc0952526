// G3: W8A8 GEMM for prefill-sized M on int8 MFMA (v_mfma_i32_16x16x64_i8).
// Weights (B) are in the tiled layout (nh_numerics.h); activations (A) are
// row-major [M][K].
//
// A workgroup of WGM x WGN waves owns a BM x BN output tile.  Its operands
// stream through a ring of S stages in LDS, each 128 bytes of K, filled by
// direct-to-LDS buffer loads (buffer_load_dwordx4 ... lds: lane l writes its
// 16 bytes at M0 + 16 l), so staging costs no VGPRs and S - 1 stages stay in
// flight.  Per stage and wave: wait for this wave's loads of the stage
// (vmcnt), one barrier, refill the slot consumed in the previous iteration,
// then two MFMA K steps of 64 bytes.  The barrier is a bare s_barrier:
// __syncthreads' release fence would wait for every in-flight LDS load
// (vmcnt(0)) and serialize the ring.
//
// Operand layout in LDS:
//  * A: each load instruction covers 8 rows x 128 bytes, i.e. whole cache
//    lines (measured: 4x the L2->LDS throughput of 16 rows x 64 bytes).
//    Lane l writes LDS slot l % 8 of row l / 8 and picks which 16-byte chunk
//    of its row to fetch, so that chunk c of local row R lands in slot
//    c ^ (R % 8) ^ ((R / 8) % 2): the 16 rows of an MFMA fragment read then
//    cover all 64 banks.
//  * B: one 1 KiB tile of the tiled weights per instruction, already in the
//    MFMA operand order (fragment reads are linear ds_read_b128), with the
//    default cache policy: every weight tile is read again by the other M
//    tiles of its column, mostly on the same XCD.  (The streaming policy that
//    suits a single pass over the weights made the loads alone take 23.8
//    instead of 18.2 us at (2048, 4096, 4096), and the kernel 150.8 instead
//    of 145.3 us at K = 21504.)
//
// Epilogue: the MFMAs take the weight fragment first, so each lane's four
// accumulators are four consecutive columns of one output row; the per-token
// and per-channel scales (+bias, +ReLU^2) are applied in registers and the
// lane stores the four results as one 8-byte (bf16) or 16-byte (f32) write,
// with no LDS staging and no barrier after the main loop.
//
// blockIdx -> tile mapping is XCD-aware: workgroups are dealt round-robin to
// the 8 XCDs, so consecutive ids are re-packed to make each XCD own a
// contiguous range of tiles (column-major: neighbours share the A panel and
// B columns stay in that XCD's L2).
#include "nh_device.h"

using namespace nh;

namespace {

typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));


// The tile's per-token scales (BM floats), per-channel scales (BN) and, when
// given, bias (BN) into LDS at `sc`, in that order: direct-to-LDS dword loads,
// 64 values per instruction, issued by one wave ahead of its stage loads (so
// its first stage wait covers them and the first barrier publishes them).
// Rows and columns past the matrix read zeros (their results are not stored).
template <int BM, int BN>
__device__ __forceinline__ void issue_scale_loads(const GemmW8A8Args& a, int m0, int n0, int8_t* sc, int lane) {
    const uint32_t l4 = (uint32_t)lane * 4u;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.sx + m0, (uint32_t)(a.M - m0) * 4u);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.sw + n0, (uint32_t)(a.N - n0) * 4u);
#pragma unroll
    for (int q = 0; q < BM / 64; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_t*)(sc + q * 256), 4, q * 256 + l4, 0, 0, 0);
#pragma unroll
    for (int q = 0; q < BN / 64; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_void_t*)(sc + BM * 4 + q * 256), 4, q * 256 + l4, 0, 0, 0);
    if (a.bias) {
        const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.bias + n0, (uint32_t)(a.N - n0) * 4u);
#pragma unroll
        for (int q = 0; q < BN / 64; ++q)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_t*)(sc + (BM + BN) * 4 + q * 256), 4, q * 256 + l4,
                                                     0, 0, 0);
    }
}

// Epilogue of a wave's tile at local offset (lm0, ln0) of the workgroup tile
// (global m0 + lm0, n0 + ln0), straight from the accumulators.  The MFMAs take
// the weight fragment first, so lane l holds C[16 i + l % 16][16 j + 4 (l / 16)
// + r] of the wave tile in register r of acc[i][j]: four consecutive columns
// of one row.  y = ((float)acc * sx[m]) * sw[n] [+ bias][ReLU^2] (the numerics
// spec's two RN multiplies), with the scales and bias read from the LDS copy
// `sc` (issue_scale_loads); each lane stores its four results as 8 bytes
// (bf16, two v_cvt_pk_bf16_f32) or 16 (f32).
//
// The epilogue is VALU-bound (a wave64 VALU instruction takes 4 cycles, and
// all 256 x 128 results of a workgroup pass through the CU's four SIMDs at
// once at the end of a single-round launch), so the usual case, a wave tile
// inside the matrix with aligned rows, is straight code with no per-element
// or per-fragment check; bias and ReLU^2 are uniform branches.  Wave tiles at
// the matrix edge or with unaligned rows take a compact general loop that
// stores element by element where four columns do not fit.
template <int BM, int BN, int FM, int FN>
__device__ __forceinline__ void store_tile(const GemmW8A8Args& a, v4i (&acc)[FM][FN], const int8_t* sc, int m0,
                                           int n0, int lm0, int ln0, int lane) {
    const int M = a.M, N = a.N;
    const int64_t ldo = a.ldo;
    const int c4 = 4 * (lane >> 4);
    const bool bf = a.out_dtype == DT_BF16;
    const bool has_bias = a.bias != nullptr, has_relu2 = a.relu2 != 0;
    const int esz = bf ? 2 : 4;
    const bool aligned = ((((uint64_t)a.out) | ((uint64_t)ldo * esz)) & (uint64_t)(4 * esz - 1)) == 0;
    const float* sx = (const float*)sc;
    const float* sw = sx + BM;
    const float* sb = sw + BN;
    if (aligned && n0 + ln0 + FN * 16 <= N && m0 + lm0 + FM * 16 <= M) {
        int8_t* base = (int8_t*)a.out + ((int64_t)(m0 + lm0 + (lane & 15)) * ldo + n0 + ln0 + c4) * esz;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const float sxm = sx[lm0 + i * 16 + (lane & 15)];
            int8_t* row = base + (int64_t)i * 16 * ldo * esz;
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int ln = ln0 + j * 16 + c4;
                const v4f w = *(const v4f*)(sw + ln);
                float y[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) y[r] = epilogue_w8a8(acc[i][j][r], sxm, w[r]);
                if (has_bias) {
                    const v4f b = *(const v4f*)(sb + ln);
#pragma unroll
                    for (int r = 0; r < 4; ++r) y[r] = y[r] + b[r];
                }
                if (has_relu2) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) y[r] = relu2(y[r]);
                }
                if (bf)
                    *(v2u*)(row + j * 32) = v2u{f32x2_to_bf16x2(y[0], y[1]), f32x2_to_bf16x2(y[2], y[3])};
                else
                    *(v4f*)(row + j * 64) = v4f{y[0], y[1], y[2], y[3]};
            }
        }
        return;
    }
    // General form: fragments through loops that are not unrolled, each
    // iteration taking the first fragment and shifting the others up.
#pragma unroll 1
    for (int i = 0; i < FM; ++i) {
        v4i cur[FN];
#pragma unroll
        for (int j = 0; j < FN; ++j) cur[j] = acc[0][j];
#pragma unroll
        for (int k = 0; k + 1 < FM; ++k)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[k][j] = acc[k + 1][j];
        const int lm = lm0 + i * 16 + (lane & 15);
        const int m = m0 + lm;
        if (m >= M) break;  // rows grow with i
        const float sxm = sx[lm];
        int8_t* row = (int8_t*)a.out + (int64_t)m * ldo * esz;
#pragma unroll 1
        for (int j = 0; j < FN; ++j) {
            const v4i q = cur[0];
#pragma unroll
            for (int k = 0; k + 1 < FN; ++k) cur[k] = cur[k + 1];
            const int ln = ln0 + j * 16 + c4;
            const int c = n0 + ln;
            const v4f w = *(const v4f*)(sw + ln);
            const v4f b = has_bias ? *(const v4f*)(sb + ln) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
            float y[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = epilogue_w8a8(q[r], sxm, w[r]);
                if (has_bias) v = v + b[r];
                y[r] = has_relu2 ? relu2(v) : v;
            }
            if (aligned && c + 3 < N) {
                if (bf)
                    *(v2u*)(row + (int64_t)c * 2) = v2u{f32x2_to_bf16x2(y[0], y[1]), f32x2_to_bf16x2(y[2], y[3])};
                else
                    *(v4f*)(row + (int64_t)c * 4) = v4f{y[0], y[1], y[2], y[3]};
            } else {
                float y0 = y[0], y1 = y[1], y2 = y[2], y3 = y[3];
#pragma unroll 1
                for (int r = 0; r < 4; ++r) {
                    if (c + r < N) {
                        if (bf)
                            ((uint16_t*)row)[c + r] = f32_to_bf16(y0);
                        else
                            ((float*)row)[c + r] = y0;
                    }
                    y0 = y1;
                    y1 = y2;
                    y2 = y3;
                }
            }
        }
    }
}

__device__ __forceinline__ int a_slot(int row, int chunk) { return chunk ^ (row & 7) ^ ((row >> 3) & 1); }

template <int BM, int BN, int WGM, int WGN, int S>
__device__ __forceinline__ void gemm_tile(const GemmW8A8Args& a, int8_t* smem) {
    constexpr int NW = WGM * WGN;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int FM = WM / 16, FN = WN / 16;
    constexpr int TB = BN / 16;
    constexpr int IA = BM / 8;                   // A load instructions per stage
    constexpr int IB = 2 * TB;                   // B load instructions per stage (two K tiles)
    constexpr int LPW = (IA + IB) / NW;
    static_assert((IA + IB) % NW == 0, "stage loads must split evenly over the waves");
    constexpr int kA = BM * 128;                 // A bytes per stage
    constexpr int kStage = kA + IB * 1024;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int M = a.M, N = a.N, K = a.K, KT = a.kt;

    const int nblk = a.tiles_m * a.tiles_n;
    int b = blockIdx.x;
    if ((nblk & 7) == 0) b = (b & 7) * (nblk >> 3) + (b >> 3);
    const int tm_idx = b % a.tiles_m, tn_idx = b / a.tiles_m;
    const int m0 = tm_idx * BM, n0 = tn_idx * BN;

    const __amdgpu_buffer_rsrc_t ra = make_rsrc(a.xq, (uint32_t)M * (uint32_t)K);
    const int nt0 = n0 / 16, ntiles = (N + 15) / 16;
    const __amdgpu_buffer_rsrc_t rb =
        make_rsrc(a.wq + (int64_t)nt0 * KT * 1024, (uint32_t)min(TB, ntiles - nt0) * (uint32_t)KT * 1024u);


    // A: instruction q covers local rows 8q .. 8q + 7; lane l -> row 8q + l / 8,
    // LDS slot l % 8, global chunk c = slot ^ (row % 8) ^ ((row / 8) % 2)
    const int a_r = lane >> 3, a_s = lane & 7;
    const uint32_t b_lane = (uint32_t)lane * 16u;
    auto issue = [&](int st, int slot) {
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int q = wave * LPW + i;  // uniform
            if (q < IA) {
                const int row = 8 * q + a_r;
                const int c = a_slot(row, a_s);  // the swizzle is an involution in the chunk
                const int k = st * 128 + c * 16;
                const uint32_t off = (uint32_t)(m0 + row) * (uint32_t)K + (uint32_t)k;
                lds_void_t* dst = (lds_void_t*)(smem + slot * kStage + q * 1024);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, dst, 16, k < K ? off : (uint32_t)kOutOfRange, 0, 0, 0);
            } else {
                const int u = q - IA;            // k tile u / TB of the stage, n tile u % TB
                const int kt = st * 2 + u / TB;
                const uint32_t off = (uint32_t)((u % TB) * KT + kt) * 1024u + b_lane;
                lds_void_t* dst = (lds_void_t*)(smem + slot * kStage + kA + u * 1024);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, dst, 16, kt < KT ? off : (uint32_t)kOutOfRange, 0, 0, 0);
            }
        }
    };

    // fragment read offsets: A row R = wm * WM + 16 i + lane % 16, chunk 4 w + lane / 16
    int a_off[FM][2];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int row = wm * WM + i * 16 + (lane & 15);
#pragma unroll
        for (int w = 0; w < 2; ++w)
            a_off[i][w] = (row >> 3) * 1024 + (row & 7) * 128 + a_slot(row, 4 * w + (lane >> 4)) * 16;
    }

    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    const int ns = (KT + 1) / 2;
    if (wave == 0) issue_scale_loads<BM, BN>(a, m0, n0, smem + S * kStage, lane);
#pragma unroll
    for (int s0 = 0; s0 < S - 1; ++s0)
        if (s0 < ns) issue(s0, s0);
    for (int st = 0; st < ns; ++st) {
        if (st + S - 2 < ns) wait_vmcnt_le((S - 2) * LPW); else wait_vmcnt_le(0);
        lds_barrier();
        if (st + S - 1 < ns) issue(st + S - 1, (st + S - 1) % S);
        const int8_t* sb = smem + (st % S) * kStage;
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            v4i af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) af[i] = *(const v4i*)(sb + a_off[i][w]);
#pragma unroll
            for (int j = 0; j < FN; ++j) bf[j] = *(const v4i*)(sb + kA + (w * TB + wn * FN + j) * 1024 + lane * 16);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[j], af[i], acc[i][j], 0, 0, 0);
        }
    }

    store_tile<BM, BN, FM, FN>(a, acc, smem + S * kStage, m0, n0, wm * WM, wn * WN, lane);
}


// Loader-wave form: NC = WGM x WGN compute waves only read LDS and run
// MFMAs; NL loader waves only issue the direct-to-LDS loads of the ring and
// wait for them.  Counters of the single-role kernel (gemm_tile) showed the
// texture-address FIFO full for long stretches, every wave stalling while
// it issued its loads; with the roles split those stalls no longer hold up
// an MFMA wave (256 x 128, 3 stages, 8 loaders: 1.78 vs 1.43 POPS at
// (2048, 4096, 4096), 2.21 vs 1.55 at K = 21504).  One bare barrier per
// stage: the loaders wait for the stage's loads (vmcnt) before it, the
// compute waves read it after it; the compute waves' reads of a stage are
// done (they fed its MFMAs) before they reach the barrier that lets the
// loaders refill its slot.
//
// ATILED: A in the weights' tiled layout ([ceil(M/16)][KT][1 KiB], written
// by the row quantizer), every A load one contiguous KiB; otherwise
// row-major A through the swizzled 8-row x 128-byte loads of gemm_tile.
// Tiled A measured 1.66 vs 1.40 POPS at (2048, 21504, 4096).
template <int BM, int BN, int WGM, int WGN, int S, int NL, bool ATILED, int KS = 2>
__device__ __forceinline__ void gemm_ws(const GemmW8A8Args& a, int8_t* smem) {
    static_assert(KS == 2 || (KS == 1 && ATILED), "row-major A loads cover 128 bytes of K per stage");
    constexpr int NC = WGM * WGN;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int FM = WM / 16, FN = WN / 16;
    constexpr int TA = BM / 16, TB = BN / 16;
    constexpr int IA = ATILED ? KS * TA : BM / 8;  // A load instructions per stage of KS K tiles
    constexpr int IB = KS * TB;
    constexpr int LPW = (IA + IB) / NL;
    static_assert((IA + IB) % NL == 0, "stage loads must split evenly over the loader waves");
    constexpr int kA = BM * 64 * KS;
    constexpr int kStage = kA + IB * 1024;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int M = a.M, N = a.N, K = a.K, KT = a.kt;
    const int nblk = a.tiles_m * a.tiles_n;
    int b = blockIdx.x;
    int tm_idx, tn_idx;
    if (a.tiles_m == 8 && (a.tiles_n & 3) == 0) {
        // 8 tile rows (M = 2048 at 256): each XCD a window of 4 tile rows x
        // tiles_n / 4 columns (2048 x 4096: 34.6-34.7 / 145.7 us against
        // 35.1-35.3 / 146.6-146.7 for 8 x 4 windows at K = 4096 / 21504)
        const int x = b & 7, l = b >> 3;
        tm_idx = (x & 1) * 4 + (l & 3);
        tn_idx = (x >> 1) * (a.tiles_n >> 2) + (l >> 2);
    } else {
        if ((nblk & 7) == 0) b = (b & 7) * (nblk >> 3) + (b >> 3);
        tm_idx = b % a.tiles_m;
        tn_idx = b / a.tiles_m;
    }
    const int m0 = tm_idx * BM, n0 = tn_idx * BN;
    const int ns = (KT + KS - 1) / KS;

    if (wave >= NC) {  // ---- loader wave
        const int mt0 = m0 / 16, mtiles = (M + 15) / 16;
        const int nt0 = n0 / 16, ntiles = (N + 15) / 16;
        const __amdgpu_buffer_rsrc_t ra =
            ATILED ? make_rsrc(a.xq + (int64_t)mt0 * KT * 1024, (uint32_t)min(TA, mtiles - mt0) * (uint32_t)KT * 1024u)
                   : make_rsrc(a.xq, (uint32_t)M * (uint32_t)K);
        const __amdgpu_buffer_rsrc_t rb =
            make_rsrc(a.wq + (int64_t)nt0 * KT * 1024, (uint32_t)min(TB, ntiles - nt0) * (uint32_t)KT * 1024u);
        const uint32_t l16 = (uint32_t)lane * 16u;
        const int a_r = lane >> 3, a_s = lane & 7;
        const int lw = wave - NC;
        if (lw == 0) issue_scale_loads<BM, BN>(a, m0, n0, smem + S * kStage, lane);
        auto issue = [&](int st, int slot) {
#pragma unroll
            for (int i = 0; i < LPW; ++i) {
                const int q = lw * LPW + i;  // uniform
                lds_void_t* dst = (lds_void_t*)(smem + slot * kStage + q * 1024);
                if (q < IA) {
                    if constexpr (ATILED) {  // K tile q / TA of the stage, M tile q % TA
                        const int kt = st * KS + q / TA;
                        const uint32_t off = (uint32_t)((q % TA) * KT + kt) * 1024u + l16;
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, dst, 16, kt < KT ? off : (uint32_t)kOutOfRange,
                                                                 0, 0, 0);
                    } else {  // local rows 8q .. 8q + 7, swizzled chunks
                        const int row = 8 * q + a_r;
                        const int k = st * 128 + a_slot(row, a_s) * 16;
                        const uint32_t off = (uint32_t)(m0 + row) * (uint32_t)K + (uint32_t)k;
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, dst, 16, k < K ? off : (uint32_t)kOutOfRange, 0,
                                                                 0, 0);
                    }
                } else {  // K tile u / TB of the stage, N tile u % TB
                    const int u = q - IA;
                    const int kt = st * KS + u / TB;
                    const uint32_t off = (uint32_t)((u % TB) * KT + kt) * 1024u + l16;
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, dst, 16, kt < KT ? off : (uint32_t)kOutOfRange, 0, 0,
                                                             0);
                }
            }
        };
#pragma unroll
        for (int s0 = 0; s0 < S - 1; ++s0)
            if (s0 < ns) issue(s0, s0);
        for (int st = 0; st < ns; ++st) {
            if (st + S - 2 < ns) wait_vmcnt_le((S - 2) * LPW); else wait_vmcnt_le(0);
            lds_barrier();
            if (st + S - 1 < ns) issue(st + S - 1, (st + S - 1) % S);
        }
        return;
    }

    // ---- compute wave
    const int wm = wave / WGN, wn = wave % WGN;
    // A fragment (M fragment i, K step w) read offsets within a stage
    int a_off[FM][KS];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int w = 0; w < KS; ++w) {
            if constexpr (ATILED) {
                a_off[i][w] = (w * TA + wm * FM + i) * 1024 + lane * 16;
            } else {
                const int row = wm * WM + i * 16 + (lane & 15);
                a_off[i][w] = (row >> 3) * 1024 + (row & 7) * 128 + a_slot(row, 4 * w + (lane >> 4)) * 16;
            }
        }
    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};
    for (int st = 0; st < ns; ++st) {
        lds_barrier();
        const int8_t* sb = smem + (st % S) * kStage;
#pragma unroll
        for (int w = 0; w < KS; ++w) {
            v4i af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) af[i] = *(const v4i*)(sb + a_off[i][w]);
#pragma unroll
            for (int j = 0; j < FN; ++j) bf[j] = *(const v4i*)(sb + kA + (w * TB + wn * FN + j) * 1024 + lane * 16);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[j], af[i], acc[i][j], 0, 0, 0);
        }
    }
    store_tile<BM, BN, FM, FN>(a, acc, smem + S * kStage, m0, n0, wm * WM, wn * WN, lane);
}

}  // namespace

// 256 x 128 tiles: 8 compute waves of 64 x 64 + 8 loader waves, 3 stages.
extern "C" __global__ __launch_bounds__(1024) void nh_gemm_w8a8_256x128_kernel(GemmW8A8Args a) {
    extern __shared__ __align__(1024) int8_t smem[];
    gemm_ws<256, 128, 4, 2, 3, 8, false>(a, smem);
}

// The same with A in the tiled layout (the linear entry point's quantizer writes it).
extern "C" __global__ __launch_bounds__(1024) void nh_gemm_w8a8_ta_256x128_kernel(GemmW8A8Args a) {
    extern __shared__ __align__(1024) int8_t smem[];
    gemm_ws<256, 128, 4, 2, 3, 8, true>(a, smem);
}

// 128 x 128 tiles, tiled A: 4 compute waves of 64 x 64 + 4 loader waves (fewer, smaller tiles).
extern "C" __global__ __launch_bounds__(512) void nh_gemm_w8a8_ta_128x128_kernel(GemmW8A8Args a) {
    extern __shared__ __align__(1024) int8_t smem[];
    gemm_ws<128, 128, 2, 2, 3, 4, true>(a, smem);
}

// 64 x 128 tiles, tiled A: 4 compute waves of 32 x 64 + 2 loader waves, for
// products whose 128 x 128 tiles would leave CUs idle (M = 128 at N = 16384:
// 256 workgroups; M = 512 with N = 2688 or 3712 took these before the 64 x 64
// tiles: the MoE layer's shared expert 338 -> 327 us against 128 x 128).
// Four compute waves keep every SIMD's MFMA unit busy (two waves of 64 x 64:
// 337 us).
extern "C" __global__ __launch_bounds__(384) void nh_gemm_w8a8_ta_64x128_kernel(GemmW8A8Args a) {
    extern __shared__ __align__(1024) int8_t smem[];
    gemm_ws<64, 128, 2, 2, 3, 2, true>(a, smem);
}

// 64 x 64 tiles, tiled A: 4 compute waves of 32 x 32 + 2 loader waves, for
// products with few rows whose larger tiles leave CUs idle (batched decode
// past 16 rows: M = 24..64 at 4096 -> 16384 on 256 workgroups, 32.5 -> 23.3 us
// against 128 workgroups of 64 x 128; the weight stream is the bound there).
extern "C" __global__ __launch_bounds__(384) void nh_gemm_w8a8_ta_64x64_kernel(GemmW8A8Args a) {
    extern __shared__ __align__(1024) int8_t smem[];
    gemm_ws<64, 64, 2, 2, 3, 2, true>(a, smem);
}

// 128 x 128 tiles, row-major A, 4 waves of 64 x 64, 3 stages (single-role).
extern "C" __global__ __launch_bounds__(256) void nh_gemm_w8a8_128x128_kernel(GemmW8A8Args a) {
    extern __shared__ __align__(1024) int8_t smem[];
    gemm_tile<128, 128, 2, 2, 3>(a, smem);
}
