// G3, persistent form: one workgroup per CU walks a list of BM x BN output
// tiles with 8 waves, each owning a (BM / WGM) x (BN / WGN) block of every
// tile, all of them streaming both operands into LDS.  Used where its tile
// fills whole rounds of CUs better than the loader-wave kernel of gemm.hip
// (the 21504-wide up projection at M = 2048: 162-164 us back to back against
// 212-236 us for the loader-wave kernel).
//
//  * 64 x 112 wave tiles on a 256 x 224 tile read 98 B/clk of LDS per CU at
//    the MFMA rate (the 64 x 64 tiles of gemm.hip: 128), and the tile needs
//    34 B/clk from L2 per CU instead of 48;
//  * stages of two K tiles (128 bytes of K), one barrier per two MFMA K steps;
//  * the first K step of stage g is read into one register set right after
//    the barrier while the MFMAs of the second K step of stage g - 1 run from
//    the other, so every barrier is followed by MFMA work already in registers;
//  * a workgroup moves from tile to tile without draining its ring, and the
//    epilogue stores go straight from the accumulators (no LDS staging);
//  * tiles are dealt so that the G / 8 workgroups of an XCD (dispatch is
//    round-robin over the 8 XCDs) hold consecutive positions of a
//    column-major order over the M tiles, sharing panels in their L2.
//
// Memory operations.  Every wave issues its share of each stage's
// direct-to-LDS loads (lane l's 16 bytes land at M0 + 16 l) through inline
// asm: the compiler, which cannot tell LDS-DMA writes from the LDS reads that
// follow, would otherwise wait for every load in flight (vmcnt(0)) before
// each fragment read.  The ring's synchronization is explicit instead: each
// wave issues a fixed number of vector-memory operations per stage (operand
// loads, one scale load or a load of zeros into a spare KiB, and per tile a
// fixed number of unconditional buffer stores; counts complete in issue
// order), so before the barrier of stage g it waits with vmcnt equal to the
// number it issued after stage g's loads -- never more than are actually
// outstanding after them -- and the barrier then publishes every wave's part
// of the stage.  The per-tile scales (sx for BM rows, sw and bias for BN
// columns) arrive the same way, with the tile's first stage, into one of
// S + 1 LDS buffers.
//
// Operand layouts: A and B both in the tiled layout (nh_numerics.h), so each
// 1 KiB tile is one MFMA operand.  The MFMA takes the weight fragment as its
// first operand and the activation fragment as its second, so lane l holds
// C[m = 16 i + l % 16][n = 16 j + 4 (l / 16) + r] in register r: four
// consecutive columns of one row, stored as 8 bytes (bf16) or 16 (f32).
//
// Host contract (launch_gemm): A tiled, KT even, M % 4 == 0 and N % 4 == 0
// (the scale rows are read 16 bytes at a time), ldo % 4 == 0, 16-byte aligned
// out, sx, sw and bias, M * ldo * esz < 2^31, LDS of NH_GEMM_P_LDS, grid <= the
// tile count (one workgroup per CU).
#include <type_traits>

#include "nh_device.h"

using namespace nh;

namespace {

// The four dwords of a raw buffer resource (the layout make_rsrc builds).
__device__ __forceinline__ v4i rsrc_words(const void* base, uint32_t bytes) {
    const uint64_t p = (uint64_t)base;
    return v4i{(int)(uint32_t)p, (int)((uint32_t)(p >> 32) & 0xffffu), (int)bytes, 0x00020000};
}

// 16 bytes per lane from rsrc + voffset into LDS at lds_addr + 16 lane.  The
// load takes its LDS base from M0, a register the compiler reserves: the asm
// saves M0 in an SGPR of its own, sets it (one wait state before the load
// reads it), issues the load and puts the saved value back, so M0 holds the
// same value after the statement as before it and needs no clobber.
__device__ __forceinline__ void lds_dma16(v4i rsrc, uint32_t voffset, uint32_t lds_addr) {
    // the resource and the LDS address are wave-uniform; say so, so that they are passed in SGPRs
    lds_addr = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_addr);
    rsrc = v4i{__builtin_amdgcn_readfirstlane(rsrc[0]), __builtin_amdgcn_readfirstlane(rsrc[1]),
               __builtin_amdgcn_readfirstlane(rsrc[2]), __builtin_amdgcn_readfirstlane(rsrc[3])};
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds_addr), "v"(voffset), "s"(rsrc)
        : "memory");
}


// s_waitcnt vmcnt(n) for a constant n in [0, 63], other counters untouched.
#define NH_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt((((n) & 15) | (7 << 4) | (15 << 8) | ((((n) >> 4) & 3) << 14)))

__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14)); }

// The same with stages of two K tiles (128 bytes of K): one barrier per two
// MFMA K steps.  Register set X holds a stage's first K step, Y its second.
// Step of stage g: barrier; X <- K step 0 of stage g; MFMAs of Y (K step 1
// of stage g - 1) -- at a tile's first stage followed by the previous tile's
// epilogue; the loads of stage g + S - 1; Y <- K step 1 of stage g (after the
// MFMAs that read Y issued); MFMAs of X.  Every barrier is followed at once
// by MFMA work whose operands are already in registers.
template <int BM, int BN, int WGM, int WGN, int S>
__device__ __forceinline__ void gemm_persistent(const GemmW8A8Args& a, int8_t* smem) {
    constexpr int NW = WGM * WGN;
    constexpr int TA = BM / 16, TB = BN / 16, TQ = TA + TB;
    constexpr int LPW = (2 * TQ + NW - 1) / NW;  // operand loads per wave per stage
    constexpr int kStage = NW * LPW * 1024;      // two K tiles; slots past 2 TQ take zeros
    constexpr int C = LPW + 1;                   // loads per wave per stage: operands + one scale load
    constexpr int FM = BM / WGM / 16, FN = BN / WGN / 16;
    static_assert(BM % (16 * WGM) == 0 && BN % (16 * WGN) == 0, "wave tiles of whole fragments");
    static_assert(BM <= 256 && BN <= 256, "one 16-byte load per lane holds a tile's scales");
    static_assert(S >= 2, "");
    constexpr int NSB = S + 1;
    constexpr int kScales = 3 * 1024;
    constexpr int NSTORE = FM * FN;
    constexpr int kAllow0 = (S - 2) * C;
    constexpr int kAllow1 = kAllow0 + NSTORE < 63 ? kAllow0 + NSTORE : 63;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const int M = a.M, N = a.N, KT = a.kt, KT2 = KT >> 1;
    const int mtiles = (M + 15) >> 4, ntiles = (N + 15) >> 4;
    const int tiles = a.tiles_m * a.tiles_n, G = gridDim.x;
    const int b = blockIdx.x;
    const int pos = (G & 7) == 0 ? (b & 7) * (G >> 3) + (b >> 3) : b;
    const int my_tiles = pos < tiles ? (tiles - 1 - pos) / G + 1 : 0;
    const int nst = my_tiles * KT2;
    if (nst == 0) return;
    typedef __attribute__((address_space(3))) int8_t lds_i8;
    const uint32_t ring0 = (uint32_t)(uintptr_t)(lds_i8*)smem;
    const uint32_t scal0 = ring0 + (uint32_t)(S * kStage);
    const uint32_t dummy = scal0 + (uint32_t)(NSB * kScales);
    const float* scales = (const float*)(smem + S * kStage);
    const int esz = a.out_dtype == DT_BF16 ? 2 : 4;
    const v4i out_r = rsrc_words(a.out, (uint32_t)M * (uint32_t)a.ldo * (uint32_t)esz);
    const v4i null_r = rsrc_words(a.out, 0u);

    int it_i = 0, kt_i = 0, s_i = 0, sb_i = 0;  // next stage to issue: tile, stage within it, slot, scale buffer
    v4i ra, rb, rsc;
    uint32_t sc_dst;
    auto set_issue_tile = [&]() {
        const int p = it_i * G + pos;
        const int m0 = (p % a.tiles_m) * BM, n0 = (p / a.tiles_m) * BN;
        const int mt0 = m0 >> 4, nt0 = n0 >> 4;
        ra = rsrc_words(a.xq + (int64_t)mt0 * KT * 1024, (uint32_t)min(TA, mtiles - mt0) * (uint32_t)KT * 1024u);
        rb = rsrc_words(a.wq + (int64_t)nt0 * KT * 1024, (uint32_t)min(TB, ntiles - nt0) * (uint32_t)KT * 1024u);
        rsc = wave == 0   ? rsrc_words(a.sx + m0, (uint32_t)(M - m0) * 4u)
              : wave == 1 ? rsrc_words(a.sw + n0, (uint32_t)(N - n0) * 4u)
              : (wave == 2 && a.bias) ? rsrc_words(a.bias + n0, (uint32_t)(N - n0) * 4u) : null_r;
        const uint32_t sb = scal0 + (uint32_t)(sb_i * kScales);
        sc_dst = wave == 0 ? sb : wave == 1 ? sb + 1024 : wave == 2 ? sb + 2048 : dummy;
    };
    set_issue_tile();
    // slot layout of a stage: [K step][A tiles, B tiles] of 1 KiB; q = h TQ + t
    auto issue = [&]() {
        const uint32_t st = ring0 + (uint32_t)(s_i * kStage);
        const int kt0 = 2 * kt_i;
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int q = wave + i * NW;  // uniform
            const int h = q >= TQ ? 1 : 0, t = q - h * TQ;
            const bool isa = t < TA;
            const int row = isa ? t : t - TA;
            const uint32_t off = q < 2 * TQ ? (uint32_t)((row * KT + kt0 + h) * 1024 + lane * 16) : (uint32_t)kOutOfRange;
            lds_dma16(isa ? ra : rb, off, st + (uint32_t)(q * 1024));
        }
        lds_dma16(kt_i == 0 ? rsc : null_r, (uint32_t)lane * 16u, kt_i == 0 ? sc_dst : dummy);
        s_i = s_i + 1 == S ? 0 : s_i + 1;
        if (++kt_i == KT2) {
            kt_i = 0;
            ++it_i;
            sb_i = sb_i + 1 == NSB ? 0 : sb_i + 1;
            if (it_i < my_tiles) set_issue_tile();
        }
    };

    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};
    v4i xa[FM], xb[FN], ya[FM], yb[FN];
    auto read = [&](v4i (&fa)[FM], v4i (&fb)[FN], int slot, int h) {
        const int8_t* st = smem + slot * kStage + h * TQ * 1024 + lane * 16;
#pragma unroll
        for (int i = 0; i < FM; ++i) fa[i] = *(const v4i*)(st + (wm * FM + i) * 1024);
#pragma unroll
        for (int j = 0; j < FN; ++j) fb[j] = *(const v4i*)(st + (TA + wn * FN + j) * 1024);
    };
    auto mma = [&](const v4i (&fa)[FM], const v4i (&fb)[FN]) {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int i = 0; i < FM; ++i) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb[j], fa[i], acc[i][j], 0, 0, 0);
    };
    int it_e = 0, sb_e = 0;
    auto epilogue = [&]() {
        const int p = it_e * G + pos;
        const int m0 = (p % a.tiles_m) * BM, n0 = (p / a.tiles_m) * BN;
        const float* sc = scales + sb_e * (kScales / 4);
        const int ml = wm * FM * 16 + (lane & 15), nl = wn * FN * 16 + 4 * (lane >> 4);
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int n = nl + 16 * j;
            const float4 sw4 = *(const float4*)(sc + 256 + n);
            const float4 b4 = a.bias ? *(const float4*)(sc + 512 + n) : make_float4(0.f, 0.f, 0.f, 0.f);
            const float swv[4] = {sw4.x, sw4.y, sw4.z, sw4.w}, bv[4] = {b4.x, b4.y, b4.z, b4.w};
            const bool nok = n0 + n < N;
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int m = ml + 16 * i;
                const float sx = sc[m];
                float y[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    y[r] = epilogue_w8a8(acc[i][j][r], sx, swv[r]);
                    if (a.bias) y[r] = y[r] + bv[r];
                    if (a.relu2) y[r] = relu2(y[r]);
                }
                const uint32_t off = (nok && m0 + m < M) ? (uint32_t)(((m0 + m) * a.ldo + n0 + n) * esz)
                                                         : (uint32_t)kOutOfRange;
                if (esz == 2) {
                    typedef uint32_t v2u __attribute__((ext_vector_type(2)));
                    const v2u v = {(uint32_t)f32_to_bf16(y[0]) | ((uint32_t)f32_to_bf16(y[1]) << 16),
                                   (uint32_t)f32_to_bf16(y[2]) | ((uint32_t)f32_to_bf16(y[3]) << 16)};
                    asm volatile("buffer_store_dwordx2 %0, %1, %2, 0 offen" : : "v"(v), "v"(off), "s"(out_r) : "memory");
                } else {
                    const v4i v = {(int)f32_bits(y[0]), (int)f32_bits(y[1]), (int)f32_bits(y[2]), (int)f32_bits(y[3])};
                    asm volatile("buffer_store_dwordx4 %0, %1, %2, 0 offen" : : "v"(v), "v"(off), "s"(out_r) : "memory");
                }
                acc[i][j] = v4i{0, 0, 0, 0};
            }
        }
        ++it_e;
        sb_e = sb_e + 1 == NSB ? 0 : sb_e + 1;
    };

#pragma unroll
    for (int s = 0; s < S - 1; ++s)
        if (s < nst) issue();
    int s_r = 0, last_epi = -S;
    // the stores of an epilogue come before the loads of its step, so they
    // follow stage g's loads when the epilogue ran in steps g - S + 2 .. g - 1
    const bool exact = KT2 >= S - 2;
    auto sync = [&](int g) {
        wait_lgkm0();
        if (!exact || g + S - 2 >= nst) NH_WAIT_VMCNT(0);
        else if (g - last_epi < S - 1) NH_WAIT_VMCNT(kAllow1);
        else NH_WAIT_VMCNT(kAllow0);
        lds_barrier();
    };
    auto second_half = [&](int g) {
        if (g + S - 1 < nst) issue();
        read(ya, yb, s_r, 1);
        s_r = s_r + 1 == S ? 0 : s_r + 1;
        __builtin_amdgcn_sched_barrier(0);
        mma(xa, xb);
    };
    auto rest_of_tile = [&](int& g) {
        for (int k2 = 1; k2 < KT2; ++k2, ++g) {
            sync(g);
            read(xa, xb, s_r, 0);
            __builtin_amdgcn_sched_barrier(0);
            mma(ya, yb);
            second_half(g);
        }
    };
    int g = 0;
    sync(0);
    read(xa, xb, s_r, 0);
    second_half(0);
    g = 1;
    rest_of_tile(g);
    for (int t = 1; t < my_tiles; ++t, ++g) {
        sync(g);
        read(xa, xb, s_r, 0);
        __builtin_amdgcn_sched_barrier(0);
        mma(ya, yb);
        epilogue();
        last_epi = g;
        second_half(g);
        ++g;
        rest_of_tile(g);
        --g;
    }
    wait_lgkm0();
    NH_WAIT_VMCNT(0);
    lds_barrier();
    mma(ya, yb);
    epilogue();
}

}  // namespace

// LDS of gemm_persistent: the ring (two K tiles per stage), S + 1 scale buffers, one spare KiB.
#define NH_GEMM_P_LDS(BM, BN, NW, S) \
    ((S) * (NW) * ((2 * ((BM) + (BN)) / 16 + (NW) - 1) / (NW)) * 1024 + ((S) + 1) * 3 * 1024 + 1024)

// 256 x 224 tiles, 8 waves of 64 x 112, 2 stages: the 21504-wide projection at
// M = 2048 is 768 tiles, three per CU.
extern "C" __global__ __launch_bounds__(512) void nh_gemm_w8a8_p256x224_kernel(GemmW8A8Args a) {
    extern __shared__ __align__(1024) int8_t smem[];
    gemm_persistent<256, 224, 4, 2, 2>(a, smem);
}
