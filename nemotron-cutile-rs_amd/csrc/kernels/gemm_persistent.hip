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
//  * the weights one stage further ahead than the activations (an A ring of
//    two slots, a B ring of three): with the weights cold in HBM, as a
//    model's layers read them, rather than in the MALL, as one matrix timed
//    over and over is, (2048, 21504, 4096) takes 181.7-184.9 us against
//    193.6-196.4 us for one common ring of two stages (170-173 us warm either way);
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
// loads, past the last stage loads of zeros from an empty resource; one
// scale load or a load of zeros into a spare KiB; and per tile a
// fixed number of unconditional buffer stores; counts complete in issue
// order), so before the barrier of stage g it waits with vmcnt equal to the
// number it issued after stage g's loads -- never more than are actually
// outstanding after them -- and the barrier then publishes every wave's part
// of the stage.  The per-tile scales (sx for BM rows, sw and bias for BN
// columns) arrive the same way, with the tile's first A stage, into one of
// three LDS buffers.
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

// Stages of two K tiles (128 bytes of K): one barrier per two MFMA K steps.
// The weight operand (B) runs one stage further ahead than the activations
// (A): a 2-slot A ring and a 3-slot B ring, each slot holding only its own
// operand's tiles (so the three B slots still fit the LDS), and a weight
// stage has two stages of MFMA time to arrive instead of one.  Register set X
// holds a stage's first K step, Y its second.  Step of stage g: barrier;
// X <- K step 0 of stage g; MFMAs of Y (K step 1 of stage g - 1) -- at a
// tile's first stage followed by the previous tile's epilogue; the A loads of
// stage g + 1 (with its tile's scales) and the B loads of stage g + 2;
// Y <- K step 1 of stage g (after the MFMAs that read Y issued); MFMAs of X.
// Every barrier is followed at once by MFMA work whose operands are already
// in registers.  Before the barrier of stage g + 1 a wave waits for all but
// its B loads of stage g + 2, the last it issued.
template <int BM, int BN, int WGM, int WGN>
__device__ __forceinline__ void gemm_persistent(const GemmW8A8Args& a, int8_t* smem) {
    constexpr int NW = WGM * WGN;
    constexpr int TA = BM / 16, TB = BN / 16;
    constexpr int LPWA = (2 * TA + NW - 1) / NW, LPWB = (2 * TB + NW - 1) / NW;
    constexpr int kA = NW * LPWA * 1024;  // an A slot: [K half][TA tiles] (+ padding slots)
    constexpr int kB = 2 * TB * 1024;     // a B slot: [K half][TB tiles]; padding loads go to the spare KiB
    constexpr int FM = BM / WGM / 16, FN = BN / WGN / 16;
    static_assert(BM % (16 * WGM) == 0 && BN % (16 * WGN) == 0, "wave tiles of whole fragments");
    static_assert(BM <= 256 && BN <= 256, "one 16-byte load per lane holds a tile's scales");
    constexpr int NSB = 3;
    constexpr int kScales = 3 * 1024;
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
    const uint32_t ringa = (uint32_t)(uintptr_t)(lds_i8*)smem;
    const uint32_t ringb = ringa + (uint32_t)(2 * kA);
    const uint32_t scal0 = ringb + (uint32_t)(3 * kB);
    const uint32_t dummy = scal0 + (uint32_t)(NSB * kScales);
    const float* scales = (const float*)(smem + 2 * kA + 3 * kB);
    const int esz = a.out_dtype == DT_BF16 ? 2 : 4;
    const v4i out_r = rsrc_words(a.out, (uint32_t)M * (uint32_t)a.ldo * (uint32_t)esz);
    const v4i null_r = rsrc_words(a.out, 0u);

    // A stream (with the tile's scales) and B stream: next stage to issue
    int ia_t = 0, ia_k = 0, sa_i = 0, sb_i = 0;
    int ib_t = 0, ib_k = 0, sbb_i = 0;
    v4i ra, rb, rsc;
    uint32_t sc_dst;
    auto set_a_tile = [&]() {
        const int p = ia_t * G + pos;
        const int m0 = (p % a.tiles_m) * BM, n0 = (p / a.tiles_m) * BN;
        const int mt0 = m0 >> 4;
        ra = rsrc_words(a.xq + (int64_t)mt0 * KT * 1024, (uint32_t)min(TA, mtiles - mt0) * (uint32_t)KT * 1024u);
        rsc = wave == 0   ? rsrc_words(a.sx + m0, (uint32_t)(M - m0) * 4u)
              : wave == 1 ? rsrc_words(a.sw + n0, (uint32_t)(N - n0) * 4u)
              : (wave == 2 && a.bias) ? rsrc_words(a.bias + n0, (uint32_t)(N - n0) * 4u) : null_r;
        const uint32_t sb = scal0 + (uint32_t)(sb_i * kScales);
        sc_dst = wave == 0 ? sb : wave == 1 ? sb + 1024 : wave == 2 ? sb + 2048 : dummy;
    };
    auto set_b_tile = [&]() {
        const int p = ib_t * G + pos;
        const int nt0 = ((p / a.tiles_m) * BN) >> 4;
        rb = rsrc_words(a.wq + (int64_t)nt0 * KT * 1024, (uint32_t)min(TB, ntiles - nt0) * (uint32_t)KT * 1024u);
    };
    set_a_tile();
    set_b_tile();
    auto issue_a = [&]() {
        const uint32_t st = ringa + (uint32_t)(sa_i * kA);
        const int kt0 = 2 * ia_k;
#pragma unroll
        for (int i = 0; i < LPWA; ++i) {
            const int q = wave + i * NW;  // uniform
            const int h = q >= TA ? 1 : 0, t = q - h * TA;
            const uint32_t off = q < 2 * TA ? (uint32_t)((t * KT + kt0 + h) * 1024 + lane * 16) : (uint32_t)kOutOfRange;
            lds_dma16(ra, off, st + (uint32_t)(q * 1024));
        }
        lds_dma16(ia_k == 0 ? rsc : null_r, (uint32_t)lane * 16u, ia_k == 0 ? sc_dst : dummy);
        sa_i ^= 1;
        if (++ia_k == KT2) {
            ia_k = 0;
            ++ia_t;
            sb_i = sb_i + 1 == NSB ? 0 : sb_i + 1;
            if (ia_t < my_tiles) set_a_tile();
        }
    };
    // the B loads of the next B stage (past the last stage: loads of zeros
    // from an empty resource into a slot no stage reads any more).  Wave w
    // issues the slots w, w + NW, ... below 2 TB: LPWB loads for the first
    // (2 TB) % NW waves, LPWB - 1 for the others, no padding loads.
    constexpr int kBFull = (2 * TB) % NW == 0 ? NW : (2 * TB) % NW;  // waves with LPWB B loads
    auto issue_b = [&]() {
        const bool live = ib_t < my_tiles;  // uniform
        const v4i rbx = live ? rb : null_r;
        const uint32_t st = ringb + (uint32_t)(sbb_i * kB);
        const int kt0 = 2 * ib_k;
#pragma unroll
        for (int i = 0; i < LPWB; ++i) {
            const int q = wave + i * NW;  // uniform
            if (i + 1 < LPWB || wave < kBFull) {
                const int h = q >= TB ? 1 : 0, t = q - h * TB;
                lds_dma16(rbx, (uint32_t)((t * KT + kt0 + h) * 1024 + lane * 16), st + (uint32_t)(q * 1024));
            }
        }
        if (live) {
            sbb_i = sbb_i + 1 == 3 ? 0 : sbb_i + 1;
            if (++ib_k == KT2) {
                ib_k = 0;
                ++ib_t;
                if (ib_t < my_tiles) set_b_tile();
            }
        }
    };

    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};
    v4i xa[FM], xb[FN], ya[FM], yb[FN];
    int rda = 0, rdb = 0;  // read slots of the A and B rings
    auto read = [&](v4i (&fa)[FM], v4i (&fb)[FN], int h) {
        const int8_t* sta = smem + rda * kA + h * TA * 1024 + lane * 16;
        const int8_t* stb = smem + 2 * kA + rdb * kB + h * TB * 1024 + lane * 16;
#pragma unroll
        for (int i = 0; i < FM; ++i) fa[i] = *(const v4i*)(sta + (wm * FM + i) * 1024);
#pragma unroll
        for (int j = 0; j < FN; ++j) fb[j] = *(const v4i*)(stb + (wn * FN + j) * 1024);
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

    // prologue: B of stage 0, A of stage 0 (and its scales), B of stage 1
    issue_b();
    issue_a();
    issue_b();
    // before the barrier of stage g: every operation but the B loads of stage
    // g + 1 (issued last) has completed
    auto sync = [&](int g) {
        wait_lgkm0();
        if (g + 1 >= nst) NH_WAIT_VMCNT(0);
        else if (wave < kBFull) NH_WAIT_VMCNT(LPWB);
        else NH_WAIT_VMCNT(LPWB - 1);
        lds_barrier();
    };
    auto second_half = [&](int g) {
        if (g + 1 < nst) {
            issue_a();
            issue_b();
        }
        read(ya, yb, 1);
        rda ^= 1;
        rdb = rdb + 1 == 3 ? 0 : rdb + 1;
        __builtin_amdgcn_sched_barrier(0);
        mma(xa, xb);
    };
    auto rest_of_tile = [&](int& g) {
        for (int k2 = 1; k2 < KT2; ++k2, ++g) {
            sync(g);
            read(xa, xb, 0);
            __builtin_amdgcn_sched_barrier(0);
            mma(ya, yb);
            second_half(g);
        }
    };
    int g = 0;
    sync(0);
    read(xa, xb, 0);
    second_half(0);
    g = 1;
    rest_of_tile(g);
    for (int t = 1; t < my_tiles; ++t, ++g) {
        sync(g);
        read(xa, xb, 0);
        __builtin_amdgcn_sched_barrier(0);
        mma(ya, yb);
        epilogue();
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

// LDS of gemm_persistent: two A slots (whole loads per wave), three B slots, three scale buffers, one spare KiB.
#define NH_GEMM_P_LDS(BM, BN, NW)                                                                      \
    (2 * (NW) * ((2 * (BM) / 16 + (NW) - 1) / (NW)) * 1024 + 3 * (2 * (BN) / 16) * 1024 + 3 * 3 * 1024 + 1024)

// 256 x 224 tiles, 8 waves of 64 x 112: the 21504-wide projection at M = 2048
// is 768 tiles, three per CU.
extern "C" __global__ __launch_bounds__(512) void nh_gemm_w8a8_p256x224_kernel(GemmW8A8Args a) {
    extern __shared__ __align__(1024) int8_t smem[];
    gemm_persistent<256, 224, 4, 2>(a, smem);
}
