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
// waits for the whole slab to have been issued.  Measured at M = 1,
// K = 4096 -> N = 16384: 2 / 4 / 6 / 8 / 12 / 16 head tiles take 12.98 /
// 12.45 / 12.05 / 12.08 / 12.38 / 12.55 us (16 cost occupancy: 143 VGPRs).
constexpr int kSlabHead = 8;

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

// y = ((float)acc * sx) * sw [+ bias] [ReLU^2] -> out (f32 or bf16 RNE).
__device__ __forceinline__ void store_y(void* out, int out_dtype, int64_t i, int32_t acc, float sx, float swn,
                                        const float* bias, float bn, int relu) {
    float y = epilogue_w8a8(acc, sx, swn);
    if (bias) y = y + bn;
    if (relu) y = relu2(y);
    store_out(out, i, y, out_dtype);
}

// The first non-finite activation of rows that hold one (the row maxima
// said so; a uniform, rare branch), from the workgroup's registers: xv[m][v]
// holds the 8 values at column (threadIdx.x + v T) 8 of row m.  The index is
// reported in the caller's whole input: this launch's rows start at row0.
template <int MM>
__device__ __forceinline__ void report_decode_rows(const LinearDecodeArgs& a, const v4i (&xv)[MM][2], int T) {
    __shared__ int red_nf[16];
    int first = 0x7fffffff;
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            const int c = (threadIdx.x + v * T) * 8;
            const int e = bf16x8_first_nonfinite(xv[m][v]);
            if (m < a.M && c < a.K && e < 8) first = min(first, m * a.K + c + e);
        }
    first = block_min_i32(first, red_nf);
    if (threadIdx.x == 0 && first != 0x7fffffff)
        report_nonfinite(a.nonfinite, 0, (int64_t)a.row0 * a.K + first,
                         bf16_to_f32(((const uint16_t*)a.x)[first]));
}

// The same for the wide decode units: xv[j] holds chunk c0 + j stride of
// the row-major [M][K] input, i.e. the values at flat index 8 chunk + e.
template <int XR>
__device__ __forceinline__ void report_decode_chunks(const LinearDecodeArgs& a, const v4i (&xv)[XR], int c0,
                                                     int stride) {
    __shared__ int red_nf[16];
    int first = 0x7fffffff;
    const int chunks = a.M * (a.K >> 3);
#pragma unroll
    for (int j = 0; j < XR; ++j) {
        const int c = c0 + j * stride;
        const int e = bf16x8_first_nonfinite(xv[j]);
        if (c < chunks && e < 8) first = min(first, c * 8 + e);
    }
    first = block_min_i32(first, red_nf);
    if (threadIdx.x == 0 && first != 0x7fffffff)
        report_nonfinite(a.nonfinite, 0, (int64_t)a.row0 * a.K + first,
                         bf16_to_f32(((const uint16_t*)a.x)[first]));
}

}  // namespace

// G1: quantized activations already in memory, M <= 16, any K <= 131072
// (waves walk their K tiles slab by slab).  The A fragments come from L2
// (at most 16 x K bytes, shared by every workgroup), issued ahead of the
// weight slab so they return first.  Two activation layouts:
//  * row-major xq [M][K] (the public entry point): a fragment is M rows x
//    64 bytes, M half-used cache lines;
//  * activation tiles [KT][4][M][16] (written by the row quantizer for the
//    linear entry point): the fragment of K tile t is the M * 64 contiguous
//    bytes at 64 M t, lane (r, g) reading 16 of them.  Measured 12.3 vs
//    12.9 us at M = 8 and 12.9 vs 15.9 us at M = 16 (K = 4096, N = 16384).
// Bytes of the last K tile past K are not read as zero by the tiled form;
// the weight tiles are zero there, so they add nothing.
template <bool XT>
__device__ __forceinline__ void gemv_w8a8(const GemvW8A8Args& a, v4i* red) {
    const int lane = threadIdx.x & 63, W = a.waves;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int M = a.M, N = a.N, K = a.K, kt = a.kt;
    const int tile = blockIdx.x;
    const __amdgpu_buffer_rsrc_t wr = row_tile_rsrc(a.wq, tile, kt);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.xq, XT ? (uint32_t)M * (uint32_t)kt * 64u : (uint32_t)M * (uint32_t)K);
    // epilogue operands first, ahead of the weight stream
    const int n = tile * 16 + r16;
    const float swn = n < N ? a.sw[n] : 0.0f;
    const float bn = (a.bias && n < N) ? a.bias[n] : 0.0f;
    float sxl[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) sxl[r] = 4 * g + r < M ? a.sx[4 * g + r] : 0.0f;
    // per-lane parts of the load offsets; the K tile enters as a scalar
    const bool xrow = r16 < M;
    const int xlane = XT ? (g * M + r16) * 16 : r16 * K + g * 16;
    const int wlane = lane * 16;
    const int steps = (kt + W - 1) / W;
    v4i acc = {0, 0, 0, 0};
    for (int s0 = 0; s0 < steps; s0 += kSlab) {
        v4i x[kSlab], b[kSlab];
        // The slab's first K tile as an opaque scalar: every offset is then
        // a per-lane invariant plus a scalar computed next to its load, so
        // no per-load offset registers are hoisted out of the loop (32 of
        // them would halve the occupancy).
        int t0 = wave + s0 * W;
        asm volatile("" : "+s"(t0));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < kSlab; ++s) {  // activation fragments (L2) first
            const int t = t0 + s * W;
            const int off = XT ? xlane + t * 64 * M : xlane + t * 64;
            x[s] = buffer_load16(xr, (xrow && (XT ? t < kt : t * 64 + g * 16 < K)) ? off : kOutOfRange);
        }
#pragma unroll
        for (int s = 0; s < kSlab; ++s)  // then the weight slab (HBM)
            b[s] = buffer_load16_stream(wr, (t0 + s * W) * 1024 + wlane);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < kSlab; ++s) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x[s], b[s], acc, 0, 0, 0);
    }
    if (reduce_waves(acc, red, W) && n < N) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (4 * g + r < M)
                store_y(a.out, a.out_dtype, (int64_t)(4 * g + r) * N + n, acc[r], sxl[r], swn, a.bias, bn, a.relu2);
    }
}

// The linear layer at M <= 16 bf16 rows as ONE launch (LinearHandoffArgs):
// the row quantizer and the tiled-A GEMV of the two-launch path, with the
// dependency between them kept inside the launch instead of at a kernel
// boundary.  The GEMV workgroups issue their weight slab first (it does not
// depend on the activations), then wait for the quantized rows, so the
// weight stream overlaps the quantization and the second launch's start-up.
// The handoff crosses XCDs, whose L2 caches are not coherent with each
// other: the producers store the codes and scales with agent-scope (sc1)
// writes and wait for them to complete before adding to the counter; the
// consumers read the counter, the codes and the scales with agent-scope
// (sc1) loads, which do not return stale L2 lines.  One lane of an extra
// wave polls (s_sleep between polls, a bounded number of polls), so the
// waves holding the weight slab never wait behind a poll; a bare s_barrier
// then releases them.  Same codes, scales and outputs as the two launches.
constexpr uint32_t kHandoffPolls = 1u << 18;  // ~0.5 s of polls: the rows take microseconds

__device__ __forceinline__ void handoff_consume(const LinearHandoffArgs& h, v4i* red) {
    const GemvW8A8Args& a = h.g;
    const int lane = threadIdx.x & 63, W = a.waves;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int M = a.M, N = a.N, kt = a.kt;
    const int tile = (int)blockIdx.x - h.q.rows;
    const int n = tile * 16 + r16;
    v4i b[kSlab];
    float swn = 0.0f, bn = 0.0f;
    if (wave < W) {
        const __amdgpu_buffer_rsrc_t wr = row_tile_rsrc(a.wq, tile, kt);
        swn = n < N ? a.sw[n] : 0.0f;
        bn = (a.bias && n < N) ? a.bias[n] : 0.0f;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < kSlab; ++s) b[s] = buffer_load16_stream(wr, (wave + s * W) * 1024 + lane * 16);
        __builtin_amdgcn_sched_barrier(0);
    } else if (lane == 0) {
        uint32_t polls = 0;
        bool ready;
        while (!(ready = __hip_atomic_load(&h.slot[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= (uint32_t)M) &&
               ++polls < kHandoffPolls)
            __builtin_amdgcn_s_sleep(2);
        if (!ready) __hip_atomic_store(&h.slot[2], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__hip_atomic_fetch_add(&h.slot[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            (uint32_t)h.consumers - 1) {  // the last workgroup past the wait: every row is in, reset the slot
            __hip_atomic_store(&h.slot[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&h.slot[1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    lds_barrier();  // the rows are in
    v4i acc = {0, 0, 0, 0};
    float sxl[4];
    if (wave < W) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            sxl[r] = 4 * g + r < M ? f32_from_bits(__hip_atomic_load((const uint32_t*)&a.sx[4 * g + r], __ATOMIC_RELAXED,
                                                                     __HIP_MEMORY_SCOPE_AGENT))
                                   : 0.0f;
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.xq, (uint32_t)M * (uint32_t)kt * 64u);
        const bool xrow = r16 < M;
        const int xlane = (g * M + r16) * 16;
        v4i x[kSlab];
#pragma unroll
        for (int s = 0; s < kSlab; ++s) {
            const int t = wave + s * W;
            x[s] = __builtin_amdgcn_raw_buffer_load_b128(xr, (xrow && t < kt) ? xlane + t * 64 * M : kOutOfRange, 0,
                                                         16 /* sc1 */);
        }
#pragma unroll
        for (int s = 0; s < kSlab; ++s) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x[s], b[s], acc, 0, 0, 0);
        red[wave * 64 + lane] = acc;
    }
    __syncthreads();
    if (wave == 0) {
        for (int w = 1; w < W; ++w) acc += red[w * 64 + lane];
        if (n < N) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (4 * g + r < M)
                    store_y(a.out, a.out_dtype, (int64_t)(4 * g + r) * N + n, acc[r], sxl[r], swn, a.bias, bn,
                            a.relu2);
        }
    }
}

extern "C" __global__ __launch_bounds__(576) void nh_linear_handoff_kernel(LinearHandoffArgs h) {
    __shared__ v4i red[8 * 64];
    __shared__ float redf[16];
    __shared__ int redi[16];
    if ((int64_t)blockIdx.x < h.q.rows) {  // a quantizer workgroup: one row, then publish it
        quantize_row_vec<DT_BF16, 2, true>(h.q, redf, redi);
        wait_vmcnt_le(0);  // this wave's codes and scale have completed
        lds_barrier();
        if (threadIdx.x == 0) __hip_atomic_fetch_add(&h.slot[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    handoff_consume(h, red);
}

extern "C" __global__ __launch_bounds__(512) void nh_gemv_w8a8_kernel(GemvW8A8Args a) {
    __shared__ v4i red[8 * 64];
    gemv_w8a8<false>(a, red);
}

extern "C" __global__ __launch_bounds__(512) void nh_gemv_w8a8_xt_kernel(GemvW8A8Args a) {
    __shared__ v4i red[8 * 64];
    gemv_w8a8<true>(a, red);
}

// int8 B operand from 8 bytes of tiled INT4 codes (16 codes of one lane):
// the low nibbles and the high nibbles of each word as bytes, i.e. K order
// 0 2 4 6 1 3 5 7 | 8 10 12 14 9 11 13 15.  The activation codes are stored
// in the same order (act_order_int4), so the MFMA pairs them correctly, and
// the zero point is folded out of the sum afterwards.
__device__ __forceinline__ v4i expand_int4(uint2 q) {
    return v4i{(int)(q.x & 0x0F0F0F0Fu), (int)((q.x >> 4) & 0x0F0F0F0Fu), (int)(q.y & 0x0F0F0F0Fu),
               (int)((q.y >> 4) & 0x0F0F0F0Fu)};
}

// 8 activation codes k0..k7 (little-endian in c0, c1) in the order of
// expand_int4: k0 k2 k4 k6 | k1 k3 k5 k7.
__device__ __forceinline__ uint2 act_order_int4(uint32_t c0, uint32_t c1) {
    return make_uint2(__builtin_amdgcn_perm(c1, c0, 0x06040200u), __builtin_amdgcn_perm(c1, c0, 0x07050301u));
}

// Decode unit for M <= MM <= 4 rows, K <= 8192: per-token quantization of
// the bf16 activation rows (Q2) fused in front of the GEMV, one N tile per
// workgroup (used for one row, and for 2..4 rows when K = 8192).  Every workgroup quantizes the row into LDS itself while its
// weight slab is in flight, so the unit is one launch and the int8
// activations never round-trip through HBM.  At one row the redundant
// quantization is cheap, and four independent workgroups per CU keep the
// weight stream smoother than one wide workgroup (12.4 vs 13.0 us at
// K = 4096, N = 16384).  The
// quantizer multiplies by the reciprocal scale (quantize8_bf16) with an exact
// tie decision for the rare value next to a rounding tie, so codes and scales
// are bit-identical to quantize_i8 in every workgroup; workgroup 0 also
// writes them out when asked.
// W4: tiled INT4 weights, half the bytes.  Each lane's 8-byte load becomes
// its MFMA operand with four bitwise ops (expand_int4) against activation
// codes stored in the matching order; the MFMA sums xq * code, and the zero
// point comes off as acc - zp * sum_k xq (exact in int32, the row sums from
// the quantizer); the per-tensor scale replaces the row scales.
template <int MM, bool W4 = false>
__device__ __forceinline__ void linear_decode_row(const LinearDecodeArgs& a, int8_t* xs) {
    __shared__ v4i red[8 * 64];
    __shared__ uint32_t redu[8][MM];
    __shared__ int redi[W4 ? 8 : 1][MM];
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
    const float swn = W4 ? a.w4_scale : n < N ? a.sw[n] : 0.0f;
    const float bn = (a.bias && n < N) ? a.bias[n] : 0.0f;
    constexpr int kTile = W4 ? 512 : 1024;  // bytes per weight tile
    // the head: kSlabHead tiles ahead of the quantizer, W4 too (all 16 of its
    // half-size tiles ahead: 8.4-8.5 vs 8.0-8.2 us at M = 1, K = 4096, and
    // 6.85 vs 6.05 us at K = 8192: more weight reads in flight delay the
    // activations' in the memory queues)
    constexpr int KH = kSlabHead;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.wq + (int64_t)tile * kt * kTile, (uint32_t)kt * kTile);
    uint2 bq[W4 ? kSlab : 1];
    auto load_tile = [&](int s) {
        if constexpr (W4)
            bq[s] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(wr, (wave + s * W) * 512 + lane * 8,
                                                                                  0, 2));
        else
            b[s] = buffer_load16_stream(wr, (wave + s * W) * 1024 + lane * 16);
    };
#pragma unroll
    for (int s = 0; s < KH; ++s) load_tile(s);
    __builtin_amdgcn_sched_barrier(0);

    // 2. row absmax over the workgroup, as the largest bf16 magnitude bit
    //    pattern (a pattern of 0x7f80 or more is an infinity or a NaN);
    //    every thread derives the scales
    float sx[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        const uint32_t mb = wave_max_u32(max(bf16x8_absmax_bits(xv[m][0]), bf16x8_absmax_bits(xv[m][1])));
        if (lane == 0) redu[wave][m] = mb;
    }
    __syncthreads();
    bool nonfinite = false;
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        uint32_t r = redu[0][m];
        for (int i = 1; i < W; ++i) r = max(r, redu[i][m]);
        sx[m] = scale_from_amax(f32_from_bits(r << 16));
        nonfinite |= r >= 0x7f80u;
    }
    if (nonfinite && a.nonfinite && blockIdx.x == 0) report_decode_rows<MM>(a, xv, T);
    // 3. codes into LDS (zeros past K and for rows >= M); W4: each thread's
    //    share of the row sums of the codes
    int rsum[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) rsum[m] = 0;
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
            if constexpr (W4) {
                rsum[m] = __builtin_amdgcn_sdot4((int)code[0], 0x01010101, rsum[m], false);
                rsum[m] = __builtin_amdgcn_sdot4((int)code[1], 0x01010101, rsum[m], false);
                *(uint2*)(xs + m * ldx + c) = act_order_int4(code[0], code[1]);
            } else {
                *(uint2*)(xs + m * ldx + c) = make_uint2(code[0], code[1]);
            }
        }
        if (blockIdx.x == 0 && threadIdx.x == 0 && a.sx_out && m < M) a.sx_out[m] = sx[m];
    }
    if constexpr (W4) {
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            int v = rsum[m];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
            if (lane == 0) redi[wave][m] = v;
        }
    }
    // the rest of the slab: its loads queue behind the head's while the MFMAs wait
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = KH; s < kSlab; ++s) load_tile(s);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    if constexpr (W4) {
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            int v = redi[0][m];
            for (int i = 1; i < W; ++i) v += redi[i][m];
            rsum[m] = v;
        }
    }

    // 4. MFMAs with A from LDS (lanes of rows >= MM read row 0: discarded outputs)
    const int8_t* xrow = xs + ((lane & 15) < MM ? (lane & 15) : 0) * ldx + (lane >> 4) * 16;
    v4i acc = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < kSlab; ++s) {
        if constexpr (W4) b[s] = expand_int4(bq[s]);
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(*(const v4i*)(xrow + (wave + s * W) * 64), b[s], acc, 0, 0, 0);
    }
    if (reduce_waves(acc, red, W) && n < N && (lane >> 4) == 0) {
#pragma unroll
        for (int r = 0; r < MM; ++r)
            if (r < M) {
                const int32_t v = W4 ? acc[r] - a.w4_zp * rsum[r] : acc[r];  // sum xq * (code - zp)
                store_y(a.out, a.out_dtype, (int64_t)r * N + n, v, sx[r], swn, a.bias, bn, a.relu2);
            }
    }
}

// Decode unit, 2 <= M <= MM <= 8, K <= 8192, K % 512 == 0: per-token
// quantization of the bf16 activation rows (Q2) fused in front of the GEMV,
// one launch (a separate quantizer launch costs ~4 us of dependent-launch
// latency on its own).  The quantizer runs in every workgroup, so one
// workgroup owns up to four 16-row N tiles (16 waves): the chip quantizes
// once per CU instead of once per N tile, and its VALU work runs while the
// weight slab is in flight:
//  1. every thread loads its XR 16-byte activation chunks (L2), the epilogue
//     operands, then the first KH KiB of its wave's 16 KiB weight slab (HBM;
//     all of it when the registers allow, else the rest after step 2: half
//     a slab per wave is 128 KiB per CU in flight, enough for its share of
//     HBM bandwidth);
//  2. it waits for the activation loads only (the slab stays in flight),
//     takes the per-row absmax (an LDS max per row), derives the row scales
//     and writes the codes into LDS in the A operand order [KT][4][MM][16];
//  3. the waves run their 16 MFMAs with A from LDS as the slab lands, the
//     K waves of each N tile meet in LDS and the first applies the epilogue.
// Codes and scales are bit-identical to quantize_i8 (quantize8_bf16); the
// first workgroup also writes them out when asked.  K % 512 == 0 keeps each
// wave's 64 consecutive chunks inside one row, so a row's partial max is a
// wave reduction plus one LDS max per wave.
template <int MM, int XR, int KH>
__device__ __forceinline__ void linear_decode_wide(const LinearDecodeArgs& a, int8_t* lds) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int W = a.waves, NTW = a.ntw, NW = W * NTW, T = 64 * NW;
    const int M = a.M, N = a.N, K = a.K, kt = a.kt;
    const int sub = wave / W, kw = wave - sub * W;  // N tile of the workgroup, K wave within it
    const int tile = blockIdx.x * NTW + sub;
    const bool live = tile < (N + 15) / 16;
    const int r16 = lane & 15, g = lane >> 4;
    const int cpr = K >> 3;  // 16-byte chunks per row
    int8_t* xs = lds;                                  // codes, kt * 64 * MM bytes
    v4i* red = (v4i*)(lds + kt * 64 * MM);             // NW * 64 partial tiles
    int* rowmax = (int*)(red + NW * 64);               // MM row absmax (f32 bits)
    if ((int)threadIdx.x < MM) rowmax[threadIdx.x] = 0;

    // 1. activation chunks, epilogue operands, then the weight slab
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, (uint32_t)M * (uint32_t)K * 2u);
    v4i xv[XR];
    v4i b[kSlab];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < XR; ++j) {
        const int c = j * T + (int)threadIdx.x;
        xv[j] = buffer_load16(xrs, c < M * cpr ? c * 16 : kOutOfRange);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int n = tile * 16 + r16;
    const float swn = (live && n < N) ? a.sw[n] : 0.0f;
    const float bn = (a.bias && live && n < N) ? a.bias[n] : 0.0f;
    const __amdgpu_buffer_rsrc_t wr = live ? row_tile_rsrc(a.wq, tile, kt) : make_rsrc(a.wq, 0);
#pragma unroll
    for (int s = 0; s < KH; ++s) b[s] = buffer_load16_stream(wr, (kw + s * W) * 1024 + lane * 16);
    __builtin_amdgcn_sched_barrier(0);

    // 2. activations in (the slab stays in flight); row absmax
    wait_vmcnt_le(KH);
    lds_publish();  // rowmax zeroed
#pragma unroll
    for (int j = 0; j < XR; ++j) {
        const int c0 = j * T + wave * 64;  // the wave's first chunk: uniform
        if (c0 < M * cpr) {
            // the largest magnitude as the f32 bits of the widened bf16
            // (non-negative: int order = value order, non-finite on top)
            const uint32_t mb = wave_max_u32(bf16x8_absmax_bits(xv[j]));
            if (lane == 0) atomicMax(&rowmax[c0 / cpr], (int)(mb << 16));
        }
    }
    lds_publish();
    if (blockIdx.x == 0 && a.nonfinite) {
        bool nonfinite = false;
        for (int r = 0; r < M; ++r) nonfinite |= (uint32_t)rowmax[r] >= 0x7f800000u;
        if (nonfinite) report_decode_chunks<XR>(a, xv, (int)threadIdx.x, T);
    }
    // codes into LDS: chunk c = 8 values of row c / cpr at k = 8 (c % cpr)
#pragma unroll
    for (int j = 0; j < XR; ++j) {
        const int c0 = j * T + wave * 64;
        if (c0 < M * cpr) {
            const int row = c0 / cpr;
            const float sx = scale_from_amax(f32_from_bits((uint32_t)rowmax[row]));
            const float rcp = 1.0f / sx;
            uint32_t code[2];
            quantize8_bf16(xv[j], sx, rcp, scale_is_pow2(sx), code);
            const int k = (c0 + lane - row * cpr) * 8;
            *(uint2*)(xs + (((k >> 6) * 4 + ((k >> 4) & 3)) * MM + row) * 16 + (k & 15)) = make_uint2(code[0], code[1]);
            if (blockIdx.x == 0 && a.xq_out) *(uint2*)(a.xq_out + (int64_t)row * K + k) = make_uint2(code[0], code[1]);
        }
    }
    if (blockIdx.x == 0 && a.sx_out && (int)threadIdx.x < M)
        a.sx_out[threadIdx.x] = scale_from_amax(f32_from_bits((uint32_t)rowmax[threadIdx.x]));
    // the rest of the slab, when its registers had to wait for the activations'
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = KH; s < kSlab; ++s) b[s] = buffer_load16_stream(wr, (kw + s * W) * 1024 + lane * 16);
    __builtin_amdgcn_sched_barrier(0);
    lds_publish();

    // 3. MFMAs with A from LDS as the slab lands (lanes of rows >= MM read
    //    row 0: their outputs are discarded; K tiles past kt meet zero weights)
    const int arow = r16 < MM ? r16 : 0;
    v4i acc = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < kSlab; ++s) {
        const int t = kw + s * W;
        const v4i xa = *(const v4i*)(xs + (((t < kt ? t : 0) * 4 + g) * MM + arow) * 16);
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, b[s], acc, 0, 0, 0);
    }
    if (W > 1) {
        red[wave * 64 + lane] = acc;
        __syncthreads();
        if (kw == 0)
            for (int w = 1; w < W; ++w) acc += red[(wave + w) * 64 + lane];
    }
    if (kw == 0 && live && n < N) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 4 * g + r;
            if (m < M) {
                const float sx = scale_from_amax(f32_from_bits((uint32_t)rowmax[m]));
                store_y(a.out, a.out_dtype, (int64_t)m * N + n, acc[r], sx, swn, a.bias, bn, a.relu2);
            }
        }
    }
}

// Streaming decode unit: up to MM bf16 rows, any N.  Each of G workgroups
// (16 waves, G <= the CU count) owns a contiguous run of N tiles (runs differ
// by at most one tile) and quantizes the activations once for all of them:
//  1. every thread loads its XR chunks of 8 activations (a wave's 64 XR
//     chunks are consecutive, so each of its 64-chunk groups lies in one
//     row), the weight scale and bias of one column of the run, then the
//     first NB rounds of weights: wave w takes K tiles [w KS, w KS + KS) of
//     the round's N tile;
//  2. it waits for the activations only, takes each row's absmax (one DPP
//     wave maximum per row the wave holds, one LDS max), derives the row
//     scales in lanes 0..MM-1 (two divisions per wave), writes the codes into
//     LDS in the A operand order [KT][4][MM][16] and moves the A operands of
//     its K tiles into registers;
//  3. per N tile of the run (a round): KS MFMAs on the landed weights, the
//     partial tile into LDS, the loads of the round two ahead, one barrier,
//     then 16 MM threads sum the 16 partials (int32: exact in any order) and
//     apply the epilogue.  NB rounds of weights stay in flight, under which
//     the quantizer runs: ~6 VALU per value, after activation loads that
//     wait behind the other CUs' weight reads in L2 (2-4 us at 64 KiB per
//     CU, 1.7 us with no weight traffic).
// With row_max (f32 out), each workgroup also leaves the largest finite |y|
// of its outputs per row, from which a consumer derives the rows' scales
// without another pass over y (the MLP's intermediate).
// Every load is unconditional (rounds past the run and K tiles past kt read
// out of range: zeros, no memory traffic), so each wait is a fixed count.
// Codes and scales are bit-identical to quantize_i8 (quantize8_bf16).
template <int MM, int XR, int KS, int NB, bool W4 = false>
__device__ __forceinline__ void linear_decode_stream(const LinearDecodeArgs& a, int8_t* lds) {
    constexpr int NW = 16;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tid = threadIdx.x;
    const int M = a.M, N = a.N, K = a.K, kt = a.kt;
    const int cpr = K >> 3;  // 16-byte chunks per row
    const int tiles = (N + 15) >> 4;
    const int G = gridDim.x;
    const int t0 = (int)(((int64_t)blockIdx.x * tiles) / G);
    const int ntl = (int)(((int64_t)(blockIdx.x + 1) * tiles) / G) - t0;
    const int r16 = lane & 15, g = lane >> 4;
    int8_t* xs = lds;                          // codes, kt * 64 * MM bytes
    v4i* red = (v4i*)(lds + kt * 64 * MM);     // [2][NW][64] partial tiles
    float* swl = (float*)(red + 2 * NW * 64);  // [1024] weight scales of the run
    float* bl = swl + 1024;                    // [1024] bias of the run
    int* rowmax = (int*)(bl + 1024);           // [MM] row absmax (f32 bits)
    float* srow = (float*)(rowmax + MM);       // [MM] row scales
    int* rowsum = (int*)(srow + MM);           // [MM] W4: the rows' code sums
    if (tid < MM) rowmax[tid] = 0;
    if (W4 && tid < MM) rowsum[tid] = 0;
    constexpr int kTile = W4 ? 512 : 1024;  // bytes per weight tile (K tile x 16 columns)

    // 1. activations, epilogue operands, the first PRE rounds of weights
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, (uint32_t)M * (uint32_t)K * 2u);
    const int cbase = wave * XR * 64;  // the wave's first chunk
    v4i xv[XR];
    using WB = std::conditional_t<W4, uint2, v4i>;  // one lane's share of a weight tile
    WB b0[KS], b1[KS], b2[KS], b3[KS];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < XR; ++j) {
        const int c = cbase + j * 64 + lane;
        xv[j] = buffer_load16(xrs, c < M * cpr ? c * 16 : kOutOfRange);
    }
    const uint32_t run_bytes = (uint32_t)min(ntl * 16, N - t0 * 16) * 4u;
    // (W4: one tensor scale, no per-column scales to stage; sw may be null)
    const float swv = f32_from_bits((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
        make_rsrc(W4 ? (const void*)a.wq : (const void*)(a.sw + t0 * 16), W4 ? 0u : run_bytes), tid * 4, 0, 0));
    const float bv = f32_from_bits((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
        make_rsrc(a.bias ? a.bias + t0 * 16 : a.sw, a.bias ? run_bytes : 0u), tid * 4, 0, 0));
    auto issue = [&](WB (&b)[KS], int r) {
        const bool in_run = r < ntl;
        const __amdgpu_buffer_rsrc_t wr =
            make_rsrc(a.wq + (int64_t)(t0 + (in_run ? r : 0)) * kt * kTile, in_run ? (uint32_t)(kt * kTile) : 0u);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            if constexpr (W4)
                b[s] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                                     wr, (wave * KS + s) * 512 + lane * 8, 0, 2));
            else
                b[s] = buffer_load16_stream(wr, (wave * KS + s) * 1024 + lane * 16);
        }
    };
    // Where the weight rounds go relative to the activations (same-box A/B,
    // the 52-layer stack at 8 rows and M = 16 at 4096 -> 16384): at 5..8
    // rows they are issued once this wave's activations have landed (stack
    // 1.727-1.729 against 1.734-1.738 ms: the activation loads otherwise
    // queue behind the whole chip's weight misses); at 9..16 rows every
    // wave's activation loads go out before any weight load (a barrier:
    // 18.51-18.73 against 19.03-19.14 us); at 3..4 rows neither helped.
    constexpr bool kLateWeights = MM == 8, kActFirst = MM == 16;
    if constexpr (kActFirst) lds_barrier();
    if constexpr (!kLateWeights) {
        issue(b0, 0);
        issue(b1, 1);
        if (NB > 2) issue(b2, 2);
        if (NB > 3) issue(b3, 3);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kLateWeights) {
        wait_vmcnt_le(2);  // the activations (the weight scale and bias loads may still fly)
        issue(b0, 0);
        issue(b1, 1);
        if (NB > 2) issue(b2, 2);
        if (NB > 3) issue(b3, 3);
        __builtin_amdgcn_sched_barrier(0);
    }

    // 2. activations in (weights in flight): row absmax, one reduction per
    //    row the wave holds (rows change only where a 64-chunk group starts)
    wait_vmcnt_le(2 + NB * KS);
    lds_publish();  // rowmax zeroed
    {
        uint32_t m = 0;
        int cur = cbase / cpr;
#pragma unroll
        for (int j = 0; j < XR; ++j) {
            const int c0 = cbase + j * 64;  // uniform
            if (c0 < M * cpr) {
                const int row = c0 / cpr;
                if (row != cur) {
                    const uint32_t mb = wave_max_dpp_u32(m);
                    if (lane == 0) atomicMax(&rowmax[cur], (int)(mb << 16));
                    m = 0;
                    cur = row;
                }
                // the largest magnitude as the bits of the widened bf16
                // (non-negative: int order = value order, non-finite on top)
                m = max(m, bf16x8_absmax_bits(xv[j]));
            }
        }
        if (cbase < M * cpr) {
            const uint32_t mb = wave_max_dpp_u32(m);
            if (lane == 0) atomicMax(&rowmax[cur], (int)(mb << 16));
        }
    }
    wait_vmcnt_le(NB * KS);  // weight scales and bias in
    swl[tid] = swv;
    bl[tid] = bv;
    lds_publish();  // row maxima complete
    // row scales in lanes 0..MM-1 of every wave
    const float sx_l = scale_from_amax(f32_from_bits((uint32_t)rowmax[lane < MM ? lane : 0]));
    const float rcp_l = 1.0f / sx_l;
    if (wave == 0 && lane < MM) srow[lane] = sx_l;
    if (blockIdx.x == 0 && a.nonfinite) {
        bool nonfinite = false;
        for (int r = 0; r < M; ++r) nonfinite |= (uint32_t)rowmax[r] >= 0x7f800000u;
        if (nonfinite) report_decode_chunks<XR>(a, xv, cbase + lane, 64);
    }
    // codes into LDS: chunk c = 8 values of row c / cpr at k = 8 (c % cpr);
    // W4: in the nibble order of expand_int4 (act_order_int4), and each row's
    // code sum (zero point, acc - zp * sum_k xq) reduced per row segment
    int csum = 0, crow = cbase / cpr;
    auto flush_sum = [&]() {
        int v = csum;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
        if (lane == 0) atomicAdd(&rowsum[crow], v);
    };
#pragma unroll
    for (int j = 0; j < XR; ++j) {
        const int c0 = cbase + j * 64;
        if (c0 < M * cpr) {
            const int row = c0 / cpr;
            const float sx = f32_from_bits((uint32_t)__builtin_amdgcn_readlane((int)f32_bits(sx_l), row));
            const float rcp = f32_from_bits((uint32_t)__builtin_amdgcn_readlane((int)f32_bits(rcp_l), row));
            uint32_t code[2];
            quantize8_bf16(xv[j], sx, rcp, scale_is_pow2(sx), code);
            const int k = (c0 + lane - row * cpr) * 8;
            uint2 st = make_uint2(code[0], code[1]);
            if constexpr (W4) {
                if (row != crow) {
                    flush_sum();
                    csum = 0;
                    crow = row;
                }
                csum = __builtin_amdgcn_sdot4((int)code[0], 0x01010101, csum, false);
                csum = __builtin_amdgcn_sdot4((int)code[1], 0x01010101, csum, false);
                st = act_order_int4(code[0], code[1]);
            }
            *(uint2*)(xs + (((k >> 6) * 4 + ((k >> 4) & 3)) * MM + row) * 16 + (k & 15)) = st;
            if (blockIdx.x == 0 && a.xq_out) *(uint2*)(a.xq_out + (int64_t)row * K + k) = make_uint2(code[0], code[1]);
        }
    }
    if (W4 && cbase < M * cpr) flush_sum();
    if (blockIdx.x == 0 && a.sx_out && tid < M) a.sx_out[tid] = sx_l;
    lds_publish();  // codes and row scales complete

    // A operands of the wave's K tiles (lanes of rows >= MM read row 0:
    // their outputs are discarded; K tiles past kt meet zero weights)
    const int arow = r16 < MM ? r16 : 0;
    v4i xa[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const int t = wave * KS + s;
        xa[s] = *(const v4i*)(xs + (((t < kt ? t : 0) * 4 + g) * MM + arow) * 16);
    }
    // the epilogue output of thread tid < 16 MM: row tid / 16, column tid % 16
    const int em = tid >> 4, en = tid & 15;
    const float sxe = srow[em < MM ? em : 0];
    const int zsum = W4 ? a.w4_zp * rowsum[em < MM ? em : 0] : 0;  // zp * sum_k xq of the row
    uint32_t ymax = 0;  // largest finite |y| of the thread's outputs (f32 bits)
    auto round = [&](WB (&b)[KS], int r) {
        const int buf = r & 1;
        wait_vmcnt_le((NB - 1) * KS);  // this round's weights in, the next NB - 1 rounds' in flight
        v4i acc = {0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            v4i bw;
            if constexpr (W4)
                bw = expand_int4(b[s]);
            else
                bw = b[s];
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[s], bw, acc, 0, 0, 0);
        }
        red[(buf * NW + wave) * 64 + lane] = acc;
        issue(b, r + NB);
        lds_publish();
        if (tid < 16 * MM && r < ntl) {
            const int n = (t0 + r) * 16 + en;
            if (em < M && n < N) {
                // C[m][n] sits in element m % 4 of lane 16 (m / 4) + n % 16
                const int32_t* rp = (const int32_t*)(red + buf * NW * 64) + (16 * (em >> 2) + en) * 4 + (em & 3);
                int32_t sum = 0;
#pragma unroll
                for (int w = 0; w < NW; ++w) sum += rp[w * 64 * 4];
                // store_y's steps, keeping y for the row maxima
                // W4: sum_k xq * (code - zp), scaled by the tensor scale
                float y = W4 ? epilogue_w8a8(sum - zsum, sxe, a.w4_scale) : epilogue_w8a8(sum, sxe, swl[r * 16 + en]);
                if (a.bias) y = y + bl[r * 16 + en];
                if (a.relu2) y = relu2(y);
                store_out(a.out, (int64_t)em * N + n, y, a.out_dtype);
                if (is_finite_f32(y)) ymax = max(ymax, f32_bits(y) & 0x7fffffffu);
            }
        }
    };
    for (int r = 0; r < ntl; r += NB) {
        round(b0, r);
        round(b1, r + 1);
        if (NB > 2) round(b2, r + 2);
        if (NB > 3) round(b3, r + 3);
    }
    // the workgroup's row maxima: the 16 threads of a row are one DPP row
    if (a.row_max && tid < 16 * MM) {
        ymax = row16_max_u32(ymax);
        if (en == 0 && em < M) a.row_max[(int64_t)blockIdx.x * M + em] = ymax;
    }
    wait_vmcnt_le(0);
}

extern "C" __global__ __launch_bounds__(512) void nh_linear_decode_w8a8_m1_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t xs[];  // [W * 1024 + 16] codes
    linear_decode_row<1>(a, xs);
}

// Rows 2..4 where the wide workgroup would own one N tile anyway (K = 8192:
// 8 K waves per tile): one N tile per workgroup, 12.5 vs 15.2 us at M = 4,
// K = 8192, N = 4096.
extern "C" __global__ __launch_bounds__(512) void nh_linear_decode_w8a8_row2_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t xs[];  // [2][W * 1024 + 16] codes
    linear_decode_row<2>(a, xs);
}

extern "C" __global__ __launch_bounds__(512) void nh_linear_decode_w8a8_row4_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t xs[];  // [4][W * 1024 + 16] codes
    linear_decode_row<4>(a, xs);
}

// The same decode unit on tiled INT4 weights (W4A8): 1, 2 or 4 rows.
extern "C" __global__ __launch_bounds__(512) void nh_linear_decode_w4a8_m1_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t xs[];
    linear_decode_row<1, true>(a, xs);
}

extern "C" __global__ __launch_bounds__(512) void nh_linear_decode_w4a8_row2_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t xs[];
    linear_decode_row<2, true>(a, xs);
}

extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void
nh_linear_decode_w4a8_row4_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t xs[];
    linear_decode_row<4, true>(a, xs);
}

extern "C" __global__ __launch_bounds__(1024) void nh_linear_decode_w8a8_m2_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t lds[];
    linear_decode_wide<2, 4, 12>(a, lds);
}

extern "C" __global__ __launch_bounds__(1024) void nh_linear_decode_w8a8_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t lds[];
    linear_decode_wide<4, 8, 8>(a, lds);
}

extern "C" __global__ __launch_bounds__(1024) void nh_linear_decode_w8a8_m8_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t lds[];
    linear_decode_wide<8, 8, 8>(a, lds);
}

// The streaming unit for 5..8 rows, K <= 4096 (4 K tiles per wave), two
// rounds of weights in flight (three: 16.9 vs 15.6 us at 4096 -> 16384, the
// extra weight reads queue ahead of the activations' in L2).
extern "C" __global__ __launch_bounds__(1024) void nh_linear_decode_stream_m8_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t lds[];
    linear_decode_stream<8, 4, 4, 2>(a, lds);
}

// The same for 3..4 rows (two activation chunks per thread).
extern "C" __global__ __launch_bounds__(1024) void nh_linear_decode_stream_m4_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t lds[];
    linear_decode_stream<4, 2, 4, 2>(a, lds);
}

// The same for 9..16 rows (eight activation chunks per thread).
extern "C" __global__ __launch_bounds__(1024) void nh_linear_decode_stream_m16_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t lds[];
    linear_decode_stream<16, 8, 4, 2>(a, lds);
}

// The streaming unit on tiled INT4 weights (W4A8), 3..4 and 5..8 rows.
extern "C" __global__ __launch_bounds__(1024) void nh_linear_decode_stream_w4_m4_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t lds[];
    linear_decode_stream<4, 2, 4, 2, true>(a, lds);
}

extern "C" __global__ __launch_bounds__(1024) void nh_linear_decode_stream_w4_m8_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t lds[];
    linear_decode_stream<8, 4, 4, 2, true>(a, lds);
}

// And for 9..16 rows (the row-group form took one launch per 4 rows).
extern "C" __global__ __launch_bounds__(1024) void nh_linear_decode_stream_w4_m16_kernel(LinearDecodeArgs a) {
    extern __shared__ __align__(16) int8_t lds[];
    linear_decode_stream<16, 8, 4, 2, true>(a, lds);
}

// G2: W8A32 dequant GEMV, y[m][n] = sum_k x[m][k] * q[n][k] * s[n].  The
// reference materialises W' = (float)q * s and sums x * W' in f64
// (linear.rs:126-131, gemm.rs:99-109).  Here each lane sums the 16 products
// of one 16-code group in f32 (one convert and one FMA per weight), adds the
// group sum to an f64 accumulator, and the row scale multiplies the f64 total
// once: every group sum carries at most 16 f32 roundings, so
// |y - exact| <= 16 u sum_k |x q s| + u |y| to first order (u = 2^-24).
//
// grid = (N tiles, ceil(M / MM)).  A workgroup owns one 16-row weight tile
// over all of K and MM activation rows; wave w takes K tiles w, w + W, ...
// in slabs of 4 whose loads are in flight together.  Lane (r, g) holds code
// row r, codes 16g .. 16g + 15 of a tile, and ONE activation per row and
// tile, x[64t + 16g + r]: the FMA for code e reads lane (e, g)'s activation
// through DPP row_newbcast:e (a 16-lane row is one g), so activations need
// no LDS, no barrier and no per-lane copies.  Loads are issued in the order
// scale, activations, weights, so the compiler's in-order vmcnt accounting
// releases each tile's FMAs as its weight load lands.
constexpr int kSlab32 = 4;

// acc += sum_e x(lane 16 g + e) * w[e] over e = 0..15 in order (f32 FMAs).
// One block: its leading s_nop gives the DPP source the two wait states a
// preceding VALU write would need, and nothing inside writes x.
__device__ __forceinline__ void fma16_row_bcast(float& acc, float x, const float (&w)[16]) {
    asm("s_nop 1\n\t"
        "v_fmac_f32_dpp %0, %1, %2 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %3 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %4 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %5 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %6 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %7 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %8 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %9 row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %10 row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %11 row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %12 row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %13 row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %14 row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %15 row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %16 row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %17 row_newbcast:15 row_mask:0xf bank_mask:0xf"
        : "+v"(acc)
        : "v"(x), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]), "v"(w[8]),
          "v"(w[9]), "v"(w[10]), "v"(w[11]), "v"(w[12]), "v"(w[13]), "v"(w[14]), "v"(w[15]));
}

template <int MM>
__device__ __forceinline__ void gemv_w8a32(const GemvW8A32Args& a) {
    __shared__ double red[16][MM][16];
    const int lane = threadIdx.x & 63, W = a.waves;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int M = a.M, N = a.N, K = a.K, kt = a.kt;
    const int tile = blockIdx.x, m0 = blockIdx.y * MM;
    const int mrows = min(MM, M - m0);
    const __amdgpu_buffer_rsrc_t wr = row_tile_rsrc(a.wq, tile, kt);
    // one resource per activation row: columns past K and rows past M load
    // as zeros, so the padding of the last K tile and K tiles past kt
    // contribute exact zeros and the tile loop needs no branch (a branch
    // around a tile would cost the in-order vmcnt accounting its precision)
    __amdgpu_buffer_rsrc_t xr[MM];
#pragma unroll
    for (int mm = 0; mm < MM; ++mm)
        xr[mm] = make_rsrc(a.x + (int64_t)(m0 + mm) * K, mm < mrows ? (uint32_t)K * 4u : 0u);
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.sw, (uint32_t)N * 4u);
    float s = 0.0f;
    double acc[MM];
#pragma unroll
    for (int mm = 0; mm < MM; ++mm) acc[mm] = 0.0;
    for (int i = 0; i < a.slabs; ++i) {
        float xv[kSlab32][MM];
        v4i b[kSlab32];
        __builtin_amdgcn_sched_barrier(0);
        // the row scale (reloaded per slab: a load pending across the loop
        // edge costs the accounting its precision)
        s = f32_from_bits((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(sr, (tile * 16 + r16) * 4, 0, 0));
#pragma unroll
        for (int st = 0; st < kSlab32; ++st)
#pragma unroll
            for (int mm = 0; mm < MM; ++mm)
                xv[st][mm] = f32_from_bits((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                    xr[mm], ((wave + (i * kSlab32 + st) * W) * 64 + lane) * 4, 0, 0));
#pragma unroll
        for (int st = 0; st < kSlab32; ++st)
            b[st] = buffer_load16_stream(wr, (wave + (i * kSlab32 + st) * W) * 1024 + lane * 16);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int st = 0; st < kSlab32; ++st) {
            float wf[16];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) wf[4 * j + e] = (float)(int8_t)(b[st][j] >> (8 * e));
#pragma unroll
            for (int mm = 0; mm < MM; ++mm) {
                if (mm >= mrows) break;
                float t = 0.0f;
                fma16_row_bcast(t, xv[st][mm], wf);
                acc[mm] += (double)t;
            }
        }
    }
    // the 4 lanes of a weight row (g = 0..3), then the waves in order
#pragma unroll
    for (int mm = 0; mm < MM; ++mm) {
        acc[mm] += __shfl_xor(acc[mm], 16, kWave);
        acc[mm] += __shfl_xor(acc[mm], 32, kWave);
        if (g == 0) red[wave][mm][r16] = acc[mm];
    }
    __syncthreads();
    const int n = tile * 16 + r16;
    if (wave == 0 && g < mrows && n < N) {
        double t = red[0][g][r16];
        for (int w = 1; w < W; ++w) t += red[w][g][r16];
        a.y[(int64_t)(m0 + g) * N + n] = (float)(t * (double)s);
    }
}

extern "C" __global__ __launch_bounds__(1024) void nh_gemv_w8a32_kernel(GemvW8A32Args a) { gemv_w8a32<4>(a); }

extern "C" __global__ __launch_bounds__(1024) void nh_gemv_w8a32_m1_kernel(GemvW8A32Args a) { gemv_w8a32<1>(a); }
