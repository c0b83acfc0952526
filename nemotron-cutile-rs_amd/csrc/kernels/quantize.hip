// Q1/Q2/Q3 and Q0d kernels: symmetric int8 row quantization, int8
// dequantization, affine INT4 dequantization.  HBM-bound elementwise work:
// one workgroup per row for the row quantizer, grid-stride loops for the
// dequantizers and the weight tiler.
#include "nh_device.h"

using namespace nh;

namespace {

// Byte of code (m, k) in the A-operand tiles with P rows per tile (the
// layout comment of QuantizeRowsArgs::act_p).
__device__ __forceinline__ int64_t act_tile_offset(int64_t m, int64_t k, int64_t p, int64_t kt) {
    return (((m / p) * kt + (k >> 6)) * 4 + ((k >> 4) & 3)) * p * 16 + (m % p) * 16 + (k & 15);
}

// Unit (row, or group of `per` rows) of workgroup b when the codes go to the
// GEMM's A tiles (P = 16).  A tile's 128-byte line holds 16 codes of each of
// 8 consecutive rows, and workgroups are dealt round-robin to the 8 XCDs, each
// with its own L2: in identity order the 8 rows of a line went to 8 XCDs, and
// every line reached HBM as 16-byte pieces from 8 caches (2048 x 4096 bf16:
// 13.4 us against 9.6 us for row-major codes).  Here the units of every line
// go to consecutive workgroups of one XCD (the M = 2048, K = 21504 linear
// layer: 186.4-186.8 us against 201.8-202.1).  A bijection on [0, units) when
// units is a multiple of 64 / per; identity otherwise.
__device__ __forceinline__ int64_t xcd_line_order(int64_t b, int64_t units, int per) {
    const int64_t g = 8 / per;  // units per line
    if (units % (8 * g) != 0) return b;
    const int64_t x = b & 7, j = b >> 3;
    return (j / g) * (8 * g) + x * g + (j % g);
}

__device__ __forceinline__ int64_t tile_line_order(const QuantizeRowsArgs& a, int64_t b, int64_t units, int per) {
    if (!a.q_act || a.act_p != 16 || a.gather) return b;
    return xcd_line_order(b, units, per);
}

// The row's first non-finite column (bad < INT_MAX) into the caller's
// non-finite word, as the flat index of the input element.
__device__ __forceinline__ void report_row(const QuantizeRowsArgs& a, int64_t src, int bad) {
    if (a.nonfinite && bad != 0x7fffffff) {
        const int64_t i = src * a.cols + bad;
        report_nonfinite(a.nonfinite, a.nonfinite_stage, i, load_as_f32(a.x, i, a.x_dtype));
    }
}

// Vector path: one workgroup per row, 16-byte chunks (8 bf16 or 4 f32
// values).  The first kRegChunks chunks of every thread stay in registers
// between the absmax pass and the code pass, so rows up to kRegChunks *
// blockDim.x chunks are read from memory once; longer rows read the rest
// again (L2), four chunks in flight per thread.
// Codes go to the row-major matrix and/or the A-operand tiles (act_p rows
// per tile: the compact [KT][4][rows][16] of the M <= 16 GEMV, or 16, the
// weights' tiled layout read by the GEMM).
// COH: the scale and the activation-tile codes are stored as agent-scope
// (sc1) writes, visible to other workgroups of the same launch once the
// stores have completed (the producer half of nh_linear_handoff_kernel).
template <int DT, int kRegChunks, bool COH = false>
__device__ __forceinline__ void quantize_row_vec(const QuantizeRowsArgs& a, float* redf, int* redi) {
    constexpr int VPC = DT == DT_BF16 ? 8 : 4;  // values per 16-byte chunk
    const int64_t row = tile_line_order(a, blockIdx.x, a.rows, 1);
    const int64_t src = a.gather ? a.gather[row] / a.gather_div : row;
    const int cols = (int)a.cols;
    const int chunks = cols / VPC;
    const uint32_t rb = (uint32_t)cols * (DT == DT_BF16 ? 2u : 4u);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc((const char*)a.x + src * (int64_t)rb, rb);
    const int T = blockDim.x;
    v4i xv[kRegChunks];
#pragma unroll
    for (int r = 0; r < kRegChunks; ++r) {
        const int c = threadIdx.x + r * T;
        xv[r] = buffer_load16(xr, c < chunks ? c * 16 : kOutOfRange);
    }
    float amax = 0.0f;
    int bad = 0x7fffffff;
    auto scan = [&](v4i v, int c) {
        float f[VPC];
        if constexpr (DT == DT_BF16) {
            unpack_bf16x8(v, f);
        } else {
#pragma unroll
            for (int j = 0; j < VPC; ++j) f[j] = f32_from_bits((uint32_t)v[j]);
        }
#pragma unroll
        for (int j = 0; j < VPC; ++j) {
            if (!is_finite_f32(f[j])) bad = min(bad, c * VPC + j);
            else amax = fmaxf(amax, fabsf(f[j]));
        }
    };
    // the row: registers, then the tail 4 loads at a time (past the row: zeros)
    auto walk = [&](auto&& f) {
#pragma unroll
        for (int r = 0; r < kRegChunks; ++r) f(xv[r], threadIdx.x + r * T);
        for (int c0 = threadIdx.x + kRegChunks * T; c0 < chunks; c0 += 4 * T) {
            v4i t[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                t[j] = buffer_load16(xr, c0 + j * T < chunks ? (c0 + j * T) * 16 : kOutOfRange);
#pragma unroll
            for (int j = 0; j < 4; ++j) f(t[j], c0 + j * T);
        }
    };
    uint32_t m = 0;
    walk([&](v4i v, int) { m = DT == DT_BF16 ? absbits_bf16x8(v, m) : absbits_f32x4(v, m); });
    m = block_max_u32(DT == DT_BF16 ? absbits_pair_f32(m) : m, redi);
    if (m < kInfBits) {
        amax = f32_from_bits(m);
    } else {  // a non-finite value: the exact scan names the first one
        walk(scan);
        amax = block_max(amax, redf);
        bad = block_min_i32(bad, redi);
    }
    const float s = scale_from_amax(amax);
    if (threadIdx.x == 0) {
        if constexpr (COH)
            __hip_atomic_store((uint32_t*)&a.scales[row], f32_bits(s), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            a.scales[row] = s;
        if (a.row_status) a.row_status[row] = bad == 0x7fffffff ? -1 : bad;
        report_row(a, src, bad);
    }
    const float rcp = s > 0.0f ? 1.0f / s : 0.0f;
    const bool pow2 = scale_is_pow2(s);
    const int64_t kt = (cols + 63) / 64;
    auto emit = [&](v4i v, int c) {
        const int k = c * VPC;
        int8_t* tile = a.q_act ? a.q_act + act_tile_offset(row, k, a.act_p, kt) : nullptr;
        if constexpr (DT == DT_BF16) {
            uint32_t code[2];
            quantize8_bf16(v, s, rcp, pow2, code);
            if (a.q) *(uint2*)(a.q + row * cols + k) = make_uint2(code[0], code[1]);
            if constexpr (COH) {
                if (tile)
                    __hip_atomic_store((uint64_t*)tile, ((uint64_t)code[1] << 32) | code[0], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            } else if (tile) {
                *(uint2*)tile = make_uint2(code[0], code[1]);
            }
        } else {
            const uint32_t code = quantize4_f32(v, s, rcp, pow2);
            if (a.q) *(uint32_t*)(a.q + row * cols + k) = code;
            if (tile) *(uint32_t*)tile = code;
        }
    };
#pragma unroll
    for (int r = 0; r < kRegChunks; ++r) {
        const int c = threadIdx.x + r * T;
        if (c < chunks) emit(xv[r], c);
    }
    for (int c0 = threadIdx.x + kRegChunks * T; c0 < chunks; c0 += 4 * T) {
        v4i t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) t[j] = buffer_load16(xr, c0 + j * T < chunks ? (c0 + j * T) * 16 : kOutOfRange);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (c0 + j * T < chunks) emit(t[j], c0 + j * T);
    }
}

// A wave's row of up to 64 * NCH chunks held in registers (chunks past the
// row read zeros): its finite absmax and first non-finite column (INT_MAX if
// none), wave-uniform.  The bit-pattern scan first; the exact scan only for a
// row with a non-finite value.
template <int DT, int NCH>
__device__ __forceinline__ void row_absmax(const v4i (&xv)[NCH], float& amax, int& bad) {
    constexpr int VPC = DT == DT_BF16 ? 8 : 4;
    const int lane = threadIdx.x & 63;
    uint32_t m = 0;
#pragma unroll
    for (int r = 0; r < NCH; ++r) m = DT == DT_BF16 ? absbits_bf16x8(xv[r], m) : absbits_f32x4(xv[r], m);
    m = wave_max_u32(DT == DT_BF16 ? absbits_pair_f32(m) : m);
    bad = 0x7fffffff;
    if (m < kInfBits) {
        amax = f32_from_bits(m);
        return;
    }
    amax = 0.0f;
#pragma unroll
    for (int r = 0; r < NCH; ++r) {
        float f[VPC];
        if constexpr (DT == DT_BF16) {
            unpack_bf16x8(xv[r], f);
        } else {
#pragma unroll
            for (int j = 0; j < VPC; ++j) f[j] = f32_from_bits((uint32_t)xv[r][j]);
        }
        const int c = lane + r * 64;
#pragma unroll
        for (int j = 0; j < VPC; ++j) {
            if (!is_finite_f32(f[j])) bad = min(bad, c * VPC + j);
            else amax = fmaxf(amax, fabsf(f[j]));
        }
    }
    amax = wave_max(amax);
    bad = wave_min_i32(bad);
}

// Wave path: one wave per row, 4 rows per 256-thread workgroup.  A row of up
// to 64 * NCH 16-byte chunks stays in registers between the absmax and the
// code pass, and both reductions are wave reductions: no barrier, and a row
// costs one round trip to memory.  Same codes and scales as the vector path
// (max and min are exact in any order).
// Its two halves, for a caller with other work to do while the row is in
// flight: the loads (the row this wave owns, or -1 past the last row), then
// the reductions and the code stores.
template <int DT, int NCH>
__device__ __forceinline__ int64_t quantize_row_wave_load(const QuantizeRowsArgs& a, v4i (&xv)[NCH], int64_t row) {
    constexpr int VPC = DT == DT_BF16 ? 8 : 4;
    const int lane = threadIdx.x & 63;
    if (row >= a.rows) return -1;  // the whole wave
    const int64_t src = a.gather ? a.gather[row] / a.gather_div : row;
    const int cols = (int)a.cols;
    const int chunks = cols / VPC;
    const uint32_t rb = (uint32_t)cols * (DT == DT_BF16 ? 2u : 4u);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc((const char*)a.x + src * (int64_t)rb, rb);
#pragma unroll
    for (int r = 0; r < NCH; ++r) {
        const int c = lane + r * 64;
        xv[r] = buffer_load16(xr, c < chunks ? c * 16 : kOutOfRange);
    }
    return row;
}

template <int DT, int NCH>
__device__ __forceinline__ void quantize_row_wave_finish(const QuantizeRowsArgs& a, const v4i (&xv)[NCH],
                                                         int64_t row) {
    constexpr int VPC = DT == DT_BF16 ? 8 : 4;
    const int lane = threadIdx.x & 63;
    const int64_t src = a.gather ? a.gather[row] / a.gather_div : row;
    const int cols = (int)a.cols;
    const int chunks = cols / VPC;
    float amax;
    int bad;
    row_absmax<DT, NCH>(xv, amax, bad);
    const float s = scale_from_amax(amax);
    if (lane == 0) {
        a.scales[row] = s;
        if (a.row_status) a.row_status[row] = bad == 0x7fffffff ? -1 : bad;
        report_row(a, src, bad);
    }
    const float rcp = s > 0.0f ? 1.0f / s : 0.0f;
    const bool pow2 = scale_is_pow2(s);
    const int64_t kt = (cols + 63) / 64;
#pragma unroll
    for (int r = 0; r < NCH; ++r) {
        const int c = lane + r * 64;
        if (c >= chunks) break;
        const int k = c * VPC;
        int8_t* tile = a.q_act ? a.q_act + act_tile_offset(row, k, a.act_p, kt) : nullptr;
        if constexpr (DT == DT_BF16) {
            uint32_t code[2];
            quantize8_bf16(xv[r], s, rcp, pow2, code);
            if (a.q) *(uint2*)(a.q + row * cols + k) = make_uint2(code[0], code[1]);
            if (tile) *(uint2*)tile = make_uint2(code[0], code[1]);
        } else {
            const uint32_t code = quantize4_f32(xv[r], s, rcp, pow2);
            if (a.q) *(uint32_t*)(a.q + row * cols + k) = code;
            if (tile) *(uint32_t*)tile = code;
        }
    }
}

template <int DT, int NCH>
__device__ __forceinline__ void quantize_row_wave(const QuantizeRowsArgs& a) {
    v4i xv[NCH];
    // (wave-uniform as the compiler sees it, so the row's buffer resource
    // sits in SGPRs and each load is one instruction)
    // (identity order: the line grouping of tile_line_order measured 1 us
    // slower here at 2048 x 4096, with 4 rows per workgroup)
    const int64_t row = quantize_row_wave_load<DT, NCH>(
        a, xv, (int64_t)blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)));
    if (row >= 0) quantize_row_wave_finish<DT, NCH>(a, xv, row);
}

// Rows into the GEMM's A tiles (act_p = 16) for many rows: 8 rows per
// workgroup, one wave per row.  A tile's 128-byte line holds 16 codes of each
// of 8 consecutive rows, so the workgroup owns whole lines: every wave
// quantizes its row into an LDS image of the 8 rows' lines, then the
// workgroup writes the lines with 16-byte stores, 8 lanes per line and 8
// lines per wave instruction (a wave storing its own row's 8-byte pieces puts
// 32 lines' pieces in every store instruction).  The row (up to 64 * NCH
// 16-byte chunks) stays in registers between the absmax and the code pass.
// Same codes, scales and non-finite reports as the vector path.
template <int DT, int NCH>
__device__ __forceinline__ void quantize_tiles(const QuantizeRowsArgs& a, int8_t* lds) {
    constexpr int VPC = DT == DT_BF16 ? 8 : 4;  // values (and codes) per 16-byte chunk
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t r0 = (int64_t)blockIdx.x * 8;
    const int64_t row = r0 + w;
    const int cols = (int)a.cols, chunks = cols / VPC;
    const int kt = (cols + 63) / 64;
    if (row < a.rows) {  // wave-uniform; a row past the matrix leaves its LDS slots to padding rows
        const uint32_t rbytes = (uint32_t)cols * (DT == DT_BF16 ? 2u : 4u);
        const __amdgpu_buffer_rsrc_t xr = make_rsrc((const char*)a.x + row * (int64_t)rbytes, rbytes);
        v4i xv[NCH];
#pragma unroll
        for (int r = 0; r < NCH; ++r) {
            const int c = lane + r * 64;
            xv[r] = buffer_load16(xr, c < chunks ? c * 16 : kOutOfRange);
        }
        float amax;
        int bad;
        row_absmax<DT, NCH>(xv, amax, bad);
        const float s = scale_from_amax(amax);
        if (lane == 0) {
            a.scales[row] = s;
            if (a.row_status) a.row_status[row] = bad == 0x7fffffff ? -1 : bad;
            report_row(a, row, bad);
        }
        const float rcp = s > 0.0f ? 1.0f / s : 0.0f;
        const bool pow2 = scale_is_pow2(s);
#pragma unroll
        for (int r = 0; r < NCH; ++r) {
            const int c = lane + r * 64;
            if (c >= chunks) break;
            const int k = c * VPC;
            const int off = (((k >> 6) * 4 + ((k >> 4) & 3)) * 8 + w) * 16 + (k & 15);  // line (K tile, group)
            if constexpr (DT == DT_BF16) {
                uint32_t code[2];
                quantize8_bf16(xv[r], s, rcp, pow2, code);
                *(uint2*)(lds + off) = make_uint2(code[0], code[1]);
                if (a.q) *(uint2*)(a.q + row * cols + k) = make_uint2(code[0], code[1]);
            } else {
                const uint32_t code = quantize4_f32(xv[r], s, rcp, pow2);
                *(uint32_t*)(lds + off) = code;
                if (a.q) *(uint32_t*)(a.q + row * cols + k) = code;
            }
        }
    }
    __syncthreads();
    // line (K tile t, group g) of this 8-row half of a 16-row block
    int8_t* dst = a.q_act + (r0 >> 4) * (int64_t)kt * 1024 + ((r0 >> 3) & 1) * 128;
    const int p = (int)(threadIdx.x & 7) * 16;
    for (int l = (int)(threadIdx.x >> 3); l < kt * 4; l += (int)(blockDim.x >> 3))
        *(v4i*)(dst + (int64_t)(l >> 2) * 1024 + (l & 3) * 256 + p) = *(const v4i*)(lds + l * 128 + p);
}

// Scalar path (any alignment, any column count): pass 1 = absmax + first
// non-finite column, pass 2 = codes; the row stays in L2 between the passes.
__device__ __forceinline__ void quantize_row_scalar(const QuantizeRowsArgs& a, float* redf, int* redi) {
    const int64_t row = blockIdx.x;
    const int64_t cols = a.cols;
    const int64_t src = a.gather ? a.gather[row] / a.gather_div : row;
    const int64_t base = src * cols;  // input row
    float amax = 0.0f;
    int bad = 0x7fffffff;
    for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
        const float v = load_as_f32(a.x, base + c, a.x_dtype);
        if (!is_finite_f32(v)) bad = min(bad, (int)c);
        else amax = fmaxf(amax, fabsf(v));
    }
    amax = block_max(amax, redf);
    bad = block_min_i32(bad, redi);
    const float s = scale_from_amax(amax);
    if (threadIdx.x == 0) {
        a.scales[row] = s;
        if (a.row_status) a.row_status[row] = bad == 0x7fffffff ? -1 : bad;
        report_row(a, src, bad);
    }
    const float r = s > 0.0f ? 1.0f / s : 0.0f;
    for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
        const int8_t code = (int8_t)quantize_i8_fast(load_as_f32(a.x, base + c, a.x_dtype), s, r);
        if (a.q) a.q[row * cols + c] = code;
        if (a.q_act) a.q_act[act_tile_offset(row, c, a.act_p, (cols + 63) / 64)] = code;
    }
}

}  // namespace

// Q1/Q2: one workgroup per row; codes bit-identical to quantize_i8 (the
// reference's division) without dividing (quantize_i8_fast).  With a gather
// list the output rows are input rows gather[r] / gather_div (the MoE's
// routes in expert order: each route's codes and scale are its token's).
extern "C" __global__ __launch_bounds__(256) void nh_quantize_rows_i8_kernel(QuantizeRowsArgs a) {
    __shared__ float redf[16];
    __shared__ int redi[16];
    if ((int64_t)blockIdx.x >= a.rows) return;
    if (!a.vec)
        quantize_row_scalar(a, redf, redi);
    else if (a.x_dtype == DT_BF16)
        quantize_row_vec<DT_BF16, 4>(a, redf, redi);
    else
        quantize_row_vec<DT_F32, 4>(a, redf, redi);
}

// The vector path for many rows of 1025..2816 16-byte chunks (the M = 2048
// linear layer's 21504-wide bf16 rows): a 256-thread workgroup per row holds
// the whole row, 11 chunks per thread, so each row is read once (the kernel
// above reads the chunks past its first 1024 twice, once per pass).  116
// registers, 4 workgroups per CU: 2048 x 21504 bf16 rows as the GEMM's A tiles
// in 3 us less than with 4 chunks per thread (171.4 against 174.4 us for the
// linear layer, three alternating runs on one box).
extern "C" __global__ __launch_bounds__(256) void nh_quantize_rows_r11_kernel(QuantizeRowsArgs a) {
    __shared__ float redf[16];
    __shared__ int redi[16];
    if ((int64_t)blockIdx.x >= a.rows) return;
    if (a.x_dtype == DT_BF16)
        quantize_row_vec<DT_BF16, 11>(a, redf, redi);
    else
        quantize_row_vec<DT_F32, 11>(a, redf, redi);
}

// The vector path for a few long rows (the decode batch's activations): 1024
// threads per row, 8 chunks each in registers, so a row of up to 8192 chunks
// (the MLP's 21504-wide f32 intermediate is 5376) costs one round trip to
// memory instead of one per 1024 chunks.
extern "C" __global__ __launch_bounds__(1024) void nh_quantize_rows_long_kernel(QuantizeRowsArgs a) {
    __shared__ float redf[16];
    __shared__ int redi[16];
    if ((int64_t)blockIdx.x >= a.rows) return;
    if (a.x_dtype == DT_BF16)
        quantize_row_vec<DT_BF16, 8>(a, redf, redi);
    else
        quantize_row_vec<DT_F32, 8>(a, redf, redi);
}

// Q2 of f32 rows whose finite absolute maxima a producer already reduced
// per workgroup (the streaming decode unit's row_max): every wave takes the
// row's maximum over the `groups` partial maxima (max is exact in any order,
// so the scale is quantize_rows' scale), then each thread quantizes one
// 16-byte chunk into the A-operand tiles.  No block-wide reduction, so a row
// spreads over many workgroups: grid = (ceil(cols / 1024), rows), 256
// threads.  Non-finite values are reported as by the row quantizer (the
// smallest flat index wins).
extern "C" __global__ __launch_bounds__(256) void nh_quantize_rows_pmax_kernel(QuantizePmaxArgs a) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.y;
    const int chunks = a.cols >> 2;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    // the chunk first (out of range past the row: zeros, no traffic), so
    // its round trip overlaps the partial maxima's
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x + (int64_t)row * a.cols, (uint32_t)a.cols * 4u);
    const v4i v = buffer_load16(xr, c < chunks ? c * 16 : kOutOfRange);
    // the partial maxima, 4 per lane in flight at once (up to 256 groups
    // in one round trip; a loop of dependent loads took one per 64 groups)
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.pmax, (uint32_t)a.groups * (uint32_t)a.rows * 4u);
    uint32_t m = 0;
    for (int g0 = 0; g0 < a.groups; g0 += 256) {
        uint32_t pm[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int g = g0 + lane + 64 * i;
            pm[i] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                pr, g < a.groups ? (g * a.rows + row) * 4 : kOutOfRange, 0, 0);
        }
        m = max(m, max(max(pm[0], pm[1]), max(pm[2], pm[3])));
    }
    m = wave_max_dpp_u32(m);
    const float s = scale_from_amax(f32_from_bits(m));
    if (blockIdx.x == 0 && threadIdx.x == 0) a.scales[row] = s;
    const float rcp = s > 0.0f ? 1.0f / s : 0.0f;
    const bool pow2 = scale_is_pow2(s);
    if (c >= chunks) return;
    if (a.nonfinite) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float f = f32_from_bits((uint32_t)v[j]);
            if (!is_finite_f32(f)) {
                report_nonfinite(a.nonfinite, a.nonfinite_stage, (int64_t)row * a.cols + c * 4 + j, f);
                break;
            }
        }
    }
    const int64_t kt = (a.cols + 63) / 64;
    *(uint32_t*)(a.q_act + act_tile_offset(row, c * 4, a.rows, kt)) = quantize4_f32(v, s, rcp, pow2);
}

// Tiled INT4 -> tiled int8 (code - zp).  INT4 lane l's 8 bytes hold the 16
// codes of int8 lane l in nibble pairs (byte j: column 2 j low, 2 j + 1
// high), so each lane expands in place of layout: two byte permutes
// interleave the low and high nibbles, and code - zp is formed per byte
// without borrows as ((v | 0x80) - zp) ^ 0x80 (v, zp in 0..15).  Padding
// nibbles hold the zero point, so they expand to the int8 layout's zeros.
extern "C" __global__ __launch_bounds__(256) void nh_expand_int4_tiles_kernel(ExpandInt4Args a) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const uint32_t zpw = (uint32_t)a.zp * 0x01010101u;
    auto expand = [&](uint32_t w, uint32_t& w0, uint32_t& w1) {
        const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
        w0 = ((__builtin_amdgcn_perm(hi, lo, 0x05010400u) | 0x80808080u) - zpw) ^ 0x80808080u;
        w1 = ((__builtin_amdgcn_perm(hi, lo, 0x07030602u) | 0x80808080u) - zpw) ^ 0x80808080u;
    };
    for (int64_t l = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; l < a.lanes; l += stride) {
        const uint2 q = ((const uint2*)a.w4)[l];
        uint4 o;
        expand(q.x, o.x, o.y);
        expand(q.y, o.z, o.w);
        ((uint4*)a.w8)[l] = o;
    }
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += stride) a.sw[i] = a.scale;
}

// Q1/Q2 for vector-path rows of up to 512 16-byte chunks (4096 bf16 / 2048
// f32 values): one wave per row (quantize_row_wave), grid = ceil(rows / 4).
extern "C" __global__ __launch_bounds__(256) void nh_quantize_rows_wave_kernel(QuantizeRowsArgs a) {
    if (a.x_dtype == DT_BF16)
        quantize_row_wave<DT_BF16, 8>(a);
    else
        quantize_row_wave<DT_F32, 8>(a);
}

// Q2 into the GEMM's A tiles (act_p = 16, no gather) for rows of up to
// 8 * 64 chunks (bf16 K <= 4096, f32 K <= 2048): grid = ceil(rows / 8), 512
// threads, dynamic LDS 8 * 64 * KT bytes.
extern "C" __global__ __launch_bounds__(512) void nh_quantize_tiles_kernel(QuantizeRowsArgs a) {
    extern __shared__ __align__(16) int8_t lds[];
    if (a.x_dtype == DT_BF16)
        quantize_tiles<DT_BF16, 8>(a, lds);
    else
        quantize_tiles<DT_F32, 8>(a, lds);
}

// Diagnostic: one read of [src, src + bytes) in 16-byte non-temporal loads,
// four per thread in flight, the contiguous KiB per wave instruction of the
// weight streams; the XOR of everything read decides a store that never
// happens for real data (it keeps the loads).  The floor the HBM-bound
// kernels are compared with.
extern "C" __global__ __launch_bounds__(256) void nh_stream_read_kernel(StreamReadArgs a) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(a.src, a.bytes);
    const uint32_t per = gridDim.x * blockDim.x * 16u;  // bytes per round of one load per thread
    const uint32_t base = blockIdx.x * blockDim.x * 16u + threadIdx.x * 16u;
    int acc = 0;
    for (uint32_t o = base; o < a.bytes; o += 4 * per) {
        v4i v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = buffer_load16_stream(r, (int)(o + i * per < a.bytes ? o + i * per : kOutOfRange));
#pragma unroll
        for (int i = 0; i < 4; ++i) acc ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
    }
    if (acc == 0x5a17c0de) a.sink[threadIdx.x] = acc;
}

// INT4 [K][N] codes, low nibble first (the reference's packed layout) -> the
// tiled INT4 layout (nh_numerics.h): thread c writes the 8 bytes of lane
// c % 64 of tile c / 64, the zero point outside the matrix.  A one-off
// repack: the reads gather nibbles N apart.
extern "C" __global__ __launch_bounds__(256) void nh_tile_weights_int4_kernel(TileInt4Args a) {
    for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < a.lanes;
         c += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = c >> 6;
        const int lane = (int)(c & 63);
        const int64_t n = (t / a.kt) * 16 + (lane & 15);
        const int64_t k0 = (t % a.kt) * 64 + (lane >> 4) * 16;
        uint32_t w[2] = {0, 0};
        for (int j = 0; j < 16; ++j) {
            uint32_t code = (uint32_t)a.zp;
            if (n < a.n && k0 + j < a.k) {
                const int64_t i = (k0 + j) * a.n + n;
                code = (a.packed[i >> 1] >> ((i & 1) * 4)) & 15u;
            }
            w[j >> 3] |= code << ((j & 7) * 4);
        }
        *(uint2*)(a.tiled + c * 8) = make_uint2(w[0], w[1]);
    }
}

// Row-major int8 [rows][cols] -> the tiled layout (nh_numerics.h): thread c
// writes 16-byte chunk c of the tiled buffer (lane c % 64 of tile c / 64),
// zeros outside the matrix.
extern "C" __global__ __launch_bounds__(256) void nh_tile_weights_kernel(TileWeightsArgs a) {
    for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < a.chunks;
         c += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = c >> 6;
        const int lane = (int)(c & 63);
        const int64_t row = (t / a.kt) * 16 + (lane & 15);
        const int64_t k0 = (t % a.kt) * 64 + (lane >> 4) * 16;
        v4i v = {0, 0, 0, 0};
        if (row < a.rows && k0 < a.cols) {
            const int8_t* src = a.w + row * a.cols + k0;
            if (k0 + 16 <= a.cols && ((uintptr_t)src & 15) == 0) {
                v = *(const v4i*)src;
            } else {
                uint8_t bytes[16];
                for (int b = 0; b < 16; ++b) bytes[b] = k0 + b < a.cols ? (uint8_t)src[b] : 0;
                for (int j = 0; j < 4; ++j)
                    v[j] = (int)(bytes[4 * j] | (bytes[4 * j + 1] << 8) | (bytes[4 * j + 2] << 16) |
                                 ((uint32_t)bytes[4 * j + 3] << 24));
            }
        }
        *(v4i*)(a.tiled + c * 16) = v;
    }
}

// The dequantizers write four f32 bytes per code byte (or per nibble), so
// they are bound by their stores.  With 16-byte aligned output (and, for
// int8, rows of whole 4-code chunks) a thread takes 4 codes: one 4-byte (or
// 2-byte) load and one 16-byte store, so a wave's store covers 1 KiB of
// consecutive whole cache lines.  Other layouts take one code per thread.
typedef float v4f __attribute__((ext_vector_type(4)));

extern "C" __global__ __launch_bounds__(256) void nh_dequantize_i8_kernel(DequantizeI8Args a) {
    const int64_t total = a.rows * a.cols;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    if (a.cols % 4 == 0 && ((((uintptr_t)a.q & 3) | ((uintptr_t)a.out & 15)) == 0)) {
        const int64_t chunks = total >> 2, cpr = a.cols >> 2;
        for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < chunks; c += stride) {
            const int64_t r = c < 0xffffffffll && cpr < 0xffffffffll ? (int64_t)((uint32_t)c / (uint32_t)cpr)
                                                                   : c / cpr;
            const float s = a.scales[r];
            const uint32_t b = *(const uint32_t*)(a.q + (c << 2));
            const v4f v = {(float)(int8_t)(b & 0xff) * s, (float)(int8_t)((b >> 8) & 0xff) * s,
                           (float)(int8_t)((b >> 16) & 0xff) * s, (float)(int8_t)(b >> 24) * s};
            *(v4f*)(a.out + (c << 2)) = v;
        }
        return;
    }
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t r = i / a.cols;
        a.out[i] = (float)a.q[i] * a.scales[r];
    }
}

// (code - zero_point) * scale straight from the packed nibbles (low nibble
// first, quantize.rs:75-77 and :110-116); the reference unpacked on the host
// and uploaded one f32 per code (quantize.rs:294-301).
extern "C" __global__ __launch_bounds__(256) void nh_dequantize_int4_kernel(DequantizeInt4Args a) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t done = 0;  // codes covered by whole 4-code chunks
    if ((((uintptr_t)a.packed & 1) | ((uintptr_t)a.out & 15)) == 0) {
        const int64_t chunks = a.value_count >> 2;
        for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < chunks; c += stride) {
            const uint32_t b = *(const uint16_t*)(a.packed + (c << 1));
            const v4f v = {((float)(b & 0x0F) - a.zero_point) * a.scale,
                           ((float)((b >> 4) & 0x0F) - a.zero_point) * a.scale,
                           ((float)((b >> 8) & 0x0F) - a.zero_point) * a.scale,
                           ((float)((b >> 12) & 0x0F) - a.zero_point) * a.scale};
            *(v4f*)(a.out + (c << 2)) = v;
        }
        done = chunks << 2;
    }
    for (int64_t i = done + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.value_count; i += stride) {
        const uint8_t byte = a.packed[i >> 1];
        const uint32_t code = (i & 1) ? ((byte >> 4) & 0x0F) : (byte & 0x0F);
        a.out[i] = ((float)code - a.zero_point) * a.scale;
    }
}
