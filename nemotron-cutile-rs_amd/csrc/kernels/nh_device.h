// Device-side helpers for the gfx950 kernels: wavefront reductions and
// vector types.  Wave size is 64 on CDNA4.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nh_kernel_args.h"
#include "nh_numerics.h"

namespace nh {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// A buffer offset past every resource: the load returns zeros without
// touching memory.
constexpr int kOutOfRange = 0x7ffffff0;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

__device__ __forceinline__ int wave_min_i32(int v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = min(v, __shfl_xor(v, off, kWave));
    return v;
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Block-wide max of non-negative floats / min of ints through LDS; every
// thread gets the result.  blockDim.x must be a multiple of 64, <= 1024.
__device__ __forceinline__ float block_max(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_max(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < nw; ++i) r = fmaxf(r, red[i]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ int block_min_i32(int v, int* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_min_i32(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    int r = red[0];
    for (int i = 1; i < nw; ++i) r = min(r, red[i]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int dtype) {
    if (dtype == DT_BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}

__device__ __forceinline__ void store_out(void* p, int64_t i, float v, int dtype) {
    if (dtype == DT_BF16)
        ((uint16_t*)p)[i] = f32_to_bf16(v);
    else
        ((float*)p)[i] = v;
}

__device__ __forceinline__ bool is_finite_f32(float v) { return (f32_bits(v) & 0x7f800000u) != 0x7f800000u; }

// Q2 codes of 8 bf16 values (one 16-byte load: value 2j in the low half of
// word j) with row scale s and r = RN(1/s), packed little-endian into
// code[0..1]: quantize_i8_fast (nh_numerics.h) vectorized, so bit-identical
// to quantize_i8.  pow2 = scale_is_pow2(s) and the zero/subnormal test are
// per row, so those branches are uniform; the exact tie decision runs only
// for a group of 8 that holds a value within 2^-15 of a half-integer.
// Non-finite inputs give unspecified codes.
__device__ __forceinline__ void quantize8_bf16(v4i xv, float s, float r, bool pow2, uint32_t (&code)[2]) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t u = (uint32_t)xv[j];
        v[2 * j] = f32_from_bits(u << 16);
        v[2 * j + 1] = f32_from_bits(u & 0xffff0000u);
    }
    uint32_t q[8];
    if (!(s >= 0x1p-126f)) {
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = (uint32_t)(int)quantize_i8(v[i], s);
    } else if (pow2) {
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = (uint32_t)(int)roundf(v[i] * r);
    } else {
        float dmax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float y = __builtin_fmaf(v[i], r, kQuantMagic);
            dmax = fmaxf(dmax, fabsf(__builtin_fmaf(v[i], r, -(y - kQuantMagic))));
            q[i] = f32_bits(y);  // low byte = the code
        }
        if (dmax >= kQuantTieBand) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float y = __builtin_fmaf(v[i], r, kQuantMagic);
                if (fabsf(__builtin_fmaf(v[i], r, -(y - kQuantMagic))) >= kQuantTieBand)
                    q[i] = (uint32_t)quantize_near_tie(v[i], s, v[i] * r);
            }
        }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t lo = __builtin_amdgcn_perm(q[4 * h + 1], q[4 * h], 0x0c0c0400u);
        const uint32_t hi = __builtin_amdgcn_perm(q[4 * h + 3], q[4 * h + 2], 0x0c0c0400u);
        code[h] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    }
}

// Raw buffer resource over [base, base + bytes): a buffer load whose offset
// falls outside returns zeros instead of touching memory (bytes < 2^31).
// Loads address through one VGPR offset plus a 12-bit immediate, so a run of
// loads at fixed strides needs a single address register.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ v4i buffer_load16(__amdgpu_buffer_rsrc_t r, int offset) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0));
}

// Streaming variant for weights that are read once per launch: the
// non-temporal policy (aux bit 1) keeps them from displacing the activations
// and scales in the caches; measured 6.3 vs 5.7 TB/s on a 64 MiB one-pass read.
__device__ __forceinline__ v4i buffer_load16_stream(__amdgpu_buffer_rsrc_t r, int offset) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 2));
}

}  // namespace nh
