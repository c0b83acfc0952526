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

__device__ __forceinline__ uint32_t wave_max_dpp_u32(uint32_t v);
__device__ __forceinline__ int wave_min_dpp_i32(int v);

// Wave maximum of non-negative floats (their bits order like the values).
__device__ __forceinline__ float wave_max(float v) { return f32_from_bits(wave_max_dpp_u32(f32_bits(v))); }

__device__ __forceinline__ int wave_min_i32(int v) { return wave_min_dpp_i32(v); }

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

__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, int* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_max_dpp_u32(v);
    if (lane == 0) red[wave] = (int)v;
    __syncthreads();
    uint32_t r = (uint32_t)red[0];
    for (int i = 1; i < nw; ++i) r = max(r, (uint32_t)red[i]);
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

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) { return wave_max_dpp_u32(v); }

// The same maximum through DPP lane moves (no LDS round trips): within rows
// of 16 lanes by quad permutes and row rotates, then across rows by the
// row broadcasts of lanes 15 and 31; lane 63 ends with the wave's maximum,
// which readlane hands to every lane.  Lanes a DPP move leaves out keep
// their own value, which a maximum absorbs.
__device__ __forceinline__ uint32_t wave_max_dpp_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xb1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4e, 0xf, 0xf, false));   // quad_perm 2,3,0,1
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x124, 0xf, 0xf, false));  // row_ror 4
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x128, 0xf, 0xf, false));  // row_ror 8
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xa, 0xf, false));  // row_bcast 15
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xc, 0xf, false));  // row_bcast 31
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// The wave minimum of ints, by the same lane moves.
__device__ __forceinline__ int wave_min_dpp_i32(int v) {
    v = min(v, __builtin_amdgcn_update_dpp(v, v, 0xb1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
    v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x4e, 0xf, 0xf, false));   // quad_perm 2,3,0,1
    v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x124, 0xf, 0xf, false));  // row_ror 4
    v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x128, 0xf, 0xf, false));  // row_ror 8
    v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x142, 0xa, 0xf, false));  // row_bcast 15
    v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x143, 0xc, 0xf, false));  // row_bcast 31
    return __builtin_amdgcn_readlane(v, 63);
}

// Maximum over each row of 16 lanes (every lane of the row gets it).
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x128, 0xf, 0xf, false));  // row_ror 8
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x124, 0xf, 0xf, false));  // row_ror 4
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x122, 0xf, 0xf, false));  // row_ror 2
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x121, 0xf, 0xf, false));  // row_ror 1
    return v;
}

// NonFiniteInput (quantize.rs:193-195: the first offending element and its
// value) from the device quantizers.  The key goes into the caller's 64-bit
// word as its complement through an atomic max, so the word keeps the
// smallest key (the lowest NonFiniteStage, then the lowest row-major index)
// and a zeroed word means that nothing was found:
//   bits 62..63  the stage (NonFiniteStage)
//   bits 24..61  the flat index (38 bits: every index the device envelope allows)
//   bit  23      the value's sign
//   bits  0..22  the value's mantissa (its exponent is all ones: NaN or infinity)
// nh_take_nonfinite decodes it.  Vector atomic only.
__device__ __forceinline__ void report_nonfinite(uint64_t* word, int stage, int64_t index, float value) {
    const uint32_t b = f32_bits(value);
    const uint64_t key = ((uint64_t)(stage & 3) << 62) | (((uint64_t)index & ((1ull << 38) - 1)) << 24) |
                         (uint64_t)((b >> 8) & 0x800000u) | (uint64_t)(b & 0x7fffffu);
    atomicMax((unsigned long long*)word, (unsigned long long)~key);
}

typedef unsigned short nh_u16x2 __attribute__((ext_vector_type(2)));

// Two f32 values to bf16 in one v_cvt_pk_bf16_f32 (gfx950), lo in the low
// half.  Bit-identical to f32_to_bf16 (round to nearest even, a NaN kept
// with its quiet bit set) on all 2^32 inputs, checked exhaustively on the
// device.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
    typedef __bf16 nh_bf16x2 __attribute__((ext_vector_type(2)));
    typedef float nh_f32x2 __attribute__((ext_vector_type(2)));
    const nh_f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, nh_bf16x2));
}

// Largest bf16 magnitude of the 8 values of one 16-byte load, as its 15-bit
// pattern (sign cleared).  Magnitude bit patterns order like the values, and
// infinities and NaNs (0x7f80 and above) order above every finite value, so
// a row's maximum pattern is its absmax and also shows a non-finite element.
// Three packed 16-bit maxima per load.
__device__ __forceinline__ uint32_t bf16x8_absmax_bits(v4i xv) {
    nh_u16x2 m = __builtin_bit_cast(nh_u16x2, (uint32_t)xv[0] & 0x7fff7fffu);
#pragma unroll
    for (int j = 1; j < 4; ++j)
        m = __builtin_elementwise_max(m, __builtin_bit_cast(nh_u16x2, (uint32_t)xv[j] & 0x7fff7fffu));
    return max((uint32_t)m.x, (uint32_t)m.y);
}

// The row quantizers' absmax scan on bit patterns (as above): one integer
// maximum per value (per bf16 pair) gives a row's absmax, or says that the
// row holds a non-finite value, and only then does a quantizer run the exact
// scan that finds the first one.
constexpr uint32_t kInfBits = 0x7f800000u;

// m: two running maxima of bf16 patterns; the pair updated with 8 values.
__device__ __forceinline__ uint32_t absbits_bf16x8(v4i v, uint32_t m) {
    nh_u16x2 acc = __builtin_bit_cast(nh_u16x2, m);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        acc = __builtin_elementwise_max(acc, __builtin_bit_cast(nh_u16x2, (uint32_t)v[j] & 0x7fff7fffu));
    return __builtin_bit_cast(uint32_t, acc);
}

// The f32 pattern of the larger bf16 pattern of a pair.
__device__ __forceinline__ uint32_t absbits_pair_f32(uint32_t m) { return max(m & 0xffffu, m >> 16) << 16; }

__device__ __forceinline__ uint32_t absbits_f32x4(v4i v, uint32_t m) {
#pragma unroll
    for (int j = 0; j < 4; ++j) m = max(m, (uint32_t)v[j] & 0x7fffffffu);
    return m;
}

// Index (0..7) of the first non-finite value of a 16-byte bf16 load, or 8.
__device__ __forceinline__ int bf16x8_first_nonfinite(v4i xv) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t h = ((uint32_t)xv[e >> 1] >> (16 * (e & 1))) & 0x7fffu;
        if (h >= 0x7f80u) return e;
    }
    return 8;
}

// Codes of NV values with row scale s and r = RN(1/s): quantize_i8_fast
// (nh_numerics.h) vectorized, so bit-identical to quantize_i8; q[i]'s low
// byte is the code.  pow2 = scale_is_pow2(s) and the zero/subnormal test are
// per row, so those branches are uniform; the exact tie decision runs only
// for a group that holds a value within 2^-15 of a half-integer.  Non-finite
// inputs give unspecified codes (the row is reported as non-finite instead).
template <int NV>
__device__ __forceinline__ void quantize_values(const float (&v)[NV], float s, float r, bool pow2, uint32_t (&q)[NV]) {
    if (!(s >= 0x1p-126f)) {
#pragma unroll
        for (int i = 0; i < NV; ++i) q[i] = (uint32_t)(int)quantize_i8(v[i], s);
    } else if (pow2) {
#pragma unroll
        for (int i = 0; i < NV; ++i) q[i] = (uint32_t)(int)roundf(v[i] * r);
    } else {
        float dmax = 0.0f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const float y = __builtin_fmaf(v[i], r, kQuantMagic);
            dmax = fmaxf(dmax, fabsf(__builtin_fmaf(v[i], r, -(y - kQuantMagic))));
            q[i] = f32_bits(y);  // low byte = the code
        }
        if (dmax >= kQuantTieBand) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const float y = __builtin_fmaf(v[i], r, kQuantMagic);
                if (fabsf(__builtin_fmaf(v[i], r, -(y - kQuantMagic))) >= kQuantTieBand)
                    q[i] = (uint32_t)quantize_near_tie(v[i], s, v[i] * r);
            }
        }
    }
}

// The low bytes of q[0..3] as one little-endian word.
__device__ __forceinline__ uint32_t pack_codes4(uint32_t q0, uint32_t q1, uint32_t q2, uint32_t q3) {
    const uint32_t lo = __builtin_amdgcn_perm(q1, q0, 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(q3, q2, 0x0c0c0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// The 8 bf16 values of one 16-byte load (value 2j in the low half of word j).
__device__ __forceinline__ void unpack_bf16x8(v4i xv, float (&v)[8]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t u = (uint32_t)xv[j];
        v[2 * j] = f32_from_bits(u << 16);
        v[2 * j + 1] = f32_from_bits(u & 0xffff0000u);
    }
}

// Codes of 8 bf16 values (one 16-byte load), packed into code[0..1].
__device__ __forceinline__ void quantize8_bf16(v4i xv, float s, float r, bool pow2, uint32_t (&code)[2]) {
    float v[8];
    unpack_bf16x8(xv, v);
    uint32_t q[8];
    quantize_values<8>(v, s, r, pow2, q);
    code[0] = pack_codes4(q[0], q[1], q[2], q[3]);
    code[1] = pack_codes4(q[4], q[5], q[6], q[7]);
}

// Codes of 4 f32 values (one 16-byte load), packed into one word.
__device__ __forceinline__ uint32_t quantize4_f32(v4i xv, float s, float r, bool pow2) {
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = f32_from_bits((uint32_t)xv[j]);
    uint32_t q[4];
    quantize_values<4>(v, s, r, pow2, q);
    return pack_codes4(q[0], q[1], q[2], q[3]);
}

// LDS destination of the direct-to-LDS buffer loads.
typedef __attribute__((address_space(3))) void lds_void_t;

// s_waitcnt vmcnt(<= n) with the other counters left alone (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] = 7 | lgkmcnt[11:8] = 15 | vmcnt[5:4] << 14).
// The wait is an immediate, hence the switch over every count (0..63).
__device__ __forceinline__ void wait_vmcnt_le(int n) {
#define NH_VMCNT(n) ((((n) & 15) | (7 << 4) | (15 << 8) | ((((n) >> 4) & 3) << 14)))
#define NH_VMCNT_CASE(n) \
    case n: __builtin_amdgcn_s_waitcnt(NH_VMCNT(n)); break;
#define NH_VMCNT_CASE8(n) NH_VMCNT_CASE(n) NH_VMCNT_CASE(n + 1) NH_VMCNT_CASE(n + 2) NH_VMCNT_CASE(n + 3) \
    NH_VMCNT_CASE(n + 4) NH_VMCNT_CASE(n + 5) NH_VMCNT_CASE(n + 6) NH_VMCNT_CASE(n + 7)
    switch (n) {
        NH_VMCNT_CASE8(0) NH_VMCNT_CASE8(8) NH_VMCNT_CASE8(16) NH_VMCNT_CASE8(24)
        NH_VMCNT_CASE8(32) NH_VMCNT_CASE8(40) NH_VMCNT_CASE8(48) NH_VMCNT_CASE8(56)
        default: __builtin_amdgcn_s_waitcnt(NH_VMCNT(0)); break;
    }
#undef NH_VMCNT_CASE8
#undef NH_VMCNT_CASE
#undef NH_VMCNT
}

// Workgroup barrier that leaves vector-memory loads in flight (__syncthreads
// would first wait for every outstanding load).  The caller waits for the
// loads whose data the barrier publishes.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// LDS stores of this wave complete (lgkmcnt(0)), then lds_barrier: the
// stores are visible to the workgroup, loads still in flight.
__device__ __forceinline__ void lds_publish() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
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
