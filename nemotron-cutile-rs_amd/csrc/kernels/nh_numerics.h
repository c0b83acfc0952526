// Scalar numerics shared by the gfx950 kernels and the library's host twins.
// Each function is the one rounding rule the path relies on; the kernels and
// the host fallback call the same code, so they agree bit for bit.
#pragma once
#include <math.h>
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define NH_HD __host__ __device__ __forceinline__
#define NH_HD_MEMBER __host__ __device__ __forceinline__
#else
#define NH_HD static inline
#define NH_HD_MEMBER inline
#endif

namespace nh {

NH_HD uint32_t f32_bits(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    return u;
}

NH_HD float f32_from_bits(uint32_t u) {
    float x;
    memcpy(&x, &u, 4);
    return x;
}

NH_HD uint64_t f64_bits(double x) {
    uint64_t u;
    memcpy(&u, &x, 8);
    return u;
}

NH_HD double f64_from_bits(uint64_t u) {
    double x;
    memcpy(&x, &u, 8);
    return x;
}

// f32 -> bf16, round to nearest even; NaN stays a quiet NaN.
NH_HD uint16_t f32_to_bf16(float x) {
    uint32_t u = f32_bits(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

NH_HD float bf16_to_f32(uint16_t b) { return f32_from_bits((uint32_t)b << 16); }

// Symmetric int8 code of v with row scale s (nemotron-kernels/src/quantize.rs:197-198
// style: one RN division, round half away from zero, clamp; zero point 0).
// s == 0 covers the all-zero row and an underflowed scale.
NH_HD int8_t quantize_i8(float v, float s) {
    if (s == 0.0f) return 0;
    float q = roundf(v / s);
    q = q > 127.0f ? 127.0f : q;
    q = q < -127.0f ? -127.0f : q;
    return (int8_t)(int)q;
}

// quantize_i8 without a division, for a row scale s = RN(amax / 127) with
// r = RN(1/s) (the per-token activation quantizer of the fused kernels):
//  * s a power of two (and normal): 1/s is exact, so v * r = v / s exactly
//    and roundf of it is the reference's rounding.
//  * otherwise y = fma(v, r, 1.5 * 2^23) holds n = round-to-nearest(v * r)
//    (exact product) in its low mantissa bits.  |v*r - v/s| and
//    |RN(v/s) - v/s| are both below 127 * 2^-24, so n equals
//    roundf(RN(v / s)) whenever v * r is more than 2^-15 from a
//    half-integer; d = fma(v, r, -n) measures that distance with one
//    rounding.  The rare value closer to a tie goes to quantize_near_tie.
//  * zero or subnormal s: the division (quantize_i8).
// |v| <= amax makes |v * r| < 127.5, so no clamp is needed.
constexpr float kQuantMagic = 0x1.8p23f;
constexpr float kQuantTieBand = 0.5f - 0x1p-15f;

NH_HD bool scale_is_pow2(float s) { return s >= 0x1p-126f && (f32_bits(s) & 0x007fffffu) == 0; }

// roundf(RN(|v| / s)) for |v| / s within 2^-14 of h = k + 0.5 (k = floor|t|,
// t = RN(v * r)), decided without dividing: RN(|v|/s) >= h exactly when
// |v| / s exceeds the midpoint m between h and its f32 predecessor, or
// equals it and h is even (round-to-nearest-even at the midpoint).  m has 25
// significant bits and s 24, so m * s is exact in f64 and the sign of
// |v| - m * s (one rounding) is exact.
NH_HD int quantize_near_tie(float v, float s, float t) {
    const float k = floorf(fabsf(t));
    const float h = k + 0.5f;
    const uint32_t hb = f32_bits(h);
    const double m = 0.5 * ((double)h + (double)f32_from_bits(hb - 1u));
    const double d = (double)fabsf(v) - m * (double)s;
    int q = (int)k + ((d > 0.0 || (d == 0.0 && (hb & 1u) == 0u)) ? 1 : 0);
    q = q > 127 ? 127 : q;
    return v < 0.0f ? -q : q;
}

NH_HD int quantize_i8_fast(float v, float s, float r) {
    if (!(s >= 0x1p-126f)) return quantize_i8(v, s);
    if (scale_is_pow2(s)) return (int)roundf(v * r);
    const float y = fmaf(v, r, kQuantMagic);
    const float n = y - kQuantMagic;
    const float d = fmaf(v, r, -n);
    if (fabsf(d) < kQuantTieBand) return (int)n;
    return quantize_near_tie(v, s, v * r);
}

// Tiled int8 weight layout: the operand order of v_mfma_i32_16x16x64_i8.
// A logical [N][K] matrix is stored as ceil(N/16) x KT tiles, KT = ceil(K/64);
// tile (nt, kt) is 1024 contiguous bytes at (nt * KT + kt) * 1024, and byte
// 16 * (16 * g + r) + b of it holds W[16 nt + r][64 kt + 16 g + b] (zero
// outside the matrix).  One 64-lane 16-byte load of a tile is exactly the B
// operand of one MFMA K step, and a row tile's KT KiB are contiguous.
NH_HD uint64_t tiled_k_tiles(uint64_t k) { return (k + 63) / 64; }
NH_HD uint64_t tiled_bytes(uint64_t n, uint64_t k) { return (n + 15) / 16 * 16 * tiled_k_tiles(k) * 64; }
NH_HD uint64_t tiled_offset(uint64_t n, uint64_t k, uint64_t kt_count) {
    return (((n >> 4) * kt_count + (k >> 6)) << 10) + (((((k >> 4) & 3) << 4) | (n & 15)) << 4) + (k & 15);
}

// Tiled INT4 weight layout: the same tiles at half the bytes.  The
// reference stores INT4 linear weights as the [K][N] matrix (input_dim x
// output_dim, linear.rs:324) packed two codes per byte, low nibble first, in
// flat order (quantize.rs:75-77).  Tiled, the logical [N][K] matrix is
// ceil(N/16) x KT tiles of 512 bytes at (nt * KT + kt) * 512; lane l = 16 g + r
// of a tile owns bytes [8 l, 8 l + 8), byte j holding W[16 nt + r][64 kt +
// 16 g + 2 j] in its low nibble and W[..][.. + 2 j + 1] in its high nibble,
// and the zero point outside the matrix.  One 64-lane 8-byte load of a tile
// expands (code - zero point) into exactly the int8 B operand of one MFMA K
// step.
NH_HD uint64_t tiled_int4_bytes(uint64_t n, uint64_t k) { return (n + 15) / 16 * tiled_k_tiles(k) * 512; }

// Row scale from the row's absolute maximum: one RN division by 127.
NH_HD float scale_from_amax(float amax) { return amax / 127.0f; }

// W8A8 epilogue: y = ((float)acc * sx) * sw [+ bias], two RN multiplies, no FMA.
NH_HD float epilogue_w8a8(int32_t acc, float sx, float sw) {
    float t = (float)acc * sx;
    return t * sw;
}

// ReLU^2 with Rust f32::max semantics (max(NaN, 0) = 0): activations.rs:68-71.
NH_HD float relu2(float x) {
    float r = x > 0.0f ? x : 0.0f;
    if (x != x) r = 0.0f;
    return r * r;
}

// expf restated from the published table-driven method used by glibc
// (ARM optimized-routines expf, Szabolcs Nagy 2017): 32-entry 2^(i/32) table,
// kd = round(x*32/ln2) via the 1.5*2^52 shift, r = x*32/ln2 - kd evaluated
// with one fused multiply-add, a degree-3 polynomial for 2^(r/32) with fused
// multiply-adds, and one final rounding to f32.  This is the x86-64 FMA build
// of that method, the one glibc selects on FMA-capable hosts; on this image it
// returns the same f32 as glibc expf for every finite input in [-104, 88.72]
// (checked exhaustively on the host).  Rust f32::exp calls glibc expf on
// linux-gnu, so routing scores computed with it match the reference's
// sigmoid_scalar (activations.rs:73-81) exactly.
NH_HD double exp2_table(uint32_t i) {
    // 2^(i/32) rounded to nearest double
    const double t[32] = {
        0x1.0000000000000p+0, 0x1.059b0d3158574p+0, 0x1.0b5586cf9890fp+0, 0x1.11301d0125b51p+0,
        0x1.172b83c7d517bp+0, 0x1.1d4873168b9aap+0, 0x1.2387a6e756238p+0, 0x1.29e9df51fdee1p+0,
        0x1.306fe0a31b715p+0, 0x1.371a7373aa9cbp+0, 0x1.3dea64c123422p+0, 0x1.44e086061892dp+0,
        0x1.4bfdad5362a27p+0, 0x1.5342b569d4f82p+0, 0x1.5ab07dd485429p+0, 0x1.6247eb03a5585p+0,
        0x1.6a09e667f3bcdp+0, 0x1.71f75e8ec5f74p+0, 0x1.7a11473eb0187p+0, 0x1.82589994cce13p+0,
        0x1.8ace5422aa0dbp+0, 0x1.93737b0cdc5e5p+0, 0x1.9c49182a3f090p+0, 0x1.a5503b23e255dp+0,
        0x1.ae89f995ad3adp+0, 0x1.b7f76f2fb5e47p+0, 0x1.c199bdd85529cp+0, 0x1.cb720dcef9069p+0,
        0x1.d5818dcfba487p+0, 0x1.dfc97337b9b5fp+0, 0x1.ea4afa2a490dap+0, 0x1.f50765b6e4540p+0};
    return t[i & 31];
}

// The method with the table entry 2^(i/32) supplied by `entry(i)` (i in
// 0..31), looked up before any input-dependent branch: the device routing
// kernel reads it from another lane of the wave (a cross-lane read needs every
// lane active) instead of from memory.
template <class Entry>
NH_HD_MEMBER float expf_rn_with(float x, Entry entry) {
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    uint64_t ki = f64_bits(kd);
    kd -= shift;
    double r = __builtin_fma(inv_ln2_n, xd, -kd);
    uint64_t t = f64_bits(entry((uint32_t)(ki % 32))) - ((uint64_t)(ki % 32) << 47);
    t += ki << 47;
    double s = f64_from_bits(t);
    double z = __builtin_fma(c0, r, c1);
    double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    if (x != x) return x + x;
    if (x > 0x1.62e42ep+6f) return __builtin_inff();  // expf overflows above 88.72283
    if (x < -0x1.9fe368p+6f) return 0.0f;              // and underflows to +0 below -103.97208
    return (float)y;
}

struct Exp2Table {
    NH_HD_MEMBER double operator()(uint32_t i) const { return exp2_table(i); }
};

NH_HD float expf_rn(float x) { return expf_rn_with(x, Exp2Table{}); }

// Numerically stable sigmoid of activations.rs:73-81, with expf_rn: exp of
// -|x| (x itself for NaN), then 1 / (1 + z) for x >= 0, z / (1 + z) below.
template <class Entry>
NH_HD_MEMBER float sigmoid_f32_with(float x, Entry entry) {
    const float z = expf_rn_with(x >= 0.0f ? -x : x, entry);
    return x >= 0.0f ? 1.0f / (1.0f + z) : z / (1.0f + z);
}

NH_HD float sigmoid_f32(float x) { return sigmoid_f32_with(x, Exp2Table{}); }

// f32::total_cmp ordering key (moe_routing.rs:176-180).
NH_HD int32_t total_cmp_key(float v) {
    int32_t b = (int32_t)f32_bits(v);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

}  // namespace nh
