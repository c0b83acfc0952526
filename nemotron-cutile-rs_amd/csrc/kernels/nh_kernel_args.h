// Kernel argument blocks shared by the host launcher and the gfx950 kernels.
// Every kernel takes exactly one of these structs by value, so the host passes
// a single kernelParams entry to hipModuleLaunchKernel and both sides agree on
// the layout by construction.
#pragma once
#include <stdint.h>

namespace nh {

enum DType : int32_t { DT_F32 = 0, DT_BF16 = 1 };

// Q1/Q2: one workgroup per row.
struct QuantizeRowsArgs {
    const void* x;        // f32 or bf16 [rows][cols]
    int8_t* q;            // [rows][cols]
    float* scales;        // [rows]
    int32_t* row_status;  // [rows] or null: -1 = all finite, else first non-finite column
    int64_t rows;
    int64_t cols;
    int32_t x_dtype;
    int32_t pad_;
};

// Q3: out[r][c] = (float)q[r][c] * scales[r]
struct DequantizeI8Args {
    const int8_t* q;
    const float* scales;
    float* out;
    int64_t rows;
    int64_t cols;
};

// Q0d: affine INT4 unpack + dequantize straight from the packed bytes.
struct DequantizeInt4Args {
    const uint8_t* packed;
    float* out;
    int64_t value_count;
    float scale;
    float zero_point;
};

// G1: W8A8 GEMV for M <= 16 on int8 MFMA.  Workgroup = ksplit waves that
// share one 16-row N tile; wave w owns K range [w*kslice, (w+1)*kslice).
struct GemvW8A8Args {
    const int8_t* xq;     // [M][K]
    const float* sx;      // [M]
    const int8_t* wq;     // [N][K]
    const float* sw;      // [N]
    const float* bias;    // [N] or null
    void* out;            // f32 or bf16 [M][N]
    int32_t M, N, K;
    int32_t kslice;       // bytes of K per wave, multiple of 64
    int32_t ntiles;       // ceil(N / 16)
    int32_t out_dtype;
};

// Decode unit: dynamic per-token quantization fused in front of the GEMV.
// Each workgroup quantizes the (few) activation rows into LDS itself.
struct LinearDecodeArgs {
    const void* x;        // f32 or bf16 [M][K]
    const int8_t* wq;
    const float* sw;
    const float* bias;
    void* out;
    int8_t* xq_out;       // optional: block 0 writes the quantized rows here
    float* sx_out;        // optional: and their scales
    int32_t M, N, K;
    int32_t kslice;
    int32_t ntiles;
    int32_t x_dtype;
    int32_t out_dtype;
    int32_t pad_;
};

// G2: W8A32 dequant GEMV (f64 accumulation of x * ((float)q * s)).
struct GemvW8A32Args {
    const float* x;       // [M][K]
    const int8_t* wq;     // [N][K]
    const float* sw;      // [N]
    float* y;             // [M][N]
    int32_t M, N, K;
    int32_t rows_per_wave;
};

// G3: W8A8 GEMM on int8 MFMA with LDS-staged tiles.
struct GemmW8A8Args {
    const int8_t* xq;     // [M][K]
    const float* sx;      // [M]
    const int8_t* wq;     // [N][K]
    const float* sw;      // [N]
    const float* bias;    // [N] or null
    void* out;            // [M][N]
    int32_t M, N, K;
    int32_t tiles_m, tiles_n;
    int32_t out_dtype;
    int32_t relu2;
    int32_t pad_;
};

// R1: sigmoid top-k routing, one wave per token.
struct RouteArgs {
    const float* scores;  // [T][E]
    int32_t* indices;     // [T][k]
    float* weights;       // [T][k]
    int32_t tokens, experts, top_k;
    int32_t renormalize;
    float scaling;
    int32_t pad_;
};

// R2: counting-sort permutation, one workgroup.
struct PermuteArgs {
    const int32_t* indices;  // [T*k] expert per route
    int32_t* offsets;        // [E+1]
    int32_t* perm;           // [T*k] route id per slot
    int32_t* pos;            // [T*k] slot per route
    int32_t routes, experts;
};

// R3: grouped W8A8 GEMM over expert segments.
struct GroupedGemmArgs {
    const int8_t* aq;        // gather ? [T][K] : [R][K]
    const float* sa;         // gather ? [T] : [R]
    const int32_t* offsets;  // [E+1]
    const int32_t* perm;     // [R]
    const int8_t* w;         // [E][N][K]
    const float* sw;         // [E][N]
    float* out;              // [R][N]
    int32_t experts, N, K;
    int32_t top_k;
    int32_t gather;
    int32_t relu2;
    int32_t ntiles;
    int32_t a_rows;          // rows of aq (tokens when gathering, routes otherwise)
};

// R4: scatter-combine.
struct CombineArgs {
    const float* slot_out;   // [R][H]
    const int32_t* pos;      // [T*k]
    const float* weights;    // [T*k]
    void* out;               // [T][H]
    int32_t tokens, top_k, hidden;
    int32_t out_dtype;
};

}  // namespace nh
