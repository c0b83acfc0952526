// Kernel argument blocks shared by the host launcher and the gfx950 kernels.
// Every kernel takes exactly one of these structs by value, so the host passes
// a single kernelParams entry to hipModuleLaunchKernel and both sides agree on
// the layout by construction.
#pragma once
#include <stdint.h>

namespace nh {

enum DType : int32_t { DT_F32 = 0, DT_BF16 = 1 };

// Where a non-finite value was found (the stage field of the non-finite key,
// report_nonfinite in nh_device.h): a smaller stage is reported first, in the
// order the reference would meet the value (MoeLayer::forward_into runs its
// shared expert before the routed experts, moe.rs:197-233).
enum NonFiniteStage : int32_t {
    kStageInput = 0,               // the layer's input x
    kStageSharedIntermediate = 1,  // the MoE shared expert's f32 intermediate [tokens][shared_inter]
    kStageIntermediate = 2,        // the layer's f32 intermediate (MLP [m][inter], MoE [routes][inter])
};

// Q1/Q2: one workgroup per row.
struct QuantizeRowsArgs {
    const void* x;        // f32 or bf16 [rows][cols]
    int8_t* q;            // [rows][cols] or null
    float* scales;        // [rows]
    int32_t* row_status;  // [rows] or null: -1 = all finite, else first non-finite column
    int8_t* q_act;        // codes in MFMA A-operand tiles (see act_p) or null
    int64_t rows;
    int64_t cols;
    int32_t x_dtype;
    int32_t vec;          // 1: rows are 16-byte aligned and a whole number of 16-byte chunks
    int32_t act_p;        // rows per tile of q_act: code (m, k) at byte
                          // ((m / P * KT + k / 64) * 4 + (k / 16) % 4) * P * 16 + (m % P) * 16 + k % 16,
                          // KT = ceil(cols / 64): P = rows (<= 16) gives the GEMV's [KT][4][rows][16],
                          // P = 16 the weights' tiled layout (the GEMM's A operand)
    int32_t gather_div;   // with gather: output row r quantizes input row gather[r] / gather_div
    const int32_t* gather;  // or null (output row r = input row r)
    uint64_t* nonfinite;  // or null: the first non-finite element (report_nonfinite, nh_device.h)
    int32_t nonfinite_stage;  // NonFiniteStage of x
    int32_t pad_;
};

// Q2 of f32 rows whose absolute maxima a producer left as per-workgroup
// partial maxima (LinearDecodeArgs::row_max): codes into the A-operand tiles
// [KT][4][rows][16] of the M <= 16 GEMV.  grid = (slices of 256 four-value
// chunks, rows).
struct QuantizePmaxArgs {
    const float* x;          // [rows][cols], 16-byte aligned rows, cols % 4 == 0
    const uint32_t* pmax;    // [groups][rows] f32 bits of finite |x| maxima
    int8_t* q_act;           // A-operand tiles
    float* scales;           // [rows]
    uint64_t* nonfinite;     // or null
    int32_t rows, cols, groups;
    int32_t nonfinite_stage;
};

// Tiled INT4 weights -> tiled int8 weights holding code - zero point (the
// W8A8 operand the reference's INT4 layer is defined by), plus the per-tensor
// scale as a per-column scale vector.  Grid-stride over the INT4 lanes.
struct ExpandInt4Args {
    const uint8_t* w4;  // tiled INT4 ([ceil(N/16)][KT][512 B])
    int8_t* w8;         // tiled int8 ([ceil(N/16)][KT][1 KiB])
    float* sw;          // [n] <- scale
    int64_t lanes;      // 8-byte INT4 lanes
    int64_t n;
    float scale;
    int32_t zp;
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

// Weights of every W8A8 / W8A32 kernel are in the tiled layout of
// nh_numerics.h: KT = ceil(K / 64) tiles of 1 KiB per 16-row N tile.

// G1 (M <= 16, activations already quantized): a workgroup owns one 16-row
// N tile; wave w of `waves` owns K tiles w, w + waves, w + 2 waves, ...
struct GemvW8A8Args {
    const int8_t* xq;     // [M][K] row-major, or activation tiles [KT][4][M][16] (x_tiled)
    const float* sx;      // [M]
    const int8_t* wq;     // tiled [N][K]
    const float* sw;      // [N]
    const float* bias;    // [N] or null
    void* out;            // f32 or bf16 [M][N]
    int32_t M, N, K;
    int32_t kt;           // ceil(K / 64)
    int32_t waves;
    int32_t out_dtype;
    int32_t x_tiled;
    int32_t relu2;        // ReLU^2 after the bias (the MLP up projection)
};

// Linear layer at M <= 16 rows in one launch with an in-launch handoff
// (nh_linear_handoff_kernel): workgroups 0 .. M-1 quantize one bf16 row each
// (q: act_p = M activation tiles, agent-scope stores), the other
// ceil(N / 16) run the tiled-A GEMV (g: one slab per wave, K <= 8192) with
// one extra wave that waits for the M rows.  `slot` is a zeroed counter
// block of the context's ring: [0] rows published, [1] GEMV workgroups past
// the wait (the last one zeroes [0] and [1] again), [2] set when a wait ran
// out of polls (never expected: the quantizer workgroups are dispatched
// first and wait for nothing).
struct LinearHandoffArgs {
    QuantizeRowsArgs q;
    GemvW8A8Args g;
    uint32_t* slot;
    int32_t consumers;
    int32_t pad_;
};

// Decode unit (M <= 16, K <= 8192, K % 512 == 0): per-token quantization
// (Q2) of bf16 rows fused in front of G1.  A workgroup owns ntw 16-row N
// tiles with `waves` waves each: blockDim = 64 * waves * ntw <= 1024 and
// waves * 1024 >= 64 * kt.
struct LinearDecodeArgs {
    const void* x;        // bf16 [M][K]
    const int8_t* wq;     // tiled [N][K]
    const float* sw;
    const float* bias;
    void* out;
    int8_t* xq_out;       // optional: block 0 writes the quantized rows here
    float* sx_out;        // optional: and their scales
    int32_t M, N, K;
    int32_t kt;
    int32_t waves;
    int32_t x_dtype;
    int32_t out_dtype;
    int32_t ntw;          // N tiles per workgroup
    int32_t relu2;        // ReLU^2 after the bias (the MLP up projection)
    int32_t w4_zp;        // INT4 weights (tiled_int4): the per-tensor zero point
    float w4_scale;       //   and scale, used in place of sw
    int32_t row0;         // first row of x in the caller's whole input (launches over groups of its rows):
                          // non-finite activations are reported at index (row0 + m) * K + k
    uint64_t* nonfinite;  // or null: the first non-finite activation (report_nonfinite, nh_device.h)
    uint32_t* row_max;    // or null (streaming unit, f32 out): [gridDim.x][M] largest finite |y| of the
                          // workgroup's outputs per row, as f32 bits (each workgroup writes its own slots)
};

// G2: W8A32 dequant GEMV; grid = (N tiles, ceil(M / rows per workgroup)).
struct GemvW8A32Args {
    const float* x;       // [M][K]
    const int8_t* wq;     // tiled [N][K]
    const float* sw;      // [N]
    float* y;             // [M][N]
    int32_t M, N, K;
    int32_t kt;
    int32_t waves;        // waves per workgroup; each takes K tiles wave, wave + waves, ...
    int32_t slabs;        // ceil(ceil(kt / waves) / 4): slabs of 4 K tiles per wave
};

// Diagnostic read stream.
struct StreamReadArgs {
    const void* src;
    int32_t* sink;        // [256], written only when the XOR of the data is a magic value
    uint32_t bytes;       // < 2^31, a multiple of 16
    uint32_t pad_;
};

// Row-major int8 [N][K] -> tiled, one 16-byte tile chunk per thread.
// INT4 [K][N] packed codes (the reference's layout) -> tiled_int4.
struct TileInt4Args {
    const uint8_t* packed;  // ceil(K * N / 2) bytes
    uint8_t* tiled;         // tiled_int4_bytes(N, K)
    int64_t n, k;
    int64_t lanes;          // tiled_int4_bytes / 8
    int32_t kt;
    int32_t zp;
};

struct TileWeightsArgs {
    const int8_t* w;      // [rows][cols] row-major
    int8_t* tiled;        // tiled_bytes(rows, cols)
    int64_t rows, cols;
    int64_t chunks;       // tiled_bytes / 16
    int32_t kt;
    int32_t pad_;
};


// G0d: f32 GEMM with f64 accumulation (the reference's gemm_into order).
struct GemmF32Args {
    const void* lhs;      // [M][K], f32 or (lhs_bf16) bf16
    const float* rhs;     // [K][N]
    float* out;           // [M][N]
    int64_t M, K, N;
    const float* bias;    // [N] or null: out = (float)acc + bias[n] in f32
    int32_t lhs_bf16;
    int32_t pad_;
};

// G3: W8A8 GEMM on int8 MFMA with LDS-staged tiles.
struct GemmW8A8Args {
    const int8_t* xq;     // [M][K]
    const float* sx;      // [M]
    const int8_t* wq;     // tiled [N][K]
    const float* sw;      // [N]
    const float* bias;    // [N] or null
    void* out;            // [M][N]
    int32_t M, N, K;
    int32_t tiles_m, tiles_n;
    int32_t out_dtype;
    int32_t relu2;
    int32_t kt;           // ceil(K / 64)
    int32_t ldo;          // elements between output rows (>= N: a launch may cover a column range)
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
    // when not null: the wave of each token also quantizes the token's row
    // of x ([T][hidden], f32 or bf16, 16-byte rows of at most 512 chunks)
    // into xq [T][hidden] and sx [T], non-finite values reported at stage 0
    const void* x;
    int8_t* xq;
    float* sx;
    uint64_t* nonfinite;
    int32_t x_dtype;
    int32_t hidden;
    // with x: the same codes also into MFMA A tiles of 16 rows (the layout
    // of the linear path's quantizer) for a GEMM over all tokens, or null
    int8_t* xq_tiles;
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
    const int8_t* w;         // [E] x tiled [N][K], expert stride tiled_bytes(N, K)
    const float* sw;         // [E][N]
    const float* bias;       // [E][N] or null: added before ReLU^2 (mlp.rs:201-205)
    float* out;              // [R][N]
    int32_t experts, N, K;
    int32_t top_k;
    int32_t gather;
    int32_t relu2;
    int32_t ntiles;
    int32_t a_rows;          // rows of aq (tokens when gathering, routes otherwise)
    int32_t kt;
    int32_t waves;
};

// R3, the MoE layer's form: A already in slot (expert) order.  grid =
// (wgs_per_expert, experts); workgroup (nb, e) owns expert e's N tiles
// [nb * tiles_per_wg, +tiles_per_wg), dealt to its `streams` waves
// (blockDim = 64 * streams), each wave computing whole tiles.
struct ExpertGemmArgs {
    const int8_t* aq;        // [R][K] codes in slot order
    const float* sa;         // [R]
    const int32_t* offsets;  // [E+1]
    const int8_t* w;         // [E] x tiled [N][K], expert stride tiled_bytes(N, K)
    const float* sw;         // [E][N]
    const float* bias;       // [E][N] or null: added before ReLU^2 (mlp.rs:201-205), staged in LDS with sw
    float* out;              // [R][N]
    int32_t N, K, kt;
    int32_t a_rows;          // R
    int32_t waves;           // unused (1)
    int32_t streams;         // waves per workgroup, each streaming its own N tiles
    int32_t tiles_per_wg;
    int32_t relu2;
    int32_t row_blocks;      // 16-row blocks of A staged per pass (1..4)
    // fused forms of the MoE layer (null when unused):
    uint32_t* omax;          // [R][2] per workgroup column range: max finite |out| of each row (f32 bits)
    const float* ah;         // [R][K] f32 A rows, quantized per row while staged (aq unused)
    const uint32_t* ahmax;   // [R][2] the omax of the launch that wrote ah
    uint64_t* nonfinite;     // non-finite outputs of the omax form are reported here
    int32_t nonfinite_stage;
    int32_t gather_div;      // with perm: A row (and sa entry) of slot s = perm[s] / gather_div
    const int32_t* perm;     // [R] or null (A rows in slot order)
    // Column-tile order of the MoE layer's f32 intermediate h (the up
    // projection's output, the down projection's A): element (row, col) of
    // an [R][C] matrix at ((col / 16) * R + row) * 16 + col % 16 (C % 16 ==
    // 0), so a 16-row block of one 16-column tile is one contiguous KiB and
    // the four stores of a lane's rows fill whole lines back to back.
    int32_t out_tcol;        // out in column-tile order with out_rows rows
    int32_t out_rows;
    int32_t ah_tcol;         // ah in column-tile order with a_rows rows
};

// R4: scatter-combine.
struct CombineArgs {
    const float* slot_out;   // [R][H]
    const int32_t* pos;      // [T*k]
    const float* weights;    // [T*k]
    void* out;               // [T][H]
    const float* shared;     // [T][H] shared-expert output, added first; or null
    int32_t tokens, top_k, hidden;
    int32_t out_dtype;
};

}  // namespace nh
