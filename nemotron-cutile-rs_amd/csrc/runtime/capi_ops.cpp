// Device entry points of the C ABI: validate on the host, then enqueue.
#include <algorithm>
#include <climits>
#include <cstdint>
#include <cmath>
#include <cstring>
#include <vector>

#include "nh_runtime.h"

using namespace nh;

namespace {

constexpr int64_t kMaxGrid = 0x7fffffff;

unsigned grid_for(int64_t items, int per_block) {
    int64_t g = (items + per_block - 1) / per_block;
    g = std::max<int64_t>(1, std::min<int64_t>(g, 1 << 20));
    return (unsigned)g;
}

// Waves per workgroup of the GEMV family: wave w owns K tiles w, w + W, ...,
// at most 16 of them per register slab; W = ceil(KT / 16) up to 8 waves
// (longer K is walked slab by slab).
int gemv_waves(int kt) { return std::max(1, std::min(8, (kt + 15) / 16)); }

// The linear entry point's M ranges: the fused decode unit (quantizer inside
// the GEMV, one launch) for up to 4 bf16 rows (K <= 8192) and for 3..16 bf16
// rows (K <= 4096, K % 512 == 0, the streaming form); other bf16 rows up to
// 16 (K <= 8192) as the handoff launch (quantizer workgroups feeding the
// tiled-A GEMV's workgroups inside one launch); otherwise quantization into
// activation tiles + the tiled-A GEMV up to 16 rows (f32 rows, K > 8192),
// and the MFMA GEMM beyond.
constexpr size_t kTiledActRows = 16;

// Fused decode unit: kernel, N tiles per workgroup, block size, LDS bytes.
struct DecodePlan {
    KernelId kid;
    int ntw, threads;
    size_t lds;
};

bool plan_decode(const nh_context* ctx, size_t m, size_t n, size_t k, DecodePlan* p) {
    if (m == 0 || m > 8 || k > 8192) return false;
    const int kt = (int)tiled_k_tiles(k);
    const int w = gemv_waves(kt);
    // one N tile per workgroup, the rows' codes in LDS (up to 4 rows)
    auto row_plan = [&]() {
        const size_t rows = m == 1 ? 1 : m <= 2 ? 2 : 4;
        const KernelId kid = m == 1 ? K_LINEAR_DECODE_M1 : m <= 2 ? K_LINEAR_DECODE_ROW2 : K_LINEAR_DECODE_ROW4;
        *p = DecodePlan{kid, 1, 64 * w, rows * ((size_t)w * 1024 + 16)};
        return p->lds <= ctx->max_shared_per_block;
    };
    if (m == 1) return row_plan();
    // several N tiles per workgroup: the widest (up to 16 waves) that still
    // gives every CU one; at one N tile the row kernel is faster up to 4 rows
    if (k % 512 == 0) {
        const int mm = m <= 2 ? 2 : m <= 4 ? 4 : 8;
        const int xr = mm == 2 ? 4 : 8;  // activation chunks each thread holds
        const KernelId kid = mm == 2 ? K_LINEAR_DECODE_M2 : mm == 4 ? K_LINEAR_DECODE : K_LINEAR_DECODE_M8;
        const size_t tiles = (n + 15) / 16;
        auto fits = [&](int ntw) {
            return m * (k / 8) <= (size_t)xr * 64 * w * ntw &&
                   (size_t)kt * 64 * mm + (size_t)w * ntw * 1024 + (size_t)mm * 4 <= ctx->max_shared_per_block;
        };
        auto wide = [&](int ntw) {
            *p = DecodePlan{kid, ntw, 64 * w * ntw, (size_t)kt * 64 * mm + (size_t)w * ntw * 1024 + (size_t)mm * 4};
            return true;
        };
        const size_t cu = (size_t)ctx->cu_count;
        for (int ntw = 16 / w; ntw >= 1; ntw /= 2) {
            // one wide workgroup per CU at a time: whole rounds only (a
            // partial second round costs a full one: 28.7 us at M = 8,
            // 4096 -> 21504, 336 workgroups, against ~20 us in two launches)
            const size_t wgs = (tiles + ntw - 1) / ntw;
            if (ntw > 1 && (wgs < cu || (wgs % cu != 0 && wgs < 4 * cu))) continue;
            if (ntw == 1 && m <= 4) break;
            if (fits(ntw)) return wide(ntw);
        }
        // (a wide workgroup on fewer CUs than the chip has loses to the
        // two-launch path: 20.0 vs ~15 us at M = 8, K = 8192, N = 4096)
    }
    return m <= 4 && row_plan();
}

// Streaming decode unit (3..16 bf16 rows, K % 512 == 0, K <= 4096, any N):
// G workgroups of 16 waves, each quantizing the rows once and walking a run
// of ceil(tiles / G) or one fewer N tiles; G is the CU count or, at the same
// number of rounds, as few workgroups as that many rounds need.  (At K = 8192
// each CU would load 128 KiB of activations, as much as its share of a
// 4096-wide output's weights: 16.4 us against 14.7 in two launches.)
bool plan_stream(const nh_context* ctx, size_t m, size_t n, size_t k, DecodePlan* p, unsigned* grid) {
    if (m < 3 || m > 16 || k % 512 != 0 || k > 4096) return false;
    const size_t mm = m <= 4 ? 4 : m <= 8 ? 8 : 16;
    const size_t tiles = (n + 15) / 16, cu = (size_t)ctx->cu_count;
    const size_t rounds = (tiles + cu - 1) / cu;
    if (rounds > 64) return false;  // a run's scales and bias: at most 1024 LDS floats each
    // codes [KT][4][MM][16], two sets of 16 partial tiles, the run's scales
    // and bias, row maxima, row scales and (W4) row code sums
    const size_t lds = (k / 64) * 64 * mm + 2 * 16 * 64 * 16 + 2 * 1024 * 4 + 3 * mm * 4;
    if (lds > ctx->max_shared_per_block) return false;
    *p = DecodePlan{mm == 4 ? K_LINEAR_DECODE_STREAM_M4 : mm == 8 ? K_LINEAR_DECODE_STREAM_M8 : K_LINEAR_DECODE_STREAM_M16,
                    0, 1024, lds};
    *grid = (unsigned)((tiles + rounds - 1) / rounds);
    return true;
}

// Dynamic LDS of the GEMM kernels: a ring of `stages` stages of `ks` K tiles
// (BM rows x 64 ks bytes of A plus ks * BN/16 weight tiles of 1 KiB), then
// the tile's scales and bias (BM + 2 BN floats) for the epilogue.
size_t gemm_lds_bytes(int bm, int bn, int stages, int ks = 2) {
    const size_t ring = (size_t)stages * ((size_t)bm * 64 * ks + (size_t)ks * (size_t)(bn / 16) * 1024);
    return ring + (size_t)(bm + 2 * bn) * 4;
}

nh_status check_dtype(nh_dtype d, nh_error* err) {
    if (d != NH_F32 && d != NH_BF16) return set_error(err, NH_INVALID_PARAMS, "unknown dtype %d", (int)d);
    return NH_OK;
}

// Shared validation of the W8A8 GEMM family (GemmError::InvalidShape for a
// zero or overflowing dimension, gemm.rs:192-208; envelope for the rest).
nh_status check_w8a8_shape(size_t m, size_t n, size_t k, nh_error* err) {
    size_t t;
    if (m == 0 || n == 0 || k == 0 || !mul_ok(m, k, &t) || !mul_ok(n, k, &t) || !mul_ok(m, n, &t))
        return set_error(err, NH_INVALID_SHAPE, "invalid GEMM shape m=%zu n=%zu k=%zu", m, n, k);
    if (!nh_supports_gemm_w8a8(m, n, k))
        return set_error(err, NH_UNSUPPORTED, "shape m=%zu n=%zu k=%zu outside the gfx950 envelope (k %% 16 == 0, "
                         "k <= 131072, dims < 2^31)", m, n, k);
    return NH_OK;
}

// Row quantizer launch (Q1/Q2): codes row-major into q and/or into the
// activation tiles q_act (rows <= 16).  The vector path needs 16-byte aligned
// rows of whole 16-byte chunks and code stores aligned to a chunk's codes.
nh_status launch_quantize(nh_context* ctx, const void* x, nh_dtype dtype, size_t rows, size_t cols, int8_t* q,
                          float* scales, int32_t* row_status, int8_t* q_act, nh_stream stream, nh_error* err,
                          int act_p = 0, const int32_t* gather = nullptr, int gather_div = 1,
                          uint64_t* nonfinite = nullptr, int nonfinite_stage = 0) {
    const size_t esz = dtype == NH_BF16 ? 2 : 4;
    const size_t row_bytes = cols * esz;
    const bool vec = aligned16(x) && row_bytes % 16 == 0 && row_bytes < (1ull << 31) &&
                     ((uintptr_t)q % (16 / esz)) == 0 && aligned16(q_act);
    QuantizeRowsArgs a{x, q, scales, row_status, q_act, (int64_t)rows, (int64_t)cols, dtype, vec ? 1 : 0,
                       act_p > 0 ? act_p : (int)rows, gather_div, gather, nonfinite, nonfinite_stage, 0};
    // the GEMM's A tiles for many rows of up to 512 chunks: 8 rows per
    // workgroup, whole 128-byte lines per store (M = 2048 linear layer,
    // 4096 -> 4096: 45.6-45.8 us against 46.1-46.7 with the wave kernel)
    if (vec && q_act && act_p == 16 && !gather && rows > 16 && row_bytes <= 512 * 16) {
        const size_t lds = 8 * 64 * tiled_k_tiles(cols);
        return launch(ctx, K_QUANTIZE_TILES, (unsigned)((rows + 7) / 8), 512, lds, stream, a, err);
    }
    // many rows of up to 512 16-byte chunks: one wave per row, no barrier
    // (3072 MoE routes: 299.6 vs 304 us per layer; a few decode rows keep a
    // workgroup each: 8 rows of 4096 on 2 workgroups cost the 52-layer stack
    // 2.26 vs 2.15 ms)
    if (vec && row_bytes <= 512 * 16 && rows >= 1024)
        return launch(ctx, K_QUANTIZE_ROWS_WAVE, (unsigned)((rows + 3) / 4), 256, 0, stream, a, err);
    // a few rows longer than a 256-thread workgroup holds in registers
    // (1024 chunks): 1024 threads per row, one round trip to memory
    if (vec && row_bytes > 1024 * 16 && rows <= 256)
        return launch(ctx, K_QUANTIZE_ROWS_LONG, (unsigned)rows, 1024, 0, stream, a, err);
    // many rows of 1025..2816 chunks: the whole row in a 256-thread workgroup's
    // registers, read once (2048 x 21504 bf16: 3 us less)
    if (vec && row_bytes > 1024 * 16 && row_bytes <= 2816 * 16)
        return launch(ctx, K_QUANTIZE_ROWS_R11, (unsigned)rows, 256, 0, stream, a, err);
    return launch(ctx, K_QUANTIZE_ROWS, (unsigned)rows, 256, 0, stream, a, err);
}

// Bytes of the activation tiles of m <= 16 rows of k codes.
size_t act_tiles_bytes(size_t m, size_t k) { return m * (size_t)tiled_k_tiles(k) * 64; }
size_t align256(size_t b) { return (b + 255) / 256 * 256; }

nh_status launch_gemv(nh_context* ctx, const int8_t* xq, const float* sx, const int8_t* wq, const float* sw,
                      const float* bias, int M, int N, int K, void* out, nh_dtype out_dtype, bool x_tiled,
                      nh_stream stream, nh_error* err, int relu2 = 0) {
    GemvW8A8Args a{};
    a.xq = xq;
    a.sx = sx;
    a.wq = wq;
    a.sw = sw;
    a.bias = bias;
    a.out = out;
    a.M = M;
    a.N = N;
    a.K = K;
    a.kt = (int)tiled_k_tiles(K);
    a.waves = gemv_waves(a.kt);
    a.out_dtype = out_dtype;
    a.x_tiled = x_tiled ? 1 : 0;
    a.relu2 = relu2;
    return launch(ctx, x_tiled ? K_GEMV_W8A8_XT : K_GEMV_W8A8, (unsigned)((N + 15) / 16), 64u * a.waves, 0, stream,
                  a, err);
}

// The persistent 256 x 224 GEMM (gemm_persistent.hip) when its contract
// holds and its tiles fill whole rounds of CUs with less work per CU than the
// loader-wave kernel's 256 x 128 tiles: rounds x tile area (the 21504-wide
// up projection at M = 2048: 3 rounds of 256 x 224 against 5.5 of 256 x 128;
// measured 201-203 against 231-236 us).
// Its LDS: two A slots of 2 x 16 tiles, three B slots of 2 x 14 tiles (the
// weights run a stage further ahead), three scale buffers, a spare KiB.
constexpr size_t kP224Lds = 2 * 8 * ((2 * 256 / 16 + 7) / 8) * 1024 + 3 * (2 * 224 / 16) * 1024 + 3 * 3 * 1024 + 1024;

bool use_persistent_224(const nh_context* ctx, const void* xq, const float* sx, const float* sw, const float* bias,
                        int M, int N, int kt, const void* out, nh_dtype out_dtype) {
    const size_t esz = out_dtype == NH_BF16 ? 2 : 4;
    if (kt % 2 != 0 || M % 4 != 0 || N % 4 != 0 || !aligned16(xq) || !aligned16(sx) || !aligned16(sw) ||
        !aligned16(bias) || !aligned16(out) || (uint64_t)M * N * esz >= (1ull << 31) ||
        kP224Lds > ctx->max_shared_per_block)
        return false;
    const int64_t cu = ctx->cu_count, tm = (M + 255) / 256;
    const int64_t tiles_p = tm * ((N + 223) / 224), tiles_o = tm * ((N + 127) / 128);
    const int64_t work_p = (tiles_p + cu - 1) / cu * 224, work_o = (tiles_o + cu - 1) / cu * 128;
    return tiles_p >= cu && work_p < work_o;
}

// G3 launch.  a_tiled: xq holds A in the weights' tiled layout (written by
// the row quantizer with 16 rows per tile), else row-major [M][K].
nh_status launch_gemm(nh_context* ctx, const int8_t* xq, const float* sx, const int8_t* wq, const float* sw,
                      const float* bias, int M, int N, int K, void* out, nh_dtype out_dtype, int relu2,
                      nh_stream stream, nh_error* err, bool a_tiled = false) {
    GemmW8A8Args a{};
    a.xq = xq;
    a.sx = sx;
    a.wq = wq;
    a.sw = sw;
    a.bias = bias;
    a.out = out;
    a.M = M;
    a.N = N;
    a.K = K;
    a.out_dtype = out_dtype;
    a.relu2 = relu2;
    a.kt = (int)tiled_k_tiles(K);
    a.ldo = N;
    if (a_tiled && use_persistent_224(ctx, xq, sx, sw, bias, M, N, a.kt, out, out_dtype)) {
        a.tiles_m = (M + 255) / 256;
        a.tiles_n = (N + 223) / 224;
        const int64_t tiles = (int64_t)a.tiles_m * a.tiles_n;
        const unsigned grid = (unsigned)std::min<int64_t>(tiles, ctx->cu_count);
        return launch(ctx, K_GEMM_P224, grid, 512u, kP224Lds, stream, a, err);
    }
    // Tile choice.  Tiled A: the largest of 256x128 (8 compute + 8 loader
    // waves), 128x128, 64x128 and 64x64 whose tiles fill every CU, else
    // 64x64 (the most tiles): M = 128 at 4096 -> 16384 took 34.4 us on 128
    // workgroups of 256x128 and 28.5 on 256 of 64x128; M = 256 41.0 -> 35.0 on
    // 128x128.  Row-major A: 256x128 unless that leaves most CUs idle, then
    // 128x128.
    struct Cfg {
        KernelId id;
        int bm, bn, threads;
        size_t lds;  // ring of stages + the tile's scales and bias
    };
    const Cfg big = {a_tiled ? K_GEMM_TA_256 : K_GEMM_W8A8, 256, 128, 1024, gemm_lds_bytes(256, 128, 3)};
    const Cfg small = a_tiled ? Cfg{K_GEMM_TA_128, 128, 128, 512, gemm_lds_bytes(128, 128, 3)}
                              : Cfg{K_GEMM_W8A8_128, 128, 128, 256, gemm_lds_bytes(128, 128, 3)};
    auto tiles = [&](const Cfg& c) { return (int64_t)((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn); };
    const Cfg tiny = {K_GEMM_TA_64, 64, 128, 384, gemm_lds_bytes(64, 128, 3)};
    const Cfg tiny2 = {K_GEMM_TA_6464, 64, 64, 384, gemm_lds_bytes(64, 64, 3)};
    const Cfg* cfg = nullptr;
    if (a_tiled) {
        for (const Cfg* c : {&big, &small, &tiny, &tiny2})
            if (!cfg && tiles(*c) >= ctx->cu_count && c->lds <= ctx->max_shared_per_block) cfg = c;
        if (!cfg && tiny2.lds <= ctx->max_shared_per_block) cfg = &tiny2;
    } else if (tiles(big) >= ctx->cu_count / 4 && big.lds <= ctx->max_shared_per_block) {
        cfg = &big;
    } else if (small.lds <= ctx->max_shared_per_block) {
        cfg = &small;
    }
    if (!cfg) {
        if (a_tiled) return set_error(err, NH_UNSUPPORTED, "LDS too small for the GEMM tiles");
        // LDS too small for the MFMA tiles: 16-row GEMV passes (still exact)
        for (int m0 = 0; m0 < M; m0 += 16) {
            const int mm = std::min(16, M - m0);
            void* o = (char*)out + (size_t)m0 * N * (out_dtype == NH_BF16 ? 2 : 4);
            nh_status st = launch_gemv(ctx, xq + (size_t)m0 * K, sx + m0, wq, sw, bias, mm, N, K, o, out_dtype,
                                       false, stream, err, relu2);
            if (st) return st;
        }
        return NH_OK;
    }
    a.tiles_m = (M + cfg->bm - 1) / cfg->bm;
    a.tiles_n = (N + cfg->bn - 1) / cfg->bn;
    // Every workgroup runs in one of ceil(tiles / CUs) rounds.  When the last
    // round of 256x128 tiles would be at most half full, the columns of the
    // whole rounds take the big tiles and the rest takes 128x128 tiles (half
    // the work each, twice as many): 2048 x 21504 x 4096 is 5 rounds + about
    // half a round instead of 6.
    const int64_t cu = ctx->cu_count;
    const int64_t nbig = (int64_t)a.tiles_m * a.tiles_n;
    if (cfg == &big && small.lds <= ctx->max_shared_per_block && nbig > cu && nbig % cu != 0 &&
        nbig % cu <= cu / 2) {
        const int tn_main = (int)(nbig / cu * cu / a.tiles_m);  // N tiles of whole rounds
        const int n_main = tn_main * big.bn;
        if (tn_main > 0 && n_main < N) {
            GemmW8A8Args r = a;
            a.N = n_main;
            a.tiles_n = tn_main;
            nh_status st =
                launch(ctx, big.id, (unsigned)(a.tiles_m * a.tiles_n), (unsigned)big.threads, big.lds, stream, a, err);
            if (st) return st;
            // columns n_main .. N: weights, scales, bias and outputs from there, rows still N apart
            const size_t esz = out_dtype == NH_BF16 ? 2 : 4;
            r.wq = wq + (size_t)(n_main / 16) * (size_t)r.kt * 1024;
            r.sw = sw + n_main;
            r.bias = bias ? bias + n_main : nullptr;
            r.out = (char*)out + (size_t)n_main * esz;
            r.N = N - n_main;
            r.tiles_m = (M + small.bm - 1) / small.bm;
            r.tiles_n = (r.N + small.bn - 1) / small.bn;
            return launch(ctx, small.id, (unsigned)(r.tiles_m * r.tiles_n), (unsigned)small.threads, small.lds, stream,
                          r, err);
        }
    }
    return launch(ctx, cfg->id, (unsigned)(a.tiles_m * a.tiles_n), (unsigned)cfg->threads, cfg->lds, stream, a, err);
}

}  // namespace

extern "C" {

int nh_supports_gemm_w8a8(size_t m, size_t n, size_t k) {
    // k <= 2^17 keeps the int32 accumulator exact: |acc| <= k * 127 * 127 < 2^31.
    // The kernels address the activations and each weight panel through
    // 32-bit buffer offsets: m * k < 2^31 (plus a tile's overshoot of at most
    // 255 rows) and the tiled weights below 2^40 bytes.
    return m > 0 && n > 0 && k > 0 && m < (1u << 31) && n < (1u << 31) && k <= (1u << 17) && (k % 16) == 0 &&
           (uint64_t)m * k < (1ull << 31) && (uint64_t)n * k < (1ull << 40);
}

nh_status nh_quantize_rows_i8(nh_context* ctx, const void* x, nh_dtype dtype, size_t rows, size_t cols, int8_t* q,
                              float* scales, int32_t* row_status, nh_stream stream, nh_error* err) {
    clear_error(err);
    nh_status st = check_dtype(dtype, err);
    if (st) return st;
    if (rows > (size_t)kMaxGrid || cols > (size_t)kMaxGrid)
        return set_error(err, NH_UNSUPPORTED, "rows/cols must be < 2^31");
    if ((st = bind_device(ctx, err))) return st;
    if (rows == 0 || cols == 0) return NH_OK;  // nothing to quantize (empty inputs are valid, quantize.rs:490-501)
    return launch_quantize(ctx, x, dtype, rows, cols, q, scales, row_status, nullptr, stream, err);
}

size_t nh_tiled_weights_bytes(size_t n, size_t k) {
    if (n == 0 || k == 0 || n > (1ull << 40) || k > (1ull << 40)) return 0;
    return (size_t)tiled_bytes(n, k);
}

nh_status nh_tile_weights_i8(nh_context* ctx, const int8_t* wq, size_t n, size_t k, int8_t* tiled, size_t tiled_len,
                             nh_stream stream, nh_error* err) {
    clear_error(err);
    if (n == 0 || k == 0) return set_error(err, NH_INVALID_SHAPE, "invalid weight shape n=%zu k=%zu", n, k);
    if (n >= (1u << 31) || k >= (1u << 31)) return set_error(err, NH_UNSUPPORTED, "n and k must be < 2^31");
    const size_t need = nh_tiled_weights_bytes(n, k);
    if (tiled_len != need) return mismatch(err, "tiled", need, tiled_len);
    if (!aligned16(tiled)) return set_error(err, NH_UNSUPPORTED, "tiled must be 16-byte aligned");
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    TileWeightsArgs a{wq, tiled, (int64_t)n, (int64_t)k, (int64_t)(need / 16), (int)tiled_k_tiles(k), 0};
    return launch(ctx, K_TILE_WEIGHTS, grid_for(a.chunks, 256), 256, 0, stream, a, err);
}

size_t nh_tiled_int4_weights_bytes(size_t n, size_t k) {
    if (n == 0 || k == 0 || n > (1ull << 40) || k > (1ull << 40)) return 0;
    return (size_t)tiled_int4_bytes(n, k);
}

nh_status nh_tile_weights_int4(nh_context* ctx, const uint8_t* packed, size_t packed_len, size_t k, size_t n,
                               uint32_t zero_point, uint8_t* tiled, size_t tiled_len, nh_stream stream, nh_error* err) {
    clear_error(err);
    size_t kn;
    if (k == 0 || n == 0 || !mul_ok(k, n, &kn)) return set_error(err, NH_INVALID_SHAPE, "invalid INT4 weight shape");
    if (packed_len != nh_packed_int4_len(kn)) return mismatch(err, "packed_weights", nh_packed_int4_len(kn), packed_len);
    if (zero_point > 0x0F) return set_error(err, NH_INVALID_PARAMS, "zero_point %u > 15", zero_point);
    if (n >= (1u << 31) || k >= (1u << 31)) return set_error(err, NH_UNSUPPORTED, "n and k must be < 2^31");
    const size_t need = nh_tiled_int4_weights_bytes(n, k);
    if (tiled_len != need) return mismatch(err, "tiled", need, tiled_len);
    if (((uintptr_t)tiled & 7u) != 0) return set_error(err, NH_UNSUPPORTED, "tiled must be 8-byte aligned");
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    TileInt4Args a{packed, tiled, (int64_t)n, (int64_t)k, (int64_t)(need / 8), (int)tiled_k_tiles(k), (int)zero_point};
    return launch(ctx, K_TILE_INT4, grid_for(a.lanes, 256), 256, 0, stream, a, err);
}

int nh_supports_linear_w4a8(size_t m, size_t n, size_t k) {
    // the fused decode unit: bf16 rows, K tiles of one slab per wave (k <= 8192), whole 16-byte chunks
    return m > 0 && m <= 16 && n > 0 && n < (1u << 31) && k > 0 && k <= 8192 && (k % 16) == 0;
}

size_t nh_linear_w4a8_workspace_size(size_t m, size_t n, size_t k) {
    if (m == 0 || n == 0 || k == 0 || m > (1ull << 31) || n > (1ull << 31) || k > (1ull << 31)) return 0;
    return align256((size_t)tiled_bytes(n, k)) + align256(n * sizeof(float)) + nh_linear_w8a8_workspace_size(m, k);
}

}  // extern "C"

namespace {
nh_status linear_w8a8(nh_context* ctx, const void* x, nh_dtype x_dtype, const int8_t* wq, const float* sw,
                      const float* bias, size_t m, size_t n, size_t k, void* out, nh_dtype out_dtype,
                      void* workspace, size_t workspace_bytes, int8_t* xq_out, float* sx_out, int relu2,
                      uint64_t* nonfinite, int nonfinite_stage, nh_stream stream, nh_error* err,
                      uint32_t* row_max = nullptr);
}  // namespace

extern "C" {

nh_status nh_linear_w4a8(nh_context* ctx, const void* x, nh_dtype x_dtype, const uint8_t* w4_tiled, float scale,
                         uint32_t zero_point, const float* bias, size_t m, size_t n, size_t k, void* out,
                         nh_dtype out_dtype, void* workspace, size_t workspace_bytes, uint64_t* nonfinite,
                         nh_stream stream, nh_error* err) {
    clear_error(err);
    nh_status st;
    // the checks of Int4LinearWeights::validate and project_into (linear.rs:113-124, 290-311)
    if (k == 0 || n == 0) return set_error(err, NH_INVALID_SHAPE, "invalid linear shape k=%zu n=%zu", k, n);
    if (!std::isfinite(scale) || scale <= 0.0f || zero_point > 0x0F)
        return set_error(err, NH_INVALID_PARAMS, "invalid INT4 params scale=%g zero_point=%u", (double)scale,
                         zero_point);
    if (m == 0) return set_error(err, NH_INVALID_ROW_COUNT, "row_count must be non-zero, got 0");
    if ((st = check_dtype(x_dtype, err)) || (st = check_dtype(out_dtype, err))) return st;
    if (((uintptr_t)w4_tiled & 7u) != 0) return set_error(err, NH_UNSUPPORTED, "w4_tiled must be 8-byte aligned");
    if (x_dtype != NH_BF16 || !nh_supports_linear_w4a8(m, n, k) || !aligned16(x)) {
        // any other shape or f32 rows: the weights expanded into int8 tiles of
        // code - zp (the layer's definition) and the W8A8 linear path on them
        if ((st = check_w8a8_shape(m, n, k, err))) return st;
        const size_t need = nh_linear_w4a8_workspace_size(m, n, k);
        if (!workspace || workspace_bytes < need) return mismatch(err, "workspace", need, workspace_bytes);
        if (!aligned16(workspace)) return set_error(err, NH_UNSUPPORTED, "workspace must be 16-byte aligned");
        if ((st = bind_device(ctx, err))) return st;
        int8_t* w8 = (int8_t*)workspace;
        float* sw = (float*)(w8 + align256((size_t)tiled_bytes(n, k)));
        void* lin = (char*)sw + align256(n * sizeof(float));
        const size_t lin_bytes = workspace_bytes - (size_t)((char*)lin - (char*)workspace);
        ExpandInt4Args e{w4_tiled, w8, sw, (int64_t)(tiled_int4_bytes(n, k) / 8), (int64_t)n, scale,
                         (int32_t)zero_point};
        if ((st = launch(ctx, K_EXPAND_INT4, grid_for(e.lanes, 256), 256, 0, stream, e, err))) return st;
        return linear_w8a8(ctx, x, x_dtype, w8, sw, bias, m, n, k, out, out_dtype, lin, lin_bytes, nullptr, nullptr,
                           0, nonfinite, 0, stream, err);
    }
    if ((st = bind_device(ctx, err))) return st;
    const int kt = (int)tiled_k_tiles(k), w = gemv_waves(kt);
    const size_t esz = out_dtype == NH_BF16 ? 2 : 4;
    DecodePlan plan;
    unsigned grid = 0;
    if (plan_stream(ctx, m, n, k, &plan, &grid)) {
        // 3..16 rows: the streaming unit, the INT4 weights streamed once
        LinearDecodeArgs a{};
        a.x = x;
        a.wq = (const int8_t*)w4_tiled;
        a.bias = bias;
        a.out = out;
        a.M = (int)m;
        a.N = (int)n;
        a.K = (int)k;
        a.kt = kt;
        a.waves = 16;
        a.x_dtype = x_dtype;
        a.out_dtype = out_dtype;
        a.w4_zp = (int)zero_point;
        a.w4_scale = scale;
        a.nonfinite = nonfinite;
        const KernelId kid = m <= 4 ? K_LINEAR_DECODE_STREAM_W4_M4
                             : m <= 8 ? K_LINEAR_DECODE_STREAM_W4_M8
                                      : K_LINEAR_DECODE_STREAM_W4_M16;
        return launch(ctx, kid, grid, 1024u, plan.lds, stream, a, err);
    }
    // groups of up to 4 rows, each a launch that streams the weights once
    for (size_t r0 = 0; r0 < m; r0 += 4) {
        const size_t rows = std::min<size_t>(4, m - r0);
        const size_t mm = rows == 1 ? 1 : rows <= 2 ? 2 : 4;
        const KernelId kid = mm == 1 ? K_LINEAR_DECODE_W4_M1 : mm == 2 ? K_LINEAR_DECODE_W4_ROW2 : K_LINEAR_DECODE_W4_ROW4;
        LinearDecodeArgs a{};
        a.x = (const uint16_t*)x + r0 * k;
        a.wq = (const int8_t*)w4_tiled;
        a.bias = bias;
        a.out = (char*)out + r0 * n * esz;
        a.M = (int)rows;
        a.N = (int)n;
        a.K = (int)k;
        a.kt = kt;
        a.waves = w;
        a.x_dtype = x_dtype;
        a.out_dtype = out_dtype;
        a.ntw = 1;
        a.w4_zp = (int)zero_point;
        a.w4_scale = scale;
        a.row0 = (int)r0;  // the group's first row: non-finite inputs are indexed in the whole x
        a.nonfinite = nonfinite;
        const size_t lds = mm * ((size_t)w * 1024 + 16);
        if (lds > ctx->max_shared_per_block) return set_error(err, NH_UNSUPPORTED, "LDS too small");
        if ((st = launch(ctx, kid, (unsigned)((n + 15) / 16), (unsigned)(64 * w), lds, stream, a, err))) return st;
    }
    return NH_OK;
}

nh_status nh_dequantize_i8(nh_context* ctx, const int8_t* q, const float* scales, size_t rows, size_t cols,
                           float* out, nh_stream stream, nh_error* err) {
    clear_error(err);
    size_t total;
    if (!mul_ok(rows, cols, &total)) return set_error(err, NH_INVALID_SHAPE, "rows*cols overflows");
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    if (total == 0) return NH_OK;
    DequantizeI8Args a{q, scales, out, (int64_t)rows, (int64_t)cols};
    // the kernel's 4-code chunks when the layout allows them (the same test)
    const bool vec = cols % 4 == 0 && ((uintptr_t)q & 3) == 0 && aligned16(out);
    return launch(ctx, K_DEQUANT_I8, grid_for((int64_t)(vec ? total / 4 : total), 256), 256, 0, stream, a, err);
}

nh_status nh_dequantize_int4(nh_context* ctx, const uint8_t* packed, size_t packed_len, size_t value_count,
                             float scale, uint32_t zero_point, float* out, size_t out_len, nh_stream stream,
                             nh_error* err) {
    clear_error(err);
    // same validation order as dequantize_int4_into_host (quantize.rs:156-178)
    if (!std::isfinite(scale) || scale <= 0.0f || zero_point > 0x0F)
        return set_error(err, NH_INVALID_PARAMS, "invalid INT4 params scale=%g zero_point=%u", (double)scale,
                         zero_point);
    if (out_len != value_count) return mismatch(err, "output", value_count, out_len);
    if (packed_len != nh_packed_int4_len(value_count))
        return mismatch(err, "packed", nh_packed_int4_len(value_count), packed_len);
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    if (value_count == 0) return NH_OK;
    DequantizeInt4Args a{packed, out, (int64_t)value_count, scale, (float)zero_point};
    // the kernel's 4-code chunks when the layout allows them (the same test)
    const bool vec = value_count >= 4 && ((uintptr_t)packed & 1) == 0 && aligned16(out);
    return launch(ctx, K_DEQUANT_INT4, grid_for((int64_t)(vec ? value_count / 4 : value_count), 256), 256, 0,
                  stream, a, err);
}

int nh_supports_gemm_f32(size_t m, size_t k, size_t n) {
    // i32 shape bounds of the reference's device GEMM (gemm.rs:247-254), any
    // alignment; the grid holds ceil(m / 64) <= 65535 row tiles
    return m > 0 && k > 0 && n > 0 && m <= INT32_MAX && k <= INT32_MAX && n <= INT32_MAX && (m + 63) / 64 <= 65535;
}

// The exact f32 product's two kernels: 64 x 64 outputs per workgroup (16 per
// lane, f64 FMAs) while those tiles fill every CU, else 16 x 16 outputs per
// workgroup on the f64 matrix cores (v_mfma_f64_4x4x4f64 chains), so a narrow
// output such as the MoE router's 128 experts still spreads its k-ordered
// chains over the chip (512 x 2688 x 128: 24.1 us against 52.3 us for one
// output per lane on f64 FMAs; 2048 x 4096 x 128: 80 against 180 us;
// 512 x 4096 x 4096 stays on the 64 x 64 tiles: 531 us against 628 on the
// matrix cores).
static nh_status launch_gemm_f32(nh_context* ctx, const GemmF32Args& a, nh_stream stream, nh_error* err) {
    const int64_t big = ((a.M + 63) / 64) * ((a.N + 63) / 64);
    if (big >= ctx->cu_count)
        return launch(ctx, K_GEMM_F32, (unsigned)((a.N + 63) / 64), 256, 0, stream, a, err,
                      (unsigned)((a.M + 63) / 64));
    // fewer than cu_count 64 x 64 tiles: at most 16 x cu_count 16 x 16 tiles;
    // its buffer loads take 32-bit byte offsets into either operand
    const uint64_t lhs_bytes = (uint64_t)a.M * (uint64_t)a.K * (a.lhs_bf16 ? 2u : 4u);
    const uint64_t rhs_bytes = (uint64_t)a.K * (uint64_t)a.N * 4u;
    if (lhs_bytes >= 0x7ffffff0u || rhs_bytes >= 0x7ffffff0u)  // the kernels' out-of-range offset
        return launch(ctx, K_GEMM_F32, (unsigned)((a.N + 63) / 64), 256, 0, stream, a, err,
                      (unsigned)((a.M + 63) / 64));
    const bool vec = aligned16(a.lhs) && aligned16(a.rhs) && a.K % (a.lhs_bf16 ? 8 : 4) == 0 && a.N % 4 == 0;
    const KernelId id = !vec ? K_GEMM_F32_MFMA_ANY : a.lhs_bf16 ? K_GEMM_F32_MFMA_BF16 : K_GEMM_F32_MFMA;
    return launch(ctx, id, (unsigned)(((a.M + 15) / 16) * ((a.N + 15) / 16)), 256, 0, stream, a, err);
}

nh_status nh_gemm_f32(nh_context* ctx, const float* lhs, size_t lhs_len, const float* rhs, size_t rhs_len, size_t m,
                      size_t k, size_t n, float* out, size_t out_len, nh_stream stream, nh_error* err) {
    clear_error(err);
    // the validation of gemm_into (gemm.rs:341-363): shape, operand lengths, output length
    size_t ll, rl, ol;
    if (m == 0 || k == 0 || n == 0 || !mul_ok(m, k, &ll) || !mul_ok(k, n, &rl) || !mul_ok(m, n, &ol))
        return set_error(err, NH_INVALID_SHAPE, "invalid GEMM shape m=%zu k=%zu n=%zu", m, k, n);
    if (lhs_len != ll) return mismatch(err, "lhs", ll, lhs_len);
    if (rhs_len != rl) return mismatch(err, "rhs", rl, rhs_len);
    if (out_len != ol) return mismatch(err, "output", ol, out_len);
    if (!nh_supports_gemm_f32(m, k, n))
        return set_error(err, NH_UNSUPPORTED, "shape m=%zu k=%zu n=%zu outside the device envelope", m, k, n);
    if (!aligned16(out)) return set_error(err, NH_UNSUPPORTED, "out must be 16-byte aligned");
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    GemmF32Args a{lhs, rhs, out, (int64_t)m, (int64_t)k, (int64_t)n, nullptr, 0, 0};
    return launch_gemm_f32(ctx, a, stream, err);
}

nh_status nh_gemm_w8a8(nh_context* ctx, const int8_t* xq, const float* sx, const int8_t* wq, const float* sw,
                       const float* bias, size_t m, size_t n, size_t k, void* out, nh_dtype out_dtype,
                       nh_stream stream, nh_error* err) {
    clear_error(err);
    nh_status st;
    if ((st = check_dtype(out_dtype, err)) || (st = check_w8a8_shape(m, n, k, err))) return st;
    if (!aligned16(xq) || !aligned16(wq))
        return set_error(err, NH_UNSUPPORTED, "xq and wq must be 16-byte aligned");
    if ((st = bind_device(ctx, err))) return st;
    if (m <= 16)
        return launch_gemv(ctx, xq, sx, wq, sw, bias, (int)m, (int)n, (int)k, out, out_dtype, false, stream, err);
    return launch_gemm(ctx, xq, sx, wq, sw, bias, (int)m, (int)n, (int)k, out, out_dtype, 0, stream, err);
}

nh_status nh_gemm_w8a8_ta(nh_context* ctx, const int8_t* xq_tiled, const float* sx, const int8_t* wq, const float* sw,
                          const float* bias, size_t m, size_t n, size_t k, void* out, nh_dtype out_dtype,
                          nh_stream stream, nh_error* err) {
    clear_error(err);
    nh_status st;
    if ((st = check_dtype(out_dtype, err)) || (st = check_w8a8_shape(m, n, k, err))) return st;
    if (!aligned16(xq_tiled) || !aligned16(wq))
        return set_error(err, NH_UNSUPPORTED, "xq_tiled and wq must be 16-byte aligned");
    if ((st = bind_device(ctx, err))) return st;
    return launch_gemm(ctx, xq_tiled, sx, wq, sw, bias, (int)m, (int)n, (int)k, out, out_dtype, 0, stream, err, true);
}

size_t nh_linear_w8a8_workspace_size(size_t m, size_t k) {
    if (m == 0 || k == 0 || m > (1ull << 31) || k > (1ull << 31)) return 0;
    if (m <= kTiledActRows) return align256(act_tiles_bytes(m, k)) + align256(m * sizeof(float));
    return align256(tiled_bytes(m, k)) + align256(m * sizeof(float));
}

}  // extern "C"

namespace {

// nh_linear_w8a8 with an optional ReLU^2 after the bias (the MLP's up
// projection, mlp.rs:205), validated by the caller up to the device binding.
nh_status linear_w8a8(nh_context* ctx, const void* x, nh_dtype x_dtype, const int8_t* wq, const float* sw,
                      const float* bias, size_t m, size_t n, size_t k, void* out, nh_dtype out_dtype,
                      void* workspace, size_t workspace_bytes, int8_t* xq_out, float* sx_out, int relu2,
                      uint64_t* nonfinite, int nonfinite_stage, nh_stream stream, nh_error* err,
                      uint32_t* row_max) {
    nh_status st;
    // bf16 rows: the fused decode unit when it fits (one launch, no workspace)
    DecodePlan plan;
    unsigned grid = 0;
    const bool streaming = plan_stream(ctx, m, n, k, &plan, &grid);
    if (x_dtype == NH_BF16 && aligned16(x) && ((uintptr_t)xq_out & 7u) == 0 &&
        (streaming || plan_decode(ctx, m, n, k, &plan))) {
        LinearDecodeArgs a{};
        a.x = x;
        a.wq = wq;
        a.sw = sw;
        a.bias = bias;
        a.out = out;
        a.xq_out = xq_out;
        a.sx_out = sx_out;
        a.M = (int)m;
        a.N = (int)n;
        a.K = (int)k;
        a.kt = (int)tiled_k_tiles(k);
        a.waves = gemv_waves(a.kt);
        a.x_dtype = x_dtype;
        a.out_dtype = out_dtype;
        a.ntw = plan.ntw;
        a.relu2 = relu2;
        a.nonfinite = nonfinite;  // the fused unit reads the caller's input only (stage 0)
        a.row_max = streaming ? row_max : nullptr;
        const size_t tiles = (n + 15) / 16;
        if (!streaming) grid = (unsigned)((tiles + plan.ntw - 1) / plan.ntw);
        return launch(ctx, plan.kid, grid, (unsigned)plan.threads, plan.lds, stream, a, err);
    }
    const size_t need = nh_linear_w8a8_workspace_size(m, k);
    if (m <= kTiledActRows) {
        // Q2 into activation tiles (and the caller's row-major xq_out), then
        // the GEMV reads each K tile's codes as M * 64 contiguous bytes
        if (!workspace || workspace_bytes < need) return mismatch(err, "workspace", need, workspace_bytes);
        if (!aligned16(workspace)) return set_error(err, NH_UNSUPPORTED, "workspace must be 16-byte aligned");
        int8_t* tiles = (int8_t*)workspace;
        float* sx = sx_out ? sx_out : (float*)((char*)workspace + align256(act_tiles_bytes(m, k)));
        if (x_dtype == NH_BF16 && aligned16(x) && k % 8 == 0 && k <= 8192 && ((uintptr_t)xq_out & 7u) == 0) {
            // one launch: the quantizer workgroups hand the rows to the GEMV
            // workgroups inside it (M = 8, 8192 -> 4096: 13.57 against 13.96
            // us in two launches; the 52-layer stack 1.733 against 1.760 ms)
            LinearHandoffArgs h{};
            h.q = QuantizeRowsArgs{x, xq_out, sx, nullptr, tiles, (int64_t)m, (int64_t)k, x_dtype, 1, (int)m, 1,
                                   nullptr, nonfinite, nonfinite_stage, 0};
            GemvW8A8Args& g = h.g;
            g.xq = tiles;
            g.sx = sx;
            g.wq = wq;
            g.sw = sw;
            g.bias = bias;
            g.out = out;
            g.M = (int)m;
            g.N = (int)n;
            g.K = (int)k;
            g.kt = (int)tiled_k_tiles(k);
            g.waves = gemv_waves(g.kt);
            g.out_dtype = out_dtype;
            g.x_tiled = 1;
            g.relu2 = relu2;
            h.consumers = (int)((n + 15) / 16);
            h.slot = ctx->handoff + (size_t)(ctx->handoff_next.fetch_add(1) % kHandoffSlots) * 16;
            return launch(ctx, K_LINEAR_HANDOFF, (unsigned)(m + h.consumers), 64u * (g.waves + 1), 0, stream, h, err);
        }
        if ((st = launch_quantize(ctx, x, x_dtype, m, k, xq_out, sx, nullptr, tiles, stream, err, 0, nullptr, 1,
                                  nonfinite, nonfinite_stage)))
            return st;
        return launch_gemv(ctx, tiles, sx, wq, sw, bias, (int)m, (int)n, (int)k, out, out_dtype, true, stream, err,
                           relu2);
    }
    // two launches: Q2 into A tiles in the workspace (and the caller's
    // row-major xq_out), then G3 on the tiled A
    if (!workspace || workspace_bytes < need) return mismatch(err, "workspace", need, workspace_bytes);
    if (!aligned16(workspace)) return set_error(err, NH_UNSUPPORTED, "workspace must be 16-byte aligned");
    int8_t* atiles = (int8_t*)workspace;
    float* sx = sx_out ? sx_out : (float*)((char*)workspace + align256(tiled_bytes(m, k)));
    if ((st = launch_quantize(ctx, x, x_dtype, m, k, xq_out, sx, nullptr, atiles, stream, err, 16, nullptr, 1,
                              nonfinite, nonfinite_stage)))
        return st;
    return launch_gemm(ctx, atiles, sx, wq, sw, bias, (int)m, (int)n, (int)k, out, out_dtype, relu2, stream, err,
                       true);
}

}  // namespace

extern "C" {

nh_status nh_linear_w8a8(nh_context* ctx, const void* x, nh_dtype x_dtype, const int8_t* wq, const float* sw,
                         const float* bias, size_t m, size_t n, size_t k, void* out, nh_dtype out_dtype,
                         void* workspace, size_t workspace_bytes, int8_t* xq_out, float* sx_out, uint64_t* nonfinite,
                         nh_stream stream, nh_error* err) {
    clear_error(err);
    if (m == 0) return set_error(err, NH_INVALID_ROW_COUNT, "row_count must be non-zero, got 0");
    nh_status st;
    if ((st = check_dtype(x_dtype, err)) || (st = check_dtype(out_dtype, err)) ||
        (st = check_w8a8_shape(m, n, k, err)))
        return st;
    if (!aligned16(wq)) return set_error(err, NH_UNSUPPORTED, "wq must be 16-byte aligned");
    if ((st = bind_device(ctx, err))) return st;
    return linear_w8a8(ctx, x, x_dtype, wq, sw, bias, m, n, k, out, out_dtype, workspace, workspace_bytes, xq_out,
                       sx_out, 0, nonfinite, 0, stream, err);
}

// The MLP's workspace: the f32 intermediate h, the up projection's
// per-workgroup row maxima of h (streaming unit: at most kMaxStreamGroups
// workgroups x 8 rows), then the linear workspace of either projection.
constexpr size_t kMaxStreamGroups = 1024;

size_t nh_mlp_w8a8_workspace_size(size_t m, size_t hidden, size_t inter) {
    if (m == 0 || hidden == 0 || inter == 0 || m > (1ull << 31) || inter > (1ull << 31)) return 0;
    const size_t a = nh_linear_w8a8_workspace_size(m, hidden), b = nh_linear_w8a8_workspace_size(m, inter);
    return align256(m * inter * sizeof(float)) + align256(kMaxStreamGroups * 8 * sizeof(uint32_t)) + (a > b ? a : b);
}

}  // extern "C"

// nh_mlp_w8a8, its f32 intermediate reported at NonFiniteStage h_stage (the
// MoE layer's shared expert: kStageSharedIntermediate).
static nh_status mlp_w8a8(nh_context* ctx, const void* x, nh_dtype x_dtype, const int8_t* w_up, const float* s_up,
                          const float* b_up, const int8_t* w_down, const float* s_down, const float* b_down, size_t m,
                          size_t hidden, size_t inter, void* out, nh_dtype out_dtype, void* workspace,
                          size_t workspace_bytes, uint64_t* nonfinite, int h_stage, nh_stream stream, nh_error* err) {
    clear_error(err);
    if (hidden == 0 || inter == 0)
        return set_error(err, NH_INVALID_SHAPE, "mlp shape must be non-zero, got hidden_dim=%zu, intermediate_dim=%zu",
                         hidden, inter);
    if (m == 0) return set_error(err, NH_INVALID_ROW_COUNT, "row_count must be non-zero, got 0");
    nh_status st;
    if ((st = check_dtype(x_dtype, err)) || (st = check_dtype(out_dtype, err)) ||
        (st = check_w8a8_shape(m, inter, hidden, err)) || (st = check_w8a8_shape(m, hidden, inter, err)))
        return st;
    if (!aligned16(w_up) || !aligned16(w_down)) return set_error(err, NH_UNSUPPORTED, "weights must be 16-byte aligned");
    const size_t need = nh_mlp_w8a8_workspace_size(m, hidden, inter);
    if (!workspace || workspace_bytes < need) return mismatch(err, "workspace", need, workspace_bytes);
    if (!aligned16(workspace)) return set_error(err, NH_UNSUPPORTED, "workspace must be 16-byte aligned");
    if ((st = bind_device(ctx, err))) return st;
    // h = ReLU^2(x W_up^T + b_up) in f32 (the reference's intermediate), then
    // out = h W_down^T + b_down with h quantized per row
    float* h = (float*)workspace;
    uint32_t* hmax = (uint32_t*)((char*)workspace + align256(m * inter * sizeof(float)));
    void* lin_ws = (char*)hmax + align256(kMaxStreamGroups * 8 * sizeof(uint32_t));
    const size_t lin_bytes = workspace_bytes - (size_t)((char*)lin_ws - (char*)workspace);
    DecodePlan plan;
    unsigned groups = 0;
    if (x_dtype == NH_BF16 && aligned16(x) && inter % 4 == 0 && plan_stream(ctx, m, inter, hidden, &plan, &groups) &&
        (size_t)groups * m <= kMaxStreamGroups * 8) {
        // 3..16 rows: the streaming unit leaves each workgroup's row maxima of
        // h, so h's quantizer needs no reduction pass over the 4 * inter-byte
        // rows and spreads each row over many workgroups (K = 21504: 8.9 us
        // as one workgroup per row)
        if ((st = linear_w8a8(ctx, x, x_dtype, w_up, s_up, b_up, m, inter, hidden, h, NH_F32, lin_ws, lin_bytes,
                              nullptr, nullptr, 1, nonfinite, kStageInput, stream, err, hmax)))
            return st;
        int8_t* tiles = (int8_t*)lin_ws;
        float* sh = (float*)((char*)lin_ws + align256(act_tiles_bytes(m, inter)));
        QuantizePmaxArgs q{h, hmax, tiles, sh, nonfinite, (int)m, (int)inter, (int)groups, h_stage};
        if ((st = launch(ctx, K_QUANTIZE_ROWS_PMAX, (unsigned)((inter / 4 + 255) / 256), 256, 0, stream, q, err,
                         (unsigned)m)))
            return st;
        return launch_gemv(ctx, tiles, sh, w_down, s_down, b_down, (int)m, (int)hidden, (int)inter, out, out_dtype,
                           true, stream, err);
    }
    if ((st = linear_w8a8(ctx, x, x_dtype, w_up, s_up, b_up, m, inter, hidden, h, NH_F32, lin_ws, lin_bytes, nullptr,
                          nullptr, 1, nonfinite, kStageInput, stream, err)))
        return st;
    // h: the layer's intermediate (h_stage of the non-finite report)
    return linear_w8a8(ctx, h, NH_F32, w_down, s_down, b_down, m, hidden, inter, out, out_dtype, lin_ws, lin_bytes,
                       nullptr, nullptr, 0, nonfinite, h_stage, stream, err);
}

extern "C" {

nh_status nh_mlp_w8a8(nh_context* ctx, const void* x, nh_dtype x_dtype, const int8_t* w_up, const float* s_up,
                      const float* b_up, const int8_t* w_down, const float* s_down, const float* b_down, size_t m,
                      size_t hidden, size_t inter, void* out, nh_dtype out_dtype, void* workspace,
                      size_t workspace_bytes, uint64_t* nonfinite, nh_stream stream, nh_error* err) {
    return mlp_w8a8(ctx, x, x_dtype, w_up, s_up, b_up, w_down, s_down, b_down, m, hidden, inter, out, out_dtype,
                    workspace, workspace_bytes, nonfinite, kStageIntermediate, stream, err);
}

nh_status nh_gemv_w8a32(nh_context* ctx, const float* x, const int8_t* wq, const float* sw, size_t m, size_t n,
                        size_t k, float* y, nh_stream stream, nh_error* err) {
    clear_error(err);
    nh_status st;
    if ((st = check_w8a8_shape(m, n, k, err))) return st;
    if (!aligned16(x) || !aligned16(wq)) return set_error(err, NH_UNSUPPORTED, "x and wq must be 16-byte aligned");
    if ((st = bind_device(ctx, err))) return st;
    if ((m + 3) / 4 > 65535 || n >= (1u << 29))
        return set_error(err, NH_UNSUPPORTED, "device W8A32 GEMV needs m <= 262140 and n < 2^29");
    GemvW8A32Args a{x, wq, sw, y, (int)m, (int)n, (int)k, 0, 0, 0};
    a.kt = (int)tiled_k_tiles(k);
    a.waves = std::max(1, std::min(16, (a.kt + 3) / 4));  // 4 K tiles per wave and slab
    a.slabs = ((a.kt + a.waves - 1) / a.waves + 3) / 4;
    // one activation row per workgroup at m = 1, else 4
    const unsigned rows = m == 1 ? 1u : 4u;
    return launch(ctx, m == 1 ? K_GEMV_W8A32_M1 : K_GEMV_W8A32, (unsigned)((n + 15) / 16), 64u * a.waves, 0, stream,
                  a, err, (unsigned)((m + rows - 1) / rows));
}

// ---- MoE ------------------------------------------------------------------
nh_status nh_moe_route_sigmoid_topk(nh_context* ctx, const float* scores, size_t tokens, size_t experts,
                                    size_t top_k, int renormalize, float scaling, int32_t* indices, float* weights,
                                    nh_stream stream, nh_error* err) {
    clear_error(err);
    if (experts == 0 || top_k == 0 || top_k > experts)  // validate_shape, moe_routing.rs:261-267
        return set_error(err, NH_INVALID_SHAPE, "invalid routing shape tokens=%zu experts=%zu top_k=%zu", tokens,
                         experts, top_k);
    if (experts > 1024 || top_k > 64 || tokens > (size_t)kMaxGrid / 4)
        return set_error(err, NH_UNSUPPORTED, "device routing needs experts <= 1024 and top_k <= 64");
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    if (tokens == 0) return NH_OK;
    RouteArgs a{scores, indices, weights, (int)tokens, (int)experts, (int)top_k, renormalize ? 1 : 0, scaling, 0,
                nullptr, nullptr, nullptr, nullptr, 0, 0, nullptr};
    return launch(ctx, K_ROUTE_SIGMOID, (unsigned)((tokens + 3) / 4), 256, 0, stream, a, err);
}

nh_status nh_moe_permute(nh_context* ctx, const int32_t* indices, size_t tokens, size_t top_k, size_t experts,
                         int32_t* offsets, int32_t* perm, int32_t* pos, nh_stream stream, nh_error* err) {
    clear_error(err);
    if (experts == 0 || top_k == 0) return set_error(err, NH_INVALID_SHAPE, "experts and top_k must be non-zero");
    size_t routes;
    if (!mul_ok(tokens, top_k, &routes) || routes > (size_t)kMaxGrid || experts > 4096)
        return set_error(err, NH_UNSUPPORTED, "device permutation needs routes < 2^31 and experts <= 4096");
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    PermuteArgs a{indices, offsets, perm, pos, (int)routes, (int)experts};
    // one workgroup per expert while their reads of the ids stay small
    // (experts x routes <= 4M: 16 MiB of L2 reads; the 512-token top-6 layer
    // with 128 experts reads 1.5 MiB) and the ids are 16-byte aligned, else
    // the single-workgroup form
    if (experts * routes <= ((size_t)1 << 22) && aligned16(indices))
        return launch(ctx, K_PERMUTE_EXPERT, (unsigned)experts, 256, 0, stream, a, err);
    return launch(ctx, K_PERMUTE, 1, 1024, 2 * experts * sizeof(int), stream, a, err);
}

}  // extern "C"

// The expert-block kernel (slot-ordered A, kernels/moe.hip) in one of its
// three forms; e carries the operands, this fills the launch shape.  Two
// workgroups per expert, each owning half of the N tiles; a pass stages as
// many 16-row blocks (up to 4) as the LDS holds next to the pass's row
// scales, 64 row maxima and the workgroup's weight scales: every pass
// re-streams the expert's weights.  NH_UNSUPPORTED when even one block does
// not fit (the caller takes the grouped kernel).
static nh_status launch_expert_gemm(nh_context* ctx, KernelId id, ExpertGemmArgs e, size_t experts, size_t n,
                                    size_t k, nh_stream stream, nh_error* err) {
    constexpr int kExpertWaves = 8;
    const int kt = (int)tiled_k_tiles(k);
    const int ntiles = (int)((n + 15) / 16);
    const int tiles_per_wg = (ntiles + 1) / 2;
    // the weight scales arrive by 64-float direct-to-LDS rows (256 bytes
    // each, also past the workgroup's last column), so their region is a
    // whole number of rows
    // (and as many for the bias, when there is one)
    auto expert_lds = [&](int rb) {
        const size_t sws_floats = ((size_t)tiles_per_wg * 16 + 63) / 64 * 64;
        return (size_t)rb * kt * 1024 + (size_t)rb * 16 * 4 + 64 * 4 + sws_floats * 4 * (e.bias ? 2 : 1);
    };
    int row_blocks = 4;
    while (row_blocks > 1 && expert_lds(row_blocks) > ctx->max_shared_per_block) --row_blocks;
    const size_t lds = expert_lds(row_blocks);
    if (lds > ctx->max_shared_per_block) return set_error(err, NH_UNSUPPORTED, "expert tiles exceed the LDS");
    e.N = (int)n;
    e.K = (int)k;
    e.kt = kt;
    e.waves = 1;
    e.streams = kExpertWaves;
    e.tiles_per_wg = tiles_per_wg;
    e.row_blocks = row_blocks;
    return launch(ctx, id, 2u, (unsigned)(64 * kExpertWaves), lds, stream, e, err, (unsigned)experts);
}

// Whether the MoE layer's two projections run as the fused expert-block
// pair: the envelope of nh_moe_grouped_gemm_w8a8 for both shapes, the f32
// intermediate within 32-bit buffer offsets, and a 16-row block of A tiles
// in the LDS for both (checked before anything is launched).
static bool expert_fused_ok(nh_context* ctx, size_t routes, size_t experts, size_t hidden, size_t inter,
                            const int8_t* w_up, const int8_t* w_down) {
    if (!nh_supports_gemm_w8a8(routes, inter, hidden) || !nh_supports_gemm_w8a8(routes, hidden, inter)) return false;
    if (experts > 65535 || hidden > 8192 || inter > 8192 || routes * inter * 4 >= (1ull << 31) ||
        routes * hidden >= (1ull << 31))
        return false;
    if (!aligned16(w_up) || !aligned16(w_down)) return false;
    // the down kernel stages each 16-row block as 4 K tiles per wave (8
    // waves): inter <= 2048
    if (tiled_k_tiles(inter) > 32) return false;
    auto fits = [&](size_t n, size_t k) {  // one row block, the weight scales and a bias
        const size_t tiles_per_wg = ((n + 15) / 16 + 1) / 2;
        const size_t sws_floats = (tiles_per_wg * 16 + 63) / 64 * 64;
        return tiled_k_tiles(k) * 1024 + 16 * 4 + 64 * 4 + 2 * sws_floats * 4 <= ctx->max_shared_per_block;
    };
    return fits(inter, hidden) && fits(hidden, inter);
}

// nh_moe_grouped_gemm_w8a8 with an optional per-expert bias [E][n], added
// before ReLU^2 (the experts' MlpLayer biases, mlp.rs:201-205).
static nh_status moe_grouped_gemm(nh_context* ctx, const int8_t* aq, const float* sa, int gather, size_t top_k,
                                  const int32_t* offsets, const int32_t* perm, size_t routes, size_t a_rows,
                                  size_t experts, const int8_t* w, const float* sw, const float* bias, size_t n,
                                  size_t k, int relu2, float* out, nh_stream stream, nh_error* err) {
    clear_error(err);
    if (experts == 0 || top_k == 0) return set_error(err, NH_INVALID_SHAPE, "experts and top_k must be non-zero");
    nh_status st;
    if ((st = check_w8a8_shape(routes ? routes : 1, n, k, err))) return st;
    if (!aligned16(aq) || !aligned16(w)) return set_error(err, NH_UNSUPPORTED, "aq and w must be 16-byte aligned");
    if (experts > 65535 || k > 8192 || a_rows * k >= (1ull << 31) || 16 * k >= (1ull << 31))
        return set_error(err, NH_UNSUPPORTED, "grouped GEMM envelope: experts <= 65535, k <= 8192, a_rows * k < 2^31");
    if ((st = bind_device(ctx, err))) return st;
    if (routes == 0) return NH_OK;
    if (!gather) {
        ExpertGemmArgs e{};
        e.aq = aq;
        e.sa = sa;
        e.offsets = offsets;
        e.w = w;
        e.sw = sw;
        e.bias = bias;
        e.out = out;
        e.a_rows = (int)a_rows;
        e.relu2 = relu2 ? 1 : 0;
        st = launch_expert_gemm(ctx, K_EXPERT_GEMM, e, experts, n, k, stream, err);
        if (st != NH_UNSUPPORTED) return st;
        clear_error(err);
    }
    GroupedGemmArgs a{};
    a.aq = aq;
    a.sa = sa;
    a.offsets = offsets;
    a.perm = perm;
    a.w = w;
    a.sw = sw;
    a.bias = bias;
    a.out = out;
    a.experts = (int)experts;
    a.N = (int)n;
    a.K = (int)k;
    a.top_k = (int)top_k;
    a.gather = gather ? 1 : 0;
    a.relu2 = relu2 ? 1 : 0;
    a.ntiles = (int)((n + 15) / 16);
    a.a_rows = (int)a_rows;
    a.kt = (int)tiled_k_tiles(k);
    a.waves = (a.kt + 15) / 16;  // k <= 8192: one 16-tile slab per wave
    return launch(ctx, K_GROUPED_GEMM, (unsigned)a.ntiles, 64u * a.waves, 0, stream, a, err, (unsigned)experts);
}

extern "C" {

nh_status nh_moe_grouped_gemm_w8a8(nh_context* ctx, const int8_t* aq, const float* sa, int gather, size_t top_k,
                                   const int32_t* offsets, const int32_t* perm, size_t routes, size_t a_rows,
                                   size_t experts, const int8_t* w, const float* sw, size_t n, size_t k, int relu2,
                                   float* out, nh_stream stream, nh_error* err) {
    return moe_grouped_gemm(ctx, aq, sa, gather, top_k, offsets, perm, routes, a_rows, experts, w, sw, nullptr, n, k,
                            relu2, out, stream, err);
}

nh_status nh_moe_combine(nh_context* ctx, const float* slot_out, const int32_t* pos, const float* weights,
                         size_t tokens, size_t top_k, size_t hidden, void* out, nh_dtype out_dtype, nh_stream stream,
                         nh_error* err) {
    return nh_moe_combine_shared(ctx, slot_out, pos, weights, nullptr, tokens, top_k, hidden, out, out_dtype, stream,
                                 err);
}

nh_status nh_moe_combine_shared(nh_context* ctx, const float* slot_out, const int32_t* pos, const float* weights,
                                const float* shared, size_t tokens, size_t top_k, size_t hidden, void* out,
                                nh_dtype out_dtype, nh_stream stream, nh_error* err) {
    clear_error(err);
    nh_status st;
    if ((st = check_dtype(out_dtype, err))) return st;
    if (tokens > (size_t)kMaxGrid || hidden > (size_t)kMaxGrid || top_k == 0)
        return set_error(err, NH_INVALID_SHAPE, "invalid combine shape");
    if ((st = bind_device(ctx, err))) return st;
    if (tokens == 0 || hidden == 0) return NH_OK;
    size_t routes;
    if (!mul_ok(tokens, top_k, &routes) || routes > (size_t)kMaxGrid)
        return set_error(err, NH_UNSUPPORTED, "tokens * top_k must be < 2^31");
    CombineArgs a{slot_out, pos, weights, out, shared, (int)tokens, (int)top_k, (int)hidden, out_dtype};
    // four columns per thread when every row starts 16-byte aligned (8 bytes for bf16 out)
    const bool vec4 = hidden % 4 == 0 && aligned16(slot_out) && aligned16(shared) &&
                      ((uintptr_t)out % (out_dtype == NH_BF16 ? 8 : 16)) == 0;
    if (vec4)
        return launch(ctx, K_COMBINE4, (unsigned)((hidden / 4 + 255) / 256), 256, 0, stream, a, err,
                      (unsigned)tokens);
    return launch(ctx, K_COMBINE, (unsigned)((hidden + 255) / 256), 256, 0, stream, a, err, (unsigned)tokens);
}

// Workspace of the fused MoE layer, 256-byte aligned fields.
static void moe_layout(size_t T, size_t H, size_t I, size_t E, size_t k, size_t off[12]) {
    const size_t R = T * k;
    size_t cur = 0;
    auto take = [&](size_t bytes) {
        size_t o = cur;
        cur += ((bytes + 255) / 256) * 256;
        return o;
    };
    off[0] = take(R * 4);        // indices
    off[1] = take(R * 4);        // weights
    off[2] = take((E + 1) * 4);  // offsets
    off[3] = take(R * 4);        // perm
    off[4] = take(R * 4);        // pos
    off[5] = take(R * H);        // xq, one row per route in expert order
    off[6] = take(R * 4);        // sx
    off[7] = take(R * I * 4);    // up output (f32, ReLU^2 applied; column-tile order on the fused path)
    off[8] = take(R * I);        // requantized up output
    off[9] = take(R * 4);        // its scales
    off[10] = take(R * H * 4);   // down output per slot (f32)
    off[11] = cur;               // total
}

size_t nh_moe_forward_w8a8_workspace_size(size_t tokens, size_t hidden, size_t inter, size_t experts,
                                          size_t top_k) {
    size_t off[12];
    moe_layout(tokens, hidden, inter, experts, top_k, off);
    return off[11];
}

void nh_moe_workspace_layout(size_t tokens, size_t hidden, size_t inter, size_t experts, size_t top_k,
                             size_t offsets_out[5]) {
    size_t off[12];
    moe_layout(tokens, hidden, inter, experts, top_k, off);
    for (int i = 0; i < 5; ++i) offsets_out[i] = off[i];
}

// The routed MoE layer, with the shared expert when w_up_sh is not null:
// shared = the int8 MLP of x (nh_mlp_w8a8, f32), added first by the combine.
// biases (optional) are the experts' and the shared expert's MlpLayer biases.
static nh_status moe_forward(nh_context* ctx, const void* x, nh_dtype x_dtype, const float* logits, size_t tokens,
                             size_t hidden, size_t inter, size_t experts, size_t top_k, int renormalize, float scaling,
                             const int8_t* w_up, const float* s_up, const int8_t* w_down, const float* s_down,
                             size_t inter_sh, const int8_t* w_up_sh, const float* s_up_sh, const int8_t* w_down_sh,
                             const float* s_down_sh, const nh_moe_biases* biases, void* out, nh_dtype out_dtype,
                             void* workspace, size_t workspace_bytes, uint64_t* nonfinite, nh_stream stream,
                             nh_error* err) {
    clear_error(err);
    if (tokens == 0) return set_error(err, NH_INVALID_ROW_COUNT, "row_count must be non-zero, got 0");
    if (hidden == 0 || experts == 0 || top_k == 0 || top_k > experts || inter == 0)
        return set_error(err, NH_INVALID_SHAPE, "invalid MoE shape");
    const bool has_shared = w_up_sh != nullptr;
    if (has_shared && (inter_sh == 0 || !s_up_sh || !w_down_sh || !s_down_sh))
        return set_error(err, NH_INVALID_SHAPE, "shared expert needs intermediate_dim > 0 and all four operands");
    const nh_moe_biases nob{nullptr, nullptr, nullptr, nullptr};
    const nh_moe_biases& b = biases ? *biases : nob;
    if (!has_shared && (b.shared_up || b.shared_down))
        return set_error(err, NH_INVALID_PARAMS, "shared expert biases given without a shared expert");
    size_t off[12];
    moe_layout(tokens, hidden, inter, experts, top_k, off);
    const size_t shared_at = off[11];
    const size_t shared_bytes = has_shared ? align256(tokens * hidden * sizeof(float)) : 0;
    const size_t need =
        off[11] + (has_shared ? shared_bytes + nh_mlp_w8a8_workspace_size(tokens, hidden, inter_sh) : 0);
    if (!workspace || workspace_bytes < need) return mismatch(err, "workspace", need, workspace_bytes);
    if (!aligned16(workspace)) return set_error(err, NH_UNSUPPORTED, "workspace must be 16-byte aligned");
    char* ws = (char*)workspace;
    int32_t* idx = (int32_t*)(ws + off[0]);
    float* wts = (float*)(ws + off[1]);
    int32_t* offsets = (int32_t*)(ws + off[2]);
    int32_t* perm = (int32_t*)(ws + off[3]);
    int32_t* pos = (int32_t*)(ws + off[4]);
    int8_t* xq = (int8_t*)(ws + off[5]);
    float* sx = (float*)(ws + off[6]);
    float* h = (float*)(ws + off[7]);
    int8_t* hq = (int8_t*)(ws + off[8]);
    float* sh = (float*)(ws + off[9]);
    float* d = (float*)(ws + off[10]);
    float* shared = has_shared ? (float*)(ws + shared_at) : nullptr;
    const size_t R = tokens * top_k;
    nh_status st;
    if ((st = check_dtype(x_dtype, err))) return st;
    const bool fused = expert_fused_ok(ctx, R, experts, hidden, inter, w_up, w_down);
    const size_t esz = x_dtype == NH_BF16 ? 2 : 4;
    // the routing wave of each token also quantizes its row (token-major)
    // when the row fits the wave quantizer; the up projection then gathers
    const bool route_q = fused && aligned16(x) && (hidden * esz) % 16 == 0 && hidden * esz <= 512 * 16 &&
                         experts <= 1024 && top_k <= 64 && tokens <= (size_t)kMaxGrid / 4;
    // The shared expert (an MLP over every token).  Past the GEMV's 16 rows
    // its up projection is a GEMM on A tiles of the same codes, so the
    // routing kernel writes them too (into the tiles of the MLP's workspace)
    // and the MLP's own quantization of x is skipped (512 tokens: 7.8 us).
    char* mlp_ws = ws + shared_at + shared_bytes;
    const size_t mlp_bytes = has_shared ? workspace_bytes - shared_at - shared_bytes : 0;
    const bool shared_tiles = has_shared && route_q && tokens > kTiledActRows && aligned16(w_up_sh) &&
                              aligned16(w_down_sh) && check_w8a8_shape(tokens, inter_sh, hidden, nullptr) == NH_OK &&
                              check_w8a8_shape(tokens, hidden, inter_sh, nullptr) == NH_OK;
    float* h_sh = (float*)mlp_ws;
    char* lin_sh = mlp_ws + align256(tokens * inter_sh * sizeof(float)) +
                   align256(kMaxStreamGroups * 8 * sizeof(uint32_t));  // nh_mlp_w8a8's layout
    // the shared expert's intermediate is reported ahead of the routed
    // experts' (the reference runs it first, moe.rs:197-219)
    if (has_shared && !shared_tiles &&
        (st = mlp_w8a8(ctx, x, x_dtype, w_up_sh, s_up_sh, b.shared_up, w_down_sh, s_down_sh, b.shared_down, tokens,
                       hidden, inter_sh, shared, NH_F32, mlp_ws, mlp_bytes, nonfinite, kStageSharedIntermediate, stream,
                       err)))
        return st;
    if (route_q) {
        if ((st = bind_device(ctx, err))) return st;
        RouteArgs ra{logits, idx, wts, (int)tokens, (int)experts, (int)top_k, renormalize ? 1 : 0, scaling, 0,
                     x, xq, sx, nonfinite, x_dtype == NH_BF16 ? DT_BF16 : DT_F32, (int)hidden,
                     shared_tiles ? (int8_t*)lin_sh : nullptr};
        // two tokens per workgroup: two waves route, two quantize
        if ((st = launch(ctx, K_ROUTE_SIGMOID, (unsigned)((tokens + 1) / 2), 256, 0, stream, ra, err))) return st;
    } else if ((st = nh_moe_route_sigmoid_topk(ctx, logits, tokens, experts, top_k, renormalize, scaling, idx, wts,
                                               stream, err))) {
        return st;
    }
    if (shared_tiles) {
        // nh_mlp_w8a8's steps from the tiles on: up (ReLU^2, f32 h), then the
        // linear path on h (its quantization: the layer's intermediate)
        if ((st = launch_gemm(ctx, (const int8_t*)lin_sh, sx, w_up_sh, s_up_sh, b.shared_up, (int)tokens,
                              (int)inter_sh, (int)hidden, h_sh, NH_F32, 1, stream, err, true)))
            return st;
        const size_t lin_bytes = mlp_bytes - (size_t)(lin_sh - mlp_ws);
        if ((st = linear_w8a8(ctx, h_sh, NH_F32, w_down_sh, s_down_sh, b.shared_down, tokens, hidden, inter_sh, shared,
                              NH_F32, lin_sh, lin_bytes, nullptr, nullptr, 0, nonfinite, kStageSharedIntermediate,
                              stream, err)))
            return st;
    }
    if ((st = nh_moe_permute(ctx, idx, tokens, top_k, experts, offsets, perm, pos, stream, err))) return st;
    // otherwise Q2 of each route's token, written in expert order (slot s =
    // token perm[s] / top_k): the up projection reads its rows contiguously
    if (!route_q && (st = launch_quantize(ctx, x, x_dtype, R, hidden, xq, sx, nullptr, nullptr, stream, err, 0, perm,
                                          (int)top_k, nonfinite, kStageInput)))
        return st;
    if (fused) {
        // up (+ bias) with ReLU^2, h in f32 plus each row's max finite |h|
        // per workgroup (non-finite h reported at kStageIntermediate: h is
        // the layer's intermediate); the down projection requantizes h per
        // row while it stages it (the codes and scales of
        // nh_quantize_rows_i8 on h), then adds its bias
        uint32_t* hmax = (uint32_t*)(ws + off[8]);  // [R][2]
        ExpertGemmArgs up{};
        up.aq = xq;
        up.sa = sx;
        if (route_q) {  // token-major codes: slot s reads token perm[s] / top_k
            up.perm = perm;
            up.gather_div = (int)top_k;
        }
        up.offsets = offsets;
        up.w = w_up;
        up.sw = s_up;
        up.bias = b.up;
        up.out = h;
        up.out_tcol = 1;  // h in column-tile order: 270.4-270.8 us per layer against 271.9-272.4 row-major
        up.out_rows = (int)R;
        up.a_rows = route_q ? (int)tokens : (int)R;
        up.relu2 = 1;
        up.omax = hmax;
        up.nonfinite = nonfinite;
        up.nonfinite_stage = kStageIntermediate;
        if ((st = launch_expert_gemm(ctx, K_EXPERT_GEMM_OMAX, up, experts, inter, hidden, stream, err))) return st;
        ExpertGemmArgs down{};
        down.ah = h;
        down.ah_tcol = 1;
        down.ahmax = hmax;
        down.offsets = offsets;
        down.w = w_down;
        down.sw = s_down;
        down.bias = b.down;
        down.out = d;
        down.a_rows = (int)R;
        if ((st = launch_expert_gemm(ctx, K_EXPERT_GEMM_QA, down, experts, hidden, inter, stream, err))) return st;
    } else {
        if ((st = moe_grouped_gemm(ctx, xq, sx, 0, top_k, offsets, perm, R, R, experts, w_up, s_up, b.up, inter,
                                   hidden, 1, h, stream, err)))
            return st;
        // the up outputs per slot: the layer's intermediate
        if ((st = launch_quantize(ctx, h, NH_F32, R, inter, hq, sh, nullptr, nullptr, stream, err, 0, nullptr, 1,
                                  nonfinite, kStageIntermediate)))
            return st;
        if ((st = moe_grouped_gemm(ctx, hq, sh, 0, top_k, offsets, perm, R, R, experts, w_down, s_down, b.down,
                                   hidden, inter, 0, d, stream, err)))
            return st;
    }
    return nh_moe_combine_shared(ctx, d, pos, wts, shared, tokens, top_k, hidden, out, out_dtype, stream, err);
}

nh_status nh_moe_forward_w8a8(nh_context* ctx, const void* x, nh_dtype x_dtype, const float* logits, size_t tokens,
                              size_t hidden, size_t inter, size_t experts, size_t top_k, int renormalize,
                              float scaling, const int8_t* w_up, const float* s_up, const int8_t* w_down,
                              const float* s_down, const nh_moe_biases* biases, void* out, nh_dtype out_dtype,
                              void* workspace, size_t workspace_bytes, uint64_t* nonfinite, nh_stream stream,
                              nh_error* err) {
    return moe_forward(ctx, x, x_dtype, logits, tokens, hidden, inter, experts, top_k, renormalize, scaling, w_up,
                       s_up, w_down, s_down, 0, nullptr, nullptr, nullptr, nullptr, biases, out, out_dtype, workspace,
                       workspace_bytes, nonfinite, stream, err);
}

size_t nh_moe_forward_shared_w8a8_workspace_size(size_t tokens, size_t hidden, size_t inter, size_t experts,
                                                 size_t top_k, size_t shared_inter) {
    size_t off[12];
    moe_layout(tokens, hidden, inter, experts, top_k, off);
    return off[11] + align256(tokens * hidden * sizeof(float)) +
           nh_mlp_w8a8_workspace_size(tokens, hidden, shared_inter);
}

nh_status nh_moe_forward_shared_w8a8(nh_context* ctx, const void* x, nh_dtype x_dtype, const float* logits,
                                     size_t tokens, size_t hidden, size_t inter, size_t experts, size_t top_k,
                                     int renormalize, float scaling, const int8_t* w_up, const float* s_up,
                                     const int8_t* w_down, const float* s_down, size_t shared_inter,
                                     const int8_t* w_up_shared, const float* s_up_shared,
                                     const int8_t* w_down_shared, const float* s_down_shared,
                                     const nh_moe_biases* biases, void* out, nh_dtype out_dtype, void* workspace,
                                     size_t workspace_bytes, uint64_t* nonfinite, nh_stream stream, nh_error* err) {
    if (!w_up_shared) {
        clear_error(err);
        return set_error(err, NH_INVALID_PARAMS, "w_up_shared must not be null (nh_moe_forward_w8a8 has no shared expert)");
    }
    return moe_forward(ctx, x, x_dtype, logits, tokens, hidden, inter, experts, top_k, renormalize, scaling, w_up,
                       s_up, w_down, s_down, shared_inter, w_up_shared, s_up_shared, w_down_shared, s_down_shared,
                       biases, out, out_dtype, workspace, workspace_bytes, nonfinite, stream, err);
}

size_t nh_moe_layer_w8a8_workspace_size(size_t tokens, size_t hidden, size_t inter, size_t experts, size_t top_k,
                                        size_t shared_inter) {
    const size_t inner = shared_inter
                             ? nh_moe_forward_shared_w8a8_workspace_size(tokens, hidden, inter, experts, top_k,
                                                                         shared_inter)
                             : nh_moe_forward_w8a8_workspace_size(tokens, hidden, inter, experts, top_k);
    return align256(inner) + align256(tokens * experts * sizeof(float));
}

// MoeLayer::forward_into (moe.rs:154-249) from its input: the dense f32
// router (router.project, moe.rs:185-188) as the f64-accumulated device GEMM
// of gemm_into_host with the bias added after the rounding to f32, its
// logits after the inner layer's workspace (so nh_moe_workspace_layout's
// offsets still hold), then the routed layer (and the shared expert) on them.
nh_status nh_moe_layer_w8a8(nh_context* ctx, const void* x, nh_dtype x_dtype, const float* router_w,
                            const float* router_b, size_t tokens, size_t hidden, size_t inter, size_t experts,
                            size_t top_k, int renormalize, float scaling, const int8_t* w_up, const float* s_up,
                            const int8_t* w_down, const float* s_down, size_t shared_inter,
                            const int8_t* w_up_shared, const float* s_up_shared, const int8_t* w_down_shared,
                            const float* s_down_shared, const nh_moe_biases* biases, void* out, nh_dtype out_dtype,
                            void* workspace, size_t workspace_bytes, uint64_t* nonfinite, nh_stream stream,
                            nh_error* err) {
    clear_error(err);
    if (tokens == 0) return set_error(err, NH_INVALID_ROW_COUNT, "row_count must be non-zero, got 0");
    if (hidden == 0 || experts == 0 || top_k == 0 || top_k > experts || inter == 0)
        return set_error(err, NH_INVALID_SHAPE, "invalid MoE shape");
    if (!router_w) return set_error(err, NH_INVALID_PARAMS, "router_w must not be null");
    if ((shared_inter != 0) != (w_up_shared != nullptr))
        return set_error(err, NH_INVALID_SHAPE, "shared_inter and w_up_shared must be given together");
    nh_status st;
    if ((st = check_dtype(x_dtype, err))) return st;
    const size_t inner = shared_inter
                             ? nh_moe_forward_shared_w8a8_workspace_size(tokens, hidden, inter, experts, top_k,
                                                                         shared_inter)
                             : nh_moe_forward_w8a8_workspace_size(tokens, hidden, inter, experts, top_k);
    const size_t need = nh_moe_layer_w8a8_workspace_size(tokens, hidden, inter, experts, top_k, shared_inter);
    if (!workspace || workspace_bytes < need) return mismatch(err, "workspace", need, workspace_bytes);
    if (!aligned16(workspace)) return set_error(err, NH_UNSUPPORTED, "workspace must be 16-byte aligned");
    size_t t;
    if (!mul_ok(tokens, hidden, &t) || !nh_supports_gemm_f32(tokens, hidden, experts))
        return set_error(err, NH_UNSUPPORTED, "router shape tokens=%zu hidden=%zu experts=%zu outside the device "
                         "envelope", tokens, hidden, experts);
    if ((st = bind_device(ctx, err))) return st;
    float* logits = (float*)((char*)workspace + align256(inner));
    GemmF32Args a{x, router_w, logits, (int64_t)tokens, (int64_t)hidden, (int64_t)experts, router_b,
                  x_dtype == NH_BF16 ? 1 : 0, 0};
    if ((st = launch_gemm_f32(ctx, a, stream, err))) return st;
    return moe_forward(ctx, x, x_dtype, logits, tokens, hidden, inter, experts, top_k, renormalize, scaling, w_up,
                       s_up, w_down, s_down, shared_inter, w_up_shared, s_up_shared, w_down_shared, s_down_shared,
                       biases, out, out_dtype, workspace, align256(inner), nonfinite, stream, err);
}

}  // extern "C"

// One read of bytes from src (device memory, 16-byte aligned, a multiple of
// 16, < 2^31): 1024 workgroups of 256 threads, four 16-byte loads per thread
// in flight.  sink: 256 device ints, normally never written.
extern "C" nh_status nh_handoff_status(nh_context* ctx, uint32_t* timeouts, uint32_t* busy, nh_error* err) {
    clear_error(err);
    if (!timeouts || !busy) return set_error(err, NH_INVALID_PARAMS, "null output pointer");
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    std::vector<uint32_t> ring((size_t)kHandoffSlots * 16);
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(ring.data(), ctx->handoff, ring.size() * 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return device_error(err, e, "nh_handoff_status");
    *timeouts = *busy = 0;
    for (uint32_t i = 0; i < kHandoffSlots; ++i) {
        *timeouts += ring[i * 16 + 2] != 0;
        *busy += ring[i * 16] != 0 || ring[i * 16 + 1] != 0;
    }
    return NH_OK;
}

extern "C" nh_status nh_stream_read(nh_context* ctx, const void* src, size_t bytes, int32_t* sink, nh_stream stream,
                                    nh_error* err) {
    clear_error(err);
    if (bytes == 0 || bytes % 16 != 0 || bytes >= (1ull << 31))
        return set_error(err, NH_INVALID_SHAPE, "stream of %zu bytes: a multiple of 16 below 2^31", bytes);
    if (!aligned16(src)) return set_error(err, NH_UNSUPPORTED, "src must be 16-byte aligned");
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    StreamReadArgs a{src, sink, (uint32_t)bytes, 0};
    const size_t chunks = bytes / 16;
    const unsigned grid = (unsigned)std::min<size_t>(1024, (chunks + 256 * 4 - 1) / (256 * 4));
    return launch(ctx, K_STREAM_READ, grid, 256, 0, stream, a, err);
}

extern "C" nh_status nh_take_nonfinite(nh_context* ctx, uint64_t* nonfinite, nh_stream stream, nh_error* err) {
    clear_error(err);
    if (!nonfinite) return set_error(err, NH_INVALID_PARAMS, "null non-finite word");
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    hipError_t e = hipStreamSynchronize((hipStream_t)stream);
    if (e != hipSuccess) return device_error(err, e, "hipStreamSynchronize");
    uint64_t word = 0;
    e = hipMemcpy(&word, nonfinite, sizeof(word), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return device_error(err, e, "hipMemcpy(DtoH)");
    if (word == 0) return NH_OK;
    const uint64_t zero = 0;  // cleared for the next call
    e = hipMemcpy(nonfinite, &zero, sizeof(zero), hipMemcpyHostToDevice);
    if (e != hipSuccess) return device_error(err, e, "hipMemcpy(HtoD)");
    // the key of report_nonfinite (nh_device.h): stage, 38-bit index, sign and mantissa
    const uint64_t key = ~word;
    const uint32_t stage = (uint32_t)(key >> 62);
    const char* what = stage == kStageInput                ? "input"
                       : stage == kStageSharedIntermediate ? "shared_intermediate"
                                                           : "intermediate";
    const uint64_t index = (key >> 24) & ((1ull << 38) - 1);
    const float value =
        f32_from_bits((uint32_t)(((key >> 23) & 1u) << 31) | 0x7f800000u | (uint32_t)(key & 0x7fffffu));
    if (err) {
        err->argument = what;
        err->index = index;
        err->value = value;
    }
    return set_error(err, NH_NON_FINITE_INPUT, "non-finite %s value %g at index %llu", what, (double)value,
                     (unsigned long long)index);
}

// nh_linear_w8a8 with the static device scratch (scratch.hip) as its
// workspace: no allocation, for callers that cannot allocate.  Validation as
// nh_linear_w8a8, then the workspace the shape needs is checked against the
// scratch before anything else touches the device.
extern "C" nh_status nh_linear_w8a8_noalloc(nh_context* ctx, const void* x, nh_dtype x_dtype, const int8_t* wq,
                                            const float* sw, const float* bias, size_t m, size_t n, size_t k,
                                            void* out, nh_dtype out_dtype, int8_t* xq_out, float* sx_out,
                                            uint64_t* nonfinite, nh_stream stream, nh_error* err) {
    clear_error(err);
    if (m == 0) return set_error(err, NH_INVALID_ROW_COUNT, "row_count must be non-zero, got 0");
    nh_status st;
    if ((st = check_dtype(x_dtype, err)) || (st = check_dtype(out_dtype, err)) ||
        (st = check_w8a8_shape(m, n, k, err)))
        return st;
    const size_t need = nh_linear_w8a8_workspace_size(m, k);
    if (need > kScratchBytes)
        return set_error(err, NH_UNSUPPORTED,
                         "m=%zu k=%zu needs a %zu-byte workspace, above the %zu-byte static scratch of "
                         "nh_linear_w8a8_noalloc (use nh_linear_w8a8 with a caller workspace)",
                         m, k, need, kScratchBytes);
    if (!aligned16(wq)) return set_error(err, NH_UNSUPPORTED, "wq must be 16-byte aligned");
    if ((st = bind_device(ctx, err))) return st;
    if (!ctx->scratch) return set_error(err, NH_DEVICE_ERROR, "static scratch unavailable: %s", ctx->scratch_error);
    return linear_w8a8(ctx, x, x_dtype, wq, sw, bias, m, n, k, out, out_dtype, ctx->scratch, kScratchBytes, xq_out,
                       sx_out, 0, nonfinite, 0, stream, err);
}
