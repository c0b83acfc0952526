// R1..R4: MoE routing, token permutation, grouped expert GEMM, combine.
//
// The reference runs every selected expert densely over ALL rows and combines
// on the host (moe.rs:207-246).  Here the routes are sorted by expert on the
// device (counting sort, deterministic, no global atomics), each expert's
// weights are streamed once against only the rows routed to it, and the
// weighted combine reads each route's row back through pos[].
#include "nh_device.h"

using namespace nh;

namespace {

// total_cmp key of the weight in the high word, ~expert in the low word: the
// maximum is the highest weight and, among equal weights, the lowest expert
// (moe_routing.rs:176-180).
__device__ __forceinline__ int64_t route_key(float w, int e) {
    return ((int64_t)total_cmp_key(w) << 32) | (int64_t)(uint32_t)(0xFFFFFFFFu - (uint32_t)e);
}

// Wave maximum of a 64-bit key through DPP lane moves (no LDS round trips):
// both halves move together each step (quad permutes and row rotates within
// rows of 16, then the row broadcasts of lanes 15 and 31), lanes a move
// leaves out keep their own key, and lane 63 ends with the maximum, which
// readlane hands to every lane.
template <int CTRL, int ROWS>
__device__ __forceinline__ int64_t dpp_max_step_i64(int64_t v) {
    const int lo = (int)(uint32_t)v, hi = (int)(v >> 32);
    const int olo = __builtin_amdgcn_update_dpp(lo, lo, CTRL, ROWS, 0xf, false);
    const int ohi = __builtin_amdgcn_update_dpp(hi, hi, CTRL, ROWS, 0xf, false);
    const int64_t o = ((int64_t)ohi << 32) | (int64_t)(uint32_t)olo;
    return o > v ? o : v;
}

__device__ __forceinline__ int64_t wave_max_i64(int64_t v) {
    v = dpp_max_step_i64<0xb1, 0xf>(v);   // quad_perm 1,0,3,2
    v = dpp_max_step_i64<0x4e, 0xf>(v);   // quad_perm 2,3,0,1
    v = dpp_max_step_i64<0x124, 0xf>(v);  // row_ror 4
    v = dpp_max_step_i64<0x128, 0xf>(v);  // row_ror 8
    v = dpp_max_step_i64<0x142, 0xa>(v);  // row_bcast 15
    v = dpp_max_step_i64<0x143, 0xc>(v);  // row_bcast 31
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(v >> 32), 63);
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

constexpr int kMaxExpertsPerLane = 16;  // E <= 1024

}  // namespace

// R1: one wave per token.  Expert e lives in lane e % 64, slot e / 64 of
// S slots (S = 2, 4 or 16: the body is instantiated per slot count, so a
// 128-expert router runs 2 inlined sigmoids per lane instead of fetching the
// code of 16).
// expf's 2^(i/32) table held across the wave (lane l: entry l % 32, f64
// bits) and read through the LDS crossbar: no memory load inside the
// sigmoid.
struct LaneExp2Table {
    uint32_t lo, hi;
    __device__ double operator()(uint32_t i) const {
        const int addr = (int)(i & 31) * 4;
        const uint32_t l = (uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)lo);
        const uint32_t h = (uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)hi);
        return f64_from_bits(((uint64_t)h << 32) | l);
    }
};

__device__ __forceinline__ LaneExp2Table lane_exp2_table(int lane) {
    const uint64_t b = f64_bits(exp2_table((uint32_t)lane & 31));
    return LaneExp2Table{(uint32_t)b, (uint32_t)(b >> 32)};
}

template <int S>
__device__ __forceinline__ void route_token(const RouteArgs& a, int token, int lane, const float (&sc)[S],
                                            const LaneExp2Table& tbl) {
    const int E = a.experts;
    int64_t key[S];
#pragma unroll
    for (int i = 0; i < S; ++i) {
        const int e = lane + 64 * i;
        const float w = sigmoid_f32_with(sc[i], tbl);  // every lane: the table reads are cross-lane
        key[i] = e < E ? route_key(w, e) : INT64_MIN;
    }
    float wsel = 0.0f;  // lane j keeps the j-th selected weight (top_k <= 64)
    int esel = 0;
    for (int j = 0; j < a.top_k; ++j) {
        int64_t best = INT64_MIN;
#pragma unroll
        for (int i = 0; i < S; ++i) best = key[i] > best ? key[i] : best;
        best = wave_max_i64(best);
        const int e = (int)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFF));
        const int32_t k32 = (int32_t)(best >> 32);
        const float w = f32_from_bits((uint32_t)total_cmp_key(f32_from_bits((uint32_t)k32)));
#pragma unroll
        for (int i = 0; i < S; ++i)  // the owner drops it
            if (lane + 64 * i == e) key[i] = INT64_MIN;
        if (lane == j) {
            wsel = w;
            esel = e;
        }
    }
    if (a.renormalize) {
        // sum in route order, as selected_total (moe_routing.rs:207-211)
        float total = 0.0f;
        for (int j = 0; j < a.top_k; ++j)
            total = total + f32_from_bits((uint32_t)__builtin_amdgcn_readlane((int)f32_bits(wsel), j));
        wsel = wsel / total;
    }
    if (a.scaling != 1.0f) wsel = wsel * a.scaling;
    if (lane < a.top_k) {
        a.indices[(int64_t)token * a.top_k + lane] = esel;
        a.weights[(int64_t)token * a.top_k + lane] = wsel;
    }
}

template <int S>
__device__ __forceinline__ void route_kernel_body(const RouteArgs& a, int token, int lane) {
    const LaneExp2Table tbl = lane_exp2_table(lane);
    // the token's scores through a buffer resource (experts past E read 0)
    float sc[S];
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.scores + (int64_t)token * a.experts, (uint32_t)a.experts * 4u);
#pragma unroll
    for (int i = 0; i < S; ++i)
        sc[i] = f32_from_bits(__builtin_amdgcn_raw_buffer_load_b32(rs, (lane + 64 * i) * 4, 0, 0));
    route_token<S>(a, token, lane, sc, tbl);
}

// The quantization half of a token when another wave routes it: Q2 of the
// token's row, token-major (and into the A tiles when given): the codes and
// scales of nh_quantize_rows_i8.
template <int DT>
__device__ __forceinline__ void quantize_token(const RouteArgs& a, int token) {
    QuantizeRowsArgs q{};
    q.x = a.x;
    q.q = a.xq;
    q.scales = a.sx;
    q.rows = a.tokens;
    q.cols = a.hidden;
    q.x_dtype = a.x_dtype;
    q.nonfinite = a.nonfinite;
    q.nonfinite_stage = 0;
    q.q_act = a.xq_tiles;
    q.act_p = 16;
    v4i xv[8];
    const int64_t row = quantize_row_wave_load<DT, 8>(q, xv, token);
    quantize_row_wave_finish<DT, 8>(q, xv, row);
}

// Without x: one wave per token routes it (4 tokens per workgroup).  With x
// (the MoE layer): 2 tokens per workgroup, waves 0 and 1 route them while
// waves 2 and 3 quantize their rows, so the two chains run side by side
// instead of one after the other in one wave (the 512-token MoE layer:
// 272.1-272.4 against 273.2-273.3 us).
extern "C" __global__ __launch_bounds__(256) void nh_moe_route_sigmoid_kernel(RouteArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int per = a.x ? 2 : 4;  // tokens per workgroup
    // with the token codes going to A tiles, a tile line's 8 tokens to one XCD (xcd_line_order)
    const int blk = a.x && a.xq_tiles ? (int)xcd_line_order(blockIdx.x, (a.tokens + per - 1) / per, per) : (int)blockIdx.x;
    const int token = blk * per + (wave & (per - 1));
    if (token >= a.tokens) return;
    if (a.x && wave >= 2) {
        if (a.x_dtype == DT_BF16)
            quantize_token<DT_BF16>(a, token);
        else
            quantize_token<DT_F32>(a, token);
        return;
    }
    if (a.experts <= 128)
        route_kernel_body<2>(a, token, lane);
    else if (a.experts <= 256)
        route_kernel_body<4>(a, token, lane);
    else
        route_kernel_body<kMaxExpertsPerLane>(a, token, lane);
}

// R2, one workgroup per expert: the same stable counting sort by (expert,
// route id) as nh_moe_permute_kernel, every expert's slots computed in
// parallel.  Thread t owns the L consecutive routes [t L, t L + L) (L = the
// routes over 256 threads, rounded up to whole 16-byte groups), so the route
// order is the thread order:
//  1. each thread counts, over its routes, the valid ids below e and the ids
//     equal to e;
//  2. one block scan: the ids below e summed over the block are the
//     expert's offset, and the exclusive prefix of the equal counts is the
//     thread's first slot within the expert;
//  3. each thread walks its routes again and places those of expert e.
// Expert 0's workgroup also marks the routes whose id lies outside [0, E)
// (pos = -1, not placed); expert E-1's writes offsets[E].  Up to 16 routes
// per thread (4096 routes) stay in registers between the passes.  (One wave
// per expert, ballots over 64 routes per step, was a serial chain of 48
// steps per pass: 6.5 us inside the kernel at 3072 routes.)
// Needs 16-byte aligned ids.
extern "C" __global__ __launch_bounds__(256) void nh_moe_permute_expert_kernel(PermuteArgs a) {
    __shared__ int wave_eq[4], wave_lt[4];
    const int e = blockIdx.x, E = a.experts, R = a.routes;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int L = ((R + 255) / 256 + 3) & ~3;
    const int r0 = tid * L;
    auto ids4 = [&](int r) {  // ids r .. r + 3, -1 past the routes
        if (r + 3 < R) return *(const v4i*)(a.indices + r);
        v4i v;
#pragma unroll
        for (int w = 0; w < 4; ++w) v[w] = r + w < R ? a.indices[r + w] : -1;
        return v;
    };
    constexpr int kKept = 4;  // 16-byte groups held in registers
    v4i kept[kKept];
    const bool in_regs = L <= 4 * kKept;
#pragma unroll
    for (int i = 0; i < kKept; ++i) kept[i] = in_regs && 4 * i < L ? ids4(r0 + 4 * i) : v4i{-1, -1, -1, -1};
    int lt = 0, eq = 0;
    auto count = [&](const v4i& v) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            lt += v[w] >= 0 && v[w] < e;
            eq += v[w] == e;
        }
    };
    if (in_regs) {
#pragma unroll
        for (int i = 0; i < kKept; ++i) count(kept[i]);
    } else {
        for (int c = 0; c < L; c += 4) count(ids4(r0 + c));
    }
    // 2. inclusive scan of eq and sum of lt within the wave, then across the 4 waves
    int incl = eq, lsum = lt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += t;
        lsum += __shfl_xor(lsum, off, kWave);
    }
    if (lane == 63) wave_eq[wave] = incl;
    if (lane == 0) wave_lt[wave] = lsum;
    __syncthreads();
    int before = 0, total = 0, offset = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        before += w < wave ? wave_eq[w] : 0;
        total += wave_eq[w];
        offset += wave_lt[w];
    }
    if (tid == 0) {
        a.offsets[e] = offset;
        if (e == E - 1) a.offsets[E] = offset + total;
    }
    if (total == 0 && e != 0) return;  // uniform
    // 3.
    int slot = offset + before + incl - eq;
    const int rend = min(R, r0 + L);  // past this thread's routes (the held groups past L read -1)
    auto place = [&](const v4i& v, int r) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            if (v[w] == e) {
                a.perm[slot] = r + w;
                a.pos[r + w] = slot;
                ++slot;
            } else if (e == 0 && r + w < rend && (v[w] < 0 || v[w] >= E)) {
                a.pos[r + w] = -1;
            }
        }
    };
    if (in_regs) {
#pragma unroll
        for (int i = 0; i < kKept; ++i) place(kept[i], r0 + 4 * i);
    } else {
        for (int c = 0; c < L; c += 4) place(ids4(r0 + c), r0 + c);
    }
}

// R2: one workgroup of 1024 threads.  Phase 1 histograms the experts (LDS
// atomics: counts do not depend on order), phase 2 scans them into offsets,
// phase 3 walks the routes in order in rounds of 1024 and gives every route
// its stable rank: inside a wave by ballot-matching equal experts, across
// waves by handing a running per-expert base from wave to wave in order.
extern "C" __global__ __launch_bounds__(1024) void nh_moe_permute_kernel(PermuteArgs a) {
    extern __shared__ int sm[];  // counts[E], base[E]
    const int E = a.experts, R = a.routes;
    int* counts = sm;
    int* running = sm + E;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
    for (int e = tid; e < E; e += blockDim.x) {
        counts[e] = 0;
        running[e] = 0;
    }
    __syncthreads();
    // an expert id outside [0, E) is not placed (pos = -1), so no slot can
    // ever leave [0, routes)
    for (int r = tid; r < R; r += blockDim.x) {
        const int e = a.indices[r];
        if (e >= 0 && e < E) atomicAdd(&counts[e], 1);
    }
    __syncthreads();
    if (wave == 0) {
        int carry = 0;
        for (int base = 0; base < E; base += 64) {
            const int e = base + lane;
            int v = e < E ? counts[e] : 0;
            // inclusive scan across the wave
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const int o = __shfl_up(v, off, kWave);
                if (lane >= off) v += o;
            }
            if (e < E) {
                const int excl = carry + v - (e < E ? counts[e] : 0);
                a.offsets[e] = excl;
                running[e] = excl;
            }
            carry += __shfl(v, 63, kWave);
        }
        if (lane == 0) a.offsets[E] = carry;
    }
    __syncthreads();
    int nbits = 0;
    while ((1 << nbits) < E) ++nbits;
    for (int round = 0; round < R; round += blockDim.x) {
        const int r = round + tid;
        const int ein = r < R ? a.indices[r] : -1;
        const bool valid = ein >= 0 && ein < E;
        const int e = valid ? ein : -1;
        if (r < R && !valid) a.pos[r] = -1;
        uint64_t mask = __ballot(valid);
        for (int b = 0; b < nbits; ++b) {
            const uint64_t bal = __ballot(valid && ((e >> b) & 1));
            mask &= ((e >> b) & 1) ? bal : ~bal;
        }
        const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
        const int rank = __popcll(mask & lt);
        const int cnt = __popcll(mask);
        const int leader = valid ? (__ffsll((long long)mask) - 1) : 0;
        for (int w = 0; w < nw; ++w) {
            int base = 0;
            if (wave == w && valid && lane == leader) {
                base = running[e];
                running[e] = base + cnt;
            }
            if (wave == w) {
                base = __shfl(base, leader, kWave);
                if (valid) {
                    const int slot = base + rank;
                    a.perm[slot] = r;
                    a.pos[r] = slot;
                }
            }
            __syncthreads();
        }
    }
}

// R3: grouped W8A8 GEMM.  grid.x = N tiles of 16 rows, grid.y = experts,
// blockDim = 64 * waves, waves = ceil(KT / 16) (K <= 8192).
// HBM-bound like the GEMV: expert e's weights are tiled (nh_numerics.h) at
// w + e * tiled_bytes(N, K); wave w owns K tiles w, w + waves, ... and issues
// the loads of all of them (at most 16, one contiguous KiB each, streaming
// policy) at once; the slab then stays in registers while the expert's
// segment is walked in blocks of 16 routed rows (two blocks for a typical
// ~24-row segment), so each expert weight byte leaves HBM once.  A rows are
// slots (the MoE layer quantizes the routes' tokens straight into slot
// order), or gathered per lane (token perm[slot] / top_k) when the public
// entry point is given token-major activations.  The first block's A loads
// go out before the weight slab and each next block's under the current
// block's reduction: behind an index load queued after the slab (the
// gathered form), the A loads would wait for the whole slab first.
// Tiles past KT and rows past the segment load from an out-of-range buffer
// offset, which returns zeros without touching memory.
constexpr int kGroupedSteps = 16;

extern "C" __global__ __launch_bounds__(512) void nh_moe_grouped_gemm_kernel(GroupedGemmArgs a) {
    __shared__ v4i red[8 * 64];
    const int e = blockIdx.y;
    const int tile = blockIdx.x;
    const int seg0 = a.offsets[e], seg1 = a.offsets[e + 1];
    if (seg0 >= seg1) return;  // no routes: this expert's weights are never read
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = a.waves;
    const int r16 = lane & 15, g = lane >> 4;
    const int N = a.N, K = a.K, kt = a.kt;
    const __amdgpu_buffer_rsrc_t wr =
        make_rsrc(a.w + (int64_t)e * tiled_bytes(N, K) + (int64_t)tile * kt * 1024, (uint32_t)kt * 1024u);
    const __amdgpu_buffer_rsrc_t ar = make_rsrc(a.aq, (uint32_t)a.a_rows * (uint32_t)K);
    const int n = tile * 16 + r16;
    const float swn = n < N ? a.sw[(int64_t)e * N + n] : 0.0f;
    const float bn = a.bias && n < N ? a.bias[(int64_t)e * N + n] : 0.0f;
    // A row of slot s (gathered rows: the public entry point's token-major
    // activations; the MoE layer passes them already in slot order)
    auto a_row = [&](int s) { return a.gather ? a.perm[s] / a.top_k : s; };
    v4i x[kGroupedSteps];
    float sa[4];
    // one 16-slot chunk's A fragments and epilogue scales
    auto load_chunk = [&](int m0) {
        const int slot = m0 + r16;
        const bool mok = slot < seg1;
        const int arow = mok ? a_row(slot) : 0;
#pragma unroll
        for (int s = 0; s < kGroupedSteps; ++s) {
            const int k = (wave + s * W) * 64 + g * 16;
            x[s] = buffer_load16(ar, (mok && k < K) ? arow * K + k : kOutOfRange);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int srow = m0 + 4 * g + r;
            sa[r] = srow < seg1 ? a.sa[a_row(srow)] : 0.0f;
        }
    };
    // the first chunk's activations ahead of the weight slab: loads return
    // in issue order, so the MFMAs wait for the slab only, not for an index
    // load queued behind it
    __builtin_amdgcn_sched_barrier(0);
    load_chunk(seg0);
    __builtin_amdgcn_sched_barrier(0);
    v4i b[kGroupedSteps];
#pragma unroll
    for (int s = 0; s < kGroupedSteps; ++s) b[s] = buffer_load16_stream(wr, (wave + s * W) * 1024 + lane * 16);
    __builtin_amdgcn_sched_barrier(0);
    for (int m0 = seg0; m0 < seg1; m0 += 16) {
        v4i acc = {0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < kGroupedSteps; ++s) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x[s], b[s], acc, 0, 0, 0);
        float sa_cur[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sa_cur[r] = sa[r];
        // the next chunk's loads run under this chunk's reduction and epilogue
        if (m0 + 16 < seg1) load_chunk(m0 + 16);
        if (W > 1) {
            red[wave * 64 + lane] = acc;
            __syncthreads();
            if (wave == 0)
                for (int w = 1; w < W; ++w) acc += red[w * 64 + lane];
        }
        if (wave == 0 && n < N) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int srow = m0 + 4 * g + r;
                if (srow < seg1) {
                    float y = epilogue_w8a8(acc[r], sa_cur[r], swn);
                    if (a.bias) y = y + bn;
                    if (a.relu2) y = relu2(y);
                    a.out[(int64_t)srow * N + n] = y;
                }
            }
        }
        if (W > 1) __syncthreads();
    }
}

// R3 for the MoE layer (A in slot order).  One workgroup per (expert, half
// of its N tiles): the chip runs one of them per CU in a single round.  The
// expert's routed rows are staged once per pass of up to 16 * row_blocks
// slots into LDS as 1 KiB MFMA A tiles (direct-to-LDS loads, lane l fetching
// row l % 16, bytes 16 (l / 16) of its 64-byte K tile, so the fragment reads
// are linear), and stay there while the 8 waves stream the weights.  Every
// wave owns whole N tiles (t_begin + wave, + 8, ...) and walks each one's K
// range in chunks of 8 K tiles held in two register slabs in ping-pong:
// while one chunk's MFMAs run, the next chunk is in flight, and a slab is
// refilled (with the chunk after next, of the same tile or of the wave's
// next one) as soon as its MFMAs are issued.  At a tile's end the wave
// writes the tile's outputs itself.  No partial sums cross waves, so a pass
// has no barrier between its staging and its end, and the waves drift apart
// like independent streams.  Measured per projection (bench routing): 120
// us; the same loads alone stream the 638 MB in 91 us, and most of the rest
// is the output rows' write-back mixed into the stream (stores aimed at a
// few L2-resident rows instead: 102 us).  The weight scales sit in LDS: a
// global load in the epilogue made every wave wait for its weights in
// flight (the compiler cannot count that load's place in the queue).
// The host sizes row_blocks to fill the LDS (3 at K = 2688, 4 at K = 1856):
// every pass re-streams the expert's weights, and since all workgroups run
// in one round the layer waits for its longest segment.  With 32-slot
// passes, the 6 of 128 experts holding 33-40 of the 3072 routes took two
// passes and doubled the projection time.
constexpr int kExpertSlab = 8;  // K tiles per register slab (two slabs in ping-pong)
constexpr int kExpertPlain = 0, kExpertOmax = 1, kExpertQuantA = 2;

// The waves' tile streams of one pass over NRB row blocks.  Straight-line
// per chunk (every load issued, past the wave's last chunk from an empty
// buffer; K tiles past kt load zeros and meet a valid A tile), so the
// compiler's wait counts see the slabs in flight and wait for one slab only.
template <int NRB, int MODE>
__device__ __forceinline__ void expert_stream(const ExpertGemmArgs& a, v4i (&b0)[kExpertSlab],
                                              v4i (&b1)[kExpertSlab], const int8_t* As, const float* sas,
                                              const float* sws, const float* sbs, const int8_t* wexp, int wave,
                                              int lane, int t_begin, int nj, int nch, int p0, int seg1,
                                              uint32_t* lmax) {
    const int N = a.N, kt = a.kt, NW = a.streams;
    const int r16 = lane & 15, g = lane >> 4;
    auto load_chunk = [&](v4i (&b)[kExpertSlab], int j) {
        const int t = t_begin + wave + (j / nch) * NW, k0 = (j % nch) * kExpertSlab;
        const __amdgpu_buffer_rsrc_t wr =
            j < nj ? make_rsrc(wexp + (int64_t)t * kt * 1024, (uint32_t)kt * 1024u) : make_rsrc(wexp, 0);
#pragma unroll
        for (int s = 0; s < kExpertSlab; ++s) b[s] = buffer_load16_stream(wr, (k0 + s) * 1024 + lane * 16);
    };
    v4i acc[NRB];
    // kExpertOmax: this lane's running max of the finite |out| of its rows
    // (its own columns; the 16 lanes of a row group meet at the pass end)
    float rmax[NRB][4];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
        for (int r = 0; r < 4; ++r) rmax[rb][r] = 0.0f;
    auto process = [&](const v4i (&b)[kExpertSlab], int j) {
        const int c = j % nch, k0 = c * kExpertSlab;
        if (c == 0) {
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb) acc[rb] = v4i{0, 0, 0, 0};
        }
        // A fragments one K tile ahead of the MFMAs (the order pinned, so the
        // fragment reads do not pile up in registers)
        v4i af[2][NRB];
        auto read_a = [&](v4i (&f)[NRB], int s) {
            const int kk = k0 + s < kt ? k0 + s : 0;
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb) f[rb] = *(const v4i*)(As + (rb * kt + kk) * 1024 + lane * 16);
        };
        read_a(af[0], 0);
#pragma unroll
        for (int s = 0; s < kExpertSlab; ++s) {
            if (s + 1 < kExpertSlab) read_a(af[(s + 1) & 1], s + 1);
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb)
                acc[rb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[s & 1][rb], b[s], acc[rb], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        const int n = (t_begin + wave + (j / nch) * NW) * 16 + r16;
        // j >= nj: the chunk after the wave's last (an odd chunk count runs
        // one past it with zero weights); its tile may belong to the other
        // workgroup of the expert, so it stores nothing
        if (j < nj && c == nch - 1 && n < N) {
            const float swn = sws[n - t_begin * 16];
            const float bn = a.bias ? sbs[n - t_begin * 16] : 0.0f;
            // one per-lane base (row p0 + 4 g, column n); rows rb * 16 + r are
            // uniform offsets (row-major, or 16 floats apart in column-tile order)
            float* ob = a.out_tcol ? a.out + ((int64_t)(n >> 4) * a.out_rows + p0 + 4 * g) * 16 + (n & 15)
                                   : a.out + (int64_t)(p0 + 4 * g) * N + n;
            const int rs = a.out_tcol ? 16 : N;
            const int rows = seg1 - p0 - 4 * g;  // rows of this lane's group in the pass
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (rb * 16 + r < rows) {
                        float y = epilogue_w8a8(acc[rb][r], sas[rb * 16 + 4 * g + r], swn);
                        if (a.bias) y = y + bn;
                        if (a.relu2) y = relu2(y);
                        ob[(rb * 16 + r) * rs] = y;
                        if constexpr (MODE == kExpertOmax) {
                            if (is_finite_f32(y))
                                rmax[rb][r] = fmaxf(rmax[rb][r], fabsf(y));
                            else if (a.nonfinite)
                                report_nonfinite(a.nonfinite, a.nonfinite_stage,
                                                 (int64_t)(p0 + 4 * g + rb * 16 + r) * N + n, y);
                        }
                    }
        }
    };
    // chunks in pairs: while one slab's MFMAs run, the other is in flight
    // (a chunk past nj has zero weights and writes nothing)
    for (int j = 0; j < nj; j += 2) {
        process(b0, j);
        load_chunk(b0, j + 2);
        process(b1, j + 1);
        load_chunk(b1, j + 3);
    }
    if constexpr (MODE == kExpertOmax) {
        // the row group's 16 lanes (one column each), then the waves (LDS max
        // of the bit patterns: non-negative floats order like their bits)
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t m = row16_max_u32(f32_bits(rmax[rb][r]));  // DPP, within the 16-lane row
                if (r16 == 0) atomicMax(&lmax[rb * 16 + 4 * g + r], m);
            }
    }
}

// The three forms of the expert-block kernel:
//  kExpertPlain  A codes in slot order (aq, sa) staged by direct-to-LDS loads;
//  kExpertOmax   the same, and each workgroup also writes, for every row of
//                its segment, the largest finite |out| over its own columns
//                (omax[row][blockIdx.x], f32 bits) and reports non-finite
//                outputs: the up projection of the MoE layer, whose output
//                the down projection requantizes per row;
//  kExpertQuantA A rows in f32 (ah), quantized per row while staged, with
//                the row scale RN(amax / 127) from amax = the larger of the
//                row's two omax entries: the max of the finite |h| over the
//                whole row, so the codes and scales are those of
//                nh_quantize_rows_i8 on h (the down projection; K <= 2048:
//                a wave stages 4 K tiles of each row block).  That fuses
//                the intermediate requantization of mlp.rs:201-208 into the
//                two projections instead of a launch and an int8 copy.
template <int MODE>
__device__ __forceinline__ void expert_gemm(const ExpertGemmArgs& a, int8_t* lds) {
    const int e = blockIdx.y;
    const int seg0 = a.offsets[e], seg1 = a.offsets[e + 1];
    if (seg0 >= seg1) return;  // no routes: the expert's weights are never read
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int NW = a.streams;
    const int r16 = lane & 15, g = lane >> 4;
    const int N = a.N, K = a.K, kt = a.kt;
    const int nch = (kt + kExpertSlab - 1) / kExpertSlab;
    const int RB = a.row_blocks, cap = 16 * RB;
    const int ntiles = (N + 15) / 16;
    const int t_begin = blockIdx.x * a.tiles_per_wg;
    const int t_end = min(t_begin + a.tiles_per_wg, ntiles);
    if (t_begin >= t_end) {  // uniform: no columns here, so no output of this range is non-zero
        if constexpr (MODE == kExpertOmax)
            for (int row = seg0 + (int)threadIdx.x; row < seg1; row += blockDim.x) a.omax[row * 2 + blockIdx.x] = 0u;
        return;
    }
    const int my_tiles = t_begin + wave < t_end ? (t_end - t_begin - wave + NW - 1) / NW : 0;
    const int nj = my_tiles * nch;  // this wave's chunks
    const int nw_cols = min(t_end * 16, N) - t_begin * 16;  // this workgroup's weight rows
    int8_t* As = lds;                                // [RB][kt] A tiles
    float* sas = (float*)(lds + RB * kt * 1024);     // [16 RB] the pass's row scales
    uint32_t* lmax = (uint32_t*)(sas + 16 * RB);     // [64] kExpertOmax: the pass's row maxima
    float* sws = (float*)(lmax + 64);                // [16 tiles_per_wg, rounded up to 64] weight scales
    float* sbs = sws + (16 * a.tiles_per_wg + 63) / 64 * 64;  // the same for the bias (when a.bias)
    const __amdgpu_buffer_rsrc_t swr = make_rsrc(a.sw + (int64_t)e * N + t_begin * 16, (uint32_t)nw_cols * 4u);
    const __amdgpu_buffer_rsrc_t sbr =
        make_rsrc(a.bias ? a.bias + (int64_t)e * N + t_begin * 16 : a.sw, a.bias ? (uint32_t)nw_cols * 4u : 0u);
    // the workgroup's weight scales (and bias) straight into LDS, 64 floats per wave instruction
    auto stage_scales = [&]() {
        for (int i = wave * 64; i < nw_cols; i += NW * 64) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(swr, (lds_void_t*)(sws + i), 4, (uint32_t)(i + lane) * 4u, 0,
                                                     0, 0);
            if (a.bias)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(sbr, (lds_void_t*)(sbs + i), 4, (uint32_t)(i + lane) * 4u,
                                                         0, 0, 0);
        }
    };
    const int8_t* wexp = a.w + (int64_t)e * tiled_bytes(N, K);
    v4i b0[kExpertSlab], b1[kExpertSlab];
    auto first = [&](v4i (&b)[kExpertSlab], int j) {
        const int t = t_begin + wave + (j / nch) * NW, k0 = (j % nch) * kExpertSlab;
        const __amdgpu_buffer_rsrc_t wr =
            j < nj ? make_rsrc(wexp + (int64_t)t * kt * 1024, (uint32_t)kt * 1024u) : make_rsrc(wexp, 0);
#pragma unroll
        for (int s = 0; s < kExpertSlab; ++s) b[s] = buffer_load16_stream(wr, (k0 + s) * 1024 + lane * 16);
    };
    for (int p0 = seg0; p0 < seg1; p0 += cap) {
        const int nrb = (min(cap, seg1 - p0) + 15) / 16;  // uniform
        if constexpr (MODE == kExpertOmax)
            if (threadIdx.x < 64) lmax[threadIdx.x] = 0u;  // published by the barrier below
        if constexpr (MODE != kExpertQuantA) {
            // 1. the pass's A tiles, the weight scales (straight to LDS: a global
            //    load in the epilogue would make the wave wait for its weight
            //    loads in flight) and the row scales, then this wave's first two chunks
            const __amdgpu_buffer_rsrc_t ar = make_rsrc(a.aq, (uint32_t)a.a_rows * (uint32_t)K);
            float sav = 0.0f;
            if (!a.perm) {
                __builtin_amdgcn_sched_barrier(0);
                for (int i = wave; i < nrb * kt; i += NW) {
                    const int rb = i / kt, t = i - rb * kt;
                    const int slot = p0 + rb * 16 + r16;
                    const uint32_t off = (uint32_t)slot * (uint32_t)K + (uint32_t)(t * 64 + g * 16);
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(ar, (lds_void_t*)(As + i * 1024), 16,
                                                             slot < seg1 ? off : (uint32_t)kOutOfRange, 0, 0, 0);
                }
                stage_scales();
                if ((int)threadIdx.x < cap && p0 + (int)threadIdx.x < seg1) sav = a.sa[p0 + threadIdx.x];
                __builtin_amdgcn_sched_barrier(0);
                first(b0, 0);
                first(b1, 1);
                __builtin_amdgcn_sched_barrier(0);
                wait_vmcnt_le(2 * kExpertSlab);  // A and scale loads in, weights in flight
            } else {
                // gathered A: row (and scale) of slot s is perm[s] / gather_div.
                // The permutation entries of this lane's rows go out ahead of
                // the weights, so waiting for them leaves the weights in
                // flight; the A rows (L2) then arrive under the weights'
                // latency (HBM).
                // (unconditional loads: entries past the segment read zeros and are masked)
                const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.perm, (uint32_t)seg1 * 4u);
                int tok[4];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int rb = 0; rb < 4; ++rb)
                    tok[rb] = __builtin_amdgcn_raw_buffer_load_b32(pr, (p0 + rb * 16 + r16) * 4, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                first(b0, 0);
                first(b1, 1);
                __builtin_amdgcn_sched_barrier(0);
                wait_vmcnt_le(2 * kExpertSlab);  // the permutation entries in, weights in flight
#pragma unroll
                for (int rb = 0; rb < 4; ++rb)
                    tok[rb] = rb < nrb && p0 + rb * 16 + r16 < seg1 ? tok[rb] / a.gather_div : -1;
                for (int i = wave; i < nrb * kt; i += NW) {
                    const int rb = i / kt, t = i - rb * kt;
                    const int tr = rb == 0 ? tok[0] : rb == 1 ? tok[1] : rb == 2 ? tok[2] : tok[3];
                    const uint32_t off = (uint32_t)tr * (uint32_t)K + (uint32_t)(t * 64 + g * 16);
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(ar, (lds_void_t*)(As + i * 1024), 16,
                                                             tr >= 0 ? off : (uint32_t)kOutOfRange, 0, 0, 0);
                }
                stage_scales();
                // thread t < cap holds slot p0 + t: row block t / 16 = g of its wave 0 lane
                if ((int)threadIdx.x < cap) {
                    const int tr = g == 0 ? tok[0] : g == 1 ? tok[1] : g == 2 ? tok[2] : tok[3];
                    if (tr >= 0) sav = a.sa[tr];
                }
                wait_vmcnt_le(0);  // A, scales and the first chunks
            }
            if ((int)threadIdx.x < cap) sas[threadIdx.x] = sav;
        } else {
            // 1. the A rows: f32 from ah, quantized with the row's scale into
            //    the MFMA tile layout of the DMA form (lane l: row l % 16 of
            //    the block, 16 codes at 16 (l / 16)); the 4 row blocks in a
            //    two-deep pipeline of 4 K tiles per lane, with this wave's
            //    first two weight chunks issued behind the first two blocks
            const __amdgpu_buffer_rsrc_t hr = make_rsrc(a.ah, (uint32_t)a.a_rows * (uint32_t)K * 4u);
            uint32_t hm[4][2];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                const int row = p0 + rb * 16 + r16;
                const bool ok = rb < nrb && row < seg1;
                hm[rb][0] = ok ? a.ahmax[row * 2] : 0u;
                hm[rb][1] = ok ? a.ahmax[row * 2 + 1] : 0u;
            }
            v4i hv[2][4][4];
            // the lane's 16 values of a K tile: 64 contiguous bytes in either order
            auto piece = [&](int row, int t) -> uint32_t {
                return a.ah_tcol ? ((uint32_t)(t * 4 + g) * (uint32_t)a.a_rows + (uint32_t)row) * 64u
                                 : ((uint32_t)row * (uint32_t)K + (uint32_t)(t * 64 + g * 16)) * 4u;
            };
            auto issue = [&](int rb, v4i (&buf)[4][4]) {
                const int row = p0 + rb * 16 + r16;
                const bool ok = rb < nrb && row < seg1;
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int t = wave + u * NW;
                        const uint32_t off = piece(row, t) + (uint32_t)(16 * q);
                        buf[u][q] = buffer_load16(hr, ok && t < kt ? (int)off : kOutOfRange);
                    }
            };
            auto consume = [&](int rb, const v4i (&buf)[4][4]) {
                if (rb >= nrb) return;  // uniform
                const float sc = scale_from_amax(fmaxf(f32_from_bits(hm[rb][0]), f32_from_bits(hm[rb][1])));
                const float rcp = sc > 0.0f ? 1.0f / sc : 0.0f;
                const bool pow2 = scale_is_pow2(sc);
                if (g == 0) sas[rb * 16 + r16] = sc;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int t = wave + u * NW;
                    if (t >= kt) break;
                    float v[16];
#pragma unroll
                    for (int q = 0; q < 4; ++q)
#pragma unroll
                        for (int w4 = 0; w4 < 4; ++w4) v[4 * q + w4] = f32_from_bits((uint32_t)buf[u][q][w4]);
                    uint32_t qc[16];
                    quantize_values<16>(v, sc, rcp, pow2, qc);
                    const v4i codes = {(int)pack_codes4(qc[0], qc[1], qc[2], qc[3]),
                                       (int)pack_codes4(qc[4], qc[5], qc[6], qc[7]),
                                       (int)pack_codes4(qc[8], qc[9], qc[10], qc[11]),
                                       (int)pack_codes4(qc[12], qc[13], qc[14], qc[15])};
                    *(v4i*)(As + (rb * kt + t) * 1024 + lane * 16) = codes;
                }
            };
            issue(0, hv[0]);
            issue(1, hv[1]);
            __builtin_amdgcn_sched_barrier(0);
            first(b0, 0);
            stage_scales();
            __builtin_amdgcn_sched_barrier(0);
            consume(0, hv[0]);
            issue(2, hv[0]);
            consume(1, hv[1]);
            issue(3, hv[1]);
            consume(2, hv[0]);
            consume(3, hv[1]);
            // the second chunk is not read before the first one's MFMAs
            __builtin_amdgcn_sched_barrier(0);
            first(b1, 1);
            __builtin_amdgcn_sched_barrier(0);
            wait_vmcnt_le(kExpertSlab);  // the weight scales' (and bias') direct-to-LDS loads in, the second chunk in flight
        }
        lds_publish();  // every wave's A tiles and the scales
        switch (nrb) {
        case 1: expert_stream<1, MODE>(a, b0, b1, As, sas, sws, sbs, wexp, wave, lane, t_begin, nj, nch, p0, seg1, lmax); break;
        case 2: expert_stream<2, MODE>(a, b0, b1, As, sas, sws, sbs, wexp, wave, lane, t_begin, nj, nch, p0, seg1, lmax); break;
        case 3: expert_stream<3, MODE>(a, b0, b1, As, sas, sws, sbs, wexp, wave, lane, t_begin, nj, nch, p0, seg1, lmax); break;
        default: expert_stream<4, MODE>(a, b0, b1, As, sas, sws, sbs, wexp, wave, lane, t_begin, nj, nch, p0, seg1, lmax); break;
        }
        lds_publish();  // the pass's A and scale reads are done before the next pass restages them
        if constexpr (MODE == kExpertOmax)
            if ((int)threadIdx.x < nrb * 16 && p0 + (int)threadIdx.x < seg1)
                a.omax[(p0 + threadIdx.x) * 2 + blockIdx.x] = lmax[threadIdx.x];
    }
}

extern "C" __global__ __launch_bounds__(512) void nh_moe_expert_gemm_kernel(ExpertGemmArgs a) {
    extern __shared__ __align__(16) int8_t lds[];
    expert_gemm<kExpertPlain>(a, lds);
}

extern "C" __global__ __launch_bounds__(512) void nh_moe_expert_gemm_omax_kernel(ExpertGemmArgs a) {
    extern __shared__ __align__(16) int8_t lds[];
    expert_gemm<kExpertOmax>(a, lds);
}

extern "C" __global__ __launch_bounds__(512) void nh_moe_expert_gemm_qa_kernel(ExpertGemmArgs a) {
    extern __shared__ __align__(16) int8_t lds[];
    expert_gemm<kExpertQuantA>(a, lds);
}

// R4: out[t][h] = sum_j w[t,j] * slot_out[pos[t*k+j]][h], j ascending, f32
// multiply then add (moe.rs:239-244).  grid = (ceil(H/256), T).
// A route whose slot is outside [0, routes) (an expert id the permutation
// did not place: pos = -1) adds nothing.
extern "C" __global__ __launch_bounds__(256) void nh_moe_combine_kernel(CombineArgs a) {
    const int t = blockIdx.y;
    const int h = blockIdx.x * blockDim.x + threadIdx.x;
    if (h >= a.hidden) return;
    const int routes = a.tokens * a.top_k;
    float v = 0.0f;
    if (a.shared) v = v + a.shared[(int64_t)t * a.hidden + h];  // the shared expert first (moe.rs:212-219)
    for (int j = 0; j < a.top_k; ++j) {
        const int r = t * a.top_k + j;
        const int slot = a.pos[r];
        if (slot < 0 || slot >= routes) continue;
        const float w = a.weights[r];
        const float x = a.slot_out[(int64_t)slot * a.hidden + h];
        const float p = w * x;
        v = v + p;
    }
    store_out(a.out, (int64_t)t * a.hidden + h, v, a.out_dtype);
}

// The same with four consecutive columns per thread (16-byte loads of the
// slot rows; hidden % 4 == 0, 16-byte aligned rows): every element is
// summed exactly as above.
extern "C" __global__ __launch_bounds__(256) void nh_moe_combine4_kernel(CombineArgs a) {
    const int t = blockIdx.y;
    const int h = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
    if (h >= a.hidden) return;
    const int routes = a.tokens * a.top_k;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (a.shared) {
        const float4 sh = *(const float4*)(a.shared + (int64_t)t * a.hidden + h);
        v[0] = v[0] + sh.x;
        v[1] = v[1] + sh.y;
        v[2] = v[2] + sh.z;
        v[3] = v[3] + sh.w;
    }
    for (int j = 0; j < a.top_k; ++j) {
        const int r = t * a.top_k + j;
        const int slot = a.pos[r];
        if (slot < 0 || slot >= routes) continue;
        const float w = a.weights[r];
        const float4 x = *(const float4*)(a.slot_out + (int64_t)slot * a.hidden + h);
        v[0] = v[0] + w * x.x;
        v[1] = v[1] + w * x.y;
        v[2] = v[2] + w * x.z;
        v[3] = v[3] + w * x.w;
    }
    const int64_t o = (int64_t)t * a.hidden + h;
    if (a.out_dtype == DT_BF16) {
        const uint32_t lo = (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
        const uint32_t hi = (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
        *(uint2*)((uint16_t*)a.out + o) = make_uint2(lo, hi);
    } else {
        *(float4*)((float*)a.out + o) = make_float4(v[0], v[1], v[2], v[3]);
    }
}
