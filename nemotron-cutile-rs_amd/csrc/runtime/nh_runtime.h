// Internal runtime of libnemotron_hip: the context (one loaded gfx950 code
// object per device), kernel launch, and error plumbing shared by the C ABI.
#pragma once
#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cstdarg>
#include <cstddef>
#include <cstdint>

#include "../kernels/nh_kernel_args.h"
#include "../kernels/nh_numerics.h"
#include "nemotron_hip.h"

namespace nh {

enum KernelId : int {
    K_QUANTIZE_ROWS = 0,
    K_DEQUANT_I8,
    K_DEQUANT_INT4,
    K_GEMV_W8A8,
    K_LINEAR_DECODE,     // M <= 4
    K_LINEAR_DECODE_M1,  // M == 1
    K_LINEAR_DECODE_M2,  // M <= 2
    K_GEMV_W8A32,
    K_GEMV_W8A32_M1,
    K_GEMM_W8A8,
    K_GEMM_W8A8_128,
    K_ROUTE_SIGMOID,
    K_PERMUTE,
    K_GROUPED_GEMM,
    K_COMBINE,
    K_TILE_WEIGHTS,
    K_GEMM_TA_256,       // tiled A, 256 x 128
    K_GEMM_TA_128,       // tiled A, 128 x 128
    K_GEMM_F32,
    K_GEMV_W8A8_XT,      // activation tiles
    K_LINEAR_DECODE_M8,  // M <= 8
    K_LINEAR_DECODE_STREAM_M8,  // 5..8 rows, any N, K <= 4096
    K_LINEAR_DECODE_STREAM_M4,  // 3..4 rows
    K_LINEAR_DECODE_STREAM_M16,  // 9..16 rows
    K_LINEAR_DECODE_STREAM_W4_M4,  // the same on tiled INT4 weights
    K_LINEAR_DECODE_STREAM_W4_M8,
    K_LINEAR_DECODE_ROW2,  // M <= 2, one N tile per workgroup
    K_LINEAR_DECODE_ROW4,  // M <= 4, one N tile per workgroup
    K_EXPERT_GEMM,         // grouped GEMM on slot-ordered A
    K_EXPERT_GEMM_OMAX,    // ... also writing per-row output maxima (MoE up projection)
    K_EXPERT_GEMM_QA,      // ... quantizing f32 A rows while staging them (MoE down projection)
    K_STREAM_READ,         // diagnostic read stream
    K_QUANTIZE_ROWS_WAVE,  // row quantizer, one wave per row
    K_QUANTIZE_TILES,      // row quantizer into GEMM A tiles, 8 rows per workgroup
    K_LINEAR_HANDOFF,      // row quantizer + tiled-A GEMV in one launch (M <= 16)
    K_QUANTIZE_ROWS_LONG,  // row quantizer, 1024 threads per row
    K_QUANTIZE_ROWS_PMAX,  // f32 rows with producer-reduced maxima, many workgroups per row
    K_EXPAND_INT4,         // tiled INT4 -> tiled int8 code - zp
    K_TILE_INT4,           // INT4 [K][N] packed -> tiled INT4
    K_LINEAR_DECODE_W4_M1,    // W4A8 decode unit, 1 row
    K_LINEAR_DECODE_W4_ROW2,  // 2 rows
    K_LINEAR_DECODE_W4_ROW4,  // 4 rows
    K_PERMUTE_EXPERT,         // R2, one workgroup per expert
    K_COMBINE4,               // R4, four columns per thread
    K_GEMM_P224,              // persistent G3, 256 x 224 tiles, tiled A
    K_GEMM_TA_64,             // G3, 64 x 128 tiles, tiled A
    K_LINEAR_DECODE_STREAM_W4_M16,  // W4A8 streaming decode unit, 9..16 rows
    K_GEMM_TA_6464,           // G3, 64 x 64 tiles, tiled A
    K_GEMM_F32_MFMA,          // G0d on the f64 matrix cores, 16 x 16 outputs per workgroup, f32 lhs
    K_GEMM_F32_MFMA_BF16,     // ... bf16 lhs
    K_GEMM_F32_MFMA_ANY,      // ... any alignment, K and N
    K_QUANTIZE_ROWS_R11,      // row quantizer, 256 threads per row, up to 2816 chunks in registers
    K_COUNT
};

extern const char* const kKernelSymbols[K_COUNT];

// Bytes of the static device scratch (scratch.hip) that nh_linear_w8a8_noalloc
// uses as its workspace.
constexpr size_t kScratchBytes = 64ull << 20;

// Counter slots of the in-launch handoff ring (64 bytes each): two calls
// that share a slot must not run at the same time, i.e. at most
// kHandoffSlots handoff launches may be in flight at once on one context.
constexpr uint32_t kHandoffSlots = 256;

}  // namespace nh

struct nh_context {
    int device;
    hipModule_t module;
    hipFunction_t fn[nh::K_COUNT];
    int max_threads[nh::K_COUNT];   // each kernel's HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK
    int static_lds[nh::K_COUNT];    // and its static LDS bytes
    int cu_count;
    size_t max_shared_per_block;
    void* scratch;             // this device's address of the static scratch, or null
    char scratch_error[128];   // why it is null
    // counter slots of the in-launch handoff (nh_linear_handoff_kernel):
    // kHandoffSlots blocks of 64 bytes, zeroed at creation; every launch
    // leaves its slot zeroed again.  Calls take the slots in turn.
    uint32_t* handoff;
    std::atomic<uint32_t> handoff_next;
};

namespace nh {

nh_status set_error(nh_error* err, nh_status st, const char* fmt, ...);
nh_status mismatch(nh_error* err, const char* argument, uint64_t expected, uint64_t actual);
nh_status device_error(nh_error* err, hipError_t e, const char* what);
void clear_error(nh_error* err);

// Makes ctx->device current for the calling thread.
nh_status bind_device(nh_context* ctx, nh_error* err);

// Device address of the static scratch on the current device (scratch.hip).
nh_status scratch_address(void** out, nh_error* err);

// Launches kernel `id`.  A block larger than the kernel's compiled limit
// (its __launch_bounds__, read from the code object at context creation) or
// LDS beyond the device's per-workgroup size is refused before it reaches the
// GPU: launched, either would run the kernel outside what it was compiled for.
template <class Args>
nh_status launch(nh_context* ctx, KernelId id, unsigned gx, unsigned bx, size_t shmem, nh_stream stream,
                 const Args& args, nh_error* err, unsigned gy = 1) {
    if (bx == 0 || (int)bx > ctx->max_threads[id])
        return set_error(err, NH_DEVICE_ERROR, "%s: launch of %u x %u blocks of %u threads (kernel limit %d)",
                         kKernelSymbols[id], gx, gy, bx, ctx->max_threads[id]);
    if (shmem + (size_t)ctx->static_lds[id] > ctx->max_shared_per_block)
        return set_error(err, NH_DEVICE_ERROR, "%s: %zu bytes of LDS requested (%zu available)", kKernelSymbols[id],
                         shmem + (size_t)ctx->static_lds[id], ctx->max_shared_per_block);
    void* params[] = {const_cast<Args*>(&args)};
    hipError_t e = hipModuleLaunchKernel(ctx->fn[id], gx, gy, 1, bx, 1, 1, (unsigned)shmem, (hipStream_t)stream,
                                         params, nullptr);
    if (e != hipSuccess) return device_error(err, e, kKernelSymbols[id]);
    return NH_OK;
}

inline bool mul_ok(size_t a, size_t b, size_t* out) { return !__builtin_mul_overflow(a, b, out); }
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace nh
