// Context, buffers, streams, registry and error plumbing of the C ABI.
#include <cstdio>
#include <cstring>
#include <new>

#include "nh_runtime.h"

// The gfx950 code object, linked in by code_object.S (.incbin).
extern "C" const unsigned char nh_gfx950_code_object[];
extern "C" const unsigned char nh_gfx950_code_object_end[];

namespace nh {

const char* const kKernelSymbols[K_COUNT] = {  // in KernelId order
    "nh_quantize_rows_i8_kernel",        // K_QUANTIZE_ROWS
    "nh_dequantize_i8_kernel",           // K_DEQUANT_I8
    "nh_dequantize_int4_kernel",         // K_DEQUANT_INT4
    "nh_gemv_w8a8_kernel",               // K_GEMV_W8A8
    "nh_linear_decode_w8a8_kernel",      // K_LINEAR_DECODE
    "nh_linear_decode_w8a8_m1_kernel",   // K_LINEAR_DECODE_M1
    "nh_linear_decode_w8a8_m2_kernel",   // K_LINEAR_DECODE_M2
    "nh_gemv_w8a32_kernel",              // K_GEMV_W8A32
    "nh_gemv_w8a32_m1_kernel",           // K_GEMV_W8A32_M1
    "nh_gemm_w8a8_256x128_kernel",       // K_GEMM_W8A8
    "nh_gemm_w8a8_128x128_kernel",       // K_GEMM_W8A8_128
    "nh_moe_route_sigmoid_kernel",       // K_ROUTE_SIGMOID
    "nh_moe_permute_kernel",             // K_PERMUTE
    "nh_moe_grouped_gemm_kernel",        // K_GROUPED_GEMM
    "nh_moe_combine_kernel",             // K_COMBINE
    "nh_tile_weights_kernel",            // K_TILE_WEIGHTS
    "nh_gemm_w8a8_ta_256x128_kernel",    // K_GEMM_TA_256
    "nh_gemm_w8a8_ta_128x128_kernel",    // K_GEMM_TA_128
    "nh_gemm_f32_kernel",                // K_GEMM_F32
    "nh_gemv_w8a8_xt_kernel",            // K_GEMV_W8A8_XT
    "nh_linear_decode_w8a8_m8_kernel",   // K_LINEAR_DECODE_M8
    "nh_linear_decode_stream_m8_kernel",  // K_LINEAR_DECODE_STREAM_M8
    "nh_linear_decode_stream_m4_kernel",  // K_LINEAR_DECODE_STREAM_M4
    "nh_linear_decode_stream_m16_kernel",  // K_LINEAR_DECODE_STREAM_M16
    "nh_linear_decode_stream_w4_m4_kernel",  // K_LINEAR_DECODE_STREAM_W4_M4
    "nh_linear_decode_stream_w4_m8_kernel",  // K_LINEAR_DECODE_STREAM_W4_M8
    "nh_linear_decode_w8a8_row2_kernel", // K_LINEAR_DECODE_ROW2
    "nh_linear_decode_w8a8_row4_kernel", // K_LINEAR_DECODE_ROW4
    "nh_moe_expert_gemm_kernel",         // K_EXPERT_GEMM
    "nh_moe_expert_gemm_omax_kernel",    // K_EXPERT_GEMM_OMAX
    "nh_moe_expert_gemm_qa_kernel",      // K_EXPERT_GEMM_QA
    "nh_stream_read_kernel",             // K_STREAM_READ
    "nh_quantize_rows_wave_kernel",      // K_QUANTIZE_ROWS_WAVE
    "nh_quantize_tiles_kernel",          // K_QUANTIZE_TILES
    "nh_linear_handoff_kernel",          // K_LINEAR_HANDOFF
    "nh_quantize_rows_long_kernel",      // K_QUANTIZE_ROWS_LONG
    "nh_quantize_rows_pmax_kernel",      // K_QUANTIZE_ROWS_PMAX
    "nh_expand_int4_tiles_kernel",       // K_EXPAND_INT4
    "nh_tile_weights_int4_kernel",       // K_TILE_INT4
    "nh_linear_decode_w4a8_m1_kernel",   // K_LINEAR_DECODE_W4_M1
    "nh_linear_decode_w4a8_row2_kernel", // K_LINEAR_DECODE_W4_ROW2
    "nh_linear_decode_w4a8_row4_kernel", // K_LINEAR_DECODE_W4_ROW4
    "nh_moe_permute_expert_kernel",      // K_PERMUTE_EXPERT
    "nh_moe_combine4_kernel",            // K_COMBINE4
    "nh_gemm_w8a8_p256x224_kernel",      // K_GEMM_P224
    "nh_gemm_w8a8_ta_64x128_kernel",     // K_GEMM_TA_64
    "nh_linear_decode_stream_w4_m16_kernel",  // K_LINEAR_DECODE_STREAM_W4_M16
    "nh_gemm_w8a8_ta_64x64_kernel",      // K_GEMM_TA_6464
    "nh_gemm_f32_mfma_kernel",           // K_GEMM_F32_MFMA
    "nh_gemm_f32_mfma_bf16_kernel",      // K_GEMM_F32_MFMA_BF16
    "nh_gemm_f32_mfma_any_kernel",       // K_GEMM_F32_MFMA_ANY
    "nh_quantize_rows_r11_kernel",       // K_QUANTIZE_ROWS_R11
};

void clear_error(nh_error* err) {
    if (err) std::memset(err, 0, sizeof(*err));
}

nh_status set_error(nh_error* err, nh_status st, const char* fmt, ...) {
    if (err) {
        va_list ap;
        va_start(ap, fmt);
        std::vsnprintf(err->message, sizeof(err->message), fmt, ap);
        va_end(ap);
    }
    return st;
}

nh_status mismatch(nh_error* err, const char* argument, uint64_t expected, uint64_t actual) {
    if (err) {
        err->argument = argument;
        err->expected = expected;
        err->actual = actual;
        std::snprintf(err->message, sizeof(err->message), "%s length mismatch: expected %llu, got %llu", argument,
                      (unsigned long long)expected, (unsigned long long)actual);
    }
    return NH_LENGTH_MISMATCH;
}

nh_status device_error(nh_error* err, hipError_t e, const char* what) {
    return set_error(err, NH_DEVICE_ERROR, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

nh_status bind_device(nh_context* ctx, nh_error* err) {
    if (!ctx) return set_error(err, NH_INVALID_PARAMS, "null context");
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return device_error(err, e, "hipGetDevice");
    if (cur != ctx->device) {
        e = hipSetDevice(ctx->device);
        if (e != hipSuccess) return device_error(err, e, "hipSetDevice");
    }
    return NH_OK;
}

}  // namespace nh

using namespace nh;

extern "C" {

int nh_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

nh_status nh_context_create(int device, const char* code_object_path, nh_context** out, nh_error* err) {
    clear_error(err);
    if (!out) return set_error(err, NH_INVALID_PARAMS, "null output pointer");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return device_error(err, e, "hipGetDeviceCount");
    if (device < 0 || device >= count)
        return set_error(err, NH_DEVICE_ERROR, "device %d out of range (%d devices)", device, count);
    e = hipSetDevice(device);
    if (e != hipSuccess) return device_error(err, e, "hipSetDevice");
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return device_error(err, e, "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return set_error(err, NH_DEVICE_ERROR, "device %d is %s; this library is built for gfx950 only", device,
                         prop.gcnArchName);
    nh_context* ctx = new (std::nothrow) nh_context();
    if (!ctx) return set_error(err, NH_DEVICE_ERROR, "out of host memory");
    ctx->device = device;
    ctx->cu_count = prop.multiProcessorCount;
    ctx->max_shared_per_block = prop.sharedMemPerBlock;
    // the static scratch's address on this device (the device is current);
    // only nh_linear_w8a8_noalloc needs it, so a failure is kept for it to report
    nh_error serr;
    clear_error(&serr);
    if (scratch_address(&ctx->scratch, &serr) != NH_OK)
        std::snprintf(ctx->scratch_error, sizeof(ctx->scratch_error), "%.120s", serr.message);
    if (code_object_path)
        e = hipModuleLoad(&ctx->module, code_object_path);
    else
        e = hipModuleLoadData(&ctx->module, nh_gfx950_code_object);
    if (e != hipSuccess) {
        delete ctx;
        return device_error(err, e, "hipModuleLoad(gfx950 code object)");
    }
    for (int i = 0; i < K_COUNT; ++i) {
        e = hipModuleGetFunction(&ctx->fn[i], ctx->module, kKernelSymbols[i]);
        if (e != hipSuccess) {
            (void)hipModuleUnload(ctx->module);
            delete ctx;
            return device_error(err, e, kKernelSymbols[i]);
        }
        e = hipFuncGetAttribute(&ctx->max_threads[i], HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, ctx->fn[i]);
        if (e == hipSuccess)
            e = hipFuncGetAttribute(&ctx->static_lds[i], HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, ctx->fn[i]);
        if (e != hipSuccess) {
            (void)hipModuleUnload(ctx->module);
            delete ctx;
            return device_error(err, e, "hipFuncGetAttribute");
        }
    }
    // the handoff ring, zeroed before any launch can use it
    void* ring = nullptr;
    e = hipMalloc(&ring, (size_t)kHandoffSlots * 64);
    if (e == hipSuccess) e = hipMemset(ring, 0, (size_t)kHandoffSlots * 64);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        if (ring) (void)hipFree(ring);
        (void)hipModuleUnload(ctx->module);
        delete ctx;
        return device_error(err, e, "handoff counters");
    }
    ctx->handoff = (uint32_t*)ring;
    ctx->handoff_next.store(0);
    *out = ctx;
    return NH_OK;
}

void nh_context_destroy(nh_context* ctx) {
    if (!ctx) return;
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) cur = -1;
    (void)hipSetDevice(ctx->device);
    if (ctx->handoff) (void)hipFree(ctx->handoff);
    (void)hipModuleUnload(ctx->module);
    if (cur >= 0) (void)hipSetDevice(cur);
    delete ctx;
}

int nh_context_device(const nh_context* ctx) { return ctx ? ctx->device : -1; }

nh_status nh_malloc(nh_context* ctx, size_t bytes, void** ptr, nh_error* err) {
    clear_error(err);
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    if (!ptr) return set_error(err, NH_INVALID_PARAMS, "null output pointer");
    hipError_t e = hipMalloc(ptr, bytes ? bytes : 1);
    if (e != hipSuccess) return device_error(err, e, "hipMalloc");
    return NH_OK;
}

nh_status nh_free(nh_context* ctx, void* ptr, nh_error* err) {
    clear_error(err);
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    hipError_t e = hipFree(ptr);
    if (e != hipSuccess) return device_error(err, e, "hipFree");
    return NH_OK;
}

nh_status nh_memcpy_htod(nh_context* ctx, void* dst, const void* src, size_t bytes, nh_error* err) {
    clear_error(err);
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    if (bytes == 0) return NH_OK;
    hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) return device_error(err, e, "hipMemcpy(HtoD)");
    return NH_OK;
}

nh_status nh_memcpy_dtoh(nh_context* ctx, void* dst, const void* src, size_t bytes, nh_error* err) {
    clear_error(err);
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    if (bytes == 0) return NH_OK;
    hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return device_error(err, e, "hipMemcpy(DtoH)");
    return NH_OK;
}

nh_status nh_memset_d8(nh_context* ctx, void* dst, int value, size_t bytes, nh_error* err) {
    clear_error(err);
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    if (bytes == 0) return NH_OK;
    hipError_t e = hipMemset(dst, value, bytes);
    if (e != hipSuccess) return device_error(err, e, "hipMemset");
    return NH_OK;
}

nh_status nh_stream_create(nh_context* ctx, nh_stream* out, nh_error* err) {
    clear_error(err);
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) return device_error(err, e, "hipStreamCreate");
    *out = (nh_stream)s;
    return NH_OK;
}

nh_status nh_stream_destroy(nh_context* ctx, nh_stream stream, nh_error* err) {
    clear_error(err);
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    hipError_t e = hipStreamDestroy((hipStream_t)stream);
    if (e != hipSuccess) return device_error(err, e, "hipStreamDestroy");
    return NH_OK;
}

nh_status nh_stream_synchronize(nh_context* ctx, nh_stream stream, nh_error* err) {
    clear_error(err);
    nh_status st = bind_device(ctx, err);
    if (st) return st;
    hipError_t e = hipStreamSynchronize((hipStream_t)stream);
    if (e != hipSuccess) return device_error(err, e, "hipStreamSynchronize");
    return NH_OK;
}

// Registry in the spirit of supported_*_kernels(): every device kernel is
// tagged 1 (gfx950), every host twin 0.
static const struct {
    const char* name;
    int backend;
} kRegistry[] = {
    {"quantize_rows_i8", 1},     {"dequantize_i8", 1},          {"int4_affine_dequantize", 1},
    {"gemv_w8a8", 1},            {"linear_decode_w8a8", 1},     {"gemv_w8a32", 1},
    {"gemm_w8a8", 1},            {"moe_sigmoid_topk", 1},       {"moe_permute", 1},
    {"moe_grouped_gemm_w8a8", 1}, {"moe_combine", 1},           {"gemm_host", 0},
    {"int4_affine_host", 0},     {"quantize_rows_i8_host", 0},  {"gemm_w8a8_host", 0},
    {"gemv_w8a32_host", 0},      {"moe_sigmoid_topk_host", 0},  {"moe_softmax_topk_host", 0},
    {"moe_permute_host", 0},     {"moe_grouped_gemm_w8a8_host", 0}, {"moe_combine_host", 0},
    {"tile_weights_i8", 1},      {"tile_weights_i8_host", 0},  {"gemm_f32", 1},
    {"mlp_w8a8", 1},             {"gemm_w8a8_tiled_a", 1},
};

int nh_kernel_count(void) { return (int)(sizeof(kRegistry) / sizeof(kRegistry[0])); }

const char* nh_kernel_name(int i, int* backend) {
    if (i < 0 || i >= nh_kernel_count()) return nullptr;
    if (backend) *backend = kRegistry[i].backend;
    return kRegistry[i].name;
}

}  // extern "C"
