"""ctypes binding of libnemotron_hip.so (the C ABI in include/nemotron_hip.h).

This is the Python-side counterpart of the Rust FFI crate a nemotron-rs
maintainer would add: one declaration per exported symbol, plus a small
device-buffer helper so tests and the benchmark can stage numpy arrays.
Nothing here computes: every op is a call into the library, and loading fails
loudly if the library has not been built.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libnemotron_hip.so")
CODE_OBJECT_PATH = os.path.join(HERE, "lib", "nh_kernels_gfx950.hsaco")

OK = 0
INVALID_SHAPE = 1
LENGTH_MISMATCH = 2
INVALID_PARAMS = 3
NON_FINITE_INPUT = 4
OUT_OF_RANGE = 5
INVALID_ROW_COUNT = 6
UNSUPPORTED = 7
DEVICE_ERROR = 8
IO_ERROR = 9
INVALID_HEADER = 10
TENSOR_NOT_FOUND = 11
STATUS_NAMES = {0: "Ok", 1: "InvalidShape", 2: "LengthMismatch", 3: "InvalidParams", 4: "NonFiniteInput",
                5: "Int4OutOfRange", 6: "InvalidRowCount", 7: "Unsupported", 8: "DeviceError", 9: "Io",
                10: "InvalidHeader", 11: "TensorNotFound"}


class TensorInfo(C.Structure):
    _fields_ = [("dtype", C.c_char * 16), ("ndim", C.c_uint32), ("shape", C.c_uint64 * 8),
                ("data_begin", C.c_uint64), ("data_bytes", C.c_uint64)]

F32 = 0
BF16 = 1


class MoeBiases(C.Structure):
    """nh_moe_biases: optional expert biases (device or host pointers, 0 = none)."""
    _fields_ = [("up", C.c_void_p), ("down", C.c_void_p), ("shared_up", C.c_void_p), ("shared_down", C.c_void_p)]


class NhError(C.Structure):
    _fields_ = [
        ("argument", C.c_char_p),
        ("expected", C.c_uint64),
        ("actual", C.c_uint64),
        ("index", C.c_uint64),
        ("value", C.c_float),
        ("byte", C.c_uint32),
        ("message", C.c_char * 256),
    ]


class NhStatusError(RuntimeError):
    def __init__(self, status, err):
        self.status = status
        self.argument = err.argument.decode() if err.argument else None
        self.expected = err.expected
        self.actual = err.actual
        self.index = err.index
        self.value = err.value
        self.byte = err.byte
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {err.message.decode(errors='replace')}")


P = C.c_void_p
SZ = C.c_size_t
ST = C.c_int
E = C.POINTER(NhError)
MB = C.POINTER(MoeBiases)

_SIGNATURES = {
    "nh_device_count": (C.c_int, []),
    "nh_context_create": (ST, [C.c_int, C.c_char_p, C.POINTER(P), E]),
    "nh_context_destroy": (None, [P]),
    "nh_context_device": (C.c_int, [P]),
    "nh_malloc": (ST, [P, SZ, C.POINTER(P), E]),
    "nh_free": (ST, [P, P, E]),
    "nh_memcpy_htod": (ST, [P, P, P, SZ, E]),
    "nh_memcpy_dtoh": (ST, [P, P, P, SZ, E]),
    "nh_memset_d8": (ST, [P, P, C.c_int, SZ, E]),
    "nh_stream_create": (ST, [P, C.POINTER(P), E]),
    "nh_stream_destroy": (ST, [P, P, E]),
    "nh_stream_synchronize": (ST, [P, P, E]),
    "nh_kernel_count": (C.c_int, []),
    "nh_kernel_name": (C.c_char_p, [C.c_int, C.POINTER(C.c_int)]),
    "nh_packed_int4_len": (SZ, [SZ]),
    "nh_pack_int4_host": (ST, [P, SZ, P, SZ, E]),
    "nh_unpack_int4_host": (ST, [P, SZ, SZ, P, SZ, E]),
    "nh_quantize_int4_host": (ST, [P, SZ, C.c_float, C.c_uint32, P, SZ, E]),
    "nh_dequantize_int4_host": (ST, [P, SZ, SZ, C.c_float, C.c_uint32, P, SZ, E]),
    "nh_dequantize_int4": (ST, [P, P, SZ, SZ, C.c_float, C.c_uint32, P, SZ, P, E]),
    "nh_quantize_rows_i8": (ST, [P, P, C.c_int, SZ, SZ, P, P, P, P, E]),
    "nh_quantize_rows_i8_host": (ST, [P, C.c_int, SZ, SZ, P, P, E]),
    "nh_dequantize_i8": (ST, [P, P, P, SZ, SZ, P, P, E]),
    "nh_dequantize_i8_host": (ST, [P, P, SZ, SZ, P, E]),
    "nh_tiled_weights_bytes": (SZ, [SZ, SZ]),
    "nh_tile_weights_i8": (ST, [P, P, SZ, SZ, P, SZ, P, E]),
    "nh_tile_weights_i8_host": (ST, [P, SZ, SZ, P, SZ, E]),
    "nh_gemm_f32_host": (ST, [P, SZ, P, SZ, SZ, SZ, SZ, P, SZ, E]),
    "nh_supports_gemm_f32": (C.c_int, [SZ, SZ, SZ]),
    "nh_gemm_f32": (ST, [P, P, SZ, P, SZ, SZ, SZ, SZ, P, SZ, P, E]),
    "nh_supports_gemm_w8a8": (C.c_int, [SZ, SZ, SZ]),
    "nh_gemm_w8a8": (ST, [P, P, P, P, P, P, SZ, SZ, SZ, P, C.c_int, P, E]),
    "nh_gemm_w8a8_ta": (ST, [P, P, P, P, P, P, SZ, SZ, SZ, P, C.c_int, P, E]),
    "nh_gemm_w8a8_host": (ST, [P, P, P, P, P, SZ, SZ, SZ, P, C.c_int, E]),
    "nh_linear_w8a8_workspace_size": (SZ, [SZ, SZ]),
    "nh_take_nonfinite": (ST, [P, P, P, E]),
    "nh_linear_w8a8": (ST, [P, P, C.c_int, P, P, P, SZ, SZ, SZ, P, C.c_int, P, SZ, P, P, P, P, E]),
    "nh_supports_linear_w8a8": (C.c_int, [SZ, SZ, SZ]),
    "nh_linear_w8a8_host": (ST, [P, C.c_int, P, P, P, SZ, SZ, SZ, P, C.c_int, P, P, E]),
    "nh_linear_w8a8_noalloc": (ST, [P, P, C.c_int, P, P, P, SZ, SZ, SZ, P, C.c_int, P, P, P, P, E]),
    "nh_mlp_w8a8_workspace_size": (SZ, [SZ, SZ, SZ]),
    "nh_mlp_w8a8": (ST, [P, P, C.c_int, P, P, P, P, P, P, SZ, SZ, SZ, P, C.c_int, P, SZ, P, P, E]),
    "nh_supports_mlp_w8a8": (C.c_int, [SZ, SZ, SZ]),
    "nh_mlp_w8a8_host": (ST, [P, C.c_int, P, P, P, P, P, P, SZ, SZ, SZ, P, C.c_int, E]),
    "nh_gemv_w8a32": (ST, [P, P, P, P, SZ, SZ, SZ, P, P, E]),
    "nh_gemv_w8a32_host": (ST, [P, P, P, SZ, SZ, SZ, P, E]),
    "nh_sigmoid_f32_host": (C.c_float, [C.c_float]),
    "nh_moe_route_sigmoid_topk": (ST, [P, P, SZ, SZ, SZ, C.c_int, C.c_float, P, P, P, E]),
    "nh_moe_route_sigmoid_topk_host": (ST, [P, SZ, SZ, SZ, SZ, C.c_int, C.c_float, P, SZ, P, SZ, E]),
    "nh_moe_route_softmax_topk_host": (ST, [P, SZ, SZ, SZ, SZ, P, SZ, P, SZ, E]),
    "nh_moe_permute": (ST, [P, P, SZ, SZ, SZ, P, P, P, P, E]),
    "nh_moe_permute_host": (ST, [P, SZ, SZ, SZ, P, P, P, E]),
    "nh_moe_grouped_gemm_w8a8": (ST, [P, P, P, C.c_int, SZ, P, P, SZ, SZ, SZ, P, P, SZ, SZ, C.c_int, P, P, E]),
    "nh_moe_grouped_gemm_w8a8_host": (ST, [P, P, C.c_int, SZ, P, P, SZ, SZ, SZ, P, P, SZ, SZ, C.c_int, P, E]),
    "nh_moe_combine": (ST, [P, P, P, P, SZ, SZ, SZ, P, C.c_int, P, E]),
    "nh_moe_combine_host": (ST, [P, P, P, SZ, SZ, SZ, P, C.c_int, E]),
    "nh_moe_forward_w8a8_workspace_size": (SZ, [SZ, SZ, SZ, SZ, SZ]),
    "nh_moe_workspace_layout": (None, [SZ, SZ, SZ, SZ, SZ, C.POINTER(SZ)]),
    "nh_moe_forward_w8a8": (ST, [P, P, C.c_int, P, SZ, SZ, SZ, SZ, SZ, C.c_int, C.c_float, P, P, P, P, MB, P,
                                 C.c_int, P, SZ, P, P, E]),
    "nh_moe_combine_shared": (ST, [P, P, P, P, P, SZ, SZ, SZ, P, C.c_int, P, E]),
    "nh_moe_combine_shared_host": (ST, [P, P, P, P, SZ, SZ, SZ, P, C.c_int, E]),
    "nh_moe_forward_shared_w8a8_workspace_size": (SZ, [SZ, SZ, SZ, SZ, SZ, SZ]),
    "nh_moe_forward_shared_w8a8": (ST, [P, P, C.c_int, P, SZ, SZ, SZ, SZ, SZ, C.c_int, C.c_float, P, P, P, P, SZ,
                                        P, P, P, P, MB, P, C.c_int, P, SZ, P, P, E]),
    "nh_moe_layer_w8a8_workspace_size": (SZ, [SZ, SZ, SZ, SZ, SZ, SZ]),
    "nh_moe_layer_w8a8": (ST, [P, P, C.c_int, P, P, SZ, SZ, SZ, SZ, SZ, C.c_int, C.c_float, P, P, P, P, SZ,
                               P, P, P, P, MB, P, C.c_int, P, SZ, P, P, E]),
    "nh_supports_moe_layer_w8a8": (C.c_int, [SZ, SZ, SZ, SZ, SZ, SZ]),
    "nh_moe_layer_w8a8_host": (ST, [P, C.c_int, P, P, SZ, SZ, SZ, SZ, SZ, C.c_int, C.c_float, P, P, P, P, SZ,
                                    P, P, P, P, MB, P, C.c_int, E]),
    "nh_stream_read": (ST, [P, P, SZ, P, P, E]),
    "nh_handoff_status": (ST, [P, P, P, E]),
    "nh_tiled_int4_weights_bytes": (SZ, [SZ, SZ]),
    "nh_tile_weights_int4": (ST, [P, P, SZ, SZ, SZ, C.c_uint32, P, SZ, P, E]),
    "nh_tile_weights_int4_host": (ST, [P, SZ, SZ, SZ, C.c_uint32, P, SZ, E]),
    "nh_supports_linear_w4a8": (C.c_int, [SZ, SZ, SZ]),
    "nh_linear_w4a8_workspace_size": (SZ, [SZ, SZ, SZ]),
    "nh_linear_w4a8": (ST, [P, P, C.c_int, P, C.c_float, C.c_uint32, P, SZ, SZ, SZ, P, C.c_int, P, SZ, P, P, E]),
    "nh_linear_w4a8_host": (ST, [P, C.c_int, P, SZ, C.c_float, C.c_uint32, P, SZ, SZ, SZ, P, C.c_int, E]),
    "nh_safetensors_tensor_info": (ST, [C.c_char_p, C.c_char_p, C.POINTER(TensorInfo), E]),
    "nh_safetensors_read": (ST, [P, C.c_char_p, C.c_char_p, P, SZ, E]),
    "nh_load_linear_i8": (ST, [P, C.c_char_p, C.c_char_p, C.c_char_p, SZ, SZ, P, SZ, P, SZ, P, E]),
    "nh_fill_normal_f32_host": (None, [C.c_uint64, C.c_float, C.c_float, P, SZ]),
}

_lib = None


def lib():
    """Load libnemotron_hip.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() (make -C nemotron-cutile-rs_amd)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    return list(_SIGNATURES)


def check(status, err):
    if status != OK:
        raise NhStatusError(status, err)


def call(name, *args):
    """Call an nh_* entry point whose last argument is nh_error*; raise on failure."""
    err = NhError()
    st = getattr(lib(), name)(*args, C.byref(err))
    check(st, err)


def call_status(name, *args):
    """Like call() but returns (status, error) instead of raising."""
    err = NhError()
    st = getattr(lib(), name)(*args, C.byref(err))
    return st, err


def ptr(a):
    if a is None:
        return None
    if isinstance(a, DeviceBuffer):
        return a.ptr
    return a.ctypes.data


class Context:
    """nh_context on one device (GpuDevice, device.rs:117-153)."""

    def __init__(self, device=0, code_object_path=None):
        self.handle = P()
        path = code_object_path.encode() if code_object_path else None
        call("nh_context_create", device, path, C.byref(self.handle))
        self.device = device

    def close(self):
        if self.handle:
            lib().nh_context_destroy(self.handle)
            self.handle = P()

    def synchronize(self, stream=None):
        call("nh_stream_synchronize", self.handle, stream)

    def empty(self, shape, dtype):
        return DeviceBuffer(self, shape, dtype)

    def upload(self, array):
        array = np.ascontiguousarray(array)
        buf = DeviceBuffer(self, array.shape, array.dtype)
        buf.copy_from(array)
        return buf


class DeviceBuffer:
    """A typed device allocation (the role of GpuTensor, tensor.rs:259-446)."""

    def __init__(self, ctx, shape, dtype):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = P()
        call("nh_malloc", ctx.handle, max(self.nbytes, 1), C.byref(p))
        self.ptr = p.value

    @property
    def size(self):
        return int(np.prod(self.shape, dtype=np.int64))

    def copy_from(self, array):
        array = np.ascontiguousarray(array, dtype=self.dtype)
        assert array.nbytes == self.nbytes, (array.nbytes, self.nbytes)
        call("nh_memcpy_htod", self.ctx.handle, self.ptr, array.ctypes.data, self.nbytes)

    def numpy(self):
        out = np.empty(self.shape, dtype=self.dtype)
        call("nh_memcpy_dtoh", self.ctx.handle, out.ctypes.data, self.ptr, self.nbytes)
        return out

    def fill_bytes(self, value):
        call("nh_memset_d8", self.ctx.handle, self.ptr, value, self.nbytes)

    def offset(self, nbytes):
        return self.ptr + nbytes

    def free(self):
        if self.ptr:
            call("nh_free", self.ctx.handle, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and self.ctx.handle:
                lib().nh_free(self.ctx.handle, self.ptr, None)
        except Exception:
            pass


# --------------------------------------------------------------------------
# HIP events for timing (plumbing for the benchmark; same runtime library).
class HipEvents:
    def __init__(self):
        self.hip = C.CDLL("libamdhip64.so.7")
        self.hip.hipEventCreate.argtypes = [C.POINTER(P)]
        self.hip.hipEventRecord.argtypes = [P, P]
        self.hip.hipEventSynchronize.argtypes = [P]
        self.hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), P, P]
        self.hip.hipEventDestroy.argtypes = [P]

    def create(self):
        e = P()
        assert self.hip.hipEventCreate(C.byref(e)) == 0
        return e

    def record(self, ev, stream=None):
        assert self.hip.hipEventRecord(ev, stream) == 0

    def elapsed_ms(self, start, stop):
        assert self.hip.hipEventSynchronize(stop) == 0
        ms = C.c_float()
        assert self.hip.hipEventElapsedTime(C.byref(ms), start, stop) == 0
        return ms.value

    def destroy(self, ev):
        self.hip.hipEventDestroy(ev)


class HipGraphs:
    """Stream capture into HIP graphs and their replay (plumbing for the
    benchmark: the library's calls are captured as issued, nothing else)."""

    CAPTURE_RELAXED = 2

    def __init__(self):
        self.hip = C.CDLL("libamdhip64.so.7")
        self.hip.hipStreamBeginCapture.argtypes = [P, C.c_int]
        self.hip.hipStreamEndCapture.argtypes = [P, C.POINTER(P)]
        self.hip.hipGraphInstantiate.argtypes = [C.POINTER(P), P, P, C.c_char_p, C.c_size_t]
        self.hip.hipGraphLaunch.argtypes = [P, P]
        self.hip.hipGraphExecDestroy.argtypes = [P]
        self.hip.hipGraphDestroy.argtypes = [P]

    def capture(self, stream, issue):
        """Runs issue() under capture on `stream`; returns (graph, exec)."""
        rc = self.hip.hipStreamBeginCapture(stream, self.CAPTURE_RELAXED)
        if rc != 0:
            raise RuntimeError(f"hipStreamBeginCapture failed ({rc})")
        try:
            issue()
        finally:
            g = P()
            rc = self.hip.hipStreamEndCapture(stream, C.byref(g))
        if rc != 0:
            raise RuntimeError(f"hipStreamEndCapture failed ({rc})")
        ex = P()
        rc = self.hip.hipGraphInstantiate(C.byref(ex), g, None, None, 0)
        if rc != 0:
            self.hip.hipGraphDestroy(g)
            raise RuntimeError(f"hipGraphInstantiate failed ({rc})")
        return g, ex

    def launch(self, ex, stream):
        rc = self.hip.hipGraphLaunch(ex, stream)
        if rc != 0:
            raise RuntimeError(f"hipGraphLaunch failed ({rc})")

    def destroy(self, g, ex):
        self.hip.hipGraphExecDestroy(ex)
        self.hip.hipGraphDestroy(g)


def tile_weights(ctx, wq_dev, n, k, stream=None):
    """Device int8 [n][k] row-major -> a new device buffer in the tiled layout."""
    nbytes = lib().nh_tiled_weights_bytes(n, k)
    out = ctx.empty(nbytes, np.int8)
    call("nh_tile_weights_i8", ctx.handle, wq_dev.ptr, n, k, out.ptr, nbytes, stream)
    return out


def normal_f32(seed, n, mean=0.0, std=1.0):
    """Seeded N(mean, std) f32 samples from the library's generator."""
    out = np.empty(n, dtype=np.float32)
    lib().nh_fill_normal_f32_host(seed, mean, std, out.ctypes.data, n)
    return out


def device_count():
    return lib().nh_device_count()
