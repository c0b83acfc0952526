"""ctypes bindings for the CPU oracle (oracle/_build/libnh_oracle.so).

Test infrastructure: the oracle is the checker the HIP path is compared with.
Arrays are numpy; every wrapper returns (status, outputs...) with status codes
mirroring the reference error enums (see oracle/nh_oracle.h).
"""
import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "_build", "libnh_oracle.so")

OK, INVALID_SHAPE, LENGTH_MISMATCH, INVALID_PARAMS, NON_FINITE_INPUT, OUT_OF_RANGE, INVALID_ROW_COUNT = range(7)


class OrError(C.Structure):
    _fields_ = [
        ("argument", C.c_char_p),
        ("expected", C.c_uint64),
        ("actual", C.c_uint64),
        ("index", C.c_uint64),
        ("value", C.c_float),
        ("byte", C.c_uint32),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            subprocess.run(["make", "-C", ORACLE_DIR], check=True, capture_output=True)
        _lib = C.CDLL(ORACLE_SO)
        _declare(_lib)
    return _lib


P = C.c_void_p
SZ = C.c_size_t


def _declare(L):
    L.or_fill_normal_f32.argtypes = [C.c_uint64, C.c_float, C.c_float, P, SZ]
    L.or_f32_to_bf16.restype = C.c_uint16
    L.or_f32_to_bf16.argtypes = [C.c_float]
    L.or_bf16_to_f32.restype = C.c_float
    L.or_bf16_to_f32.argtypes = [C.c_uint16]
    L.or_f32_to_bf16_array.argtypes = [P, P, SZ]
    L.or_packed_int4_len.restype = SZ
    L.or_packed_int4_len.argtypes = [SZ]
    L.or_pack_int4.argtypes = [P, SZ, P, SZ, C.POINTER(OrError)]
    L.or_unpack_int4.argtypes = [P, SZ, SZ, P, SZ, C.POINTER(OrError)]
    L.or_quantize_int4.argtypes = [P, SZ, C.c_float, C.c_uint32, P, SZ, C.POINTER(OrError)]
    L.or_dequantize_int4.argtypes = [P, SZ, SZ, C.c_float, C.c_uint32, P, SZ, C.POINTER(OrError)]
    L.or_quantize_rows_i8_f32.argtypes = [P, SZ, SZ, P, P, C.POINTER(OrError)]
    L.or_quantize_rows_i8_bf16.argtypes = [P, SZ, SZ, P, P, C.POINTER(OrError)]
    L.or_dequantize_i8.argtypes = [P, P, SZ, SZ, P]
    L.or_gemm_f32.argtypes = [P, SZ, P, SZ, SZ, SZ, SZ, P, SZ, C.POINTER(OrError)]
    L.or_gemm_f32_col_range.argtypes = [P, P, SZ, SZ, SZ, SZ, SZ, P]
    L.or_gemm_f32_col_range.restype = None
    L.or_gemm_i8_i32.argtypes = [P, P, SZ, SZ, SZ, P]
    L.or_epilogue_w8a8.argtypes = [P, P, P, P, SZ, SZ, C.c_int, C.c_int, P]
    L.or_linear_w8a8.argtypes = [P, P, P, P, P, SZ, SZ, SZ, C.c_int, P]
    L.or_gemv_w8a32.argtypes = [P, P, P, SZ, SZ, SZ, P]
    L.or_sigmoid.restype = C.c_float
    L.or_sigmoid.argtypes = [C.c_float]
    L.or_relu2.restype = C.c_float
    L.or_relu2.argtypes = [C.c_float]
    L.or_route_sigmoid_topk.argtypes = [P, SZ, SZ, SZ, SZ, C.c_int, C.c_float, P, SZ, P, SZ, C.POINTER(OrError)]
    L.or_route_softmax_topk.argtypes = [P, SZ, SZ, SZ, SZ, P, SZ, P, SZ, C.POINTER(OrError)]
    L.or_moe_permute.argtypes = [P, SZ, SZ, SZ, P, P, P]
    L.or_moe_grouped_w8a8.argtypes = [P, P, C.c_int, SZ, P, P, SZ, P, P, P, SZ, SZ, C.c_int, P]
    L.or_moe_combine.argtypes = [P, P, P, SZ, SZ, SZ, C.c_int, P]
    L.or_moe_forward_w8a8.argtypes = [P, P, SZ, SZ, SZ, SZ, SZ, C.c_int, C.c_float, P, P, P, P, P, P, P, P, P, P]
    L.or_linear_project.argtypes = [P, SZ, SZ, P, SZ, SZ, P, P, SZ, C.POINTER(OrError)]
    L.or_mlp_forward.argtypes = [P, SZ, SZ, SZ, P, P, P, P, P]
    L.or_moe_forward_dense.argtypes = [P, SZ, SZ, SZ, SZ, P, P, SZ, P, P, P, P, SZ, P, P, P, P, P]
    L.or_moe_combine_shared.argtypes = [P, P, P, P, SZ, SZ, SZ, C.c_int, P]
    L.or_linear_w4a8.argtypes = [P, SZ, SZ, P, SZ, C.c_float, C.c_uint32, P, C.c_int, P]
    L.or_mlp_w8a8.argtypes = [P, SZ, SZ, SZ, P, P, P, P, P, P, P]
    L.or_moe_forward_shared_w8a8.argtypes = [P, P, SZ, SZ, SZ, SZ, SZ, C.c_int, C.c_float, P, P, P, P, SZ, P, P, P,
                                             P, P, P, P, P, P, P, P]


def ptr(a):
    """Data pointer of a numpy array (None passes NULL)."""
    if a is None:
        return None
    return a.ctypes.data


def normal_f32(seed, n, mean=0.0, std=1.0):
    out = np.empty(n, dtype=np.float32)
    lib().or_fill_normal_f32(seed, mean, std, ptr(out), n)
    return out


def to_bf16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().or_f32_to_bf16_array(ptr(x), ptr(out), x.size)
    return out


def bf16_to_f32(b):
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def quantize_rows_f32(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    q = np.zeros((rows, cols), dtype=np.int8)
    s = np.zeros(rows, dtype=np.float32)
    err = OrError()
    st = lib().or_quantize_rows_i8_f32(ptr(x), rows, cols, ptr(q), ptr(s), C.byref(err))
    return st, q, s, err


def quantize_rows_bf16(xb):
    xb = np.ascontiguousarray(xb, dtype=np.uint16)
    rows, cols = xb.shape
    q = np.zeros((rows, cols), dtype=np.int8)
    s = np.zeros(rows, dtype=np.float32)
    err = OrError()
    st = lib().or_quantize_rows_i8_bf16(ptr(xb), rows, cols, ptr(q), ptr(s), C.byref(err))
    return st, q, s, err


def dequantize_i8(q, s):
    q = np.ascontiguousarray(q, dtype=np.int8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    rows, cols = q.shape
    out = np.empty((rows, cols), dtype=np.float32)
    lib().or_dequantize_i8(ptr(q), ptr(s), rows, cols, ptr(out))
    return out


def gemm_f32(lhs, rhs, m, k, n, out_len=None):
    lhs = np.ascontiguousarray(lhs, dtype=np.float32).ravel()
    rhs = np.ascontiguousarray(rhs, dtype=np.float32).ravel()
    out_len = m * n if out_len is None else out_len
    out = np.zeros(max(out_len, 1), dtype=np.float32)
    err = OrError()
    st = lib().or_gemm_f32(ptr(lhs), lhs.size, ptr(rhs), rhs.size, m, k, n, ptr(out), out_len, C.byref(err))
    return st, out[:out_len], err


def gemm_f32_col_range(lhs, rhs, m, k, n, col0, col1, out):
    """or_gemm_f32's loop over output columns [col0, col1) of out ([m][n], f32), in place."""
    lib().or_gemm_f32_col_range(ptr(lhs), ptr(rhs), m, k, n, col0, col1, ptr(out))


def gemm_i8_i32(xq, wq):
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    m, k = xq.shape
    n = wq.shape[0]
    acc = np.empty((m, n), dtype=np.int32)
    lib().or_gemm_i8_i32(ptr(xq), ptr(wq), m, n, k, ptr(acc))
    return acc


def epilogue(acc, sx, sw, bias=None, relu2=False, out_bf16=False):
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    m, n = acc.shape
    out = np.empty((m, n), dtype=np.uint16 if out_bf16 else np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    sx = np.ascontiguousarray(sx, dtype=np.float32)
    sw = np.ascontiguousarray(sw, dtype=np.float32)
    lib().or_epilogue_w8a8(ptr(acc), ptr(sx), ptr(sw), ptr(b), m, n, int(relu2), int(out_bf16), ptr(out))
    return out


def linear_w8a8(xq, sx, wq, sw, bias=None, out_bf16=False):
    return epilogue(gemm_i8_i32(xq, wq), sx, sw, bias=bias, out_bf16=out_bf16)


def gemv_w8a32(x, wq, sw):
    x = np.ascontiguousarray(x, dtype=np.float32)
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    m, k = x.shape
    n = wq.shape[0]
    sw = np.ascontiguousarray(sw, dtype=np.float32)
    y = np.empty((m, n), dtype=np.float32)
    lib().or_gemv_w8a32(ptr(x), ptr(wq), ptr(sw), m, n, k, ptr(y))
    return y


def route_sigmoid(scores, tokens, experts, top_k, renormalize=False, scaling=1.0,
                  indices_len=None, weights_len=None, scores_len=None):
    scores = np.ascontiguousarray(scores, dtype=np.float32).ravel()
    scores_len = scores.size if scores_len is None else scores_len
    il = tokens * top_k if indices_len is None else indices_len
    wl = tokens * top_k if weights_len is None else weights_len
    idx = np.zeros(max(il, 1), dtype=np.int32)
    w = np.zeros(max(wl, 1), dtype=np.float32)
    err = OrError()
    st = lib().or_route_sigmoid_topk(ptr(scores), scores_len, tokens, experts, top_k, int(renormalize),
                                     scaling, ptr(idx), il, ptr(w), wl, C.byref(err))
    return st, idx[:il], w[:wl], err


def route_softmax(scores, tokens, experts, top_k):
    scores = np.ascontiguousarray(scores, dtype=np.float32).ravel()
    il = tokens * top_k
    idx = np.zeros(max(il, 1), dtype=np.int32)
    w = np.zeros(max(il, 1), dtype=np.float32)
    err = OrError()
    st = lib().or_route_softmax_topk(ptr(scores), scores.size, tokens, experts, top_k, ptr(idx), il,
                                     ptr(w), il, C.byref(err))
    return st, idx[:il], w[:il], err


def moe_permute(indices, tokens, top_k, experts):
    indices = np.ascontiguousarray(indices, dtype=np.int32)  # kept alive for the call
    routes = tokens * top_k
    offsets = np.zeros(experts + 1, dtype=np.int32)
    perm = np.zeros(max(routes, 1), dtype=np.int32)
    pos = np.zeros(max(routes, 1), dtype=np.int32)
    lib().or_moe_permute(ptr(indices), tokens, top_k, experts, ptr(offsets), ptr(perm), ptr(pos))
    return offsets, perm[:routes], pos[:routes]


def moe_grouped(aq, sa, gather_tokens, top_k, offsets, perm, w, sw, relu2, bias=None):
    experts, n, k = w.shape
    routes = int(offsets[-1])
    out = np.zeros((max(routes, 1), n), dtype=np.float32)
    aq = np.ascontiguousarray(aq, dtype=np.int8)
    sa = np.ascontiguousarray(sa, dtype=np.float32)
    offsets = np.ascontiguousarray(offsets, dtype=np.int32)
    perm = np.ascontiguousarray(perm, dtype=np.int32)
    w = np.ascontiguousarray(w, dtype=np.int8)
    sw = np.ascontiguousarray(sw, dtype=np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().or_moe_grouped_w8a8(ptr(aq), ptr(sa), int(gather_tokens), top_k, ptr(offsets), ptr(perm), experts,
                              ptr(w), ptr(sw), ptr(bias), n, k, int(relu2), ptr(out))
    return out[:routes]


def moe_combine(slot_out, pos, weights, tokens, top_k, hidden, out_bf16=False):
    out = np.zeros((tokens, hidden), dtype=np.uint16 if out_bf16 else np.float32)
    slot_out = np.ascontiguousarray(slot_out, dtype=np.float32)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    lib().or_moe_combine(ptr(slot_out), ptr(pos), ptr(weights), tokens, top_k, hidden, int(out_bf16), ptr(out))
    return out


def moe_forward_w8a8(x_bf16, logits, w_up, s_up, w_down, s_down, top_k, renormalize=True, scaling=1.0):
    tokens, hidden = x_bf16.shape
    experts, inter, _ = w_up.shape
    routes = tokens * top_k
    out = np.zeros((tokens, hidden), dtype=np.uint16)
    idx = np.zeros(routes, dtype=np.int32)
    w = np.zeros(routes, dtype=np.float32)
    offsets = np.zeros(experts + 1, dtype=np.int32)
    perm = np.zeros(routes, dtype=np.int32)
    pos = np.zeros(routes, dtype=np.int32)
    x_bf16 = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    w_up, s_up = np.ascontiguousarray(w_up, dtype=np.int8), np.ascontiguousarray(s_up, dtype=np.float32)
    w_down, s_down = np.ascontiguousarray(w_down, dtype=np.int8), np.ascontiguousarray(s_down, dtype=np.float32)
    st = lib().or_moe_forward_w8a8(ptr(x_bf16), ptr(logits),
                                   tokens, hidden, inter, experts, top_k, int(renormalize), scaling,
                                   ptr(w_up), ptr(s_up), ptr(w_down), ptr(s_down), ptr(out), ptr(idx), ptr(w),
                                   ptr(offsets), ptr(perm), ptr(pos))
    return st, out, idx, w, offsets, perm, pos


def moe_combine_shared(slot_out, pos, weights, shared, tokens, top_k, hidden, out_bf16=False):
    out = np.zeros((tokens, hidden), dtype=np.uint16 if out_bf16 else np.float32)
    slot_out = np.ascontiguousarray(slot_out, dtype=np.float32)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    shared = None if shared is None else np.ascontiguousarray(shared, dtype=np.float32)
    lib().or_moe_combine_shared(ptr(slot_out), ptr(pos), ptr(weights), ptr(shared), tokens, top_k, hidden,
                                int(out_bf16), ptr(out))
    return out


def _f32_or_none(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def mlp_w8a8(x_bf16, w_up, s_up, w_down, s_down, b_up=None, b_down=None):
    """int8 MLP of bf16 rows: Q2 -> up (+ b_up, ReLU^2, f32) -> Q2 -> down (+ b_down, f32)."""
    x_bf16 = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    rows, hidden = x_bf16.shape
    inter = w_up.shape[0]
    out = np.zeros((rows, hidden), dtype=np.float32)
    b_up, b_down = _f32_or_none(b_up), _f32_or_none(b_down)
    st = lib().or_mlp_w8a8(ptr(x_bf16), rows, hidden, inter, ptr(np.ascontiguousarray(w_up, dtype=np.int8)),
                           ptr(np.ascontiguousarray(s_up, dtype=np.float32)), ptr(b_up),
                           ptr(np.ascontiguousarray(w_down, dtype=np.int8)),
                           ptr(np.ascontiguousarray(s_down, dtype=np.float32)), ptr(b_down), ptr(out))
    return st, out


def moe_forward_shared_w8a8(x_bf16, logits, w_up, s_up, w_down, s_down, top_k, sh_up, sh_su, sh_down, sh_sd,
                            renormalize=True, scaling=1.0, biases=None):
    """The int8 MoE layer with a shared expert (sh_up None: without one);
    biases = (up [E][inter], down [E][hidden], shared up, shared down), each
    None or an array."""
    tokens, hidden = x_bf16.shape
    experts, inter, _ = w_up.shape
    routes = tokens * top_k
    out = np.zeros((tokens, hidden), dtype=np.uint16)
    idx = np.zeros(routes, dtype=np.int32)
    w = np.zeros(routes, dtype=np.float32)
    offsets = np.zeros(experts + 1, dtype=np.int32)
    perm = np.zeros(routes, dtype=np.int32)
    pos = np.zeros(routes, dtype=np.int32)
    keep = [None if a is None else np.ascontiguousarray(a, dtype=d)
            for a, d in ((x_bf16, np.uint16), (logits, np.float32), (w_up, np.int8), (s_up, np.float32),
                         (w_down, np.int8), (s_down, np.float32), (sh_up, np.int8), (sh_su, np.float32),
                         (sh_down, np.int8), (sh_sd, np.float32))]
    bkeep = [_f32_or_none(b) for b in (biases or (None,) * 4)]
    bptrs = (C.c_void_p * 4)(*[ptr(b) for b in bkeep]) if biases is not None else None
    st = lib().or_moe_forward_shared_w8a8(ptr(keep[0]), ptr(keep[1]), tokens, hidden, inter, experts, top_k,
                                          int(renormalize), scaling, ptr(keep[2]), ptr(keep[3]), ptr(keep[4]),
                                          ptr(keep[5]), 0 if sh_up is None else sh_up.shape[0], ptr(keep[6]),
                                          ptr(keep[7]), ptr(keep[8]), ptr(keep[9]), bptrs, ptr(out), ptr(idx), ptr(w),
                                          ptr(offsets), ptr(perm), ptr(pos))
    return st, out, idx, w, offsets, perm, pos


def quantize_int4(values, scale, zp):
    values = np.ascontiguousarray(values, dtype=np.float32)
    packed = np.zeros((values.size + 1) // 2, dtype=np.uint8)
    err = OrError()
    st = lib().or_quantize_int4(ptr(values), values.size, scale, zp, ptr(packed), packed.size, C.byref(err))
    return st, packed, err


def dequantize_int4(packed, count, scale, zp):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.zeros(count, dtype=np.float32)
    err = OrError()
    st = lib().or_dequantize_int4(ptr(packed), packed.size, count, scale, zp, ptr(out), count, C.byref(err))
    return st, out, err


def linear_w4a8(x_bf16, packed, n, scale, zp, bias=None, out_bf16=False):
    """W4A8 linear on the reference's packed [K][N] INT4 codes."""
    x_bf16 = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    m, k = x_bf16.shape
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    out = np.zeros((m, n), dtype=np.uint16 if out_bf16 else np.float32)
    st = lib().or_linear_w4a8(ptr(x_bf16), m, k, ptr(packed), n, scale, zp, ptr(bias), int(out_bf16), ptr(out))
    return st, out


def sigmoid(x):
    return lib().or_sigmoid(float(x))
