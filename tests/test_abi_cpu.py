"""CPU-side checks of libnemotron_hip.so: it loads, exports every symbol the
C header declares, validates arguments before touching a device, and its host
twins (the reference's *_host functions) agree with the oracle bit for bit.
No device compute runs here."""
import ctypes as C
import json
import math
import os
import re
import struct

import numpy as np
import pytest

import nemotron_hip as NH
import oracle_ctypes as O
from tiling import tile_16x64, tile_experts, tiled_bytes

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nemotron_hip.h")
KATS = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_kats.json")))


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = NH.lib()
    declared = header_functions()
    assert len(declared) > 40
    missing = [name for name in declared if not hasattr(L, name)]
    assert missing == []
    # and the Python binding declares exactly the header's functions
    assert sorted(NH.exported_symbols()) == declared


def test_code_object_is_gfx950_only():
    data = open(NH.CODE_OBJECT_PATH, "rb").read()
    assert data[:4] == b"\x7fELF"
    assert b"gfx950" in data
    for other in (b"gfx942", b"gfx90a", b"sm_"):
        assert other not in data


def test_kernel_registry_lists_device_and_host_backends():
    L = NH.lib()
    names = {}
    for i in range(L.nh_kernel_count()):
        b = C.c_int(-1)
        name = L.nh_kernel_name(i, C.byref(b)).decode()
        names[name] = b.value
    assert names["gemm_w8a8"] == 1 and names["moe_sigmoid_topk"] == 1 and names["gemv_w8a8"] == 1
    assert names["gemm_host"] == 0 and names["moe_sigmoid_topk_host"] == 0
    assert L.nh_kernel_name(L.nh_kernel_count(), None) is None


def test_mlp_validates_like_mlp_layer_before_touching_a_device():
    """nh_mlp_w8a8 (MlpLayer::forward_into, mlp.rs:157-211): InvalidShape for a
    zero dimension (mlp.rs:230-236), InvalidRowCount for m == 0 (:163-165),
    then the workspace, all before the (NULL) context is used."""
    mlp = lambda m, hidden, inter, ws, ws_bytes: NH.call_status(
        "nh_mlp_w8a8", None, None, NH.BF16, None, None, None, None, None, None, m, hidden, inter, None, NH.BF16,
        ws, ws_bytes, None, None)
    assert mlp(1, 0, 64, None, 0)[0] == NH.INVALID_SHAPE
    assert mlp(1, 64, 0, None, 0)[0] == NH.INVALID_SHAPE
    assert mlp(0, 64, 64, None, 0)[0] == NH.INVALID_ROW_COUNT
    assert mlp(2, 64, 40, None, 0)[0] == NH.UNSUPPORTED  # inter % 16 != 0: the host path's job
    need = NH.lib().nh_mlp_w8a8_workspace_size(8, 4096, 21504)
    # h (f32 [8][21504]) + the up projection's per-workgroup row maxima (1024
    # workgroups x 8 rows) + the larger projection workspace (activation tiles + scales)
    assert need == 8 * 21504 * 4 + 1024 * 8 * 4 + (8 * 21504 + 255) // 256 * 256 + 256
    st, err = mlp(8, 4096, 21504, None, need - 1)
    assert st == NH.LENGTH_MISMATCH and err.argument == b"workspace" and (err.expected, err.actual) == (need, need - 1)
    assert NH.lib().nh_mlp_w8a8_workspace_size(0, 4096, 21504) == 0


def test_linear_workspace_sizes():
    L = NH.lib()
    # m <= 16: activation tiles (K rounded up to 64) + scales; beyond: row-major codes + scales
    assert L.nh_linear_w8a8_workspace_size(8, 4096) == 8 * 4096 + 256
    assert L.nh_linear_w8a8_workspace_size(3, 4112) == (3 * 4160 + 255) // 256 * 256 + 256
    assert L.nh_linear_w8a8_workspace_size(2048, 4096) == 2048 * 4096 + 8192
    assert L.nh_linear_w8a8_workspace_size(0, 4096) == 0


def test_device_entry_points_validate_before_touching_a_device():
    # NULL context: validation errors must win over the missing device
    st, err = NH.call_status("nh_gemm_w8a8", None, None, None, None, None, None, 0, 4, 16, None, NH.F32, None)
    assert st == NH.INVALID_SHAPE
    st, err = NH.call_status("nh_gemm_w8a8", None, None, None, None, None, None, 2, 4, 12, None, NH.F32, None)
    assert st == NH.UNSUPPORTED  # k % 16 != 0 -> caller uses the host twin
    st, err = NH.call_status("nh_linear_w8a8", None, None, NH.BF16, None, None, None, 0, 4, 16, None, NH.BF16,
                             None, 0, None, None, None, None)
    assert st == NH.INVALID_ROW_COUNT
    st, err = NH.call_status("nh_moe_route_sigmoid_topk", None, None, 1, 2, 3, 0, 1.0, None, None, None)
    assert st == NH.INVALID_SHAPE
    st, err = NH.call_status("nh_dequantize_int4", None, None, 1, 2, 0.0, 8, None, 2, None)
    assert st == NH.INVALID_PARAMS
    st, err = NH.call_status("nh_dequantize_int4", None, None, 1, 2, 1.0, 0, None, 1, None)
    assert st == NH.LENGTH_MISMATCH and err.argument == b"output" and (err.expected, err.actual) == (2, 1)
    assert NH.lib().nh_supports_gemm_w8a8(2048, 4096, 4096) == 1
    assert NH.lib().nh_supports_gemm_w8a8(2048, 4096, 4095) == 0
    assert NH.lib().nh_supports_gemm_w8a8(0, 4096, 4096) == 0
    # int32 accumulator exactness bound: 131072 * 127^2 < 2^31
    assert NH.lib().nh_supports_gemm_w8a8(1, 16, 131072) == 1
    assert NH.lib().nh_supports_gemm_w8a8(1, 16, 131088) == 0
    # 32-bit buffer offsets of the activation panel: m * k < 2^31
    assert NH.lib().nh_supports_gemm_w8a8(16384, 16, 131072) == 0
    assert NH.lib().nh_supports_gemm_w8a8(16383, 16, 131072) == 1


def test_generator_matches_oracle_bit_for_bit():
    for seed, mean, std, n in [(0, 0.0, 0.02, 10001), (1, 0.0, 1.0, 4096), (102, 0.5, 3.0, 7)]:
        assert np.array_equal(NH.normal_f32(seed, n, mean, std), O.normal_f32(seed, n, mean, std))


# ---- host twins vs oracle ---------------------------------------------------
@pytest.mark.parametrize("kat", [k for k in KATS["int4"] if k["op"] in ("quantize_dequantize", "quantize_into")],
                         ids=lambda k: k["src"].split("/")[-1])
def test_int4_host_twin_reference_kats(kat):
    vals = np.array(kat["values"], dtype=np.float32)
    packed = np.zeros(len(kat["packed"]), dtype=np.uint8)
    NH.call("nh_quantize_int4_host", vals.ctypes.data, vals.size, kat["scale"], kat["zero_point"],
            packed.ctypes.data, packed.size)
    assert packed.tolist() == kat["packed"]
    out = np.zeros(vals.size, dtype=np.float32)
    NH.call("nh_dequantize_int4_host", packed.ctypes.data, packed.size, vals.size, kat["scale"], kat["zero_point"],
            out.ctypes.data, out.size)
    if "dequantized" in kat:
        assert np.all(np.abs(out - np.array(kat["dequantized"])) <= kat["tol"])


def test_int4_host_twin_errors_match_reference():
    nan = np.array([np.nan], dtype=np.float32)
    packed = np.zeros(1, dtype=np.uint8)
    st, err = NH.call_status("nh_quantize_int4_host", nan.ctypes.data, 1, 1.0, 8, packed.ctypes.data, 1)
    assert st == NH.NON_FINITE_INPUT and err.index == 0 and math.isnan(err.value)
    st, err = NH.call_status("nh_pack_int4_host", np.array([16], dtype=np.uint8).ctypes.data, 1, packed.ctypes.data, 1)
    assert st == NH.OUT_OF_RANGE and err.byte == 16
    two = np.array([0.0, 1.0], dtype=np.float32)
    st, err = NH.call_status("nh_quantize_int4_host", two.ctypes.data, 2, 1.0, 8, packed.ctypes.data, 0)
    assert st == NH.LENGTH_MISMATCH and (err.argument, err.expected, err.actual) == (b"packed", 1, 0)


def test_quantize_rows_host_twin_matches_oracle():
    x = O.normal_f32(4, 37 * 129).reshape(37, 129)
    _, q_ref, s_ref, _ = O.quantize_rows_f32(x)
    q = np.zeros_like(q_ref)
    s = np.zeros_like(s_ref)
    NH.call("nh_quantize_rows_i8_host", x.ctypes.data, NH.F32, 37, 129, q.ctypes.data, s.ctypes.data)
    assert np.array_equal(q, q_ref) and np.array_equal(s, s_ref)
    xb = O.to_bf16(x)
    _, qb_ref, sb_ref, _ = O.quantize_rows_bf16(xb)
    NH.call("nh_quantize_rows_i8_host", xb.ctypes.data, NH.BF16, 37, 129, q.ctypes.data, s.ctypes.data)
    assert np.array_equal(q, qb_ref) and np.array_equal(s, sb_ref)
    x[3, 5] = np.inf
    st, err = NH.call_status("nh_quantize_rows_i8_host", x.ctypes.data, NH.F32, 37, 129, q.ctypes.data, s.ctypes.data)
    assert st == NH.NON_FINITE_INPUT and err.index == 3 * 129 + 5


def _bf16_rows_every_value(amax_bits_list):
    """One row per row maximum: every finite bf16 value v with |v| <= amax, both signs, and amax itself."""
    pos = np.arange(0, 0x7f80, dtype=np.uint32)
    rows = []
    for ab in amax_bits_list:
        p = pos[pos <= ab].astype(np.uint16)
        rows.append(np.concatenate([p, p | 0x8000, [ab]]).astype(np.uint16))
    width = max(r.size for r in rows)
    # pad with zeros (they quantize to 0 and do not change the row maximum)
    return np.stack([np.concatenate([r, np.zeros(width - r.size, np.uint16)]) for r in rows])


@pytest.mark.slow
def test_quantize_rows_host_twin_every_bf16_value():
    """The division-free quantizer (quantize_i8_fast: multiply by the
    reciprocal, exact tie decision next to half-integers, power-of-two scales
    rounded exactly; the fused decode kernels run the same rule) against the
    oracle's division, on every bf16 value below each of 96 row maxima.  The
    maxima include 127 * 2^e (power-of-two scales: hundreds of exact ties per
    row) and random ones (the value amax / 2 is an exact tie of every row)."""
    rng = np.random.default_rng(21)
    special = [127.0 * 2.0 ** e for e in (-20, -5, 0, 3)] + [3.96875, 4.125, 1.0, 0.1, 250.0, 1e-30]
    specials = O.to_bf16(np.array(special, dtype=np.float32)).ravel()
    rand = rng.integers(0x3000, 0x4800, size=86).astype(np.uint16)
    xb = _bf16_rows_every_value([int(b) for b in np.concatenate([specials, rand])])
    rows, cols = xb.shape
    _, q_ref, s_ref, _ = O.quantize_rows_bf16(xb)
    q = np.zeros_like(q_ref)
    s = np.zeros_like(s_ref)
    NH.call("nh_quantize_rows_i8_host", xb.ctypes.data, NH.BF16, rows, cols, q.ctypes.data, s.ctypes.data)
    assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q, q_ref)
    # the sweep does reach the tie branches: exact half-integer quotients exist
    t = O.bf16_to_f32(xb).astype(np.float64) / s_ref[:, None].astype(np.float64)
    assert int(np.sum(np.abs(t - np.floor(t) - 0.5) < 2.0 ** -15)) > 1000


def test_quantize_rows_host_twin_f32_near_ties():
    """f32 values placed within a few ulps of (j + 0.5) * s for non-power-of-two
    scales, where the reciprocal multiply alone would round the wrong way."""
    rng = np.random.default_rng(22)
    rows = []
    for _ in range(64):
        amax = np.float32(rng.uniform(0.01, 100.0))
        s = np.float32(amax / np.float32(127.0))
        j = rng.integers(0, 127, size=500)
        base = ((j + 0.5) * np.float64(s)).astype(np.float32)
        ulp = rng.integers(-3, 4, size=500).astype(np.int32)
        vals = (base.view(np.int32) + ulp).view(np.float32) * rng.choice([-1, 1], size=500).astype(np.float32)
        vals = np.clip(vals, -amax, amax)
        rows.append(np.concatenate([[amax], vals]).astype(np.float32))
    x = np.stack(rows)
    _, q_ref, s_ref, _ = O.quantize_rows_f32(x)
    q = np.zeros_like(q_ref)
    s = np.zeros_like(s_ref)
    NH.call("nh_quantize_rows_i8_host", x.ctypes.data, NH.F32, x.shape[0], x.shape[1], q.ctypes.data, s.ctypes.data)
    assert np.array_equal(q, q_ref)


@pytest.mark.parametrize("kat", KATS["gemm"] + [dict(KATS["gemm_pattern"][0], lhs=None)],
                         ids=lambda k: k["src"].split("/")[-1])
def test_gemm_f32_host_twin_matches_oracle(kat):
    m, k, n = kat["m"], kat["k"], kat["n"]
    if kat["lhs"] is None:
        lhs = np.array([((i % 11) - 5) * 0.25 for i in range(m * k)], dtype=np.float32)
        rhs = np.array([((i % 7) - 3) * 0.5 for i in range(k * n)], dtype=np.float32)
    else:
        lhs = np.array(kat["lhs"], dtype=np.float32)
        rhs = np.array(kat["rhs"], dtype=np.float32)
    out = np.zeros(m * n, dtype=np.float32)
    NH.call("nh_gemm_f32_host", lhs.ctypes.data, lhs.size, rhs.ctypes.data, rhs.size, m, k, n, out.ctypes.data, out.size)
    _, ref, _ = O.gemm_f32(lhs, rhs, m, k, n)
    assert np.array_equal(out, ref)


def test_gemm_f32_host_twin_errors_match_reference():
    one = np.ones(4, dtype=np.float32)
    st, err = NH.call_status("nh_gemm_f32_host", one.ctypes.data, 1, one.ctypes.data, 2, 1, 2, 1, one.ctypes.data, 1)
    assert st == NH.LENGTH_MISMATCH and (err.argument, err.expected, err.actual) == (b"lhs", 2, 1)
    st, err = NH.call_status("nh_gemm_f32_host", one.ctypes.data, 1, one.ctypes.data, 1, 2, (1 << 64) - 1, 1,
                             one.ctypes.data, 2)
    assert st == NH.INVALID_SHAPE


@pytest.mark.parametrize("kat", KATS["gemm_errors"], ids=lambda k: k["src"].split(":")[-1])
def test_device_gemm_f32_validates_like_gemm_into(kat):
    """G0d's device entry point returns the reference's error variants and
    payloads (gemm.rs:490-621) before it touches a device (NULL context)."""
    usize_max = (1 << 64) - 1
    k = usize_max if kat["k"] == "usize::MAX" else kat["k"]
    st, err = NH.call_status("nh_gemm_f32", None, None, kat["lhs_len"], None, kat["rhs_len"], kat["m"], k, kat["n"],
                             None, kat["out_len"], None)
    if kat["error"] == "InvalidShape":
        assert st == NH.INVALID_SHAPE
    else:
        assert st == NH.LENGTH_MISMATCH
        assert (err.argument.decode(), err.expected, err.actual) == (kat["argument"], kat["expected"], kat["actual"])
    assert NH.lib().nh_supports_gemm_f32(3, 5, 7) == 1 and NH.lib().nh_supports_gemm_f32(0, 5, 7) == 0
    assert NH.lib().nh_supports_gemm_f32(1 << 31, 1, 1) == 0


def test_w8a8_and_w8a32_host_twins_match_oracle():
    rng = np.random.default_rng(2)
    m, n, k = 5, 33, 96
    xq = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    wq = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sx = rng.uniform(1e-3, 1e-2, m).astype(np.float32)
    sw = rng.uniform(1e-4, 1e-3, n).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    wt = tile_16x64(wq)
    for dt, npdt, bf in ((NH.F32, np.float32, False), (NH.BF16, np.uint16, True)):
        out = np.zeros((m, n), dtype=npdt)
        NH.call("nh_gemm_w8a8_host", xq.ctypes.data, sx.ctypes.data, wt.ctypes.data, sw.ctypes.data, bias.ctypes.data,
                m, n, k, out.ctypes.data, dt)
        assert np.array_equal(out, O.linear_w8a8(xq, sx, wq, sw, bias=bias, out_bf16=bf))
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = np.zeros((m, n), dtype=np.float32)
    NH.call("nh_gemv_w8a32_host", x.ctypes.data, wt.ctypes.data, sw.ctypes.data, m, n, k, y.ctypes.data)
    assert np.array_equal(y, O.gemv_w8a32(x, wq, sw))


@pytest.mark.parametrize("n,k", [(1, 1), (16, 64), (33, 96), (17, 200), (48, 4112)])
def test_tile_weights_host_twin_matches_layout(n, k):
    rng = np.random.default_rng(n * 1000 + k)
    wq = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    nbytes = NH.lib().nh_tiled_weights_bytes(n, k)
    assert nbytes == tiled_bytes(n, k) == -(-n // 16) * 16 * -(-k // 64) * 64
    out = np.full(nbytes, 0x55, dtype=np.int8)
    NH.call("nh_tile_weights_i8_host", wq.ctypes.data, n, k, out.ctypes.data, nbytes)
    ref = tile_16x64(wq)
    assert np.array_equal(out, ref)
    # spot check of the layout formula itself: W[n][k] sits at tile (n/16, k/64), byte 16*(16*g + r) + b
    kt = -(-k // 64)
    for (r_, c_) in [(0, 0), (n - 1, k - 1), (n // 2, k // 3)]:
        off = ((r_ // 16) * kt + c_ // 64) * 1024 + 16 * (16 * ((c_ % 64) // 16) + r_ % 16) + c_ % 16
        assert out[off] == wq[r_, c_]
    # the padding is zero and every matrix byte appears once
    assert np.count_nonzero(out) == np.count_nonzero(wq)


def test_tile_weights_host_twin_errors():
    one = np.zeros(64, dtype=np.int8)
    st, err = NH.call_status("nh_tile_weights_i8_host", one.ctypes.data, 1, 1, one.ctypes.data, 63)
    assert st == NH.LENGTH_MISMATCH and (err.argument, err.expected, err.actual) == (b"tiled", 1024, 63)
    st, _ = NH.call_status("nh_tile_weights_i8_host", one.ctypes.data, 0, 1, one.ctypes.data, 0)
    assert st == NH.INVALID_SHAPE
    assert NH.lib().nh_tiled_weights_bytes(0, 5) == 0
    st, _ = NH.call_status("nh_tile_weights_i8", None, one.ctypes.data, 1, 1, one.ctypes.data, 63, None)
    assert st == NH.LENGTH_MISMATCH  # validated before the (absent) device is touched


def test_sigmoid_host_twin_equals_glibc_expf_sigmoid():
    # The library evaluates expf with a restated table method; the oracle
    # calls glibc expf.  Dense sweep of the N(0,1)-relevant range plus a
    # strided sweep of every float exponent.
    L = NH.lib()
    xs = np.concatenate([np.linspace(-12, 12, 200001, dtype=np.float32),
                         np.array([0.0, -0.0, 1e-30, -1e-30, 88.7, -88.7, 103.9, -103.9, 200.0, -200.0],
                                  dtype=np.float32)])
    bits = np.arange(0, 0x7F800000, 7919, dtype=np.uint32)
    xs = np.concatenate([xs, bits.view(np.float32), (bits | 0x80000000).view(np.float32)])
    lib_s = np.array([L.nh_sigmoid_f32_host(float(v)) for v in xs[::3]], dtype=np.float32)
    ora_s = np.array([O.sigmoid(float(v)) for v in xs[::3]], dtype=np.float32)
    assert np.array_equal(lib_s.view(np.uint32), ora_s.view(np.uint32))


@pytest.mark.parametrize("kat", KATS["routing_sigmoid"], ids=lambda k: k["src"].split("/")[-1])
def test_route_host_twin_reference_kats(kat):
    t, e, k = kat["tokens"], kat["experts"], kat["top_k"]
    scores = np.array(kat["scores"], dtype=np.float32)
    idx = np.zeros(max(t * k, 1), dtype=np.int32)
    w = np.zeros(max(t * k, 1), dtype=np.float32)
    NH.call("nh_moe_route_sigmoid_topk_host", scores.ctypes.data, scores.size, t, e, k, 0, 1.0, idx.ctypes.data,
            t * k, w.ctypes.data, t * k)
    _, ridx, rw, _ = O.route_sigmoid(scores, t, e, k)
    assert np.array_equal(idx[:t * k], ridx) and np.array_equal(w[:t * k], rw)


def test_route_host_twins_match_oracle_on_random_logits():
    t, e, k = 64, 128, 6
    scores = O.normal_f32(2, t * e)
    for renorm, scaling in ((0, 1.0), (1, 1.0), (1, 2.5)):
        idx = np.zeros(t * k, dtype=np.int32)
        w = np.zeros(t * k, dtype=np.float32)
        NH.call("nh_moe_route_sigmoid_topk_host", scores.ctypes.data, scores.size, t, e, k, renorm, scaling,
                idx.ctypes.data, t * k, w.ctypes.data, t * k)
        _, ridx, rw, _ = O.route_sigmoid(scores, t, e, k, renormalize=bool(renorm), scaling=scaling)
        assert np.array_equal(idx, ridx) and np.array_equal(w, rw)
    idx = np.zeros(t * k, dtype=np.int32)
    w = np.zeros(t * k, dtype=np.float32)
    NH.call("nh_moe_route_softmax_topk_host", scores.ctypes.data, scores.size, t, e, k, idx.ctypes.data, t * k,
            w.ctypes.data, t * k)
    _, ridx, rw, _ = O.route_softmax(scores, t, e, k)
    assert np.array_equal(idx, ridx) and np.array_equal(w, rw)


@pytest.mark.parametrize("kat", KATS["routing_errors"], ids=lambda k: k["src"].split("/")[-1])
def test_route_host_twin_reference_error_kats(kat):
    buf = np.zeros(8, dtype=np.float32)
    ibuf = np.zeros(8, dtype=np.int32)
    st, err = NH.call_status("nh_moe_route_sigmoid_topk_host", buf.ctypes.data, kat["scores_len"], kat["tokens"],
                             kat["experts"], kat["top_k"], 0, 1.0, ibuf.ctypes.data, kat["indices_len"],
                             buf.ctypes.data, kat["weights_len"])
    if kat["error"] == "InvalidShape":
        assert st == NH.INVALID_SHAPE
    else:
        assert st == NH.LENGTH_MISMATCH
        assert (err.argument.decode(), err.expected, err.actual) == (kat["argument"], kat["expected"], kat["actual"])


def test_moe_host_twins_match_oracle():
    rng = np.random.default_rng(11)
    tokens, k_top, experts, hidden, inter = 19, 3, 7, 64, 32
    idx = np.stack([rng.choice(experts, size=k_top, replace=False) for _ in range(tokens)]).astype(np.int32).ravel()
    R = tokens * k_top
    offsets = np.zeros(experts + 1, dtype=np.int32)
    perm = np.zeros(R, dtype=np.int32)
    pos = np.zeros(R, dtype=np.int32)
    NH.call("nh_moe_permute_host", idx.ctypes.data, tokens, k_top, experts, offsets.ctypes.data, perm.ctypes.data,
            pos.ctypes.data)
    o_off, o_perm, o_pos = O.moe_permute(idx, tokens, k_top, experts)
    assert np.array_equal(offsets, o_off) and np.array_equal(perm, o_perm) and np.array_equal(pos, o_pos)
    xq = rng.integers(-127, 128, size=(tokens, hidden), dtype=np.int8)
    sx = rng.uniform(1e-3, 1e-2, tokens).astype(np.float32)
    w = rng.integers(-127, 128, size=(experts, inter, hidden), dtype=np.int8)
    sw = rng.uniform(1e-4, 1e-3, (experts, inter)).astype(np.float32)
    out = np.zeros((R, inter), dtype=np.float32)
    wt = tile_experts(w)
    NH.call("nh_moe_grouped_gemm_w8a8_host", xq.ctypes.data, sx.ctypes.data, 1, k_top, offsets.ctypes.data,
            perm.ctypes.data, R, tokens, experts, wt.ctypes.data, sw.ctypes.data, inter, hidden, 1, out.ctypes.data)
    ref = O.moe_grouped(xq, sx, True, k_top, offsets, perm, w, sw, relu2=True)
    assert np.array_equal(out, ref)
    weights = rng.uniform(0, 1, R).astype(np.float32)
    comb = np.zeros((tokens, inter), dtype=np.uint16)
    NH.call("nh_moe_combine_host", out.ctypes.data, pos.ctypes.data, weights.ctypes.data, tokens, k_top, inter,
            comb.ctypes.data, NH.BF16)
    assert np.array_equal(comb, O.moe_combine(out, pos, weights, tokens, k_top, inter, out_bf16=True))

    # with a shared expert's rows, added ahead of the routes
    shared = rng.standard_normal((tokens, inter)).astype(np.float32)
    comb_sh = np.zeros((tokens, inter), dtype=np.float32)
    NH.call("nh_moe_combine_shared_host", out.ctypes.data, pos.ctypes.data, weights.ctypes.data, shared.ctypes.data,
            tokens, k_top, inter, comb_sh.ctypes.data, NH.F32)
    assert np.array_equal(comb_sh, O.moe_combine_shared(out, pos, weights, shared, tokens, k_top, inter))


def test_moe_forward_shared_validation_before_any_launch():
    """nh_moe_forward_shared_w8a8 rejects a missing shared expert, an empty
    shared intermediate and a short workspace before touching the device
    (NULL context)."""
    T, H, I, E, K, SI = 4, 64, 32, 8, 2, 48
    need = NH.lib().nh_moe_forward_shared_w8a8_workspace_size(T, H, I, E, K, SI)
    assert need > NH.lib().nh_moe_forward_w8a8_workspace_size(T, H, I, E, K)

    def call(si, up_sh, ws_bytes, tokens=T):
        dummy = 16
        return NH.call_status("nh_moe_forward_shared_w8a8", None, dummy, NH.BF16, dummy, tokens, H, I, E, K, 1, 1.0,
                              dummy, dummy, dummy, dummy, si, up_sh, dummy, dummy, dummy, None, dummy, NH.BF16,
                              dummy if ws_bytes else None, ws_bytes, None, None)

    assert call(SI, None, need)[0] == NH.INVALID_PARAMS
    assert call(0, 16, need)[0] == NH.INVALID_SHAPE
    assert call(SI, 16, need, tokens=0)[0] == NH.INVALID_ROW_COUNT
    st, err = call(SI, 16, need - 1)
    assert st == NH.LENGTH_MISMATCH and err.argument.decode() == "workspace" and err.expected == need


def test_int4_host_twins_match_oracle_and_layout():
    from tiling import tile_int4
    rng = np.random.default_rng(12)
    for (m, k, n, zp) in [(1, 64, 16, 8), (3, 200, 33, 0), (5, 1040, 100, 15)]:
        packed = rng.integers(0, 256, size=(k * n + 1) // 2, dtype=np.uint8)
        need = NH.lib().nh_tiled_int4_weights_bytes(n, k)
        assert need == (n + 15) // 16 * ((k + 63) // 64) * 512
        tiled = np.zeros(need, dtype=np.uint8)
        NH.call("nh_tile_weights_int4_host", packed.ctypes.data, packed.size, k, n, zp, tiled.ctypes.data, need)
        assert np.array_equal(tiled, tile_int4(packed, k, n, zp))
        x = O.to_bf16(O.normal_f32(7, m * k)).reshape(m, k)
        bias = rng.standard_normal(n).astype(np.float32)
        for out_dtype, bf in ((NH.BF16, True), (NH.F32, False)):
            y = np.zeros((m, n), dtype=np.uint16 if bf else np.float32)
            NH.call("nh_linear_w4a8_host", x.ctypes.data, NH.BF16, packed.ctypes.data, packed.size, 0.0123, zp,
                    bias.ctypes.data, m, n, k, y.ctypes.data, out_dtype)
            st, ref = O.linear_w4a8(x, packed, n, 0.0123, zp, bias=bias, out_bf16=bf)
            assert st == O.OK and np.array_equal(y, ref)
        # f32 rows holding bf16 values quantize exactly like the bf16 rows
        xf = (x.astype(np.uint32) << 16).view(np.float32)
        y = np.zeros((m, n), dtype=np.float32)
        NH.call("nh_linear_w4a8_host", xf.ctypes.data, NH.F32, packed.ctypes.data, packed.size, 0.0123, zp,
                None, m, n, k, y.ctypes.data, NH.F32)
        assert np.array_equal(y, O.linear_w4a8(x, packed, n, 0.0123, zp)[1])


def test_int4_validation_in_the_reference_order():
    packed = np.zeros(2, dtype=np.uint8)
    y = np.zeros(4, dtype=np.float32)
    x = np.zeros(4, dtype=np.float32)

    def host(k, n, plen, scale, zp, m):
        return NH.call_status("nh_linear_w4a8_host", x.ctypes.data, NH.F32, packed.ctypes.data, plen, scale, zp,
                              None, m, n, k, y.ctypes.data, NH.F32)
    assert host(0, 2, 0, 0.5, 8, 1)[0] == NH.INVALID_SHAPE
    st, err = host(2, 2, 1, 0.5, 8, 1)  # linear.rs:113-121
    assert st == NH.LENGTH_MISMATCH and (err.argument.decode(), err.expected, err.actual) == ("packed_weights", 2, 1)
    assert host(2, 2, 2, 0.0, 8, 1)[0] == NH.INVALID_PARAMS  # quantize.rs:180-186
    assert host(2, 2, 2, float("nan"), 8, 1)[0] == NH.INVALID_PARAMS
    assert host(2, 2, 2, 0.5, 16, 1)[0] == NH.INVALID_PARAMS
    assert host(2, 2, 2, 0.5, 8, 0)[0] == NH.INVALID_ROW_COUNT
    # the device entry point validates before touching the (NULL) context
    dev = lambda m, n, k, scale=0.5, zp=8, dt=NH.BF16: NH.call_status(  # noqa: E731
        "nh_linear_w4a8", None, 16, dt, 16, scale, zp, None, m, n, k, 16, NH.BF16, None, 0, None, None)
    assert dev(1, 0, 64)[0] == NH.INVALID_SHAPE
    assert dev(1, 16, 64, scale=-1.0)[0] == NH.INVALID_PARAMS
    assert dev(0, 16, 64)[0] == NH.INVALID_ROW_COUNT
    # past the fused unit (m > 16, k > 8192, f32 rows): the expanded form needs its workspace
    for st, err in (dev(17, 16, 64), dev(1, 16, 8192 + 16), dev(1, 16, 64, dt=NH.F32)):
        assert st == NH.LENGTH_MISMATCH and err.argument == b"workspace" and err.actual == 0
    assert dev(1, 16, 72)[0] == NH.UNSUPPORTED  # k % 16 != 0: the W8A8 envelope
    L = NH.lib()
    assert L.nh_linear_w4a8_workspace_size(2048, 4096, 4096) == (
        4096 * 4096 + 4096 * 4 + L.nh_linear_w8a8_workspace_size(2048, 4096))
    assert L.nh_linear_w4a8_workspace_size(0, 4096, 4096) == 0
    st, err = NH.call_status("nh_tile_weights_int4", None, 16, 3, 2, 2, 8, 16, 512, None)
    assert st == NH.LENGTH_MISMATCH and err.argument.decode() == "packed_weights"


def test_combine_skips_routes_without_a_slot():
    """A route the permutation did not place (pos -1) adds nothing, on the
    host twin as in the oracle."""
    slot_out = np.array([[1.0, 2.0], [3.0, 4.0]], dtype=np.float32)
    pos = np.array([1, -1], dtype=np.int32)
    w = np.array([0.5, 0.25], dtype=np.float32)
    out = np.zeros((1, 2), dtype=np.float32)
    NH.call("nh_moe_combine_host", slot_out.ctypes.data, pos.ctypes.data, w.ctypes.data, 1, 2, 2, out.ctypes.data,
            NH.F32)
    assert np.array_equal(out, np.array([[1.5, 2.0]], dtype=np.float32))
    assert np.array_equal(out, O.moe_combine(slot_out, pos, w, 1, 2, 2))


def test_linear_noalloc_rejects_a_workspace_above_its_scratch_before_the_device():
    # 2048 x 32768 needs 64 MiB of A tiles + 8 KiB of scales: above the 64 MiB
    # static scratch, refused before the (null) context is touched
    st, err = NH.call_status("nh_linear_w8a8_noalloc", None, None, NH.BF16, None, None, None, 2048, 64, 32768, None,
                             NH.BF16, None, None, None, None)
    assert st == NH.UNSUPPORTED and b"static scratch" in err.message
    assert NH.lib().nh_linear_w8a8_workspace_size(2048, 32768) > 64 << 20
    assert NH.lib().nh_linear_w8a8_workspace_size(2048, 32704) <= 64 << 20
    # m == 0 and shape errors keep the order of nh_linear_w8a8
    assert NH.call_status("nh_linear_w8a8_noalloc", None, None, NH.BF16, None, None, None, 0, 64, 64, None, NH.BF16,
                          None, None, None, None)[0] == NH.INVALID_ROW_COUNT


# ---- layer host twins (the host-fallback contract, gemm.rs:290-310) ----------
@pytest.mark.parametrize("m,n,k,xdt,odt", [(3, 37, 100, "f32", "f32"),   # k % 16 != 0: outside the device envelope
                                           (5, 33, 96, "bf16", "bf16"), (1, 20, 1, "bf16", "f32"),
                                           (17, 9, 200, "f32", "bf16")])
def test_linear_host_twin_matches_oracle(m, n, k, xdt, odt):
    """nh_linear_w8a8_host = Q2 + the W8A8 product + bias (the oracle's parts),
    bit for bit, on shapes the device rejects (k % 16 != 0) and accepts; the
    device entry point returns Unsupported outside nh_supports_linear_w8a8
    before touching a device, so a caller takes this twin there."""
    rng = np.random.default_rng(m * 100 + k)
    w = O.normal_f32(0, n * k, 0.0, 0.02).reshape(n, k)
    _, wq, sw, _ = O.quantize_rows_f32(w)
    bias = rng.standard_normal(n).astype(np.float32)
    xf = O.normal_f32(1, m * k).reshape(m, k)
    if xdt == "bf16":
        x = O.to_bf16(xf)
        st, xq, sx, _ = O.quantize_rows_bf16(x)
    else:
        x = xf
        st, xq, sx, _ = O.quantize_rows_f32(x)
    assert st == O.OK
    bf = odt == "bf16"
    ref = O.linear_w8a8(xq, sx, wq, sw, bias=bias, out_bf16=bf)
    out = np.zeros((m, n), dtype=np.uint16 if bf else np.float32)
    xq_out = np.zeros((m, k), dtype=np.int8)
    sx_out = np.zeros(m, dtype=np.float32)
    wt = tile_16x64(wq)
    NH.call("nh_linear_w8a8_host", x.ctypes.data, NH.BF16 if xdt == "bf16" else NH.F32, wt.ctypes.data,
            sw.ctypes.data, bias.ctypes.data, m, n, k, out.ctypes.data, NH.BF16 if bf else NH.F32,
            xq_out.ctypes.data, sx_out.ctypes.data)
    assert np.array_equal(out, ref)
    assert np.array_equal(xq_out, xq) and np.array_equal(sx_out.view(np.uint32), sx.view(np.uint32))
    supported = NH.lib().nh_supports_linear_w8a8(m, n, k)
    assert supported == (k % 16 == 0)
    if not supported:
        st, err = NH.call_status("nh_linear_w8a8", None, 16, NH.F32, 16, 16, None, m, n, k, 16, NH.F32, 16, 1 << 30,
                                 None, None, None, None)
        assert st == NH.UNSUPPORTED


def test_linear_host_twin_errors_and_nonfinite():
    k, n = 48, 8
    x = O.normal_f32(3, 2 * k).reshape(2, k)
    x[1, 7] = np.nan
    x[1, 9] = np.inf
    _, wq, sw, _ = O.quantize_rows_f32(O.normal_f32(0, n * k, 0.0, 0.02).reshape(n, k))
    wt = tile_16x64(wq)
    out = np.zeros((2, n), dtype=np.float32)
    st, err = NH.call_status("nh_linear_w8a8_host", x.ctypes.data, NH.F32, wt.ctypes.data, sw.ctypes.data, None, 2,
                             n, k, out.ctypes.data, NH.F32, None, None)
    assert st == NH.NON_FINITE_INPUT and err.argument == b"input" and err.index == k + 7 and math.isnan(err.value)
    for m_, n_, k_, want in ((0, n, k, NH.INVALID_ROW_COUNT), (2, 0, k, NH.INVALID_SHAPE), (2, n, 0, NH.INVALID_SHAPE)):
        st, _ = NH.call_status("nh_linear_w8a8_host", x.ctypes.data, NH.F32, wt.ctypes.data, sw.ctypes.data, None, m_,
                               n_, k_, out.ctypes.data, NH.F32, None, None)
        assert st == want


@pytest.mark.parametrize("m,hidden,inter", [(3, 40, 24), (2, 64, 32), (1, 17, 5)])
def test_mlp_host_twin_matches_oracle(m, hidden, inter):
    """nh_mlp_w8a8_host = the oracle's int8 MLP with biases (or_mlp_w8a8),
    bit for bit, also at hidden / inter not multiples of 16 (no device form);
    an overflowing intermediate is NonFiniteInput "intermediate" at the
    oracle's index, a non-finite x "input"."""
    rng = np.random.default_rng(hidden)
    x = O.to_bf16(O.normal_f32(7, m * hidden)).reshape(m, hidden)
    _, wu, su, _ = O.quantize_rows_f32(O.normal_f32(8, inter * hidden, 0, 0.02).reshape(inter, hidden))
    _, wd, sd, _ = O.quantize_rows_f32(O.normal_f32(9, hidden * inter, 0, 0.02).reshape(hidden, inter))
    bu = rng.standard_normal(inter).astype(np.float32)
    bd = rng.standard_normal(hidden).astype(np.float32)
    st, ref = O.mlp_w8a8(x, wu, su, wd, sd, b_up=bu, b_down=bd)
    assert st == O.OK
    wut, wdt = tile_16x64(wu), tile_16x64(wd)
    out = np.zeros((m, hidden), dtype=np.float32)
    args = lambda xx, b_up: (xx.ctypes.data, NH.BF16, wut.ctypes.data, su.ctypes.data, b_up.ctypes.data,
                             wdt.ctypes.data, sd.ctypes.data, bd.ctypes.data, m, hidden, inter, out.ctypes.data, NH.F32)
    NH.call("nh_mlp_w8a8_host", *args(x, bu))
    assert np.array_equal(out, ref)
    assert NH.lib().nh_supports_mlp_w8a8(m, hidden, inter) == (hidden % 16 == 0 and inter % 16 == 0)
    # the intermediate overflows: ReLU^2 of a 3e38 biased output is +inf
    big = bu.copy()
    big[inter - 1] = 3e38
    _, xq, sx, _ = O.quantize_rows_bf16(x)
    h = O.epilogue(O.gemm_i8_i32(xq, wu), sx, su, bias=big, relu2=True)
    ost, _, _, oerr = O.quantize_rows_f32(h)
    assert ost == O.NON_FINITE_INPUT
    st, err = NH.call_status("nh_mlp_w8a8_host", *args(x, big))
    assert st == NH.NON_FINITE_INPUT and err.argument == b"intermediate" and err.index == oerr.index
    assert np.isinf(err.value)
    xb = x.copy()
    xb[m - 1, 2] = 0x7fc0  # bf16 NaN: the input wins over the intermediate
    st, err = NH.call_status("nh_mlp_w8a8_host", *args(xb, big))
    assert st == NH.NON_FINITE_INPUT and err.argument == b"input" and err.index == (m - 1) * hidden + 2


def _moe_host_case(tokens, hidden, inter, experts, top_k, sh_inter, seed=3):
    rng = np.random.default_rng(seed)
    x = O.to_bf16(O.normal_f32(1, tokens * hidden)).reshape(tokens, hidden)
    rw = O.normal_f32(2, hidden * experts, 0.0, 0.1)
    rb = rng.standard_normal(experts).astype(np.float32)
    _, qu, su, _ = O.quantize_rows_f32(O.normal_f32(3, experts * inter * hidden, 0, 0.02).reshape(-1, hidden))
    _, qd, sd, _ = O.quantize_rows_f32(O.normal_f32(4, experts * hidden * inter, 0, 0.02).reshape(-1, inter))
    qu, su = qu.reshape(experts, inter, hidden), su.reshape(experts, inter)
    qd, sd = qd.reshape(experts, hidden, inter), sd.reshape(experts, hidden)
    sh = None
    if sh_inter:
        _, hu, hsu, _ = O.quantize_rows_f32(O.normal_f32(5, sh_inter * hidden, 0, 0.02).reshape(sh_inter, hidden))
        _, hd, hsd, _ = O.quantize_rows_f32(O.normal_f32(6, hidden * sh_inter, 0, 0.02).reshape(hidden, sh_inter))
        sh = (hu, hsu, hd, hsd)
    biases = [rng.standard_normal((experts, inter)).astype(np.float32) * 0.5,
              rng.standard_normal((experts, hidden)).astype(np.float32),
              rng.standard_normal(sh_inter).astype(np.float32) * 0.5 if sh_inter else None,
              rng.standard_normal(hidden).astype(np.float32) if sh_inter else None]
    return x, rw, rb, qu, su, qd, sd, sh, biases


def _moe_host_call(x, xdt, rw, rb, qu, su, qd, sd, sh, biases, top_k, renorm, scaling, out_dtype=NH.BF16):
    tokens, hidden = x.shape
    experts, inter, _ = qu.shape
    sh_inter = sh[0].shape[0] if sh is not None else 0
    tiles = [tile_experts(qu), tile_experts(qd)] + ([tile_16x64(sh[0]), tile_16x64(sh[2])] if sh is not None else [])
    shp = [tiles[2].ctypes.data, sh[1].ctypes.data, tiles[3].ctypes.data, sh[3].ctypes.data] if sh is not None \
        else [None] * 4
    mb = NH.MoeBiases(*[None if b is None else b.ctypes.data for b in biases]) if biases is not None else None
    out = np.zeros((tokens, hidden), dtype=np.uint16 if out_dtype == NH.BF16 else np.float32)
    st, err = NH.call_status("nh_moe_layer_w8a8_host", x.ctypes.data, xdt, rw.ctypes.data, rb.ctypes.data, tokens,
                             hidden, inter, experts, top_k, renorm, C.c_float(scaling), tiles[0].ctypes.data,
                             su.ctypes.data, tiles[1].ctypes.data, sd.ctypes.data, sh_inter, *shp, mb,
                             out.ctypes.data, out_dtype)
    return st, err, out


@pytest.mark.parametrize("tokens,hidden,inter,experts,top_k,sh_inter,renorm,scaling",
                         [(9, 64, 32, 8, 3, 48, 0, 1.0), (7, 40, 24, 5, 2, 0, 1, 2.5),  # 40 / 24: no device form
                          (5, 48, 20, 6, 6, 12, 1, 1.0)])
def test_moe_layer_host_twin_matches_oracle(tokens, hidden, inter, experts, top_k, sh_inter, renorm, scaling):
    """nh_moe_layer_w8a8_host = router.project (gemm_into_host then the bias,
    linear.rs:325-339: or_linear_project) + the oracle's int8 MoE with its
    shared expert and all four biases, bit for bit; with f32 x of bf16 values
    the same output."""
    x, rw, rb, qu, su, qd, sd, sh, b = _moe_host_case(tokens, hidden, inter, experts, top_k, sh_inter)
    logits = np.zeros(tokens * experts, dtype=np.float32)
    xf = O.bf16_to_f32(x)
    err = O.OrError()
    assert O.lib().or_linear_project(O.ptr(xf), xf.size, tokens, O.ptr(rw), hidden, experts, O.ptr(rb),
                                     O.ptr(logits), logits.size, C.byref(err)) == O.OK
    shargs = sh if sh is not None else (None, None, None, None)
    st, ref, *_ = O.moe_forward_shared_w8a8(x, logits, qu, su, qd, sd, top_k, *shargs, renormalize=bool(renorm),
                                            scaling=scaling, biases=tuple(b))
    assert st == O.OK
    st, e, out = _moe_host_call(x, NH.BF16, rw, rb, qu, su, qd, sd, sh, b, top_k, renorm, scaling)
    assert st == NH.OK, e.message
    assert np.array_equal(out, ref)
    st, e, out_f = _moe_host_call(np.ascontiguousarray(xf), NH.F32, rw, rb, qu, su, qd, sd, sh, b, top_k, renorm,
                                  scaling)
    assert st == NH.OK and np.array_equal(out_f, ref)
    supported = NH.lib().nh_supports_moe_layer_w8a8(tokens, hidden, inter, experts, top_k, sh_inter)
    assert supported == (hidden % 16 == 0 and inter % 16 == 0 and (sh_inter % 16 == 0))


def test_moe_layer_host_twin_nonfinite_order_and_errors():
    """Input first, then the shared expert's intermediate, then the routed
    experts' (the order MoeLayer::forward_into meets them, moe.rs:197-233, and
    the device word's stages)."""
    tokens, hidden, inter, experts, top_k, sh_inter = 6, 32, 16, 4, 2, 16
    x, rw, rb, qu, su, qd, sd, sh, b = _moe_host_case(tokens, hidden, inter, experts, top_k, sh_inter)
    b_sh_big = list(b)
    b_sh_big[2] = b[2].copy()
    b_sh_big[2][3] = 3e38
    st, e, _ = _moe_host_call(x, NH.BF16, rw, rb, qu, su, qd, sd, sh, b_sh_big, top_k, 0, 1.0)
    assert st == NH.NON_FINITE_INPUT and e.argument == b"shared_intermediate" and np.isinf(e.value)
    assert e.index % sh_inter == 3
    b_all_big = list(b_sh_big)
    b_all_big[0] = b[0].copy()
    b_all_big[0][:, 5] = 3e38
    st, e, _ = _moe_host_call(x, NH.BF16, rw, rb, qu, su, qd, sd, sh, b_all_big, top_k, 0, 1.0)
    assert st == NH.NON_FINITE_INPUT and e.argument == b"shared_intermediate"
    st, e, _ = _moe_host_call(x, NH.BF16, rw, rb, qu, su, qd, sd, sh, [b_all_big[0], b[1], b[2], b[3]], top_k, 0, 1.0)
    assert st == NH.NON_FINITE_INPUT and e.argument == b"intermediate" and e.index == 5  # slot 0, column 5
    xb = x.copy()
    xb[2, 4] = 0xff80  # -inf
    st, e, _ = _moe_host_call(xb, NH.BF16, rw, rb, qu, su, qd, sd, sh, b_all_big, top_k, 0, 1.0)
    assert st == NH.NON_FINITE_INPUT and e.argument == b"input" and e.index == 2 * hidden + 4 and e.value < 0
    # shared biases without a shared expert
    st, e, _ = _moe_host_call(x, NH.BF16, rw, rb, qu, su, qd, sd, None, [None, None, b[2], None], top_k, 0, 1.0)
    assert st == NH.INVALID_PARAMS
    st, e, _ = _moe_host_call(x[:0], NH.BF16, rw, rb, qu, su, qd, sd, sh, b, top_k, 0, 1.0)
    assert st == NH.INVALID_ROW_COUNT
