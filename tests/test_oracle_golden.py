"""Pins the CPU oracle before anything is compared with it.

Three kinds of check, chosen so that a plausible slip in the oracle (dropped
term, wrong sign or index, transposed operand, wrong rounding mode) fails one:
  1. the reference's own known-answer tests, transcribed in
     tests/golden/reference_kats.json (each entry cites its source file:line);
  2. closed forms / textbook routines (numpy int64 and float64 matmul, sorted()
     with an explicit key, numpy stable argsort, Python's float arithmetic);
  3. invariants of the spec-defined int8 functions (range, absmax code, half-
     step error bound, tie rounding, zero rows, non-finite reporting).
"""
import ctypes as C
import json
import math
import os
import struct

import numpy as np
import pytest

import oracle_ctypes as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")
KATS = json.load(open(GOLDEN))


def f32(v):
    return float("nan") if v == "NaN" else float(v)


def assert_close(got, want, tol):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape
    assert np.all(np.abs(got - want) <= tol), (got, want)


# --------------------------------------------------------------------------
# INT4 (quantize.rs KATs)
@pytest.mark.parametrize("kat", KATS["int4"], ids=lambda k: k["src"].split("/")[-1])
def test_int4_reference_kats(kat):
    L = O.lib()
    op = kat["op"]
    err = O.OrError()
    if op == "pack":
        vals = np.array(kat["values"], dtype=np.uint8)
        packed = np.zeros(len(kat["packed"]), dtype=np.uint8)
        assert L.or_pack_int4(O.ptr(vals), vals.size, O.ptr(packed), packed.size, C.byref(err)) == O.OK
        assert packed.tolist() == kat["packed"]
        out = np.zeros(vals.size, dtype=np.uint8)
        assert L.or_unpack_int4(O.ptr(packed), packed.size, vals.size, O.ptr(out), out.size, C.byref(err)) == O.OK
        assert out.tolist() == kat["values"]
    elif op in ("quantize_dequantize", "quantize_into", "device_dequantize", "dequantize_into"):
        if "values" in kat:
            vals = np.array([f32(v) for v in kat["values"]], dtype=np.float32)
            packed = np.array(kat.get("packed_init", [0] * len(kat["packed"])), dtype=np.uint8)
            st = L.or_quantize_int4(O.ptr(vals), vals.size, kat["scale"], kat["zero_point"], O.ptr(packed),
                                    packed.size, C.byref(err))
            assert st == O.OK
            assert packed.tolist() == kat["packed"]
        if "dequantized" in kat:
            packed = np.array(kat["packed"], dtype=np.uint8)
            n = kat.get("value_count", len(kat.get("values", [])))
            out = np.full(n, -1.0, dtype=np.float32)
            st = L.or_dequantize_int4(O.ptr(packed), packed.size, n, kat["scale"], kat["zero_point"], O.ptr(out),
                                      n, C.byref(err))
            assert st == O.OK
            assert_close(out, kat["dequantized"], kat["tol"])
    elif op == "empty":
        z = np.zeros(1, dtype=np.uint8)
        zf = np.zeros(1, dtype=np.float32)
        assert L.or_pack_int4(O.ptr(z), 0, O.ptr(z), 0, C.byref(err)) == O.OK
        assert L.or_unpack_int4(O.ptr(z), 0, 0, O.ptr(z), 0, C.byref(err)) == O.OK
        assert L.or_quantize_int4(O.ptr(zf), 0, kat["scale"], kat["zero_point"], O.ptr(z), 0, C.byref(err)) == O.OK
        assert L.or_dequantize_int4(O.ptr(z), 0, 0, kat["scale"], kat["zero_point"], O.ptr(zf), 0,
                                    C.byref(err)) == O.OK
    elif op == "quantize_error":
        vals = np.array([f32(v) for v in kat["values"]], dtype=np.float32)
        packed = np.zeros(max(kat["packed_len"], 1), dtype=np.uint8)
        st = L.or_quantize_int4(O.ptr(vals), vals.size, kat["scale"], kat["zero_point"], O.ptr(packed),
                                kat["packed_len"], C.byref(err))
        expect = {"InvalidParams": O.INVALID_PARAMS, "LengthMismatch": O.LENGTH_MISMATCH,
                  "NonFiniteInput": O.NON_FINITE_INPUT}[kat["error"]]
        assert st == expect
        if kat["error"] == "LengthMismatch":
            assert (err.argument.decode(), err.expected, err.actual) == (kat["argument"], kat["expected"], kat["actual"])
        if kat["error"] == "NonFiniteInput":
            assert err.index == kat["index"] and math.isnan(err.value)
    elif op == "pack_error":
        vals = np.array(kat["values"], dtype=np.uint8)
        packed = np.zeros(1, dtype=np.uint8)
        assert L.or_pack_int4(O.ptr(vals), vals.size, O.ptr(packed), 1, C.byref(err)) == O.OUT_OF_RANGE
        assert err.byte == kat["byte"]
    elif op in ("dequantize_error", "device_dequantize_error"):
        packed = np.array(kat["packed"], dtype=np.uint8)
        out_len = kat.get("out_len", kat["value_count"])
        out = np.zeros(max(out_len, 1), dtype=np.float32)
        st = L.or_dequantize_int4(O.ptr(packed), packed.size, kat["value_count"], kat["scale"], kat["zero_point"],
                                  O.ptr(out), out_len, C.byref(err))
        if kat["error"] == "InvalidParams":
            assert st == O.INVALID_PARAMS
        else:
            assert st == O.LENGTH_MISMATCH
            assert (err.argument.decode(), err.expected, err.actual) == (kat["argument"], kat["expected"], kat["actual"])
    else:
        raise AssertionError(op)


def test_int4_quantize_rounds_half_away_from_zero():
    # f32::round semantics (quantize.rs:198): 0.5 -> 1 and, with zp=8, -0.5 -> 8-1.
    vals = np.array([0.5, 1.5, 2.5, -0.5, -1.5], dtype=np.float32)
    packed = np.zeros(3, dtype=np.uint8)
    err = O.OrError()
    assert O.lib().or_quantize_int4(O.ptr(vals), 5, 1.0, 8, O.ptr(packed), 3, C.byref(err)) == O.OK
    codes = [(b >> s) & 15 for b in packed.tolist() for s in (0, 4)][:5]
    # v/s + zp = 8.5, 9.5, 10.5, 7.5, 6.5 -> half away from zero
    assert codes == [9, 10, 11, 8, 7]


# --------------------------------------------------------------------------
# G0 (gemm.rs KATs + closed form)
@pytest.mark.parametrize("kat", KATS["gemm"], ids=lambda k: k["src"].split("/")[-1])
def test_gemm_reference_kats(kat):
    st, out, _ = O.gemm_f32(kat["lhs"], kat["rhs"], kat["m"], kat["k"], kat["n"])
    assert st == O.OK
    assert_close(out, kat["out"], kat["tol"])


@pytest.mark.parametrize("kat", KATS["gemm_errors"], ids=lambda k: k["src"].split("/")[-1])
def test_gemm_reference_error_kats(kat):
    k = (1 << 64) - 1 if kat["k"] == "usize::MAX" else kat["k"]
    lhs = np.zeros(max(kat["lhs_len"], 1), dtype=np.float32)
    rhs = np.zeros(max(kat["rhs_len"], 1), dtype=np.float32)
    out = np.zeros(max(kat["out_len"], 1), dtype=np.float32)
    err = O.OrError()
    st = O.lib().or_gemm_f32(O.ptr(lhs), kat["lhs_len"], O.ptr(rhs), kat["rhs_len"], kat["m"], k, kat["n"],
                             O.ptr(out), kat["out_len"], C.byref(err))
    if kat["error"] == "InvalidShape":
        assert st == O.INVALID_SHAPE
    else:
        assert st == O.LENGTH_MISMATCH
        assert (err.argument.decode(), err.expected, err.actual) == (kat["argument"], kat["expected"], kat["actual"])


def test_gemm_pattern_matches_float64_closed_form():
    kat = KATS["gemm_pattern"][0]
    m, k, n = kat["m"], kat["k"], kat["n"]
    lhs = np.array([((i % 11) - 5) * 0.25 for i in range(m * k)], dtype=np.float32)
    rhs = np.array([((i % 7) - 3) * 0.5 for i in range(k * n)], dtype=np.float32)
    st, out, _ = O.gemm_f32(lhs, rhs, m, k, n)
    assert st == O.OK
    # every product and partial sum is a small dyadic rational: float64 is exact
    ref = (lhs.astype(np.float64).reshape(m, k) @ rhs.astype(np.float64).reshape(k, n)).astype(np.float32)
    assert np.array_equal(out.reshape(m, n), ref)


def test_gemm_f64_accumulation_differs_from_f32_accumulation():
    # gemm.rs:464-471 catches f32 accumulation; here a case where f32 accumulation
    # would lose the small term entirely while f64 keeps it.
    lhs = np.array([1.0, 1.0, 1.0], dtype=np.float32)
    rhs = np.array([2.0 ** 24, 1.0, 1.0], dtype=np.float32)
    st, out, _ = O.gemm_f32(lhs, rhs, 1, 3, 1)
    assert st == O.OK and out[0] == np.float32(2.0 ** 24 + 2.0)


def test_gemm_random_matches_float64_reference_rounded_once():
    rng = np.random.default_rng(7)
    m, k, n = 5, 37, 9
    lhs = rng.standard_normal(m * k).astype(np.float32)
    rhs = rng.standard_normal(k * n).astype(np.float32)
    st, out, _ = O.gemm_f32(lhs, rhs, m, k, n)
    ref = lhs.astype(np.float64).reshape(m, k) @ rhs.astype(np.float64).reshape(k, n)
    # f64 sums in a different order agree to ~1e-15 relative before the f32 rounding
    assert np.allclose(out.reshape(m, n), ref, rtol=1e-6, atol=1e-6)
    # a transposed operand would not agree
    assert not np.allclose(out.reshape(m, n), lhs.reshape(m, k) @ rhs.reshape(n, k).T, rtol=1e-3)


def test_gemm_col_range_pieces_equal_the_whole_gemm():
    """The multi-core CPU baseline's column ranges: disjoint ranges over the
    one shared [K][N] matrix write exactly or_gemm_f32's output (every bit),
    and a range writes nothing outside itself."""
    rng = np.random.default_rng(11)
    m, k, n = 3, 53, 41
    lhs = rng.standard_normal(m * k).astype(np.float32)
    rhs = rng.standard_normal(k * n).astype(np.float32)
    st, whole, _ = O.gemm_f32(lhs, rhs, m, k, n)
    assert st == O.OK
    out = np.full(m * n, np.nan, dtype=np.float32)
    for c0, c1 in ((0, 7), (7, 8), (8, 30), (30, 41)):
        O.gemm_f32_col_range(lhs, rhs, m, k, n, c0, c1, out)
    assert np.array_equal(out.view(np.uint32), whole.view(np.uint32))
    part = np.full(m * n, np.nan, dtype=np.float32)
    O.gemm_f32_col_range(lhs, rhs, m, k, n, 8, 30, part)
    p = part.reshape(m, n)
    assert np.all(np.isnan(p[:, :8])) and np.all(np.isnan(p[:, 30:]))
    assert np.array_equal(p[:, 8:30].view(np.uint32), whole.reshape(m, n)[:, 8:30].view(np.uint32))


# --------------------------------------------------------------------------
# bf16 and the synthetic generator
def test_bf16_round_to_nearest_even():
    L = O.lib()
    cases = {
        0x3F800000: 0x3F80,  # 1.0
        0x3F808000: 0x3F80,  # tie, even stays
        0x3F818000: 0x3F82,  # tie, odd rounds up
        0x3F808001: 0x3F81,  # above tie
        0x80000000: 0x8000,  # -0
        0x7F800000: 0x7F80,  # inf
        0x7F7FFFFF: 0x7F80,  # overflow to inf
        0xC0490FDB: 0xC049,  # -pi
    }
    for bits, want in cases.items():
        x = struct.unpack("<f", struct.pack("<I", bits))[0]
        assert L.or_f32_to_bf16(x) == want, hex(bits)
    nan = L.or_f32_to_bf16(float("nan"))
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0
    for b in (0x3F80, 0xC049, 0x0001, 0x7F7F):
        assert O.bf16_to_f32(np.array([b], dtype=np.uint16))[0] == struct.unpack("<f", struct.pack("<I", b << 16))[0]


def test_splitmix64_known_first_outputs():
    L = O.lib()
    L.or_splitmix64_next.restype = C.c_uint64
    L.or_splitmix64_next.argtypes = [C.POINTER(C.c_uint64)]
    state = C.c_uint64(0)
    # published first outputs of splitmix64 seeded with 0
    assert L.or_splitmix64_next(C.byref(state)) == 0xE220A8397B1DCDAF
    assert L.or_splitmix64_next(C.byref(state)) == 0x6E789E6AA1B965F4


def test_normal_generator_moments_and_determinism():
    a = O.normal_f32(0, 200_001, 0.0, 0.02)
    b = O.normal_f32(0, 200_001, 0.0, 0.02)
    assert np.array_equal(a, b)
    assert abs(a.mean()) < 3 * 0.02 / math.sqrt(a.size)
    assert abs(a.std() - 0.02) < 0.0005
    c = O.normal_f32(1, 10)
    assert not np.array_equal(c, O.normal_f32(2, 10))


# --------------------------------------------------------------------------
# Q1/Q2/Q3 spec invariants
def test_quantize_rows_invariants_on_random_rows():
    x = O.normal_f32(0, 64 * 300, 0.0, 0.02).reshape(64, 300)
    st, q, s, _ = O.quantize_rows_f32(x)
    assert st == O.OK
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    amax = np.abs(x).max(axis=1)
    assert np.array_equal(s, (amax / np.float32(127.0)).astype(np.float32))
    # the absmax element maps to +-127
    arg = np.abs(x).argmax(axis=1)
    assert np.all(np.abs(q[np.arange(64), arg].astype(np.int32)) == 127)
    # half-step error bound (plus one f32 rounding of the quotient)
    deq = O.dequantize_i8(q, s)
    assert np.all(np.abs(deq - x) <= 0.5 * s[:, None] * (1 + 1e-5) + 1e-12)
    # sign preserved for non-tiny values
    big = np.abs(x) > s[:, None]
    assert np.all(np.sign(q[big]) == np.sign(x[big]))


def test_quantize_rows_tie_rounds_half_away_from_zero():
    # amax 127 -> s = 1 exactly, so v/s = v: 2.5 -> 3, -2.5 -> -3, 0.5 -> 1, -0.5 -> -1
    x = np.array([[127.0, 2.5, -2.5, 0.5, -0.5, 1.49999988, -126.5]], dtype=np.float32)
    st, q, s, _ = O.quantize_rows_f32(x)
    assert st == O.OK and s[0] == 1.0
    assert q[0].tolist() == [127, 3, -3, 1, -1, 1, -127]


def test_quantize_rows_zero_and_underflow_rows():
    tiny = np.float32(1e-45)  # smallest subnormal; tiny/127 underflows to 0
    x = np.array([[0.0, 0.0, -0.0], [tiny, 0.0, -tiny]], dtype=np.float32)
    st, q, s, _ = O.quantize_rows_f32(x)
    assert st == O.OK
    assert s.tolist() == [0.0, 0.0]
    assert q.tolist() == [[0, 0, 0], [0, 0, 0]]


def test_quantize_rows_reports_first_non_finite_in_row_major_order():
    x = np.ones((3, 4), dtype=np.float32)
    x[2, 1] = np.inf
    x[1, 3] = np.nan
    st, _, _, err = O.quantize_rows_f32(x)
    assert st == O.NON_FINITE_INPUT and err.index == 7 and math.isnan(err.value)


def test_quantize_rows_bf16_widens_exactly():
    x = O.normal_f32(3, 8 * 64).reshape(8, 64)
    xb = O.to_bf16(x)
    st1, q1, s1, _ = O.quantize_rows_bf16(xb)
    st2, q2, s2, _ = O.quantize_rows_f32(O.bf16_to_f32(xb).reshape(8, 64))
    assert st1 == st2 == O.OK
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)


def test_quantize_rows_matches_textbook_python_formula():
    # independent restatement with Python floats rounded to f32 at each step
    x = O.normal_f32(11, 4 * 50).reshape(4, 50)
    st, q, s, _ = O.quantize_rows_f32(x)

    def r32(v):
        return struct.unpack("<f", struct.pack("<f", v))[0]

    for r in range(4):
        amax = max(abs(float(v)) for v in x[r])
        sc = r32(amax / 127.0)
        assert sc == float(s[r])
        for c in range(50):
            quo = r32(float(x[r, c]) / sc)
            code = math.floor(abs(quo) + 0.5) * (1 if quo >= 0 else -1)
            assert max(-127, min(127, code)) == int(q[r, c])


# --------------------------------------------------------------------------
# G1/G3 (W8A8): brute force + epilogue KAT
def test_gemm_i8_i32_matches_int64_brute_force():
    rng = np.random.default_rng(1)
    xq = rng.integers(-127, 128, size=(7, 129), dtype=np.int8)
    wq = rng.integers(-127, 128, size=(11, 129), dtype=np.int8)
    acc = O.gemm_i8_i32(xq, wq)
    assert np.array_equal(acc, xq.astype(np.int64) @ wq.astype(np.int64).T)


def test_gemm_i8_i32_extreme_accumulator():
    k = 21504  # largest K in the configs: 21504 * 127^2 < 2^31
    xq = np.full((1, k), -127, dtype=np.int8)
    wq = np.full((2, k), 127, dtype=np.int8)
    wq[1] = -127
    acc = O.gemm_i8_i32(xq, wq)
    assert acc.tolist() == [[-k * 127 * 127, k * 127 * 127]]


def test_epilogue_hand_computed():
    acc = np.array([[100, -3], [0, 7]], dtype=np.int32)
    sx = np.array([0.5, 2.0], dtype=np.float32)
    sw = np.array([0.25, 2.0], dtype=np.float32)
    bias = np.array([1.0, 0.0], dtype=np.float32)
    out = O.epilogue(acc, sx, sw, bias=bias)
    assert out.tolist() == [[13.5, -3.0], [1.0, 28.0]]
    r2 = O.epilogue(acc, sx, sw, bias=bias, relu2=True)
    assert r2.tolist() == [[182.25, 0.0], [1.0, 784.0]]
    bf = O.epilogue(acc, sx, sw, bias=bias, out_bf16=True)
    assert O.bf16_to_f32(bf).reshape(2, 2).tolist() == [[13.5, -3.0], [1.0, 28.0]]


def test_epilogue_multiplies_in_two_rounded_steps():
    # ((float)acc * sx) * sw, not (float)acc * (sx * sw)
    acc = np.array([[3]], dtype=np.int32)
    sx = np.array([np.float32(1.0) / np.float32(3.0)], dtype=np.float32)
    sw = np.array([np.float32(0.1)], dtype=np.float32)
    out = O.epilogue(acc, sx, sw)[0, 0]
    two_step = np.float32(np.float32(np.float32(3.0) * sx[0]) * sw[0])
    assert out == two_step


# --------------------------------------------------------------------------
# G2: W8A32 dequant GEMV == G0 on the materialised weights
def test_gemv_w8a32_equals_reference_gemm_on_materialised_weights():
    k, n = 96, 40
    w = O.normal_f32(0, n * k, 0.0, 0.02).reshape(n, k)
    x = O.normal_f32(1, 2 * k).reshape(2, k)
    st, q, s, _ = O.quantize_rows_f32(w)
    y = O.gemv_w8a32(x, q, s)
    w_mat = (q.astype(np.float32) * s[:, None]).T.copy()  # [K, N] reference layout (linear.rs:324)
    st, ref, _ = O.gemm_f32(x, w_mat, 2, k, n)
    assert np.array_equal(y.ravel(), ref)


# --------------------------------------------------------------------------
# Sigmoid / routing (moe_routing.rs KATs + brute force)
def test_sigmoid_matches_float64_closed_form():
    for x in np.linspace(-30, 30, 2001, dtype=np.float32):
        s = O.sigmoid(x)
        ref = 1.0 / (1.0 + math.exp(-float(x)))
        assert abs(s - ref) <= 2.5e-7 * max(ref, 1e-30) + 1e-40


@pytest.mark.parametrize("kat", KATS["routing_sigmoid"], ids=lambda k: k["src"].split("/")[-1])
def test_routing_sigmoid_reference_kats(kat):
    st, idx, w, _ = O.route_sigmoid(kat["scores"], kat["tokens"], kat["experts"], kat["top_k"])
    assert st == O.OK
    if kat["indices"] == "host":
        ref_idx, ref_w = brute_force_sigmoid_topk(kat["scores"], kat["tokens"], kat["experts"], kat["top_k"])
        assert idx.tolist() == ref_idx
        assert_close(w, ref_w, 0.0)
    else:
        assert idx.tolist() == kat["indices"]
        assert_close(w, kat["weights"], kat["tol"])


def brute_force_sigmoid_topk(scores, tokens, experts, top_k):
    idx, w = [], []
    for t in range(tokens):
        sig = [O.sigmoid(scores[t * experts + e]) for e in range(experts)]
        order = sorted(range(experts), key=lambda e: (-sig[e], e))[:top_k]
        idx += order
        w += [sig[e] for e in order]
    return idx, w


def test_routing_sigmoid_pattern_has_ties_and_matches_brute_force():
    kat = KATS["routing_pattern"][0]
    t_, e_, k_ = kat["tokens"], kat["experts"], kat["top_k"]
    scores = np.array([((e % 17) - 8.0) * 0.375 + t * 0.125 - 0.05 for t in range(t_) for e in range(e_)],
                      dtype=np.float32)
    st, idx, w, _ = O.route_sigmoid(scores, t_, e_, k_)
    ref_idx, ref_w = brute_force_sigmoid_topk(scores.tolist(), t_, e_, k_)
    assert idx.tolist() == ref_idx and w.tolist() == ref_w
    # the pattern repeats every 17 experts: the top-6 are ties broken toward lower index
    assert idx[:6].tolist() == [16, 33, 50, 67, 84, 101]


def test_routing_sigmoid_random_matches_brute_force():
    scores = O.normal_f32(2, 9 * 128)
    st, idx, w, _ = O.route_sigmoid(scores, 9, 128, 6)
    ref_idx, ref_w = brute_force_sigmoid_topk(scores.tolist(), 9, 128, 6)
    assert idx.tolist() == ref_idx and w.tolist() == ref_w


def test_routing_sigmoid_renormalised_weights_sum_to_one():
    scores = O.normal_f32(2, 16 * 128)
    st, idx, raw, _ = O.route_sigmoid(scores, 16, 128, 6)
    st, idx2, w, _ = O.route_sigmoid(scores, 16, 128, 6, renormalize=True)
    assert np.array_equal(idx, idx2)
    w = w.reshape(16, 6)
    raw = raw.reshape(16, 6)
    assert np.allclose(w.sum(axis=1), 1.0, atol=1e-6)
    for t in range(16):
        tot = np.float32(0.0)
        for j in range(6):
            tot = np.float32(tot + raw[t, j])
        assert np.array_equal(w[t], (raw[t] / tot).astype(np.float32))
    st, _, ws, _ = O.route_sigmoid(scores, 16, 128, 6, renormalize=True, scaling=2.5)
    assert np.array_equal(ws.reshape(16, 6), (w * np.float32(2.5)).astype(np.float32))


@pytest.mark.parametrize("kat", KATS["routing_softmax"], ids=lambda k: k["src"].split("/")[-1])
def test_routing_softmax_reference_kats(kat):
    st, idx, w, _ = O.route_softmax(kat["scores"], kat["tokens"], kat["experts"], kat["top_k"])
    assert st == O.OK
    if kat["indices"] == "host":
        # brute force with float64 softmax: same ranking, weights within f32 noise
        s = np.array(kat["scores"], dtype=np.float64).reshape(kat["tokens"], kat["experts"])
        for t in range(kat["tokens"]):
            p = np.exp(s[t] - s[t].max())
            p /= p.sum()
            order = sorted(range(kat["experts"]), key=lambda e: (-p[e], e))[: kat["top_k"]]
            assert idx[t * kat["top_k"]:(t + 1) * kat["top_k"]].tolist() == order
            sel = p[order] / p[order].sum()
            assert_close(w[t * kat["top_k"]:(t + 1) * kat["top_k"]], sel, 1e-6)
    else:
        assert idx.tolist() == kat["indices"]
        assert_close(w, kat["weights"], kat["tol"])


@pytest.mark.parametrize("kat", KATS["routing_errors"], ids=lambda k: k["src"].split("/")[-1])
def test_routing_reference_error_kats(kat):
    scores = np.zeros(max(kat["scores_len"], 1), dtype=np.float32)
    st, _, _, err = O.route_sigmoid(scores, kat["tokens"], kat["experts"], kat["top_k"],
                                    indices_len=kat["indices_len"], weights_len=kat["weights_len"],
                                    scores_len=kat["scores_len"])
    if kat["error"] == "InvalidShape":
        assert st == O.INVALID_SHAPE
    else:
        assert st == O.LENGTH_MISMATCH
        assert (err.argument.decode(), err.expected, err.actual) == (kat["argument"], kat["expected"], kat["actual"])


# --------------------------------------------------------------------------
# R2 permutation (spec) against numpy's stable argsort
def test_permute_matches_stable_argsort_and_invariants():
    rng = np.random.default_rng(5)
    tokens, k, experts = 37, 6, 16
    idx = np.stack([rng.choice(experts, size=k, replace=False) for _ in range(tokens)]).astype(np.int32).ravel()
    offsets, perm, pos = O.moe_permute(idx, tokens, k, experts)
    counts = np.bincount(idx, minlength=experts)
    assert offsets.tolist() == [0] + np.cumsum(counts).tolist()
    assert np.array_equal(perm, np.argsort(idx, kind="stable"))
    assert np.array_equal(pos[perm], np.arange(tokens * k))
    assert sorted(perm.tolist()) == list(range(tokens * k))


def test_permute_empty_experts_and_single_route():
    offsets, perm, pos = O.moe_permute(np.array([3], dtype=np.int32), 1, 1, 5)
    assert offsets.tolist() == [0, 0, 0, 0, 1, 1] and perm.tolist() == [0] and pos.tolist() == [0]


# --------------------------------------------------------------------------
# R3 grouped GEMM: per-expert dense brute force
def test_grouped_gemm_matches_dense_per_expert_brute_force():
    rng = np.random.default_rng(9)
    tokens, k_top, experts, hidden, inter = 13, 2, 5, 64, 24
    idx = np.stack([rng.choice(experts, size=k_top, replace=False) for _ in range(tokens)]).astype(np.int32).ravel()
    offsets, perm, pos = O.moe_permute(idx, tokens, k_top, experts)
    xq = rng.integers(-127, 128, size=(tokens, hidden), dtype=np.int8)
    sx = rng.uniform(0.001, 0.01, size=tokens).astype(np.float32)
    w = rng.integers(-127, 128, size=(experts, inter, hidden), dtype=np.int8)
    sw = rng.uniform(0.0001, 0.001, size=(experts, inter)).astype(np.float32)
    out = O.moe_grouped(xq, sx, True, k_top, offsets, perm, w, sw, relu2=True)
    for r in range(tokens * k_top):
        t, e = r // k_top, idx[r]
        acc = xq[t].astype(np.int64) @ w[e].astype(np.int64).T
        y = (acc.astype(np.float32) * sx[t]).astype(np.float32) * sw[e]
        y = np.maximum(y, np.float32(0)) ** 2
        assert np.array_equal(out[pos[r]], y.astype(np.float32))


def test_combine_hand_computed_and_identity():
    slot = np.array([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], dtype=np.float32)
    pos = np.array([2, 0, 1], dtype=np.int32)
    w = np.array([0.5, 0.25, 1.0], dtype=np.float32)
    out = O.moe_combine(slot, pos, w, tokens=1, top_k=3, hidden=2)
    assert out.tolist() == [[0.5 * 5 + 0.25 * 1 + 3.0, 0.5 * 6 + 0.25 * 2 + 4.0]]
    ident = O.moe_combine(slot, np.array([1, 2, 0], dtype=np.int32), np.ones(3, dtype=np.float32), 3, 1, 2)
    assert np.array_equal(ident, slot[[1, 2, 0]])


# --------------------------------------------------------------------------
# L1/L2/MoE layer KATs (linear.rs, mlp.rs, moe.rs)
@pytest.mark.parametrize("kat", KATS["linear"], ids=lambda k: k["src"].split("/")[-1])
def test_linear_reference_kats(kat):
    inp = np.array(kat["input"], dtype=np.float32)
    w = np.array(kat["weights"], dtype=np.float32)
    b = None if kat["bias"] is None else np.array(kat["bias"], dtype=np.float32)
    out = np.full(kat["rows"] * kat["out_dim"], -1.0, dtype=np.float32)
    err = O.OrError()
    st = O.lib().or_linear_project(O.ptr(inp), inp.size, kat["rows"], O.ptr(w), kat["in_dim"], kat["out_dim"],
                                   O.ptr(b), O.ptr(out), out.size, C.byref(err))
    assert st == O.OK
    assert_close(out, kat["out"], kat["tol"])


@pytest.mark.parametrize("kat", KATS["linear_errors"], ids=lambda k: k["src"].split("/")[-1])
def test_linear_reference_error_kats(kat):
    z = np.zeros(8, dtype=np.float32)
    err = O.OrError()
    st = O.lib().or_linear_project(O.ptr(z), kat.get("input_len", 0), kat.get("rows", 1), O.ptr(z), kat["in_dim"],
                                   kat["out_dim"], None, O.ptr(z), kat.get("out_len", 0), C.byref(err))
    want = {"InvalidShape": O.INVALID_SHAPE, "InvalidRowCount": O.INVALID_ROW_COUNT,
            "LengthMismatch": O.LENGTH_MISMATCH}[kat["error"]]
    assert st == want
    if want == O.LENGTH_MISMATCH:
        assert (err.argument.decode(), err.expected, err.actual) == (kat["argument"], kat["expected"], kat["actual"])


@pytest.mark.parametrize("kat", KATS["mlp"], ids=lambda k: k["src"].split("/")[-1])
def test_mlp_reference_kats(kat):
    f = lambda v: None if v is None else np.array(v, dtype=np.float32)
    inp, wu, bu, wd, bd = (f(kat[key]) for key in ("input", "w_up", "b_up", "w_down", "b_down"))
    out = np.full(kat["rows"] * kat["hidden"], -1.0, dtype=np.float32)
    st = O.lib().or_mlp_forward(O.ptr(inp), kat["rows"], kat["hidden"], kat["inter"], O.ptr(wu), O.ptr(bu),
                                O.ptr(wd), O.ptr(bd), O.ptr(out))
    assert st == O.OK
    assert_close(out, kat["out"], kat["tol"])


@pytest.mark.parametrize("kat", KATS["moe"], ids=lambda k: k["src"].split("/")[-1])
def test_moe_layer_reference_kats(kat):
    E = kat["experts"]
    ups = [np.array([1.0], dtype=np.float32) for _ in range(E)]
    downs = [np.array([s], dtype=np.float32) for s in kat["expert_scales"]]
    up_ptrs = (C.c_void_p * E)(*[O.ptr(a) for a in ups])
    down_ptrs = (C.c_void_p * E)(*[O.ptr(a) for a in downs])
    shared_up = np.array([1.0], dtype=np.float32) if kat["shared_scale"] is not None else None
    shared_down = np.array([kat["shared_scale"]], dtype=np.float32) if kat["shared_scale"] is not None else None
    inp = np.array(kat["input"], dtype=np.float32)
    rw = np.array(kat["router_w"], dtype=np.float32)
    rb = np.array(kat["router_b"], dtype=np.float32)
    out = np.full(kat["rows"] * kat["hidden"], -1.0, dtype=np.float32)
    st = O.lib().or_moe_forward_dense(O.ptr(inp), kat["rows"], kat["hidden"], E, kat["top_k"], O.ptr(rw), O.ptr(rb),
                                      1, up_ptrs, down_ptrs, None, None, 1, O.ptr(shared_up), O.ptr(shared_down),
                                      None, None, O.ptr(out))
    assert st == O.OK
    assert_close(out, kat["out"], kat["tol"])


# --------------------------------------------------------------------------
# Full int8 MoE composition: equal to its parts and to the dense reference
# semantics where quantization is lossless.
def test_moe_forward_w8a8_composes_its_parts():
    tokens, hidden, inter, experts, top_k = 12, 64, 32, 8, 3
    x = O.to_bf16(O.normal_f32(1, tokens * hidden)).reshape(tokens, hidden)
    logits = O.normal_f32(2, tokens * experts)
    wu = O.normal_f32(3, experts * inter * hidden, 0, 0.02).reshape(experts * inter, hidden)
    wd = O.normal_f32(4, experts * hidden * inter, 0, 0.02).reshape(experts * hidden, inter)
    _, qu, su, _ = O.quantize_rows_f32(wu)
    _, qd, sd, _ = O.quantize_rows_f32(wd)
    qu = qu.reshape(experts, inter, hidden)
    qd = qd.reshape(experts, hidden, inter)
    su = su.reshape(experts, inter)
    sd = sd.reshape(experts, hidden)
    st, out, idx, w, offsets, perm, pos = O.moe_forward_w8a8(x, logits, qu, su, qd, sd, top_k)
    assert st == O.OK
    _, xq, sx, _ = O.quantize_rows_bf16(x)
    _, idx2, w2, _ = O.route_sigmoid(logits, tokens, experts, top_k, renormalize=True)
    assert np.array_equal(idx, idx2) and np.array_equal(w, w2)
    off2, perm2, pos2 = O.moe_permute(idx, tokens, top_k, experts)
    assert np.array_equal(offsets, off2) and np.array_equal(perm, perm2) and np.array_equal(pos, pos2)
    h = O.moe_grouped(xq, sx, True, top_k, offsets, perm, qu, su, relu2=True)
    _, hq, sh, _ = O.quantize_rows_f32(h)
    d = O.moe_grouped(hq, sh, False, top_k, offsets, perm, qd, sd, relu2=False)
    ref = O.moe_combine(d, pos, w, tokens, top_k, hidden, out_bf16=True)
    assert np.array_equal(out, ref)


def test_moe_int8_pipeline_equals_dense_reference_when_lossless():
    # Integer-valued activations/weights with absmax 127 per row quantize
    # losslessly (scale 1), so the int8 pipeline must reproduce the reference
    # MoE layer (moe.rs:154-249) with raw sigmoid weights, up to bf16 output.
    rng = np.random.default_rng(3)
    tokens, hidden, inter, experts, top_k = 4, 8, 4, 4, 2
    x = rng.integers(-3, 4, size=(tokens, hidden)).astype(np.float32)
    x[:, 0] = 127.0
    wu = rng.integers(-2, 3, size=(experts, inter, hidden)).astype(np.float32)
    wu[:, :, 1] = 127.0
    logits = O.normal_f32(5, tokens * experts)
    # relu2 output must also quantize losslessly: too strong an assumption in
    # general, so compare only the up projection + routing here and the
    # combine via an identity down projection on lossless inputs.
    _, qu, su, _ = O.quantize_rows_f32(wu.reshape(-1, hidden))
    assert np.all(su == 1.0)
    _, xq, sx, _ = O.quantize_rows_bf16(O.to_bf16(x))
    assert np.all(sx == 1.0) and np.array_equal(xq.astype(np.float32), x)
    st, idx, w, _ = O.route_sigmoid(logits, tokens, experts, top_k)
    offsets, perm, pos = O.moe_permute(idx, tokens, top_k, experts)
    h = O.moe_grouped(xq, sx, True, top_k, offsets, perm, qu.reshape(experts, inter, hidden),
                      su.reshape(experts, inter), relu2=True)
    for r in range(tokens * top_k):
        t, e = r // top_k, idx[r]
        dense = np.maximum(x[t] @ wu[e].T, 0) ** 2
        assert np.array_equal(h[pos[r]], dense.astype(np.float32))


# --------------------------------------------------------------------------
# Shared expert (moe.rs:195-244): the output row starts at 0.0, the shared
# expert's row is added first, then each route's weighted output in route
# order.  The values make the order visible in f32: shared first gives
# (1e8 - 1e8) + 3 = 3; the routes first would give (-1e8 + 3) + 1e8 = 0
# (f32 spacing at 1e8 is 8).
def test_moe_combine_shared_adds_the_shared_row_first():
    slot_out = np.array([[-1e8], [3.0]], dtype=np.float32)
    pos = np.array([0, 1], dtype=np.int32)
    w = np.array([1.0, 1.0], dtype=np.float32)
    shared = np.array([[1e8]], dtype=np.float32)
    assert O.moe_combine_shared(slot_out, pos, w, shared, 1, 2, 1)[0, 0] == 3.0
    # without the shared row: exactly or_moe_combine (0 + (-1e8) + 3 = -1e8 in f32)
    no_sh = O.moe_combine_shared(slot_out, pos, w, None, 1, 2, 1)
    assert np.array_equal(no_sh, O.moe_combine(slot_out, pos, w, 1, 2, 1))
    assert no_sh[0, 0] == np.float32(-1e8)
    # 0.0 + (-0.0) = +0.0: the output starts at +0.0 as output.fill(0.0) does
    z = O.moe_combine_shared(np.zeros((1, 1), np.float32), np.zeros(1, np.int32), np.zeros(1, np.float32),
                             np.array([[-0.0]], dtype=np.float32), 1, 1, 1)
    assert np.signbit(z[0, 0]) == False  # noqa: E712


def test_moe_combine_shared_matches_the_dense_reference_layer_kat():
    # moe.rs:417-435 (pinned through or_moe_forward_dense above): 0.5*4 +
    # 0.880797*8 + 0.7310586*12 with the shared row first
    kat = [k for k in KATS["moe"] if k["shared_scale"] is not None][0]
    x = kat["input"][0]
    shared = np.array([[kat["shared_scale"] * max(x, 0.0) ** 2]], dtype=np.float32)
    scores = np.array([O.sigmoid(b) for b in kat["router_b"]], dtype=np.float32)
    order = sorted(range(kat["experts"]), key=lambda e: (-scores[e], e))[:kat["top_k"]]
    slot_out = np.array([[kat["expert_scales"][e] * x * x] for e in order], dtype=np.float32)
    w = scores[order]
    got = O.moe_combine_shared(slot_out, np.arange(len(order), dtype=np.int32), w, shared, 1, len(order), 1)
    assert_close(got.ravel(), kat["out"], kat["tol"])


def test_mlp_w8a8_composes_its_parts():
    rows, hidden, inter = 9, 96, 40
    x = O.to_bf16(O.normal_f32(7, rows * hidden)).reshape(rows, hidden)
    _, wu, su, _ = O.quantize_rows_f32(O.normal_f32(8, inter * hidden, 0, 0.02).reshape(inter, hidden))
    _, wd, sd, _ = O.quantize_rows_f32(O.normal_f32(9, hidden * inter, 0, 0.02).reshape(hidden, inter))
    st, out = O.mlp_w8a8(x, wu, su, wd, sd)
    assert st == O.OK
    _, xq, sx, _ = O.quantize_rows_bf16(x)
    h = O.epilogue(O.gemm_i8_i32(xq, wu), sx, su, relu2=True)
    _, hq, sh, _ = O.quantize_rows_f32(h)
    assert np.array_equal(out, O.linear_w8a8(hq, sh, wd, sd))


def test_moe_forward_shared_composes_its_parts():
    tokens, hidden, inter, experts, top_k, sh_inter = 12, 64, 32, 8, 3, 48
    x = O.to_bf16(O.normal_f32(1, tokens * hidden)).reshape(tokens, hidden)
    logits = O.normal_f32(2, tokens * experts)
    _, qu, su, _ = O.quantize_rows_f32(O.normal_f32(3, experts * inter * hidden, 0, 0.02).reshape(-1, hidden))
    _, qd, sd, _ = O.quantize_rows_f32(O.normal_f32(4, experts * hidden * inter, 0, 0.02).reshape(-1, inter))
    _, hu, hsu, _ = O.quantize_rows_f32(O.normal_f32(5, sh_inter * hidden, 0, 0.02).reshape(sh_inter, hidden))
    _, hd, hsd, _ = O.quantize_rows_f32(O.normal_f32(6, hidden * sh_inter, 0, 0.02).reshape(hidden, sh_inter))
    qu, su = qu.reshape(experts, inter, hidden), su.reshape(experts, inter)
    qd, sd = qd.reshape(experts, hidden, inter), sd.reshape(experts, hidden)
    st, out, idx, w, offsets, perm, pos = O.moe_forward_shared_w8a8(x, logits, qu, su, qd, sd, top_k, hu, hsu, hd, hsd)
    assert st == O.OK
    st0, out0, idx0, w0, off0, perm0, pos0 = O.moe_forward_w8a8(x, logits, qu, su, qd, sd, top_k)
    assert np.array_equal(idx, idx0) and np.array_equal(w, w0) and np.array_equal(pos, pos0)
    _, xq, sx, _ = O.quantize_rows_bf16(x)
    h = O.moe_grouped(xq, sx, True, top_k, offsets, perm, qu, su, relu2=True)
    _, hq, sh, _ = O.quantize_rows_f32(h)
    d = O.moe_grouped(hq, sh, False, top_k, offsets, perm, qd, sd, relu2=False)
    _, shared = O.mlp_w8a8(x, hu, hsu, hd, hsd)
    assert np.array_equal(out, O.moe_combine_shared(d, pos, w, shared, tokens, top_k, hidden, out_bf16=True))
    assert not np.array_equal(out, out0)  # the shared expert contributes


# --------------------------------------------------------------------------
# Expert biases.  The reference's experts and shared expert are MlpLayers
# with optional biases (mlp.rs:79-96, moe.rs:60-65): up bias before ReLU^2,
# down bias on the expert's own output, i.e. before the combine weight
# (mlp.rs:201-208).  or_mlp_forward's bias handling is pinned by the
# mlp.rs:347-363 KAT above.
def _mlp_dense(x, wu, bu, wd, bd):
    rows, hidden = x.shape
    inter = wu.shape[1]
    out = np.zeros(rows * hidden, dtype=np.float32)
    st = O.lib().or_mlp_forward(O.ptr(np.ascontiguousarray(x)), rows, hidden, inter, O.ptr(wu), O.ptr(bu),
                                O.ptr(wd), O.ptr(bd), O.ptr(out))
    assert st == O.OK
    return out.reshape(rows, hidden)


def test_moe_dense_reference_with_biases_composes_its_biased_mlps():
    """or_moe_forward_dense with expert and shared biases: output 0, + the
    shared expert's biased MLP, + w * the selected expert's biased MLP in route
    order (moe.rs:195-244), each MLP the KAT-pinned or_mlp_forward."""
    rng = np.random.default_rng(21)
    rows, hidden, inter, E, top_k, sh_inter = 3, 5, 4, 4, 2, 3
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    rw = rng.standard_normal((hidden, E)).astype(np.float32)
    rb = rng.standard_normal(E).astype(np.float32)
    wu = [rng.standard_normal((hidden, inter)).astype(np.float32) for _ in range(E)]
    wd = [rng.standard_normal((inter, hidden)).astype(np.float32) for _ in range(E)]
    bu = [rng.standard_normal(inter).astype(np.float32) for _ in range(E)]
    bd = [rng.standard_normal(hidden).astype(np.float32) for _ in range(E)]
    shu, shd = rng.standard_normal((hidden, sh_inter)).astype(np.float32), rng.standard_normal((sh_inter, hidden)).astype(np.float32)
    shbu, shbd = rng.standard_normal(sh_inter).astype(np.float32), rng.standard_normal(hidden).astype(np.float32)
    arr = lambda lst: (C.c_void_p * E)(*[O.ptr(a) for a in lst])
    out = np.full(rows * hidden, -1.0, dtype=np.float32)
    st = O.lib().or_moe_forward_dense(O.ptr(x), rows, hidden, E, top_k, O.ptr(rw), O.ptr(rb), inter, arr(wu), arr(wd),
                                      arr(bu), arr(bd), sh_inter, O.ptr(shu), O.ptr(shd), O.ptr(shbu), O.ptr(shbd),
                                      O.ptr(out))
    assert st == O.OK
    scores = np.zeros(rows * E, dtype=np.float32)
    err = O.OrError()
    assert O.lib().or_linear_project(O.ptr(x), x.size, rows, O.ptr(rw), hidden, E, O.ptr(rb), O.ptr(scores),
                                     scores.size, C.byref(err)) == O.OK
    st, idx, w, _ = O.route_sigmoid(scores, rows, E, top_k)
    shared = _mlp_dense(x, shu, shbu, shd, shbd)
    experts = [_mlp_dense(x, wu[e], bu[e], wd[e], bd[e]) for e in range(E)]
    want = np.zeros((rows, hidden), dtype=np.float32)
    for t in range(rows):
        v = np.float32(0.0) + shared[t]
        for j in range(top_k):
            v = v + np.float32(w[t * top_k + j]) * experts[idx[t * top_k + j]][t]
        want[t] = v
    assert np.array_equal(out.reshape(rows, hidden), want)
    # the biases matter: without them the layer differs
    out0 = np.full(rows * hidden, -1.0, dtype=np.float32)
    O.lib().or_moe_forward_dense(O.ptr(x), rows, hidden, E, top_k, O.ptr(rw), O.ptr(rb), inter, arr(wu), arr(wd),
                                 None, None, sh_inter, O.ptr(shu), O.ptr(shd), None, None, O.ptr(out0))
    assert not np.allclose(out0, out, atol=1e-3)


def _biased_moe_case(seed=31):
    tokens, hidden, inter, experts, top_k, sh_inter = 12, 64, 32, 8, 3, 48
    rng = np.random.default_rng(seed)
    x = O.to_bf16(O.normal_f32(1, tokens * hidden)).reshape(tokens, hidden)
    logits = O.normal_f32(2, tokens * experts)
    _, qu, su, _ = O.quantize_rows_f32(O.normal_f32(3, experts * inter * hidden, 0, 0.02).reshape(-1, hidden))
    _, qd, sd, _ = O.quantize_rows_f32(O.normal_f32(4, experts * hidden * inter, 0, 0.02).reshape(-1, inter))
    _, hu, hsu, _ = O.quantize_rows_f32(O.normal_f32(5, sh_inter * hidden, 0, 0.02).reshape(sh_inter, hidden))
    _, hd, hsd, _ = O.quantize_rows_f32(O.normal_f32(6, hidden * sh_inter, 0, 0.02).reshape(hidden, sh_inter))
    qu, su = qu.reshape(experts, inter, hidden), su.reshape(experts, inter)
    qd, sd = qd.reshape(experts, hidden, inter), sd.reshape(experts, hidden)
    biases = (rng.standard_normal((experts, inter)).astype(np.float32) * 0.5,
              rng.standard_normal((experts, hidden)).astype(np.float32),
              rng.standard_normal(sh_inter).astype(np.float32) * 0.5,
              rng.standard_normal(hidden).astype(np.float32))
    return tokens, hidden, top_k, x, logits, qu, su, qd, sd, hu, hsu, hd, hsd, biases


def test_moe_int8_biases_compose_their_parts():
    """or_moe_forward_shared_w8a8 with all four biases = R3 with the up bias
    (before ReLU^2), Q2, R3 with the down bias, the biased shared MLP, the
    combine; each bias changes the output."""
    tokens, hidden, top_k, x, logits, qu, su, qd, sd, hu, hsu, hd, hsd, b = _biased_moe_case()
    st, out, idx, w, offsets, perm, pos = O.moe_forward_shared_w8a8(x, logits, qu, su, qd, sd, top_k, hu, hsu, hd,
                                                                    hsd, biases=b)
    assert st == O.OK
    _, xq, sx, _ = O.quantize_rows_bf16(x)
    h = O.moe_grouped(xq, sx, True, top_k, offsets, perm, qu, su, relu2=True, bias=b[0])
    _, hq, sh, _ = O.quantize_rows_f32(h)
    d = O.moe_grouped(hq, sh, False, top_k, offsets, perm, qd, sd, relu2=False, bias=b[1])
    _, shared = O.mlp_w8a8(x, hu, hsu, hd, hsd, b_up=b[2], b_down=b[3])
    assert np.array_equal(out, O.moe_combine_shared(d, pos, w, shared, tokens, top_k, hidden, out_bf16=True))
    for i in range(4):
        partial = tuple(v if j != i else None for j, v in enumerate(b))
        _, o2, *_ = O.moe_forward_shared_w8a8(x, logits, qu, su, qd, sd, top_k, hu, hsu, hd, hsd, biases=partial)
        assert not np.array_equal(o2, out), f"bias {i} has no effect"


def test_moe_int8_down_bias_is_weighted_by_the_route():
    """Down bias on the expert's own output, before the combine weight
    (mlp.rs:208 inside the expert, moe.rs:239-244 after it): with raw
    (un-renormalised) sigmoid weights and a different constant bias per
    expert, the layer moves by sum_j w_j b[e_j], not by the unweighted sum."""
    tokens, hidden, top_k, x, logits, qu, su, qd, sd, hu, hsu, hd, hsd, _ = _biased_moe_case()
    experts = qu.shape[0]
    bd = np.repeat(np.arange(1, experts + 1, dtype=np.float32)[:, None] * 4.0, hidden, axis=1)
    none = (None, None, None, None)
    st, o0, idx, w, *_ = O.moe_forward_shared_w8a8(x, logits, qu, su, qd, sd, top_k, None, None, None, None,
                                                   renormalize=False, biases=none)
    st1, o1, *_ = O.moe_forward_shared_w8a8(x, logits, qu, su, qd, sd, top_k, None, None, None, None,
                                           renormalize=False, biases=(None, bd, None, None))
    assert st == st1 == O.OK
    shift = O.bf16_to_f32(o1).astype(np.float64) - O.bf16_to_f32(o0).astype(np.float64)
    want = np.array([sum(w[t * top_k + j] * bd[idx[t * top_k + j], 0] for j in range(top_k)) for t in range(tokens)])
    unweighted = np.array([sum(bd[idx[t * top_k + j], 0] for j in range(top_k)) for t in range(tokens)])
    tol = 2.0 ** -7 * (np.abs(O.bf16_to_f32(o1)).max() + 1.0)  # two bf16 roundings
    assert np.all(np.abs(shift - want[:, None]) <= tol)
    assert np.all(np.abs(shift - unweighted[:, None]).max(axis=1) > tol)


def test_moe_int8_up_bias_lossless_equals_dense_reference():
    """On lossless inputs (integer rows with absmax 127, scale 1) the up
    projection with an integer bias is exactly relu2(x W_e^T + b_e) of the
    reference's expert (mlp.rs:201-205): the bias before ReLU^2, per expert."""
    rng = np.random.default_rng(5)
    tokens, hidden, inter, experts, top_k = 4, 8, 4, 4, 2
    x = rng.integers(-3, 4, size=(tokens, hidden)).astype(np.float32)
    x[:, 0] = 127.0
    wu = rng.integers(-2, 3, size=(experts, inter, hidden)).astype(np.float32)
    wu[:, :, 1] = 127.0
    bu = rng.integers(-300, 301, size=(experts, inter)).astype(np.float32)
    logits = O.normal_f32(5, tokens * experts)
    _, qu, su, _ = O.quantize_rows_f32(wu.reshape(-1, hidden))
    _, xq, sx, _ = O.quantize_rows_bf16(O.to_bf16(x))
    assert np.all(su == 1.0) and np.all(sx == 1.0)
    st, idx, w, _ = O.route_sigmoid(logits, tokens, experts, top_k)
    offsets, perm, pos = O.moe_permute(idx, tokens, top_k, experts)
    h = O.moe_grouped(xq, sx, True, top_k, offsets, perm, qu.reshape(experts, inter, hidden),
                      su.reshape(experts, inter), relu2=True, bias=bu)
    for r in range(tokens * top_k):
        t, e = r // top_k, idx[r]
        dense = np.maximum(x[t] @ wu[e].T + bu[e], 0) ** 2
        assert np.array_equal(h[pos[r]], dense.astype(np.float32))
    assert np.any(h == 0.0)  # some biased outputs went negative before ReLU^2


# --------------------------------------------------------------------------
# W4A8: the reference's INT4 linear weights (packed [K][N] affine codes) with
# per-token int8 activations.
def _int4_codes(packed, k, n):
    flat = np.empty(packed.size * 2, dtype=np.int64)
    flat[0::2], flat[1::2] = packed & 15, packed >> 4
    return flat[:k * n].reshape(k, n)


def test_linear_w4a8_reference_int4_layer_kat():
    # linear.rs:493-502: params (0.5, 8), values [0.5, 1.0, -0.5, 0.0] as a
    # 2 x 2 [input][output] layer materialise to the same values; projected
    # on the lossless row x = [127, -3] (scale 1): [127*0.5 + 3*0.5, 127*1.0]
    st, packed, _ = O.quantize_int4(np.array([0.5, 1.0, -0.5, 0.0], dtype=np.float32), 0.5, 8)
    assert st == O.OK
    st, dense, _ = O.dequantize_int4(packed, 4, 0.5, 8)
    assert st == O.OK and np.array_equal(dense, np.array([0.5, 1.0, -0.5, 0.0], dtype=np.float32))
    x = O.to_bf16(np.array([[127.0, -3.0]], dtype=np.float32))
    st, y = O.linear_w4a8(x, packed, 2, 0.5, 8)
    assert st == O.OK
    assert np.array_equal(y, np.array([[65.0, 127.0]], dtype=np.float32))


def test_linear_w4a8_equals_reference_dense_path_when_lossless():
    # Integer activations with a 127 in every row quantize with scale 1; a
    # power-of-two weight scale makes every (code - zp) * s exact, and the
    # sums are exact in f64: then W4A8 must equal materialize_dense +
    # gemm_into_host + bias (linear.rs:126-131, 325-339) to the bit.
    rng = np.random.default_rng(4)
    m, k, n, zp, scale = 3, 96, 40, 6, 2.0 ** -6
    packed = rng.integers(0, 256, size=k * n // 2, dtype=np.uint8)
    x = rng.integers(-100, 101, size=(m, k)).astype(np.float32)
    x[:, 5] = 127.0
    bias = rng.integers(-8, 9, size=n).astype(np.float32)
    st, y = O.linear_w4a8(O.to_bf16(x), packed, n, scale, zp, bias=bias)
    assert st == O.OK
    st, dense, _ = O.dequantize_int4(packed, k * n, scale, zp)
    assert st == O.OK
    ref = np.zeros(m * n, dtype=np.float32)
    st = O.lib().or_linear_project(O.ptr(x), m * k, m, O.ptr(dense), k, n, O.ptr(bias), O.ptr(ref), m * n, None)
    assert st == O.OK
    assert np.array_equal(y.ravel(), ref)


def test_linear_w4a8_brute_force():
    rng = np.random.default_rng(5)
    m, k, n, zp, scale = 4, 200, 33, 11, 0.0173
    packed = rng.integers(0, 256, size=(k * n + 1) // 2, dtype=np.uint8)
    x = O.to_bf16(O.normal_f32(6, m * k)).reshape(m, k)
    st, y = O.linear_w4a8(x, packed, n, scale, zp)
    assert st == O.OK
    _, xq, sx, _ = O.quantize_rows_bf16(x)
    acc = xq.astype(np.int64) @ (_int4_codes(packed, k, n) - zp)  # [m][n]
    assert np.abs(acc).max() < 2 ** 31
    ref = (acc.astype(np.float32) * sx[:, None]).astype(np.float32) * np.float32(scale)
    assert np.array_equal(y, ref.astype(np.float32))
