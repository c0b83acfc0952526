"""Pins tests/exact_int.py (the exact float64-BLAS accumulators used by the
full-size GPU parity tests) against the oracle's own integer loops, so a
full-size comparison is a comparison with the oracle."""
import numpy as np

import oracle_ctypes as O
from exact_int import gemm_i8_exact, linear_w8a8_exact, moe_forward_exact, moe_grouped_exact


def test_gemm_exact_equals_oracle_random():
    rng = np.random.default_rng(5)
    for m, n, k in [(7, 11, 129), (33, 65, 4096), (3, 5, 21504)]:
        xq = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
        wq = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        assert np.array_equal(gemm_i8_exact(xq, wq), O.gemm_i8_i32(xq, wq))


def test_gemm_exact_extreme_accumulators():
    # the largest |acc| the device envelope allows: K = 131072 codes of +-127
    k = 131072
    xq = np.full((2, k), 127, dtype=np.int8)
    xq[1] = -127
    wq = np.full((2, k), 127, dtype=np.int8)
    wq[1, ::2] = -127
    got = gemm_i8_exact(xq, wq)
    assert np.array_equal(got, O.gemm_i8_i32(xq, wq))
    assert got[0, 0] == k * 127 * 127 and got[1, 0] == -k * 127 * 127 and got[0, 1] == 0


def test_linear_exact_equals_oracle_linear():
    rng = np.random.default_rng(6)
    xq = rng.integers(-127, 128, size=(9, 1000), dtype=np.int8)
    wq = rng.integers(-127, 128, size=(40, 1000), dtype=np.int8)
    sx = rng.uniform(1e-3, 1e-1, size=9).astype(np.float32)
    sw = rng.uniform(1e-4, 1e-2, size=40).astype(np.float32)
    bias = rng.standard_normal(40).astype(np.float32)
    for bf in (False, True):
        assert np.array_equal(linear_w8a8_exact(xq, sx, wq, sw, bias=bias, out_bf16=bf),
                              O.linear_w8a8(xq, sx, wq, sw, bias=bias, out_bf16=bf))


def test_moe_exact_equals_oracle_composition():
    for tokens, hidden, inter, experts, top_k in [(12, 64, 32, 8, 3), (96, 128, 64, 16, 6)]:
        x = O.to_bf16(O.normal_f32(1, tokens * hidden)).reshape(tokens, hidden)
        logits = O.normal_f32(2, tokens * experts)
        wu = O.normal_f32(3, experts * inter * hidden, 0, 0.02).reshape(experts * inter, hidden)
        wd = O.normal_f32(4, experts * hidden * inter, 0, 0.02).reshape(experts * hidden, inter)
        _, qu, su, _ = O.quantize_rows_f32(wu)
        _, qd, sd, _ = O.quantize_rows_f32(wd)
        qu, su = qu.reshape(experts, inter, hidden), su.reshape(experts, inter)
        qd, sd = qd.reshape(experts, hidden, inter), sd.reshape(experts, hidden)
        st, out, idx, w, offsets, perm, pos = O.moe_forward_w8a8(x, logits, qu, su, qd, sd, top_k)
        assert st == O.OK
        got = moe_forward_exact(x, logits, qu, su, qd, sd, top_k)
        for a, b in zip(got[:6], (out, idx, w, offsets, perm, pos)):
            assert np.array_equal(a, b)
        # the stages themselves against the oracle's grouped GEMM
        _, xq, sx, _ = O.quantize_rows_bf16(x)
        assert np.array_equal(got[6], O.moe_grouped(xq, sx, True, top_k, offsets, perm, qu, su, relu2=True))
        h = got[6]
        _, hq, sh, _ = O.quantize_rows_f32(h)
        assert np.array_equal(got[7], moe_grouped_exact(hq, sh, False, top_k, offsets, perm, qd, sd, False))
        assert np.array_equal(got[7], O.moe_grouped(hq, sh, False, top_k, offsets, perm, qd, sd, relu2=False))
