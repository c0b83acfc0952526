"""Exact int8 x int8 -> int32 accumulators through float64 BLAS, for checking
the device at the BASELINE.json configs' full sizes in seconds.

Every product of two int8 codes is an integer of magnitude <= 127^2, and every
partial sum of K of them stays below K * 127^2 < 2^53 for K < 5.5e11, so each
float64 addition BLAS performs, in whatever order and blocking, is exact: the
float64 result is the integer sum, identical to the oracle's int32 loop
(or_gemm_i8_i32) whenever that fits in int32, which the device envelope
guarantees (K <= 131072).  tests/test_exact_int.py pins these helpers against
the oracle on random and extreme inputs; the epilogues and the MoE stages other
than the accumulation are the oracle's own functions.
"""
import numpy as np

import oracle_ctypes as O


def gemm_i8_exact(xq, wq):
    """acc[m][n] = sum_k xq[m][k] * wq[n][k] (int32), via an exact float64 matmul."""
    a = np.asarray(xq, dtype=np.int8).astype(np.float64)
    b = np.asarray(wq, dtype=np.int8).astype(np.float64)
    acc = a @ b.T
    assert np.all(np.abs(acc) < 2.0 ** 31)
    return acc.astype(np.int32)


def linear_w8a8_exact(xq, sx, wq, sw, bias=None, relu2=False, out_bf16=False):
    """The oracle's W8A8 linear (or_linear_w8a8) with the accumulators from gemm_i8_exact."""
    return O.epilogue(gemm_i8_exact(xq, wq), sx, sw, bias=bias, relu2=relu2, out_bf16=out_bf16)


def moe_grouped_exact(aq, sa, gather_tokens, top_k, offsets, perm, w, sw, relu2):
    """or_moe_grouped_w8a8 with exact BLAS accumulators: the rows of slot
    segment e (token perm[s] / top_k when gathering, slot s otherwise) times
    expert e's weights, the oracle's epilogue."""
    experts, n, _ = w.shape
    routes = int(offsets[-1])
    out = np.zeros((routes, n), dtype=np.float32)
    for e in range(experts):
        s0, s1 = int(offsets[e]), int(offsets[e + 1])
        if s0 == s1:
            continue
        rows = np.asarray(perm[s0:s1]) // top_k if gather_tokens else np.arange(s0, s1)
        out[s0:s1] = O.epilogue(gemm_i8_exact(aq[rows], w[e]), sa[rows], sw[e], relu2=relu2)
    return out


def moe_forward_exact(x_bf16, logits, w_up, s_up, w_down, s_down, top_k, renormalize=True, scaling=1.0):
    """or_moe_forward_w8a8's composition (Q2 -> R1 -> R2 -> up, ReLU^2 -> Q2 ->
    down -> R4), each stage the oracle's, the expert accumulations exact
    through BLAS.  Returns (out bf16, idx, w, offsets, perm, pos, h, d)."""
    tokens, _ = x_bf16.shape
    experts = w_up.shape[0]
    st, xq, sx, _ = O.quantize_rows_bf16(x_bf16)
    assert st == O.OK
    st, idx, w, _ = O.route_sigmoid(logits, tokens, experts, top_k, renormalize=renormalize, scaling=scaling)
    assert st == O.OK
    offsets, perm, pos = O.moe_permute(idx, tokens, top_k, experts)
    h = moe_grouped_exact(xq, sx, True, top_k, offsets, perm, w_up, s_up, relu2=True)
    st, hq, sh, _ = O.quantize_rows_f32(h)
    assert st == O.OK
    d = moe_grouped_exact(hq, sh, False, top_k, offsets, perm, w_down, s_down, relu2=False)
    out = O.moe_combine(d, pos, w, tokens, top_k, x_bf16.shape[1], out_bf16=True)
    return out, idx, w, offsets, perm, pos, h, d
