"""Parity of the gfx950 path with the CPU oracle, through the C ABI.

Bar: int8 codes, scales, int32 accumulators,
routing indices and permutations bit-exact; float outputs bit-exact where the
arithmetic is the same sequence of IEEE operations (the W8A8 epilogue,
combine), and within max_i |y-r| / max(|r_i|, 1e-6 max|r|) <= 1e-3 (f32) /
1e-2 (bf16) where the summation order differs (W8A32).
Inputs: the seeded generator (splitmix64 + Box-Muller), W ~ N(0, 0.02) seed 0,
activations ~ N(0, 1) seed 1, router logits seed 2, expert e seed 100 + e.
"""
import ctypes
import functools
import json
import os
import sys

import numpy as np
import pytest

import nemotron_hip as NH
import oracle_ctypes as O
from exact_int import linear_w8a8_exact, moe_forward_exact, moe_grouped_exact
from tiling import tile_16x64, tile_experts

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = NH.Context(0)
    yield c
    c.close()


def rel_err(y, r):
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    floor = 1e-6 * np.max(np.abs(r)) if r.size else 0.0
    return float(np.max(np.abs(y - r) / np.maximum(np.abs(r), floor))) if r.size else 0.0


@functools.lru_cache(maxsize=8)
def quantized_weights(n, k, seed=0):
    w = O.normal_f32(seed, n * k, 0.0, 0.02).reshape(n, k)
    st, q, s, _ = O.quantize_rows_f32(w)
    assert st == O.OK
    return w, q, s


def activations_bf16(m, k, seed=1):
    return O.to_bf16(O.normal_f32(seed, m * k)).reshape(m, k)


# ---- Q1/Q2/Q3 ----------------------------------------------------------------
@pytest.mark.parametrize("rows,cols,dtype", [(1, 4096, "bf16"), (16, 8192, "bf16"), (3072, 1856, "f32"),
                                             (4096, 4096, "f32"), (7, 33, "f32"), (5, 1, "bf16"),
                                             (3, 21504, "f32"), (2, 40000, "bf16"), (4, 12, "f32"),
                                             # past the 8192 chunks the 1024-thread kernel holds in registers
                                             (2, 70000, "bf16")])
def test_quantize_rows_bit_exact(ctx, rows, cols, dtype):
    note(f"quantize_rows {rows}x{cols} {dtype}")
    x = O.normal_f32(5, rows * cols, 0.0, 0.02 if dtype == "f32" else 1.0).reshape(rows, cols)
    if dtype == "bf16":
        xb = O.to_bf16(x)
        st, q_ref, s_ref, _ = O.quantize_rows_bf16(xb)
        dx, dt = ctx.upload(xb), NH.BF16
    else:
        st, q_ref, s_ref, _ = O.quantize_rows_f32(x)
        dx, dt = ctx.upload(x), NH.F32
    dq = ctx.empty((rows, cols), np.int8)
    ds = ctx.empty(rows, np.float32)
    dstat = ctx.empty(rows, np.int32)
    NH.call("nh_quantize_rows_i8", ctx.handle, dx.ptr, dt, rows, cols, dq.ptr, ds.ptr, dstat.ptr, None)
    ctx.synchronize()
    assert np.array_equal(dq.numpy(), q_ref)
    assert np.array_equal(ds.numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.all(dstat.numpy() == -1)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_quantize_rows_unaligned_rows_take_the_scalar_path(ctx, dtype):
    """Rows that start off a 16-byte boundary (x offset by one element) give
    the same codes as aligned ones."""
    rows, cols = 6, 520
    note(f"quantize_rows unaligned {dtype}")
    x = O.normal_f32(9, rows * cols + 1).astype(np.float32)
    if dtype == "bf16":
        xs = O.to_bf16(x)
        st, q_ref, s_ref, _ = O.quantize_rows_bf16(xs[1:].reshape(rows, cols))
        dx, dt, esz = ctx.upload(xs), NH.BF16, 2
    else:
        xs = x
        st, q_ref, s_ref, _ = O.quantize_rows_f32(xs[1:].reshape(rows, cols))
        dx, dt, esz = ctx.upload(xs), NH.F32, 4
    dq = ctx.empty((rows, cols), np.int8)
    ds = ctx.empty(rows, np.float32)
    NH.call("nh_quantize_rows_i8", ctx.handle, dx.offset(esz), dt, rows, cols, dq.ptr, ds.ptr, None, None)
    ctx.synchronize()
    assert np.array_equal(dq.numpy(), q_ref)
    assert np.array_equal(ds.numpy().view(np.uint32), s_ref.view(np.uint32))


def test_quantize_rows_special_rows(ctx):
    note("quantize_rows special rows")
    tiny = np.float32(1e-45)
    x = np.zeros((5, 64), dtype=np.float32)
    x[1, :7] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.49999988, -126.5]  # ties, s = 1
    x[2, :3] = [tiny, 0.0, -tiny]                               # underflowed scale
    x[3] = np.linspace(-3e-39, 3e-39, 64, dtype=np.float32)     # subnormal row
    x[4] = 1.0
    x[4, 9] = np.nan
    x[4, 20] = np.inf
    st, q_ref, s_ref, err = O.quantize_rows_f32(x[:4])
    dx = ctx.upload(x)
    dq = ctx.empty((5, 64), np.int8)
    ds = ctx.empty(5, np.float32)
    dstat = ctx.empty(5, np.int32)
    NH.call("nh_quantize_rows_i8", ctx.handle, dx.ptr, NH.F32, 5, 64, dq.ptr, ds.ptr, dstat.ptr, None)
    ctx.synchronize()
    assert np.array_equal(dq.numpy()[:4], q_ref)
    assert np.array_equal(ds.numpy()[:4].view(np.uint32), s_ref.view(np.uint32))
    assert dstat.numpy().tolist() == [-1, -1, -1, -1, 9]


@pytest.mark.parametrize("cols,dtype", [(2688, "bf16"), (1856, "f32"), (4096, "bf16"), (2048, "f32"), (8, "bf16"),
                                        (4, "f32"),
                                        # whole rows of 1025..2816 chunks in a workgroup's registers
                                        (21504, "bf16"), (8200, "bf16"), (22528, "bf16"), (11264, "f32")])
def test_quantize_many_rows_bit_exact(ctx, cols, dtype):
    """1100 rows: the one-wave-per-row quantizer (rows of up to 512 16-byte
    chunks, 1024 rows or more) and the whole-row workgroup quantizer (rows of
    1025..2816 chunks), with tie, tiny, subnormal and non-finite rows among
    them."""
    rows = 1100
    note(f"quantize_rows many {rows}x{cols} {dtype}")
    x = O.normal_f32(11, rows * cols, 0.0, 0.02 if dtype == "f32" else 1.0).reshape(rows, cols)
    n = min(cols, 7)
    x[3, :n] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.49999988, -126.5][:n]
    x[3, n:] = 0.0
    x[500, :] = 0.0
    x[500, 0] = np.float32(1e-45)
    x[700] = np.linspace(-3e-39, 3e-39, cols, dtype=np.float32)
    x[1099, :] = 1.0
    x[1099, cols // 2] = np.nan
    x[1099, cols - 1] = np.inf
    if dtype == "bf16":
        xs = O.to_bf16(x)
        st, q_ref, s_ref, _ = O.quantize_rows_bf16(xs[:rows - 1])
        dx, dt = ctx.upload(xs), NH.BF16
    else:
        st, q_ref, s_ref, _ = O.quantize_rows_f32(x[:rows - 1])
        dx, dt = ctx.upload(x), NH.F32
    dq = ctx.empty((rows, cols), np.int8)
    ds = ctx.empty(rows, np.float32)
    dstat = ctx.empty(rows, np.int32)
    NH.call("nh_quantize_rows_i8", ctx.handle, dx.ptr, dt, rows, cols, dq.ptr, ds.ptr, dstat.ptr, None)
    ctx.synchronize()
    assert np.array_equal(dq.numpy()[:rows - 1], q_ref)
    assert np.array_equal(ds.numpy()[:rows - 1].view(np.uint32), s_ref.view(np.uint32))
    stat = dstat.numpy()
    assert np.all(stat[:rows - 1] == -1) and stat[rows - 1] == cols // 2


@pytest.mark.parametrize("rows,cols,shift", [(256, 1024, 0), (37, 100, 0), (7, 30, 0), (5, 48, 1)],
                         ids=["chunks", "chunks-100", "ragged-cols", "unaligned-codes"])
def test_dequantize_i8_bit_exact(ctx, rows, cols, shift):
    """4-code chunks (cols % 4 == 0, codes 4-byte and output 16-byte aligned)
    and the per-code path (ragged columns, or codes one byte into their
    allocation)."""
    note(f"dequantize_i8 {rows}x{cols} shift={shift}")
    _, q, s = quantized_weights(rows, cols)
    dq, ds = ctx.upload(np.concatenate([np.zeros(shift, np.int8), q.ravel()])), ctx.upload(s)
    out = ctx.empty(q.shape, np.float32)
    NH.call("nh_dequantize_i8", ctx.handle, dq.ptr + shift, ds.ptr, rows, cols, out.ptr, None)
    ctx.synchronize()
    assert np.array_equal(out.numpy(), O.dequantize_i8(q, s))


# ---- Q0d --------------------------------------------------------------------
@pytest.mark.parametrize("packed,count,scale,zp", [([0x76, 0x98, 0x0A], 5, 0.5, 8), ([0x76, 0x98], 4, 0.5, 8),
                                                   (None, 1_000_003, 0.037, 3), (None, 64, 0.25, 0),
                                                   (None, 33, 1.5, 15), (None, 3, 2.0, 1)])
def test_dequantize_int4_matches_host_reference(ctx, packed, count, scale, zp):
    note(f"dequantize_int4 n={count}")
    if packed is None:
        rng = np.random.default_rng(0)
        packed = rng.integers(0, 256, size=(count + 1) // 2, dtype=np.uint8)
    packed = np.array(packed, dtype=np.uint8)
    ref = np.zeros(count, dtype=np.float32)
    err = O.OrError()
    assert O.lib().or_dequantize_int4(O.ptr(packed), packed.size, count, scale, zp, O.ptr(ref), count,
                                      O.C.byref(err)) == O.OK
    dp = ctx.upload(packed)
    out = ctx.empty(count, np.float32)
    NH.call("nh_dequantize_int4", ctx.handle, dp.ptr, packed.size, count, scale, zp, out.ptr, count, None)
    ctx.synchronize()
    assert np.array_equal(out.numpy(), ref)  # reference tolerance 1e-6 (quantize.rs:585-617); exact here


# ---- tiled weight layout -----------------------------------------------------------
@pytest.mark.parametrize("n,k", [(1, 1), (33, 96), (17, 200), (4096, 4096), (20, 4112)])
def test_tile_weights_on_device_matches_layout(ctx, n, k):
    note(f"tile_weights n={n} k={k}")
    wq = np.random.default_rng(n + k).integers(-127, 128, size=(n, k), dtype=np.int8)
    dwq = ctx.upload(wq)
    t = NH.tile_weights(ctx, dwq, n, k)
    ctx.synchronize()
    assert np.array_equal(t.numpy(), tile_16x64(wq))


# ---- G0d: f32 device GEMM (f64 accumulation, the host order) ----------------------
def _gemm_f32_case(kat):
    m, k, n = kat["m"], kat["k"], kat["n"]
    if kat.get("lhs") is None:
        lhs = np.array([((i % 11) - 5) * 0.25 for i in range(m * k)], dtype=np.float32)
        rhs = np.array([((i % 7) - 3) * 0.5 for i in range(k * n)], dtype=np.float32)
    else:
        lhs = np.array(kat["lhs"], dtype=np.float32)
        rhs = np.array(kat["rhs"], dtype=np.float32)
    return m, k, n, lhs, rhs


_GEMM_KATS = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                         "reference_kats.json")))


@pytest.mark.parametrize("case", _GEMM_KATS["gemm"] + [dict(_GEMM_KATS["gemm_pattern"][0], lhs=None)]
                         + [dict(m=m, k=k, n=n, lhs="rand") for (m, k, n) in
                            [(1, 4096, 4096), (37, 100, 65), (130, 257, 71), (64, 16, 64), (3, 1, 5),
                             (512, 2688, 128), (5, 130, 200), (1024, 300, 1030),
                             # the f64 matrix-core path (16 x 16 tiles, 128-k chunks): one
                             # partial chunk, a chunk and a 1-k tail, whole chunks, K below
                             # one 4-k step, partial tiles both ways, two chunks and a tail
                             (1, 64, 1), (3, 65, 130), (4, 128, 64), (7, 63, 70), (17, 3, 17),
                             (33, 257, 31), (2, 384, 3),
                             # 64 x 64 tiles filling 256 CUs with a 1-k tail step
                             (1024, 33, 1024)]],
                         ids=lambda c: f"{c['m']}x{c['k']}x{c['n']}")
def test_gemm_f32_device_bit_exact_with_host_order(ctx, case):
    note(f"gemm_f32 {case['m']}x{case['k']}x{case['n']}")
    if case.get("lhs") == "rand":
        m, k, n = case["m"], case["k"], case["n"]
        lhs = O.normal_f32(31, m * k)
        rhs = O.normal_f32(32, k * n, 0.0, 0.02)
    else:
        m, k, n, lhs, rhs = _gemm_f32_case(case)
    _, ref, _ = O.gemm_f32(lhs, rhs, m, k, n)
    dl, dr = ctx.upload(lhs), ctx.upload(rhs)
    out = ctx.empty(m * n, np.float32)
    NH.call("nh_gemm_f32", ctx.handle, dl.ptr, lhs.size, dr.ptr, rhs.size, m, k, n, out.ptr, m * n, None)
    ctx.synchronize()
    got = out.numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    if "out" in case:  # the reference KAT's own expected values (tolerance 1e-6)
        assert np.all(np.abs(got - np.array(case["out"], dtype=np.float32)) <= case["tol"])


def test_gemm_f32_device_signed_zero_and_specials(ctx):
    """Signed zeros, Inf and NaN propagate as on the host (NaN compared by
    position: the host's default NaN is negative, the GPU's positive)."""
    m, k, n = 2, 3, 2
    lhs = np.array([-0.0, -0.0, -0.0, 1.0, np.inf, 2.0], dtype=np.float32)
    rhs = np.array([1.0, 2.0, 3.0, 0.0, -1.0, np.nan], dtype=np.float32)
    _, ref, _ = O.gemm_f32(lhs, rhs, m, k, n)
    dl, dr = ctx.upload(lhs), ctx.upload(rhs)
    out = ctx.empty(m * n, np.float32)
    NH.call("nh_gemm_f32", ctx.handle, dl.ptr, lhs.size, dr.ptr, rhs.size, m, k, n, out.ptr, m * n, None)
    ctx.synchronize()
    got = out.numpy()
    assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.isnan(ref).sum() == 2
    keep = ~np.isnan(ref)
    assert np.array_equal(got[keep].view(np.uint32), ref[keep].view(np.uint32))


# ---- G1: W8A8 GEMV (M <= 16) ----------------------------------------------------
@pytest.mark.parametrize("m,n,k", [(1, 16384, 4096), (4, 16384, 4096), (16, 16384, 4096), (1, 4096, 8192),
                                   (4, 4096, 8192), (16, 4096, 8192), (3, 1000, 80), (16, 20, 4112)])
def test_gemv_w8a8_bit_exact(ctx, m, n, k):
    note(f"gemv_w8a8 m={m} n={n} k={k}")
    _, wq, sw = quantized_weights(n, k)
    x = activations_bf16(m, k)
    _, xq, sx, _ = O.quantize_rows_bf16(x)
    bias = O.normal_f32(7, n, 0.0, 0.1)
    d = {name: ctx.upload(a) for name, a in dict(xq=xq, sx=sx, wq=tile_16x64(wq), sw=sw, bias=bias).items()}
    for out_dt, np_dt, use_bias in ((NH.BF16, np.uint16, False), (NH.F32, np.float32, True)):
        out = ctx.empty((m, n), np_dt)
        NH.call("nh_gemm_w8a8", ctx.handle, d["xq"].ptr, d["sx"].ptr, d["wq"].ptr, d["sw"].ptr,
                d["bias"].ptr if use_bias else None, m, n, k, out.ptr, out_dt, None)
        ctx.synchronize()
        ref = O.linear_w8a8(xq, sx, wq, sw, bias=bias if use_bias else None, out_bf16=(out_dt == NH.BF16))
        got = out.numpy()
        assert np.array_equal(got, ref), f"max diff {np.max(np.abs(got.astype(np.float64) - ref))}"


@pytest.mark.parametrize("m,n,k", [(m, 16384, 4096) for m in (1, 2, 3, 4, 5, 8, 13, 16)] +
                         # configs[1]'s out_proj-like shape: the one-tile decode unit with 8 K waves
                         # (M = 1..4), the two-launch path beyond
                         [(m, 4096, 8192) for m in (1, 2, 4, 8, 16)])
def test_linear_decode_unit_bit_exact(ctx, m, n, k):
    note(f"linear_w8a8 decode m={m} n={n} k={k}")
    _, wq, sw = quantized_weights(n, k)
    x = activations_bf16(m, k, seed=1 + m)
    _, xq_ref, sx_ref, _ = O.quantize_rows_bf16(x)
    ref = O.linear_w8a8(xq_ref, sx_ref, wq, sw, out_bf16=True)
    dwq = ctx.upload(wq)
    dx, dw, ds = ctx.upload(x), NH.tile_weights(ctx, dwq, n, k), ctx.upload(sw)  # the device tiler
    out = ctx.empty((m, n), np.uint16)
    xq = ctx.empty((m, k), np.int8)
    sx = ctx.empty(m, np.float32)
    ws_bytes = NH.lib().nh_linear_w8a8_workspace_size(m, k)
    ws = ctx.empty(max(ws_bytes, 1), np.uint8)
    NH.call("nh_linear_w8a8", ctx.handle, dx.ptr, NH.BF16, dw.ptr, ds.ptr, None, m, n, k, out.ptr, NH.BF16,
            ws.ptr, ws_bytes, xq.ptr, sx.ptr, None, None)
    ctx.synchronize()
    assert np.array_equal(xq.numpy(), xq_ref)
    assert np.array_equal(sx.numpy().view(np.uint32), sx_ref.view(np.uint32))
    assert np.array_equal(out.numpy(), ref)
    # without the optional quantized outputs (workspace path for m > 4)
    out2 = ctx.empty((m, n), np.uint16)
    NH.call("nh_linear_w8a8", ctx.handle, dx.ptr, NH.BF16, dw.ptr, ds.ptr, None, m, n, k, out2.ptr, NH.BF16,
            ws.ptr, ws_bytes, None, None, None, None)
    ctx.synchronize()
    assert np.array_equal(out2.numpy(), ref)


@pytest.mark.parametrize("m,n,k,dtype", [(8, 4096, 21504, "bf16"), (8, 1040, 4112, "bf16"), (5, 528, 4160, "f32"),
                                         (1, 4096, 16384, "bf16"), (16, 96, 64, "f32"), (2, 300, 8192, "f32"),
                                         (3, 4096, 8192, "bf16"), (2, 1000, 4112, "bf16"), (7, 4096, 8192, "bf16"),
                                         (6, 6144, 4096, "bf16"), (17, 300, 4160, "bf16"), (100, 2688, 1856, "f32"),
                                         (257, 1024, 4096, "bf16"),
                                         # the streaming decode unit (5..8 rows): a ragged last N tile
                                         # in runs of 5 and 6 tiles, fewer N tiles than CUs, K = 512
                                         # (most waves past kt), K = 6144 on the 8-tile form, 17 rounds
                                         (8, 21512, 4096, "bf16"), (8, 100, 4096, "bf16"), (5, 4000, 512, "bf16"),
                                         (8, 3000, 6144, "bf16"), (6, 65544, 512, "bf16"),
                                         # the persistent 256 x 224 GEMM with a bias and f32 out
                                         (1000, 14236, 384, "bf16"), (1024, 14336, 256, "f32"),
                                         # batched decode past 16 rows: 64 x 64 tiles (M = 24, 64),
                                         # 64 x 128 (M = 128), 128 x 128 (M = 256), ragged N and K
                                         (24, 16384, 4096, "bf16"), (64, 5000, 1040, "bf16"),
                                         (128, 16390, 512, "bf16"), (256, 16384, 2048, "f32")])
def test_linear_small_m_shapes_bit_exact(ctx, m, n, k, dtype):
    """The linear path off the headline shape (and past 16 rows, the GEMM on
    A tiles written by the quantizer, M and K tails included): several K slabs per
    wave (K = 16384, 21504), a last K tile only partly inside the matrix
    (K = 4112, 4160: the activation tiles hold stale bytes there and meet
    zero weight padding), N not a multiple of 16, f32 activations, the
    one-tile-per-workgroup decode kernels for 2..4 rows (K = 8192 or
    K % 512 != 0) and the streaming one for 5..8 rows (runs of N tiles per
    workgroup, odd and even run lengths, a ragged last tile)."""
    note(f"linear_w8a8 m={m} n={n} k={k} {dtype}")
    _, wq, sw = quantized_weights(n, k)
    bias = O.normal_f32(3, n, 0.0, 0.1)
    if dtype == "bf16":
        x = activations_bf16(m, k, seed=40 + m)
        _, xq_ref, sx_ref, _ = O.quantize_rows_bf16(x)
        dt = NH.BF16
    else:
        x = O.normal_f32(40 + m, m * k).reshape(m, k)
        _, xq_ref, sx_ref, _ = O.quantize_rows_f32(x)
        dt = NH.F32
    ref = linear_w8a8_exact(xq_ref, sx_ref, wq, sw, bias=bias, out_bf16=False)
    dx, dw, ds, db = ctx.upload(x), ctx.upload(tile_16x64(wq)), ctx.upload(sw), ctx.upload(bias)
    ws_bytes = NH.lib().nh_linear_w8a8_workspace_size(m, k)
    ws = ctx.empty(max(ws_bytes, 1), np.uint8)
    ws.fill_bytes(0x5a)  # stale bytes in the activation tiles
    out = ctx.empty((m, n), np.float32)
    xq = ctx.empty((m, k), np.int8)
    sx = ctx.empty(m, np.float32)
    NH.call("nh_linear_w8a8", ctx.handle, dx.ptr, dt, dw.ptr, ds.ptr, db.ptr, m, n, k, out.ptr, NH.F32,
            ws.ptr, ws_bytes, xq.ptr, sx.ptr, None, None)
    ctx.synchronize()
    assert np.array_equal(xq.numpy(), xq_ref)
    assert np.array_equal(sx.numpy().view(np.uint32), sx_ref.view(np.uint32))
    assert np.array_equal(out.numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("n,k", [(6144, 4096), (4096, 4096)], ids=["qkv", "o"])
@pytest.mark.parametrize("out_dtype", ["bf16", "f32"])
@pytest.mark.parametrize("with_bias", [False, True])
def test_linear_decode_stack_attention_shapes(ctx, n, k, out_dtype, with_bias):
    """The decode stack's attention projections at its batch of 8 rows (QKV
    4096 -> 6144 and O 4096 -> 4096): the streaming decode unit's runs over
    384 and 256 N tiles.  bf16 rows in; bf16 and f32 out, with and without a
    bias, against LinearProjection::project_into's order (linear.rs:325-339:
    GEMM, then the bias)."""
    m = 8
    note(f"linear_w8a8 attention m={m} n={n} k={k} out={out_dtype} bias={with_bias}")
    _, wq, sw = quantized_weights(n, k, seed=7)
    bias = O.normal_f32(9, n, 0.0, 0.1) if with_bias else None
    x = activations_bf16(m, k, seed=60)
    _, xq_ref, sx_ref, _ = O.quantize_rows_bf16(x)
    ref = linear_w8a8_exact(xq_ref, sx_ref, wq, sw, bias=bias, out_bf16=out_dtype == "bf16")
    dx, dw, ds = ctx.upload(x), ctx.upload(tile_16x64(wq)), ctx.upload(sw)
    db = ctx.upload(bias) if with_bias else None
    ws_bytes = NH.lib().nh_linear_w8a8_workspace_size(m, k)
    ws = ctx.empty(max(ws_bytes, 1), np.uint8)
    odt = NH.BF16 if out_dtype == "bf16" else NH.F32
    out = ctx.empty((m, n), np.uint16 if out_dtype == "bf16" else np.float32)
    NH.call("nh_linear_w8a8", ctx.handle, dx.ptr, NH.BF16, dw.ptr, ds.ptr, db.ptr if db else None, m, n, k, out.ptr,
            odt, ws.ptr, ws_bytes, None, None, None, None)
    ctx.synchronize()
    got = out.numpy()
    if out_dtype == "bf16":
        assert np.array_equal(got, ref)
    else:
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


# ---- the in-launch handoff (quantizer + tiled-A GEMV as one launch, M <= 16) ------
def handoff_status(ctx):
    timeouts, busy = ctypes.c_uint32(0), ctypes.c_uint32(0)
    NH.call("nh_handoff_status", ctx.handle, ctypes.addressof(timeouts), ctypes.addressof(busy))
    return timeouts.value, busy.value


@pytest.mark.parametrize("m,n,k,out_dtype,with_bias", [(5, 100, 16, "f32", True), (9, 1000, 80, "bf16", False),
                                                       (13, 4096, 528, "f32", False), (16, 4100, 8192, "bf16", True),
                                                       (11, 16, 4112, "bf16", True), (8, 4096, 8192, "f32", True),
                                                       (6, 2000, 4160, "bf16", False), (16, 300, 6144, "f32", True)])
def test_linear_handoff_bit_exact(ctx, m, n, k, out_dtype, with_bias):
    """5..16 bf16 rows that no fused decode unit takes (K % 512 != 0, K past
    4096, or 9..16 rows at K past 4096): the quantizer's workgroups hand the
    rows to the GEMV's workgroups inside one launch.  Codes, scales and
    outputs bit-exact against Q2 and linear.rs:325-339's order; the context's
    handoff slots all back at zero, no wait out of polls."""
    note(f"linear_w8a8 handoff m={m} n={n} k={k} out={out_dtype} bias={with_bias}")
    _, wq, sw = quantized_weights(n, k, seed=11)
    bias = O.normal_f32(13, n, 0.0, 0.1) if with_bias else None
    x = activations_bf16(m, k, seed=80 + m)
    _, xq_ref, sx_ref, _ = O.quantize_rows_bf16(x)
    ref = linear_w8a8_exact(xq_ref, sx_ref, wq, sw, bias=bias, out_bf16=out_dtype == "bf16")
    dx, dw, ds = ctx.upload(x), ctx.upload(tile_16x64(wq)), ctx.upload(sw)
    db = ctx.upload(bias) if with_bias else None
    ws_bytes = NH.lib().nh_linear_w8a8_workspace_size(m, k)
    ws = ctx.empty(max(ws_bytes, 1), np.uint8)
    ws.fill_bytes(0x5a)
    odt = NH.BF16 if out_dtype == "bf16" else NH.F32
    out = ctx.empty((m, n), np.uint16 if out_dtype == "bf16" else np.float32)
    xq, sx = ctx.empty((m, k), np.int8), ctx.empty(m, np.float32)
    NH.call("nh_linear_w8a8", ctx.handle, dx.ptr, NH.BF16, dw.ptr, ds.ptr, db.ptr if db else None, m, n, k, out.ptr,
            odt, ws.ptr, ws_bytes, xq.ptr, sx.ptr, None, None)
    ctx.synchronize()
    assert np.array_equal(xq.numpy(), xq_ref)
    assert np.array_equal(sx.numpy().view(np.uint32), sx_ref.view(np.uint32))
    got = out.numpy()
    assert np.array_equal(got if out_dtype == "bf16" else got.view(np.uint32),
                          ref if out_dtype == "bf16" else ref.view(np.uint32))
    assert handoff_status(ctx) == (0, 0)


def test_linear_handoff_slots_wrap_and_graph_replays(ctx):
    """More handoff launches than the context has counter slots (each slot
    must come back to zero for its next user), each against its own oracle
    result; then three calls captured in a HIP graph, replayed four times with
    eager calls and synchronizations between the replays, every replay
    checked."""
    m, n, k = 8, 512, 1040
    note(f"linear_w8a8 handoff ring m={m} n={n} k={k}")
    _, wq, sw = quantized_weights(n, k, seed=12)
    dw, ds = ctx.upload(tile_16x64(wq)), ctx.upload(sw)
    ws_bytes = NH.lib().nh_linear_w8a8_workspace_size(m, k)
    ws = ctx.empty(ws_bytes, np.uint8)
    xs = [activations_bf16(m, k, seed=500 + i) for i in range(6)]
    refs = []
    for x in xs:
        _, xq_ref, sx_ref, _ = O.quantize_rows_bf16(x)
        refs.append(linear_w8a8_exact(xq_ref, sx_ref, wq, sw, out_bf16=True))
    dxs = [ctx.upload(x) for x in xs]
    out = ctx.empty((m, n), np.uint16)

    def run(i, stream=None):
        NH.call("nh_linear_w8a8", ctx.handle, dxs[i].ptr, NH.BF16, dw.ptr, ds.ptr, None, m, n, k, out.ptr, NH.BF16,
                ws.ptr, ws_bytes, None, None, None, stream)

    for c in range(300):
        run(c % 6)
        ctx.synchronize()
        assert np.array_equal(out.numpy(), refs[c % 6]), f"call {c}"
    assert handoff_status(ctx) == (0, 0)
    stream = ctypes.c_void_p()
    NH.call("nh_stream_create", ctx.handle, ctypes.byref(stream))
    graphs = NH.HipGraphs()
    outs = [ctx.empty((m, n), np.uint16) for _ in range(3)]

    def issue():
        for j in range(3):
            NH.call("nh_linear_w8a8", ctx.handle, dxs[j].ptr, NH.BF16, dw.ptr, ds.ptr, None, m, n, k, outs[j].ptr,
                    NH.BF16, ws.ptr, ws_bytes, None, None, None, stream)

    g, ex = graphs.capture(stream, issue)
    try:
        for rep in range(4):
            for o in outs:
                o.fill_bytes(0)
            ctx.synchronize()
            graphs.launch(ex, stream)
            ctx.synchronize(stream)
            for j in range(3):
                assert np.array_equal(outs[j].numpy(), refs[j]), f"replay {rep}, call {j}"
            run(3 + rep % 3)
            ctx.synchronize()
            assert np.array_equal(out.numpy(), refs[3 + rep % 3])
    finally:
        graphs.destroy(g, ex)
        NH.call("nh_stream_destroy", ctx.handle, stream)
    assert handoff_status(ctx) == (0, 0)


# ---- L2: int8 MLP layer (MlpLayer::forward_into, mlp.rs:157-211) -----------------
def mlp_oracle(x, xdt, w_up, s_up, b_up, w_down, s_down, b_down, out_bf16):
    """Per-token Q2, up projection + bias, ReLU^2 (mlp.rs:205) in f32, Q2 of
    the f32 intermediate, down projection + bias: the oracle's parts."""
    _, xq, sx, _ = O.quantize_rows_bf16(x) if xdt == NH.BF16 else O.quantize_rows_f32(x)
    h = linear_w8a8_exact(xq, sx, w_up, s_up, bias=b_up, relu2=True)
    st, hq, sh, _ = O.quantize_rows_f32(h)
    assert st == O.OK
    return h, linear_w8a8_exact(hq, sh, w_down, s_down, bias=b_down, out_bf16=out_bf16)


@functools.lru_cache(maxsize=2)
def mlp_weights(hidden, inter):
    _, w_up, s_up = quantized_weights(inter, hidden, seed=20)
    _, w_down, s_down = quantized_weights(hidden, inter, seed=21)
    return w_up, s_up, w_down, s_down


@pytest.mark.parametrize("m,hidden,inter,dtype", [(8, 4096, 21504, "bf16"), (1, 4096, 21504, "bf16"),
                                                  (37, 1024, 2560, "bf16"), (5, 512, 1856, "f32"),
                                                  # the streaming up projection's row maxima feeding h's
                                                  # quantizer: a last K tile partly past inter = 1872, one
                                                  # N tile per workgroup
                                                  (6, 512, 1872, "bf16"), (7, 1024, 4096, "bf16"),
                                                  (12, 1024, 2048, "bf16"), (4, 4096, 1024, "bf16"),
                                                  # the up projection (bias, ReLU^2, f32 out) on the persistent GEMM
                                                  (1024, 512, 14336, "bf16"),
                                                  # the MoE layer's shared expert on 64 x 128 tiles
                                                  (512, 2688, 3712, "bf16")])
def test_mlp_bit_exact(ctx, m, hidden, inter, dtype):
    note(f"mlp_w8a8 m={m} hidden={hidden} inter={inter} {dtype}")
    w_up, s_up, w_down, s_down = mlp_weights(hidden, inter)
    b_up = O.normal_f32(22, inter, 0.0, 0.05)
    b_down = O.normal_f32(23, hidden, 0.0, 0.05)
    if dtype == "bf16":
        x, xdt = activations_bf16(m, hidden, seed=24), NH.BF16
    else:
        x, xdt = O.normal_f32(24, m * hidden).reshape(m, hidden), NH.F32
    _, ref = mlp_oracle(x, xdt, w_up, s_up, b_up, w_down, s_down, b_down, out_bf16=True)
    dx, db_up, db_down = ctx.upload(x), ctx.upload(b_up), ctx.upload(b_down)
    dwu, dsu = ctx.upload(tile_16x64(w_up)), ctx.upload(s_up)
    dwd, dsd = ctx.upload(tile_16x64(w_down)), ctx.upload(s_down)
    ws_bytes = NH.lib().nh_mlp_w8a8_workspace_size(m, hidden, inter)
    ws = ctx.empty(ws_bytes, np.uint8)
    out = ctx.empty((m, hidden), np.uint16)
    NH.call("nh_mlp_w8a8", ctx.handle, dx.ptr, xdt, dwu.ptr, dsu.ptr, db_up.ptr, dwd.ptr, dsd.ptr, db_down.ptr,
            m, hidden, inter, out.ptr, NH.BF16, ws.ptr, ws_bytes, None, None)
    ctx.synchronize()
    assert np.array_equal(out.numpy(), ref)


@pytest.mark.parametrize("m", [1, 3, 7])
def test_linear_decode_unit_rounding_ties(ctx, m):
    """Rows whose scale is a power of two carry exact half-integer quotients
    (x/s = j + 0.5): round-half-away-from-zero and round-half-even disagree on
    every one of them, so a fused quantizer that rounds ties the wrong way, or
    skips its exact-division fallback next to a tie, changes codes."""
    n, k = 4096, 4096
    note(f"linear_w8a8 decode rounding ties m={m}")
    _, wq, sw = quantized_weights(n, k)
    rng = np.random.default_rng(11 + m)
    rows = []
    for r in range(m):
        e = (0, -3, 2)[r % 3]
        amax = 127.0 * 2.0 ** e
        row = np.clip(rng.standard_normal(k) * amax / 4, -amax, amax).astype(np.float32)
        ties = np.array([(j + 0.5) * 2.0 ** e for j in range(127)], dtype=np.float32)
        vals = np.concatenate([[amax], ties, -ties])
        cols = rng.permutation(k)[:vals.size]
        row[cols] = vals
        rows.append(row)
    x = O.to_bf16(np.stack(rows))
    _, xq_ref, sx_ref, _ = O.quantize_rows_bf16(x)
    xf = O.bf16_to_f32(x)
    for r in range(m):
        e = (0, -3, 2)[r % 3]
        assert sx_ref[r] == np.float32(2.0 ** e)  # power-of-two scale: every j + 0.5 is an exact tie
        t = xf[r] / sx_ref[r]
        tie = (t - np.floor(t)) == 0.5
        assert tie.sum() >= 254
        assert np.array_equal(xq_ref[r][tie], (np.sign(t[tie]) * np.ceil(np.abs(t[tie]))).astype(np.int8))
    ref = O.linear_w8a8(xq_ref, sx_ref, wq, sw, out_bf16=True)
    dx, dw, ds = ctx.upload(x), ctx.upload(tile_16x64(wq)), ctx.upload(sw)
    out = ctx.empty((m, n), np.uint16)
    xq = ctx.empty((m, k), np.int8)
    sx = ctx.empty(m, np.float32)
    ws_bytes = NH.lib().nh_linear_w8a8_workspace_size(m, k)
    ws = ctx.empty(max(ws_bytes, 1), np.uint8)
    NH.call("nh_linear_w8a8", ctx.handle, dx.ptr, NH.BF16, dw.ptr, ds.ptr, None, m, n, k, out.ptr, NH.BF16,
            ws.ptr, ws_bytes, xq.ptr, sx.ptr, None, None)
    ctx.synchronize()
    assert np.array_equal(sx.numpy().view(np.uint32), sx_ref.view(np.uint32))
    assert np.array_equal(xq.numpy(), xq_ref)
    assert np.array_equal(out.numpy(), ref)


# ---- G2: W8A32 dequant GEMV ------------------------------------
@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (2, 1000, 80), (5, 300, 1040), (3, 64, 20480), (1, 1000, 20480),
                                   (4, 4096, 4096), (8, 333, 8192), (1, 17, 16)])
def test_gemv_w8a32_within_tolerance(ctx, m, n, k):
    note(f"gemv_w8a32 m={m} n={n} k={k}")
    _, wq, sw = quantized_weights(n, k)
    x = O.normal_f32(1, m * k).reshape(m, k)
    ref = O.gemv_w8a32(x, wq, sw)
    dx, dw, ds = ctx.upload(x), ctx.upload(tile_16x64(wq)), ctx.upload(sw)
    y = ctx.empty((m, n), np.float32)
    NH.call("nh_gemv_w8a32", ctx.handle, dx.ptr, dw.ptr, ds.ptr, m, n, k, y.ptr, None)
    ctx.synchronize()
    got = y.numpy()
    assert rel_err(got, ref) <= 1e-3  # north_star f32 tolerance
    # each lane sums the 16 products of a 16-code group in f32 (16 roundings)
    # and the group sums in f64, so |got - exact| <= 16 u sum|x q s| + u |y|
    # to first order; the reference path adds one rounding of q * s per term.
    # A dropped group, a wrong activation lane or a wrong row's scale exceeds
    # this by orders of magnitude.
    w = wq.astype(np.float64) * sw.astype(np.float64)[:, None]
    exact = x.astype(np.float64) @ w.T
    mag = np.abs(x.astype(np.float64)) @ np.abs(w).T
    u = 2.0 ** -24
    assert np.all(np.abs(got - exact) <= 18 * u * mag + u * np.abs(exact))
    assert np.all(np.abs(ref - exact) <= 2 * u * mag + u * np.abs(exact))


# ---- W4A8: the reference's INT4 linear weights, tiled, with the fused quantizer ----
@pytest.mark.parametrize("m,n,k,zp,dtype", [(1, 16384, 4096, 8, "bf16"), (1, 4096, 8192, 0, "bf16"),
                                            (2, 100, 1040, 15, "bf16"), (3, 4096, 4096, 7, "bf16"),
                                            (4, 33, 64, 8, "bf16"), (7, 4096, 4096, 3, "bf16"),
                                            (16, 1000, 2048, 9, "bf16"),
                                            # the streaming unit on INT4 tiles (3..16 rows, K % 512 == 0,
                                            # K <= 4096): bias, fewer N tiles than CUs, a ragged N over
                                            # several rounds, zero points 0 and 15, K = 512
                                            (5, 1000, 512, 4, "bf16"), (8, 16384, 4096, 8, "bf16"),
                                            (6, 100, 2048, 15, "bf16"), (4, 21520, 1024, 0, "bf16"),
                                            (12, 16384, 4096, 1, "bf16"), (9, 6000, 512, 15, "bf16"),
                                            # the expanded form: f32 rows, K past the fused unit's 8192,
                                            # prefill-sized M on the GEMM (M and N tails)
                                            (3, 1000, 2048, 6, "f32"), (1, 600, 16384, 5, "bf16"),
                                            (17, 300, 1024, 11, "bf16"), (300, 2050, 1024, 8, "bf16"),
                                            (129, 520, 4096, 2, "f32")])
def test_linear_w4a8_bit_exact(ctx, m, n, k, zp, dtype):
    """nh_linear_w4a8 against the layer's definition: or_linear_w4a8 for bf16
    rows; for f32 rows the oracle's parts (quantize_rows_f32, then the W8A8
    product with weights code - zp and every row scale = scale)."""
    from tiling import tile_int4
    note(f"linear_w4a8 m={m} n={n} k={k} zp={zp} {dtype}")
    rng = np.random.default_rng(m * 1000 + zp)
    packed = rng.integers(0, 256, size=(k * n + 1) // 2, dtype=np.uint8)
    scale = 0.0137
    if dtype == "bf16":
        x, xdt = activations_bf16(m, k), NH.BF16
    else:
        x, xdt = O.normal_f32(90 + m, m * k).reshape(m, k), NH.F32
    bias = rng.standard_normal(n).astype(np.float32) if m % 2 else None
    need = NH.lib().nh_tiled_int4_weights_bytes(n, k)
    dp, dt = ctx.upload(packed), ctx.empty(need, np.uint8)
    NH.call("nh_tile_weights_int4", ctx.handle, dp.ptr, packed.size, k, n, zp, dt.ptr, need, None)
    ctx.synchronize()
    assert np.array_equal(dt.numpy(), tile_int4(packed, k, n, zp))
    fused = dtype == "bf16" and NH.lib().nh_supports_linear_w4a8(m, n, k)
    ws_bytes = NH.lib().nh_linear_w4a8_workspace_size(m, n, k)
    ws = ctx.empty(ws_bytes, np.uint8)
    dx = ctx.upload(x)
    db = ctx.upload(bias) if bias is not None else None
    if dtype == "f32":
        st, xq, sx, _ = O.quantize_rows_f32(x)
        assert st == O.OK
        codes = np.stack([packed & 15, packed >> 4], axis=1).reshape(-1)[:k * n].reshape(k, n)
        w = (codes.astype(np.int16) - zp).astype(np.int8).T.copy()  # [N][K] = code - zp
    for out_dtype, bf in ((NH.BF16, True), (NH.F32, False)):
        out = ctx.empty((m, n), np.uint16 if bf else np.float32)
        # the fused unit needs no workspace
        NH.call("nh_linear_w4a8", ctx.handle, dx.ptr, xdt, dt.ptr, scale, zp, db.ptr if db else None, m, n, k,
                out.ptr, out_dtype, None if fused else ws.ptr, 0 if fused else ws_bytes, None, None)
        ctx.synchronize()
        if dtype == "bf16":
            st, ref = O.linear_w4a8(x, packed, n, scale, zp, bias=bias, out_bf16=bf)
            assert st == O.OK
        else:
            ref = linear_w8a8_exact(xq, sx, w, np.full(n, scale, np.float32), bias=bias, out_bf16=bf)
        assert np.array_equal(out.numpy(), ref)


# ---- G3: W8A8 GEMM (prefill) -----------------------------------------------------
@pytest.mark.parametrize("m,n,k", [(2048, 4096, 4096), (2048, 21504, 4096), (2048, 4096, 21504), (37, 100, 64),
                                   (300, 130, 272), (17, 4096, 4096), (513, 2688, 1856),
                                   # 256 x 128 tiles at their edges: one K step, fewer K steps than
                                   # ring slots, an odd K-tile count with a partial last tile, ragged
                                   # M and N (a half-valid last weight tile)
                                   (512, 8192, 64), (1000, 2000, 192), (777, 8200, 1040),
                                   # a sparse last round of 256 x 128 tiles: whole rounds, then the
                                   # remaining columns as 128 x 128 tiles (also at 777 x 8200)
                                   (1100, 9000, 128),
                                   # the persistent 256 x 224 kernel (tiled A; also 2048 x 21504): one tile
                                   # per CU, and ragged last tiles in M and N with several tiles per CU
                                   (1024, 14336, 256), (1000, 14236, 384), (2000, 21484, 128)])
@pytest.mark.parametrize("a_layout", ["row-major", "tiled"])
def test_gemm_w8a8_bit_exact(ctx, m, n, k, a_layout):
    note(f"gemm_w8a8 m={m} n={n} k={k} A {a_layout}")
    _, wq, sw = quantized_weights(n, k)
    x = activations_bf16(m, k)
    _, xq, sx, _ = O.quantize_rows_bf16(x)
    dxq = ctx.upload(xq if a_layout == "row-major" else tile_16x64(xq))
    dsx, dw, dsw = ctx.upload(sx), ctx.upload(tile_16x64(wq)), ctx.upload(sw)
    out = ctx.empty((m, n), np.uint16)
    fn = "nh_gemm_w8a8" if a_layout == "row-major" else "nh_gemm_w8a8_ta"
    NH.call(fn, ctx.handle, dxq.ptr, dsx.ptr, dw.ptr, dsw.ptr, None, m, n, k, out.ptr, NH.BF16, None)
    ctx.synchronize()
    got = out.numpy()
    # every row and column: the oracle's epilogue on exact accumulators (the
    # oracle's own int32 loop for small shapes, exact float64 BLAS for the
    # M = 2048 configs, pinned against it in test_exact_int.py)
    ref = O.linear_w8a8(xq, sx, wq, sw, out_bf16=True) if m * n * k <= 2e9 else \
        linear_w8a8_exact(xq, sx, wq, sw, out_bf16=True)
    assert np.array_equal(got, ref)


# ---- R1..R4: MoE -----------------------------------------------------------------
def route_on_device(ctx, scores, t, e, k, renorm, scaling=1.0):
    ds = ctx.upload(scores)
    di = ctx.empty(t * k, np.int32)
    dw = ctx.empty(t * k, np.float32)
    NH.call("nh_moe_route_sigmoid_topk", ctx.handle, ds.ptr, t, e, k, renorm, scaling, di.ptr, dw.ptr, None)
    ctx.synchronize()
    return di.numpy(), dw.numpy()


@pytest.mark.parametrize("t,e,k,renorm,scaling", [(512, 128, 6, 1, 1.0), (512, 128, 6, 0, 1.0), (64, 128, 6, 1, 2.5),
                                                  (3, 1000, 8, 1, 1.0), (5, 7, 7, 0, 1.0), (17, 129, 4, 0, 1.0),
                                                  (40, 200, 6, 1, 1.0), (9, 256, 8, 1, 1.0), (6, 257, 3, 0, 1.0)])
def test_route_sigmoid_bit_exact(ctx, t, e, k, renorm, scaling):
    note(f"route t={t} e={e} k={k} renorm={renorm}")
    scores = O.normal_f32(2, t * e)
    idx, w = route_on_device(ctx, scores, t, e, k, renorm, scaling)
    _, ridx, rw, _ = O.route_sigmoid(scores, t, e, k, renormalize=bool(renorm), scaling=scaling)
    assert np.array_equal(idx, ridx)
    assert np.array_equal(w.view(np.uint32), rw.view(np.uint32))


def test_route_reference_kats_on_device(ctx):
    note("route KATs")
    for scores, t, e, k, want_idx, want_w in [
            ([0.0, 1.0, -1.0, 2.0], 1, 4, 2, [3, 1], [0.880797, 0.7310586]),  # moe_routing.rs:618-623
            ([0.0, 1.0, -1.0, 2.0, 5.0, -5.0, 0.5, 0.6], 2, 4, 2, [3, 1, 0, 3],
             [0.880797, 0.7310586, 0.9933072, 0.6456563]),                       # :629-641
            ([0.0, 0.0, 1.0], 1, 3, 2, [2, 0], [0.7310586, 0.5]),                # :647-653 ties
            ([0.1, 0.9, 0.4, 0.6], 2, 2, 1, None, None)]:                        # :809-822
        s = np.array(scores, dtype=np.float32)
        idx, w = route_on_device(ctx, s, t, e, k, 0)
        _, ridx, rw, _ = O.route_sigmoid(s, t, e, k)
        assert np.array_equal(idx, ridx) and np.all(np.abs(w - rw) <= 5e-6)
        if want_idx is not None:
            assert idx.tolist() == want_idx and np.all(np.abs(w - np.array(want_w)) <= 1e-6)
    # moe_routing.rs:846-864: 128 experts, top-6, heavily tied pattern
    t, e, k = 2, 128, 6
    s = np.array([((x % 17) - 8.0) * 0.375 + tt * 0.125 - 0.05 for tt in range(t) for x in range(e)], dtype=np.float32)
    idx, w = route_on_device(ctx, s, t, e, k, 0)
    _, ridx, rw, _ = O.route_sigmoid(s, t, e, k)
    assert np.array_equal(idx, ridx) and np.array_equal(w, rw)


@pytest.mark.parametrize("t,k,e", [(512, 6, 128), (1, 1, 1), (1000, 8, 64), (3, 2, 1000), (2000, 6, 128),
                                   (300, 2, 3),  # long same-expert runs inside every wave
                                   (600, 5, 100), (700, 8, 16),
                                   (70000, 8, 8)])  # experts x routes past the one-wave-per-expert form
def test_permute_bit_exact(ctx, t, k, e):
    note(f"permute t={t} k={k} e={e}")
    rng = np.random.default_rng(t + e)
    idx = np.stack([rng.choice(e, size=k, replace=False) for _ in range(t)]).astype(np.int32).ravel()
    ref = O.moe_permute(idx, t, k, e)
    di = ctx.upload(idx)
    off = ctx.empty(e + 1, np.int32)
    perm = ctx.empty(t * k, np.int32)
    pos = ctx.empty(t * k, np.int32)
    NH.call("nh_moe_permute", ctx.handle, di.ptr, t, k, e, off.ptr, perm.ptr, pos.ptr, None)
    ctx.synchronize()
    assert np.array_equal(off.numpy(), ref[0])
    assert np.array_equal(perm.numpy(), ref[1])
    assert np.array_equal(pos.numpy(), ref[2])


@pytest.mark.parametrize("t,k,e", [(512, 6, 128), (40, 3, 5)])
def test_permute_ids_outside_the_experts(ctx, t, k, e):
    """Expert ids outside [0, E) are not placed (pos = -1) and take no slot;
    the valid routes keep the stable (expert, route id) order."""
    note(f"permute invalid ids t={t} k={k} e={e}")
    rng = np.random.default_rng(7 + e)
    idx = rng.integers(0, e, size=t * k).astype(np.int32)
    bad = rng.choice(t * k, size=t * k // 7, replace=False)
    idx[bad] = rng.choice([-1, -5, e, e + 3], size=bad.size)
    valid = (idx >= 0) & (idx < e)
    order = sorted(np.flatnonzero(valid).tolist(), key=lambda r: (idx[r], r))
    want_off = np.zeros(e + 1, np.int32)
    np.add.at(want_off, idx[valid] + 1, 1)
    want_off = np.cumsum(want_off).astype(np.int32)
    want_pos = np.full(t * k, -1, np.int32)
    want_pos[order] = np.arange(len(order), dtype=np.int32)
    di = ctx.upload(idx)
    off = ctx.empty(e + 1, np.int32)
    perm = ctx.empty(t * k, np.int32)
    pos = ctx.empty(t * k, np.int32)
    NH.call("nh_moe_permute", ctx.handle, di.ptr, t, k, e, off.ptr, perm.ptr, pos.ptr, None)
    ctx.synchronize()
    assert np.array_equal(off.numpy(), want_off)
    assert np.array_equal(perm.numpy()[:len(order)], np.array(order, np.int32))
    assert np.array_equal(pos.numpy(), want_pos)


@pytest.mark.parametrize("tokens,top_k,hidden", [(512, 6, 2688), (7, 3, 37), (5, 2, 8)])
@pytest.mark.parametrize("with_shared", [False, True])
def test_combine_bit_exact(ctx, tokens, top_k, hidden, with_shared):
    """R4 on the device: the four-column kernel (hidden % 4 == 0) and the
    scalar one (37), f32 and bf16 out, with an unplaced route (pos -1)."""
    note(f"combine t={tokens} k={top_k} h={hidden} shared={with_shared}")
    rng = np.random.default_rng(tokens + hidden)
    R = tokens * top_k
    slot_out = rng.standard_normal((R, hidden)).astype(np.float32)
    pos = rng.permutation(R).astype(np.int32)
    pos[R // 2] = -1
    w = rng.random(R).astype(np.float32)
    shared = rng.standard_normal((tokens, hidden)).astype(np.float32) if with_shared else None
    d = [ctx.upload(a) for a in (slot_out, pos, w)]
    dsh = ctx.upload(shared) if with_shared else None
    for out_dtype, bf in ((NH.F32, False), (NH.BF16, True)):
        out = ctx.empty((tokens, hidden), np.uint16 if bf else np.float32)
        NH.call("nh_moe_combine_shared", ctx.handle, d[0].ptr, d[1].ptr, d[2].ptr, dsh.ptr if dsh else None, tokens,
                top_k, hidden, out.ptr, out_dtype, None)
        ctx.synchronize()
        ref = O.moe_combine_shared(slot_out, pos, w, shared, tokens, top_k, hidden, out_bf16=bf)
        assert np.array_equal(out.numpy(), ref)


def moe_weights(experts, inter, hidden):
    up = np.empty((experts, inter, hidden), dtype=np.int8)
    down = np.empty((experts, hidden, inter), dtype=np.int8)
    su = np.empty((experts, inter), dtype=np.float32)
    sd = np.empty((experts, hidden), dtype=np.float32)
    for e in range(experts):
        w = O.normal_f32(100 + e, inter * hidden + hidden * inter, 0.0, 0.02)
        _, q, s, _ = O.quantize_rows_f32(w[: inter * hidden].reshape(inter, hidden))
        up[e], su[e] = q, s
        _, q, s, _ = O.quantize_rows_f32(w[inter * hidden:].reshape(hidden, inter))
        down[e], sd[e] = q, s
    return up, su, down, sd


@functools.lru_cache(maxsize=1)
def moe_weights_cached(experts, inter, hidden):
    return moe_weights(experts, inter, hidden)


@functools.lru_cache(maxsize=2)
def moe_case(tokens, hidden, inter, experts, top_k):
    x = activations_bf16(tokens, hidden)
    logits = O.normal_f32(2, tokens * experts)
    up, su, down, sd = moe_weights_cached(experts, inter, hidden)
    return x, logits, up, su, down, sd


@pytest.mark.parametrize("tokens,hidden,inter,experts,top_k", [(64, 2688, 1856, 128, 6), (13, 64, 32, 8, 3)])
def test_moe_stages_bit_exact(ctx, tokens, hidden, inter, experts, top_k):
    note(f"moe stages t={tokens} h={hidden} i={inter} e={experts} k={top_k}")
    x, logits, up, su, down, sd = moe_case(tokens, hidden, inter, experts, top_k)
    _, xq, sx, _ = O.quantize_rows_bf16(x)
    _, idx, w, _ = O.route_sigmoid(logits, tokens, experts, top_k, renormalize=True)
    offsets, perm, pos = O.moe_permute(idx, tokens, top_k, experts)
    R = tokens * top_k
    h_ref = O.moe_grouped(xq, sx, True, top_k, offsets, perm, up, su, relu2=True)
    d = {n: ctx.upload(a) for n, a in dict(xq=xq, sx=sx, off=offsets, perm=perm, pos=pos, w=w, up=tile_experts(up),
                                           su=su, down=tile_experts(down), sd=sd).items()}
    h = ctx.empty((R, inter), np.float32)
    NH.call("nh_moe_grouped_gemm_w8a8", ctx.handle, d["xq"].ptr, d["sx"].ptr, 1, top_k, d["off"].ptr, d["perm"].ptr,
            R, tokens, experts, d["up"].ptr, d["su"].ptr, inter, hidden, 1, h.ptr, None)
    ctx.synchronize()
    assert np.array_equal(h.numpy(), h_ref)
    _, hq, sh, _ = O.quantize_rows_f32(h_ref)
    d_ref = O.moe_grouped(hq, sh, False, top_k, offsets, perm, down, sd, relu2=False)
    dhq, dsh = ctx.upload(hq), ctx.upload(sh)
    dd = ctx.empty((R, hidden), np.float32)
    NH.call("nh_moe_grouped_gemm_w8a8", ctx.handle, dhq.ptr, dsh.ptr, 0, top_k, d["off"].ptr, d["perm"].ptr, R, R,
            experts, d["down"].ptr, d["sd"].ptr, hidden, inter, 0, dd.ptr, None)
    ctx.synchronize()
    assert np.array_equal(dd.numpy(), d_ref)
    out = ctx.empty((tokens, hidden), np.uint16)
    NH.call("nh_moe_combine", ctx.handle, dd.ptr, d["pos"].ptr, d["w"].ptr, tokens, top_k, hidden, out.ptr, NH.BF16,
            None)
    ctx.synchronize()
    assert np.array_equal(out.numpy(), O.moe_combine(d_ref, pos, w, tokens, top_k, hidden, out_bf16=True))


@pytest.mark.parametrize("n,k", [(1856, 2688), (2688, 1856), (40, 64), (256, 64), (160, 512)])
def test_expert_gemm_long_segments_bit_exact(ctx, n, k):
    """Slot-ordered grouped GEMM (the MoE layer's expert-block kernel) with
    segments around every pass boundary: a pass stages 48 rows at K = 2688,
    64 at K = 1856, 64 at K = 64, and longer segments take several passes."""
    note(f"expert gemm long segments n={n} k={k}")
    counts = [0, 1, 17, 33, 47, 48, 49, 64, 65, 100, 130, 0, 16]
    experts = len(counts)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    R = int(offsets[-1])
    rng = np.random.default_rng(n + k)
    aq = rng.integers(-127, 128, size=(R, k), dtype=np.int8)
    sa = rng.uniform(1e-3, 2e-2, size=R).astype(np.float32)
    w = rng.integers(-127, 128, size=(experts, n, k), dtype=np.int8)
    sw = rng.uniform(1e-4, 1e-3, size=(experts, n)).astype(np.float32)
    perm = np.arange(R, dtype=np.int32)
    for relu2 in (0, 1):
        ref = O.moe_grouped(aq, sa, False, 1, offsets, perm, w, sw, relu2=relu2)
        d = {nm: ctx.upload(a) for nm, a in dict(aq=aq, sa=sa, off=offsets, perm=perm, w=tile_experts(w), sw=sw).items()}
        out = ctx.empty((R, n), np.float32)
        NH.call("nh_moe_grouped_gemm_w8a8", ctx.handle, d["aq"].ptr, d["sa"].ptr, 0, 1, d["off"].ptr, d["perm"].ptr,
                R, R, experts, d["w"].ptr, d["sw"].ptr, n, k, relu2, out.ptr, None)
        ctx.synchronize()
        assert np.array_equal(out.numpy(), ref)


@pytest.mark.parametrize("tokens,hidden,inter,experts,top_k,sh_inter", [(64, 2688, 1856, 128, 6, 3712),
                                                                         (13, 64, 32, 8, 3, 48)])
def test_moe_forward_shared_expert_bit_exact(ctx, tokens, hidden, inter, experts, top_k, sh_inter):
    """The layer with its shared expert (moe.rs:197-219; 3712 wide in the
    reference config, config.rs:227): the int8 MLP of every token, added to
    the output row ahead of the routed experts."""
    note(f"moe forward + shared t={tokens} h={hidden} i={inter} e={experts} k={top_k} si={sh_inter}")
    x, logits, up, su, down, sd = moe_case(tokens, hidden, inter, experts, top_k)
    _, hu, hsu = quantized_weights(sh_inter, hidden, seed=30)
    _, hd, hsd = quantized_weights(hidden, sh_inter, seed=31)
    st, ref, *_ = O.moe_forward_shared_w8a8(x, logits, up, su, down, sd, top_k, hu, hsu, hd, hsd)
    assert st == O.OK
    ws_bytes = NH.lib().nh_moe_forward_shared_w8a8_workspace_size(tokens, hidden, inter, experts, top_k, sh_inter)
    ws = ctx.empty(ws_bytes, np.uint8)
    dx, dl = ctx.upload(x), ctx.upload(logits)
    dup, dsu, ddown, dsd = ctx.upload(tile_experts(up)), ctx.upload(su), ctx.upload(tile_experts(down)), ctx.upload(sd)
    dhu, dhsu, dhd, dhsd = ctx.upload(tile_16x64(hu)), ctx.upload(hsu), ctx.upload(tile_16x64(hd)), ctx.upload(hsd)
    out = ctx.empty((tokens, hidden), np.uint16)
    NH.call("nh_moe_forward_shared_w8a8", ctx.handle, dx.ptr, NH.BF16, dl.ptr, tokens, hidden, inter, experts, top_k,
            1, 1.0, dup.ptr, dsu.ptr, ddown.ptr, dsd.ptr, sh_inter, dhu.ptr, dhsu.ptr, dhd.ptr, dhsd.ptr, None, out.ptr,
            NH.BF16, ws.ptr, ws_bytes, None, None)
    ctx.synchronize()
    assert np.array_equal(out.numpy(), ref)


@pytest.mark.parametrize("tokens,hidden,inter,experts,top_k", [(64, 2688, 1856, 128, 6), (13, 64, 32, 8, 3),
                                                                (256, 64, 32, 16, 6), (40, 256, 160, 8, 3),
                                                                (24, 512, 256, 4, 2)])
def test_moe_forward_bit_exact(ctx, tokens, hidden, inter, experts, top_k):
    note(f"moe forward t={tokens} h={hidden} i={inter} e={experts} k={top_k}")
    x, logits, up, su, down, sd = moe_case(tokens, hidden, inter, experts, top_k)
    st, ref, idx, w, offsets, perm, pos = O.moe_forward_w8a8(x, logits, up, su, down, sd, top_k, renormalize=True)
    assert st == O.OK
    ws_bytes = NH.lib().nh_moe_forward_w8a8_workspace_size(tokens, hidden, inter, experts, top_k)
    ws = ctx.empty(ws_bytes, np.uint8)
    dx, dl = ctx.upload(x), ctx.upload(logits)
    dup, dsu, ddown, dsd = ctx.upload(tile_experts(up)), ctx.upload(su), ctx.upload(tile_experts(down)), ctx.upload(sd)
    out = ctx.empty((tokens, hidden), np.uint16)
    NH.call("nh_moe_forward_w8a8", ctx.handle, dx.ptr, NH.BF16, dl.ptr, tokens, hidden, inter, experts, top_k, 1, 1.0,
            dup.ptr, dsu.ptr, ddown.ptr, dsd.ptr, None, out.ptr, NH.BF16, ws.ptr, ws_bytes, None, None)
    ctx.synchronize()
    lay = (ctypes.c_size_t * 5)()
    NH.lib().nh_moe_workspace_layout(tokens, hidden, inter, experts, top_k, lay)
    wsh = ws.numpy()
    R = tokens * top_k
    assert np.array_equal(wsh[lay[0]:lay[0] + 4 * R].view(np.int32), idx)
    assert np.array_equal(wsh[lay[2]:lay[2] + 4 * (experts + 1)].view(np.int32), offsets)
    assert np.array_equal(wsh[lay[3]:lay[3] + 4 * R].view(np.int32), perm)
    assert np.array_equal(out.numpy(), ref)


# ---- configs[3] at its full size: 512 tokens, 128 experts, top-6 ----------------
CONFIG3 = (512, 2688, 1856, 128, 6)


@functools.lru_cache(maxsize=1)
def config3_reference():
    """The oracle's composition at configs[3]: the stages are the oracle's,
    the expert accumulations exact through float64 BLAS (exact_int.py)."""
    tokens, hidden, inter, experts, top_k = CONFIG3
    x, logits, up, su, down, sd = moe_case(*CONFIG3)
    return moe_forward_exact(x, logits, up, su, down, sd, top_k)


def test_moe_forward_config3_bit_exact(ctx):
    """nh_moe_forward_w8a8 at configs[3] (the bench's layer): every routing
    index and weight, the offsets, the permutation and its inverse from the
    workspace, and every output element against the oracle."""
    tokens, hidden, inter, experts, top_k = CONFIG3
    note(f"moe forward configs[3] t={tokens} h={hidden} i={inter} e={experts} k={top_k}")
    x, logits, up, su, down, sd = moe_case(*CONFIG3)
    ref, idx, w, offsets, perm, pos, _, _ = config3_reference()
    counts = np.diff(offsets)
    note(f"routes per expert: min {counts.min()} max {counts.max()} (expert kernel passes: 48 rows at K=2688)")
    ws_bytes = NH.lib().nh_moe_forward_w8a8_workspace_size(tokens, hidden, inter, experts, top_k)
    ws = ctx.empty(ws_bytes, np.uint8)
    ws.fill_bytes(0xa5)
    dx, dl = ctx.upload(x), ctx.upload(logits)
    dup, dsu, ddown, dsd = ctx.upload(tile_experts(up)), ctx.upload(su), ctx.upload(tile_experts(down)), ctx.upload(sd)
    out = ctx.empty((tokens, hidden), np.uint16)
    NH.call("nh_moe_forward_w8a8", ctx.handle, dx.ptr, NH.BF16, dl.ptr, tokens, hidden, inter, experts, top_k, 1, 1.0,
            dup.ptr, dsu.ptr, ddown.ptr, dsd.ptr, None, out.ptr, NH.BF16, ws.ptr, ws_bytes, None, None)
    ctx.synchronize()
    lay = (ctypes.c_size_t * 5)()
    NH.lib().nh_moe_workspace_layout(tokens, hidden, inter, experts, top_k, lay)
    wsh = ws.numpy()
    R = tokens * top_k
    assert np.array_equal(wsh[lay[0]:lay[0] + 4 * R].view(np.int32), idx)
    assert np.array_equal(wsh[lay[1]:lay[1] + 4 * R].view(np.uint32), w.view(np.uint32))
    assert np.array_equal(wsh[lay[2]:lay[2] + 4 * (experts + 1)].view(np.int32), offsets)
    assert np.array_equal(wsh[lay[3]:lay[3] + 4 * R].view(np.int32), perm)
    assert np.array_equal(wsh[lay[4]:lay[4] + 4 * R].view(np.int32), pos)
    got = out.numpy()
    assert np.array_equal(got, ref), f"{(got != ref).sum()} of {ref.size} outputs differ"


def router_case(tokens, hidden, experts, seed=40):
    """The dense f32 router of MoeLayer ([hidden][experts] weights and a bias)
    and the logits the reference computes from bf16 x: gemm_into_host on the
    widened input (the oracle's f64-accumulated GEMM), then the bias added in
    f32 (linear.rs:330-336)."""
    rw = O.normal_f32(seed, hidden * experts, 0.0, 0.02).reshape(hidden, experts)
    rb = O.normal_f32(seed + 1, experts, 0.0, 0.1)
    return rw, rb


def router_logits(x_bf16, rw, rb):
    tokens, hidden = x_bf16.shape
    experts = rw.shape[1]
    xf = (x_bf16.astype(np.uint32) << 16).view(np.float32)
    st, logits, _ = O.gemm_f32(xf, rw, tokens, hidden, experts)
    assert st == O.OK
    return (logits.reshape(tokens, experts) + rb[None, :]).astype(np.float32).ravel()


@pytest.mark.parametrize("tokens,hidden,inter,experts,top_k,sh_inter", [(13, 64, 32, 8, 3, 0), (64, 2688, 1856, 128, 6, 3712),
                                                                         (512, 2688, 1856, 128, 6, 0)])
def test_moe_layer_with_router_bit_exact(ctx, tokens, hidden, inter, experts, top_k, sh_inter):
    """nh_moe_layer_w8a8: MoeLayer::forward_into from its input (moe.rs:154-249),
    the dense router on the device, routing as moe_route_host (no
    renormalization, scale 1).  The logits in the workspace and every output
    element against the oracle."""
    note(f"moe layer + router t={tokens} h={hidden} i={inter} e={experts} k={top_k} si={sh_inter}")
    x, _, up, su, down, sd = moe_case(tokens, hidden, inter, experts, top_k)
    rw, rb = router_case(tokens, hidden, experts)
    logits = router_logits(x, rw, rb)
    if sh_inter:
        _, hu, hsu = quantized_weights(sh_inter, hidden, seed=30)
        _, hd, hsd = quantized_weights(hidden, sh_inter, seed=31)
        st, ref, idx, *_ = O.moe_forward_shared_w8a8(x, logits, up, su, down, sd, top_k, hu, hsu, hd, hsd,
                                                     renormalize=False)
        assert st == O.OK
    elif tokens > 64:
        ref, idx, *_ = moe_forward_exact(x, logits, up, su, down, sd, top_k, renormalize=False)
    else:
        st, ref, idx, *_ = O.moe_forward_w8a8(x, logits, up, su, down, sd, top_k, renormalize=False)
        assert st == O.OK
    lib = NH.lib()
    ws_bytes = lib.nh_moe_layer_w8a8_workspace_size(tokens, hidden, inter, experts, top_k, sh_inter)
    inner = (lib.nh_moe_forward_shared_w8a8_workspace_size(tokens, hidden, inter, experts, top_k, sh_inter) if sh_inter
             else lib.nh_moe_forward_w8a8_workspace_size(tokens, hidden, inter, experts, top_k))
    ws = ctx.empty(ws_bytes, np.uint8)
    ws.fill_bytes(0x5a)
    dx, drw, drb = ctx.upload(x), ctx.upload(rw), ctx.upload(rb)
    dup, dsu, ddown, dsd = ctx.upload(tile_experts(up)), ctx.upload(su), ctx.upload(tile_experts(down)), ctx.upload(sd)
    sh = [None] * 4
    if sh_inter:
        dhu, dhsu, dhd, dhsd = (ctx.upload(tile_16x64(hu)), ctx.upload(hsu), ctx.upload(tile_16x64(hd)),
                                ctx.upload(hsd))
        sh = [dhu.ptr, dhsu.ptr, dhd.ptr, dhsd.ptr]
    out = ctx.empty((tokens, hidden), np.uint16)
    NH.call("nh_moe_layer_w8a8", ctx.handle, dx.ptr, NH.BF16, drw.ptr, drb.ptr, tokens, hidden, inter, experts,
            top_k, 0, 1.0, dup.ptr, dsu.ptr, ddown.ptr, dsd.ptr, sh_inter, *sh, None, out.ptr, NH.BF16, ws.ptr, ws_bytes,
            None, None)
    ctx.synchronize()
    wsh = ws.numpy()
    at = (inner + 255) // 256 * 256
    assert np.array_equal(wsh[at:at + 4 * tokens * experts].view(np.uint32), logits.view(np.uint32))
    lay = (ctypes.c_size_t * 5)()
    lib.nh_moe_workspace_layout(tokens, hidden, inter, experts, top_k, lay)
    assert np.array_equal(wsh[lay[0]:lay[0] + 4 * tokens * top_k].view(np.int32), idx)
    got = out.numpy()
    assert np.array_equal(got, ref), f"{(got != ref).sum()} of {ref.size} outputs differ"


def moe_biases_case(experts, inter, hidden, sh_inter, seed=50):
    """Expert and shared-expert biases (the reference's MlpLayer biases,
    mlp.rs:79-96), N(0, 0.5) up and N(0, 1) down."""
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((experts, inter)).astype(np.float32) * 0.5,
            rng.standard_normal((experts, hidden)).astype(np.float32),
            rng.standard_normal(sh_inter).astype(np.float32) * 0.5 if sh_inter else None,
            rng.standard_normal(hidden).astype(np.float32) if sh_inter else None)


@pytest.mark.parametrize("tokens,hidden,inter,experts,top_k,sh_inter", [(13, 64, 32, 8, 3, 16), (64, 2688, 1856, 128, 6, 3712),
                                                                         (40, 2688, 1856, 128, 6, 0),
                                                                         (7, 64, 2112, 4, 2, 0)])  # unfused: inter > 2048
def test_moe_layer_with_biases_bit_exact(ctx, tokens, hidden, inter, experts, top_k, sh_inter):
    """nh_moe_layer_w8a8 with the routed experts' up and down biases and the
    shared expert's (the up bias before ReLU^2, the down bias on the expert's
    output before the combine weight, mlp.rs:201-208) against the oracle's
    int8 layer with the same biases, every output; and against the host twin."""
    note(f"moe layer + biases t={tokens} h={hidden} i={inter} e={experts} k={top_k} si={sh_inter}")
    x, _, up, su, down, sd = moe_case(tokens, hidden, inter, experts, top_k)
    rw, rb = router_case(tokens, hidden, experts)
    logits = router_logits(x, rw, rb)
    b = moe_biases_case(experts, inter, hidden, sh_inter)
    shw = (None, None, None, None)
    if sh_inter:
        _, hu, hsu = quantized_weights(sh_inter, hidden, seed=30)
        _, hd, hsd = quantized_weights(hidden, sh_inter, seed=31)
        shw = (hu, hsu, hd, hsd)
    st, ref, idx, *_ = O.moe_forward_shared_w8a8(x, logits, up, su, down, sd, top_k, *shw, renormalize=False,
                                                 biases=b)
    assert st == O.OK
    lib = NH.lib()
    ws_bytes = lib.nh_moe_layer_w8a8_workspace_size(tokens, hidden, inter, experts, top_k, sh_inter)
    ws = ctx.empty(ws_bytes, np.uint8)
    ws.fill_bytes(0x5a)
    dx, drw, drb = ctx.upload(x), ctx.upload(rw), ctx.upload(rb)
    dup, dsu, ddown, dsd = ctx.upload(tile_experts(up)), ctx.upload(su), ctx.upload(tile_experts(down)), ctx.upload(sd)
    dbs = [ctx.upload(v) if v is not None else None for v in b]
    mb = NH.MoeBiases(*[d.ptr if d is not None else None for d in dbs])
    sh = [None] * 4
    if sh_inter:
        dsh = [ctx.upload(tile_16x64(hu)), ctx.upload(hsu), ctx.upload(tile_16x64(hd)), ctx.upload(hsd)]
        sh = [d.ptr for d in dsh]
    out = ctx.empty((tokens, hidden), np.uint16)
    NH.call("nh_moe_layer_w8a8", ctx.handle, dx.ptr, NH.BF16, drw.ptr, drb.ptr, tokens, hidden, inter, experts,
            top_k, 0, 1.0, dup.ptr, dsu.ptr, ddown.ptr, dsd.ptr, sh_inter, *sh, mb, out.ptr, NH.BF16, ws.ptr,
            ws_bytes, None, None)
    ctx.synchronize()
    got = out.numpy()
    assert np.array_equal(got, ref), f"{(got != ref).sum()} of {ref.size} outputs differ"
    if tokens <= 13:  # the host twin on the same operands (the fallback path), bit for bit
        tiles = [tile_experts(up), tile_experts(down)] + ([tile_16x64(hu), tile_16x64(hd)] if sh_inter else [])
        hsh = [tiles[2].ctypes.data, hsu.ctypes.data, tiles[3].ctypes.data, hsd.ctypes.data] if sh_inter else [None] * 4
        hb = NH.MoeBiases(*[v.ctypes.data if v is not None else None for v in b])
        hout = np.zeros((tokens, hidden), np.uint16)
        NH.call("nh_moe_layer_w8a8_host", x.ctypes.data, NH.BF16, rw.ctypes.data, rb.ctypes.data, tokens, hidden,
                inter, experts, top_k, 0, ctypes.c_float(1.0), tiles[0].ctypes.data, su.ctypes.data,
                tiles[1].ctypes.data, sd.ctypes.data, sh_inter, *hsh, hb, hout.ctypes.data, NH.BF16)
        assert np.array_equal(hout, got)


def test_moe_shared_intermediate_reported_ahead_of_the_routed_experts(ctx):
    """The shared expert's overflowing intermediate is reported as
    "shared_intermediate" (its own [tokens][shared_inter] index), ahead of an
    overflow in the routed experts' intermediate, as MoeLayer::forward_into
    meets the shared expert first (moe.rs:197-219); a routed overflow alone is
    "intermediate"."""
    tokens, hidden, inter, experts, top_k, sh_inter = 64, 2688, 1856, 128, 6, 3712
    note(f"moe shared-intermediate non-finite t={tokens} si={sh_inter}")
    x, logits, up, su, down, sd = moe_case(tokens, hidden, inter, experts, top_k)
    _, hu, hsu = quantized_weights(sh_inter, hidden, seed=30)
    _, hd, hsd = quantized_weights(hidden, sh_inter, seed=31)
    b_up = np.zeros((experts, inter), np.float32)
    b_up[:, 7] = 3e38  # every routed row overflows at column 7
    b_sh = np.zeros(sh_inter, np.float32)
    b_sh[100] = 3e38   # every shared row overflows at column 100
    lib = NH.lib()
    ws_bytes = lib.nh_moe_forward_shared_w8a8_workspace_size(tokens, hidden, inter, experts, top_k, sh_inter)
    ws = ctx.empty(ws_bytes, np.uint8)
    dx, dl = ctx.upload(x), ctx.upload(logits)
    dup, dsu, ddown, dsd = ctx.upload(tile_experts(up)), ctx.upload(su), ctx.upload(tile_experts(down)), ctx.upload(sd)
    dsh = [ctx.upload(tile_16x64(hu)), ctx.upload(hsu), ctx.upload(tile_16x64(hd)), ctx.upload(hsd)]
    dbu, dbs = ctx.upload(b_up), ctx.upload(b_sh)
    word = ctx.upload(np.zeros(1, dtype=np.uint64))
    out = ctx.empty((tokens, hidden), np.uint16)
    for mb, want, index in ((NH.MoeBiases(dbu.ptr, None, dbs.ptr, None), b"shared_intermediate", 100),
                            (NH.MoeBiases(dbu.ptr, None, None, None), b"intermediate", 7)):
        NH.call("nh_moe_forward_shared_w8a8", ctx.handle, dx.ptr, NH.BF16, dl.ptr, tokens, hidden, inter, experts,
                top_k, 1, 1.0, dup.ptr, dsu.ptr, ddown.ptr, dsd.ptr, sh_inter, *[d.ptr for d in dsh], mb, out.ptr,
                NH.BF16, ws.ptr, ws_bytes, word.ptr, None)
        st, err = take_nonfinite(ctx, word)
        assert st == NH.NON_FINITE_INPUT and err.argument == want and err.index == index
        assert np.isinf(err.value) and err.value > 0


def test_moe_layer_router_reads_bf16_rows_off_a_4_byte_boundary(ctx):
    """The router GEMM widens bf16 rows that start on a 2-byte boundary (x one
    element into its allocation) exactly as aligned ones: logits and the
    layer's output against the oracle."""
    tokens, hidden, inter, experts, top_k = 13, 64, 32, 8, 3
    note(f"moe layer + router, x at +2 bytes t={tokens} h={hidden}")
    x, _, up, su, down, sd = moe_case(tokens, hidden, inter, experts, top_k)
    rw, rb = router_case(tokens, hidden, experts)
    logits = router_logits(x, rw, rb)
    st, ref, idx, *_ = O.moe_forward_w8a8(x, logits, up, su, down, sd, top_k, renormalize=False)
    assert st == O.OK
    lib = NH.lib()
    ws_bytes = lib.nh_moe_layer_w8a8_workspace_size(tokens, hidden, inter, experts, top_k, 0)
    inner = lib.nh_moe_forward_w8a8_workspace_size(tokens, hidden, inter, experts, top_k)
    ws = ctx.empty(ws_bytes, np.uint8)
    dx = ctx.upload(np.concatenate([np.zeros(1, np.uint16), x.ravel()]))
    drw, drb = ctx.upload(rw), ctx.upload(rb)
    dup, dsu, ddown, dsd = ctx.upload(tile_experts(up)), ctx.upload(su), ctx.upload(tile_experts(down)), ctx.upload(sd)
    out = ctx.empty((tokens, hidden), np.uint16)
    NH.call("nh_moe_layer_w8a8", ctx.handle, dx.ptr + 2, NH.BF16, drw.ptr, drb.ptr, tokens, hidden, inter, experts,
            top_k, 0, 1.0, dup.ptr, dsu.ptr, ddown.ptr, dsd.ptr, 0, None, None, None, None, None, out.ptr, NH.BF16, ws.ptr,
            ws_bytes, None, None)
    ctx.synchronize()
    wsh = ws.numpy()
    at = (inner + 255) // 256 * 256
    assert np.array_equal(wsh[at:at + 4 * tokens * experts].view(np.uint32), logits.view(np.uint32))
    assert np.array_equal(out.numpy(), ref)


def test_moe_layer_rejects_before_the_device(ctx):
    err = NH.NhError()
    L = NH.lib()
    st = L.nh_moe_layer_w8a8(ctx.handle, None, NH.BF16, None, None, 0, 64, 32, 8, 3, 0, 1.0, None, None, None, None,
                             0, None, None, None, None, None, None, NH.BF16, None, 0, None, None, ctypes.byref(err))
    assert st == NH.INVALID_ROW_COUNT
    st = L.nh_moe_layer_w8a8(ctx.handle, None, NH.BF16, None, None, 4, 64, 32, 8, 3, 0, 1.0, None, None, None, None,
                             0, None, None, None, None, None, None, NH.BF16, None, 0, None, None, ctypes.byref(err))
    assert st == NH.INVALID_PARAMS
    ws_need = L.nh_moe_layer_w8a8_workspace_size(4, 64, 32, 8, 3, 0)
    st = L.nh_moe_layer_w8a8(ctx.handle, None, NH.BF16, ctypes.c_void_p(16), None, 4, 64, 32, 8, 3, 0, 1.0, None,
                             None, None, None, 0, None, None, None, None, None, None, NH.BF16, None, 0, None, None,
                             ctypes.byref(err))
    assert st == NH.LENGTH_MISMATCH and err.argument == b"workspace" and err.expected == ws_need


def test_grouped_gemm_config3_routes_bit_exact(ctx):
    """nh_moe_grouped_gemm_w8a8 on the 3072 routes of configs[3]: the up
    projection gathered from token-major codes (the grouped kernel) and from
    slot-ordered codes (the MoE layer's expert-block kernel), and the down
    projection, every output against the oracle."""
    tokens, hidden, inter, experts, top_k = CONFIG3
    note(f"grouped gemm configs[3] routes={tokens * top_k}")
    x, logits, up, su, down, sd = moe_case(*CONFIG3)
    _, idx, w, offsets, perm, pos, h_ref, d_ref = config3_reference()
    _, xq, sx, _ = O.quantize_rows_bf16(x)
    R = tokens * top_k
    d = {nm: ctx.upload(a) for nm, a in dict(xq=xq, sx=sx, xs=xq[perm // top_k], ss=sx[perm // top_k], off=offsets,
                                               perm=perm, up=tile_experts(up), su=su, down=tile_experts(down),
                                               sd=sd).items()}
    h = ctx.empty((R, inter), np.float32)
    NH.call("nh_moe_grouped_gemm_w8a8", ctx.handle, d["xq"].ptr, d["sx"].ptr, 1, top_k, d["off"].ptr, d["perm"].ptr,
            R, tokens, experts, d["up"].ptr, d["su"].ptr, inter, hidden, 1, h.ptr, None)
    ctx.synchronize()
    assert np.array_equal(h.numpy(), h_ref)
    h2 = ctx.empty((R, inter), np.float32)
    NH.call("nh_moe_grouped_gemm_w8a8", ctx.handle, d["xs"].ptr, d["ss"].ptr, 0, top_k, d["off"].ptr, d["perm"].ptr,
            R, R, experts, d["up"].ptr, d["su"].ptr, inter, hidden, 1, h2.ptr, None)
    ctx.synchronize()
    assert np.array_equal(h2.numpy(), h_ref)
    _, hq, sh, _ = O.quantize_rows_f32(h_ref)
    dhq, dsh = ctx.upload(hq), ctx.upload(sh)
    dd = ctx.empty((R, hidden), np.float32)
    NH.call("nh_moe_grouped_gemm_w8a8", ctx.handle, dhq.ptr, dsh.ptr, 0, top_k, d["off"].ptr, d["perm"].ptr, R, R,
            experts, d["down"].ptr, d["sd"].ptr, hidden, inter, 0, dd.ptr, None)
    ctx.synchronize()
    assert np.array_equal(dd.numpy(), d_ref)


# ---- NonFiniteInput from the device quantizers -----------------------------------
def take_nonfinite(ctx, word):
    return NH.call_status("nh_take_nonfinite", ctx.handle, word.ptr, None)


@pytest.mark.parametrize("m,n,k,dtype", [(1, 4096, 4096, "bf16"),    # fused one-row unit
                                         (3, 4096, 8192, "bf16"),    # fused 4-row unit, one N tile per workgroup
                                         (6, 16384, 4096, "bf16"),   # fused streaming unit
                                         (8, 4096, 8192, "bf16"),    # streaming unit, 8 K tiles per wave
                                         (12, 1024, 4096, "bf16"),   # quantizer into activation tiles + GEMV
                                         (2, 1024, 4096, "f32"),     # f32 rows: the row quantizer
                                         (40, 512, 1024, "bf16"),    # quantizer into A tiles + GEMM
                                         (41, 512, 1024, "f32"),     # the same, f32 rows, a partial 8-row group
                                         (300, 256, 21504, "bf16"),  # long rows: a workgroup per row, re-read tail
                                         (20, 256, 21504, "f32")])   # long rows: 1024 threads per row
def test_linear_nonfinite_input_reported(ctx, m, n, k, dtype):
    """A NaN or infinity in x: nh_take_nonfinite returns NonFiniteInput with
    the oracle's first non-finite index (row-major) and value, then the word is
    clear; a finite call leaves it clear."""
    note(f"linear nonfinite m={m} n={n} k={k} {dtype}")
    _, wq, sw = quantized_weights(n, k)
    xf = O.normal_f32(60 + m, m * k).reshape(m, k)
    xf[m - 1, 5] = np.inf
    xf[m // 2, k - 3] = np.nan
    xf[m // 2, k - 1] = -np.inf
    x = O.to_bf16(xf) if dtype == "bf16" else xf
    st, _, _, oerr = O.quantize_rows_bf16(x) if dtype == "bf16" else O.quantize_rows_f32(x)
    assert st == O.NON_FINITE_INPUT
    dx, dw, ds = ctx.upload(x), ctx.upload(tile_16x64(wq)), ctx.upload(sw)
    word = ctx.upload(np.zeros(1, dtype=np.uint64))
    ws_bytes = NH.lib().nh_linear_w8a8_workspace_size(m, k)
    ws = ctx.empty(max(ws_bytes, 1), np.uint8)
    out = ctx.empty((m, n), np.uint16)
    dt = NH.BF16 if dtype == "bf16" else NH.F32
    NH.call("nh_linear_w8a8", ctx.handle, dx.ptr, dt, dw.ptr, ds.ptr, None, m, n, k, out.ptr, NH.BF16, ws.ptr,
            ws_bytes, None, None, word.ptr, None)
    st, err = take_nonfinite(ctx, word)
    assert st == NH.NON_FINITE_INPUT
    first = int(np.flatnonzero(~np.isfinite(xf))[0])
    assert err.argument == b"input" and err.index == oerr.index == first
    want = xf.flat[first]
    assert (np.isnan(err.value) and np.isnan(want)) or err.value == want
    assert take_nonfinite(ctx, word)[0] == NH.OK  # cleared
    xc = np.where(np.isfinite(xf), xf, 0.0).astype(np.float32)
    dxc = ctx.upload(O.to_bf16(xc) if dtype == "bf16" else xc)
    NH.call("nh_linear_w8a8", ctx.handle, dxc.ptr, dt, dw.ptr, ds.ptr, None, m, n, k, out.ptr, NH.BF16, ws.ptr,
            ws_bytes, None, None, word.ptr, None)
    assert take_nonfinite(ctx, word)[0] == NH.OK
    assert np.array_equal(word.numpy(), np.zeros(1, dtype=np.uint64))


@pytest.mark.parametrize("m,n,k,bad", [(8, 1024, 8192, [(5, 7)]),            # groups of 4 rows: row 5 is group 2
                                       (8, 1024, 8192, [(6, 3), (2, 100)]),  # the earlier group's index wins
                                       (6, 1024, 4096, [(4, 9)])])          # the streaming unit (one launch)
def test_linear_w4a8_nonfinite_input_reported(ctx, m, n, k, bad):
    """nh_linear_w4a8 reports a non-finite activation at its index in the
    whole input, also where it runs the rows in groups of 4 launches
    (K = 8192): a NaN in row 5 is reported as 5 K + c, not as its index inside
    the second group."""
    note(f"linear_w4a8 nonfinite m={m} n={n} k={k} bad={bad}")
    zp, scale = 8, 0.01
    packed = np.random.default_rng(m).integers(0, 256, size=(k * n + 1) // 2, dtype=np.uint8)
    xf = O.normal_f32(70 + m, m * k).reshape(m, k)
    for r, c in bad:
        xf[r, c] = np.nan
    x = O.to_bf16(xf)
    first = int(np.flatnonzero(~np.isfinite(O.bf16_to_f32(x)))[0])
    assert first == min(r * k + c for r, c in bad)
    tiled_len = NH.lib().nh_tiled_int4_weights_bytes(n, k)
    dpk = ctx.upload(packed)
    dt4 = ctx.empty(tiled_len, np.uint8)
    NH.call("nh_tile_weights_int4", ctx.handle, dpk.ptr, packed.size, k, n, zp, dt4.ptr, tiled_len, None)
    dx = ctx.upload(x)
    word = ctx.upload(np.zeros(1, dtype=np.uint64))
    ws_bytes = NH.lib().nh_linear_w4a8_workspace_size(m, n, k)
    ws = ctx.empty(max(ws_bytes, 1), np.uint8)
    out = ctx.empty((m, n), np.uint16)
    NH.call("nh_linear_w4a8", ctx.handle, dx.ptr, NH.BF16, dt4.ptr, ctypes.c_float(scale), zp, None, m, n, k,
            out.ptr, NH.BF16, ws.ptr, ws_bytes, word.ptr, None)
    st, err = take_nonfinite(ctx, word)
    assert st == NH.NON_FINITE_INPUT
    assert err.argument == b"input" and err.index == first
    assert np.isnan(err.value)
    assert take_nonfinite(ctx, word)[0] == NH.OK  # cleared


@pytest.mark.parametrize("m", [2, 6])
def test_mlp_nonfinite_intermediate_and_input_reported(ctx, m):
    """The MLP's f32 intermediate overflows (ReLU^2 of a 3e38 biased output is
    +inf): reported as "intermediate" at its row-major index; a NaN in x takes
    precedence as "input".  m = 6: the intermediate's quantizer works from the
    up projection's per-workgroup row maxima."""
    hidden, inter = 512, 1024
    note(f"mlp nonfinite m={m}")
    w_up, s_up, w_down, s_down = mlp_weights(hidden, inter)
    b_up = np.zeros(inter, dtype=np.float32)
    b_up[3] = 3e38
    x = activations_bf16(m, hidden, seed=70)
    d = {nm: ctx.upload(a) for nm, a in dict(x=x, bu=b_up, wu=tile_16x64(w_up), su=s_up, wd=tile_16x64(w_down),
                                               sd=s_down).items()}
    ws_bytes = NH.lib().nh_mlp_w8a8_workspace_size(m, hidden, inter)
    ws = ctx.empty(ws_bytes, np.uint8)
    out = ctx.empty((m, hidden), np.uint16)
    word = ctx.upload(np.zeros(1, dtype=np.uint64))

    def run(dx):
        NH.call("nh_mlp_w8a8", ctx.handle, dx.ptr, NH.BF16, d["wu"].ptr, d["su"].ptr, d["bu"].ptr, d["wd"].ptr,
                d["sd"].ptr, None, m, hidden, inter, out.ptr, NH.BF16, ws.ptr, ws_bytes, word.ptr, None)
        return take_nonfinite(ctx, word)

    st, err = run(d["x"])
    assert st == NH.NON_FINITE_INPUT and err.argument == b"intermediate" and err.index == 3
    assert np.isinf(err.value) and err.value > 0
    xb = x.copy()
    xb[1, 17] = O.to_bf16(np.array([np.nan], dtype=np.float32))[0]
    st, err = run(ctx.upload(xb))
    assert st == NH.NON_FINITE_INPUT and err.argument == b"input" and err.index == hidden + 17


def test_stream_read_diagnostic_reads_and_leaves_the_sink(ctx):
    """nh_stream_read over a buffer of ones: returns OK, writes nothing
    (the data's XOR is not the magic value), rejects unaligned sizes."""
    note("stream read diagnostic")
    src = ctx.upload(np.ones(1 << 22, dtype=np.int32))
    sink = ctx.upload(np.zeros(256, dtype=np.int32))
    NH.call("nh_stream_read", ctx.handle, src.ptr, 16 << 20, sink.ptr, None)
    ctx.synchronize()
    assert not sink.numpy().any()
    err = NH.NhError()
    assert NH.lib().nh_stream_read(ctx.handle, src.ptr, 17, sink.ptr, None, ctypes.byref(err)) == NH.INVALID_SHAPE


def test_moe_nonfinite_intermediate_reported(ctx):
    """An expert's up output overflows (a 3e38 weight scale): the fused up
    epilogue reports it as "intermediate" at its index into the
    [routes][inter] up output in slot order, the lowest such index; the down
    projection requantizes the finite rows as before."""
    tokens, hidden, inter, experts, top_k = 13, 64, 32, 8, 3
    note("moe nonfinite intermediate")
    x, logits, up, su, down, sd = moe_case(tokens, hidden, inter, experts, top_k)
    _, idx, w, _ = O.route_sigmoid(logits, tokens, experts, top_k, renormalize=True)
    offsets, perm, pos = O.moe_permute(idx, tokens, top_k, experts)
    e = int(np.argmax(np.diff(offsets)))  # the busiest expert
    su2 = su.copy()
    su2[e, 5] = 3e38
    _, xq, sx, _ = O.quantize_rows_bf16(x)
    h = O.moe_grouped(xq, sx, True, top_k, offsets, perm, up, su2, relu2=True)
    bad = np.flatnonzero(~np.isfinite(h.ravel()))
    assert bad.size > 0
    ws_bytes = NH.lib().nh_moe_forward_w8a8_workspace_size(tokens, hidden, inter, experts, top_k)
    ws = ctx.empty(ws_bytes, np.uint8)
    dx, dl = ctx.upload(x), ctx.upload(logits)
    dup, dsu, ddown, dsd = ctx.upload(tile_experts(up)), ctx.upload(su2), ctx.upload(tile_experts(down)), ctx.upload(sd)
    out = ctx.empty((tokens, hidden), np.uint16)
    word = ctx.upload(np.zeros(1, dtype=np.uint64))
    NH.call("nh_moe_forward_w8a8", ctx.handle, dx.ptr, NH.BF16, dl.ptr, tokens, hidden, inter, experts, top_k, 1, 1.0,
            dup.ptr, dsu.ptr, ddown.ptr, dsd.ptr, None, out.ptr, NH.BF16, ws.ptr, ws_bytes, word.ptr, None)
    st, err = take_nonfinite(ctx, word)
    assert st == NH.NON_FINITE_INPUT and err.argument == b"intermediate" and err.index == bad[0]
    assert np.isinf(err.value) and err.value > 0
    # the word was cleared: a clean call reports nothing
    dsu_clean = ctx.upload(su)
    NH.call("nh_moe_forward_w8a8", ctx.handle, dx.ptr, NH.BF16, dl.ptr, tokens, hidden, inter, experts, top_k, 1, 1.0,
            dup.ptr, dsu_clean.ptr, ddown.ptr, dsd.ptr, None, out.ptr, NH.BF16, ws.ptr, ws_bytes, word.ptr, None)
    st, _ = take_nonfinite(ctx, word)
    assert st == NH.OK


def test_moe_nonfinite_input_reported(ctx):
    tokens, hidden, inter, experts, top_k = 13, 64, 32, 8, 3
    note("moe nonfinite")
    x, logits, up, su, down, sd = moe_case(tokens, hidden, inter, experts, top_k)
    xb = x.copy()
    xb[5, 10] = O.to_bf16(np.array([-np.inf], dtype=np.float32))[0]
    ws_bytes = NH.lib().nh_moe_forward_w8a8_workspace_size(tokens, hidden, inter, experts, top_k)
    ws = ctx.empty(ws_bytes, np.uint8)
    dx, dl = ctx.upload(xb), ctx.upload(logits)
    dup, dsu, ddown, dsd = ctx.upload(tile_experts(up)), ctx.upload(su), ctx.upload(tile_experts(down)), ctx.upload(sd)
    out = ctx.empty((tokens, hidden), np.uint16)
    word = ctx.upload(np.zeros(1, dtype=np.uint64))
    NH.call("nh_moe_forward_w8a8", ctx.handle, dx.ptr, NH.BF16, dl.ptr, tokens, hidden, inter, experts, top_k, 1, 1.0,
            dup.ptr, dsu.ptr, ddown.ptr, dsd.ptr, None, out.ptr, NH.BF16, ws.ptr, ws_bytes, word.ptr, None)
    st, err = take_nonfinite(ctx, word)
    assert st == NH.NON_FINITE_INPUT and err.argument == b"input" and err.index == 5 * hidden + 10
    assert np.isinf(err.value) and err.value < 0
