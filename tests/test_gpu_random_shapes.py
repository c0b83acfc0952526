"""Seeded random shapes through the linear, MLP, W4A8 and MoE entry points,
checked against the oracle bit-exactly (the bar of test_gpu_parity.py).

The fixed-shape tests pin each kernel at the shapes it was written for; these
draws cross the dispatch boundaries in combinations nobody picked: rows across
1..16 (the one-tile, wide and streaming decode units, the two-launch GEMV),
17..513 (the GEMM on 64 x 128, 128 x 128 and 256 x 128 tiles), K on both sides
of 512-multiples, 4096 and 8192, ragged N from one tile to several rounds of
CUs, bf16 and f32 rows, bf16 and f32 outputs, with and without bias; MoE
layers from 2 to 160 experts, top-1..8, with and without renormalization and
routed scaling, several passes of rows per expert.  Each case is reproducible
from its index (numpy's default_rng(seed)).
"""
import sys

import numpy as np
import pytest

import nemotron_hip as NH
import oracle_ctypes as O
from exact_int import linear_w8a8_exact
from tiling import tile_16x64, tile_int4

pytestmark = pytest.mark.gpu

M_CHOICES = [1, 1, 2, 3, 4, 5, 6, 7, 8, 8, 9, 12, 16, 17, 24, 64, 100, 256, 300, 513]
K_CHOICES = [64, 128, 448, 512, 1024, 1040, 2048, 3072, 4096, 4096, 4160, 6144, 8192, 8256, 12288]


def note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = NH.Context(0)
    yield c
    c.close()


def draw_n(rng, wide):
    if wide:  # several rounds of N tiles over the CUs, ragged last tile
        return int(rng.integers(256, 1500)) * 16 + int(rng.choice([0, 0, 5, 11]))
    return int(rng.integers(1, 48)) * 16 + int(rng.choice([0, 0, 3, 9]))


def draw_linear(i):
    rng = np.random.default_rng(7000 + i)
    while True:
        m, k = int(rng.choice(M_CHOICES)), int(rng.choice(K_CHOICES))
        n = draw_n(rng, rng.random() < 0.35)
        if m * n * k <= 4_000_000_000:
            break
    dtype = "f32" if rng.random() < 0.2 else "bf16"
    out_bf16 = bool(rng.random() < 0.5)
    with_bias = bool(rng.random() < 0.5)
    return m, n, k, dtype, out_bf16, with_bias, int(rng.integers(0, 1 << 30))


@pytest.mark.parametrize("case", range(40))
def test_linear_random_shapes_bit_exact(ctx, case):
    m, n, k, dtype, out_bf16, with_bias, seed = draw_linear(case)
    note(f"random linear #{case}: m={m} n={n} k={k} {dtype} out={'bf16' if out_bf16 else 'f32'} bias={with_bias}")
    w = O.normal_f32(seed, n * k, 0.0, 0.02).reshape(n, k)
    st, wq, sw, _ = O.quantize_rows_f32(w)
    assert st == O.OK
    bias = O.normal_f32(seed + 1, n, 0.0, 0.1) if with_bias else None
    if dtype == "bf16":
        x, xdt = O.to_bf16(O.normal_f32(seed + 2, m * k)).reshape(m, k), NH.BF16
        _, xq_ref, sx_ref, _ = O.quantize_rows_bf16(x)
    else:
        x, xdt = O.normal_f32(seed + 2, m * k).reshape(m, k), NH.F32
        _, xq_ref, sx_ref, _ = O.quantize_rows_f32(x)
    ref = linear_w8a8_exact(xq_ref, sx_ref, wq, sw, bias=bias, out_bf16=out_bf16)
    dx, dw, ds = ctx.upload(x), ctx.upload(tile_16x64(wq)), ctx.upload(sw)
    db = ctx.upload(bias) if bias is not None else None
    ws_bytes = NH.lib().nh_linear_w8a8_workspace_size(m, k)
    ws = ctx.empty(max(ws_bytes, 1), np.uint8)
    ws.fill_bytes(0xa5)  # stale bytes wherever a path leaves padding unwritten
    out = ctx.empty((m, n), np.uint16 if out_bf16 else np.float32)
    NH.call("nh_linear_w8a8", ctx.handle, dx.ptr, xdt, dw.ptr, ds.ptr, db.ptr if db else None, m, n, k, out.ptr,
            NH.BF16 if out_bf16 else NH.F32, ws.ptr, ws_bytes, None, None, None, None)
    ctx.synchronize()
    got = out.numpy()
    assert np.array_equal(got if out_bf16 else got.view(np.uint32), ref if out_bf16 else ref.view(np.uint32))


def draw_mlp(i):
    rng = np.random.default_rng(8000 + i)
    while True:
        m = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 16, 20, 64]))
        hidden = int(rng.choice([256, 512, 1024, 2048, 4096]))
        inter = int(rng.integers(4, 160)) * 16  # the down projection's K: a multiple of 16
        if m * hidden * inter <= 1_000_000_000:
            return m, hidden, inter, int(rng.integers(0, 1 << 30))


@pytest.mark.parametrize("case", range(12))
def test_mlp_random_shapes_bit_exact(ctx, case):
    m, hidden, inter, seed = draw_mlp(case)
    note(f"random mlp #{case}: m={m} hidden={hidden} inter={inter}")
    w_up = O.normal_f32(seed, inter * hidden, 0.0, 0.02).reshape(inter, hidden)
    w_down = O.normal_f32(seed + 1, hidden * inter, 0.0, 0.02).reshape(hidden, inter)
    _, q_up, s_up, _ = O.quantize_rows_f32(w_up)
    _, q_down, s_down, _ = O.quantize_rows_f32(w_down)
    b_up = O.normal_f32(seed + 2, inter, 0.0, 0.05)
    b_down = O.normal_f32(seed + 3, hidden, 0.0, 0.05)
    x = O.to_bf16(O.normal_f32(seed + 4, m * hidden)).reshape(m, hidden)
    _, xq, sx, _ = O.quantize_rows_bf16(x)
    h = linear_w8a8_exact(xq, sx, q_up, s_up, bias=b_up, relu2=True)
    st, hq, sh, _ = O.quantize_rows_f32(h)
    assert st == O.OK
    ref = linear_w8a8_exact(hq, sh, q_down, s_down, bias=b_down, out_bf16=True)
    dx, dbu, dbd = ctx.upload(x), ctx.upload(b_up), ctx.upload(b_down)
    dwu, dsu = ctx.upload(tile_16x64(q_up)), ctx.upload(s_up)
    dwd, dsd = ctx.upload(tile_16x64(q_down)), ctx.upload(s_down)
    ws_bytes = NH.lib().nh_mlp_w8a8_workspace_size(m, hidden, inter)
    ws = ctx.empty(ws_bytes, np.uint8)
    ws.fill_bytes(0xa5)
    out = ctx.empty((m, hidden), np.uint16)
    NH.call("nh_mlp_w8a8", ctx.handle, dx.ptr, NH.BF16, dwu.ptr, dsu.ptr, dbu.ptr, dwd.ptr, dsd.ptr, dbd.ptr,
            m, hidden, inter, out.ptr, NH.BF16, ws.ptr, ws_bytes, None, None)
    ctx.synchronize()
    assert np.array_equal(out.numpy(), ref)


def draw_w4a8(i):
    rng = np.random.default_rng(9000 + i)
    while True:
        m = int(rng.choice([1, 2, 3, 4, 5, 8, 9, 13, 16, 17, 40]))
        k = int(rng.choice([64, 512, 1024, 1040, 2048, 4096, 6144, 8192]))
        n = draw_n(rng, False) + (int(rng.integers(0, 300)) * 16 if rng.random() < 0.3 else 0)
        if m * n * k <= 150_000_000:
            return m, n, k, int(rng.integers(0, 16)), int(rng.integers(0, 1 << 30))


@pytest.mark.parametrize("case", range(12))
def test_linear_w4a8_random_shapes_bit_exact(ctx, case):
    m, n, k, zp, seed = draw_w4a8(case)
    note(f"random w4a8 #{case}: m={m} n={n} k={k} zp={zp}")
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, size=(k * n + 1) // 2, dtype=np.uint8)
    scale = float(np.float32(0.001 + rng.random() * 0.05))
    x = O.to_bf16(O.normal_f32(seed + 1, m * k)).reshape(m, k)
    bias = rng.standard_normal(n).astype(np.float32) if case % 2 else None
    need = NH.lib().nh_tiled_int4_weights_bytes(n, k)
    dp, dt = ctx.upload(packed), ctx.empty(need, np.uint8)
    NH.call("nh_tile_weights_int4", ctx.handle, dp.ptr, packed.size, k, n, zp, dt.ptr, need, None)
    ctx.synchronize()
    assert np.array_equal(dt.numpy(), tile_int4(packed, k, n, zp))
    ws_bytes = NH.lib().nh_linear_w4a8_workspace_size(m, n, k)
    ws = ctx.empty(ws_bytes, np.uint8)
    dx = ctx.upload(x)
    db = ctx.upload(bias) if bias is not None else None
    out = ctx.empty((m, n), np.uint16)
    NH.call("nh_linear_w4a8", ctx.handle, dx.ptr, NH.BF16, dt.ptr, scale, zp, db.ptr if db else None, m, n, k,
            out.ptr, NH.BF16, ws.ptr, ws_bytes, None, None)
    ctx.synchronize()
    st, ref = O.linear_w4a8(x, packed, n, scale, zp, bias=bias, out_bf16=True)
    assert st == O.OK
    assert np.array_equal(out.numpy(), ref)


def draw_moe(i):
    rng = np.random.default_rng(10000 + i)
    while True:
        experts = int(rng.choice([2, 5, 8, 16, 64, 128, 160]))
        top_k = int(rng.integers(1, min(8, experts) + 1))
        tokens = int(rng.integers(1, 600))
        hidden = int(rng.integers(1, 129)) * 16
        inter = int(rng.integers(1, 129)) * 16
        if experts * hidden * inter <= 200_000_000 and tokens * top_k * hidden * inter <= 3_000_000_000:
            break
    renorm = int(rng.random() < 0.7)
    scaling = float(rng.choice([1.0, 2.5]))
    return tokens, hidden, inter, experts, top_k, renorm, scaling, int(rng.integers(0, 1 << 30))


@pytest.mark.parametrize("case", range(10))
def test_moe_forward_random_shapes_bit_exact(ctx, case):
    """nh_moe_forward_w8a8 (route, permute, up with ReLU^2, the fused
    requantization, down, combine) against the oracle's composition."""
    from exact_int import moe_forward_exact
    from tiling import tile_experts
    tokens, hidden, inter, experts, top_k, renorm, scaling, seed = draw_moe(case)
    note(f"random moe #{case}: t={tokens} h={hidden} i={inter} e={experts} k={top_k} renorm={renorm} "
         f"scaling={scaling}")
    rng = np.random.default_rng(seed)
    x = O.to_bf16(O.normal_f32(seed + 1, tokens * hidden)).reshape(tokens, hidden)
    logits = O.normal_f32(seed + 2, tokens * experts)
    up = rng.integers(-127, 128, size=(experts, inter, hidden), dtype=np.int8)
    down = rng.integers(-127, 128, size=(experts, hidden, inter), dtype=np.int8)
    su = rng.uniform(1e-4, 1e-3, size=(experts, inter)).astype(np.float32)
    sd = rng.uniform(1e-4, 1e-3, size=(experts, hidden)).astype(np.float32)
    ref, idx, w, offsets, perm, pos, _, _ = moe_forward_exact(x, logits, up, su, down, sd, top_k,
                                                              renormalize=bool(renorm), scaling=scaling)
    ws_bytes = NH.lib().nh_moe_forward_w8a8_workspace_size(tokens, hidden, inter, experts, top_k)
    ws = ctx.empty(ws_bytes, np.uint8)
    ws.fill_bytes(0xa5)
    dx, dl = ctx.upload(x), ctx.upload(logits)
    dup, dsu, ddown, dsd = ctx.upload(tile_experts(up)), ctx.upload(su), ctx.upload(tile_experts(down)), ctx.upload(sd)
    out = ctx.empty((tokens, hidden), np.uint16)
    NH.call("nh_moe_forward_w8a8", ctx.handle, dx.ptr, NH.BF16, dl.ptr, tokens, hidden, inter, experts, top_k,
            renorm, scaling, dup.ptr, dsu.ptr, ddown.ptr, dsd.ptr, None, out.ptr, NH.BF16, ws.ptr, ws_bytes, None, None)
    ctx.synchronize()
    import ctypes
    lay = (ctypes.c_size_t * 5)()
    NH.lib().nh_moe_workspace_layout(tokens, hidden, inter, experts, top_k, lay)
    wsh = ws.numpy()
    routes = tokens * top_k
    assert np.array_equal(wsh[lay[0]:lay[0] + 4 * routes].view(np.int32), idx)
    assert np.array_equal(wsh[lay[2]:lay[2] + 4 * (experts + 1)].view(np.int32), offsets)
    assert np.array_equal(wsh[lay[3]:lay[3] + 4 * routes].view(np.int32), perm)
    assert np.array_equal(out.numpy(), ref)
