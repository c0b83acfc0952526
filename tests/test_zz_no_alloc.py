"""nh_linear_w8a8_noalloc (the allocation-free entry point, static device
scratch as its workspace) against nh_linear_w8a8 with a caller workspace, to
the same bar as every linear test: codes, scales and outputs bit-exact, and
both equal to the oracle."""
import numpy as np
import pytest

import nemotron_hip as NH
import oracle_ctypes as O
from exact_int import linear_w8a8_exact
from tiling import tile_16x64

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = NH.Context(0)
    yield c
    c.close()


def run_pair(ctx, m, n, k, dtype, seed):
    """One call of each entry point on the same inputs; returns both results
    and the oracle's."""
    print(f"[gpu-case] noalloc m={m} n={n} k={k} {dtype}", flush=True)
    w = O.normal_f32(seed, n * k, 0.0, 0.02).reshape(n, k)
    _, wq, sw, _ = O.quantize_rows_f32(w)
    if dtype == "bf16":
        x = O.to_bf16(O.normal_f32(seed + 1, m * k)).reshape(m, k)
        _, xq_ref, sx_ref, _ = O.quantize_rows_bf16(x)
        dt = NH.BF16
    else:
        x = O.normal_f32(seed + 1, m * k).reshape(m, k)
        _, xq_ref, sx_ref, _ = O.quantize_rows_f32(x)
        dt = NH.F32
    bias = O.normal_f32(seed + 2, n, 0.0, 0.1)
    ref = linear_w8a8_exact(xq_ref, sx_ref, wq, sw, bias=bias, out_bf16=True)
    dx, dw, ds, db = ctx.upload(x), ctx.upload(tile_16x64(wq)), ctx.upload(sw), ctx.upload(bias)
    res = []
    for noalloc in (False, True):
        out = ctx.empty((m, n), np.uint16)
        xq = ctx.empty((m, k), np.int8)
        sx = ctx.empty(m, np.float32)
        if noalloc:
            NH.call("nh_linear_w8a8_noalloc", ctx.handle, dx.ptr, dt, dw.ptr, ds.ptr, db.ptr, m, n, k, out.ptr,
                    NH.BF16, xq.ptr, sx.ptr, None, None)
        else:
            ws_bytes = NH.lib().nh_linear_w8a8_workspace_size(m, k)
            ws = ctx.empty(ws_bytes, np.uint8)
            NH.call("nh_linear_w8a8", ctx.handle, dx.ptr, dt, dw.ptr, ds.ptr, db.ptr, m, n, k, out.ptr, NH.BF16,
                    ws.ptr, ws_bytes, xq.ptr, sx.ptr, None, None)
        ctx.synchronize()
        res.append((out.numpy(), xq.numpy(), sx.numpy()))
    return res, (ref, xq_ref, sx_ref)


def test_noalloc_equals_workspace_entry_two_calls_second_smaller(ctx):
    # first call: 300 rows through the GEMM on A tiles in the scratch (2.4 MB
    # of it); second, smaller: 12 rows through the activation tiles + GEMV
    # (the scratch keeps the first call's bytes past what the second writes);
    # third: 12 bf16 rows at K = 8192, the one-launch handoff whose quantizer
    # workgroups write the activation tiles into the scratch
    for (m, n, k, dtype, seed) in [(300, 2048, 8192, "bf16", 80), (12, 1024, 4096, "f32", 90),
                                   (12, 1024, 8192, "bf16", 100)]:
        (a, b), (ref, xq_ref, sx_ref) = run_pair(ctx, m, n, k, dtype, seed)
        assert np.array_equal(b[0], a[0]), f"{(b[0] != a[0]).sum()} outputs differ"
        assert np.array_equal(b[1], a[1]) and np.array_equal(b[2].view(np.uint32), a[2].view(np.uint32))
        assert np.array_equal(a[0], ref)
        assert np.array_equal(a[1], xq_ref) and np.array_equal(a[2].view(np.uint32), sx_ref.view(np.uint32))


def test_noalloc_rejects_a_workspace_above_the_scratch(ctx):
    # 2048 x 32768: 64 MiB of A tiles + the row scales, past the 64 MiB scratch
    st, err = NH.call_status("nh_linear_w8a8_noalloc", ctx.handle, None, NH.BF16, None, None, None, 2048, 64, 32768,
                             None, NH.BF16, None, None, None, None)
    assert st == NH.UNSUPPORTED and b"static scratch" in err.message
