"""Benchmark of the int8 quantized-linear path on one MI355X.

Headline (M=1): the decode unit of an SSM
in_proj-like layer, K=4096 -> N=16384: bf16 activations are quantized per
token and multiplied by int8 per-row weights, bf16 out, in ONE fused gfx950
kernel.  value = algorithmic bytes of the unit / time per unit, in GB/s.
Weights rotate through a >512 MiB pool so the 256 MiB Infinity Cache never
serves them.  The same JSON line also reports the prefill GEMM (M=2048, TOPS
vs the int8 MFMA peak) and the M=2048 linear layer around it (per-token
quantization of bf16 rows + the GEMM), the other decode shapes, the W8A32 GEMV
the MoE layer and the 52-layer decode stack at batch 8, plus
the reference's CPU path timed on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import ctypes
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nemotron-cutile-rs_amd"))

import numpy as np  # noqa: E402

import nemotron_hip as NH  # noqa: E402

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0     # MI355X dense int8 MFMA, published (5.0 POPS)
POOL_BYTES = 640 << 20      # > 512 MiB: weights never resident in the 256 MiB MALL


def decode_bytes(m, n, k):
    # int8 weights + f32 row scales + bf16 activations in + bf16 out + f32 token scales
    return n * k + 4 * n + 2 * m * k + 2 * m * n + 4 * m


class Bench:
    def __init__(self):
        self.ctx = NH.Context(0)
        self.ev = NH.HipEvents()
        self.e0, self.e1 = self.ev.create(), self.ev.create()
        self.last_timing = {}
        self.graphs = NH.HipGraphs()
        s = ctypes.c_void_p()
        NH.call("nh_stream_create", self.ctx.handle, ctypes.byref(s))
        self.stream = s

    def time_ms(self, fn, steps, warmup, per_graph=None, out=None):
        """Mean time per step of fn(i) on self.stream.  `warmup` eager calls;
        then the calls of steps warmup .. warmup + steps - 1 are captured from
        the same entry points into HIP graphs of `per_graph` steps each (the
        replay issues exactly the captured launches, without the ~12 us of
        Python/ctypes work per eager call).  After a synchronize, the graphs
        are replayed back to back on the stream: untimed replays for ~10 ms
        (the warm-up of sustained use), then the timed one between two events.
        The first event fires when the last untimed replay ends, and the timed
        graphs were dispatched while it ran, so the interval holds exactly the
        `steps` timed steps and not the fixed cost of dispatching a graph onto
        an idle stream.  That cold figure (one replay right after a
        synchronize) is kept in self.last_timing.  With `out`, the replayed
        result must equal an eager call of the last step."""
        for i in range(warmup):
            fn(i)
        fn(warmup + steps - 1)
        self.ctx.synchronize(self.stream)
        eager = out.numpy() if out is not None else None
        per = per_graph or steps
        graphs = []
        for c0 in range(0, steps, per):
            idx = range(warmup + c0, warmup + min(steps, c0 + per))
            graphs.append(self.graphs.capture(self.stream, lambda idx=idx: [fn(i) for i in idx]))

        def replay():
            for _, ex in graphs:
                self.graphs.launch(ex, self.stream)

        replay()  # first replay: graph upload and warm-up
        self.ctx.synchronize(self.stream)
        self.ev.record(self.e0, self.stream)
        replay()
        self.ev.record(self.e1, self.stream)
        cold = self.ev.elapsed_ms(self.e0, self.e1)
        self.ctx.synchronize(self.stream)
        # untimed replays back to back for ~10 ms (clocks and power state
        # settle as in sustained use); the last keeps the stream busy while
        # the timed replay is dispatched
        for _ in range(max(1, int(np.ceil(10.0 / max(cold, 1e-3))))):
            replay()
        self.ev.record(self.e0, self.stream)
        replay()
        self.ev.record(self.e1, self.stream)
        hot = self.ev.elapsed_ms(self.e0, self.e1)
        self.ctx.synchronize(self.stream)
        for g, ex in graphs:
            self.graphs.destroy(g, ex)
        if eager is not None and not np.array_equal(out.numpy(), eager):
            raise AssertionError("graph replay differs from the eager call of the same step")
        self.last_timing = {"back_to_back_ms": hot, "after_sync_ms": cold}
        return hot / steps

    def time_eager_ms(self, fn, steps, warmup):
        """The same timing with eager calls from this Python loop (reported
        beside the headline: it includes the per-call host overhead)."""
        for i in range(warmup):
            fn(i)
        self.ctx.synchronize(self.stream)
        self.ev.record(self.e0, self.stream)
        for i in range(steps):
            fn(warmup + i)
        self.ev.record(self.e1, self.stream)
        ms = self.ev.elapsed_ms(self.e0, self.e1)
        self.ctx.synchronize(self.stream)
        return ms / steps

    def quantized_pool(self, n, k, copies, seed=0):
        """copies x (tiled int8 [n][k], f32 [n]) quantized on the device from N(0, 0.02) and tiled
        (nh_quantize_rows_i8 then nh_tile_weights_i8, the offline weight path)."""
        w = NH.normal_f32(seed, n * k, 0.0, 0.02)
        dw = self.ctx.upload(w)
        del w
        q = self.ctx.empty((n, k), np.int8)
        s = self.ctx.empty(n, np.float32)
        NH.call("nh_quantize_rows_i8", self.ctx.handle, dw.ptr, NH.F32, n, k, q.ptr, s.ptr, None, None)
        pool = [(NH.tile_weights(self.ctx, q, n, k), s) for _ in range(copies)]
        self.ctx.synchronize()
        dw.free()
        q.free()
        return pool

    # ---- decode unit ---------------------------------------------------------
    def decode(self, m, n, k, steps, warmup, pool=None, eager_only=False):
        """nh_linear_w8a8 on bf16 rows (bf16 out) over a pool of tiled weights.
        Returns (ms per call, pool, x, out); eager_only times eager calls
        (no graph capture: the profiling runs of the K = 8192 shapes)."""
        copies = max(2, -(-POOL_BYTES // (n * k)))
        pool = pool or self.quantized_pool(n, k, copies)
        x = self.ctx.upload(NH_bf16(NH.normal_f32(1, m * k)).reshape(m, k))
        out = self.ctx.empty((m, n), np.uint16)
        ws_bytes = NH.lib().nh_linear_w8a8_workspace_size(m, k)
        ws = self.ctx.empty(max(ws_bytes, 1), np.uint8)
        L, h = NH.lib(), self.ctx.handle
        err = NH.NhError()

        def step(i):
            q, s = pool[i % len(pool)]
            st = L.nh_linear_w8a8(h, x.ptr, NH.BF16, q.ptr, s.ptr, None, m, n, k, out.ptr, NH.BF16, ws.ptr,
                                  ws_bytes, None, None, None, self.stream, ctypes.byref(err))
            if st:
                NH.check(st, err)

        ms = self.time_eager_ms(step, steps, warmup) if eager_only else self.time_ms(step, steps, warmup, out=out)
        self.last_step = step
        return ms, pool, x, out

    def w4a8(self, m, n, k, steps, warmup, eager_only=False):
        """The W4A8 decode unit (nh_linear_w4a8): bf16 rows quantized per token
        in the GEMV over tiled INT4 weights (per-tensor scale 0.01, zero point
        8), rotating through a > 512 MiB pool of random codes; eager_only
        times eager calls (for tracing)."""
        copies = max(2, -(-POOL_BYTES // (n * k // 2)))
        L, h = NH.lib(), self.ctx.handle
        packed = np.random.default_rng(7).integers(0, 256, size=(k * n + 1) // 2, dtype=np.uint8)
        dp = self.ctx.upload(packed)
        need = L.nh_tiled_int4_weights_bytes(n, k)
        pool = []
        for _ in range(copies):
            t = self.ctx.empty(need, np.uint8)
            NH.call("nh_tile_weights_int4", h, dp.ptr, packed.size, k, n, 8, t.ptr, need, None)
            pool.append(t)
        self.ctx.synchronize()
        dp.free()
        x = self.ctx.upload(NH_bf16(NH.normal_f32(1, m * k)).reshape(m, k))
        out = self.ctx.empty((m, n), np.uint16)
        err = NH.NhError()

        def step(i):
            st = L.nh_linear_w4a8(h, x.ptr, NH.BF16, pool[i % len(pool)].ptr, 0.01, 8, None, m, n, k, out.ptr,
                                  NH.BF16, None, 0, None, self.stream, ctypes.byref(err))
            if st:
                NH.check(st, err)

        if eager_only:
            return self.time_eager_ms(step, steps, warmup)
        return self.time_ms(step, steps, warmup, out=out)

    def gemm(self, m, n, k, steps, warmup):
        """G3 on pre-quantized activations: nh_gemm_w8a8_ta (A in the tiled
        layout, as the linear entry point feeds it) and nh_gemm_w8a8 (row-major
        A).  Returns (ms tiled A, ms row-major A)."""
        (q, s), = self.quantized_pool(n, k, 1)
        xq = self.ctx.upload(np.random.default_rng(1).integers(-127, 128, size=(m, k), dtype=np.int8))
        xt = NH.tile_weights(self.ctx, xq, m, k)
        sx = self.ctx.upload(np.full(m, 0.01, dtype=np.float32))
        out = self.ctx.empty((m, n), np.uint16)
        L, h = NH.lib(), self.ctx.handle
        err = NH.NhError()

        def run(fn, a):
            def step(i):
                st = fn(h, a.ptr, sx.ptr, q.ptr, s.ptr, None, m, n, k, out.ptr, NH.BF16, self.stream,
                        ctypes.byref(err))
                if st:
                    NH.check(st, err)
            return self.time_ms(step, steps, warmup, out=out)

        return run(L.nh_gemm_w8a8_ta, xt), run(L.nh_gemm_w8a8, xq)

    def w8a32(self, n, k, steps, warmup):
        copies = max(2, -(-POOL_BYTES // (n * k)))
        pool = self.quantized_pool(n, k, copies)
        x = self.ctx.upload(NH.normal_f32(1, k))
        y = self.ctx.empty(n, np.float32)
        L, h = NH.lib(), self.ctx.handle
        err = NH.NhError()

        def step(i):
            q, s = pool[i % len(pool)]
            st = L.nh_gemv_w8a32(h, x.ptr, q.ptr, s.ptr, 1, n, k, y.ptr, self.stream, ctypes.byref(err))
            if st:
                NH.check(st, err)

        return self.time_ms(step, steps, warmup, out=y)

    def gemm_f32(self, m, k, n, steps, warmup):
        """G0d: nh_gemm_f32 (f64 accumulation in k order, bit-identical to the
        host GEMM) on N(0, 1) operands.  Returns ms per call."""
        L, h = NH.lib(), self.ctx.handle
        err = NH.NhError()
        lhs = self.ctx.upload(NH.normal_f32(7, m * k))
        rhs = self.ctx.upload(NH.normal_f32(8, k * n))
        out = self.ctx.empty(m * n, np.float32)

        def step(i):
            st = L.nh_gemm_f32(h, lhs.ptr, m * k, rhs.ptr, k * n, m, k, n, out.ptr, m * n, self.stream,
                               ctypes.byref(err))
            if st:
                NH.check(st, err)

        return self.time_ms(step, steps, warmup, out=out)

    def dequant(self, n, k, steps, warmup):
        """Q0d and Q3 on an [n][k] matrix: nh_dequantize_int4 (packed codes,
        one tensor scale and zero point) and nh_dequantize_i8 (row scales), both
        to f32.  Returns (ms int4, ms int8)."""
        L, h = NH.lib(), self.ctx.handle
        err = NH.NhError()
        rng = np.random.default_rng(5)
        packed = self.ctx.upload(rng.integers(0, 256, size=n * k // 2, dtype=np.uint8))
        codes = self.ctx.upload(rng.integers(-127, 128, size=n * k, dtype=np.int8))
        scales = self.ctx.upload(NH.normal_f32(6, n, 0.01, 0.001))
        out = self.ctx.empty(n * k, np.float32)

        def step4(i):
            st = L.nh_dequantize_int4(h, packed.ptr, n * k // 2, n * k, 0.0125, 8, out.ptr, n * k, self.stream,
                                      ctypes.byref(err))
            if st:
                NH.check(st, err)

        def step8(i):
            st = L.nh_dequantize_i8(h, codes.ptr, scales.ptr, n, k, out.ptr, self.stream, ctypes.byref(err))
            if st:
                NH.check(st, err)

        return self.time_ms(step4, steps, warmup, out=out), self.time_ms(step8, steps, warmup, out=out)

    def moe(self, steps, warmup, tokens=512, hidden=2688, inter=1856, experts=128, top_k=6, shared_inter=0,
            router=False):
        """The MoE layer on synthetic expert weights.  With router=True it is
        nh_moe_layer_w8a8, MoeLayer::forward_into from its input: the dense
        f32 router (N(0, 0.02) weights, N(0, 0.1) bias) computes the logits
        on the device first; otherwise the logits are given."""
        L = NH.lib()
        tb_up, tb_down = L.nh_tiled_weights_bytes(inter, hidden), L.nh_tiled_weights_bytes(hidden, inter)
        up_q = self.ctx.empty(experts * tb_up, np.int8)
        down_q = self.ctx.empty(experts * tb_down, np.int8)
        rows_q = self.ctx.empty(inter * hidden, np.int8)
        up_s = self.ctx.empty((experts, inter), np.float32)
        down_s = self.ctx.empty((experts, hidden), np.float32)
        h = self.ctx.handle
        # 8 distinct N(0, 0.02) expert weight sets (seeds 100..107) reused
        # cyclically: the timing does not depend on the values, and drawing
        # 1.28 G normals on the host would dominate the run
        sets = []
        for i in range(8):
            sets.append(self.ctx.upload(NH.normal_f32(100 + i, 2 * inter * hidden, 0.0, 0.02)))
        for e in range(experts):
            dw = sets[e % 8]
            NH.call("nh_quantize_rows_i8", h, dw.ptr, NH.F32, inter, hidden, rows_q.ptr, up_s.offset(4 * e * inter),
                    None, None)
            NH.call("nh_tile_weights_i8", h, rows_q.ptr, inter, hidden, up_q.offset(e * tb_up), tb_up, None)
            NH.call("nh_quantize_rows_i8", h, dw.offset(4 * inter * hidden), NH.F32, hidden, inter, rows_q.ptr,
                    down_s.offset(4 * e * hidden), None, None)
            NH.call("nh_tile_weights_i8", h, rows_q.ptr, hidden, inter, down_q.offset(e * tb_down), tb_down, None)
        self.ctx.synchronize()
        rows_q.free()
        for dw in sets:
            dw.free()
        x = self.ctx.upload(NH_bf16(NH.normal_f32(1, tokens * hidden)))
        logits = self.ctx.upload(NH.normal_f32(2, tokens * experts))
        out = self.ctx.empty((tokens, hidden), np.uint16)
        err = NH.NhError()
        if shared_inter:
            # the shared expert (the reference config's 3712-wide MLP), N(0, 0.02) seeds 120 / 121
            sh = []
            for seed, (n, k) in ((120, (shared_inter, hidden)), (121, (hidden, shared_inter))):
                (q, s_), = self.quantized_pool(n, k, 1, seed=seed)
                sh += [q, s_]
            ws_bytes = L.nh_moe_forward_shared_w8a8_workspace_size(tokens, hidden, inter, experts, top_k,
                                                                   shared_inter)
        else:
            ws_bytes = L.nh_moe_forward_w8a8_workspace_size(tokens, hidden, inter, experts, top_k)
        if router:
            rw = self.ctx.upload(NH.normal_f32(3, hidden * experts, 0.0, 0.02))
            rb = self.ctx.upload(NH.normal_f32(4, experts, 0.0, 0.1))
            ws_bytes = L.nh_moe_layer_w8a8_workspace_size(tokens, hidden, inter, experts, top_k, shared_inter)
        ws = self.ctx.empty(ws_bytes, np.uint8)

        def step(i):
            if router:
                shp = [q.ptr for q in sh] if shared_inter else [None] * 4
                st = L.nh_moe_layer_w8a8(h, x.ptr, NH.BF16, rw.ptr, rb.ptr, tokens, hidden, inter, experts, top_k, 1,
                                         1.0, up_q.ptr, up_s.ptr, down_q.ptr, down_s.ptr, shared_inter, *shp, None, out.ptr,
                                         NH.BF16, ws.ptr, ws_bytes, None, self.stream, ctypes.byref(err))
            elif shared_inter:
                st = L.nh_moe_forward_shared_w8a8(h, x.ptr, NH.BF16, logits.ptr, tokens, hidden, inter, experts, top_k,
                                                  1, 1.0, up_q.ptr, up_s.ptr, down_q.ptr, down_s.ptr, shared_inter,
                                                  sh[0].ptr, sh[1].ptr, sh[2].ptr, sh[3].ptr, None, out.ptr, NH.BF16, ws.ptr,
                                                  ws_bytes, None, self.stream, ctypes.byref(err))
            else:
                st = L.nh_moe_forward_w8a8(h, x.ptr, NH.BF16, logits.ptr, tokens, hidden, inter, experts, top_k, 1,
                                           1.0, up_q.ptr, up_s.ptr, down_q.ptr, down_s.ptr, None, out.ptr, NH.BF16, ws.ptr,
                                           ws_bytes, None, self.stream, ctypes.byref(err))
            if st:
                NH.check(st, err)

        ms = self.time_ms(step, steps, warmup, out=out)
        # weights of the experts that received routes + scales + activations
        wbytes = experts * (inter * hidden + hidden * inter) + experts * 4 * (inter + hidden)
        wbytes += 2 * shared_inter * hidden + 4 * (shared_inter + hidden) if shared_inter else 0
        abytes = tokens * hidden * 2 + tokens * experts * 4 + tokens * hidden * 2
        wbytes += 4 * (hidden * experts + experts) if router else 0
        return ms, wbytes + abytes, 2.0 * tokens * (top_k * inter + shared_inter) * hidden * 2


    def decode_stack(self, steps, warmup, m=8):
        """the 52 linear layers of one decode step of a
        Nemotron-H-8B-like stack at batch m: 24 Mamba blocks (in_proj
        4096 -> 16384, out_proj 8192 -> 4096), 4 attention blocks (qkv
        4096 -> 6144, o 4096 -> 4096) and 24 MLPs (4096 -> 21504 -> 4096,
        nh_mlp_w8a8), every layer with its own tiled int8 weights (6.81 GB
        resident in HBM).  The mixers between the projections (SSM scan,
        attention core) are not part of this path: the out/o projections read
        a fixed bf16 activation of their width.  Returns (ms per step, weight
        + scale bytes per step)."""
        L, h = NH.lib(), self.ctx.handle
        shapes = {"in": (16384, 4096), "out": (4096, 8192), "qkv": (6144, 4096), "o": (4096, 4096),
                  "up": (21504, 4096), "down": (4096, 21504)}
        # 24 x (Mamba, MLP) with an attention block after every 6th pair
        pattern = []
        for i in range(24):
            pattern += ["M", "-"]
            if i % 6 == 5:
                pattern.append("*")
        counts = {"in": 24, "out": 24, "qkv": 4, "o": 4, "up": 24, "down": 24}
        layers, wbytes = {}, 0
        for j, (name, (n, k)) in enumerate(shapes.items()):
            # one N(0, 0.02) matrix per shape, quantized once on the device and
            # tiled into every layer's own buffer
            dw = self.ctx.upload(NH.normal_f32(200 + j, n * k, 0.0, 0.02))
            q = self.ctx.empty((n, k), np.int8)
            s = self.ctx.empty(n, np.float32)
            NH.call("nh_quantize_rows_i8", h, dw.ptr, NH.F32, n, k, q.ptr, s.ptr, None, None)
            dw.free()
            tb = L.nh_tiled_weights_bytes(n, k)
            bufs = []
            for _ in range(counts[name]):
                d = self.ctx.empty(tb, np.int8)
                NH.call("nh_tile_weights_i8", h, q.ptr, n, k, d.ptr, tb, None)
                bufs.append(d)
                wbytes += n * k + 4 * n
            self.ctx.synchronize()
            q.free()
            layers[name] = (bufs, s)
        acts = {w: self.ctx.upload(NH_bf16(NH.normal_f32(300 + w, m * w))) for w in (4096, 8192)}
        outs = {n: self.ctx.empty((m, n), np.uint16) for n in (16384, 6144, 4096)}
        lin_ws = max(L.nh_linear_w8a8_workspace_size(m, k) for (n, k) in shapes.values())
        ws = self.ctx.empty(max(lin_ws, L.nh_mlp_w8a8_workspace_size(m, 4096, 21504)), np.uint8)
        err = NH.NhError()
        eb = ctypes.byref(err)

        def linear(name, idx, x):
            (n, k), (bufs, s) = shapes[name], layers[name]
            st = L.nh_linear_w8a8(h, x.ptr, NH.BF16, bufs[idx].ptr, s.ptr, None, m, n, k, outs[n].ptr, NH.BF16,
                                  ws.ptr, ws.nbytes, None, None, None, self.stream, eb)
            if st:
                NH.check(st, err)

        def step(_):
            cnt = {"M": 0, "*": 0, "-": 0}
            for t in pattern:
                i = cnt[t]
                cnt[t] += 1
                if t == "M":
                    linear("in", i, acts[4096])
                    linear("out", i, acts[8192])
                elif t == "*":
                    linear("qkv", i, acts[4096])
                    linear("o", i, acts[4096])
                else:
                    (bu, su), (bd, sd) = layers["up"], layers["down"]
                    st = L.nh_mlp_w8a8(h, acts[4096].ptr, NH.BF16, bu[i].ptr, su.ptr, None, bd[i].ptr, sd.ptr, None,
                                       m, 4096, 21504, outs[4096].ptr, NH.BF16, ws.ptr, ws.nbytes, None, self.stream,
                                       eb)
                    if st:
                        NH.check(st, err)

        ms = self.time_ms(step, steps, warmup, per_graph=5, out=outs[4096])
        for bufs, s in layers.values():
            for d in bufs:
                d.free()
        return ms, wbytes


def NH_bf16(x):
    """f32 -> bf16 bits, round to nearest even (numpy)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def cpu_model():
    """The host CPU's model string (/proc/cpuinfo), else the platform's."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_threads():
    """Threads for the all-cores baselines: the CPUs this process may use,
    capped at 16 (a one-GPU box's share of the host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def _parallel(fn, items, threads):
    """fn over items on `threads` host threads (the oracle's C calls release
    the GIL), wall time in seconds."""
    from concurrent.futures import ThreadPoolExecutor
    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=threads) as ex:
        list(ex.map(fn, items))
    return time.perf_counter() - t0


def cpu_baselines(budget_s=10.0):
    """The reference's host path on this host, timed on bounded samples
    (restated by the oracle, which is only the checker elsewhere):
    gemm_into_host (f64 accumulation, gemm.rs:91-112) on f32 weights
    materialised from the int8 codes (linear.rs:126-131), and MoeLayer's
    dense experts (moe.rs:207-246: every selected expert's MlpLayer over all
    rows).  Returns (the headline object, the list of all baselines)."""
    import ctypes
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_ctypes as O

    T = cpu_threads()
    model = cpu_model()
    out = []
    # one M=1 decode step, K=4096 -> N=16384
    m, n, k = 1, 16384, 4096
    w = O.normal_f32(0, n * k, 0.0, 0.02).reshape(n, k)
    st, q, s, _ = O.quantize_rows_f32(w)
    del w
    w_mat = np.ascontiguousarray((q.astype(np.float32) * s[:, None]).T)  # [K][N], linear.rs:324 layout
    del q
    x = O.normal_f32(1, m * k)
    runs, t0 = 0, time.perf_counter()
    while True:
        O.gemm_f32(x, w_mat, m, k, n)
        runs += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= budget_s or runs >= 20:
            break
    per1 = elapsed / runs
    out.append({"workload": "decode_m1_k4096_n16384", "value": round(decode_bytes(m, n, k) / per1 / 1e9, 4),
                "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"{runs} full M=1 steps, {per1 * 1e3:.0f} ms/step"})
    # the same step with its output columns split over T threads, every
    # thread walking the one shared [K][N] matrix (the reference's layout and
    # loop; the gain over one core is the threads alone)
    cols = np.array_split(np.arange(n), T)
    yT = np.empty(m * n, dtype=np.float32)
    reps, tt = 0, 0.0
    while tt < budget_s / 2 and reps < 20:
        tt += _parallel(lambda c: O.gemm_f32_col_range(x, w_mat, m, k, n, int(c[0]), int(c[-1]) + 1, yT), cols, T)
        reps += 1
    perT = tt / reps
    out.append({"workload": "decode_m1_k4096_n16384", "value": round(decode_bytes(m, n, k) / perT / 1e9, 4),
                "unit": "GB/s", "cores": T, "kind": "port",
                "sample": f"{reps} full M=1 steps, output columns split over {T} threads on the one shared [K][N] "
                          f"matrix, {perT * 1e3:.0f} ms/step"})
    del w_mat
    # configs[2] first shape: M=2048, K=4096 -> N=4096, timed on T rows (one per thread)
    M2, N2, K2 = 2048, 4096, 4096
    w2 = np.ascontiguousarray(O.normal_f32(3, K2 * N2, 0.0, 0.02).reshape(K2, N2))
    rows = [O.normal_f32(100 + i, K2) for i in range(T)]
    t_rows, nrows = 0.0, 0
    while t_rows < 1.0 and nrows < M2:
        t_rows += _parallel(lambda r: O.gemm_f32(r, w2, 1, K2, N2), rows, T)
        nrows += T
    t_full = t_rows * M2 / nrows
    out.append({"workload": "gemm_m2048_n4096_k4096", "value": round(2 * M2 * N2 * K2 / t_full / 1e12, 6),
                "unit": "TOPS", "cores": T, "kind": "port",
                "sample": f"{nrows} of {M2} rows ({t_rows:.2f} s), extrapolated linearly to all rows: {t_full:.0f} s"})
    del w2, rows
    # MoeLayer::forward_into runs every selected expert's dense
    # f32 MLP over all 512 rows (moe.rs:226-233); timed on T (expert, row)
    # pairs of one expert's weights, extrapolated to 128 experts x 512 rows
    H, I, E, TOK = 2688, 1856, 128, 512
    wu = np.ascontiguousarray(O.normal_f32(4, H * I, 0.0, 0.02))  # [H][I]
    wd = np.ascontiguousarray(O.normal_f32(5, I * H, 0.0, 0.02))  # [I][H]
    lib = O.lib()
    lib.or_mlp_forward.restype = ctypes.c_int
    P = ctypes.c_void_p

    def mlp_row(r):
        o = np.empty(H, dtype=np.float32)
        lib.or_mlp_forward(P(r.ctypes.data), ctypes.c_size_t(1), ctypes.c_size_t(H), ctypes.c_size_t(I),
                           P(wu.ctypes.data), None, P(wd.ctypes.data), None, P(o.ctypes.data))
    rows = [O.normal_f32(200 + i, H) for i in range(T)]
    t_pairs, npairs = 0.0, 0
    while t_pairs < 1.0 and npairs < E * TOK:
        t_pairs += _parallel(mlp_row, rows, T)
        npairs += T
    t_layer = t_pairs * E * TOK / npairs
    moe_bytes = 2 * E * H * I  # the int8 layer's expert weight bytes, the device line's GB/s basis
    out.append({"workload": "moe_512tok_2688h_1856i_128e_top6", "value": round(moe_bytes / t_layer / 1e9, 6),
                "unit": "GB/s", "cores": T, "kind": "port",
                "sample": f"{npairs} (expert, row) dense MLPs ({t_pairs:.2f} s), extrapolated to {E} experts x {TOK} "
                          f"rows (the reference's dense experts; all {E} are selected at top-6 of 512 tokens): "
                          f"{t_layer:.0f} s per layer"})
    # the W8A32 dequant GEMV, K=4096 -> N=4096, one core: the
    # reference's path, materialize_dense then gemm_into_host on [K][N]
    wq = O.normal_f32(6, 4096 * 4096, 0.0, 0.02).reshape(4096, 4096)
    _, q0, s0, _ = O.quantize_rows_f32(wq)
    w0 = np.ascontiguousarray((q0.astype(np.float32) * s0[:, None]).T)
    del wq, q0
    x0 = O.normal_f32(7, 4096)
    runs0, t0 = 0, time.perf_counter()
    while True:
        O.gemm_f32(x0, w0, 1, 4096, 4096)
        runs0 += 1
        t_w32 = (time.perf_counter() - t0) / runs0
        if t_w32 * runs0 >= 1.0 or runs0 >= 20:
            break
    out.append({"workload": "w8a32_gemv_k4096_n4096", "value": round((4096 * 4096 + 3 * 4 * 4096) / t_w32 / 1e9, 4),
                "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"{runs0} full GEMVs (materialised f32 weights, gemm_into_host), {t_w32 * 1e3:.0f} ms each"})
    for b in out:
        b["sample"] += f" ({model})"
    head = dict(out[0])
    head.pop("workload")
    head["sample"] = ("configs[1] decode step K=4096->N=16384 through the oracle's restatement of gemm_into_host "
                      "(f64 accumulation, single-threaded like the reference) on materialised f32 weights [K][N]; "
                      "GB/s counts the int8 unit's algorithmic bytes; " + head["sample"] +
                      f"; {out[1]['cores']} threads on the same matrix: {out[1]['value']} GB/s")
    return head, out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--quick", action="store_true", help="headline only")
    ap.add_argument("--only", choices=["moe", "moe_shared", "moe_router", "gemm", "stack", "decode", "decode_eager",
                                       "w8a32", "w4a8", "w4a8_eager", "dequant", "gemm_f32"],
                    default=None,
                    help="run one secondary workload only (for profiling) and print its figures")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 5 plain device-to-device copies of MIB MiB (torch's copy kernel), the "
                         "calibration run for the FETCH_SIZE / WRITE_SIZE counters, and exit")
    ap.add_argument("--stream", type=int, nargs="+", default=None, metavar="MIB",
                    help="only time one read of MIB MiB with nh_stream_read (the weight streams' load pattern) "
                         "over a 640 MiB pool, the HBM floor of the bandwidth-bound kernels, and exit")
    args = ap.parse_args()
    if args.stream:
        b = Bench()
        L, h = NH.lib(), b.ctx.handle
        err = NH.NhError()
        sink = b.ctx.empty(256, np.int32)
        res = {}
        for mib in args.stream:
            nbytes = mib << 20
            copies = max(2, -(-POOL_BYTES // nbytes))
            pool = b.ctx.empty(copies * nbytes, np.uint8)
            pool.fill_bytes(1)

            def step(i, pool=pool, nbytes=nbytes, copies=copies):
                st = L.nh_stream_read(h, pool.ptr + (i % copies) * nbytes, nbytes, sink.ptr,
                                      b.stream, ctypes.byref(err))
                if st:
                    NH.check(st, err)

            t = b.time_ms(step, max(40, 4 * copies), 5)
            res[f"{mib}MiB"] = {"us": round(t * 1e3, 2), "GBps": round(nbytes / (t * 1e-3) / 1e9, 1),
                                "frac_hbm_peak": round(nbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
            pool.free()
        print(json.dumps({"stream": res}), flush=True)
        return
    if args.copy_probe:
        import torch

        nbytes = args.copy_probe << 20
        src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_read": nbytes, "copy_probe_bytes_written": nbytes, "launches": 5}))
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the int8 linear path has no "
              f"multi-GPU mode in this build", file=sys.stderr)
        sys.exit(2)

    b = Bench()
    if args.only:
        res = {}
        if args.only in ("moe", "moe_shared", "moe_router"):
            t, mbytes, mops = b.moe(10, 2, shared_inter=3712 if args.only == "moe_shared" else 0,
                                    router=args.only == "moe_router")
            res = {"us": round(t * 1e3, 1), "GBps": round(mbytes / (t * 1e-3) / 1e9, 1)}
        elif args.only == "gemm":
            for (mm, nn, kk) in [(2048, 4096, 4096), (2048, 21504, 4096), (2048, 4096, 21504)]:
                t, t_rm = b.gemm(mm, nn, kk, 50, 5)
                t_lin, _, _, _ = b.decode(mm, nn, kk, 50, 5)
                res[f"m{mm}_n{nn}_k{kk}"] = {"us": round(t * 1e3, 1), "row_major_a_us": round(t_rm * 1e3, 1),
                                             "linear_bf16_us": round(t_lin * 1e3, 1)}
        elif args.only == "w4a8":
            for (mm, nn, kk) in [(1, 16384, 4096), (4, 16384, 4096), (8, 16384, 4096), (16, 16384, 4096),
                                 (1, 4096, 8192)]:
                res[f"m{mm}_k{kk}_n{nn}"] = round(b.w4a8(mm, nn, kk, 50, 5) * 1e3, 2)
        elif args.only == "w8a32":
            res = {"us": round(b.w8a32(4096, 4096, 200, 20) * 1e3, 2)}
        elif args.only == "gemm_f32":
            for (mm, kk, nn) in [(512, 2688, 128), (64, 2688, 128), (2048, 4096, 128), (512, 4096, 4096)]:
                res[f"m{mm}_k{kk}_n{nn}"] = round(b.gemm_f32(mm, kk, nn, 20, 3) * 1e3, 1)
        elif args.only == "dequant":
            t4, t8 = b.dequant(4096, 4096, 50, 5)
            res = {"int4_us": round(t4 * 1e3, 2), "i8_us": round(t8 * 1e3, 2)}
        elif args.only == "decode_eager":
            # M = 16 and 8 at 8192 -> 4096 (out_proj), then M = 4, 8 and 16 at
            # 4096 -> 16384 (the streaming unit), eager calls only: 110 each
            for (mm, nn, kk) in [(16, 4096, 8192), (8, 4096, 8192), (4, 16384, 4096), (8, 16384, 4096),
                                 (16, 16384, 4096)]:
                t, _, _, _ = b.decode(mm, nn, kk, 100, 10, eager_only=True)
                res[f"m{mm}_k{kk}_n{nn}_eager"] = round(t * 1e3, 2)
        elif args.only == "w4a8_eager":
            # the W4A8 decode units at 4096 -> 16384, M = 1, 4, 8, 16: eager calls only, 110 each
            for mm in (1, 4, 8, 16):
                res[f"m{mm}_k4096_n16384_eager"] = round(b.w4a8(mm, 16384, 4096, 100, 10, eager_only=True) * 1e3, 2)
        elif args.only == "stack":
            t, sbytes = b.decode_stack(20, 3)
            res = {"ms": round(t, 4), "GBps": round(sbytes / (t * 1e-3) / 1e9, 1)}
        else:
            for (mm, nn, kk) in [(4, 16384, 4096), (8, 16384, 4096), (16, 16384, 4096), (8, 4096, 8192)]:
                t, _, _, _ = b.decode(mm, nn, kk, 50, 5)
                res[f"m{mm}_k{kk}_n{nn}"] = round(t * 1e3, 2)
        print(json.dumps({"only": args.only, **res}), flush=True)
        return
    m, n, k = 1, 16384, 4096
    log = lambda s: print(s, file=sys.stderr, flush=True)  # noqa: E731
    log("[bench] headline decode unit m=1 k=4096 n=16384")
    ms, pool, x, out = b.decode(m, n, k, args.steps, args.warmup)
    head_timing = dict(b.last_timing)
    eager_ms = b.time_eager_ms(b.last_step, args.steps, args.warmup)
    nbytes = decode_bytes(m, n, k)
    gbs = nbytes / (ms * 1e-3) / 1e9
    extra = {}
    if not args.quick:
        sweep = {}
        # (32..128 rows: batched decode on the GEMM's small tiles)
        for (mm, nn, kk) in [(4, 16384, 4096), (8, 16384, 4096), (16, 16384, 4096), (32, 16384, 4096),
                             (64, 16384, 4096), (128, 16384, 4096), (1, 4096, 8192), (4, 4096, 8192),
                             (8, 4096, 8192), (16, 4096, 8192)]:
            log(f"[bench] decode m={mm} k={kk} n={nn}")
            p = pool if (nn, kk) == (n, k) else None
            t, _, _, _ = b.decode(mm, nn, kk, max(20, args.steps), 5, pool=p)
            sweep[f"m{mm}_k{kk}_n{nn}"] = {"us": round(t * 1e3, 2),
                                          "GBps": round(decode_bytes(mm, nn, kk) / (t * 1e-3) / 1e9, 1)}
        extra["decode_sweep"] = sweep
        del pool
        w4 = {}
        for (mm, nn, kk) in [(1, 16384, 4096), (4, 16384, 4096), (8, 16384, 4096), (16, 16384, 4096),
                             (1, 4096, 8192)]:
            log(f"[bench] w4a8 decode m={mm} k={kk} n={nn}")
            t = b.w4a8(mm, nn, kk, max(20, args.steps), 5)
            # int4 codes + bf16 x + bf16 y + f32 token scales (one scale and zero point per tensor)
            wbytes = nn * kk // 2 + 2 * mm * kk + 2 * mm * nn + 4 * mm + 8
            w4[f"m{mm}_k{kk}_n{nn}"] = {"us": round(t * 1e3, 2), "GBps": round(wbytes / (t * 1e-3) / 1e9, 1),
                                        "frac_hbm_peak": round(wbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        extra["w4a8_decode_int4_weights"] = w4
        log("[bench] w8a32 gemv k=4096 n=4096")
        t = b.w8a32(4096, 4096, max(20, args.steps), 5)
        w32_bytes = 4096 * 4096 + 4 * 4096 + 4 * 4096 + 4 * 4096
        extra["w8a32_gemv_k4096_n4096"] = {"us": round(t * 1e3, 2), "GBps": round(w32_bytes / (t * 1e-3) / 1e9, 1)}
        log("[bench] dequantization to f32, 4096 x 4096 (INT4 and int8 codes)")
        t4, t8 = b.dequant(4096, 4096, max(20, args.steps // 10), 5)
        nk = 4096 * 4096
        extra["dequant_f32_4096x4096"] = {
            "int4_us": round(t4 * 1e3, 2), "int4_GBps": round((nk // 2 + 4 * nk) / (t4 * 1e-3) / 1e9, 1),
            "i8_us": round(t8 * 1e3, 2), "i8_GBps": round((nk + 4 * 4096 + 4 * nk) / (t8 * 1e-3) / 1e9, 1)}
        gemms = {}
        for (mm, nn, kk) in [(2048, 4096, 4096), (2048, 21504, 4096), (2048, 4096, 21504)]:
            log(f"[bench] prefill gemm m={mm} n={nn} k={kk}")
            t, t_rm = b.gemm(mm, nn, kk, 50, 5)
            ops = 2.0 * mm * nn * kk
            tops = ops / (t * 1e-3) / 1e12
            gemms[f"m{mm}_n{nn}_k{kk}"] = {"us": round(t * 1e3, 1), "TOPS": round(tops, 1),
                                          "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                                          "row_major_a_us": round(t_rm * 1e3, 1),
                                          "row_major_a_TOPS": round(ops / (t_rm * 1e-3) / 1e12, 1)}
        extra["prefill_gemm"] = gemms
        lins = {}
        for (mm, nn, kk) in [(2048, 4096, 4096), (2048, 21504, 4096), (2048, 4096, 21504)]:
            log(f"[bench] prefill linear layer m={mm} n={nn} k={kk} (bf16 rows quantized per token, then the GEMM)")
            t, _, _, _ = b.decode(mm, nn, kk, 50, 5)
            ops = 2.0 * mm * nn * kk
            lins[f"m{mm}_n{nn}_k{kk}"] = {"us": round(t * 1e3, 1), "TOPS": round(ops / (t * 1e-3) / 1e12, 1),
                                         "frac_int8_peak": round(ops / (t * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4)}
        extra["prefill_linear_bf16"] = lins
        log("[bench] decode stack, 52 layers, m=8")
        t, sbytes = b.decode_stack(20, 3)
        extra["decode_stack_52l_m8"] = {"ms": round(t, 4), "GBps": round(sbytes / (t * 1e-3) / 1e9, 1),
                                        "frac_hbm_peak": round(sbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                        "weight_bytes": sbytes}
        log("[bench] moe layer 512 tokens, 128 experts, top-6")
        t, mbytes, mops = b.moe(40, 3)
        extra["moe_512tok_128exp_top6"] = {"us": round(t * 1e3, 1), "GBps": round(mbytes / (t * 1e-3) / 1e9, 1),
                                           "frac_hbm_peak": round(mbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                           "TOPS": round(mops / (t * 1e-3) / 1e12, 2)}
        log("[bench] moe layer from its input (the dense f32 router on the device)")
        t, mbytes, mops = b.moe(40, 3, router=True)
        extra["moe_layer_with_router_512tok"] = {"us": round(t * 1e3, 1), "GBps": round(mbytes / (t * 1e-3) / 1e9, 1),
                                                 "frac_hbm_peak": round(mbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        log("[bench] moe layer with its 3712-wide shared expert")
        t, mbytes, mops = b.moe(40, 3, shared_inter=3712)
        extra["moe_512tok_128exp_top6_shared3712"] = {
            "us": round(t * 1e3, 1), "GBps": round(mbytes / (t * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round(mbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "TOPS": round(mops / (t * 1e-3) / 1e12, 2)}
    cpu, cpu_all = None, None
    if not args.no_cpu:
        log("[bench] cpu baselines")
        cpu, cpu_all = cpu_baselines()

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "decode_unit_m1_k4096_n16384_traffic.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("hbm_bytes_per_launch")

    line = {
        "metric": "int8 GEMV GB/s (% HBM peak) at M=1; int8 GEMM TOPS (% MFMA peak) at M=2048",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "decode unit (per-token int8 quantization + W8A8 GEMV), M=1, K=4096 -> N=16384, "
                               "bf16 in/out, int8 per-row weights from N(0,0.02) (BASELINE configs[1])",
                   "m": m, "k": k, "n": n, "weight_pool_MiB": POOL_BYTES >> 20,
                   "timing": (f"{args.steps} steps captured in a HIP graph; the timed replay follows ~10 ms "
                              f"of untimed replays back to back on the stream, events around it "
                              f"({head_timing['back_to_back_ms'] * 1e3 / args.steps:.2f} us/step); the same "
                              f"replay launched onto an idle stream after a synchronize "
                              f"{head_timing['after_sync_ms'] * 1e3 / args.steps:.2f} us/step (graph dispatch "
                              f"included); eager Python-loop {eager_ms * 1e3:.2f} us/step")},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "nh_linear_decode_w8a8_m1_kernel", "bytes_per_launch": nbytes},
        "cpu_baseline": cpu,
    }
    if cpu_all is not None:
        line["cpu_baselines"] = cpu_all
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
