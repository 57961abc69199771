"""Benchmark of the W8A8 linear-layer path on one MI355X.

Headline (``value``): decode GEMV HBM throughput at M=1 over one token's
worth of projections -- BASELINE configs 2 + 3: 36 layers x {qkv 6144x4096,
o 4096x4096, gate_up 24576x4096, down 4096x12288} plus the W8A8 lm_head
151936x4096 with fused greedy argmax -- all with distinct seeded weights
(7.58 GB, far above the 256 MB MALL), activations already quantized to int8
(the metric's byte formula counts int8 activations as the GEMV input).
One step = those 145 launches, captured once in a hip graph and replayed.

    bytes per projection = N*K + 4N + K + 4 + 2N   (weights, scales, q, s, bf16 out)
    lm_head              = N*K + 4N + K + 4 + 4    (token instead of logits)

Also reported (same JSON line): per-shape GEMV GB/s; the same step with a
per-token quantize kernel before every projection; prefill INT8 TOPS at
M=512 and HBM GB/s at M=129 on the four layer shapes (config 4); ragged
M in {4,16,64} for the dot4 GEMV and the MFMA GEMM (config 5); the roofline
of the dominant kernel; and the CPU baseline (the C oracle: quantize +
integer GEMM + epilogue, OpenMP over output channels) timed on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extras] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
WARM_SECONDS = 0.25            # minimum replay time before the timed steps
INT8_PEAK_TOPS = 5000.0        # MI355X dense INT8 MFMA, 5.0 POP/s
SEED_W, SEED_S = 1, 2


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gemv_bytes(n: int, k: int, m: int = 1, out_bytes: int = 2) -> int:
    return n * k + 4 * n + m * k + 4 * m + out_bytes * m * n


def measured_traffic():
    """HBM bytes per gate_up launch from the committed FETCH_SIZE/WRITE_SIZE
    profile (profiles/gemv_m1_gate_up_traffic.txt), or None."""
    f = ROOT / "profiles" / "gemv_m1_gate_up_traffic.txt"
    try:
        for line in f.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def traffic_run() -> int:
    """Workload for the counter passes: 36 gate_up GEMVs (distinct weights),
    three times, eager launches; then a 256 MiB device copy three times as the
    calibration kernel of known traffic (reads and writes 256 MiB)."""
    from inferrous_amd import CudaContext, DeviceBuffer, load, synth
    from inferrous_amd import _lib
    ctx = CudaContext(0)
    mod = load(ctx)
    s = ctx.new_stream()
    n, k = 24576, 4096
    ws_ = []
    for layer in range(synth.LAYERS):
        w = DeviceBuffer.zeroed(s, n * k, np.int8)
        sc = DeviceBuffer.zeroed(s, n, np.float32)
        mod.synth_i8(s, w, SEED_W, synth.weight_stream(layer, 2))
        mod.synth_f32(s, sc, SEED_S, synth.scale_stream(layer, 2), 1e-3, 1e-2)
        ws_.append((w, sc))
    x = DeviceBuffer.from_host(s, synth.normal_rows(40, 1, k).reshape(-1))
    q = DeviceBuffer.zeroed(s, k, np.int8)
    sc1 = DeviceBuffer.zeroed(s, 1, np.float32)
    mod.quantize(s, None, x, k, q, sc1)
    out = DeviceBuffer.zeroed(s, n, np.uint16)
    for _ in range(3):
        for (w, sc) in ws_:
            mod.linear(s, None, q, sc1, w, sc, k, out)
    s.synchronize()
    src = DeviceBuffer.zeroed(s, 256 << 20, np.uint8)
    dst = DeviceBuffer.zeroed(s, 256 << 20, np.uint8)
    for _ in range(3):
        _lib.check(_lib.lib().w8a8_memcpy_dtod(dst.ptr, src.ptr, 256 << 20, s.handle))
    s.synchronize()
    print("traffic run done", flush=True)
    return 0


def packed_head_setup(mod, s, hn):
    """The reference model's BF16 head, packed: 4096 distinct rows of
    N(0, 0.02) weights packed on the host, the packed rows replicated on the
    device up to hn rows (every row streams from HBM; the exception list is
    shared, so offsets repeat), and one activation row."""
    from inferrous_amd import DeviceBuffer, PackedBf16, synth
    from inferrous_amd import _lib as L
    base_rows = 4096
    wbase = (np.random.default_rng(46).standard_normal((base_rows, 4096)).astype(np.float32)
             * np.float32(0.02)).view(np.uint32) >> 16
    pk = PackedBf16.new(wbase.astype(np.uint16))
    words = DeviceBuffer.zeroed(s, hn * 1536, np.uint32)
    wb = DeviceBuffer.from_host(s, pk.words)
    for r0 in range(0, hn, base_rows):
        nr = min(base_rows, hn - r0)
        L.check(L.lib().w8a8_memcpy_dtod(words.ptr + r0 * 1536 * 4, wb.ptr, nr * 1536 * 4, s.handle))
    offs = DeviceBuffer.from_host(s, np.tile(pk.offsets.reshape(base_rows, 16), (hn // base_rows + 1, 1))[:hn]
                                  .reshape(-1))
    exc = DeviceBuffer.from_host(s, pk.exceptions)
    hx = DeviceBuffer.from_host(s, synth.normal_rows(47, 1, 4096).reshape(-1))
    logits = DeviceBuffer.zeroed(s, hn, np.float32)
    s.synchronize()
    return pk, words, offs, exc, hx, logits


def head_profile_run() -> int:
    """Workload for a kernel-trace profile of the packed BF16 head: 20 eager
    head_packed + select_token passes over the 151,936-row head."""
    from inferrous_amd import CudaContext, DeviceBuffer, load, synth
    ctx = CudaContext(0)
    mod = load(ctx)
    s = ctx.new_stream()
    pk, words, offs, exc, hx, logits = packed_head_setup(mod, s, synth.VOCAB)
    token = DeviceBuffer.zeroed(s, 1, np.uint32)
    for _ in range(20):
        mod.head_packed(s, None, hx, words, offs, exc, logits)
        mod.select_token(s, None, logits, token)
    s.synchronize()
    print("head profile done", flush=True)
    return 0


def prefill_profile_run(warm_seconds: float = 0.0) -> int:
    """Workload for a kernel-trace profile of the prefill GEMMs: 8 layers of
    distinct weights (1.5 GB, above the MALL), the four projections at
    M = 512 and M = 129, three eager passes each (no graphs), each M's
    passes preceded by eager passes for warm_seconds (the count is printed,
    so that a summary can skip them); then a 256 MiB device copy three
    times, the calibration kernel of known traffic for counter passes
    (reads and writes 256 MiB)."""
    from inferrous_amd import CudaContext, DeviceBuffer, load, synth
    from inferrous_amd import _lib
    ctx = CudaContext(0)
    mod = load(ctx)
    s = ctx.new_stream()
    nl = 8
    mats = []
    for layer in range(nl):
        for si, (name, n, k) in enumerate(synth.DECODE_SHAPES):
            w = DeviceBuffer.zeroed(s, n * k, np.int8)
            ws = DeviceBuffer.zeroed(s, n, np.float32)
            mod.synth_i8(s, w, SEED_W, synth.weight_stream(layer, si))
            mod.synth_f32(s, ws, SEED_S, synth.scale_stream(layer, si), 1e-3, 1e-2)
            mats.append((name, n, k, w, ws))
    for m in (512, 129):
        pq = {}
        for k, seed in ((4096, 700), (12288, 703)):
            x = synth.student_t_rows(seed, m, k).reshape(-1)
            q = DeviceBuffer.zeroed(s, m * k, np.int8)
            sc = DeviceBuffer.zeroed(s, m, np.float32)
            mod.quantize(s, None, DeviceBuffer.from_host(s, x), k, q, sc)
            pq[k] = (q, sc)
        outs = {name: DeviceBuffer.zeroed(s, m * n, np.uint16) for (name, n, _) in synth.DECODE_SHAPES}

        def one_pass():
            for (name, n, k, w, ws) in mats:
                mod.linear(s, None, pq[k][0], pq[k][1], w, ws, k, outs[name])
        warm, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < warm_seconds:
            one_pass()
            s.synchronize()
            warm += 1
        for _ in range(3):
            one_pass()
        s.synchronize()
        print(f"prefill M={m} done after {warm} warm passes", flush=True)
    src = DeviceBuffer.zeroed(s, 256 << 20, np.uint8)
    dst = DeviceBuffer.zeroed(s, 256 << 20, np.uint8)
    for _ in range(3):
        _lib.check(_lib.lib().w8a8_memcpy_dtod(dst.ptr, src.ptr, 256 << 20, s.handle))
    s.synchronize()
    print("calibration copies done", flush=True)
    return 0


def ragged_profile_run() -> int:
    """Workload for a kernel-trace or counter profile of the ragged small
    batches (config 5): 8 layers of distinct gate_up and down weights (1.2 GB),
    M = 4, 16 and 64 per-row-seeded rows, the dot4 GEMV and the MFMA GEMM
    forced in turn, three eager passes each (no graphs); then a 256 MiB device
    copy three times, the calibration kernel of known traffic for counter
    passes (reads and writes 256 MiB)."""
    from inferrous_amd import CudaContext, DeviceBuffer, load, synth
    from inferrous_amd import _lib
    ctx = CudaContext(0)
    mod = load(ctx)
    s = ctx.new_stream()
    nl = 8
    mats = []
    for layer in range(nl):
        for si in (2, 3):
            name, n, k = synth.DECODE_SHAPES[si]
            w = DeviceBuffer.zeroed(s, n * k, np.int8)
            ws = DeviceBuffer.zeroed(s, n, np.float32)
            mod.synth_i8(s, w, SEED_W, synth.weight_stream(layer, si))
            mod.synth_f32(s, ws, SEED_S, synth.scale_stream(layer, si), 1e-3, 1e-2)
            mats.append((name, n, k, w, ws))
    for m in (4, 16, 64):
        pq, outs = {}, {}
        for (name, n, k, _, _) in mats[:2]:
            x = synth.ragged_rows(range(9000 + 100 * m, 9000 + 100 * m + m), k).reshape(-1)
            q = DeviceBuffer.zeroed(s, m * k, np.int8)
            sc = DeviceBuffer.zeroed(s, m, np.float32)
            mod.quantize(s, None, DeviceBuffer.from_host(s, x), k, q, sc)
            pq[k] = (q, sc)
            outs[name] = DeviceBuffer.zeroed(s, m * n, np.uint16)
        for fam in ("linear_dot4", "linear_mfma"):
            for _ in range(3):
                for (name, n, k, w, ws) in mats:
                    getattr(mod, fam)(s, None, pq[k][0], pq[k][1], w, ws, k, outs[name])
            s.synchronize()
            print(f"ragged M={m} {fam} done", flush=True)
    src = DeviceBuffer.zeroed(s, 256 << 20, np.uint8)
    dst = DeviceBuffer.zeroed(s, 256 << 20, np.uint8)
    for _ in range(3):
        _lib.check(_lib.lib().w8a8_memcpy_dtod(dst.ptr, src.ptr, 256 << 20, s.handle), "memcpy_dtod")
    s.synchronize()
    print("calibration copies done", flush=True)
    return 0


def chain_profile_run() -> int:
    """Workload for a kernel-trace profile of the decode layer chain
    (src/gpu.rs:571-790 order) at M = 1: 8 layers of distinct weights, the
    reference call sequence, the chain with linear_swiglu_quantize, that
    chain with every K = 4096 producer folded into its GEMV, and the same with
    the MLP block as norm_quantize_mlp (the act row tail folded into the down
    GEMV), each captured once and replayed 5 times."""
    from inferrous_amd import CudaContext, DeviceBuffer, Graph, load, synth
    ctx = CudaContext(0)
    mod = load(ctx)
    s = ctx.new_stream()
    nl, ffn, h = 8, 12288, 4096
    layers = []
    for layer in range(nl):
        mats = []
        for si, (name, n, k) in enumerate(synth.DECODE_SHAPES):
            w = DeviceBuffer.zeroed(s, n * k, np.int8)
            ws = DeviceBuffer.zeroed(s, n, np.float32)
            mod.synth_i8(s, w, SEED_W, synth.weight_stream(layer, si))
            mod.synth_f32(s, ws, SEED_S, synth.scale_stream(layer, si), 1e-3, 1e-2)
            mats.append((w, ws))
        (gw, gws) = mats[2]
        halves = (DeviceBuffer.view_of(gw, 0, ffn * h), DeviceBuffer.view_of(gws, 0, ffn),
                  DeviceBuffer.view_of(gw, ffn * h, ffn * h), DeviceBuffer.view_of(gws, ffn, ffn))
        layers.append((mats, halves))
    x = DeviceBuffer.from_host(s, synth.normal_rows(40, 1, h).reshape(-1))
    resid = DeviceBuffer.from_host(s, synth.normal_rows(43, 1, h).reshape(-1))
    gains = [DeviceBuffer.from_host(s, (1 + 0.1 * synth.normal_rows(44 + i, 1, h)).astype(np.float32).reshape(-1))
             for i in range(2)]
    normed = DeviceBuffer.zeroed(s, h, np.float32)
    q4, sc4 = DeviceBuffer.zeroed(s, h, np.int8), DeviceBuffer.zeroed(s, 1, np.float32)
    q12, sc12 = DeviceBuffer.zeroed(s, ffn, np.int8), DeviceBuffer.zeroed(s, 1, np.float32)
    mx = DeviceBuffer.zeroed(s, 1, np.uint32)
    gbuf, ubuf, act = (DeviceBuffer.zeroed(s, ffn, np.float32) for _ in range(3))
    qkv, o, down = (DeviceBuffer.zeroed(s, n, np.uint16) for n in (6144, h, h))
    comb = DeviceBuffer.zeroed(s, h, np.uint16)

    def chain(mode: int):
        # 0: the reference's calls; 1: linear_swiglu_quantize for the MLP
        # pair; 2: every K = 4096 producer folded into its GEMV; 3: and the
        # MLP block in two launches
        for (mats, (wg_, sg_, wu_, su_)) in layers:
            (wqkv, sqkv), (wo, so), _, (wd, sd) = mats
            if mode >= 2:
                mod.norm_quantize_linear(s, None, x, gains[0], normed, q4, sc4, mx, wqkv, sqkv, qkv)
                mod.quantize_linear(s, None, x, q4, sc4, wo, so, o, resid, comb)
                if mode == 3:
                    mod.norm_quantize_mlp(s, None, x, gains[1], normed, q4, sc4, wg_, sg_, gbuf, wu_, su_, ubuf,
                                          act, mx, wd, sd, down, resid, comb, q12, sc12)
                    continue
                mod.norm_quantize_linear_swiglu(s, None, x, gains[1], normed, q4, sc4, wg_, sg_, gbuf, wu_, su_,
                                                ubuf, act, mx, q12, sc12)
                mod.linear_residual(s, None, q12, sc12, wd, sd, ffn, resid, down, comb)
                continue
            else:
                mod.norm_quantize(s, None, x, gains[0], normed, q4, sc4, mx)
                mod.linear(s, None, q4, sc4, wqkv, sqkv, h, qkv)
                mod.quantize(s, None, x, h, q4, sc4)
                mod.linear_residual(s, None, q4, sc4, wo, so, h, resid, o, comb)
            mod.norm_quantize(s, None, x, gains[1], normed, q4, sc4, mx)
            if mode >= 1:
                mod.linear_swiglu_quantize(s, None, q4, sc4, h, wg_, sg_, gbuf, wu_, su_, ubuf, act, mx, q12, sc12)
                mod.linear_residual(s, None, q12, sc12, wd, sd, ffn, resid, down, comb)
            else:
                mod.linear_swiglu(s, None, q4, sc4, h, wg_, sg_, gbuf, wu_, su_, ubuf, act, mx)
                mod.linear_quantize_with_max(s, None, act, ffn, mx, q12, sc12, wd, sd, down, resid, comb)

    for mode, label in ((0, "reference calls"), (1, "fused MLP tail"), (2, "fused producers"),
                        (3, "fused MLP block")):
        chain(mode)
        s.synchronize()
        g = Graph(s)
        with g:
            chain(mode)
        for _ in range(5):
            g.launch()
        s.synchronize()
        print(f"chain profile ({label}) done", flush=True)
    return 0


def timeline_run() -> int:
    """Where a decode GEMV launch spends its time, without a profiler.  For
    each decode shape, 36 distinct-weight launches of the timed one-matrix
    M = 1 GEMV (w8a8_diag_linear_timeline: the kernel body and launch shape
    of w8a8_linear, plus per-wave stamps of the 100 MHz device clock) are
    captured as one graph and replayed 20 times.  From the last replay, per
    launch: `gap`, the previous launch's last wave end to this launch's first
    wave start; `first` and `last`, the first wave start to the first and to
    the last wave whose loads have all landed; `tail`, the last landing to
    the last acknowledged store; `launch`, end to end; `TB/s`, the launch's
    bytes over `last`.  Medians over launches 2..35; one line per shape."""
    from inferrous_amd import CudaContext, DeviceBuffer, Graph, load, synth
    from inferrous_amd import _lib
    ctx = CudaContext(0)
    mod = load(ctx)
    s = ctx.new_stream()
    L = _lib.lib()
    nl, tick_us = 36, 0.01   # s_memrealtime: 100 MHz
    print(f"{'shape':8s} {'N x K':>12s} {'waves':>6s} {'gap':>6s} {'first':>6s} {'last':>6s} {'tail':>6s} "
          f"{'launch':>7s} {'TB/s':>6s}   (us, medians of launches 2..35)", flush=True)
    for si, (name, n, k) in enumerate(synth.DECODE_SHAPES):
        mats = []
        for layer in range(nl):
            w = DeviceBuffer.zeroed(s, n * k, np.int8)
            ws = DeviceBuffer.zeroed(s, n, np.float32)
            mod.synth_i8(s, w, SEED_W, synth.weight_stream(layer, si))
            mod.synth_f32(s, ws, SEED_S, synth.scale_stream(layer, si), 1e-3, 1e-2)
            mats.append((w, ws))
        x = DeviceBuffer.from_host(s, synth.normal_rows(40, 1, k).reshape(-1))
        q, sc = DeviceBuffer.zeroed(s, k, np.int8), DeviceBuffer.zeroed(s, 1, np.float32)
        mod.quantize(s, None, x, k, q, sc)
        out = DeviceBuffer.zeroed(s, n, np.uint16)
        need = L.w8a8_diag_linear_timeline_stamps(n, k)
        stamps = DeviceBuffer.zeroed(s, nl * need, np.uint64)

        def launches():
            for i, (w, ws) in enumerate(mats):
                _lib.check(L.w8a8_diag_linear_timeline(s.handle, q.ptr, sc.ptr, w.ptr, ws.ptr, n, k, out.ptr,
                                                       _lib.OUT_BF16, stamps.ptr + i * need * 8, need),
                           "diag_linear_timeline")
        launches()
        s.synchronize()
        g = Graph(s)
        with g:
            launches()
        for _ in range(20):
            g.launch()
        s.synchronize()
        t = stamps.to_host_vec(s).astype(np.int64).reshape(nl, need // 3, 3)
        start, landed, end = t[:, :, 0].min(1), t[:, :, 1], t[:, :, 2].max(1)
        first, last = landed.min(1), landed.max(1)
        gap = (start[1:] - end[:-1])[1:] * tick_us
        to_first = (first - start)[2:] * tick_us
        to_last = (last - start)[2:] * tick_us
        tail = (end - last)[2:] * tick_us
        launch = (end[1:] - end[:-1])[1:] * tick_us
        med = lambda a: float(np.median(a))
        rate = gemv_bytes(n, k) / (med(to_last) * 1e-6) / 1e12
        print(f"{name:8s} {n:>5d} x {k:<5d} {need // 3:6d} {med(gap):6.2f} {med(to_first):6.2f} {med(to_last):6.2f} "
              f"{med(tail):6.2f} {med(launch):7.2f} {rate:6.2f}", flush=True)
        del mats, stamps, g
    return 0


def gemm_timeline_run() -> int:
    """Where a gemm_tall launch spends its time (M = 129 on the four layer
    shapes, the ragged M = 24 / 64 down and M = 16 gate_up), without a
    profiler.  For each shape, 36 distinct-weight launches of
    w8a8_diag_gemm_timeline (the kernel and launch of w8a8_linear_ex's
    gemm_tall route with per-wave stamps of the 100 MHz clock, and the same
    split-K slab epilogue launch) are captured as one graph and replayed 20
    times; the last replay is read.  Per launch, medians of launches 2..35,
    in us from the launch's first wave start: `prologue`, the median and the
    last wave to have stage 0 of both rings landed; `stream`, the median and
    the last wave to have issued its last MFMA (or DMA, for waves holding no
    rows); `end`, the last store acknowledged; `between`, this launch's end to
    the next launch's first wave (the slab epilogue launch and two launch
    gaps for a split route, one gap otherwise); `period`, end to end.  The
    per-CU pull model: each workgroup's (rows loaded + BN) x K range bytes
    at 30 B/clk and the clock the stamps imply.  `plain us`: the same graph
    through w8a8_linear_ex."""
    from inferrous_amd import CudaContext, DeviceBuffer, Event, Graph, load, synth
    from inferrous_amd import _lib
    ctx = CudaContext(0)
    mod = load(ctx)
    s = ctx.new_stream()
    L = _lib.lib()
    nl, tick_us = 36, 0.01
    shapes = [(129, si) for si in range(4)] + [(24, 3), (64, 3), (16, 2)]
    print(f"{'shape':14s} {'M':>4s} {'WGs':>4s} {'split':>5s} {'prologue':>13s} {'stream':>13s} {'end':>6s} "
          f"{'between':>7s} {'period':>6s} {'plain us':>8s} {'pull us':>7s} {'HBM us':>6s}   "
          f"(us, medians of launches 2..35; med/last wave)", flush=True)
    for m, si in shapes:
        name, n, k = synth.DECODE_SHAPES[si]
        mats = []
        for layer in range(nl):
            w = DeviceBuffer.zeroed(s, n * k, np.int8)
            ws = DeviceBuffer.zeroed(s, n, np.float32)
            mod.synth_i8(s, w, SEED_W, synth.weight_stream(layer, si))
            mod.synth_f32(s, ws, SEED_S, synth.scale_stream(layer, si), 1e-3, 1e-2)
            mats.append((w, ws))
        x = synth.student_t_rows(700 + si, m, k)
        q, sc = DeviceBuffer.zeroed(s, m * k, np.int8), DeviceBuffer.zeroed(s, m, np.float32)
        mod.quantize(s, None, DeviceBuffer.from_host(s, x.reshape(-1)), k, q, sc)
        out = DeviceBuffer.zeroed(s, m * n, np.uint16)
        wsb = int(L.w8a8_linear_workspace_bytes(m, n, k))
        work = DeviceBuffer.zeroed(s, max(wsb, 16), np.uint8)
        need = int(L.w8a8_diag_gemm_timeline_stamps(m, n, k, wsb))
        if need == 0:
            print(f"{name:14s} {m:4d}: not a gemm_tall route", flush=True)
            continue
        stamps = DeviceBuffer.zeroed(s, nl * need, np.uint64)
        route = np.zeros(20, np.int32)
        _lib.check(L.w8a8_diag_linear_route(m, n, k, _lib.OUT_BF16, 0, 0, wsb, route.ctypes.data, 20), "route")
        wgs, splits, bn, ma = int(route[1]), int(route[14]), int(route[5]), int(route[10])

        def launches():
            for i, (w, ws) in enumerate(mats):
                _lib.check(L.w8a8_diag_gemm_timeline(s.handle, q.ptr, sc.ptr, m, w.ptr, ws.ptr, n, k, out.ptr,
                                                     work.ptr, wsb, stamps.ptr + i * need * 8, need),
                           "diag_gemm_timeline")

        def plain():
            for (w, ws) in mats:
                mod.linear(s, None, q, sc, w, ws, k, out)
        launches()
        s.synchronize()
        g = Graph(s)
        with g:
            launches()
        for _ in range(20):
            g.launch()
        s.synchronize()
        t = stamps.to_host_vec(s).astype(np.int64).reshape(nl, need // 4, 4)
        start, end = t[:, :, 0].min(1), t[:, :, 3].max(1)
        rel = (t - start[:, None, None]) * tick_us
        med = lambda a: float(np.median(a))
        pro_m, pro_x = med(np.median(rel[:, :, 1], 1)[2:]), med(rel[:, :, 1].max(1)[2:])
        st_m, st_x = med(np.median(rel[:, :, 2], 1)[2:]), med(rel[:, :, 2].max(1)[2:])
        e = med(rel[:, :, 3].max(1)[2:])
        between = med(((start[1:] - end[:-1]) * tick_us)[1:])
        period = med(((end[1:] - end[:-1]) * tick_us)[1:])
        plain()  # eager first: reserves the stream's split-K workspace outside capture
        s.synchronize()
        pg = Graph(s)
        with pg:
            plain()
        for _ in range(5):
            pg.launch()
        s.synchronize()
        e0, e1 = Event(), Event()
        e0.record(s)
        for _ in range(20):
            pg.launch()
        e1.record(s)
        e1.synchronize()
        plain_us = e0.elapsed_ms(e1) * 1e3 / 20 / nl
        rows = -(-m // 8) * 8
        pull = wgs * (rows + bn) * (k // splits)            # bytes pulled L2 -> CU
        pull_us = (pull / wgs) / 30.0 / 2.1e3                 # 30 B/clk at 2.1 GHz, per CU
        hbm_us = (n * k + m * k) / 8e12 * 1e6
        print(f"{name:14s} {m:4d} {wgs:4d} {splits:5d} {pro_m:6.2f}/{pro_x:6.2f} {st_m:6.2f}/{st_x:6.2f} {e:6.2f} "
              f"{between:7.2f} {period:6.2f} {plain_us:8.2f} {pull_us:7.2f} {hbm_us:6.2f}", flush=True)
        del mats, stamps, g, pg
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-extras", action="store_true", help="headline + roofline only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--traffic", action="store_true",
                    help="run only the counter-profiling workload (gate_up GEMVs + calibration copy)")
    ap.add_argument("--prefill-profile", action="store_true",
                    help="run only the prefill GEMM workload for a kernel-trace profile")
    ap.add_argument("--head-profile", action="store_true",
                    help="run only the packed BF16 head workload for a kernel-trace profile")
    ap.add_argument("--chain-profile", action="store_true",
                    help="run only the decode layer chain workload for a kernel-trace profile")
    ap.add_argument("--ragged-profile", action="store_true",
                    help="run only the ragged small-batch workload for a kernel-trace profile")
    ap.add_argument("--warm-seconds", type=float, default=0.0,
                    help="--prefill-profile: eager passes before each M's three profiled passes")
    ap.add_argument("--timeline", action="store_true",
                    help="run only the per-wave clock timeline of the decode GEMV launches")
    ap.add_argument("--gemm-timeline", action="store_true",
                    help="run only the per-wave clock timeline of gemm_tall at M = 129 and the ragged batches")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this W8A8 path has no multi-GPU mode "
              "(column/row/vocab sharding is a design note, not built); run with --gpus 1.",
              file=sys.stderr)
        return 2

    if args.traffic:
        return traffic_run()
    if args.prefill_profile:
        return prefill_profile_run(args.warm_seconds)
    if args.head_profile:
        return head_profile_run()
    if args.ragged_profile:
        return ragged_profile_run()
    if args.timeline:
        return timeline_run()
    if args.gemm_timeline:
        return gemm_timeline_run()
    if args.chain_profile:
        return chain_profile_run()

    from inferrous_amd import CudaContext, DeviceBuffer, Event, Graph, load, synth

    ctx = CudaContext(0)
    cu, arch = ctx.info()
    clock_mhz = ctx.clock_khz() / 1e3
    mod = load(ctx)
    s = ctx.new_stream()
    # dense INT8 MFMA peak re-derived from the reported clock: CUs x 4 SIMDs x
    # 2048 ops/clk (v_mfma_i32_32x32x32_i8: 65536 ops in 32 cycles per SIMD)
    int8_peak_derived = cu * 4 * 2048 * clock_mhz * 1e6 / 1e12
    log(f"device {arch} with {cu} CUs at {clock_mhz:.0f} MHz peak; "
        f"INT8 MFMA peak {int8_peak_derived:.0f} TOPS derived, {INT8_PEAK_TOPS:.0f} published")

    # ------------------------------------------------------------ weights
    t0 = time.time()
    layers = []
    for layer in range(synth.LAYERS):
        mats = []
        for si, (name, n, k) in enumerate(synth.DECODE_SHAPES):
            w = DeviceBuffer.zeroed(s, n * k, np.int8)
            ws = DeviceBuffer.zeroed(s, n, np.float32)
            mod.synth_i8(s, w, SEED_W, synth.weight_stream(layer, si))
            mod.synth_f32(s, ws, SEED_S, synth.scale_stream(layer, si), 1e-3, 1e-2)
            mats.append((name, n, k, w, ws))
        layers.append(mats)
    hn, hk = synth.VOCAB, synth.HIDDEN
    head_w = DeviceBuffer.zeroed(s, hn * hk, np.int8)
    head_s = DeviceBuffer.zeroed(s, hn, np.float32)
    mod.synth_i8(s, head_w, SEED_W, 9001)
    mod.synth_f32(s, head_s, SEED_S, 9101, 1e-3, 1e-2)
    s.synchronize()
    weight_bytes = sum(n * k for (_, n, k, _, _) in layers[0]) * synth.LAYERS + hn * hk
    log(f"generated {weight_bytes / 1e9:.2f} GB of int8 weights in {time.time() - t0:.1f}s")

    # ------------------------------------------------------------ activations
    xs, qs = {}, {}
    for k, seed in ((4096, 40), (12288, 41)):
        x = synth.normal_rows(seed, 1, k).reshape(-1)
        xs[k] = DeviceBuffer.from_host(s, x)
        q = DeviceBuffer.zeroed(s, k, np.int8)
        sc = DeviceBuffer.zeroed(s, 1, np.float32)
        mod.quantize(s, None, xs[k], k, q, sc)
        qs[k] = (q, sc)
    outs = {name: DeviceBuffer.zeroed(s, n, np.uint16) for (name, n, _, _, _) in layers[0]}
    token = DeviceBuffer.zeroed(s, 1, np.uint32)

    def decode_step(with_quant: bool = False):
        for mats in layers:
            for (name, n, k, w, ws) in mats:
                q, sc = qs[k]
                if with_quant:
                    mod.quantize(s, None, xs[k], k, q, sc)
                mod.linear(s, None, q, sc, w, ws, k, outs[name])
        q, sc = qs[hk]
        if with_quant:
            mod.quantize(s, None, xs[hk], hk, q, sc)
        mod.linear_argmax(s, q, sc, head_w, head_s, hk, token)

    step_bytes = sum(gemv_bytes(n, k) for (_, n, k, _, _) in layers[0]) * synth.LAYERS \
        + gemv_bytes(hn, hk, out_bytes=0) + 4

    def capture(fn) -> Graph:
        g = Graph(s)
        with g:
            fn()
        return g

    def time_graph(g: Graph, reps: int, warm: int = 2) -> float:
        """Mean over reps of graph replays, HIP events on `s` (ms), after at
        least `warm` replays and WARM_SECONDS of them.  Measured on MI355X: the
        36-layer prefill graphs timed after one warm replay, with the device
        idle for 0.5 s before (as after the host builds the next inputs), took
        5.02 ms at M = 512 and 2.92 ms at M = 129; after 0.3 s of replays
        4.81-4.83 and 2.65 ms, and the same after a further second."""
        t0 = time.perf_counter()
        done = 0
        while done < warm or time.perf_counter() - t0 < WARM_SECONDS:
            for _ in range(4):
                g.launch()
            done += 4
            s.synchronize()
        e0, e1 = Event(), Event()
        e0.record(s)
        for _ in range(reps):
            g.launch()
        e1.record(s)
        e1.synchronize()
        return e0.elapsed_ms(e1) / reps

    decode_step()          # eager pass: allocates the selection workspace outside capture
    s.synchronize()
    g_step = capture(decode_step)
    # Warm-up: the W requested steps, and at least WARM_SECONDS of replays in
    # all.  Measured on MI355X: after 5 warm-up steps (7 ms) the timed step
    # came out at 1.305-1.335 ms across runs, after 100 at 1.302-1.305 ms --
    # the device leaves its idle power state only after tenths of a second of
    # load.  The timed region below is exactly K steps either way.
    warm_t0 = time.perf_counter()
    warm_run = 0
    while warm_run < args.warmup or time.perf_counter() - warm_t0 < WARM_SECONDS:
        for _ in range(10):
            g_step.launch()
        warm_run += 10
        s.synchronize()
    e0, e1 = Event(), Event()
    t_start = time.perf_counter()
    e0.record(s)
    for _ in range(args.steps):
        g_step.launch()
    e1.record(s)
    s.synchronize()
    t_end = time.perf_counter()
    wall_ms = (t_end - t_start) * 1e3 / args.steps
    ev_ms = e0.elapsed_ms(e1) / args.steps
    value = step_bytes / (wall_ms * 1e-3) / 1e9
    log(f"decode step: {wall_ms * 1e3:.1f} us wall, {ev_ms * 1e3:.1f} us events, "
        f"{value:.0f} GB/s ({value / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)")

    # Dispatch gap between dependent launches in a graph: a chain of 145
    # one-workgroup fill kernels (16 bytes each) -- the floor every kernel
    # boundary of the step pays on this runtime.
    scratch = DeviceBuffer.zeroed(s, 16, np.uint8)
    launches = 4 * synth.LAYERS + 2          # 144 GEMVs + lm_head GEMV + select finalize
    gap_ms = time_graph(capture(lambda: [scratch.fill_zero(s) for _ in range(launches)]), 20)
    gap_us = gap_ms * 1e3 / launches
    in_kernel_gbs = step_bytes / ((ev_ms - gap_ms) * 1e-3) / 1e9
    log(f"dispatch gap {gap_us:.2f} us/launch; in-kernel rate {in_kernel_gbs:.0f} GB/s")

    # ------------------------------------------------------------ roofline
    # Dominant kernel: gemv_m1_one<1,4,0,4>, the gate_up GEMV (24576 x 4096, one row
    # per wave) -- the largest share of the step.  Timed as a graph of the 36
    # distinct-weight launches of one token, HIP events on the launch stream.
    gu = [mats[2] for mats in layers]
    gu_bytes = gemv_bytes(24576, 4096)

    def gate_up_chain():
        for (name, n, k, w, ws) in gu:
            mod.linear(s, None, qs[k][0], qs[k][1], w, ws, k, outs[name])

    dom_ms = time_graph(capture(gate_up_chain), max(10, args.steps // 2))
    dom_avg_us = dom_ms * 1e3 / len(gu)
    dom_gbs = gu_bytes / (dom_avg_us * 1e-6) / 1e9
    roofline = {"kernel": "gemv_m1_one<1,4,0,4> (gate_up 24576x4096, M=1)", "bound": "hbm",
                "achieved": round(dom_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dom_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                "avg_launch_us": round(dom_avg_us, 3), "bytes_per_launch": gu_bytes}
    log(f"dominant GEMV (gate_up): {dom_avg_us:.2f} us/launch avg, {dom_gbs:.0f} GB/s")

    result = {
        "metric": "decode GEMV HBM GB/s (% peak) at M=1; prefill INT8 TOPS (% peak) at M=512",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall_ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic: seeded int8 weights U[-127,127], f32 scales U[1e-3,1e-2], BF16 N(0,1) activations",
        "config": {"workload": "C2+C3 decode: 36 x (qkv 6144x4096, o 4096x4096, gate_up 24576x4096, "
                               "down 4096x12288) + W8A8 lm_head 151936x4096 + fused argmax, M=1",
                   "bytes_per_step": step_bytes, "gemv_launches_per_step": 4 * synth.LAYERS + 1,
                   "pct_hbm_peak": round(value / HBM_PEAK_GBS * 100, 2),
                   "event_ms_per_step": round(ev_ms, 4),
                   "warmup_steps_run": warm_run,
                   "launches_in_graph": launches,
                   "dispatch_gap_us_per_launch": round(gap_us, 3),
                   "in_kernel_GB/s": round(in_kernel_gbs, 1),
                   "in_kernel_pct_hbm_peak": round(in_kernel_gbs / HBM_PEAK_GBS * 100, 2)},
        "roofline": roofline,
    }

    if not args.no_extras:
        extras = {}
        # per-shape GEMV throughput (36 launches each, distinct weights)
        per = {}
        for si, (name, n, k) in enumerate(synth.DECODE_SHAPES):
            def chain(si=si):
                for mats in layers:
                    (nm, nn, kk, w, ws) = mats[si]
                    q, sc = qs[kk]
                    mod.linear(s, None, q, sc, w, ws, kk, outs[nm])
            ms = time_graph(capture(chain), 20)
            us = ms * 1e3 / synth.LAYERS
            per[name] = {"us": round(us, 2), "GB/s": round(gemv_bytes(n, k) / (us * 1e-6) / 1e9, 1)}
        ms = time_graph(capture(lambda: mod.linear_argmax(s, qs[hk][0], qs[hk][1], head_w, head_s,
                                                          hk, token)), 20)
        per["lm_head_argmax"] = {"us": round(ms * 1e3, 2),
                                 "GB/s": round(gemv_bytes(hn, hk, out_bytes=0) / (ms * 1e-3) / 1e9, 1)}
        extras["per_shape_gemv"] = per
        log(f"per shape: {per}")
        # The same 145 projections as one launch (w8a8_linear_sequence: a
        # device-wide barrier between dependent entries, weights requested
        # ahead of it), against the graph of 146 launches above.
        mod.sequence_reset()
        seq_entries = [dict(q=qs[k][0], asc=qs[k][1], w=w, ws=ws, out=outs[name])
                       for mats in layers for (name, n, k, w, ws) in mats]
        seq_entries.append(dict(q=qs[hk][0], asc=qs[hk][1], w=head_w, ws=head_s, out=None, select=True))
        plan = mod.prepare_sequence(seq_entries)
        seq_token = DeviceBuffer.zeroed(s, 1, np.uint32)
        seq_t0, seq_warm = time.perf_counter(), 0
        while seq_warm < 20 or time.perf_counter() - seq_t0 < WARM_SECONDS:
            for _ in range(10):
                mod.linear_sequence(s, plan, seq_token)
            seq_warm += 10
            s.synchronize()
        e0, e1 = Event(), Event()
        e0.record(s)
        for _ in range(50):
            mod.linear_sequence(s, plan, seq_token)
        e1.record(s)
        e1.synchronize()
        ms = e0.elapsed_ms(e1) / 50
        seq_status = mod.sequence_status()
        extras["decode_sequence_one_launch"] = {
            "ms": round(ms, 4), "GB/s": round(step_bytes / (ms * 1e-3) / 1e9, 1), "status": seq_status,
            "token_matches_graph": int(seq_token.to_host_vec(s)[0]) == int(token.to_host_vec(s)[0]),
            "entries": len(seq_entries)}
        log(f"decode step as one sequence launch: {ms * 1e3:.1f} us (status {seq_status})")
        # step including a per-token quantize kernel before every projection
        ms = time_graph(capture(lambda: decode_step(with_quant=True)), 20)
        extras["decode_step_with_quantize"] = {"ms": round(ms, 4),
                                               "GB/s": round(step_bytes / (ms * 1e-3) / 1e9, 1)}
        # The reference's decode layer chain (src/gpu.rs:571-790) with this
        # library's ops: quantize (maxima reset) -> qkv; quantize -> o with
        # residual; quantize (reset) -> linear_swiglu (publishes max |act|)
        # -> quantize_with_max + down with residual.  gate and up
        # are the two halves of the gate_up matrix.  Weight bytes as the
        # headline (the small activation/output traffic is not counted).
        ffn = 12288
        resid = DeviceBuffer.from_host(s, synth.normal_rows(43, 1, 4096).reshape(-1))
        mx = DeviceBuffer.zeroed(s, 1, np.uint32)
        gbuf = DeviceBuffer.zeroed(s, ffn, np.float32)
        ubuf = DeviceBuffer.zeroed(s, ffn, np.float32)
        act = DeviceBuffer.zeroed(s, ffn, np.float32)
        comb = DeviceBuffer.zeroed(s, 4096, np.uint16)
        gains = [DeviceBuffer.from_host(s, (1 + 0.1 * synth.normal_rows(44 + i, 1, 4096)).astype(np.float32)
                                        .reshape(-1)) for i in range(2)]
        normed = DeviceBuffer.zeroed(s, 4096, np.float32)
        q4, sc4 = qs[4096]
        q12, sc12 = qs[12288]
        halves = []
        for mats in layers:
            (_, _, _, gw, gws) = mats[2]
            halves.append((DeviceBuffer.view_of(gw, 0, ffn * 4096), DeviceBuffer.view_of(gws, 0, ffn),
                           DeviceBuffer.view_of(gw, ffn * 4096, ffn * 4096),
                           DeviceBuffer.view_of(gws, ffn, ffn)))

        def layer_chain(fused_mlp: bool = False, fused_producers: bool = False, mlp_bufs=None):
            gb_, ub_, ab_ = mlp_bufs or (gbuf, ubuf, act)
            for mats, (wg_, sg_, wu_, su_) in zip(layers, halves):
                (_, _, _, wqkv, sqkv), (_, _, _, wo, so), _, (_, _, _, wd, sd) = mats
                if fused_producers:
                    # norm_quantize + qkv and quantize + o, one launch each
                    mod.norm_quantize_linear(s, None, xs[4096], gains[0], normed, q4, sc4, mx, wqkv, sqkv,
                                             outs["qkv"])
                    mod.quantize_linear(s, None, xs[4096], q4, sc4, wo, so, outs["o"], resid, comb)
                else:
                    mod.norm_quantize(s, None, xs[4096], gains[0], normed, q4, sc4, mx)
                    mod.linear(s, None, q4, sc4, wqkv, sqkv, 4096, outs["qkv"])
                    mod.quantize(s, None, xs[4096], 4096, q4, sc4)
                    mod.linear_residual(s, None, q4, sc4, wo, so, 4096, resid, outs["o"], comb)
                if fused_producers:
                    # the MLP block in two launches: norm_quantize folded into
                    # the SwiGLU GEMV, the act row tail into the down GEMV
                    mod.norm_quantize_mlp(s, None, xs[4096], gains[1], normed, q4, sc4, wg_, sg_, gb_, wu_, su_,
                                          ub_, ab_, mx, wd, sd, outs["down"], resid, comb, q12, sc12)
                    continue
                mod.norm_quantize(s, None, xs[4096], gains[1], normed, q4, sc4, mx)
                if fused_mlp:
                    mod.linear_swiglu_quantize(s, None, q4, sc4, 4096, wg_, sg_, gbuf, wu_, su_, ubuf, act, mx,
                                               q12, sc12)
                    mod.linear_residual(s, None, q12, sc12, wd, sd, ffn, resid, outs["down"], comb)
                else:
                    mod.linear_swiglu(s, None, q4, sc4, 4096, wg_, sg_, gbuf, wu_, su_, ubuf, act, mx)
                    mod.linear_quantize_with_max(s, None, act, ffn, mx, q12, sc12, wd, sd, outs["down"],
                                                 resid, comb)
            mod.quantize(s, None, xs[hk], hk, q4, sc4)
            mod.linear_argmax(s, q4, sc4, head_w, head_s, hk, token)

        layer_chain()
        s.synchronize()
        ms = time_graph(capture(layer_chain), 20)
        # launches per layer: norm_quantize, qkv, quantize, o, norm_quantize,
        # swiglu GEMV + its row-maximum workgroup, quantize_with_max, down
        extras["decode_reference_chain"] = {
            "ms": round(ms, 4), "GB/s": round(step_bytes / (ms * 1e-3) / 1e9, 1),
            "launches": 9 * synth.LAYERS + 3,
            "chain": "norm_quantize, qkv, quantize, o+residual, norm_quantize, linear_swiglu, quantize_with_max, down+residual; lm_head"}
        log(f"reference decode chain: {ms * 1e3:.1f} us ({extras['decode_reference_chain']['GB/s']} GB/s)")
        # the same chain with the MLP pair linear_swiglu + quantize_with_max
        # as one linear_swiglu_quantize call (its row tail folds the maximum
        # and quantizes the down input in one workgroup)
        ms = time_graph(capture(lambda: layer_chain(fused_mlp=True)), 20)
        extras["decode_chain_fused_mlp"] = {
            "ms": round(ms, 4), "GB/s": round(step_bytes / (ms * 1e-3) / 1e9, 1),
            "launches": 8 * synth.LAYERS + 3,
            "chain": "norm_quantize, qkv, quantize, o+residual, norm_quantize, linear_swiglu_quantize, down+residual; lm_head"}
        log(f"decode chain, fused MLP tail: {ms * 1e3:.1f} us ({extras['decode_chain_fused_mlp']['GB/s']} GB/s)")
        # and with every producer folded into the GEMV that consumes it
        # (w8a8_norm_quantize_linear, w8a8_quantize_linear, and the MLP block
        # as w8a8_norm_quantize_mlp)
        ms = time_graph(capture(lambda: layer_chain(fused_mlp=True, fused_producers=True)), 20)
        extras["decode_chain_fused_producers"] = {
            "ms": round(ms, 4), "GB/s": round(step_bytes / (ms * 1e-3) / 1e9, 1),
            "launches": 4 * synth.LAYERS + 3,
            "chain": "norm_quantize_linear (qkv), quantize_linear (o+residual), norm_quantize_mlp "
                     "(SwiGLU GEMV with the norm folded in, down+residual GEMV with the act row tail folded in); "
                     "lm_head"}
        log(f"decode chain, fused producers: {ms * 1e3:.1f} us "
            f"({extras['decode_chain_fused_producers']['GB/s']} GB/s)")
        # the same with BF16 gate / up / act buffers: act is bf(silu(g) u),
        # a BF16 value, so the codes and every output are the same bits, and
        # the down GEMV's producers read a 24 KiB act row instead of 48 KiB
        bf_bufs = tuple(DeviceBuffer.zeroed(s, ffn, np.uint16) for _ in range(3))
        ms = time_graph(capture(lambda: layer_chain(fused_mlp=True, fused_producers=True, mlp_bufs=bf_bufs)), 20)
        extras["decode_chain_fused_producers_bf16_mlp"] = {
            "ms": round(ms, 4), "GB/s": round(step_bytes / (ms * 1e-3) / 1e9, 1),
            "launches": 4 * synth.LAYERS + 3, "gate_up_act_dtype": "bf16"}
        log(f"decode chain, fused producers, BF16 gate/up/act: {ms * 1e3:.1f} us")
        # latency-bound producers at M = 1: per call in a graph of 100
        # stream-ordered calls (launch gap included)
        act12 = DeviceBuffer.from_host(s, synth.normal_rows(45, 1, ffn).reshape(-1))
        lat_ops = {
            "quantize_4096": lambda: mod.quantize(s, None, xs[4096], 4096, q4, sc4),
            "quantize_with_max_12288": lambda: mod.quantize_with_max(s, None, act12, ffn, mx, q12, sc12),
            "norm_quantize_4096": lambda: mod.norm_quantize(s, None, xs[4096], gains[0], normed, q4, sc4, mx),
        }
        lat = {}
        for name, fn in lat_ops.items():
            def hundred(fn=fn):
                for _ in range(100):
                    fn()
            lat[name] = round(time_graph(capture(hundred), 5) / 100 * 1e3, 2)
        extras["producer_us_per_call"] = lat
        log(f"producers (us per call in a graph): {lat}")
        # the reference model's own head: BF16 151936 x 4096, losslessly packed
        # (src/kernels.rs:2258-2373), then select_token.
        pk, words, offs, exc, hx, logits = packed_head_setup(mod, s, hn)
        head_bytes = hn * 1536 * 4 + hn * 16 * 4 + 4096 * 4 + hn * 4
        t_head = time_graph(capture(lambda: mod.head_packed(s, None, hx, words, offs, exc, logits)), 20)
        t_sel = time_graph(capture(lambda: (mod.head_packed(s, None, hx, words, offs, exc, logits),
                                            mod.select_token(s, None, logits, token))), 20)
        extras["bf16_packed_head"] = {
            "us": round(t_head * 1e3, 2), "GB/s": round(head_bytes / (t_head * 1e-3) / 1e9, 1),
            "pct_hbm_peak": round(head_bytes / (t_head * 1e-3) / 1e9 / HBM_PEAK_GBS * 100, 2),
            "us_with_select_token": round(t_sel * 1e3, 2), "bytes": head_bytes,
            "escapes_per_value": round(pk.exceptions.size / (4096 * 4096), 4),
            "reference_us": 574.0, "reference_hw": "RTX PRO 6000 Blackwell Max-Q, docs/qwen3-8b-w8a8/optimization/round-6.md:14"}
        log(f"packed BF16 head: {extras['bf16_packed_head']}")
        # prefill (config 4): M = 512 TOPS and M = 129 HBM GB/s, 36 layers x 4 shapes
        pre = {}
        for m in (512, 129):
            pq = {}
            for k, seed in ((4096, 700), (12288, 703)):
                x = synth.student_t_rows(seed, m, k).reshape(-1)
                q = DeviceBuffer.zeroed(s, m * k, np.int8)
                sc = DeviceBuffer.zeroed(s, m, np.float32)
                mod.quantize(s, None, DeviceBuffer.from_host(s, x), k, q, sc)
                pq[k] = (q, sc)
            pouts = {name: DeviceBuffer.zeroed(s, m * n, np.uint16) for (name, n, _, _, _) in layers[0]}

            def prefill_chain(pq=pq, pouts=pouts):
                for mats in layers:
                    for (name, n, k, w, ws) in mats:
                        mod.linear(s, None, pq[k][0], pq[k][1], w, ws, k, pouts[name])

            prefill_chain()       # eager pass: sizes the module's split-K workspace
            s.synchronize()
            ms = time_graph(capture(prefill_chain), 5, warm=1)
            ops = sum(2 * m * n * k for (_, n, k, _, _) in layers[0]) * synth.LAYERS
            byts = sum(gemv_bytes(n, k, m) for (_, n, k, _, _) in layers[0]) * synth.LAYERS
            shp = {}
            for si, (name, n, k) in enumerate(synth.DECODE_SHAPES):
                def one(si=si, pq=pq, pouts=pouts):
                    for mats in layers:
                        (nm, nn, kk, w, ws) = mats[si]
                        mod.linear(s, None, pq[kk][0], pq[kk][1], w, ws, kk, pouts[nm])
                sms = time_graph(capture(one), 5, warm=1) / synth.LAYERS
                shp[name] = {"us": round(sms * 1e3, 2),
                             "TOPS": round(2 * m * n * k / (sms * 1e-3) / 1e12, 1)}
            pre[f"M{m}"] = {"ms_36_layers": round(ms, 4),
                            "TOPS": round(ops / (ms * 1e-3) / 1e12, 1),
                            "pct_int8_peak": round(ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS * 100, 2),
                            "GB/s": round(byts / (ms * 1e-3) / 1e9, 1),
                            "pct_hbm_peak": round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS * 100, 2),
                            "per_shape": shp}
            log(f"prefill M={m}: {pre[f'M{m}']}")
        extras["prefill"] = pre
        extras["int8_peak"] = {"published_TOPS": INT8_PEAK_TOPS, "derived_TOPS": round(int8_peak_derived, 1),
                               "cu": cu, "peak_clock_MHz": round(clock_mhz, 1),
                               "derivation": "CUs x 4 SIMDs x 2048 ops/clk x peak engine clock"}
        # ragged small batches (config 5): dot4 GEMV vs MFMA GEMM
        rag = {}
        for m in (1, 2, 4, 8, 16, 32, 64):
            entry = {}
            for si in (2, 3):
                name, n, k = synth.DECODE_SHAPES[si]
                x = synth.ragged_rows(range(9000 + 100 * m, 9000 + 100 * m + m), k).reshape(-1)
                q = DeviceBuffer.zeroed(s, m * k, np.int8)
                sc = DeviceBuffer.zeroed(s, m, np.float32)
                mod.quantize(s, None, DeviceBuffer.from_host(s, x), k, q, sc)
                o = DeviceBuffer.zeroed(s, m * n, np.uint16)
                for fam in ("linear_dot4", "linear_mfma"):
                    def chain(si=si, q=q, sc=sc, o=o, fam=fam, k=k):
                        for mats in layers:
                            (_, _, _, w, ws) = mats[si]
                            getattr(mod, fam)(s, None, q, sc, w, ws, k, o)
                    us = time_graph(capture(chain), 10) * 1e3 / synth.LAYERS
                    entry[f"{name}_{fam.split('_')[1]}_GB/s"] = round(
                        gemv_bytes(n, k, m) / (us * 1e-6) / 1e9, 1)
            rag[f"M{m}"] = entry
        extras["ragged"] = rag
        log(f"ragged: {rag}")
        result["extras"] = extras

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)
    return 0


C2_NAME = "C2 decode layers 0-3: qkv, o, gate_up, down at M=1"


def cpu_baseline() -> dict:
    """The C oracle (quantize + exact integer GEMV/GEMM + epilogue, OpenMP
    over output channels; argmax for the head) timed on this host on every
    BASELINE config, each at all the cores this process may use, 8 threads
    (the reference fixture's setting, tools/operator_fixtures.py:17) and 1
    thread; median of 5 or more runs after one warmup run.  "All cores" is
    nproc, capped by OMP_NUM_THREADS when that is set (the GPU box sets it to
    its one-GPU share of the host); the cap is reported.  Samples: C1 one
    4096x4096 projection; C2 four decode layers' sixteen projections
    (layers 0-3, 772 MB of weights: larger than any host L3, so the figure is
    a DRAM rate); C3 the whole 151,936-row head with argmax; C4 the o shape
    (4096x4096) at M = 129 and 512 on Student-t rows; C5 the down shape
    (4096x12288) at M = 4, 16 and 64 on per-row-seeded rows.  `value` is C2
    at all cores."""
    import oracle
    from inferrous_amd import synth

    t0 = time.time()
    nproc = os.cpu_count() or 1
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    nthreads = max(1, min(nproc, cap) if cap > 0 else nproc)
    thread_counts = sorted({nthreads, 8, 1}, reverse=True)
    c2_layers = 4

    def weights(layer: int, si: int):
        _, n, k = synth.DECODE_SHAPES[si]
        return (oracle.synth_i8(SEED_W, synth.weight_stream(layer, si), 0, n * k),
                oracle.synth_f32(SEED_S, synth.scale_stream(layer, si), 0, n, 1e-3, 1e-2))

    layer_mats = [[(n, k) + weights(layer, si) for si, (_, n, k) in enumerate(synth.DECODE_SHAPES)]
                  for layer in range(c2_layers)]
    mats = layer_mats[0]
    xs = {4096: synth.normal_rows(40, 1, 4096).reshape(-1), 12288: synth.normal_rows(41, 1, 12288).reshape(-1)}
    hn, hk = synth.VOCAB, synth.HIDDEN
    hw = oracle.synth_i8(SEED_W, 9001, 0, hn * hk)
    hs = oracle.synth_f32(SEED_S, 9101, 0, hn, 1e-3, 1e-2)
    xh = synth.normal_rows(42, 1, hk).reshape(-1)
    (_, _, wo, so), (_, _, wd, sd) = mats[1], mats[3]
    log(f"cpu baseline: host weights ready in {time.time() - t0:.1f}s")

    def linear_pass(x, m, n, k, w, ws, threads):
        q, sc = oracle.quantize(x, k)
        oracle.linear(q, sc, w, ws, k, threads=threads)

    # (name, algorithmic bytes, integer ops 2*M*N*K, pass at `threads`)
    configs = [("C1 linear M=1 4096x4096", gemv_bytes(4096, 4096), 2 * 4096 * 4096,
                lambda th: linear_pass(xs[4096], 1, 4096, 4096, wo, so, th)),
               (C2_NAME,
                c2_layers * sum(gemv_bytes(n, k) for (n, k, _, _) in mats),
                c2_layers * sum(2 * n * k for (n, k, _, _) in mats),
                lambda th: [linear_pass(xs[k], 1, n, k, w, ws, th) for lm in layer_mats for (n, k, w, ws) in lm]),
               ("C3 lm_head 151936x4096 + argmax, M=1", gemv_bytes(hn, hk, out_bytes=0) + 4, 2 * hn * hk,
                lambda th: oracle.linear_argmax(*oracle.quantize(xh, hk), hw, hs, hk, threads=th))]
    for m in (129, 512):
        x = synth.student_t_rows(700, m, 4096).reshape(-1)
        configs.append((f"C4 prefill o 4096x4096 at M={m}", gemv_bytes(4096, 4096, m), 2 * m * 4096 * 4096,
                        lambda th, x=x, m=m: linear_pass(x, m, 4096, 4096, wo, so, th)))
    for m in (4, 16, 64):
        x = synth.ragged_rows(range(9000 + 100 * m, 9000 + 100 * m + m), 12288).reshape(-1)
        configs.append((f"C5 ragged down 4096x12288 at M={m}", gemv_bytes(4096, 12288, m), 2 * m * 4096 * 12288,
                        lambda th, x=x, m=m: linear_pass(x, m, 4096, 12288, wd, sd, th)))

    def median_seconds(fn) -> float:
        fn()  # warmup
        times = []
        start = time.perf_counter()
        while len(times) < 5 or (time.perf_counter() - start < 0.6 and len(times) < 9):
            t = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t)
        return float(np.median(times))

    per = {}
    for name, nbytes, ops, fn in configs:
        gbs, gops = {}, {}
        for th in thread_counts:
            sec = median_seconds(lambda: fn(th))
            gbs[str(th)] = round(nbytes / sec / 1e9, 3)
            gops[str(th)] = round(ops / sec / 1e9, 3)
        per[name] = {"GB/s_by_threads": gbs, "GOPS_by_threads": gops}
        log(f"cpu baseline {name}: GB/s {gbs}, GOPS {gops}")
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    c2 = per[C2_NAME]["GB/s_by_threads"]
    c2_mb = c2_layers * sum(gemv_bytes(n, k) for (n, k, _, _) in mats) / 1e6
    return {"value": c2[str(nthreads)], "unit": "GB/s", "cores": nthreads, "kind": "port",
            "sample": (f"C oracle (quantize + int32 GEMV/GEMM + BF16 epilogue; argmax for C3), median of >=5 "
                       f"runs after 1 warmup per point; value = C2 (decode layers 0-{c2_layers - 1}, 16 projections "
                       f"at M=1, {c2_mb:.1f} MB of weights) at {nthreads} threads; {cpu_model}, {nproc} logical CPUs"
                       + (f", threads capped at OMP_NUM_THREADS={cap}" if 0 < cap < nproc else "")),
            "cpu_model": cpu_model, "logical_cpus": nproc,
            "thread_cap": {"OMP_NUM_THREADS": cap or None, "applied": bool(0 < cap < nproc)},
            "per_config": per}


if __name__ == "__main__":
    sys.exit(main())
