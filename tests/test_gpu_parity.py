"""GPU parity: every op through the C ABI against the CPU oracle, the committed
fixtures and the reference's own test vectors.  Bit-exact for int8 codes,
scales, i32 accumulators, BF16 outputs and token ids (the north-star bar is
1 BF16 ulp; nothing here needs it).

Layout follows crates/inferrous-qwen3/src/conformance.rs: each op is called
as ``module.op(stream, cfg, ...)`` on the same inputs as the reference's
tests, and each kernel family is forced on every fixture.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import (argmax_cases, argmax_expected, rounding_expected, rounding_probe_inputs,
                      seeded_linear_shapes)
from inferrous_amd import (CudaContext, DeviceBuffer, Event, Graph, W8A8Error, cfg, load, rows)
from inferrous_amd import synth

pytestmark = pytest.mark.gpu

F32 = np.float32


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def env():
    ctx = CudaContext(0)
    stream = ctx.new_stream()
    return ctx, load(ctx), stream


def dev(stream, a):
    return DeviceBuffer.from_host(stream, np.ascontiguousarray(a))


# ------------------------------------------------------------------ rounding
def test_rounding_probe_reference_set(env):
    ctx, mod, s = env
    x = rounding_probe_inputs()
    out = DeviceBuffer.zeroed(s, x.size, np.int8)
    mod.rounding_probe(s, cfg(x.size), dev(s, x), out)
    got = out.to_host_vec(s)
    want = rounding_expected(x)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"first mismatch input bits {x[bad[0]].view(np.uint32):08x}"


# ------------------------------------------------------------------ quantize
def test_quantize_fixtures(env, fixtures):
    ctx, mod, s = env
    for c in fixtures.cases("quantize"):
        w = c["width"]
        x = fixtures.tensor(c, "x").reshape(-1)
        q = DeviceBuffer.zeroed(s, x.size, np.int8)
        sc = DeviceBuffer.zeroed(s, x.size // w, np.float32)
        maxima = dev(s, np.full(x.size // w, 7, np.uint32))
        mod.quantize(s, rows(x.size // w, 1024), dev(s, x), w, q, sc, maxima_reset=maxima)
        assert np.array_equal(q.to_host_vec(s), fixtures.tensor(c, "q").reshape(-1)), c["name"]
        assert np.array_equal(bits(sc.to_host_vec(s)), bits(fixtures.tensor(c, "scale").reshape(-1)))
        assert np.all(maxima.to_host_vec(s) == np.float32(1e-8).view(np.uint32))
        # producer-max path reproduces the scan (src/conformance.rs:129-152)
        mx = np.array([oracle.absmax_bits(r) for r in x.reshape(-1, w)], np.uint32)
        q2 = DeviceBuffer.zeroed(s, x.size, np.int8)
        sc2 = DeviceBuffer.zeroed(s, x.size // w, np.float32)
        mod.quantize_with_max(s, cfg(x.size), dev(s, x), w, dev(s, mx), q2, sc2)
        assert np.array_equal(q2.to_host_vec(s), fixtures.tensor(c, "q").reshape(-1))
        assert np.array_equal(bits(sc2.to_host_vec(s)), bits(fixtures.tensor(c, "scale").reshape(-1)))


def test_weight_quantize_fixture(env, fixtures):
    """tools/prepare.py:79-83 on the device (w8a8_quantize_bf16, one row per
    output channel)."""
    ctx, mod, s = env
    (c,) = fixtures.cases("weight_quantize")
    w = fixtures.tensor(c, "w").view(np.uint16)
    n, k = w.shape
    q = DeviceBuffer.zeroed(s, n * k, np.int8)
    sc = DeviceBuffer.zeroed(s, n, np.float32)
    mod.quantize_weights(s, dev(s, w.reshape(-1)), k, q, sc)
    assert np.array_equal(q.to_host_vec(s), fixtures.tensor(c, "q").reshape(-1))
    assert np.array_equal(bits(sc.to_host_vec(s)), bits(fixtures.tensor(c, "scale")))


@pytest.mark.parametrize("width", [16, 128, 1000, 1001, 4096, 12288, 16400, 20000])
def test_quantize_widths_edges_and_bf16(env, width):
    ctx, mod, s = env
    rng = np.random.default_rng(width)
    m = 6
    x = synth.student_t_rows(width, m, width)
    x[1] = 0.0                                   # floor scale
    x[2, :: max(1, width // 7)] = np.nan         # NaN ignored by the max, quantizes to 0
    x[3, 5 % width] = np.inf                     # inf scale -> all zero codes
    x[4] *= np.float32(1e-30)                    # tiny values
    x[5, :4] = [127, -127, 0.5, -0.5][: min(4, width)]
    for dtype in ("f32", "bf16"):
        if dtype == "f32":
            xin = x.reshape(-1)
            wq, ws = oracle.quantize(xin, width)
        else:
            xin = (bits(x) >> 16).astype(np.uint16).reshape(-1)
            wq, ws = oracle.quantize_bf16(xin, width)
        q = DeviceBuffer.zeroed(s, m * width, np.int8)
        sc = DeviceBuffer.zeroed(s, m, np.float32)
        mod.quantize(s, rows(m, 1024), dev(s, xin), width, q, sc)
        assert np.array_equal(q.to_host_vec(s), wq), dtype
        assert np.array_equal(bits(sc.to_host_vec(s)), bits(ws)), dtype
    del rng


# ------------------------------------------------------------------ linear
# The route each op forces: AUTO (w8a8_linear's own dispatch), the v_dot4
# GEMV family at any M, and the MFMA GEMM family at any M.
LINEAR_ROUTES = ("linear", "linear_dot4", "linear_mfma")
# The reference's four M > 1 tensor-core entry points (src/kernels.rs:846-1289)
# are names for the MFMA route here.
MFMA_ALIASES = ("linear_prefill", "linear_splitk", "linear_tiled", "linear_large")


def test_linear_fixtures_auto_dot4_and_mfma_routes(env, fixtures):
    ctx, mod, s = env
    for c in fixtures.cases("linear"):
        k = c["width"]
        q, asc, w, ws = (dev(s, fixtures.tensor(c, key)) for key in ("q", "asc", "w", "ws"))
        want = fixtures.tensor(c, "out").reshape(-1)
        want_acc = fixtures.tensor(c, "acc").reshape(-1)
        for op in LINEAR_ROUTES:
            for dtype, expect in ((np.float32, bits(want)), (np.uint16, (bits(want) >> 16).astype(np.uint16)),
                                  (np.int32, want_acc)):
                out = DeviceBuffer.zeroed(s, want.size, dtype)
                getattr(mod, op)(s, cfg(want.size * 32), q, asc, w, ws, k, out)
                got = out.to_host_vec(s)
                if dtype is np.float32:
                    got = bits(got)
                assert np.array_equal(got, expect), f"{op} {np.dtype(dtype)} {c['name']}"


def test_reference_tensor_core_names_take_the_mfma_route(env, fixtures):
    """linear_prefill / _splitk / _tiled / _large keep the reference's call
    sites working; each is the MFMA route, checked once per fixture."""
    ctx, mod, s = env
    for c in fixtures.cases("linear"):
        k = c["width"]
        q, asc, w, ws = (dev(s, fixtures.tensor(c, key)) for key in ("q", "asc", "w", "ws"))
        want_acc = fixtures.tensor(c, "acc").reshape(-1)
        for op in MFMA_ALIASES:
            out = DeviceBuffer.zeroed(s, want_acc.size, np.int32)
            getattr(mod, op)(s, None, q, asc, w, ws, k, out)
            assert np.array_equal(out.to_host_vec(s), want_acc), f"{op} {c['name']}"


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 200, 256])
def test_linear_random_shapes(env, m):
    ctx, mod, s = env
    rng = np.random.default_rng(1000 + m)
    for n, k in ((1, 16), (17, 112), (33, 128), (100, 1040), (257, 4096), (64, 12288)):
        if m * k * n > 64 * 12288 * 257:
            continue
        q = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
        w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        if m > 1:
            q[0] = 127
            w[0] = -127
        asc = (rng.random(m) / 64).astype(F32)
        ws = (rng.random(n) / 64).astype(F32)
        acc, out, outb = oracle.linear(q, asc, w, ws, k)
        dq, da, dw, dws = dev(s, q), dev(s, asc), dev(s, w), dev(s, ws)
        for op in ("linear", "linear_dot4", "linear_mfma"):
            o32 = DeviceBuffer.zeroed(s, m * n, np.int32)
            getattr(mod, op)(s, None, dq, da, dw, dws, k, o32)
            assert np.array_equal(o32.to_host_vec(s), acc), f"{op} acc m={m} n={n} k={k}"
            ob = DeviceBuffer.zeroed(s, m * n, np.uint16)
            getattr(mod, op)(s, None, dq, da, dw, dws, k, ob)
            assert np.array_equal(ob.to_host_vec(s), outb), f"{op} bf16 m={m} n={n} k={k}"


@pytest.mark.parametrize("m,n,k", seeded_linear_shapes())
def test_linear_seeded_shape_sweep(env, m, n, k):
    """Every family -- AUTO with the module's split-K workspace, the dot4
    GEMV forced and the MFMA family forced -- at seeded random shapes that
    land on every route and its tails: i32 accumulators, BF16 outputs and,
    through linear_residual, f32 outputs with the residual sum, each bit for
    bit against the oracle."""
    ctx, mod, s = env
    print(f"sweep m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(m * 1_000_003 + n * 101 + k)
    q = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    q[0] = 127
    w[-1] = -127
    asc = (rng.random(m) / 64).astype(F32)
    ws = (rng.random(n) / 64).astype(F32)
    res = rng.standard_normal(m * n).astype(F32)
    acc, out, outb = oracle.linear(q, asc, w, ws, k)
    comb_want = oracle.residual(res, out.reshape(-1))
    dq, da, dw, dws, dres = dev(s, q), dev(s, asc), dev(s, w), dev(s, ws), dev(s, res)
    for op in ("linear", "linear_dot4", "linear_mfma"):
        o32 = DeviceBuffer.zeroed(s, m * n, np.int32)
        getattr(mod, op)(s, None, dq, da, dw, dws, k, o32)
        assert np.array_equal(o32.to_host_vec(s), acc.reshape(-1)), f"{op} acc m={m} n={n} k={k}"
        ob = DeviceBuffer.zeroed(s, m * n, np.uint16)
        getattr(mod, op)(s, None, dq, da, dw, dws, k, ob)
        assert np.array_equal(ob.to_host_vec(s), outb.reshape(-1)), f"{op} bf16 m={m} n={n} k={k}"
    of, cf = DeviceBuffer.zeroed(s, m * n, np.float32), DeviceBuffer.zeroed(s, m * n, np.float32)
    mod.linear_residual(s, None, dq, da, dw, dws, k, dres, of, cf)
    assert np.array_equal(bits(of.to_host_vec(s)), bits(out.reshape(-1))), f"residual out m={m} n={n} k={k}"
    assert np.array_equal(bits(cf.to_host_vec(s)), bits(comb_want)), f"residual sum m={m} n={n} k={k}"


@pytest.mark.parametrize("m", [7, 8, 12, 16, 17, 23, 24, 32, 33])
@pytest.mark.parametrize("n", [6144, 4096])
def test_small_batch_qkv_o_routes(env, m, n):
    """The small-batch boundary at K = 4096 on narrow N: the narrow kernel
    up to M = 16 (and up to M = 32 for N <= 4096), the one-M-tile split-K
    route above (with the module's workspace).  AUTO and the forced MFMA
    family equal the oracle bit for bit on both sides of each boundary."""
    ctx, mod, s = env
    k = 4096
    print(f"small-batch route m={m} n={n}", flush=True)
    rng = np.random.default_rng(7000 + m + n)
    q = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    q[-1] = 127
    w[-1] = -127
    asc = (rng.random(m) / 64 + 1e-4).astype(F32)
    ws = (rng.random(n) / 64 + 1e-4).astype(F32)
    acc, out, outb = oracle.linear(q, asc, w, ws, k, threads=8)
    dq, da, dw, dws = dev(s, q), dev(s, asc), dev(s, w), dev(s, ws)
    for op in ("linear", "linear_mfma"):
        o32 = DeviceBuffer.zeroed(s, m * n, np.int32)
        getattr(mod, op)(s, None, dq, da, dw, dws, k, o32)
        assert np.array_equal(o32.to_host_vec(s), acc), f"{op} acc"
        ob = DeviceBuffer.zeroed(s, m * n, np.uint16)
        getattr(mod, op)(s, None, dq, da, dw, dws, k, ob)
        assert np.array_equal(ob.to_host_vec(s), outb), f"{op} bf16"


def test_linear_residual(env, fixtures):
    ctx, mod, s = env
    for c in fixtures.cases("linear"):
        k = c["width"]
        q, asc, w, ws = (dev(s, fixtures.tensor(c, key)) for key in ("q", "asc", "w", "ws"))
        want = fixtures.tensor(c, "out").reshape(-1)
        res = ((np.arange(want.size) % 17).astype(F32) - 8) * F32(0.0625)   # src/conformance.rs:236-241
        comb_want = oracle.residual(res, want)
        for dtype in (np.float32, np.uint16):
            out = DeviceBuffer.zeroed(s, want.size, dtype)
            comb = DeviceBuffer.zeroed(s, want.size, dtype)
            mod.linear_residual(s, None, q, asc, w, ws, k, dev(s, res), out, comb, k)
            o, cb = out.to_host_vec(s), comb.to_host_vec(s)
            if dtype is np.float32:
                assert np.array_equal(bits(o), bits(want)) and np.array_equal(bits(cb), bits(comb_want))
            else:
                assert np.array_equal(o, (bits(want) >> 16).astype(np.uint16))
                assert np.array_equal(cb, (bits(comb_want) >> 16).astype(np.uint16))


@pytest.mark.parametrize("k,n", [(4096, 8191), (4096, 8192), (4096, 8193), (4096, 12289), (12288, 4097),
                                 (12288, 3)])
def test_decode_gemv_one_matrix_routes(env, k, n):
    """M = 1 on one matrix runs the scalar-argument GEMV entry: two rows per
    wave up to N = 8192 at K = 4096, one row per wave above that and at
    K = 12288.  These N leave the last workgroup partly empty, so its tail
    waves clamp their rows to the last one and must not write.  Every output
    dtype, the residual epilogue (src/kernels.rs:577-618) in f32 and BF16,
    and a one-member grouped call (the same entry) against the oracle; each
    output sits in a larger buffer whose guard elements past N must come
    back untouched."""
    ctx, mod, s = env
    rng = np.random.default_rng(9100 + n + k)
    q = rng.integers(-127, 128, size=(1, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    w[-1, :] = -127                          # the row the tail waves clamp to
    asc = np.array([rng.random() / 64 + 1e-4], F32)
    ws = (rng.random(n) / 64 + 1e-4).astype(F32)
    acc, out, outb = oracle.linear(q, asc, w, ws, k)
    res = rng.standard_normal(n).astype(F32)
    comb = oracle.residual(res, out.reshape(-1))
    dq, da, dw, dws, dres = dev(s, q), dev(s, asc), dev(s, w), dev(s, ws), dev(s, res)
    guard = 64

    def guarded(dtype):
        fill = np.full(n + guard, 0x5A5A, dtype)
        base = DeviceBuffer.from_host(s, fill)
        return base, DeviceBuffer.view_of(base, 0, n)

    def check(base, exp, what):
        got = base.to_host_vec(s)
        if got.dtype == np.float32:
            assert np.array_equal(bits(got[:n]), bits(exp.reshape(-1))), what
        else:
            assert np.array_equal(got[:n], exp.reshape(-1)), what
        assert np.all(got[n:] == got.dtype.type(0x5A5A)), f"{what}: write past N"

    for dtype, exp in ((np.int32, acc), (np.uint16, outb), (np.float32, out)):
        base, o = guarded(dtype)
        mod.linear(s, None, dq, da, dw, dws, k, o)
        check(base, exp, f"linear {np.dtype(dtype)}")
        base, o = guarded(dtype)
        mod.linear_grouped(s, dq, da, k, [(dw, dws, o)])
        check(base, exp, f"grouped(1) {np.dtype(dtype)}")
    for dtype in (np.float32, np.uint16):
        (bo, o), (bc, c) = guarded(dtype), guarded(dtype)
        mod.linear_residual(s, None, dq, da, dw, dws, k, dres, o, c, k)
        if dtype is np.float32:
            check(bo, out, "residual out f32")
            check(bc, comb, "residual combined f32")
        else:
            check(bo, (bits(out) >> 16).astype(np.uint16), "residual out bf16")
            check(bc, (bits(comb) >> 16).astype(np.uint16), "residual combined bf16")


@pytest.mark.parametrize("m,n,k", [(129, 4096, 4096), (129, 24576, 4096), (24, 4096, 12288), (200, 6100, 4096),
                                   (64, 4096, 12288)])
def test_diag_gemm_timeline_matches_linear(env, m, n, k):
    """The timed gemm_tall route (w8a8_diag_gemm_timeline) writes the BF16
    values w8a8_linear writes with the same workspace -- split-K routes
    included -- and four ordered stamps per wave."""
    from inferrous_amd import _lib
    ctx, mod, s = env
    L = _lib.lib()
    rng = np.random.default_rng(9400 + m + n)
    q = dev(s, rng.integers(-127, 128, size=(m, k), dtype=np.int8))
    w = dev(s, rng.integers(-127, 128, size=(n, k), dtype=np.int8))
    asc = dev(s, (rng.random(m) / 64 + 1e-4).astype(F32))
    ws = dev(s, (rng.random(n) / 64 + 1e-4).astype(F32))
    wsb = int(L.w8a8_linear_workspace_bytes(m, n, k))
    work = DeviceBuffer.zeroed(s, max(wsb, 16), np.uint8)
    need = int(L.w8a8_diag_gemm_timeline_stamps(m, n, k, wsb))
    assert need > 0 and need % 32 == 0
    stamps = DeviceBuffer.zeroed(s, need, np.uint64)
    got = DeviceBuffer.zeroed(s, m * n, np.uint16)
    _lib.check(L.w8a8_diag_gemm_timeline(s.handle, q.ptr, asc.ptr, m, w.ptr, ws.ptr, n, k, got.ptr, work.ptr, wsb,
                                         stamps.ptr, need), "diag_gemm_timeline")
    want = DeviceBuffer.zeroed(s, m * n, np.uint16)
    mod.linear(s, None, q, asc, w, ws, k, want)
    assert np.array_equal(got.to_host_vec(s), want.to_host_vec(s))
    t = stamps.to_host_vec(s).astype(np.int64).reshape(-1, 4)
    assert (t > 0).all() and (np.diff(t, axis=1) >= 0).all()


@pytest.mark.parametrize("k,n", [(4096, 6144), (4096, 8193), (12288, 4097)])
def test_diag_timeline_matches_linear(env, k, n):
    """The timed diagnostics GEMV writes the values w8a8_linear writes, and
    one stamp triple per wave of its launch: start <= loads landed <= store
    acknowledged, all within the call."""
    from inferrous_amd import _lib
    ctx, mod, s = env
    L = _lib.lib()
    rng = np.random.default_rng(9300 + n + k)
    q = rng.integers(-127, 128, size=(1, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    asc = np.array([rng.random() / 64 + 1e-4], F32)
    ws = (rng.random(n) / 64 + 1e-4).astype(F32)
    dq, da, dw, dws = dev(s, q), dev(s, asc), dev(s, w), dev(s, ws)
    need = L.w8a8_diag_linear_timeline_stamps(n, k)
    assert need % 3 == 0 and need // 3 >= (n + 1) // 2
    want = DeviceBuffer.zeroed(s, n, np.uint16)
    mod.linear(s, None, dq, da, dw, dws, k, want)
    got = DeviceBuffer.zeroed(s, n, np.uint16)
    stamps = DeviceBuffer.zeroed(s, need, np.uint64)
    _lib.check(L.w8a8_diag_linear_timeline(s.handle, dq.ptr, da.ptr, dw.ptr, dws.ptr, n, k, got.ptr,
                                           _lib.OUT_BF16, stamps.ptr, need), "diag_linear_timeline")
    assert np.array_equal(got.to_host_vec(s), want.to_host_vec(s))
    t = stamps.to_host_vec(s).reshape(-1, 3).astype(np.int64)
    assert np.all(t[:, 0] > 0)
    assert np.all(t[:, 0] <= t[:, 1]) and np.all(t[:, 1] <= t[:, 2])
    assert t[:, 2].max() - t[:, 0].min() < 100_000      # < 1 ms of the 100 MHz clock


def test_pair_triple_share_activations(env, fixtures):
    """src/conformance.rs:263-300: the same matrix in every sibling slot
    reproduces the single projection bit for bit."""
    ctx, mod, s = env
    for c in fixtures.cases("linear"):
        k = c["width"]
        q, asc, w, ws = (dev(s, fixtures.tensor(c, key)) for key in ("q", "asc", "w", "ws"))
        want = bits(fixtures.tensor(c, "out").reshape(-1))
        outs = [DeviceBuffer.zeroed(s, want.size, np.float32) for _ in range(3)]
        mod.linear_pair(s, None, q, asc, k, w, ws, outs[0], w, ws, outs[1])
        assert all(np.array_equal(bits(o.to_host_vec(s)), want) for o in outs[:2])
        outs = [DeviceBuffer.zeroed(s, want.size, np.float32) for _ in range(3)]
        mod.linear_triple(s, None, q, asc, k, w, ws, outs[0], w, ws, outs[1], w, ws, outs[2])
        assert all(np.array_equal(bits(o.to_host_vec(s)), want) for o in outs)


@pytest.mark.parametrize("m", [1, 2, 3])
@pytest.mark.parametrize("k,ns", [(4096, (4096, 1024, 1024)),       # qkv call site, src/gpu.rs:571-590
                                  (4096, (33, 1000, 4099, 7)),      # count 4, unequal and ragged N
                                  (12288, (4096, 1024)),
                                  (1040, (517, 64, 3))])
def test_grouped_distinct_matrices(env, m, k, ns):
    """linear_triple (src/kernels.rs:736-806) / linear_pair / count 4 with a
    different matrix, scale vector and N in every slot: each output equals
    its own projection in the oracle (i32, BF16 and f32), so a slot that read
    a neighbour's matrix, scales or row range would fail.  m = 1 runs the
    one-launch GEMV (gemv_m1 with two rows per wave at k = 4096 here), m = 2
    the multi-row GEMV (gemv_mt), m = 3 one MFMA launch per member."""
    ctx, mod, s = env
    rng = np.random.default_rng(7000 + 31 * m + len(ns) + k)
    q = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    asc = (rng.random(m) / 64 + 1e-4).astype(F32)
    mats = []
    for i, n in enumerate(ns):
        w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        w[0, :] = 127 - i                       # a distinct first row per slot
        ws = (rng.random(n) / 64 + 1e-4 * (i + 1)).astype(F32)
        mats.append((w, ws))
    dq, da = dev(s, q), dev(s, asc)
    dmats = [(dev(s, w), dev(s, ws)) for w, ws in mats]
    want = [oracle.linear(q, asc, w, ws, k) for w, ws in mats]
    for dtype in (np.int32, np.uint16, np.float32):
        outs = [DeviceBuffer.zeroed(s, m * n, dtype) for n in ns]
        mod.linear_grouped(s, dq, da, k, [(dw, dws, o) for (dw, dws), o in zip(dmats, outs)])
        for i, (o, (acc, out, outb)) in enumerate(zip(outs, want)):
            got = o.to_host_vec(s)
            exp = acc if dtype is np.int32 else outb if dtype is np.uint16 else out
            if dtype is np.float32:
                got, exp = bits(got), bits(exp)
            assert np.array_equal(got, exp.reshape(-1)), f"slot {i} n={ns[i]} {np.dtype(dtype)}"
    if len(ns) == 3:
        outs = [DeviceBuffer.zeroed(s, m * n, np.uint16) for n in ns]
        (w0, s0), (w1, s1), (w2, s2) = dmats
        mod.linear_triple(s, None, dq, da, k, w0, s0, outs[0], w1, s1, outs[1], w2, s2, outs[2])
        for i, (o, (_, _, outb)) in enumerate(zip(outs, want)):
            assert np.array_equal(o.to_host_vec(s), outb.reshape(-1)), f"linear_triple slot {i}"


@pytest.mark.parametrize("k,n", [(128, 33), (4096, 12288)])
def test_gate_up_deterministic_inputs(env, k, n):
    """Inputs of src/conformance.rs:746-777; gate/up bits equal separate
    projections and the oracle."""
    ctx, mod, s = env
    i = np.arange(k, dtype=np.int64)
    q = ((i * 13 % 255) - 127).astype(np.int8)
    j = np.arange(k * n, dtype=np.int64)
    w0 = ((j * 31 % 255) - 127).astype(np.int8)
    w1 = ((j * 17 % 251) - 125).astype(np.int8)
    asc = np.array([0.002], F32)
    c = np.arange(n)
    s0 = (F32(0.0001) * ((c % 7) + 1).astype(F32)).astype(F32)
    s1 = (F32(0.0001) * ((c % 11) + 1).astype(F32)).astype(F32)
    dq, da = dev(s, q), dev(s, asc)
    dw0, dw1, ds0, ds1 = dev(s, w0), dev(s, w1), dev(s, s0), dev(s, s1)
    g, u = DeviceBuffer.zeroed(s, n, np.float32), DeviceBuffer.zeroed(s, n, np.float32)
    mod.linear_gate_up(s, rows((n + 7) // 8, 256), dq, da, k, dw0, ds0, g, dw1, ds1, u)
    g1, u1 = DeviceBuffer.zeroed(s, n, np.float32), DeviceBuffer.zeroed(s, n, np.float32)
    mod.linear(s, None, dq, da, dw0, ds0, k, g1)
    mod.linear(s, None, dq, da, dw1, ds1, k, u1)
    _, og, _ = oracle.linear(q, asc, w0, s0, k)
    _, ou, _ = oracle.linear(q, asc, w1, s1, k)
    assert np.array_equal(bits(g.to_host_vec(s)), bits(g1.to_host_vec(s)))
    assert np.array_equal(bits(u.to_host_vec(s)), bits(u1.to_host_vec(s)))
    assert np.array_equal(bits(g.to_host_vec(s)), bits(og))
    assert np.array_equal(bits(u.to_host_vec(s)), bits(ou))


# ------------------------------------------------------------------ selection
def test_select_token_reference_cases(env):
    ctx, mod, s = env
    for x in argmax_cases() + [np.array([1, 3, 3], F32), np.array([np.nan], F32),
                                np.array([np.inf], F32), np.array([-0.0, 0.0], F32)]:
        out = DeviceBuffer.zeroed(s, 1, np.uint32)
        mod.select_token(s, rows(1, 1024), dev(s, x), out)
        assert int(out.to_host_vec(s)[0]) == argmax_expected(x), x[:8]
    # empty input -> sentinel
    out = DeviceBuffer.zeroed(s, 1, np.uint32)
    empty = DeviceBuffer.zeroed(s, 0, np.float32)
    mod.select_token(s, None, empty, out)
    assert int(out.to_host_vec(s)[0]) == 0xFFFFFFFF


def test_select_token_random_ties(env):
    ctx, mod, s = env
    rng = np.random.default_rng(77)
    for n in (1, 63, 64, 65, 4095, 4097, 151936, 300001):
        x = synth.bf16_round((rng.integers(-50, 50, n)).astype(F32) * F32(0.25))
        out = DeviceBuffer.zeroed(s, 1, np.uint32)
        mod.select_token(s, None, dev(s, x), out)
        assert int(out.to_host_vec(s)[0]) == oracle.argmax(x) == int(np.argmax(x))


@pytest.mark.parametrize("k", [4096, 12288, 1024])
def test_linear_argmax_fused(env, k):
    ctx, mod, s = env
    rng = np.random.default_rng(k)
    n = 20000 if k != 4096 else 151936
    q = rng.integers(-127, 128, size=k, dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    w[n - 3] = 127 * np.sign(q).astype(np.int8)          # strong max ...
    w[n // 3] = w[n - 3]                                  # ... tied at a lower index
    ws = np.full(n, 0.004, F32)
    asc = np.array([0.01], F32)
    tok, logits = oracle.linear_argmax(q, asc, w, ws, k)
    assert tok == n // 3
    dq, da, dw, dws = dev(s, q), dev(s, asc), dev(s, w), dev(s, ws)
    for with_logits in (False, True):
        t = DeviceBuffer.zeroed(s, 1, np.uint32)
        lg = DeviceBuffer.zeroed(s, n, np.float32) if with_logits else None
        mod.linear_argmax(s, dq, da, dw, dws, k, t, lg)
        assert int(t.to_host_vec(s)[0]) == tok
        if with_logits:
            assert np.array_equal(bits(lg.to_host_vec(s)), bits(logits))
    # a non-finite logit (scale overflow) gives the sentinel
    ws2 = ws.copy()
    ws2[5] = F32(3e38)
    t = DeviceBuffer.zeroed(s, 1, np.uint32)
    mod.linear_argmax(s, dq, da, dw, dev(s, ws2), k, t)
    tok2, lg2 = oracle.linear_argmax(q, asc, w, ws2, k)
    assert int(t.to_host_vec(s)[0]) == tok2
    assert (tok2 == 0xFFFFFFFF) == (not np.all(np.isfinite(lg2)))


@pytest.mark.parametrize("k,n", [(4096, 4099), (4096, 5), (12288, 1001), (12288, 17), (4096, 1)])
def test_linear_argmax_partial_last_workgroup(env, k, n):
    """Row counts that leave the last selection workgroup partly empty (its
    waves past the last row publish no key): the maximum in the last row,
    then tied with row 0."""
    ctx, mod, s = env
    print(f"argmax partial k={k} n={n}", flush=True)
    rng = np.random.default_rng(k + n)
    q = rng.integers(-127, 128, size=k, dtype=np.int8)
    w = rng.integers(-64, 65, size=(n, k), dtype=np.int8)
    w[n - 1] = 127 * np.sign(q).astype(np.int8)
    ws = np.full(n, 0.004, F32)
    asc = np.array([0.01], F32)
    dq, da, dws = dev(s, q), dev(s, asc), dev(s, ws)
    for tie in (False, True):
        if tie:
            w[0] = w[n - 1]
        tok, logits = oracle.linear_argmax(q, asc, w, ws, k)
        assert tok == (0 if tie else n - 1)
        t = DeviceBuffer.zeroed(s, 1, np.uint32)
        lg = DeviceBuffer.zeroed(s, n, np.float32)
        mod.linear_argmax(s, dq, da, dev(s, w), dws, k, t, lg)
        assert int(t.to_host_vec(s)[0]) == tok, tie
        assert np.array_equal(bits(lg.to_host_vec(s)), bits(logits))


def test_linear_argmax_consecutive_calls_smaller_max(env):
    """The selection slots are reused across calls: a call whose maximum is
    far below the previous call's must still find its own token."""
    ctx, mod, s = env
    rng = np.random.default_rng(99)
    k, n = 4096, 50000
    q = rng.integers(-127, 128, size=k, dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    dq, dw = dev(s, q), dev(s, w)
    tok = DeviceBuffer.zeroed(s, 1, np.uint32)
    for scale, asc_v in ((8e-3, 0.05), (1e-5, 1e-4), (3e-3, 0.02), (2e-6, 1e-5)):
        ws = (rng.random(n) * scale + scale * 0.1).astype(F32)
        asc = np.array([asc_v], F32)
        want, _ = oracle.linear_argmax(q, asc, w, ws, k)
        mod.linear_argmax(s, dq, dev(s, asc), dw, dev(s, ws), k, tok)
        assert int(tok.to_host_vec(s)[0]) == want, (scale, asc_v)


# ------------------------------------------------------------------ graphs
def test_graph_replay_matches_eager(env):
    """Quantize -> linear -> fused lm_head argmax captured once and replayed
    several times with eager work in between; every replay equals eager."""
    ctx, mod, s = env
    k, n, vocab = 4096, 4096, 32000
    x = synth.normal_rows(5, 1, k).reshape(-1)
    w = DeviceBuffer.zeroed(s, n * k, np.int8)
    wh = DeviceBuffer.zeroed(s, vocab * k, np.int8)
    ws = DeviceBuffer.zeroed(s, n, np.float32)
    wsh = DeviceBuffer.zeroed(s, vocab, np.float32)
    mod.synth_i8(s, w, 1, 11)
    mod.synth_i8(s, wh, 1, 12)
    mod.synth_f32(s, ws, 2, 11, 1e-3, 1e-2)
    mod.synth_f32(s, wsh, 2, 12, 1e-3, 1e-2)
    dx = dev(s, x)
    q = DeviceBuffer.zeroed(s, k, np.int8)
    sc = DeviceBuffer.zeroed(s, 1, np.float32)
    h = DeviceBuffer.zeroed(s, n, np.float32)
    q2 = DeviceBuffer.zeroed(s, n, np.int8)
    sc2 = DeviceBuffer.zeroed(s, 1, np.float32)
    tok = DeviceBuffer.zeroed(s, 1, np.uint32)
    lg = DeviceBuffer.zeroed(s, vocab, np.uint16)

    def step():
        mod.quantize(s, None, dx, k, q, sc)
        mod.linear(s, None, q, sc, w, ws, k, h)
        mod.quantize(s, None, h, n, q2, sc2)
        mod.linear_argmax(s, q2, sc2, wh, wsh, n, tok, lg)

    step()
    s.synchronize()
    eager = (h.to_host_vec(s).copy(), lg.to_host_vec(s).copy(), int(tok.to_host_vec(s)[0]))
    g = Graph(s)
    with g:
        step()
    for rep in range(4):
        for b in (h, lg, tok):
            b.fill_zero(s)
        g.launch()
        s.synchronize()
        assert np.array_equal(bits(h.to_host_vec(s)), bits(eager[0])), rep
        assert np.array_equal(lg.to_host_vec(s), eager[1]), rep
        assert int(tok.to_host_vec(s)[0]) == eager[2], rep
        step()  # eager work between replays
        s.synchronize()
        assert int(tok.to_host_vec(s)[0]) == eager[2]


def test_selection_workspace_growth_keeps_captured_graph_valid(env):
    """A graph captured with select_token keeps its workspace address: an
    eager linear_argmax that needs a larger selection workspace retires the
    old buffer instead of freeing it, so every replay still writes live
    memory and returns the right token.  Growing under capture is refused."""
    ctx, mod0, s = env
    mod = load(ctx)                       # fresh workspaces
    x = (np.arange(5000) % 97).astype(F32)
    x[617] = 4000.0
    dx, tok = dev(s, x), DeviceBuffer.zeroed(s, 1, np.uint32)
    mod.select_token(s, None, dx, tok)
    s.synchronize()
    assert int(tok.to_host_vec(s)[0]) == 617
    g = Graph(s)
    with g:
        mod.select_token(s, None, dx, tok)
    # grow: 400,000 vocabulary rows need more keys than the first buffer holds
    n, k = 400_000, 16
    rng = np.random.default_rng(5)
    q = rng.integers(-127, 128, size=(1, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    asc, ws = np.array([0.01], F32), (rng.random(n) / 64 + 1e-4).astype(F32)
    want, _ = oracle.linear_argmax(q, asc, w, ws, k)
    before = len(mod._retired)
    t2 = DeviceBuffer.zeroed(s, 1, np.uint32)
    mod.linear_argmax(s, dev(s, q), dev(s, asc), dev(s, w), dev(s, ws), k, t2)
    s.synchronize()
    assert int(t2.to_host_vec(s)[0]) == want
    assert len(mod._retired) == before + 1
    for rep in range(3):
        tok.fill_zero(s)
        g.launch()
        s.synchronize()
        assert int(tok.to_host_vec(s)[0]) == 617, rep
    mod3 = load(ctx)
    with pytest.raises(W8A8Error):
        with Graph(s):
            mod3.select_token(s, None, dx, tok)


# ------------------------------------------------------------------ synthetic
def test_device_synth_matches_host_definition(env):
    ctx, mod, s = env
    n = (1 << 20) + 13
    a = DeviceBuffer.zeroed(s, n, np.int8)
    mod.synth_i8(s, a, 1, 1003)
    got = a.to_host_vec(s)
    assert np.array_equal(got, oracle.synth_i8(1, 1003, 0, n))
    f = DeviceBuffer.zeroed(s, 4097, np.float32)
    mod.synth_f32(s, f, 2, 1103, 1e-3, 1e-2)
    assert np.array_equal(bits(f.to_host_vec(s)), bits(oracle.synth_f32(2, 1103, 0, 4097, 1e-3, 1e-2)))


def test_errors_raise_not_fall_back(env):
    ctx, mod, s = env
    q = DeviceBuffer.zeroed(s, 4095, np.int8)
    asc = DeviceBuffer.zeroed(s, 1, np.float32)
    with pytest.raises(W8A8Error):
        mod.linear(s, None, q, asc, q, asc, 4095, DeviceBuffer.zeroed(s, 1, np.float32))


# ------------------------------------------------------------------ split-K workspace
@pytest.mark.parametrize("m,n,k", [(129, 4096, 12288), (512, 4096, 12288), (129, 4096, 4096), (129, 6144, 4096),
                                   (24, 4096, 12288), (64, 4096, 12288), (40, 6144, 4096),
                                   (100, 96, 12288), (255, 1024, 4096), (100, 4096, 12288), (65, 4100, 12288),
                                   (128, 4096, 4096),
                                   (129, 4100, 4096), (64, 4100, 12288), (512, 4100, 12288),
                                   (17, 4100, 12288), (100, 1024, 4096), (3, 4100, 8448), (7, 1024, 8448),
                                   (255, 4096, 4096)])
@pytest.mark.parametrize("dtype,res", [(np.float32, False), (np.uint16, True), (np.int32, False)])
def test_linear_split_k_workspace_identical(env, m, n, k, dtype, res):
    """w8a8_linear_ex with a workspace (split-K partials + exact i32 epilogue)
    equals the call without one and the oracle, bit for bit -- also on a
    second call with the same workspace, which carries nothing between calls.
    Up to M = 16 the narrow kernel takes every K it can split over its waves;
    K >= 8192 with K % 1024 != 0 still splits there (3 x 4100 x 8448 under
    AUTO's MFMA route from M = 3, 7 x 1024 x 8448).
    The shapes cover both slab policies with the 16-byte epilogue (M > 200,
    N % 8 == 0) and the 4-column one: streamed (gemm_tall from 3 MiB of
    slabs: 129 x 4096 x 4096 and 64 x 4100 x 12288 on 4 columns, 255 x 4096
    x 4096 on 16 bytes) and plain (smaller gemm_tall sets such as 17 x 4100 x
    12288, 100 x 96 x 12288 and 100 x 1024 x 4096, and gemm_dma's split route
    above M = 256: 512 x 4096 x 12288 on 16 bytes, 512 x 4100 x 12288 on 4
    columns)."""
    from inferrous_amd import _lib
    ctx, mod, s = env
    print(f"split-K m={m} n={n} k={k} {np.dtype(dtype).name} res={res}", flush=True)
    lib = _lib.lib()
    need = lib.w8a8_linear_workspace_bytes(m, n, k)
    assert need > 0 and need % (4 * m * n) == 0
    rng = np.random.default_rng(m * 31 + n + k)
    q = rng.integers(-127, 128, (m, k), dtype=np.int8)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    q[0] = 127
    w[0] = 127
    asc = (rng.random(m) / 64 + 1e-4).astype(F32)
    ws = (rng.random(n) / 64 + 1e-4).astype(F32)
    resid = oracle.bf16_rne(rng.standard_normal(m * n).astype(F32))
    dq, da, dw, dws, dres = dev(s, q), dev(s, asc), dev(s, w), dev(s, ws), dev(s, resid)
    work = DeviceBuffer.zeroed(s, need, np.uint8)
    dt = {np.float32: _lib.OUT_F32, np.uint16: _lib.OUT_BF16, np.int32: _lib.OUT_I32}[dtype]
    outs = []
    for wp, wb in ((work.ptr, need), (None, 0), (work.ptr, need - 1), (work.ptr, need)):
        out = DeviceBuffer.zeroed(s, m * n, dtype)
        comb = DeviceBuffer.zeroed(s, m * n, dtype) if res else None
        _lib.check(lib.w8a8_linear_ex(s.handle, dq.ptr, da.ptr, m, dw.ptr, dws.ptr, n, k,
                                      dres.ptr if res else None, out.ptr,
                                      comb.ptr if res else None, dt, _lib.PATH_AUTO, wp, wb))
        outs.append((out.to_host_vec(s), comb.to_host_vec(s) if res else None))
    for o, c in outs[1:]:
        assert np.array_equal(o.view(np.uint8), outs[0][0].view(np.uint8))
        if res:
            assert np.array_equal(c, outs[0][1])
    acc, of, ob = oracle.linear(q, asc, w, ws, k, threads=8)
    got = outs[0][0]
    if dtype == np.int32:
        assert np.array_equal(got, acc)
    elif dtype == np.uint16:
        assert np.array_equal(got, ob)
        want = (bits(oracle.residual(resid, of)) >> 16).astype(np.uint16)
        assert np.array_equal(outs[0][1], want)
    else:
        assert np.array_equal(bits(got), bits(of))


def test_split_k_workspace_shared_by_shapes(env):
    """One workspace used by split-K launches of different shapes in turn
    (different slab counts and sizes, each call overwriting what the last
    left): every call is bit-exact against the oracle."""
    from inferrous_amd import _lib
    ctx, mod, s = env
    lib = _lib.lib()
    shapes = [(129, 4096, 12288), (512, 4096, 12288), (129, 6144, 4096), (40, 6144, 4096), (129, 4096, 12288),
              (255, 1024, 4096), (512, 4096, 12288)]
    need = max(lib.w8a8_linear_workspace_bytes(m, n, k) for m, n, k in shapes)
    work = DeviceBuffer.zeroed(s, need, np.uint8)
    for i, (m, n, k) in enumerate(shapes):
        print(f"shared workspace call {i}: m={m} n={n} k={k}", flush=True)
        assert lib.w8a8_linear_workspace_bytes(m, n, k) > 0
        rng = np.random.default_rng(i * 101 + m)
        q = rng.integers(-127, 128, (m, k), dtype=np.int8)
        w = rng.integers(-127, 128, (n, k), dtype=np.int8)
        asc = (rng.random(m) / 64 + 1e-4).astype(F32)
        ws = (rng.random(n) / 64 + 1e-4).astype(F32)
        dq, da, dw, dws = dev(s, q), dev(s, asc), dev(s, w), dev(s, ws)
        out = DeviceBuffer.zeroed(s, m * n, np.uint16)
        _lib.check(lib.w8a8_linear_ex(s.handle, dq.ptr, da.ptr, m, dw.ptr, dws.ptr, n, k, None, out.ptr, None,
                                      _lib.OUT_BF16, _lib.PATH_AUTO, work.ptr, need))
        _, _, ob = oracle.linear(q, asc, w, ws, k, threads=8)
        assert np.array_equal(out.to_host_vec(s), ob), f"call {i}"


def test_large_row_counts_beyond_grid_y(env):
    """More rows than a grid's y extent holds (65,535): the quantizer over
    70,000 rows, and a split-K GEMM whose epilogue loops its rows
    (M = 70,000, K = 8192, residual), both bit-exact."""
    from inferrous_amd import _lib
    ctx, mod, s = env
    print("large rows: quantize 70000 x 32, then split-K linear m=70000 n=64 k=8192", flush=True)
    lib = _lib.lib()
    rows_, width = 70000, 32
    rng = np.random.default_rng(70000)
    x = rng.standard_normal(rows_ * width).astype(F32)
    q = DeviceBuffer.zeroed(s, rows_ * width, np.int8)
    sc = DeviceBuffer.zeroed(s, rows_, np.float32)
    dx = dev(s, x)
    mod.quantize(s, None, dx, width, q, sc)
    wq, wsc = oracle.quantize(x, width)
    assert np.array_equal(q.to_host_vec(s), wq)
    assert np.array_equal(bits(sc.to_host_vec(s)), bits(wsc))
    m, n, k = 70000, 64, 8192
    need = lib.w8a8_linear_workspace_bytes(m, n, k)
    assert need > 0  # the split-K plan runs
    qa = rng.integers(-127, 128, (m, k), dtype=np.int8)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    asc = (rng.random(m) / 64 + 1e-4).astype(F32)
    ws = (rng.random(n) / 64 + 1e-4).astype(F32)
    resid = oracle.bf16_rne(rng.standard_normal(m * n).astype(F32))
    acc, of, ob = oracle.linear(qa, asc, w, ws, k, threads=8)
    out = DeviceBuffer.zeroed(s, m * n, np.uint16)
    comb = DeviceBuffer.zeroed(s, m * n, np.uint16)
    work = DeviceBuffer.zeroed(s, need, np.uint8)
    # named, so that no buffer is freed before the kernels that read it ran
    dq, da, dw, dws, dres = dev(s, qa), dev(s, asc), dev(s, w), dev(s, ws), dev(s, resid)
    _lib.check(lib.w8a8_linear_ex(s.handle, dq.ptr, da.ptr, m, dw.ptr, dws.ptr, n, k, dres.ptr, out.ptr,
                                  comb.ptr, _lib.OUT_BF16, _lib.PATH_AUTO, work.ptr, need))
    assert np.array_equal(out.to_host_vec(s), ob)
    assert np.array_equal(comb.to_host_vec(s), (bits(oracle.residual(resid, of)) >> 16).astype(np.uint16))


def test_linear_split_k_unaligned_outputs(env):
    """The split-K epilogue at outputs, residuals and scales that do not start
    on 16 bytes (offset views inside larger buffers): the 4-column epilogue
    runs in place of the 16-byte one, with the same bits."""
    from inferrous_amd import _lib
    ctx, mod, s = env
    lib = _lib.lib()
    m, n, k = 129, 4096, 12288
    need = lib.w8a8_linear_workspace_bytes(m, n, k)
    assert need > 0
    rng = np.random.default_rng(4242)
    q = rng.integers(-127, 128, (m, k), dtype=np.int8)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    asc = (rng.random(m) / 64 + 1e-4).astype(F32)
    ws = (rng.random(n) / 64 + 1e-4).astype(F32)
    resid = oracle.bf16_rne(rng.standard_normal(m * n).astype(F32))
    acc, of, ob = oracle.linear(q, asc, w, ws, k, threads=8)
    want_comb = (bits(oracle.residual(resid, of)) >> 16).astype(np.uint16)
    dq, da, dw = dev(s, q), dev(s, asc), dev(s, w)
    dws = dev(s, np.concatenate([np.zeros(1, F32), ws]))          # ws at +4 bytes
    dres = dev(s, np.concatenate([np.zeros(1, F32), resid]))      # residual at +4 bytes
    work = DeviceBuffer.zeroed(s, need, np.uint8)
    out = DeviceBuffer.zeroed(s, m * n + 1, np.uint16)              # outputs at +2 bytes
    comb = DeviceBuffer.zeroed(s, m * n + 1, np.uint16)
    _lib.check(lib.w8a8_linear_ex(s.handle, dq.ptr, da.ptr, m, dw.ptr, dws.ptr + 4, n, k, dres.ptr + 4,
                                  out.ptr + 2, comb.ptr + 2, _lib.OUT_BF16, _lib.PATH_AUTO, work.ptr, need))
    assert np.array_equal(out.to_host_vec(s)[1:], ob)
    assert np.array_equal(comb.to_host_vec(s)[1:], want_comb)


@pytest.mark.parametrize("m", [1, 2, 3, 5, 7, 8, 16, 33, 40, 64, 65, 100, 128, 129, 193, 256])
@pytest.mark.parametrize("dtype,res", [(np.float32, False), (np.uint16, True), (np.int32, False)])
def test_linear_one_m_tile_wide_n(env, m, dtype, res):
    """1 <= M <= 256 on a wide N (the gate_up regime): one M tile, one
    32 x 32 block per wave up to M = 64 (one to six blocks busy) and 32-row
    slices above, waves without work idle, activation rows past M never
    loaded, a ragged last column tile; bit-exact against the oracle with and
    without a workspace.  M <= 2 forces the MFMA family (AUTO runs dot4 at
    M = 1)."""
    from inferrous_amd import _lib
    ctx, mod, s = env
    n, k = 21601, 1024
    path = _lib.PATH_MFMA if m <= 2 else _lib.PATH_AUTO
    print(f"one-M-tile m={m} n={n} k={k} {np.dtype(dtype).name} res={res}", flush=True)
    lib = _lib.lib()
    rng = np.random.default_rng(m * 7 + 3)
    q = rng.integers(-127, 128, (m, k), dtype=np.int8)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    q[-1] = 127
    w[-1] = -127
    asc = (rng.random(m) / 64 + 1e-4).astype(F32)
    ws = (rng.random(n) / 64 + 1e-4).astype(F32)
    resid = oracle.bf16_rne(rng.standard_normal(m * n).astype(F32))
    dq, da, dw, dws, dres = dev(s, q), dev(s, asc), dev(s, w), dev(s, ws), dev(s, resid)
    dt = {np.float32: _lib.OUT_F32, np.uint16: _lib.OUT_BF16, np.int32: _lib.OUT_I32}[dtype]
    work = DeviceBuffer.zeroed(s, 4 * m * n * 4, np.uint8)
    outs = []
    for wp, wb in ((None, 0), (work.ptr, 4 * m * n * 4)):
        out = DeviceBuffer.zeroed(s, m * n, dtype)
        comb = DeviceBuffer.zeroed(s, m * n, dtype) if res else None
        _lib.check(lib.w8a8_linear_ex(s.handle, dq.ptr, da.ptr, m, dw.ptr, dws.ptr, n, k,
                                      dres.ptr if res else None, out.ptr,
                                      comb.ptr if res else None, dt, path, wp, wb))
        outs.append((out.to_host_vec(s), comb.to_host_vec(s) if res else None))
    assert np.array_equal(outs[1][0].view(np.uint8), outs[0][0].view(np.uint8))
    acc, of, ob = oracle.linear(q, asc, w, ws, k, threads=8)
    got = outs[0][0]
    if dtype == np.int32:
        assert np.array_equal(got, acc)
    elif dtype == np.uint16:
        assert np.array_equal(got, ob)
        want = (bits(oracle.residual(resid, of)) >> 16).astype(np.uint16)
        assert np.array_equal(outs[0][1], want)
    else:
        assert np.array_equal(bits(got), bits(of))



@pytest.mark.parametrize("n,k", [(1000, 512), (4100, 4096), (333, 2048), (1000, 8192), (4096, 12288), (17, 12288)])
@pytest.mark.parametrize("dtype,res", [(np.uint16, True), (np.float32, False), (np.int32, False)])
def test_linear_narrow_every_m(env, n, k, dtype, res):
    """The narrow kernel (small M on narrow N, K split over the workgroup's
    waves, no slabs): M from 1 to 32 across its one to four live activation
    loads per stage, four and eight waves (K below and from 8192), a
    one-stage slice (K = 512), N not a multiple of 16; bit-exact against the
    oracle in every output type, with the residual sum.  The forced MFMA
    family runs it at M = 1 (AUTO runs dot4 there); the route is checked
    on the host."""
    from inferrous_amd import _lib
    ctx, mod, s = env
    lib = _lib.lib()
    dt = {np.float32: _lib.OUT_F32, np.uint16: _lib.OUT_BF16, np.int32: _lib.OUT_I32}[dtype]
    took = 0
    for m in (1, 2, 3, 8, 9, 16, 17, 24, 25, 32):
        route = np.zeros(20, np.int32)
        _lib.check(lib.w8a8_diag_linear_route(m, n, k, dt, int(res), _lib.PATH_MFMA, 0, route.ctypes.data, 20),
                   "route")
        took += int(route[0]) == 15
        print(f"narrow m={m} n={n} k={k} {np.dtype(dtype).name} res={res} family={int(route[0])}", flush=True)
        rng = np.random.default_rng(31 * m + n + k)
        q = rng.integers(-127, 128, (m, k), dtype=np.int8)
        w = rng.integers(-127, 128, (n, k), dtype=np.int8)
        q[-1] = 127
        w[-1] = -127
        asc = (rng.random(m) / 64 + 1e-4).astype(F32)
        ws = (rng.random(n) / 64 + 1e-4).astype(F32)
        resid = oracle.bf16_rne(rng.standard_normal(m * n).astype(F32))
        dq, da, dw, dws, dres = dev(s, q), dev(s, asc), dev(s, w), dev(s, ws), dev(s, resid)
        out = DeviceBuffer.zeroed(s, m * n, dtype)
        comb = DeviceBuffer.zeroed(s, m * n, dtype) if res else None
        _lib.check(lib.w8a8_linear_ex(s.handle, dq.ptr, da.ptr, m, dw.ptr, dws.ptr, n, k,
                                      dres.ptr if res else None, out.ptr, comb.ptr if res else None, dt,
                                      _lib.PATH_MFMA, None, 0))
        acc, of, ob = oracle.linear(q, asc, w, ws, k, threads=8)
        got = out.to_host_vec(s)
        if dtype == np.int32:
            assert np.array_equal(got, acc), f"m={m}"
        elif dtype == np.uint16:
            assert np.array_equal(got, ob), f"m={m}"
            want = (bits(oracle.residual(resid, of)) >> 16).astype(np.uint16)
            assert np.array_equal(comb.to_host_vec(s), want), f"m={m} combined"
        else:
            assert np.array_equal(bits(got), bits(of)), f"m={m}"
    assert took >= 6


@pytest.mark.parametrize("n,tile", [(23100, "256x192"), (15300, "128x192"), (6200, "128x128"), (1000, "128x64")])
@pytest.mark.parametrize("dtype,res", [(np.uint16, True), (np.int32, False)])
def test_linear_large_m_every_tile(env, n, tile, dtype, res):
    """M = 300 (one full and one ragged 256-row tile; three 128-row tiles,
    the last ragged) on the widths that select each gemm_dma tile, with a
    ragged last column tile and K = 640 (five stages: both rings wrap).
    Residual outputs of the 256x192 width take the 128x192 tile."""
    from inferrous_amd import _lib
    ctx, mod, s = env
    m, k = 300, 640
    print(f"large-M m={m} n={n} k={k} tile {tile} {np.dtype(dtype).name} res={res}", flush=True)
    lib = _lib.lib()
    assert lib.w8a8_linear_workspace_bytes(m, n, k) == 0  # no split-K plan: the tile route runs
    rng = np.random.default_rng(n + 17)
    q = rng.integers(-127, 128, (m, k), dtype=np.int8)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    q[-1] = -127
    w[-1] = 127
    asc = (rng.random(m) / 64 + 1e-4).astype(F32)
    ws = (rng.random(n) / 64 + 1e-4).astype(F32)
    resid = oracle.bf16_rne(rng.standard_normal(m * n).astype(F32))
    dq, da, dw, dws, dres = dev(s, q), dev(s, asc), dev(s, w), dev(s, ws), dev(s, resid)
    dt = _lib.OUT_BF16 if dtype == np.uint16 else _lib.OUT_I32
    out = DeviceBuffer.zeroed(s, m * n, dtype)
    comb = DeviceBuffer.zeroed(s, m * n, dtype) if res else None
    _lib.check(lib.w8a8_linear_ex(s.handle, dq.ptr, da.ptr, m, dw.ptr, dws.ptr, n, k,
                                  dres.ptr if res else None, out.ptr,
                                  comb.ptr if res else None, dt, _lib.PATH_AUTO, None, 0))
    acc, of, ob = oracle.linear(q, asc, w, ws, k, threads=8)
    got = out.to_host_vec(s)
    if dtype == np.int32:
        assert np.array_equal(got, acc)
    else:
        assert np.array_equal(got, ob)
        want = (bits(oracle.residual(resid, of)) >> 16).astype(np.uint16)
        assert np.array_equal(comb.to_host_vec(s), want)


def test_linear_split_k_graph_replay(env):
    """The module's split-K workspace under graph capture: replays reuse the
    slabs and equal the eager result every time."""
    ctx, mod, s = env
    m, n, k = 129, 4096, 12288
    rng = np.random.default_rng(5150)
    q = dev(s, rng.integers(-127, 128, (m, k), dtype=np.int8))
    w = dev(s, rng.integers(-127, 128, (n, k), dtype=np.int8))
    asc = dev(s, (rng.random(m) / 64 + 1e-4).astype(F32))
    ws = dev(s, (rng.random(n) / 64 + 1e-4).astype(F32))
    out = DeviceBuffer.zeroed(s, m * n, np.float32)
    mod.linear(s, None, q, asc, w, ws, k, out)     # eager: sizes the workspace
    want = out.to_host_vec(s).copy()
    g = Graph(s)
    with g:
        mod.linear(s, None, q, asc, w, ws, k, out)
    for rep in range(3):
        out.fill_zero(s)
        s.synchronize()
        g.launch()
        s.synchronize()
        assert np.array_equal(bits(out.to_host_vec(s)), bits(want)), f"replay {rep}"
