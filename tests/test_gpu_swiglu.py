"""GPU parity of the SwiGLU producers: `linear_swiglu` (src/kernels.rs:619-695)
and `swiglu` (src/kernels.rs:2172-2190), and the decode MLP chain they feed
(src/gpu.rs:713-790: norm-quantize reset -> linear_swiglu -> quantize_with_max
-> linear_residual).

gate and up are linear epilogues: bit-exact against the oracle.  act uses an
exponential the reference computes with an approximate exp2; it is checked
against the oracle within the reference's own tolerance
(src/conformance.rs:663, |a-b| <= 2e-4 + 0.01|b|, relative L2 <= 0.005) and,
tighter, within one BF16 ulp.  Like the reference's test
(src/conformance.rs:741-838), the fused kernel must equal the separate
projections + swiglu bit for bit, and the published maximum must equal
fold(1e-8, max |act|) of the values actually written.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import bf16_ulp_distance, reference_tolerance_ok
from inferrous_amd import CudaContext, DeviceBuffer, Graph, load, rows

pytestmark = pytest.mark.gpu

F32 = np.float32
FLOOR = int(np.array([1e-8], F32).view(np.uint32)[0])


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def env():
    ctx = CudaContext(0)
    stream = ctx.new_stream()
    return ctx, load(ctx), stream


def dev(stream, a):
    return DeviceBuffer.from_host(stream, np.ascontiguousarray(a))


def fold_max(act) -> int:
    a = np.abs(np.asarray(act, F32).reshape(-1))
    a = a[~np.isnan(a)]
    return int(max(FLOOR, int(bits(a).max()) if a.size else 0))


def act_close(got, gate, up):
    want, _ = oracle.swiglu(gate, up)
    assert reference_tolerance_ok(got, want)
    same = (np.sign(got) == np.sign(want)) & (want != 0)
    assert bf16_ulp_distance(got[same], want[same]).max(initial=0) <= 1


def deterministic_inputs(k, n):
    """src/conformance.rs:746-777."""
    i = np.arange(k, dtype=np.int64)
    q = ((i * 13 % 255) - 127).astype(np.int8)
    j = np.arange(k * n, dtype=np.int64)
    w0 = ((j * 31 % 255) - 127).astype(np.int8)
    w1 = ((j * 17 % 251) - 125).astype(np.int8)
    asc = np.array([0.002], F32)
    c = np.arange(n)
    s0 = (F32(0.0001) * ((c % 7) + 1).astype(F32)).astype(F32)
    s1 = (F32(0.0001) * ((c % 11) + 1).astype(F32)).astype(F32)
    return q, asc, w0, s0, w1, s1


@pytest.mark.parametrize("k,n", [(128, 33), (4096, 12288), (12288, 33), (4096, 4099)])
def test_fused_gate_up_matches_separate(env, k, n):
    ctx, mod, s = env
    print(f"linear_swiglu k={k} n={n}", flush=True)
    q, asc, w0, s0, w1, s1 = deterministic_inputs(k, n)
    dq, da = dev(s, q), dev(s, asc)
    dw0, ds0, dw1, ds1 = dev(s, w0), dev(s, s0), dev(s, w1), dev(s, s1)
    z = lambda: DeviceBuffer.zeroed(s, n, np.float32)  # noqa: E731
    g, u, act = z(), z(), z()
    maximum = dev(s, np.array([FLOOR], np.uint32))
    mod.linear_pair(s, None, dq, da, k, dw0, ds0, g, dw1, ds1, u)
    mod.swiglu(s, None, g, u, act, maximum)
    exp_g, exp_u, exp_act = (b.to_host_vec(s) for b in (g, u, act))
    exp_max = fold_max(exp_act)
    if n == 12288:   # the reference's swiglu publishes only for the decode row
        assert int(maximum.to_host_vec(s)[0]) == exp_max
    else:
        assert int(maximum.to_host_vec(s)[0]) == FLOOR

    g2, u2, act2 = z(), z(), z()
    maximum.copy_from_host(s, np.array([FLOOR], np.uint32))
    mod.linear_swiglu(s, rows((n + 7) // 8, 256), dq, da, k, dw0, ds0, g2, dw1, ds1, u2, act2,
                      maximum)
    assert np.array_equal(bits(g2.to_host_vec(s)), bits(exp_g)), "gate bits"
    assert np.array_equal(bits(u2.to_host_vec(s)), bits(exp_u)), "up bits"
    assert np.array_equal(bits(act2.to_host_vec(s)), bits(exp_act)), "activation bits"
    assert int(maximum.to_host_vec(s)[0]) == exp_max, "activation maximum"

    _, og, _ = oracle.linear(q, asc, w0, s0, k)
    _, ou, _ = oracle.linear(q, asc, w1, s1, k)
    assert np.array_equal(bits(exp_g), bits(og))
    assert np.array_equal(bits(exp_u), bits(ou))
    act_close(exp_act, og, ou)


def test_swiglu_fixture(env, fixtures):
    ctx, mod, s = env
    (case,) = fixtures.cases("swiglu")
    g, u, want = (fixtures.tensor(case, key) for key in ("gate", "up", "out"))
    out = DeviceBuffer.zeroed(s, g.size, np.float32)
    maxima = dev(s, np.array([FLOOR], np.uint32))
    mod.swiglu(s, None, dev(s, g), dev(s, u), out, maxima)
    got = out.to_host_vec(s)
    assert reference_tolerance_ok(got, want)
    act_close(got, g, u)
    assert int(maxima.to_host_vec(s)[0]) == fold_max(got)


@pytest.mark.parametrize("m,k,n", [(1, 1024, 300), (2, 4096, 12288), (4, 4096, 12288),
                                   (17, 4096, 1000), (129, 4096, 12288)])
@pytest.mark.parametrize("dtype", [np.float32, np.uint16])
def test_linear_swiglu_rows(env, m, k, n, dtype):
    """Any M (the reference kernel is M = 1 only): per-row maxima, BF16 and
    f32 outputs, both GEMV and MFMA families underneath."""
    ctx, mod, s = env
    print(f"linear_swiglu m={m} k={k} n={n} dtype={np.dtype(dtype).name}", flush=True)
    rng = np.random.default_rng(m * 7 + k + n)
    q = rng.integers(-127, 128, (m, k), dtype=np.int8)
    asc = (rng.random(m) / 512 + 1e-4).astype(F32)
    w0 = rng.integers(-127, 128, (n, k), dtype=np.int8)
    w1 = rng.integers(-127, 128, (n, k), dtype=np.int8)
    s0 = (rng.random(n) / 256 + 1e-4).astype(F32)
    s1 = (rng.random(n) / 256 + 1e-4).astype(F32)
    z = lambda: DeviceBuffer.zeroed(s, m * n, dtype)  # noqa: E731
    g, u, act = z(), z(), z()
    maxima = dev(s, np.full(m, FLOOR, np.uint32))
    mod.linear_swiglu(s, None, dev(s, q), dev(s, asc), k, dev(s, w0), dev(s, s0), g, dev(s, w1),
                      dev(s, s1), u, act, maxima)

    def host(b):
        v = b.to_host_vec(s)
        return (v.astype(np.uint32) << 16).view(F32) if dtype == np.uint16 else v

    _, og, _ = oracle.linear(q, asc, w0, s0, k, threads=8)
    _, ou, _ = oracle.linear(q, asc, w1, s1, k, threads=8)
    hg, hu, ha = host(g), host(u), host(act)
    assert np.array_equal(bits(hg), bits(og))
    assert np.array_equal(bits(hu), bits(ou))
    act_close(ha, og, ou)
    mx = maxima.to_host_vec(s)
    for r in range(m):
        assert int(mx[r]) == fold_max(ha.reshape(m, n)[r]), f"row {r}"


def test_decode_mlp_chain_and_graph_replay(env):
    """src/gpu.rs:713-790 at decode shapes: the norm quantize resets maxima,
    linear_swiglu publishes max |act|, quantize_with_max (K=12288) uses it,
    linear_residual (down) closes the block.  Replayed from a graph three
    times with eager work in between; each replay equals the eager pass."""
    ctx, mod, s = env
    rng = np.random.default_rng(2024)
    h, f = 4096, 12288
    x = oracle.bf16_rne(rng.standard_normal(h).astype(F32))
    res = oracle.bf16_rne(rng.standard_normal(h).astype(F32))
    wg = rng.integers(-127, 128, (f, h), dtype=np.int8)
    wu = rng.integers(-127, 128, (f, h), dtype=np.int8)
    wd = rng.integers(-127, 128, (h, f), dtype=np.int8)
    sg, su = (rng.random(f) / 4096 + 1e-5).astype(F32), (rng.random(f) / 4096 + 1e-5).astype(F32)
    sd = (rng.random(h) / 4096 + 1e-5).astype(F32)
    dx, dres = dev(s, x), dev(s, res)
    dwg, dwu, dwd = dev(s, wg), dev(s, wu), dev(s, wd)
    dsg, dsu, dsd = dev(s, sg), dev(s, su), dev(s, sd)
    q4, q12 = DeviceBuffer.zeroed(s, h, np.int8), DeviceBuffer.zeroed(s, f, np.int8)
    sc4, sc12 = DeviceBuffer.zeroed(s, 1, np.float32), DeviceBuffer.zeroed(s, 1, np.float32)
    maxima = DeviceBuffer.zeroed(s, 1, np.uint32)
    g, u, act = (DeviceBuffer.zeroed(s, f, np.float32) for _ in range(3))
    down, hidden = DeviceBuffer.zeroed(s, h, np.float32), DeviceBuffer.zeroed(s, h, np.float32)

    def block():
        mod.quantize(s, None, dx, h, q4, sc4, maxima_reset=maxima)
        mod.linear_swiglu(s, None, q4, sc4, h, dwg, dsg, g, dwu, dsu, u, act, maxima)
        mod.quantize_with_max(s, None, act, f, maxima, q12, sc12)
        mod.linear_residual(s, None, q12, sc12, dwd, dsd, f, dres, down, hidden)

    block()
    eager = {name: b.to_host_vec(s).copy() for name, b in
             (("act", act), ("q12", q12), ("sc12", sc12), ("max", maxima), ("hidden", hidden))}

    # oracle chain on the same inputs; act comes from the GPU (tolerance op)
    oq4, osc4 = oracle.quantize(x, h)
    _, og, _ = oracle.linear(oq4, osc4, wg, sg, h, threads=8)
    _, ou, _ = oracle.linear(oq4, osc4, wu, su, h, threads=8)
    assert np.array_equal(bits(g.to_host_vec(s)), bits(og))
    assert np.array_equal(bits(u.to_host_vec(s)), bits(ou))
    act_close(eager["act"], og, ou)
    assert int(eager["max"][0]) == oracle.absmax_bits(eager["act"])
    oq12, osc12 = oracle.quantize(eager["act"], f)
    assert np.array_equal(eager["q12"], oq12)
    assert np.array_equal(bits(eager["sc12"]), bits(osc12))
    _, od, _ = oracle.linear(oq12, osc12, wd, sd, f, threads=8)
    assert np.array_equal(bits(eager["hidden"]), bits(oracle.residual(res, od)))

    graph = Graph(s)
    with graph:
        block()
    for rep in range(3):
        for b in (act, q12, hidden):
            b.fill_zero(s)
        maxima.copy_from_host(s, np.array([0xFFFFFFFF >> 1], np.uint32))  # stale large value
        s.synchronize()
        graph.launch()
        s.synchronize()
        for name, b in (("act", act), ("q12", q12), ("sc12", sc12), ("max", maxima),
                        ("hidden", hidden)):
            assert np.array_equal(b.to_host_vec(s).view(np.uint8), eager[name].view(np.uint8)), \
                f"replay {rep}: {name}"


@pytest.mark.parametrize("m,k,n,res,dtype", [(1, 12288, 4096, True, np.float32),
                                             (1, 12288, 4099, True, np.uint16),
                                             (1, 4096, 12288, False, np.float32),
                                             (1, 4096, 33, False, np.int32),
                                             (3, 12288, 100, True, np.float32),
                                             (1, 1024, 64, False, np.float32)])
def test_linear_quantize_with_max_matches_two_steps(env, m, k, n, res, dtype):
    """The combined quantize_with_max + linear(_residual) entry point equals
    the two separate calls (src/gpu.rs:371-406) and the oracle, bit for bit."""
    ctx, mod, s = env
    print(f"linear_quantize_with_max m={m} k={k} n={n} res={res} {np.dtype(dtype).name}", flush=True)
    rng = np.random.default_rng(k + n + m)
    x = oracle.bf16_rne((rng.standard_normal(m * k) * 3).astype(F32))
    x[5] = 0.0
    mx = np.array([oracle.absmax_bits(r) for r in x.reshape(m, k)], np.uint32)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    ws = (rng.random(n) / 512 + 1e-5).astype(F32)
    resid = oracle.bf16_rne(rng.standard_normal(m * n).astype(F32))
    dx, dmx, dw, dws, dres = dev(s, x), dev(s, mx), dev(s, w), dev(s, ws), dev(s, resid)

    def outputs():
        q = DeviceBuffer.zeroed(s, m * k, np.int8)
        sc = DeviceBuffer.zeroed(s, m, np.float32)
        out = DeviceBuffer.zeroed(s, m * n, dtype)
        comb = DeviceBuffer.zeroed(s, m * n, dtype) if res else None
        return q, sc, out, comb

    q1, sc1, out1, comb1 = outputs()
    mod.linear_quantize_with_max(s, None, dx, k, dmx, q1, sc1, dw, dws, out1,
                                 dres if res else None, comb1)
    q2, sc2, out2, comb2 = outputs()
    mod.quantize_with_max(s, None, dx, k, dmx, q2, sc2)
    if res:
        mod.linear_residual(s, None, q2, sc2, dw, dws, k, dres, out2, comb2)
    else:
        mod.linear(s, None, q2, sc2, dw, dws, k, out2)
    for a, b in ((q1, q2), (sc1, sc2), (out1, out2)) + (((comb1, comb2),) if res else ()):
        assert np.array_equal(a.to_host_vec(s).view(np.uint8), b.to_host_vec(s).view(np.uint8))
    oq, osc = oracle.quantize_with_max(x, k, mx)
    assert np.array_equal(q1.to_host_vec(s), oq)
    acc, of, ob = oracle.linear(oq, osc, w, ws, k, threads=8)
    got = out1.to_host_vec(s)
    if dtype == np.int32:
        assert np.array_equal(got, acc)
    elif dtype == np.uint16:
        assert np.array_equal(got, ob)
    else:
        assert np.array_equal(bits(got), bits(of))
    if res:
        want = oracle.residual(resid, of)
        gotc = comb1.to_host_vec(s)
        if dtype == np.uint16:
            assert np.array_equal(gotc, (bits(want) >> 16).astype(np.uint16))
        else:
            assert np.array_equal(bits(gotc), bits(want))


def test_decode_mlp_chain_combined_down_entry(env):
    """The decode MLP block through the combined down entry point
    (linear_quantize_with_max) equals the chain of separate calls bit for
    bit, eagerly and under graph replay."""
    ctx, mod, s = env
    rng = np.random.default_rng(77)
    h, f = 4096, 12288
    x = oracle.bf16_rne(rng.standard_normal(h).astype(F32))
    res = oracle.bf16_rne(rng.standard_normal(h).astype(F32))
    wg = dev(s, rng.integers(-127, 128, (f, h), dtype=np.int8))
    wu = dev(s, rng.integers(-127, 128, (f, h), dtype=np.int8))
    wd = dev(s, rng.integers(-127, 128, (h, f), dtype=np.int8))
    sg = dev(s, (rng.random(f) / 4096 + 1e-5).astype(F32))
    su = dev(s, (rng.random(f) / 4096 + 1e-5).astype(F32))
    sd = dev(s, (rng.random(h) / 4096 + 1e-5).astype(F32))
    dx, dres = dev(s, x), dev(s, res)

    def buffers():
        return dict(q4=DeviceBuffer.zeroed(s, h, np.int8), sc4=DeviceBuffer.zeroed(s, 1, np.float32),
                    mx=DeviceBuffer.zeroed(s, 1, np.uint32),
                    g=DeviceBuffer.zeroed(s, f, np.float32), u=DeviceBuffer.zeroed(s, f, np.float32),
                    act=DeviceBuffer.zeroed(s, f, np.float32),
                    q12=DeviceBuffer.zeroed(s, f, np.int8), sc12=DeviceBuffer.zeroed(s, 1, np.float32),
                    down=DeviceBuffer.zeroed(s, h, np.float32), hid=DeviceBuffer.zeroed(s, h, np.float32))

    def block(b, fused):
        mod.quantize(s, None, dx, h, b["q4"], b["sc4"], maxima_reset=b["mx"])
        mod.linear_swiglu(s, None, b["q4"], b["sc4"], h, wg, sg, b["g"], wu, su, b["u"], b["act"], b["mx"])
        if fused:
            mod.linear_quantize_with_max(s, None, b["act"], f, b["mx"], b["q12"], b["sc12"], wd, sd,
                                         b["down"], dres, b["hid"])
        else:
            mod.quantize_with_max(s, None, b["act"], f, b["mx"], b["q12"], b["sc12"])
            mod.linear_residual(s, None, b["q12"], b["sc12"], wd, sd, f, dres, b["down"], b["hid"])

    ref, fus = buffers(), buffers()
    block(ref, False)
    block(fus, True)
    names = ("q12", "sc12", "down", "hid", "mx")
    want = {k: ref[k].to_host_vec(s).view(np.uint8).copy() for k in names}
    for k in names:
        assert np.array_equal(fus[k].to_host_vec(s).view(np.uint8), want[k]), k
    graph = Graph(s)
    with graph:
        block(fus, True)
    for rep in range(3):
        for k in ("q12", "down", "hid"):
            fus[k].fill_zero(s)
        s.synchronize()
        graph.launch()
        s.synchronize()
        for k in names:
            assert np.array_equal(fus[k].to_host_vec(s).view(np.uint8), want[k]), f"replay {rep}: {k}"


@pytest.mark.parametrize("m,k,n,dtype", [(1, 4096, 12288, np.float32), (1, 4096, 12288, np.uint16),
                                         (1, 4096, 20000, np.float32), (1, 4096, 20000, np.uint16),
                                         (1, 12288, 1000, np.float32), (1, 128, 33, np.uint16),
                                         (3, 4096, 4099, np.float32), (2, 1024, 5000, np.uint16)])
def test_linear_swiglu_quantize_matches_separate_calls(env, m, k, n, dtype):
    """w8a8_linear_swiglu_quantize (the decode pair src/gpu.rs:730 + :381 in
    one call) writes the same gate / up / act / maxima bits as
    w8a8_linear_swiglu, and q_out / scales_out equal quantize_with_max of
    act with the folded maxima (the oracle restatement of
    src/kernels.rs:453-475) -- at M = 1 on the fused GEMV (one workgroup
    folds the maximum and quantizes), and on the grouped / MFMA route.
    n = 20000 at M = 1 exceeds the row tail's register-held width (16,384),
    so its re-reading fold and quantize loops run too.  The maxima start at a reset floor on one row and at a large stale value
    on another, so the fold (not the row maximum) sets the scale."""
    ctx, mod, s = env
    print(f"linear_swiglu_quantize m={m} k={k} n={n} dtype={np.dtype(dtype).name}", flush=True)
    rng = np.random.default_rng(m * 1009 + k + n)
    q = rng.integers(-127, 128, (m, k), dtype=np.int8)
    asc = (rng.random(m) / 512 + 1e-4).astype(F32)
    w0 = rng.integers(-127, 128, (n, k), dtype=np.int8)
    w1 = rng.integers(-127, 128, (n, k), dtype=np.int8)
    s0 = (rng.random(n) / 256 + 1e-4).astype(F32)
    s1 = (rng.random(n) / 256 + 1e-4).astype(F32)
    start = np.full(m, FLOOR, np.uint32)
    if m > 1:
        start[-1] = int(np.array([1e4], F32).view(np.uint32)[0])   # larger than any |act| here
    dq, da, dw0, dw1, ds0, ds1 = dev(s, q), dev(s, asc), dev(s, w0), dev(s, w1), dev(s, s0), dev(s, s1)
    outs = []
    for fused in (False, True):
        g, u, act = (DeviceBuffer.zeroed(s, m * n, dtype) for _ in range(3))
        maxima = dev(s, start)
        q_out = DeviceBuffer.zeroed(s, m * n, np.int8)
        sc_out = DeviceBuffer.zeroed(s, m, np.float32)
        if fused:
            mod.linear_swiglu_quantize(s, None, dq, da, k, dw0, ds0, g, dw1, ds1, u, act, maxima, q_out, sc_out)
        else:
            mod.linear_swiglu(s, None, dq, da, k, dw0, ds0, g, dw1, ds1, u, act, maxima)
        outs.append({name: b.to_host_vec(s).copy() for name, b in
                     (("g", g), ("u", u), ("act", act), ("max", maxima), ("q", q_out), ("sc", sc_out))})
    for name in ("g", "u", "act", "max"):
        assert np.array_equal(outs[1][name].view(np.uint8), outs[0][name].view(np.uint8)), name
    act_v = outs[1]["act"]
    if dtype == np.uint16:
        act_v = (act_v.astype(np.uint32) << 16).view(F32)
    want_q, want_s = oracle.quantize_with_max(act_v, n, outs[1]["max"])
    assert np.array_equal(outs[1]["q"], want_q)
    assert np.array_equal(bits(outs[1]["sc"]), bits(want_s))
    for r in range(m):
        assert int(outs[1]["max"][r]) == max(int(start[r]), fold_max(act_v.reshape(m, n)[r])), f"row {r}"
