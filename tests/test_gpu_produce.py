"""GPU parity of the producers folded into the decode GEMV's prologue:
`w8a8_norm_quantize_linear` (norm_quantize, src/kernels.rs:476-575, then
linear / linear_residual) and `w8a8_quantize_linear` (quantize,
src/kernels.rs:433-451, then the same), one launch each, and
`w8a8_norm_quantize_linear_swiglu` (norm_quantize, then linear_swiglu,
src/kernels.rs:619-695, and optionally the act's quantize_with_max), and
`w8a8_norm_quantize_mlp` (that GEMV, then the act's row tail --
maximum fold and quantize_with_max, src/kernels.rs:453-475 -- folded into the
down GEMV with its residual).

Every workgroup recomputes the row's codes with the producer's arithmetic, so
every output must equal the two-call sequence bit for bit: the codes, the
scale, the normalised row, the maxima reset, and the projection's out and
combined.  They are also checked against the oracle: the codes and scale
against oracle.norm_quantize / oracle.quantize, and the projection against
oracle.linear on those codes (with oracle.residual for combined).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from inferrous_amd import CudaContext, DeviceBuffer, Graph, load

pytestmark = pytest.mark.gpu

F32 = np.float32
FLOOR = int(np.array([1e-8], F32).view(np.uint32)[0])
JUNK = 0x12345678


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def env():
    ctx = CudaContext(0)
    stream = ctx.new_stream()
    return ctx, load(ctx), stream


def dev(stream, a):
    return DeviceBuffer.from_host(stream, np.ascontiguousarray(a))


def make_row(rng, kind="normal"):
    x = (rng.standard_normal(4096) * np.exp(rng.uniform(-2, 2))).astype(F32)
    x[rng.integers(0, 4096, 8)] *= F32(50)          # outlier channels
    if kind == "zero":
        x[:] = 0
    elif kind == "nan":
        x[[3, 2048]] = np.nan
    elif kind == "huge":
        x *= F32(1e20)                             # squares overflow in the norm
    elif kind == "tiny":
        x *= F32(1e-3)
    return x


def run_both(env, producer, x, gain, w, ws, resid, dtype, with_normed=True, with_maxima=True):
    """(two-call outputs, fused outputs), each a dict of host arrays."""
    _, mod, s = env
    n = ws.size
    xb, wb, wsb = dev(s, x), dev(s, w), dev(s, ws)
    gb = dev(s, gain) if gain is not None else None
    rb = dev(s, resid) if resid is not None else None
    res = {}
    for mode in ("two", "fused"):
        q = DeviceBuffer.zeroed(s, 4096, np.int8)
        sc = DeviceBuffer.zeroed(s, 1, np.float32)
        mx = dev(s, np.array([JUNK], np.uint32))
        nb = DeviceBuffer.zeroed(s, 4096, np.float32)
        out = DeviceBuffer.zeroed(s, n, dtype)
        comb = DeviceBuffer.zeroed(s, n, dtype) if resid is not None else None
        if mode == "two":
            if producer == "norm":
                mod.norm_quantize(s, None, xb, gb, nb, q, sc, mx)
            else:
                mod.quantize(s, None, xb, 4096, q, sc, maxima_reset=mx)
            if resid is not None:
                mod.linear_residual(s, None, q, sc, wb, wsb, 4096, rb, out, comb)
            else:
                mod.linear(s, None, q, sc, wb, wsb, 4096, out)
        elif producer == "norm":
            mod.norm_quantize_linear(s, None, xb, gb, nb if with_normed else None, q, sc,
                                     mx if with_maxima else None, wb, wsb, out, rb, comb)
        else:
            mod.quantize_linear(s, None, xb, q, sc, wb, wsb, out, rb, comb,
                                maxima_reset=mx if with_maxima else None)
        s.synchronize()
        res[mode] = dict(q=q.to_host_vec(s), sc=sc.to_host_vec(s), mx=mx.to_host_vec(s),
                         normed=nb.to_host_vec(s), out=out.to_host_vec(s),
                         comb=comb.to_host_vec(s) if comb is not None else None)
    return res["two"], res["fused"]


def same_bits(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float32:
        return np.array_equal(bits(a), bits(b))
    return np.array_equal(a, b)


def check_against_oracle(producer, x, gain, w, ws, resid, dtype, got):
    if producer == "norm":
        wn, wq, wsc, _ = oracle.norm_quantize(x[None, :], gain)
        wn = wn.reshape(-1)
    else:
        wq, wsc = oracle.quantize(x, 4096)
        wn = None
    assert np.array_equal(got["q"], wq.reshape(-1)), "codes"
    assert np.array_equal(bits(got["sc"]), bits(wsc)), "scale"
    acc, of, ob = oracle.linear(wq.reshape(1, -1), wsc, w, ws, 4096, threads=8)
    if dtype == np.int32:
        assert np.array_equal(got["out"], acc)
    elif dtype == np.uint16:
        assert np.array_equal(got["out"], ob)
    else:
        assert np.array_equal(bits(got["out"]), bits(of))
    if resid is not None:
        comb = oracle.residual(resid, of)
        want = (bits(comb) >> 16).astype(np.uint16) if dtype == np.uint16 else comb
        assert same_bits(got["comb"], want), "combined"
    return wn


@pytest.mark.parametrize("producer", ["norm", "quant"])
@pytest.mark.parametrize("dtype,res", [(np.uint16, False), (np.uint16, True), (np.float32, True),
                                       (np.float32, False), (np.int32, False)])
@pytest.mark.parametrize("n", [1, 33, 6144, 8193])
def test_producer_linear_matches_two_calls(env, producer, dtype, res, n):
    """n = 8193 takes the one-row-per-wave form; the others two rows per wave
    (n = 1 and 33: a ragged last workgroup, tail rows clamped)."""
    print(f"producer+linear {producer} n={n} {np.dtype(dtype).name} res={res}", flush=True)
    rng = np.random.default_rng(n * 7 + (3 if producer == "norm" else 5) + (11 if res else 0))
    x = make_row(rng)
    gain = (1 + 0.3 * rng.standard_normal(4096)).astype(F32) if producer == "norm" else None
    w = rng.integers(-127, 128, (n, 4096), dtype=np.int8)
    ws = (rng.random(n) / 64 + 1e-4).astype(F32)
    resid = oracle.bf16_rne(rng.standard_normal(n).astype(F32)) if res else None
    two, fused = run_both(env, producer, x, gain, w, ws, resid, dtype)
    for key in ("q", "sc", "mx", "out") + (("normed",) if producer == "norm" else ()) + (("comb",) if res else ()):
        assert same_bits(fused[key], two[key]), key
    assert fused["mx"][0] == FLOOR
    wn = check_against_oracle(producer, x, gain, w, ws, resid, dtype, fused)
    if producer == "norm":
        assert np.array_equal(bits(fused["normed"]), bits(wn)), "normalised row"


@pytest.mark.parametrize("producer", ["norm", "quant"])
@pytest.mark.parametrize("kind", ["zero", "nan", "huge", "tiny"])
def test_producer_linear_special_rows(env, producer, kind):
    """Zero rows (scale at its floor, codes 0), NaN coordinates (codes 0; with
    the norm every output NaN), squares that overflow the norm's sum, and a
    tiny row where the norm's epsilon matters: the fused call still equals the
    two calls, NaN for NaN."""
    print(f"producer+linear special row {kind} {producer}", flush=True)
    rng = np.random.default_rng(17 + len(kind))
    x = make_row(rng, kind)
    gain = (1 + 0.3 * rng.standard_normal(4096)).astype(F32) if producer == "norm" else None
    n = 4096
    w = rng.integers(-127, 128, (n, 4096), dtype=np.int8)
    ws = (rng.random(n) / 64 + 1e-4).astype(F32)
    resid = oracle.bf16_rne(rng.standard_normal(n).astype(F32))
    two, fused = run_both(env, producer, x, gain, w, ws, resid, np.float32)
    for key in ("q", "sc", "mx", "out", "comb") + (("normed",) if producer == "norm" else ()):
        a, b = fused[key], two[key]
        if a.dtype == np.float32:
            ok = (bits(a) == bits(b)) | (np.isnan(a) & np.isnan(b))
            assert ok.all(), key
        else:
            assert np.array_equal(a, b), key
    if kind == "zero":
        assert np.all(fused["q"] == 0) and fused["sc"][0] == F32(1e-8) / F32(127)
    if kind == "nan":
        assert np.all(fused["q"][[3, 2048]] == 0)


def test_producer_linear_optional_outputs(env):
    """out_norm and maxima may be NULL: nothing else changes."""
    rng = np.random.default_rng(23)
    x = make_row(rng)
    gain = (1 + 0.3 * rng.standard_normal(4096)).astype(F32)
    n = 6144
    w = rng.integers(-127, 128, (n, 4096), dtype=np.int8)
    ws = (rng.random(n) / 64 + 1e-4).astype(F32)
    two, fused = run_both(env, "norm", x, gain, w, ws, None, np.uint16, with_normed=False, with_maxima=False)
    assert np.all(fused["normed"] == 0) and fused["mx"][0] == JUNK
    for key in ("q", "sc", "out"):
        assert same_bits(fused[key], two[key]), key
    two, fused = run_both(env, "quant", x, None, w, ws, None, np.uint16, with_maxima=False)
    assert fused["mx"][0] == JUNK
    for key in ("q", "sc", "out"):
        assert same_bits(fused[key], two[key]), key


def test_producer_linear_graph_replay(env):
    """Both fused calls captured in one graph (no allocation, no host sync):
    every replay reproduces the eager result, with eager work between."""
    _, mod, s = env
    rng = np.random.default_rng(29)
    x = make_row(rng)
    gain = (1 + 0.3 * rng.standard_normal(4096)).astype(F32)
    n = 4096
    w = rng.integers(-127, 128, (n, 4096), dtype=np.int8)
    ws = (rng.random(n) / 64 + 1e-4).astype(F32)
    resid = oracle.bf16_rne(rng.standard_normal(n).astype(F32))
    xb, gb, wb, wsb, rb = dev(s, x), dev(s, gain), dev(s, w), dev(s, ws), dev(s, resid)
    q = DeviceBuffer.zeroed(s, 4096, np.int8)
    sc = DeviceBuffer.zeroed(s, 1, np.float32)
    mx = DeviceBuffer.zeroed(s, 1, np.uint32)
    nb = DeviceBuffer.zeroed(s, 4096, np.float32)
    o1 = DeviceBuffer.zeroed(s, n, np.uint16)
    o2 = DeviceBuffer.zeroed(s, n, np.uint16)
    c2 = DeviceBuffer.zeroed(s, n, np.uint16)

    def calls():
        mod.norm_quantize_linear(s, None, xb, gb, nb, q, sc, mx, wb, wsb, o1)
        mod.quantize_linear(s, None, xb, q, sc, wb, wsb, o2, rb, c2)

    calls()
    s.synchronize()
    want = [b.to_host_vec(s) for b in (o1, o2, c2, q, sc)]
    g = Graph(s)
    with g:
        calls()
    for _ in range(3):
        for b in (o1, o2, c2, q, sc):
            b.fill_zero(s)
        s.synchronize()
        g.launch()
        s.synchronize()
        got = [b.to_host_vec(s) for b in (o1, o2, c2, q, sc)]
        for a, b in zip(got, want):
            assert same_bits(a, b)


def run_swiglu_both(env, x, gain, wg, sg, wu, su, dtype, quantize):
    """(separate calls, folded call): norm_quantize then linear_swiglu or
    linear_swiglu_quantize, against norm_quantize_linear_swiglu."""
    _, mod, s = env
    n = sg.size
    xb, gb = dev(s, x), dev(s, gain)
    wgb, sgb, wub, sub = dev(s, wg), dev(s, sg), dev(s, wu), dev(s, su)
    res = {}
    for mode in ("calls", "folded"):
        q = DeviceBuffer.zeroed(s, 4096, np.int8)
        sc = DeviceBuffer.zeroed(s, 1, np.float32)
        nb = DeviceBuffer.zeroed(s, 4096, np.float32)
        mx = dev(s, np.array([JUNK], np.uint32))
        gate, up, act = (DeviceBuffer.zeroed(s, n, dtype) for _ in range(3))
        qo = DeviceBuffer.zeroed(s, n, np.int8) if quantize else None
        so = DeviceBuffer.zeroed(s, 1, np.float32) if quantize else None
        if mode == "calls":
            mod.norm_quantize(s, None, xb, gb, nb, q, sc, mx)
            if quantize:
                mod.linear_swiglu_quantize(s, None, q, sc, 4096, wgb, sgb, gate, wub, sub, up, act, mx, qo, so)
            else:
                mod.linear_swiglu(s, None, q, sc, 4096, wgb, sgb, gate, wub, sub, up, act, mx)
        else:
            mod.norm_quantize_linear_swiglu(s, None, xb, gb, nb, q, sc, wgb, sgb, gate, wub, sub, up, act, mx,
                                            qo, so)
        s.synchronize()
        res[mode] = dict(q=q.to_host_vec(s), sc=sc.to_host_vec(s), normed=nb.to_host_vec(s),
                         mx=mx.to_host_vec(s), gate=gate.to_host_vec(s), up=up.to_host_vec(s),
                         act=act.to_host_vec(s), qo=qo.to_host_vec(s) if quantize else None,
                         so=so.to_host_vec(s) if quantize else None)
    return res["calls"], res["folded"]


def nan_same(a, b):
    if a.dtype == np.float32:
        return bool(((bits(a) == bits(b)) | (np.isnan(a) & np.isnan(b))).all())
    return np.array_equal(a, b)


@pytest.mark.parametrize("quantize", [False, True])
@pytest.mark.parametrize("dtype", [np.float32, np.uint16])
@pytest.mark.parametrize("n,kind", [(12288, "normal"), (1, "normal"), (33, "normal"), (8191, "normal"),
                                    (12288, "zero"), (12288, "nan")])
def test_norm_swiglu_matches_calls(env, quantize, dtype, n, kind):
    """Two coordinates per wave: n = 1 and 33 leave a ragged last wave (its
    tail coordinate clamped); n = 8191 an odd count.  gate, up and act,
    the codes, scale, normalised row, the maximum (reset, then folded) and
    the act's codes and scale all equal the separate calls' bits."""
    print(f"norm+swiglu n={n} {kind} {np.dtype(dtype).name} quantize={quantize}", flush=True)
    rng = np.random.default_rng(n + (7 if quantize else 0) + len(kind))
    x = make_row(rng, kind)
    gain = (1 + 0.3 * rng.standard_normal(4096)).astype(F32)
    wg = rng.integers(-127, 128, (n, 4096), dtype=np.int8)
    wu = rng.integers(-127, 128, (n, 4096), dtype=np.int8)
    sg = (rng.random(n) / 64 + 1e-4).astype(F32)
    su = (rng.random(n) / 64 + 1e-4).astype(F32)
    calls, folded = run_swiglu_both(env, x, gain, wg, sg, wu, su, dtype, quantize)
    for key in ("q", "sc", "normed", "mx", "gate", "up", "act") + (("qo", "so") if quantize else ()):
        assert nan_same(folded[key], calls[key]), key
    if kind == "normal":
        _, wq, wsc, _ = oracle.norm_quantize(x[None, :], gain)
        assert np.array_equal(folded["q"], wq.reshape(-1)) and np.array_equal(bits(folded["sc"]), bits(wsc))
        acc, of, ob = oracle.linear(wq.reshape(1, -1), wsc, wg, sg, 4096, threads=8)
        want_gate = ob if dtype == np.uint16 else of
        assert same_bits(folded["gate"], want_gate), "gate against the oracle"


def run_mlp_both(env, x, gain, wg, sg, wu, su, wd, sd, resid, act_dtype, out_dtype, optional=True):
    """(separate calls, folded call): norm_quantize_linear_swiglu with the
    act's codes, then linear_residual (linear without a residual) on them,
    against norm_quantize_mlp."""
    _, mod, s = env
    n_ff, n = sg.size, sd.size
    xb, gb = dev(s, x), dev(s, gain)
    wgb, sgb, wub, sub, wdb, sdb = dev(s, wg), dev(s, sg), dev(s, wu), dev(s, su), dev(s, wd), dev(s, sd)
    rb = dev(s, resid) if resid is not None else None
    res = {}
    for mode in ("calls", "folded"):
        q = DeviceBuffer.zeroed(s, 4096, np.int8)
        sc = DeviceBuffer.zeroed(s, 1, np.float32)
        nb = DeviceBuffer.zeroed(s, 4096, np.float32)
        mx = dev(s, np.array([JUNK], np.uint32))
        gate, up, act = (DeviceBuffer.zeroed(s, n_ff, act_dtype) for _ in range(3))
        qa = DeviceBuffer.zeroed(s, n_ff, np.int8)
        sa = DeviceBuffer.zeroed(s, 1, np.float32)
        out = DeviceBuffer.zeroed(s, n, out_dtype)
        comb = DeviceBuffer.zeroed(s, n, out_dtype) if resid is not None else None
        if mode == "calls":
            mod.norm_quantize_linear_swiglu(s, None, xb, gb, nb, q, sc, wgb, sgb, gate, wub, sub, up, act, mx,
                                            qa, sa)
            if resid is not None:
                mod.linear_residual(s, None, qa, sa, wdb, sdb, n_ff, rb, out, comb)
            else:
                mod.linear(s, None, qa, sa, wdb, sdb, n_ff, out)
        else:
            mod.norm_quantize_mlp(s, None, xb, gb, nb if optional else None, q, sc, wgb, sgb, gate, wub, sub, up,
                                  act, mx, wdb, sdb, out, rb, comb, qa if optional else None,
                                  sa if optional else None)
        s.synchronize()
        res[mode] = dict(q=q.to_host_vec(s), sc=sc.to_host_vec(s), normed=nb.to_host_vec(s),
                         mx=mx.to_host_vec(s), gate=gate.to_host_vec(s), up=up.to_host_vec(s),
                         act=act.to_host_vec(s), qa=qa.to_host_vec(s), sa=sa.to_host_vec(s),
                         out=out.to_host_vec(s), comb=comb.to_host_vec(s) if comb is not None else None)
    return res["calls"], res["folded"]


def mlp_weights(rng, n):
    wg = rng.integers(-127, 128, (12288, 4096), dtype=np.int8)
    wu = rng.integers(-127, 128, (12288, 4096), dtype=np.int8)
    sg = (rng.random(12288) / 64 + 1e-4).astype(F32)
    su = (rng.random(12288) / 64 + 1e-4).astype(F32)
    wd = rng.integers(-127, 128, (n, 12288), dtype=np.int8)
    sd = (rng.random(n) / 64 + 1e-4).astype(F32)
    return wg, sg, wu, su, wd, sd


@pytest.mark.parametrize("act_dtype,out_dtype,res", [(np.float32, np.uint16, True), (np.uint16, np.uint16, True),
                                                     (np.float32, np.float32, True), (np.uint16, np.float32, False)])
@pytest.mark.parametrize("n,kind", [(4096, "normal"), (1000, "normal"), (1, "normal"), (4096, "zero"),
                                    (4096, "nan")])
def test_norm_mlp_matches_calls(env, act_dtype, out_dtype, res, n, kind):
    """The MLP block in two launches against norm_quantize_linear_swiglu
    (with the act's codes) then linear_residual / linear: the norm's codes,
    scale and row, gate / up / act, the maximum (reset by the norm, then the
    act maximum folded in by the down GEMV's first workgroup), the act's
    codes and scale, out and combined, bit for bit.  n = 1000 and 1 leave a
    partly empty last 16-row workgroup (its rows clamped, not stored); the
    zero row gives an all-zero act (scale from the floor), the NaN row NaN
    gate / up / act (the maximum skips NaN).  The down outputs are also
    checked against the oracle's quantize_with_max and linear."""
    print(f"norm mlp n={n} {kind} act={np.dtype(act_dtype).name} out={np.dtype(out_dtype).name} res={res}",
          flush=True)
    rng = np.random.default_rng(n * 3 + len(kind) + (1 if res else 0))
    x = make_row(rng, kind)
    gain = (1 + 0.3 * rng.standard_normal(4096)).astype(F32)
    wg, sg, wu, su, wd, sd = mlp_weights(rng, n)
    resid = oracle.bf16_rne(rng.standard_normal(n).astype(F32)) if res else None
    calls, folded = run_mlp_both(env, x, gain, wg, sg, wu, su, wd, sd, resid, act_dtype, out_dtype)
    for key in ("q", "sc", "normed", "mx", "gate", "up", "act", "qa", "sa", "out") + (("comb",) if res else ()):
        assert nan_same(folded[key], calls[key]), key
    if kind != "nan":
        act = folded["act"]
        act32 = (act.astype(np.uint32) << 16).view(F32) if act_dtype == np.uint16 else act
        wq, wsc = oracle.quantize_with_max(act32, 12288, folded["mx"])
        assert np.array_equal(folded["qa"], wq) and np.array_equal(bits(folded["sa"]), bits(wsc))
        acc, of, ob = oracle.linear(wq.reshape(1, -1), wsc, wd, sd, 12288, threads=8)
        assert same_bits(folded["out"], ob if out_dtype == np.uint16 else of), "out against the oracle"
        if res:
            want = bits(oracle.residual(resid, of))
            want = (want >> 16).astype(np.uint16) if out_dtype == np.uint16 else want.view(F32)
            assert same_bits(folded["comb"], want), "combined against the oracle"


def test_norm_mlp_optional_outputs(env):
    """Without the normalised row and the act's codes / scale the required
    outputs are unchanged."""
    rng = np.random.default_rng(41)
    x = make_row(rng)
    gain = (1 + 0.3 * rng.standard_normal(4096)).astype(F32)
    wg, sg, wu, su, wd, sd = mlp_weights(rng, 4096)
    resid = oracle.bf16_rne(rng.standard_normal(4096).astype(F32))
    calls, folded = run_mlp_both(env, x, gain, wg, sg, wu, su, wd, sd, resid, np.float32, np.uint16,
                                 optional=False)
    for key in ("q", "sc", "mx", "gate", "up", "act", "out", "comb"):
        assert nan_same(folded[key], calls[key]), key


def test_norm_mlp_graph_replay(env):
    """The MLP block captured in a graph: every replay reproduces the eager
    result (maxima restored to junk between replays, outputs cleared), with
    eager work between the replays."""
    _, mod, s = env
    rng = np.random.default_rng(43)
    x = make_row(rng)
    gain = (1 + 0.3 * rng.standard_normal(4096)).astype(F32)
    n = 4096
    wg, sg, wu, su, wd, sd = mlp_weights(rng, n)
    resid = oracle.bf16_rne(rng.standard_normal(n).astype(F32))
    xb, gb, rb = dev(s, x), dev(s, gain), dev(s, resid)
    wgb, sgb, wub, sub, wdb, sdb = dev(s, wg), dev(s, sg), dev(s, wu), dev(s, su), dev(s, wd), dev(s, sd)
    q = DeviceBuffer.zeroed(s, 4096, np.int8)
    sc = DeviceBuffer.zeroed(s, 1, np.float32)
    mx = dev(s, np.array([JUNK], np.uint32))
    gate, up, act = (DeviceBuffer.zeroed(s, 12288, np.float32) for _ in range(3))
    qa = DeviceBuffer.zeroed(s, 12288, np.int8)
    sa = DeviceBuffer.zeroed(s, 1, np.float32)
    out = DeviceBuffer.zeroed(s, n, np.uint16)
    comb = DeviceBuffer.zeroed(s, n, np.uint16)

    def block():
        mod.norm_quantize_mlp(s, None, xb, gb, None, q, sc, wgb, sgb, gate, wub, sub, up, act, mx, wdb, sdb, out,
                              rb, comb, qa, sa)

    bufs = (q, sc, mx, gate, up, act, qa, sa, out, comb)
    block()
    s.synchronize()
    want = [b.to_host_vec(s) for b in bufs]
    g = Graph(s)
    with g:
        block()
    for _ in range(3):
        for b in bufs:
            b.fill_zero(s)
        mx.copy_from_host(s, np.array([JUNK], np.uint32))
        s.synchronize()
        g.launch()
        s.synchronize()
        got = [b.to_host_vec(s) for b in bufs]
        for a, b in zip(got, want):
            assert nan_same(a, b)
