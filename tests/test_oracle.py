"""Pin the CPU oracle (oracle/) before it is trusted as the GPU checker.

Each oracle function is checked against something it does not compute
itself: the committed torch-CPU fixtures (reference fixture recipe), the
reference's own deterministic test sets and KATs, closed forms evaluated in
f64 / numpy, or brute force.  A second group plants plausible mistakes (in
Python, on the CPU) and shows the same checks reject them.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from conftest import (argmax_cases, argmax_expected, bf16_ulp_distance,
                      reference_tolerance_ok, rounding_expected, rounding_probe_inputs)

F32 = np.float32


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# --------------------------------------------------------------- bf16 / round
def test_bf16_matches_torch_rne_on_finite_values():
    rng = np.random.default_rng(1)
    u = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    # force a block of exact ties (low half 0x8000) with both parities
    u[:4096] = (u[:4096] & 0xFFFF0000) | 0x8000
    x = u.view(np.float32)
    x = x[np.isfinite(x) & (np.abs(x) < np.finfo(np.float32).max / 2)]
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    got = oracle.bf16_rne(x)
    assert np.array_equal(bits(got), bits(want))
    # the C scalar agrees with the vectorised formula
    L = oracle.lib()
    for v in x[:2000]:
        assert np.float32(L.orc_bf16_rne(float(v))).view(np.uint32) == oracle.bf16_rne(np.array([v]))[0].view(np.uint32)


def test_bf16_idempotent_on_every_bf16_encoding():
    enc = (np.arange(65536, dtype=np.uint32) << 16)
    x = enc.view(np.float32)
    fin = np.isfinite(x)
    assert np.array_equal(bits(oracle.bf16_rne(x[fin])), enc[fin])


def test_round_matches_reference_probe_set():
    x = rounding_probe_inputs()
    assert x.size == 1_328_443
    assert np.array_equal(oracle.round_i8(x), rounding_expected(x))


# --------------------------------------------------------------- quantize
def test_quantize_matches_fixtures(fixtures):
    cases = fixtures.cases("quantize")
    assert len(cases) == 3
    for c in cases:
        x = fixtures.tensor(c, "x")
        q, s = oracle.quantize(x, c["width"])
        assert np.array_equal(q, fixtures.tensor(c, "q").reshape(-1)), c["name"]
        assert np.array_equal(bits(s), bits(fixtures.tensor(c, "scale").reshape(-1))), c["name"]


def test_weight_quantize_matches_prepare_recipe(fixtures):
    # tools/prepare.py:79-83: per-output-channel quantization of BF16 weights
    (c,) = fixtures.cases("weight_quantize")
    w = fixtures.tensor(c, "w").view(np.uint16)
    q, s = oracle.quantize_bf16(w, w.shape[1])
    assert np.array_equal(q, fixtures.tensor(c, "q").reshape(-1))
    assert np.array_equal(bits(s), bits(fixtures.tensor(c, "scale")))
    assert q.min() >= -127 and (s > 0).all()


def test_quantize_kats():
    # zero row: scale is the floor 1e-8/127, all q zero
    q, s = oracle.quantize(np.zeros(4096, F32), 4096)
    assert bits(s)[0] == bits(np.array([F32(1e-8) / F32(127)]))[0]
    assert not q.any()
    # absmax 127 -> scale exactly 1.0; ties go to even
    x = np.zeros(128, F32)
    x[:8] = [127, -127, .5, -.5, 1.5, -1.5, 2.5, -2.5]
    q, s = oracle.quantize(x, 128)
    assert s[0] == 1.0
    assert list(q[:8]) == [127, -127, 0, 0, 2, -2, 2, -2]
    # NaN is ignored by the max and quantizes to 0; inf saturates the scale
    x = np.array([np.nan, 2.0, -4.0, 1.0], F32)
    q, s = oracle.quantize(x, 4)
    assert s[0] == F32(4.0) / F32(127.0)
    assert list(q) == [0, 64, -127, 32]
    x = np.array([np.inf, 1.0, -1.0, 0.0], F32)
    q, s = oracle.quantize(x, 4)
    assert np.isinf(s[0]) and list(q) == [0, 0, 0, 0]


def test_quantize_closed_form_random_rows():
    rng = np.random.default_rng(7)
    x = oracle.bf16_rne(rng.standard_normal(5 * 4096).astype(F32))
    x[3 * 4096 + 17] *= 50
    q, s = oracle.quantize(x, 4096)
    xr = x.reshape(5, 4096)
    want_s = np.maximum(np.abs(xr).max(1), F32(1e-8)).astype(F32) / F32(127)
    assert np.array_equal(bits(s), bits(want_s.astype(F32)))
    ratio = (xr / want_s[:, None].astype(F32)).astype(F32)  # numpy f32 RN division
    want_q = np.clip(np.rint(ratio.astype(np.float64)), -127, 127).astype(np.int8)
    assert np.array_equal(q.reshape(5, 4096), want_q)


def test_quantize_bf16_input_matches_f32_input():
    rng = np.random.default_rng(3)
    x = oracle.bf16_rne(rng.standard_t(3, size=3 * 12288).astype(F32) * 3)
    xb = (bits(x) >> 16).astype(np.uint16)
    assert np.array_equal(np.concatenate(oracle.quantize(x, 12288)[:1]),
                          oracle.quantize_bf16(xb, 12288)[0])
    assert np.array_equal(bits(oracle.quantize(x, 12288)[1]), bits(oracle.quantize_bf16(xb, 12288)[1]))


def test_quantize_with_max_equals_scan(fixtures):
    # src/conformance.rs:129-152: the producer-max path reproduces the scan
    for c in fixtures.cases("quantize"):
        x = fixtures.tensor(c, "x").reshape(-1)
        w = c["width"]
        maxima = np.array([oracle.absmax_bits(r) for r in x.reshape(-1, w)], np.uint32)
        q, s = oracle.quantize_with_max(x, w, maxima)
        assert np.array_equal(q, fixtures.tensor(c, "q").reshape(-1))
        assert np.array_equal(bits(s), bits(fixtures.tensor(c, "scale").reshape(-1)))


# --------------------------------------------------------------- linear
def test_linear_matches_fixtures(fixtures):
    cases = fixtures.cases("linear")
    assert len(cases) == 5
    for c in cases:
        k = c["width"]
        q, asc, w, ws = (fixtures.tensor(c, key) for key in ("q", "asc", "w", "ws"))
        acc, out, outb = oracle.linear(q, asc, w, ws, k)
        assert np.array_equal(acc, fixtures.tensor(c, "acc").reshape(-1)), c["name"]
        assert np.array_equal(bits(out), bits(fixtures.tensor(c, "out").reshape(-1))), c["name"]
        assert np.array_equal(outb, (bits(out) >> 16).astype(np.uint16))


def test_linear_worst_case_accumulator():
    k = 12288
    q = np.full(k, 127, np.int8)
    w = np.stack([np.full(k, 127, np.int8), np.full(k, -127, np.int8)])
    acc = oracle.linear_i32(q, w, 1, 2, k)
    assert list(acc) == [198_193_152, -198_193_152]


def test_linear_bruteforce_int64_and_numpy_epilogue():
    rng = np.random.default_rng(11)
    for m, n, k in ((1, 7, 16), (3, 33, 128), (17, 5, 4096), (4, 65, 12288)):
        q = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
        w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        asc = (rng.random(m) / 64).astype(F32)
        ws = (rng.random(n) / 64).astype(F32)
        acc, out, outb = oracle.linear(q, asc, w, ws, k, threads=4)
        want = q.astype(np.int64) @ w.astype(np.int64).T
        assert np.array_equal(acc.reshape(m, n), want)
        t = (want.astype(np.int32).astype(F32) * asc[:, None]).astype(F32)
        t = (t * ws[None, :]).astype(F32)
        assert np.array_equal(bits(out), bits(oracle.bf16_rne(t.reshape(-1))))
        assert np.array_equal(oracle.linear_i32(q, w, m, n, k, threads=1), acc)


def test_residual_closed_form():
    rng = np.random.default_rng(5)
    out = oracle.bf16_rne(rng.standard_normal(4096).astype(F32))
    res = ((np.arange(4096) % 17).astype(F32) - 8) * F32(0.0625)   # src/conformance.rs:236-241
    want = torch.from_numpy((res + out).astype(F32)).bfloat16().float().numpy()
    assert np.array_equal(bits(oracle.residual(res, out)), bits(want))


# --------------------------------------------------------------- swiglu
def test_swiglu_matches_fixture_within_reference_tolerance(fixtures):
    (case,) = fixtures.cases("swiglu")
    g, u = fixtures.tensor(case, "gate"), fixtures.tensor(case, "up")
    want = fixtures.tensor(case, "out")
    act, mx = oracle.swiglu(g, u)
    assert reference_tolerance_ok(act, want)
    # torch evaluates silu as x * sigmoid(x): a different rounding order, so
    # values may differ by one BF16 ulp, never more.
    same_sign = np.sign(act) == np.sign(want)
    assert bf16_ulp_distance(act[same_sign], want[same_sign]).max() <= 1
    assert mx == int(bits(np.maximum(np.abs(act).max(), F32(1e-8)))[0])


def test_silu_mul_against_float64_and_closed_forms():
    rng = np.random.default_rng(11)
    g = oracle.bf16_rne(rng.uniform(-90, 90, 200_000).astype(F32))
    u = oracle.bf16_rne(rng.standard_normal(200_000).astype(F32))
    act, _ = oracle.swiglu(g, u)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    exact = g64 / (1.0 + np.exp(-g64)) * u64
    want = oracle.bf16_rne(exact.astype(F32))
    assert reference_tolerance_ok(act, want)
    nz = (want != 0) & (np.sign(act) == np.sign(want))
    d = bf16_ulp_distance(act[nz], want[nz])
    assert d.max() <= 1 and np.mean(d) < 0.01
    # closed forms: silu(0) = 0; silu(g) = g for large g; silu(g) -> 0- for very negative g
    assert oracle.lib().orc_silu_mul(0.0, 3.0) == 0.0
    assert oracle.lib().orc_silu_mul(100.0, 1.5) == 150.0
    assert abs(oracle.lib().orc_silu_mul(-100.0, 1.0)) < 1e-40
    # a planted operand swap (silu(up) * gate) is far outside the tolerance
    swapped, _ = oracle.swiglu(u, g)
    assert not reference_tolerance_ok(swapped, want)


def test_swiglu_maximum_ignores_nan_and_keeps_floor():
    act, mx = oracle.swiglu(np.zeros(8, F32), np.ones(8, F32))
    assert mx == int(bits(F32(1e-8))[0])
    g = np.array([1.0, np.nan, -4.0], F32)
    act, mx = oracle.swiglu(g, np.ones(3, F32))
    assert np.isnan(act[1])
    assert mx == int(bits(np.abs(act[[0, 2]]).max())[0])


# --------------------------------------------------------------- argmax
def test_argmax_reference_cases():
    cases = argmax_cases()
    assert len(cases) == 20
    for x in cases:
        assert oracle.argmax(x) == argmax_expected(x)
    # src/model.rs:268-272
    assert oracle.argmax(np.array([1, 3, 3], F32)) == 1
    assert oracle.argmax(np.array([np.nan], F32)) == oracle.SENTINEL
    assert oracle.argmax(np.array([], F32)) == oracle.SENTINEL
    assert oracle.argmax(np.array([np.inf], F32)) == oracle.SENTINEL
    assert oracle.argmax(np.array([-0.0, 0.0], F32)) == 0


def test_argmax_matches_numpy_first_occurrence():
    rng = np.random.default_rng(9)
    for _ in range(50):
        x = oracle.bf16_rne(rng.standard_normal(2000).astype(F32)) * 4
        x = oracle.bf16_rne(x)
        assert oracle.argmax(x) == int(np.argmax(x))


def test_linear_argmax_composition():
    rng = np.random.default_rng(13)
    k, n = 256, 3000
    q = rng.integers(-127, 128, size=k, dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    w[2500] = w[1200]          # a guaranteed tie: lower index must win
    w[1200] = 127 * np.sign(q)
    w[2500] = w[1200]
    ws = np.full(n, 0.01, F32)
    tok, logits = oracle.linear_argmax(q, np.array([0.05], F32), w, ws, k)
    _, out, _ = oracle.linear(q, np.array([0.05], F32), w, ws, k)
    assert np.array_equal(bits(logits), bits(out))
    assert tok == 1200 == argmax_expected(logits)


# --------------------------------------------------------------- synthetic
def test_mix64_splitmix_vectors():
    # Vigna's splitmix64 seeded with 0: the first outputs are the finaliser
    # applied to k * 0x9E3779B97F4A7C15.
    g = 0x9E3779B97F4A7C15
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    for i, v in enumerate(want, start=1):
        assert oracle.mix64((i * g) & (2**64 - 1)) == v


def test_synth_ranges_and_spread():
    v = oracle.synth_i8(1, 7, 0, 1 << 20)
    assert v.min() == -127 and v.max() == 127
    counts = np.bincount(v.astype(np.int64) + 127, minlength=255)
    assert counts.size == 255 and counts.min() > 0.9 * counts.mean()
    # windows agree with the whole
    assert np.array_equal(oracle.synth_i8(1, 7, 12345, 1000), v[12345:13345])
    f = oracle.synth_f32(2, 3, 0, 100000, 1e-3, 1e-2)
    assert f.min() >= F32(1e-3) and f.max() < F32(1e-2)
    assert abs(float(f.mean()) - 5.5e-3) < 1e-4
    assert not np.array_equal(oracle.synth_i8(1, 8, 0, 64), v[:64])


# --------------------------------------------------------------- planted mistakes
def test_epilogue_order_is_pinned():
    """(acc*asc)*ws, not acc*(asc*ws): random triples where the two orders
    land on different BF16 values exist, and the oracle follows the
    reference order (src/kernels.rs:290) on all of them."""
    rng = np.random.default_rng(21)
    m = n = 1024
    acc = rng.integers(-198_193_152, 198_193_153, size=m * n).astype(np.int32)
    asc = (rng.random(m) / 64).astype(F32)
    ws = (rng.random(n) / 64).astype(F32)
    out, _ = oracle.epilogue(acc, asc, ws)
    a = acc.reshape(m, n).astype(F32)
    ref = oracle.bf16_rne(((a * asc[:, None]).astype(F32) * ws[None, :]).astype(F32).reshape(-1))
    fused = oracle.bf16_rne((a * (asc[:, None] * ws[None, :]).astype(F32)).astype(F32).reshape(-1))
    assert np.array_equal(bits(out), bits(ref))
    assert np.any(bits(fused) != bits(ref))
    # truncation instead of RNE is rejected by the fixtures' values too
    trunc = bits((a * asc[:, None]).astype(F32) * ws[None, :]).reshape(-1) & 0xFFFF0000
    assert np.any(trunc != bits(ref))


def test_division_not_reciprocal_is_pinned():
    """RN division x/s (src/kernels.rs:446): pairs exist where x*(1/s)
    rounds to another integer; the oracle follows the division."""
    rng = np.random.default_rng(0)
    mx = (rng.random(200000).astype(F32) * F32(8) + F32(0.25))
    s = (mx / F32(127)).astype(F32)
    x = ((rng.integers(-126, 126, 200000) + 0.5).astype(F32) * s).astype(F32)
    by_div = np.rint((x / s).astype(F32).astype(np.float64))
    by_rcp = np.rint((x * (F32(1) / s)).astype(F32).astype(np.float64))
    hit = np.flatnonzero(by_div != by_rcp)
    assert hit.size > 0
    for i in hit[:50]:
        q, sc = oracle.quantize_with_max(x[i:i + 1], 1, mx[i:i + 1].view(np.uint32))
        assert sc[0] == s[i]
        assert q[0] == by_div[i] != by_rcp[i]


def test_planted_operand_and_tie_mistakes_are_rejected(fixtures):
    lin = fixtures.cases("linear")[3]          # 65 rows, width 4096
    q, asc, w, ws = (fixtures.tensor(lin, key) for key in ("q", "asc", "w", "ws"))
    acc = fixtures.tensor(lin, "acc").reshape(-1)
    # transposed / reversed weight operand
    wt = np.ascontiguousarray(w.reshape(33, 4096)[:, ::-1])
    assert not np.array_equal(oracle.linear(q, asc, wt, ws, 4096)[0], acc)
    # dropped last K term
    q2 = q.copy().reshape(65, 4096)
    q2[:, -1] = 0
    assert not np.array_equal(oracle.linear(q2, asc, w, ws, 4096)[0], acc)
    # rounding ties away from zero instead of to even
    qc = fixtures.cases("quantize")[2]
    x = fixtures.tensor(qc, "x").reshape(3, -1)
    s = fixtures.tensor(qc, "scale").reshape(3, 1)
    away = np.clip(np.sign(x / s) * np.floor(np.abs(x / s) + 0.5), -127, 127).astype(np.int8)
    assert not np.array_equal(away, fixtures.tensor(qc, "q"))
    # argmax keeping the last of tied maxima
    x = argmax_cases()[-1]
    assert int(x.size - 1 - np.argmax(x[::-1])) != oracle.argmax(x)


# ------------------------------------------------------------------ norm_quantize
def _tree_sum_numpy(row: np.ndarray) -> np.float32:
    """Independent numpy form of the reference's sum tree (src/kernels.rs:354-392):
    partial t = sequential f32 sum over x[t::256]**2, then p[:d] += p[d:2d]."""
    sq = (row.astype(np.float32) * row.astype(np.float32)).astype(np.float32).reshape(16, 256)
    p = np.zeros(256, np.float32)
    for i in range(16):
        p = (p + sq[i]).astype(np.float32)
    d = 128
    while d:
        p[:d] = (p[:d] + p[d:2 * d]).astype(np.float32)
        d //= 2
    return p[0]


def test_norm_sum_tree_order_is_pinned():
    rng = np.random.default_rng(71)
    rows = (rng.standard_normal((8, 4096)) * np.exp(rng.uniform(-6, 6, (8, 4096)))).astype(np.float32)
    differs = 0
    for row in rows:
        got = oracle.norm_sum_sq(row)
        assert np.float32(got) == _tree_sum_numpy(row)
        seq = np.float32(0)
        for v in row:
            seq = np.float32(seq + np.float32(v * v))
        differs += np.float32(got) != seq
        assert abs(got - float(np.sum(row.astype(np.float64) ** 2))) <= 1e-5 * float(np.sum(row.astype(np.float64) ** 2))
    assert differs > 0, "inputs must distinguish the tree from a sequential sum"


def test_norm_sum_exact_on_representable_squares():
    rng = np.random.default_rng(72)
    row = rng.choice(np.array([-3, -2, -1, -0.5, 0, 0.5, 1, 2, 3], np.float32), 4096)
    assert oracle.norm_sum_sq(row) == float(np.sum(row.astype(np.float64) ** 2))


def test_norm_quantize_kats():
    gain = np.ones(4096, np.float32)
    # all ones: mean 1, inv = 1/sqrt(f32(1 + 1e-6)) -> out rounds to BF16 1.0, q = 127
    out, q, s, mx = oracle.norm_quantize(np.ones((1, 4096), np.float32), gain)
    assert np.all(out == 1.0) and np.all(q == 127)
    assert s[0] == np.float32(1.0) / np.float32(127.0) and mx[0] == int(np.float32(1e-8).view(np.uint32))
    # zero row: out 0, q 0, scale at the 1e-8 floor
    out, q, s, _ = oracle.norm_quantize(np.zeros((1, 4096), np.float32), gain)
    assert np.all(out == 0) and np.all(q == 0) and s[0] == np.float32(1e-8) / np.float32(127.0)
    # a NaN anywhere: every output NaN, quantized to 0
    x = np.ones((1, 4096), np.float32)
    x[0, 7] = np.nan
    out, q, s, _ = oracle.norm_quantize(x, gain)
    assert np.isnan(out).all() and np.all(q == 0)


def test_norm_against_float64_and_fixture(fixtures):
    (case,) = fixtures.cases("norm")
    x, gain, want = (fixtures.tensor(case, k) for k in ("x", "gain", "out"))
    got = oracle.norm_rows(x, gain)
    assert reference_tolerance_ok(got, want)
    assert np.all(got[0] == 0)
    rng = np.random.default_rng(73)
    x = (rng.standard_normal((5, 4096)) * [[1e-3], [1], [30], [1e3], [1]]).astype(np.float32)
    g = (1 + 0.25 * rng.standard_normal(4096)).astype(np.float32)
    got = oracle.norm_rows(x, g)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-6) * g
    # one BF16 rounding (at most 2^-8 of the value) plus the f32 steps before
    # it; the 1e-3 row has mean(x^2) = 1e-6, where the epsilon halves 1/rms
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -7.95)


def test_norm_quantize_equals_norm_then_quantize():
    """src/conformance.rs:166-199: the fused operator equals `norm`, then `quantize`."""
    rng = np.random.default_rng(74)
    x = rng.standard_normal((4, 4096)).astype(np.float32)
    g = rng.standard_normal(4096).astype(np.float32)
    out, q, s, mx = oracle.norm_quantize(x, g)
    assert np.array_equal(out, oracle.norm_rows(x, g))
    q2, s2 = oracle.quantize(out, 4096)
    assert np.array_equal(q.reshape(-1), q2) and np.array_equal(s, s2)
    assert np.all(mx == np.float32(1e-8).view(np.uint32))


# ------------------------------------------------------------------ packed BF16 head
def _unpack_all_numpy(words, offsets, exceptions, n):
    """Independent vectorised decoder of src/kernels.rs:295-314."""
    i = np.arange(n, dtype=np.int64)
    step = (i % 256) // 32
    word = i // 256 * 96 + i % 32 + (step * 12 // 32) * 32
    shift = (step * 12 % 32).astype(np.uint64)
    lo = words[word].astype(np.uint64)
    hi = np.where(word + 32 < words.size, words[np.minimum(word + 32, words.size - 1)], 0).astype(np.uint64)
    code = ((lo | (hi << np.uint64(32))) >> shift) & np.uint64(4095)
    code = code.astype(np.int64)
    direct = ((code & 128) << 8) | (((code >> 8) + 109) << 7) | (code & 127)
    esc = exceptions[np.minimum(offsets[i // 256].astype(np.int64) + (code & 255), exceptions.size - 1)]
    return np.where(code >> 8 == 15, esc, direct).astype(np.uint16)


def _reference_exhaustive_input():
    """src/packing.rs tests and src/conformance.rs:716-720: every BF16 pattern,
    then (i * 40503) mod 2^16 for i < 65536 (mixed chunks)."""
    a = np.arange(65536, dtype=np.uint32)
    return np.concatenate([a, (a * 40503) % 65536]).astype(np.uint16)


def test_bf16_pack_round_trips_every_pattern():
    v = _reference_exhaustive_input()
    words, offsets, exc = oracle.bf16_pack(v)
    assert np.array_equal(_unpack_all_numpy(words, offsets, exc, v.size), v)
    for i in range(0, v.size, 4099):
        assert oracle.bf16_unpack_at(words, offsets, exc, i) == v[i]


def test_bf16_pack_format_kats():
    v = np.zeros(256, np.uint16)
    v[0] = np.float32(2.0 ** -18).view(np.uint32) >> 16        # exponent 109: direct code 0x000
    v[1] = (np.float32(-0.1).view(np.uint32) >> 16)            # exponent 123: direct, sign bit
    v[2] = np.float32(0.125).view(np.uint32) >> 16             # exponent 124: escapes
    v[32] = 0x3C00                                             # lane 0, second code
    words, offsets, exc = oracle.bf16_pack(v)
    assert words.size == 96 and offsets.tolist() == [0]
    # lane 0's first code sits in bits 0-11 of word 0, its second in bits 12-23
    assert words[0] & 0xFFF == 0 and (words[0] >> 12) & 0xFFF == ((0x3C00 >> 7 & 255) - 109) << 8
    assert (words[1] & 0xFFF) == (((v[1] >> 7) & 255) - 109) << 8 | 128 | (v[1] & 127)
    # 0.125 is the chunk's first escape (index 0); the 252 zeros (exponent 0)
    # escape after it, in value order -> 253 exceptions
    assert exc.size == 253 and exc[0] == v[2] and (words[2] & 0xFFF) == 0xF00
    assert (words[3] & 0xFFF) == 0xF01 and exc[1] == 0


def _head_numpy(x4096, w_bits):
    """Independent numpy statement of src/kernels.rs:2233-2257's order."""
    w = (w_bits.astype(np.uint32) << 16).view(np.float32).reshape(-1, 4096)
    x = x4096.astype(np.float32)
    prod = (x[None, :] * w).astype(np.float32).reshape(w.shape[0], 128, 32)
    lane = np.zeros((w.shape[0], 32), np.float32)
    for i in range(128):
        lane = (lane + prod[:, i, :]).astype(np.float32)
    d = 16
    while d:
        lane[:, :d] = (lane[:, :d] + lane[:, d:2 * d]).astype(np.float32)
        d //= 2
    return lane[:, 0]


def test_head_order_is_pinned(fixtures):
    (case,) = fixtures.cases("head")
    x, w, want = (fixtures.tensor(case, k) for k in ("x", "w", "out"))
    got = oracle.head_bf16(x, w.view(np.uint16))
    assert reference_tolerance_ok(got, want)
    rng = np.random.default_rng(81)
    x = (rng.standard_normal(4096) * np.exp(rng.uniform(-4, 4, 4096))).astype(np.float32)
    wb = (rng.standard_normal((64, 4096)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    got = oracle.head_bf16(x, wb)
    tree = _head_numpy(x, wb)
    # before the final BF16 rounding the tree sums agree bit for bit
    assert np.array_equal(got.view(np.uint32), oracle.bf16_rne(tree).view(np.uint32))
    # the tree sum (before BF16) separates the reference order from a
    # sequential one on these rows
    wf = (wb.astype(np.uint32) << 16).view(np.float32)
    differs = 0
    for r in range(8):
        s = np.float32(0)
        for j in range(4096):
            s = np.float32(s + np.float32(x[j] * wf[r, j]))
        differs += s != tree[r]
    assert differs > 0
