"""CPU check of quant_code (inferrous_amd/csrc/device_common.hpp), the
division-free form of quantize's code used where a workgroup recomputes a
row's codes: round_i8(RN(v * RN(1 / s))) with the division taken instead
when v * r lies within 2^-12 of a half-integer.  The claim is that it equals
round_i8(RN(v / s)) (src/kernels.rs:441-449) whenever s = RN(m / 127) for a
maximum m >= |v|.  numpy float32 arithmetic is IEEE round-to-nearest, like
the device's v_mul_f32 and its correctly rounded division; the reference side
is the oracle's orc_round_i8 of the float32 quotient.  Inputs: uniform rows
over 60 orders of magnitude of m, the floor maximum, and values a few ulps
either side of every half-integer boundary k + 0.5 (the only places the two
forms could part), plus zeros, +-m and NaN."""
from __future__ import annotations

import numpy as np

import oracle

F = np.float32
THR = F(0.5) - F(2.0 ** -12)


def quant_code(v, s):
    r = F(1) / s
    y = (v * r).astype(F)
    ry = np.rint(y)
    fast = np.abs(y - ry) < THR
    q = np.where(fast, np.clip(ry, -127, 127), 0).astype(np.int8)
    q[~fast] = oracle.round_i8((v[~fast] / s).astype(F))
    return q, fast


def test_quant_code_equals_the_division():
    rng = np.random.default_rng(5)
    taken = 0
    for trial in range(60):
        m = F(1e-8) if trial == 0 else F(np.exp(rng.uniform(-30, 30)))
        s = F(m / F(127))
        v = (rng.uniform(-1, 1, 200_000) * m).astype(F)
        near = ((rng.integers(-127, 127, 50_000).astype(F) + F(0.5)) * s).astype(F)
        for _ in range(4):
            step = np.where(rng.random(near.size) < 0.5, F(np.inf), F(-np.inf)).astype(F)
            near = np.where(rng.random(near.size) < 0.7, np.nextafter(near, step), near).astype(F)
        near = np.clip(near, -m, m).astype(F)
        v = np.concatenate([v, near, np.array([0, -0.0, m, -m, np.nan], F)])
        want = oracle.round_i8((v / s).astype(F))
        got, fast = quant_code(v, s)
        assert np.array_equal(got, want), f"m={m}"
        taken += int((~fast).sum())
    assert taken > 0  # the division path is exercised


def test_quant_code_rejects_a_wider_window():
    """The 2^-12 window is needed: with no window at all (always the
    reciprocal), values next to a half-integer come out differently."""
    rng = np.random.default_rng(6)
    diffs = 0
    for _ in range(20):
        m = F(np.exp(rng.uniform(-10, 10)))
        s = F(m / F(127))
        near = ((rng.integers(-127, 127, 100_000).astype(F) + F(0.5)) * s).astype(F)
        for _ in range(2):
            near = np.nextafter(near, np.where(rng.random(near.size) < 0.5, F(np.inf), F(-np.inf)).astype(F))
        near = np.clip(near, -m, m).astype(F)
        y = (near * (F(1) / s)).astype(F)
        plain = np.clip(np.rint(y), -127, 127).astype(np.int8)
        diffs += int((plain != oracle.round_i8((near / s).astype(F))).sum())
    assert diffs > 0
