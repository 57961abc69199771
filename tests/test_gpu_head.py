"""GPU parity of the reference's packed BF16 lm_head: `unpack_head`
(src/kernels.rs:2376-2388) and `head_packed` (src/kernels.rs:2258-2373).

The packed logits keep the reference's FP32 order (32 lane sums, halving
tree), so they are compared bit for bit with the oracle's `head`
(src/kernels.rs:2233-2257) -- the same equality src/conformance.rs:611-641
asserts between the reference's two kernels -- and within the reference's
tolerance with the torch fixture.  Greedy selection over the packed logits
must give the oracle's token.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import reference_tolerance_ok
from inferrous_amd import CudaContext, DeviceBuffer, PackedBf16, load

pytestmark = pytest.mark.gpu

F32 = np.float32


@pytest.fixture(scope="module")
def env():
    ctx = CudaContext(0)
    stream = ctx.new_stream()
    return ctx, load(ctx), stream


def dev(stream, a):
    return DeviceBuffer.from_host(stream, np.ascontiguousarray(a))


def to_bits(a):
    return (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def packed_logits(env, x, w_bits):
    _, mod, s = env
    rows = w_bits.size // 4096
    p = PackedBf16.new(w_bits)
    out = DeviceBuffer.zeroed(s, rows, np.float32)
    mod.head_packed(s, None, dev(s, x.reshape(-1)), dev(s, p.words), dev(s, p.offsets), dev(s, p.exceptions),
                    out, 6144)
    s.synchronize()
    return out.to_host_vec(s), p


def test_unpack_round_trips_reference_exhaustive_input(env):
    """src/conformance.rs:715-738."""
    _, mod, s = env
    v = ((np.arange(131072, dtype=np.uint32) * 40503) % 65536).astype(np.uint16)
    p = PackedBf16.new(v)
    out = DeviceBuffer.zeroed(s, v.size, np.uint16)
    mod.unpack_head(s, None, dev(s, p.words), dev(s, p.offsets), dev(s, p.exceptions), out)
    s.synchronize()
    assert np.array_equal(out.to_host_vec(s), v)


def test_head_fixture(env, fixtures):
    (case,) = fixtures.cases("head")
    x, w, want = (fixtures.tensor(case, k) for k in ("x", "w", "out"))
    got, _ = packed_logits(env, x, w.view(np.uint16))
    assert np.array_equal(got.view(np.uint32), oracle.head_bf16(x, w.view(np.uint16)).view(np.uint32))
    assert reference_tolerance_ok(got, want)


@pytest.mark.parametrize("rows,scale,seed", [(33, 0.02, 1), (4099, 0.02, 2), (517, 1.0, 3)])
def test_head_packed_bit_exact(env, rows, scale, seed):
    """Trained-like weights (|w| ~ 0.02: few escapes) and N(0, 1) weights
    (most values escape), an activation of several rows (the last is used)."""
    rng = np.random.default_rng(seed)
    x = oracle.bf16_rne(rng.standard_normal((2, 4096)).astype(F32))
    w = to_bits(rng.standard_normal((rows, 4096)).astype(F32) * F32(scale))
    w[0, :256] = 0            # an all-escape chunk
    w[-1, 7] = 0x7F80         # +inf weight: an escaped special value
    got, p = packed_logits(env, x, w)
    want = oracle.head_bf16(x, w)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()
    if scale < 0.1:
        assert p.exceptions.size < w.size // 50


def test_select_over_packed_logits(env):
    _, mod, s = env
    rng = np.random.default_rng(5)
    rows = 8192
    x = oracle.bf16_rne(rng.standard_normal(4096).astype(F32))
    w = to_bits(rng.standard_normal((rows, 4096)).astype(F32) * F32(0.02))
    logits, _ = packed_logits(env, x, w)
    token = DeviceBuffer.zeroed(s, 1, np.uint32)
    mod.select_token(s, None, dev(s, logits), token)
    s.synchronize()
    assert int(token.to_host_vec(s)[0]) == oracle.argmax(oracle.head_bf16(x, w))


def test_head_packed_many_rows_mixed_escapes(env):
    """Enough rows that every workgroup of the persistent grid runs several
    steps with both register sets, a row count that is not a multiple of 8,
    and rows of every escape regime side by side (none, up to 32 -- held one
    per lane --, exactly 32, 33, and most values)."""
    rng = np.random.default_rng(9)
    rows = 20011
    x = oracle.bf16_rne(rng.standard_normal(4096).astype(F32))
    w = to_bits(rng.standard_normal((rows, 4096)).astype(F32) * F32(0.02))
    r = np.arange(rows)
    w[r % 7 == 3] = to_bits(rng.standard_normal((int(np.sum(r % 7 == 3)), 4096)).astype(F32))
    for sel, k in ((r % 11 == 5, 32), (r % 13 == 6, 33), (r % 17 == 8, 1)):
        for i in np.nonzero(sel)[0]:
            w[i] = to_bits(rng.uniform(0.01, 0.1, 4096).astype(F32))  # no natural escapes
            w[i, rng.choice(4096, k, replace=False)] = 0
    w[-1, 4095] = 0
    got, p = packed_logits(env, x, w)
    per_row = np.diff(np.append(p.offsets.reshape(rows, 16)[:, 0], p.exceptions.size))
    assert {0, 1, 32, 33}.issubset(set(per_row.tolist())) and per_row.max() > 1000
    want = oracle.head_bf16(x, w)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    again, _ = packed_logits(env, x, w)
    assert np.array_equal(again.view(np.uint32), got.view(np.uint32))
