"""GPU parity of `norm_quantize` (src/kernels.rs:476-575): RMSNorm of each
4096-wide row, then its quantization, with the maxima reset.

The kernel and the oracle evaluate 1/sqrt in binary64, so `out`, `q`,
`scales` and `maxima` are compared bit for bit with the oracle.  Against the
reference's torch fixture (tools/operator_fixtures.py:36-40, whose rsqrt and
sum order are torch's) `out` is compared within the reference's tolerance
(src/conformance.rs:660-673).  As in src/conformance.rs:166-199, the fused
operator must equal `quantize` applied to its own output.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import reference_tolerance_ok
from inferrous_amd import CudaContext, DeviceBuffer, Graph, load, rows

pytestmark = pytest.mark.gpu

F32 = np.float32
FLOOR = int(np.array([1e-8], F32).view(np.uint32)[0])


@pytest.fixture(scope="module")
def env():
    ctx = CudaContext(0)
    stream = ctx.new_stream()
    return ctx, load(ctx), stream


def dev(stream, a):
    return DeviceBuffer.from_host(stream, np.ascontiguousarray(a))


def run(env, x, gain):
    _, mod, s = env
    m = x.shape[0]
    out = DeviceBuffer.zeroed(s, m * 4096, np.float32)
    q = DeviceBuffer.zeroed(s, m * 4096, np.int8)
    sc = DeviceBuffer.zeroed(s, m, np.float32)
    mx = dev(s, np.full(m, 0x12345678, np.uint32))
    mod.norm_quantize(s, rows(m, 1024), dev(s, x), dev(s, gain), out, q, sc, mx)
    s.synchronize()
    return (out.to_host_vec(s).reshape(m, 4096), q.to_host_vec(s).reshape(m, 4096), sc.to_host_vec(s),
            mx.to_host_vec(s))


def special_rows(rng):
    x = rng.standard_normal((6, 4096)).astype(F32)
    x[0] = 0                       # zero row: scale floor, q = 0
    x[1] = 1                       # mean 1: out rounds to 1.0, q = 127
    x[2, 11] = np.nan              # NaN: every output NaN, q = 0
    x[3] *= F32(1e-3)              # mean(x^2) ~ 1e-6: the epsilon matters
    x[4] *= F32(1e20)              # squares overflow: sum inf, inv 0
    x[5] = np.where(np.arange(4096) % 2, F32(2.5), F32(-2.5))
    return x


@pytest.mark.parametrize("m,seed", [(1, 1), (3, 2), (129, 3)])
def test_norm_quantize_bit_exact_vs_oracle(env, m, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((m, 4096)) * np.exp(rng.uniform(-3, 3, (m, 1)))).astype(F32)
    gain = (1 + 0.3 * rng.standard_normal(4096)).astype(F32)
    got = run(env, x, gain)
    want = oracle.norm_quantize(x, gain)
    assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32)), "out"
    assert np.array_equal(got[1], want[1]), "q"
    assert np.array_equal(got[2].view(np.uint32), want[2].view(np.uint32)), "scales"
    assert np.all(got[3] == FLOOR), "maxima reset"


def test_norm_quantize_special_rows(env):
    x = special_rows(np.random.default_rng(4))
    gain = np.random.default_rng(5).standard_normal(4096).astype(F32)
    out, q, sc, mx = run(env, x, gain)
    wout, wq, wsc, _ = oracle.norm_quantize(x, gain)
    same = (out.view(np.uint32) == wout.view(np.uint32)) | (np.isnan(out) & np.isnan(wout))
    assert same.all()
    assert np.array_equal(q, wq) and np.array_equal(sc.view(np.uint32), wsc.view(np.uint32))
    assert np.all(out[0] == 0) and np.all(q[0] == 0) and sc[0] == F32(1e-8) / F32(127)
    assert np.isnan(out[2]).all() and np.all(q[2] == 0)
    assert np.all(out[4] == 0) and np.all(q[4] == 0)
    assert np.all(mx == FLOOR)


def test_norm_matches_reference_fixture_within_tolerance(env, fixtures):
    (case,) = fixtures.cases("norm")
    x, gain, want = (fixtures.tensor(case, k) for k in ("x", "gain", "out"))
    out, _, _, _ = run(env, x, gain)
    assert reference_tolerance_ok(out, want)
    assert np.all(out[0] == 0)


def test_fused_equals_quantize_of_its_output(env):
    """src/conformance.rs:166-199 (the fused operator against norm, then quantize)."""
    _, mod, s = env
    rng = np.random.default_rng(6)
    x = rng.standard_normal((17, 4096)).astype(F32)
    gain = rng.standard_normal(4096).astype(F32)
    out, q, sc, _ = run(env, x, gain)
    q2 = DeviceBuffer.zeroed(s, 17 * 4096, np.int8)
    sc2 = DeviceBuffer.zeroed(s, 17, np.float32)
    mod.quantize(s, None, dev(s, out.reshape(-1)), 4096, q2, sc2)
    s.synchronize()
    assert np.array_equal(q.reshape(-1), q2.to_host_vec(s))
    assert np.array_equal(sc.view(np.uint32), sc2.to_host_vec(s).view(np.uint32))


def test_norm_quantize_graph_replay(env):
    """Capturable (no allocation, no host sync): replays reproduce the eager result."""
    _, mod, s = env
    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, 4096)).astype(F32)
    gain = rng.standard_normal(4096).astype(F32)
    xb, gb = dev(s, x), dev(s, gain)
    out = DeviceBuffer.zeroed(s, 2 * 4096, np.float32)
    q = DeviceBuffer.zeroed(s, 2 * 4096, np.int8)
    sc = DeviceBuffer.zeroed(s, 2, np.float32)
    mx = DeviceBuffer.zeroed(s, 2, np.uint32)
    want = oracle.norm_quantize(x, gain)
    g = Graph(s)
    with g:
        mod.norm_quantize(s, None, xb, gb, out, q, sc, mx)
    for _ in range(3):
        out.fill_zero(s)
        q.fill_zero(s)
        s.synchronize()
        g.launch()
        s.synchronize()
        assert np.array_equal(out.to_host_vec(s).view(np.uint32), want[0].reshape(-1).view(np.uint32))
        assert np.array_equal(q.to_host_vec(s), want[1].reshape(-1))
