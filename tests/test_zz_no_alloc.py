"""w8a8_linear_argmax_noalloc against w8a8_linear_argmax, through the C ABI.

The allocation-free entry point keeps its selection keys in a fixed device
array inside the library.  Two calls in a row -- the second over fewer
vocabulary rows, so the array still holds the first call's larger key set --
must each give exactly the token and logits of the workspace entry point
(and of the CPU oracle).  A graph captured around it replays with the same
results, and nothing is allocated while capturing.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from inferrous_amd import CudaContext, DeviceBuffer, Graph, W8A8Error, load
from inferrous_amd import _lib

pytestmark = pytest.mark.gpu
F32 = np.float32


@pytest.fixture(scope="module")
def env():
    ctx = CudaContext(0)
    return ctx, load(ctx), ctx.new_stream()


def dev(s, a):
    return DeviceBuffer.from_host(s, np.ascontiguousarray(a))


def case(seed, n, k):
    rng = np.random.default_rng(seed)
    q = rng.integers(-127, 128, size=(1, k), dtype=np.int8)
    w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    asc = np.array([0.0123], F32)
    ws = (rng.random(n) / 128 + 1e-3).astype(F32)
    return q, asc, w, ws


def run_both(mod, s, q, asc, w, ws, k):
    n = len(ws)
    dq, da, dw, dws = dev(s, q), dev(s, asc), dev(s, w), dev(s, ws)
    t_ref, t_na = DeviceBuffer.zeroed(s, 1, np.uint32), DeviceBuffer.zeroed(s, 1, np.uint32)
    l_ref, l_na = DeviceBuffer.zeroed(s, n, np.uint16), DeviceBuffer.zeroed(s, n, np.uint16)
    mod.linear_argmax(s, dq, da, dw, dws, k, t_ref, l_ref)
    mod.linear_argmax_noalloc(s, dq, da, dw, dws, k, t_na, l_na)
    s.synchronize()
    return (int(t_ref.to_host_vec(s)[0]), l_ref.to_host_vec(s), int(t_na.to_host_vec(s)[0]),
            l_na.to_host_vec(s))


def test_noalloc_matches_workspace_entry_two_calls_shrinking(env):
    ctx, mod, s = env
    k = 4096
    for seed, n in ((1, 151936), (2, 40001)):       # second call: fewer rows, stale keys beyond
        q, asc, w, ws = case(seed, n, k)
        t_ref, l_ref, t_na, l_na = run_both(mod, s, q, asc, w, ws, k)
        want, logits = oracle.linear_argmax(q, asc, w, ws, k)
        print(f"noalloc n={n} token {t_na} (workspace {t_ref}, oracle {want})", flush=True)
        assert t_na == t_ref == want, n
        assert np.array_equal(l_na, l_ref), n
        assert np.array_equal(l_na, (logits.view(np.uint32) >> 16).astype(np.uint16)), n


def test_noalloc_without_logits_ties_and_sentinel(env):
    """Token only; a planted tie on the largest value resolves to the lowest
    index; a non-finite scale gives the sentinel; then a clean call again."""
    ctx, mod, s = env
    k = 1024
    q, asc, w, ws = case(3, 9000, k)
    w[123] = np.where(q[0] >= 0, 127, -127)          # the largest accumulator possible
    w[7000] = w[123]
    ws[7000] = ws[123] = F32(0.5)                    # rows 123 and 7000 tie and dominate
    want, _ = oracle.linear_argmax(q, asc, w, ws, k)
    assert want == 123
    t = DeviceBuffer.zeroed(s, 1, np.uint32)
    mod.linear_argmax_noalloc(s, dev(s, q), dev(s, asc), dev(s, w), dev(s, ws), k, t)
    s.synchronize()
    assert int(t.to_host_vec(s)[0]) == 123
    ws_bad = ws.copy()
    ws_bad[4500] = np.inf
    mod.linear_argmax_noalloc(s, dev(s, q), dev(s, asc), dev(s, w), dev(s, ws_bad), k, t)
    s.synchronize()
    assert int(t.to_host_vec(s)[0]) == 0xFFFFFFFF
    mod.linear_argmax_noalloc(s, dev(s, q), dev(s, asc), dev(s, w), dev(s, ws), k, t)
    s.synchronize()
    assert int(t.to_host_vec(s)[0]) == 123


def test_noalloc_graph_replay_and_limit(env):
    ctx, mod, s = env
    k = 4096
    q, asc, w, ws = case(4, 70000, k)
    want, _ = oracle.linear_argmax(q, asc, w, ws, k)
    dq, da, dw, dws = dev(s, q), dev(s, asc), dev(s, w), dev(s, ws)
    t = DeviceBuffer.zeroed(s, 1, np.uint32)
    g = Graph(s)
    with g:
        mod.linear_argmax_noalloc(s, dq, da, dw, dws, k, t)
    q2, asc2, w2, ws2 = case(5, 3000, k)
    want2, _ = oracle.linear_argmax(q2, asc2, w2, ws2, k)
    t2 = DeviceBuffer.zeroed(s, 1, np.uint32)
    for rep in range(3):
        t.fill_zero(s)
        g.launch()
        s.synchronize()
        assert int(t.to_host_vec(s)[0]) == want, rep
        # eager call on the same array between replays
        mod.linear_argmax_noalloc(s, dev(s, q2), dev(s, asc2), dev(s, w2), dev(s, ws2), k, t2)
        s.synchronize()
        assert int(t2.to_host_vec(s)[0]) == want2, rep
    too_many = _lib.NOALLOC_MAX_ROWS + 1
    status = _lib.lib().w8a8_linear_argmax_noalloc(s.handle, dq.ptr, da.ptr, dw.ptr, dws.ptr, too_many, k,
                                                   t.ptr, None, 0)
    assert status == _lib.ESHAPE
    with pytest.raises((W8A8Error, ValueError)):
        mod.linear_argmax_noalloc(s, dq, da, dw, DeviceBuffer.view_of(dws, 0, 1), k, t,
                                  DeviceBuffer.zeroed(s, 2, np.uint16))
