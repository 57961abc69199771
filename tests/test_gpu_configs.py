"""Parity at the benchmark configurations' real shapes (configs 1-5 of the
W8A8 baseline), on the same seeded synthetic tensors the bench uses.

Weights are generated on the device; the checker regenerates the same rows
on the host (oracle.synth_*) and compares every output: the 36-layer decode
set, the lm_head, every row of the four prefill shapes at M = 129 and 512
(the threaded C oracle runs those 198 G int8 ops in about a second), and
the ragged small-M batches.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from inferrous_amd import CudaContext, DeviceBuffer, load
from inferrous_amd import synth

pytestmark = pytest.mark.gpu
F32 = np.float32
SEED_W, SEED_S = 1, 2


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def env():
    ctx = CudaContext(0)
    return ctx, load(ctx), ctx.new_stream()


def dev(s, a):
    return DeviceBuffer.from_host(s, np.ascontiguousarray(a))


def make_weights(mod, s, n, k, wstream, sstream):
    w = DeviceBuffer.zeroed(s, n * k, np.int8)
    ws = DeviceBuffer.zeroed(s, n, np.float32)
    mod.synth_i8(s, w, SEED_W, wstream)
    mod.synth_f32(s, ws, SEED_S, sstream, 1e-3, 1e-2)
    return w, ws


def host_weights(n, k, wstream, sstream, rows_idx=None):
    if rows_idx is None:
        return (oracle.synth_i8(SEED_W, wstream, 0, n * k).reshape(n, k),
                oracle.synth_f32(SEED_S, sstream, 0, n, 1e-3, 1e-2))
    w = np.stack([oracle.synth_i8(SEED_W, wstream, int(r) * k, k) for r in rows_idx])
    ws = oracle.synth_f32(SEED_S, sstream, 0, n, 1e-3, 1e-2)[rows_idx]
    return w, ws


def quantize_dev(mod, s, x, k):
    m = x.shape[0]
    q = DeviceBuffer.zeroed(s, m * k, np.int8)
    sc = DeviceBuffer.zeroed(s, m, np.float32)
    mod.quantize(s, None, dev(s, x.reshape(-1)), k, q, sc)
    wq, wsc = oracle.quantize(x.reshape(-1), k)
    assert np.array_equal(q.to_host_vec(s), wq)
    assert np.array_equal(bits(sc.to_host_vec(s)), bits(wsc))
    return q, sc, wq.reshape(m, k), wsc


def test_config1_single_linear_full(env):
    """M=1, K=N=4096: i32 accumulators and BF16 output, every element."""
    ctx, mod, s = env
    k = n = 4096
    w, ws = make_weights(mod, s, n, k, 1, 101)
    x = synth.normal_rows(3, 1, k)
    q, sc, hq, hsc = quantize_dev(mod, s, x, k)
    hw, hws = host_weights(n, k, 1, 101)
    acc, out, outb = oracle.linear(hq, hsc, hw, hws, k)
    for op in ("linear", "linear_dot4", "linear_mfma"):
        o32 = DeviceBuffer.zeroed(s, n, np.int32)
        getattr(mod, op)(s, None, q, sc, w, ws, k, o32)
        assert np.array_equal(o32.to_host_vec(s), acc), op
        ob = DeviceBuffer.zeroed(s, n, np.uint16)
        getattr(mod, op)(s, None, q, sc, w, ws, k, ob)
        assert np.array_equal(ob.to_host_vec(s), outb), op


def test_config2_decode_layer_set(env):
    """36 layers x {qkv, o, gate_up, down} at M=1, every output of every
    layer: the i32 accumulators and the BF16 outputs equal the oracle's on
    the host-regenerated weights (7 GB of int8 regenerated layer by layer)."""
    ctx, mod, s = env
    xs = {4096: synth.normal_rows(40, 1, 4096), 12288: synth.normal_rows(41, 1, 12288)}
    qs = {k: quantize_dev(mod, s, x, k) for k, x in xs.items()}
    for layer in range(36):
        for si, (name, n, k) in enumerate(synth.DECODE_SHAPES):
            ws_id, ss_id = synth.weight_stream(layer, si), synth.scale_stream(layer, si)
            w, ws = make_weights(mod, s, n, k, ws_id, ss_id)
            q, sc, hq, hsc = qs[k]
            o32 = DeviceBuffer.zeroed(s, n, np.int32)
            mod.linear(s, None, q, sc, w, ws, k, o32)
            ob = DeviceBuffer.zeroed(s, n, np.uint16)
            mod.linear(s, None, q, sc, w, ws, k, ob)
            hw, hws = host_weights(n, k, ws_id, ss_id)
            a2, _, b2 = oracle.linear(hq, hsc, hw, hws, k)
            assert np.array_equal(o32.to_host_vec(s), a2), (layer, name)
            assert np.array_equal(ob.to_host_vec(s), b2), (layer, name)
            del w, ws, hw


def test_config3_lm_head_argmax_full(env):
    ctx, mod, s = env
    n, k = synth.VOCAB, synth.HIDDEN
    w, ws = make_weights(mod, s, n, k, 9001, 9101)
    x = synth.normal_rows(4, 1, k)
    q, sc, hq, hsc = quantize_dev(mod, s, x, k)
    hw, hws = host_weights(n, k, 9001, 9101)
    tok, logits = oracle.linear_argmax(hq, hsc, hw, hws, k)
    t = DeviceBuffer.zeroed(s, 1, np.uint32)
    lg = DeviceBuffer.zeroed(s, n, np.float32)
    mod.linear_argmax(s, q, sc, w, ws, k, t, lg)
    assert int(t.to_host_vec(s)[0]) == tok
    assert np.array_equal(bits(lg.to_host_vec(s)), bits(logits))
    t2 = DeviceBuffer.zeroed(s, 1, np.uint32)
    mod.select_token(s, None, lg, t2)
    assert int(t2.to_host_vec(s)[0]) == tok


@pytest.mark.parametrize("m", [129, 512])
def test_config4_prefill_shapes(env, m):
    """Student-t(3) activations with 8 x50 outlier channels, per-token
    quantization, then the MFMA GEMM on all four layer shapes: every row of
    the i32 accumulators and of the BF16 outputs against the oracle."""
    ctx, mod, s = env
    for si, (name, n, k) in enumerate(synth.DECODE_SHAPES):
        x = synth.student_t_rows(700 + si, m, k)
        q, sc, hq, hsc = quantize_dev(mod, s, x, k)
        w, ws = make_weights(mod, s, n, k, 5000 + si, 5100 + si)
        o32 = DeviceBuffer.zeroed(s, m * n, np.int32)
        mod.linear(s, None, q, sc, w, ws, k, o32)
        ob = DeviceBuffer.zeroed(s, m * n, np.uint16)
        mod.linear(s, None, q, sc, w, ws, k, ob)
        acc = o32.to_host_vec(s).reshape(m, n)
        outb = ob.to_host_vec(s).reshape(m, n)
        hw, hws = host_weights(n, k, 5000 + si, 5100 + si)
        a2, _, b2 = oracle.linear(hq, hsc, hw, hws, k)
        bad = np.flatnonzero((acc != a2.reshape(m, n)).any(1))
        assert bad.size == 0, f"{name}: {bad.size} rows of acc differ, first row {bad[:1]}"
        bad = np.flatnonzero((outb != b2.reshape(m, n)).any(1))
        assert bad.size == 0, f"{name}: {bad.size} rows of the BF16 output differ, first row {bad[:1]}"


@pytest.mark.parametrize("m", [4, 16, 64])
def test_config5_ragged_rows_both_families(env, m):
    ctx, mod, s = env
    for si in (2, 3):
        name, n, k = synth.DECODE_SHAPES[si]
        x = synth.ragged_rows(range(9000 + 100 * m, 9000 + 100 * m + m), k)
        q, sc, hq, hsc = quantize_dev(mod, s, x, k)
        w, ws = make_weights(mod, s, n, k, 6000 + si, 6100 + si)
        hw, hws = host_weights(n, k, 6000 + si, 6100 + si)
        acc, _, outb = oracle.linear(hq, hsc, hw, hws, k)
        for op in ("linear_dot4", "linear_mfma", "linear"):
            o32 = DeviceBuffer.zeroed(s, m * n, np.int32)
            getattr(mod, op)(s, None, q, sc, w, ws, k, o32)
            assert np.array_equal(o32.to_host_vec(s), acc), (op, name)
            ob = DeviceBuffer.zeroed(s, m * n, np.uint16)
            getattr(mod, op)(s, None, q, sc, w, ws, k, ob)
            assert np.array_equal(ob.to_host_vec(s), outb), (op, name)
