"""A dependent multi-layer decode chain, fused against the reference's calls.

Four Qwen3-8B-shaped layers with distinct weights, wired the way the decode
step wires them (src/gpu.rs:571-790): the layer's residual stream h feeds the
attention norm; norm_quantize -> qkv; the attention output (out of scope
here: a stand-in row, the first 4096 values of the qkv output, so that o
depends on qkv) -> quantize -> o + residual h = h1; norm_quantize(h1) ->
linear_swiglu -> quantize_with_max -> down + residual h1 = the next layer's
h; after the last layer the lm_head GEMV with greedy selection.

The same chain with every producer folded into its consumer
(w8a8_norm_quantize_linear, w8a8_quantize_linear, w8a8_norm_quantize_mlp:
147 launches per token at 36 layers instead of 327) must produce every
intermediate -- codes, scales, qkv, the residual streams, gate/up/act, the
token -- bit for bit, eagerly and as a replayed graph.  Each single fold is
checked against the oracle in test_gpu_produce.py; this file checks that the
folds compose across layers, where each layer's inputs are the previous
layer's outputs.
"""
from __future__ import annotations

import numpy as np
import pytest

from inferrous_amd import CudaContext, DeviceBuffer, Graph, load, synth

pytestmark = pytest.mark.gpu
LAYERS, H, FFN = 4, 4096, 12288


@pytest.fixture(scope="module")
def env():
    ctx = CudaContext(0)
    mod = load(ctx)
    s = ctx.new_stream()
    layers = []
    for layer in range(LAYERS):
        mats = []
        for si, (name, n, k) in enumerate(synth.DECODE_SHAPES):
            w = DeviceBuffer.zeroed(s, n * k, np.int8)
            ws = DeviceBuffer.zeroed(s, n, np.float32)
            mod.synth_i8(s, w, 11, 1000 + 10 * layer + si)
            mod.synth_f32(s, ws, 12, 2000 + 10 * layer + si, 1e-3, 1e-2)
            mats.append((w, ws))
        (gw, gws) = mats[2]
        halves = (DeviceBuffer.view_of(gw, 0, FFN * H), DeviceBuffer.view_of(gws, 0, FFN),
                  DeviceBuffer.view_of(gw, FFN * H, FFN * H), DeviceBuffer.view_of(gws, FFN, FFN))
        gains = [DeviceBuffer.from_host(s, (1 + 0.2 * synth.normal_rows(3000 + 2 * layer + i, 1, H))
                                        .astype(np.float32).reshape(-1)) for i in range(2)]
        layers.append((mats, halves, gains))
    head_w = DeviceBuffer.zeroed(s, 50000 * H, np.int8)
    head_s = DeviceBuffer.zeroed(s, 50000, np.float32)
    mod.synth_i8(s, head_w, 11, 4000)
    mod.synth_f32(s, head_s, 12, 4001, 1e-3, 1e-2)
    return ctx, mod, s, layers, (head_w, head_s)


class State:
    """Every intermediate of the chain: one buffer per layer for the values
    that flow between launches, so that all of them can be compared."""

    def __init__(self, s):
        z = DeviceBuffer.zeroed
        self.h = [DeviceBuffer.from_host(s, (2.0 * synth.normal_rows(77, 1, H)).reshape(-1))] + \
                 [z(s, H, np.float32) for _ in range(LAYERS)]          # residual stream per layer boundary
        self.h1 = [z(s, H, np.float32) for _ in range(LAYERS)]          # after o + residual
        self.qkv = [z(s, 6144, np.float32) for _ in range(LAYERS)]
        self.o = [z(s, H, np.float32) for _ in range(LAYERS)]
        self.down = [z(s, H, np.float32) for _ in range(LAYERS)]
        self.gate = [z(s, FFN, np.float32) for _ in range(LAYERS)]
        self.up = [z(s, FFN, np.float32) for _ in range(LAYERS)]
        self.act = [z(s, FFN, np.float32) for _ in range(LAYERS)]
        self.q4 = [z(s, H, np.int8) for _ in range(3 * LAYERS + 1)]     # qkv, o, swiglu codes per layer; head
        self.s4 = [z(s, 1, np.float32) for _ in range(3 * LAYERS + 1)]
        self.q12 = [z(s, FFN, np.int8) for _ in range(LAYERS)]
        self.s12 = [z(s, 1, np.float32) for _ in range(LAYERS)]
        self.normed = z(s, H, np.float32)
        self.mx = z(s, 1, np.uint32)
        self.token = z(s, 1, np.uint32)
        self.logits = z(s, 50000, np.float32)

    def buffers(self):
        return (self.h + self.h1 + self.qkv + self.o + self.down + self.gate + self.up + self.act + self.q4
                + self.s4 + self.q12 + self.s12 + [self.token, self.logits])

    def clear(self, s):
        for b in self.buffers()[1:]:
            b.fill_zero(s)


def attention_stand_in(st, layer):
    """The attention output row of the layer (out of scope): the first 4096
    values of the qkv output, so that o depends on qkv."""
    return DeviceBuffer.view_of(st.qkv[layer], 0, H)


def chain_calls(mod, s, layers, head, st):
    """The reference's order: 9 launches per layer (src/gpu.rs:571-790)."""
    for ly, (mats, (wg_, sg_, wu_, su_), gains) in enumerate(layers):
        (wqkv, sqkv), (wo, so), _, (wd, sd) = mats
        h, q = st.h[ly], st.q4
        mod.norm_quantize(s, None, h, gains[0], st.normed, q[3 * ly], st.s4[3 * ly], st.mx)
        mod.linear(s, None, q[3 * ly], st.s4[3 * ly], wqkv, sqkv, H, st.qkv[ly])
        mod.quantize(s, None, attention_stand_in(st, ly), H, q[3 * ly + 1], st.s4[3 * ly + 1])
        mod.linear_residual(s, None, q[3 * ly + 1], st.s4[3 * ly + 1], wo, so, H, h, st.o[ly], st.h1[ly])
        mod.norm_quantize(s, None, st.h1[ly], gains[1], st.normed, q[3 * ly + 2], st.s4[3 * ly + 2], st.mx)
        mod.linear_swiglu(s, None, q[3 * ly + 2], st.s4[3 * ly + 2], H, wg_, sg_, st.gate[ly], wu_, su_,
                          st.up[ly], st.act[ly], st.mx)
        mod.linear_quantize_with_max(s, None, st.act[ly], FFN, st.mx, st.q12[ly], st.s12[ly], wd, sd,
                                     st.down[ly], st.h1[ly], st.h[ly + 1])
    mod.quantize(s, None, st.h[LAYERS], H, st.q4[-1], st.s4[-1])
    mod.linear_argmax(s, st.q4[-1], st.s4[-1], head[0], head[1], H, st.token, st.logits)


def chain_fused(mod, s, layers, head, st):
    """Every producer folded into its consumer: 4 launches per layer."""
    for ly, (mats, (wg_, sg_, wu_, su_), gains) in enumerate(layers):
        (wqkv, sqkv), (wo, so), _, (wd, sd) = mats
        h, q = st.h[ly], st.q4
        mod.norm_quantize_linear(s, None, h, gains[0], st.normed, q[3 * ly], st.s4[3 * ly], st.mx, wqkv, sqkv,
                                 st.qkv[ly])
        mod.quantize_linear(s, None, attention_stand_in(st, ly), q[3 * ly + 1], st.s4[3 * ly + 1], wo, so,
                            st.o[ly], h, st.h1[ly])
        mod.norm_quantize_mlp(s, None, st.h1[ly], gains[1], st.normed, q[3 * ly + 2], st.s4[3 * ly + 2], wg_, sg_,
                              st.gate[ly], wu_, su_, st.up[ly], st.act[ly], st.mx, wd, sd, st.down[ly], st.h1[ly],
                              st.h[ly + 1], st.q12[ly], st.s12[ly])
    mod.quantize(s, None, st.h[LAYERS], H, st.q4[-1], st.s4[-1])
    mod.linear_argmax(s, st.q4[-1], st.s4[-1], head[0], head[1], H, st.token, st.logits)


def snapshot(s, st):
    return [b.to_host_vec(s).copy() for b in st.buffers()]


def compare(got, want, what):
    for i, (g, w) in enumerate(zip(got, want)):
        gb, wb = g.view(np.uint8), w.view(np.uint8)
        bad = np.flatnonzero(gb != wb)
        assert bad.size == 0, f"{what}: buffer {i} differs at byte {bad[0]} ({bad.size} bytes)"


def test_fused_chain_matches_reference_calls(env):
    ctx, mod, s, layers, head = env
    ref, fused = State(s), State(s)
    chain_calls(mod, s, layers, head, ref)
    chain_fused(mod, s, layers, head, fused)
    s.synchronize()
    want = snapshot(s, ref)
    compare(snapshot(s, fused), want, "fused chain")
    # the chain really flows: every layer's residual stream differs from its input
    for ly in range(LAYERS):
        assert not np.array_equal(want[ly], want[ly + 1]), f"layer {ly} left the residual stream unchanged"
    assert int(want[-2][0]) < 50000


def test_fused_chain_graph_replays(env):
    """The fused chain captured once, replayed three times with its
    intermediates cleared and eager work in between: every replay equals the
    eager reference chain."""
    ctx, mod, s, layers, head = env
    ref = State(s)
    chain_calls(mod, s, layers, head, ref)
    s.synchronize()
    want = snapshot(s, ref)
    st = State(s)
    chain_fused(mod, s, layers, head, st)  # eager first: workspaces exist before capture
    s.synchronize()
    g = Graph(s)
    with g:
        chain_fused(mod, s, layers, head, st)
    for rep in range(3):
        st.clear(s)
        mod.quantize(s, None, st.h[0], H, st.q4[0], st.s4[0])  # eager work between replays
        s.synchronize()
        g.launch()
        s.synchronize()
        compare(snapshot(s, st), want, f"replay {rep}")
