"""GPU parity of the one-launch decode sequence (w8a8_linear_sequence).

The sequence runs M = 1 projections as one launch, with a device-wide
barrier between consecutive entries (the reference's decode graph with
programmatic edges, crates/inferrous-qwen3/src/graph.rs:56-110).  Every
output must equal the per-entry call -- linear (src/kernels.rs:807-845),
linear_residual (:577-618), linear_argmax (the head GEMV + select_token,
:2191-2231) -- bit for bit; those calls are themselves checked against the
CPU oracle in test_gpu_parity.py, and two entries here are checked against
the oracle directly.  Shapes cover fewer rows than waves, a row count one
past a whole round of waves, K of 4096 / 8192 / 12288, both output dtypes,
residual entries and a selecting last entry, and the Qwen3-8B decode shapes.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from inferrous_amd import CudaContext, DeviceBuffer, Graph, W8A8Error, load, synth

pytestmark = pytest.mark.gpu

F32 = np.float32


@pytest.fixture(scope="module")
def env():
    ctx = CudaContext(0)
    stream = ctx.new_stream()
    mod = load(ctx)
    mod.sequence_reset()
    return ctx, mod, stream


def dev(stream, a):
    return DeviceBuffer.from_host(stream, np.ascontiguousarray(a))


def waves(ctx):
    """Compute waves of a sequence launch: 15 per CU."""
    return 15 * ctx.info()[0]


class Proj:
    """One projection's operands on the device (seeded weights, one quantized
    activation row) and its output buffers."""

    def __init__(self, s, mod, n, k, seed, dtype=np.uint16, residual=False, select=False):
        self.n, self.k, self.seed, self.dtype = n, k, seed, dtype
        self.w = DeviceBuffer.zeroed(s, n * k, np.int8)
        self.ws = DeviceBuffer.zeroed(s, n, np.float32)
        mod.synth_i8(s, self.w, 31, seed)
        mod.synth_f32(s, self.ws, 32, seed, 1e-3, 1e-2)
        self.x = synth.normal_rows(seed, 1, k).reshape(-1)
        self.q = DeviceBuffer.zeroed(s, k, np.int8)
        self.asc = DeviceBuffer.zeroed(s, 1, np.float32)
        mod.quantize(s, None, dev(s, self.x), k, self.q, self.asc)
        self.select = select
        self.out = DeviceBuffer.zeroed(s, n, dtype)
        self.res = dev(s, synth.normal_rows(seed + 7, 1, n).reshape(-1)) if residual else None
        self.comb = DeviceBuffer.zeroed(s, n, dtype) if residual else None

    def entry(self):
        e = dict(q=self.q, asc=self.asc, w=self.w, ws=self.ws, out=self.out, select=self.select)
        if self.res is not None:
            e.update(residual=self.res, combined=self.comb)
        return e

    def clear(self, s):
        for b in (self.out, self.comb):
            if b is not None:
                b.fill_zero(s)

    def outputs(self, s):
        return [b.to_host_vec(s).copy() for b in (self.out, self.comb) if b is not None]

    def per_call(self, s, mod, token=None):
        """The same projection through the per-entry ops."""
        out = DeviceBuffer.zeroed(s, self.n, self.dtype)
        if self.select:
            mod.linear_argmax(s, self.q, self.asc, self.w, self.ws, self.k, token, out)
            return [out.to_host_vec(s).copy()]
        if self.res is not None:
            comb = DeviceBuffer.zeroed(s, self.n, self.dtype)
            mod.linear_residual(s, None, self.q, self.asc, self.w, self.ws, self.k, self.res, out, comb)
            return [out.to_host_vec(s).copy(), comb.to_host_vec(s).copy()]
        mod.linear(s, None, self.q, self.asc, self.w, self.ws, self.k, out)
        return [out.to_host_vec(s).copy()]


def check_against_per_call(s, mod, projs, got_token=None):
    want_token = DeviceBuffer.zeroed(s, 1, np.uint32)
    for i, p in enumerate(projs):
        got = p.outputs(s)
        want = p.per_call(s, mod, want_token if p.select else None)
        for g, w in zip(got, want):
            if g.dtype == np.float32:
                g, w = g.view(np.uint32), w.view(np.uint32)
            bad = np.flatnonzero(g != w)
            assert bad.size == 0, f"entry {i} (n={p.n}, k={p.k}): {bad.size} outputs differ, first row {bad[0]}"
    if got_token is not None:
        assert int(got_token) == int(want_token.to_host_vec(s)[0])


def test_sequence_mixed_entries_match_per_call(env):
    ctx, mod, s = env
    nw = waves(ctx)
    print(f"sequence mixed entries, {nw} compute waves", flush=True)
    projs = [
        Proj(s, mod, 33, 4096, 101, np.float32),                  # fewer rows than waves
        Proj(s, mod, 6144, 4096, 102),                            # qkv
        Proj(s, mod, 4096, 12288, 103, residual=True),            # down + residual
        Proj(s, mod, 5000, 8192, 104, np.float32, residual=True),
        Proj(s, mod, 1, 4096, 105),
        Proj(s, mod, nw + 1, 4096, 106),                          # one wave takes a second row
        Proj(s, mod, 24576, 4096, 107, np.float32),               # gate_up
        Proj(s, mod, 50000, 4096, 108, np.uint16, select=True),   # selecting head with logits
    ]
    plan = mod.prepare_sequence([p.entry() for p in projs])
    token = DeviceBuffer.zeroed(s, 1, np.uint32)
    tokens = []
    for rep in range(3):  # repeated calls: the barrier epochs carry over
        for p in projs:
            p.clear(s)
        token.fill_zero(s)
        mod.linear_sequence(s, plan, token)
        s.synchronize()
        assert mod.sequence_status() == 0
        tokens.append(int(token.to_host_vec(s)[0]))
        if rep == 0:
            check_against_per_call(s, mod, projs, tokens[0])
            first = [p.outputs(s) for p in projs]
        else:
            for i, p in enumerate(projs):
                for g, w in zip(p.outputs(s), first[i]):
                    assert np.array_equal(g.view(np.uint8), w.view(np.uint8)), \
                        f"call {rep}, entry {i} differs from the first call"
    assert len(set(tokens)) == 1
    # Two entries against the oracle directly.
    for p in (projs[0], projs[2]):
        wq, wsc = oracle.quantize(p.x, p.k)
        w = oracle.synth_i8(31, p.seed, 0, p.n * p.k)
        ws = oracle.synth_f32(32, p.seed, 0, p.n, 1e-3, 1e-2)
        _, out_f32, out_bf16 = oracle.linear(wq, wsc, w, ws, p.k)
        got = p.outputs(s)[0]
        if p.dtype == np.float32:
            assert np.array_equal(got.view(np.uint32), np.asarray(out_f32, F32).view(np.uint32))
        else:
            assert np.array_equal(got, out_bf16)


def test_sequence_without_selection(env):
    ctx, mod, s = env
    projs = [Proj(s, mod, 4096, 4096, 201), Proj(s, mod, 2048, 12288, 202, np.float32, residual=True)]
    plan = mod.prepare_sequence([p.entry() for p in projs])
    mod.linear_sequence(s, plan)
    s.synchronize()
    assert mod.sequence_status() == 0
    check_against_per_call(s, mod, projs)


def test_sequence_decode_shapes(env):
    """Two Qwen3-8B decoder layers' projections (qkv 6144x4096, o 4096x4096
    with residual, gate_up 24576x4096, down 4096x12288 with residual) and the
    151,936-row W8A8 lm_head with selection, as one launch."""
    ctx, mod, s = env
    projs = []
    for layer in range(2):
        base = 300 + 10 * layer
        projs += [Proj(s, mod, 6144, 4096, base + 1), Proj(s, mod, 4096, 4096, base + 2, residual=True),
                  Proj(s, mod, 24576, 4096, base + 3), Proj(s, mod, 4096, 12288, base + 4, residual=True)]
    projs.append(Proj(s, mod, 151936, 4096, 399, np.float32, select=True))
    plan = mod.prepare_sequence([p.entry() for p in projs])
    token = DeviceBuffer.zeroed(s, 1, np.uint32)
    mod.linear_sequence(s, plan, token)
    s.synchronize()
    assert mod.sequence_status() == 0
    check_against_per_call(s, mod, projs, token.to_host_vec(s)[0])


def test_sequence_wait_limit_abort_and_reset(env):
    """A wait limit of 1 us cannot be met at the first entry boundary of
    large entries: the launch marks the state aborted and ends (every wave
    leaves its waits); later launches do nothing until the reset, after
    which the sequence runs correctly again."""
    ctx, mod, s = env
    projs = [Proj(s, mod, 24576, 4096, 400 + i) for i in range(4)]
    plan = mod.prepare_sequence([p.entry() for p in projs])
    mod.linear_sequence(s, plan, wait_us=1)
    s.synchronize()
    status = mod.sequence_status()
    print(f"status after a 1 us wait limit: {status}", flush=True)
    assert status in (0, 1)
    if status == 1:
        for p in projs:
            p.clear(s)
        mod.linear_sequence(s, plan)  # returns at once: the state is aborted
        s.synchronize()
        assert mod.sequence_status() == 1
        assert all(not np.any(o) for p in projs for o in p.outputs(s))
    mod.sequence_reset()
    assert mod.sequence_status() == 0
    for p in projs:
        p.clear(s)
    mod.linear_sequence(s, plan)
    s.synchronize()
    assert mod.sequence_status() == 0
    check_against_per_call(s, mod, projs)


def test_sequence_refuses_misuse(env):
    ctx, mod, s = env
    projs = [Proj(s, mod, 512, 4096, 501), Proj(s, mod, 512, 4096, 502, select=True)]
    plan = mod.prepare_sequence([p.entry() for p in projs])
    with pytest.raises(ValueError, match="token"):
        mod.linear_sequence(s, plan)
    token = DeviceBuffer.zeroed(s, 1, np.uint32)
    plan.count = 1  # a count other than the prepared one
    with pytest.raises(W8A8Error):
        mod.linear_sequence(s, plan, token)
    plan.count = 2
    g = Graph(s)
    with pytest.raises(W8A8Error):  # not capturable
        with g:
            mod.linear_sequence(s, plan, token)
    s.synchronize()
    assert mod.sequence_status() == 0
