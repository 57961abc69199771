"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and rejects malformed arguments on the host (negative status
codes) before any HIP call.  With no device present, well-formed calls stop at
the init check (W8A8_EINIT) -- never at a launch."""
from __future__ import annotations

import ctypes
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from inferrous_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "inferrous_w8a8.h"
DIAG_HEADER = ROOT / "include" / "inferrous_w8a8_diag.h"


def declared_symbols(header: Path = HEADER) -> set[str]:
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(w8a8_[a-z0-9_]+)\s*\(", text))


def test_header_declarations_match_binding():
    assert declared_symbols() == set(_lib.SIGNATURES)
    assert declared_symbols(DIAG_HEADER) == set(_lib.DIAG_SIGNATURES)
    assert not declared_symbols() & declared_symbols(DIAG_HEADER)


def declared_arity() -> dict[str, int]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(w8a8_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_integration_rust_binding_covers_header():
    """The Rust FFI block a maintainer would add binds every declared entry
    point, each with the header's number of parameters."""
    doc = (ROOT / "INTEGRATION.md").read_text()
    bound = {}
    for name, params in re.findall(r"pub fn (w8a8_[a-z0-9_]+)\(([^)]*)\)", doc, flags=re.S):
        params = re.sub(r"//[^\n]*", "", params).strip()
        bound[name] = 0 if not params else params.count(",") + 1
    assert bound == declared_arity()


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = (declared_symbols() | declared_symbols(DIAG_HEADER)) - exported
    assert not missing, missing
    L = _lib.lib()
    for name in declared_symbols() | declared_symbols(DIAG_HEADER):
        assert getattr(L, name) is not None


def test_library_targets_gfx950_only():
    """The offload bundle ids embedded in our own build name gfx950 only."""
    blob = _lib.LIB_PATH.read_bytes()
    arches = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-z]+)", blob))
    assert arches == {b"gfx950"}, arches


def test_abi_version_and_status_strings():
    L = _lib.lib()
    assert L.w8a8_abi_version() == 1
    for code in (_lib.OK, _lib.ENULL, _lib.ESHAPE, _lib.EALIGN, _lib.EINIT, _lib.EWORKSPACE,
                 _lib.EARG, _lib.ENODEV):
        assert L.w8a8_status_string(code)


A = 0x10000  # fake, aligned device addresses: validation never dereferences them


def lin(**kw):
    args = dict(stream=None, q=A, asc=A, m=1, w=A, ws=A, n=33, k=4096, out=A, dtype=_lib.OUT_F32,
                path=_lib.PATH_AUTO)
    args.update(kw)
    return _lib.lib().w8a8_linear_path(args["stream"], args["q"], args["asc"], args["m"], args["w"],
                                       args["ws"], args["n"], args["k"], args["out"], args["dtype"],
                                       args["path"])


def no_device_status():
    c = ctypes.c_int()
    _lib.lib().w8a8_device_count(ctypes.byref(c))
    return c.value


def test_diag_timeline_stamp_count():
    """Three stamps per wave of the one-matrix M = 1 launch: two rows per wave
    up to N = 8192 at K = 4096, one above it and at K = 12288, four waves per
    workgroup; other widths are not built (0)."""
    L = _lib.lib()
    assert L.w8a8_diag_linear_timeline_stamps(6144, 4096) == 3 * 3072
    assert L.w8a8_diag_linear_timeline_stamps(8193, 4096) == 3 * 8196
    assert L.w8a8_diag_linear_timeline_stamps(24576, 4096) == 3 * 24576
    assert L.w8a8_diag_linear_timeline_stamps(4097, 12288) == 3 * 4100
    assert L.w8a8_diag_linear_timeline_stamps(1, 4096) == 3 * 4
    assert L.w8a8_diag_linear_timeline_stamps(4096, 1024) == 0
    assert L.w8a8_diag_linear_timeline_stamps(0, 4096) == 0


def test_diag_gemm_timeline_stamp_count():
    """Four stamps per wave of the gemm_tall launch (8 waves per workgroup,
    the route's grid); 0 where the route is not gemm_tall."""
    L = _lib.lib()
    route = np.zeros(20, np.int32)
    for (m, n, k) in [(129, 4096, 4096), (129, 24576, 4096), (24, 4096, 12288), (200, 6100, 4096)]:
        wsb = L.w8a8_linear_workspace_bytes(m, n, k)
        assert L.w8a8_diag_linear_route(m, n, k, _lib.OUT_BF16, 0, 0, wsb, route.ctypes.data, 20) == 0
        assert route[0] == 12
        assert L.w8a8_diag_gemm_timeline_stamps(m, n, k, wsb) == 4 * 8 * route[1]
    assert L.w8a8_diag_gemm_timeline_stamps(512, 4096, 4096, 0) == 0      # gemm_dma
    assert L.w8a8_diag_gemm_timeline_stamps(3, 4096, 4096, 0) == 0        # gemm_narrow
    assert L.w8a8_diag_gemm_timeline_stamps(16, 4096, 12288, 0) == 0      # gemm_narrow
    assert L.w8a8_diag_gemm_timeline_stamps(3, 4096, 1040, 0) == 0        # gemm_skinny
    assert L.w8a8_diag_gemm_timeline_stamps(129, 4096, 4100, 0) == 0      # K % 16 != 0
    assert L.w8a8_diag_gemm_timeline_stamps(0, 4096, 4096, 0) == 0


@pytest.mark.skipif(no_device_status() > 0, reason="validation-order test assumes no GPU")
def test_diag_timeline_validation_precedes_device():
    L = _lib.lib()
    need = L.w8a8_diag_linear_timeline_stamps(4096, 4096)

    def tl(**kw):
        a = dict(q=A, asc=A, w=A, ws=A, n=4096, k=4096, out=A, dt=_lib.OUT_BF16, st=A, sl=need)
        a.update(kw)
        return L.w8a8_diag_linear_timeline(None, a["q"], a["asc"], a["w"], a["ws"], a["n"], a["k"], a["out"],
                                           a["dt"], a["st"], a["sl"])
    assert tl() == _lib.EINIT
    assert tl(n=0) == _lib.OK
    assert tl(k=1024) == _lib.ESHAPE
    assert tl(k=4100) == _lib.ESHAPE
    assert tl(st=None) == _lib.ENULL
    assert tl(st=A + 4) == _lib.EALIGN
    assert tl(sl=need - 1) == _lib.EWORKSPACE
    assert tl(q=None) == _lib.ENULL
    assert tl(dt=7) == _lib.EARG


@pytest.mark.skipif(no_device_status() > 0, reason="validation-order test assumes no GPU")
def test_producer_linear_validation_precedes_device():
    """w8a8_norm_quantize_linear, w8a8_quantize_linear and
    w8a8_norm_quantize_linear_swiglu reject malformed calls on the host,
    including any output that shares bytes with the row every workgroup
    reads."""
    L = _lib.lib()
    B = A + 0x100000  # outputs, clear of x [A, A + 16 KiB) and gain [A + 16 KiB, A + 32 KiB)

    def nql(**kw):
        a = dict(x=A, gain=A + 0x4000, norm=B, q=B + 0x8000, sc=B + 0x9000, mx=B + 0x9010, w=B + 0x10000,
                 ws=B + 0x20000, n=4096, res=None, out=B + 0x30000, comb=None, dt=_lib.OUT_BF16)
        a.update(kw)
        return L.w8a8_norm_quantize_linear(None, a["x"], a["gain"], a["norm"], a["q"], a["sc"], a["mx"], a["w"],
                                           a["ws"], a["n"], a["res"], a["out"], a["comb"], a["dt"])

    def ql(**kw):
        a = dict(x=A, width=4096, q=B + 0x8000, sc=B + 0x9000, mx=None, w=B + 0x10000, ws=B + 0x20000, n=4096,
                 res=B + 0x40000, out=B + 0x30000, comb=B + 0x50000, dt=_lib.OUT_F32)
        a.update(kw)
        return L.w8a8_quantize_linear(None, a["x"], a["width"], a["q"], a["sc"], a["mx"], a["w"], a["ws"], a["n"],
                                      a["res"], a["out"], a["comb"], a["dt"])

    assert nql() == _lib.EINIT
    assert nql(norm=None, mx=None) == _lib.EINIT
    assert nql(n=0) == _lib.ESHAPE
    assert nql(n=1 << 33) == _lib.ESHAPE
    assert nql(gain=None) == _lib.ENULL
    assert nql(q=None) == _lib.ENULL and nql(sc=None) == _lib.ENULL and nql(out=None) == _lib.ENULL
    assert nql(res=B + 0x40000) == _lib.ENULL          # a residual needs combined
    assert nql(q=B + 0x8004) == _lib.EALIGN            # codes are written 16 bytes at a time
    assert nql(x=A + 2) == _lib.EALIGN
    assert nql(dt=7) == _lib.EARG
    assert nql(res=B + 0x40000, comb=B + 0x50000, dt=_lib.OUT_I32) == _lib.EARG
    assert nql(norm=A + 0x10) == _lib.EARG             # the normalised row over x
    assert nql(out=A + 0x4100) == _lib.EARG            # out over the gains
    assert nql(q=A + 0x3ff0) == _lib.EARG              # codes over x's last bytes

    def nqs(**kw):
        a = dict(x=A, gain=A + 0x4000, norm=None, q=B + 0x8000, sc=B + 0x9000, wg=B + 0x10000, sg=B + 0x20000,
                 wu=B + 0x30000, su=B + 0x40000, n=12288, gate=B + 0x50000, up=B + 0x60000, act=B + 0x70000,
                 mx=B + 0x9010, qo=B + 0x80000, so=B + 0x9020, dt=_lib.OUT_F32)
        a.update(kw)
        return L.w8a8_norm_quantize_linear_swiglu(None, a["x"], a["gain"], a["norm"], a["q"], a["sc"], a["wg"],
                                                  a["sg"], a["wu"], a["su"], a["n"], a["gate"], a["up"], a["act"],
                                                  a["mx"], a["qo"], a["so"], a["dt"])

    assert nqs() == _lib.EINIT
    assert nqs(qo=None, so=None) == _lib.EINIT
    assert nqs(n=0) == _lib.ESHAPE
    assert nqs(dt=_lib.OUT_I32) == _lib.EARG
    assert nqs(mx=None) == _lib.ENULL                  # the norm resets it, the row tail folds into it
    assert nqs(so=None) == _lib.ENULL                  # q_out and scales_out go together
    assert nqs(act=None) == _lib.ENULL and nqs(gain=None) == _lib.ENULL
    assert nqs(wu=B + 0x30008) == _lib.EALIGN and nqs(q=B + 0x8008) == _lib.EALIGN
    assert nqs(act=A + 0x100) == _lib.EARG             # act over x
    assert nqs(mx=A + 0x4000) == _lib.EARG             # maxima over the gains
    assert ql() == _lib.EINIT
    assert ql(res=None, comb=None) == _lib.EINIT
    assert ql(width=4095) == _lib.ESHAPE and ql(width=12288) == _lib.ESHAPE
    assert ql(q=None) == _lib.ENULL
    assert ql(comb=None) == _lib.ENULL
    assert ql(comb=A) == _lib.EARG                      # combined over x


@pytest.mark.skipif(no_device_status() > 0, reason="validation-order test assumes no GPU")
def test_norm_quantize_mlp_validation_precedes_device():
    """w8a8_norm_quantize_mlp rejects malformed calls on the host: dtypes,
    the MLP width (12288 only), required and paired pointers, alignment, and
    outputs over x, the gains or (for the down GEMV's outputs) act."""
    L = _lib.lib()
    B = A + 0x100000  # outputs, clear of x [A, A + 16 KiB) and gain [A + 16 KiB, A + 32 KiB)

    def mlp(**kw):
        a = dict(x=A, gain=A + 0x4000, norm=None, q=B + 0x8000, sc=B + 0x9000, wg=B + 0x10000, sg=B + 0x20000,
                 wu=B + 0x30000, su=B + 0x40000, nff=12288, gate=B + 0x50000, up=B + 0x60000, act=B + 0x70000,
                 adt=_lib.OUT_F32, mx=B + 0x9010, qa=B + 0x80000, sa=B + 0x9020, wd=B + 0x90000, sd=B + 0xA0000,
                 n=4096, res=B + 0xB0000, out=B + 0xC0000, comb=B + 0xD0000, dt=_lib.OUT_BF16)
        a.update(kw)
        return L.w8a8_norm_quantize_mlp(None, a["x"], a["gain"], a["norm"], a["q"], a["sc"], a["wg"], a["sg"],
                                        a["wu"], a["su"], a["nff"], a["gate"], a["up"], a["act"], a["adt"], a["mx"],
                                        a["qa"], a["sa"], a["wd"], a["sd"], a["n"], a["res"], a["out"], a["comb"],
                                        a["dt"])

    assert mlp() == _lib.EINIT
    assert mlp(qa=None, sa=None, res=None, comb=None, norm=B) == _lib.EINIT
    assert mlp(adt=_lib.OUT_I32) == _lib.EARG and mlp(dt=_lib.OUT_I32) == _lib.EARG and mlp(dt=9) == _lib.EARG
    assert mlp(nff=4096) == _lib.ESHAPE and mlp(nff=12289) == _lib.ESHAPE
    assert mlp(n=0) == _lib.ESHAPE and mlp(n=1 << 33) == _lib.ESHAPE
    assert mlp(mx=None) == _lib.ENULL and mlp(out=None) == _lib.ENULL and mlp(wd=None) == _lib.ENULL
    assert mlp(sa=None) == _lib.ENULL                  # q_act and scale_act go together
    assert mlp(comb=None) == _lib.ENULL                # a residual needs combined
    assert mlp(qa=B + 0x80008) == _lib.EALIGN and mlp(wd=B + 0x90004) == _lib.EALIGN
    assert mlp(act=B + 0x70002) == _lib.EALIGN and mlp(out=B + 0xC0001) == _lib.EALIGN
    assert mlp(act=A + 0x100) == _lib.EARG             # act over x
    assert mlp(out=A + 0x4000) == _lib.EARG            # out over the gains
    assert mlp(out=B + 0x70000 + 4 * 12000) == _lib.EARG   # out over act, read by every workgroup
    assert mlp(mx=B + 0x70010) == _lib.EARG            # maxima over act


@pytest.mark.skipif(no_device_status() > 0, reason="validation-order test assumes no GPU")
def test_linear_validation_precedes_device():
    assert lin() == _lib.EINIT                       # well formed: stops at init
    assert lin(k=4095) == _lib.ESHAPE                # k % 16
    assert lin(k=0) == _lib.ESHAPE
    assert lin(m=1 << 33) == _lib.ESHAPE
    assert lin(q=None) == _lib.ENULL
    assert lin(ws=None) == _lib.ENULL
    assert lin(q=A + 8) == _lib.EALIGN               # 16-byte operand alignment
    assert lin(w=A + 4) == _lib.EALIGN
    assert lin(out=A + 2) == _lib.EALIGN             # f32 output needs 4 bytes
    assert lin(out=A + 2, dtype=_lib.OUT_BF16) == _lib.EINIT
    assert lin(dtype=7) == _lib.EARG
    assert lin(path=9) == _lib.EARG
    assert lin(m=0) == _lib.OK and lin(n=0) == _lib.OK  # empty problems are no-ops


@pytest.mark.skipif(no_device_status() > 0, reason="validation-order test assumes no GPU")
def test_other_ops_validation():
    L = _lib.lib()
    assert L.w8a8_quantize(None, A, 4096, 1, A, A, None) == _lib.EINIT
    assert L.w8a8_quantize(None, None, 4096, 1, A, A, None) == _lib.ENULL
    assert L.w8a8_quantize(None, A, 0, 1, A, A, None) == _lib.ESHAPE
    assert L.w8a8_quantize(None, A + 2, 4096, 1, A, A, None) == _lib.EALIGN
    assert L.w8a8_quantize_bf16(None, A + 2, 4096, 1, A, A, None) == _lib.EINIT
    assert L.w8a8_quantize_with_max(None, A, 4096, 1, None, A, A) == _lib.ENULL
    assert L.w8a8_rounding_probe(None, A, 10, None) == _lib.ENULL
    # residual needs both extra buffers and a float epilogue
    assert L.w8a8_linear_residual(None, A, A, 1, A, A, 8, 4096, None, A, A, _lib.OUT_F32) == _lib.ENULL
    assert L.w8a8_linear_residual(None, A, A, 1, A, A, 8, 4096, A, A, A, _lib.OUT_I32) == _lib.EARG
    # grouped: 1..4 projections
    W = (ctypes.c_void_p * 4)(A, A, A, A)
    N = (ctypes.c_size_t * 4)(8, 8, 8, 8)
    assert L.w8a8_linear_grouped(None, A, A, 1, 4096, 0, W, W, N, W, 0) == _lib.EARG
    assert L.w8a8_linear_grouped(None, A, A, 1, 4096, 5, W, W, N, W, 0) == _lib.EARG
    assert L.w8a8_linear_grouped(None, A, A, 1, 4096, 3, W, W, N, W, 0) == _lib.EINIT
    # selection workspaces
    need = L.w8a8_select_workspace_bytes(151936)
    assert need >= 16
    assert L.w8a8_select_token(None, A, 151936, A, A, need - 8) == _lib.EWORKSPACE
    assert L.w8a8_select_token(None, A, 151936, A, None, need) == _lib.EWORKSPACE
    assert L.w8a8_select_token(None, A, 151936, A, A, need) == _lib.EINIT
    need = L.w8a8_linear_argmax_workspace_bytes(151936)
    assert L.w8a8_linear_argmax(None, A, A, A, A, 151936, 4096, A, None, 0, A, need) == _lib.EINIT
    assert L.w8a8_linear_argmax(None, A, A, A, A, 151936, 4096, A, None, 0, A, 8) == _lib.EWORKSPACE
    assert L.w8a8_linear_argmax(None, A, A, A, A, 151936, 4096, None, None, 0, A, need) == _lib.ENULL
    assert L.w8a8_linear_argmax(None, A, A, A, A, 151936, 4096, A, A, _lib.OUT_I32, A, need) == _lib.EARG
    assert L.w8a8_synth_i8(None, A + 1, 100, 1, 2) == _lib.EALIGN
    assert L.w8a8_synth_f32(None, A, 100, 1, 2, 2.0, 1.0) == _lib.EARG
    # runtime primitives refuse to run before init
    p = ctypes.c_void_p()
    assert L.w8a8_malloc(ctypes.byref(p), 64) == _lib.EINIT
    assert L.w8a8_stream_create(ctypes.byref(p)) == _lib.EINIT
    assert L.w8a8_init(-1) == _lib.EARG
    assert L.w8a8_init(0) == _lib.ENODEV


@pytest.mark.skipif(no_device_status() > 0, reason="validation-order test assumes no GPU")
def test_fused_and_workspace_entries_validation():
    L = _lib.lib()
    F32, BF16, I32 = _lib.OUT_F32, _lib.OUT_BF16, _lib.OUT_I32
    # swiglu: dtype, empty no-op, nulls, alignment
    assert L.w8a8_swiglu(None, A, A, 1, 12288, A, A, BF16) == _lib.EINIT
    assert L.w8a8_swiglu(None, A, A, 1, 12288, A, A, I32) == _lib.EARG
    assert L.w8a8_swiglu(None, A, A, 0, 12288, A, A, F32) == _lib.OK
    assert L.w8a8_swiglu(None, A, None, 1, 12288, A, A, F32) == _lib.ENULL
    assert L.w8a8_swiglu(None, A, A, 1, 12288, A + 2, A, F32) == _lib.EALIGN
    assert L.w8a8_swiglu(None, A, A, 1, 12288, A, A + 2, BF16) == _lib.EALIGN
    # linear_swiglu(q, asc, m, k, w_gate, ws_gate, w_up, ws_up, n, gate, up, act, maxima, dtype)
    sw = lambda **kw: L.w8a8_linear_swiglu(  # noqa: E731
        None, kw.get("q", A), A, kw.get("m", 1), kw.get("k", 4096), A, A, kw.get("wu", A), A,
        kw.get("n", 12288), A, A, kw.get("act", A), kw.get("maxima", A), kw.get("dtype", F32))
    assert sw() == _lib.EINIT
    assert sw(dtype=I32) == _lib.EARG
    assert sw(k=4095) == _lib.ESHAPE
    assert sw(wu=None) == _lib.ENULL
    assert sw(act=None) == _lib.ENULL
    assert sw(act=A + 2) == _lib.EALIGN
    assert sw(maxima=A + 1) == _lib.EALIGN
    assert sw(m=0) == _lib.OK and sw(n=0) == _lib.OK
    # linear_swiglu_quantize: linear_swiglu's arguments, then maxima, q_out, scales_out (all required)
    swq = lambda **kw: L.w8a8_linear_swiglu_quantize(  # noqa: E731
        None, A, A, kw.get("m", 1), kw.get("k", 4096), A, A, A, A, 12288, A, A, kw.get("act", A),
        kw.get("maxima", A), kw.get("qo", A), kw.get("so", A), kw.get("dtype", F32))
    assert swq() == _lib.EINIT
    assert swq(maxima=None) == _lib.ENULL
    assert swq(qo=None) == _lib.ENULL and swq(so=None) == _lib.ENULL
    assert swq(dtype=I32) == _lib.EARG
    assert swq(k=4095) == _lib.ESHAPE
    assert swq(so=A + 2) == _lib.EALIGN and swq(maxima=A + 1) == _lib.EALIGN
    assert swq(act=A + 2) == _lib.EALIGN
    assert swq(m=0) == _lib.OK
    # linear_quantize_with_max(x, maxima, m, k, q, scales, w, ws, n, residual, out, combined, dtype)
    qm = lambda **kw: L.w8a8_linear_quantize_with_max(  # noqa: E731
        None, kw.get("x", A), kw.get("maxima", A), kw.get("m", 1), 12288, A, A, A, A, 4096,
        kw.get("res"), A, kw.get("comb"), kw.get("dtype", BF16))
    assert qm() == _lib.EINIT
    assert qm(x=None) == _lib.ENULL
    assert qm(maxima=None) == _lib.ENULL
    assert qm(x=A + 4) == _lib.EALIGN
    assert qm(res=A) == _lib.ENULL                   # residual without combined
    assert qm(res=A, comb=A, dtype=I32) == _lib.EARG
    assert qm(res=A, comb=A) == _lib.EINIT
    assert qm(m=0) == _lib.OK
    # norm_quantize(x, gain, rows, width, out, q, scales, maxima): width 4096 only
    nq = lambda **kw: L.w8a8_norm_quantize(  # noqa: E731
        None, kw.get("x", A), A, kw.get("m", 2), kw.get("width", 4096), kw.get("out", A), A, A,
        kw.get("maxima", A))
    assert nq() == _lib.EINIT
    assert nq(width=4095) == _lib.ESHAPE and nq(width=2048) == _lib.ESHAPE
    assert nq(m=0) == _lib.OK
    assert nq(x=None) == _lib.ENULL and nq(maxima=None) == _lib.ENULL
    assert nq(out=A + 2) == _lib.EALIGN
    # linear_ex: the split-K workspace is optional, never required
    # the MFMA family's split plan for down at m = 24 (4 slabs); below m = 17 the narrow kernel needs none
    assert L.w8a8_linear_workspace_bytes(24, 4096, 12288) == 4 * 24 * 4096 * 4
    assert L.w8a8_linear_workspace_bytes(1, 4096, 12288) == 0      # narrow kernel: none
    assert L.w8a8_linear_workspace_bytes(4, 4096, 4096) == 0       # narrow kernel: none
    assert L.w8a8_linear_workspace_bytes(4, 4096, 1040) == 0       # skinny kernel: none
    assert L.w8a8_linear_workspace_bytes(512, 4096, 12288) > 0     # 128x128 split in two
    assert L.w8a8_linear_workspace_bytes(512, 4096, 12288) == 2 * 512 * 4096 * 4
    ex = lambda **kw: L.w8a8_linear_ex(  # noqa: E731
        None, A, A, kw.get("m", 512), A, A, 4096, 12288, None, A, None, F32,
        kw.get("path", _lib.PATH_AUTO), kw.get("wsp", A), kw.get("wsb", 1 << 24))
    assert ex() == _lib.EINIT
    assert ex(wsp=None, wsb=0) == _lib.EINIT
    assert ex(wsb=16) == _lib.EINIT                   # too small: runs unsplit
    assert ex(wsp=A + 8) == _lib.EALIGN
    assert ex(path=9) == _lib.EARG


def test_module_requires_library_not_oracle():
    """The product package never imports the oracle."""
    for py in (ROOT / "inferrous_amd").rglob("*.py"):
        text = py.read_text()
        assert "import oracle" not in text and "from oracle" not in text, py


def test_bf16_packer_is_host_side_and_matches_oracle():
    """w8a8_bf16_pack needs no device: the library's packer against the oracle's."""
    import numpy as np

    import oracle
    from inferrous_amd import PackedBf16
    a = np.arange(65536, dtype=np.uint32)
    rng = np.random.default_rng(9)
    trained = (rng.standard_normal(4096 * 4).astype(np.float32) * 0.02).view(np.uint32) >> 16
    v = np.concatenate([a, (a * 40503) % 65536, trained]).astype(np.uint16)
    p = PackedBf16.new(v)
    w, o, e = oracle.bf16_pack(v)
    assert np.array_equal(p.words, w) and np.array_equal(p.offsets, o) and np.array_equal(p.exceptions, e)
    L = _lib.lib()
    n = ctypes.c_size_t()
    buf = np.zeros(512, np.uint32)
    exc = np.zeros(1, np.uint16)
    zeros = np.zeros(256, np.uint16)        # every value escapes: capacity 1 is too small
    assert L.w8a8_bf16_pack(zeros.ctypes.data, 256, buf.ctypes.data, buf.ctypes.data, exc.ctypes.data, 1,
                            ctypes.byref(n)) == _lib.EWORKSPACE
    assert L.w8a8_bf16_pack(zeros.ctypes.data, 255, buf.ctypes.data, buf.ctypes.data, exc.ctypes.data, 1,
                            ctypes.byref(n)) == _lib.ESHAPE
    assert L.w8a8_bf16_pack(zeros.ctypes.data, 256, buf.ctypes.data, buf.ctypes.data, exc.ctypes.data, 1,
                            None) == _lib.ENULL


@pytest.mark.skipif(no_device_status() > 0, reason="validation-order test assumes no GPU")
def test_head_entries_validation():
    L = _lib.lib()
    assert L.w8a8_head_packed(None, A, 4096, A, A, A, 1, 33, A) == _lib.EINIT
    assert L.w8a8_head_packed(None, A, 4095, A, A, A, 1, 33, A) == _lib.ESHAPE
    assert L.w8a8_head_packed(None, A, 4096, A, A, A, 0, 33, A) == _lib.ESHAPE
    assert L.w8a8_head_packed(None, A, 4096, A, A, A, 1, 0, A) == _lib.OK
    assert L.w8a8_head_packed(None, A, 4096, None, A, A, 1, 33, A) == _lib.ENULL
    assert L.w8a8_head_packed(None, A + 2, 4096, A, A, A, 1, 33, A) == _lib.EALIGN
    assert L.w8a8_unpack_bf16(None, A, A, A, 256, A) == _lib.EINIT
    assert L.w8a8_unpack_bf16(None, A, A, A, 255, A) == _lib.ESHAPE
    assert L.w8a8_unpack_bf16(None, A, A, A, 256, A + 1) == _lib.EALIGN


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus 2 exits with status 2 and a message,
    before anything touches a device."""
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_bench_reads_the_committed_traffic_profile():
    """roofline.traffic comes from the committed FETCH_SIZE / WRITE_SIZE
    summary of the gate_up GEMV: the bench parses it, and it is within 2%
    above the launch's algorithmic bytes (N K + 4 N + K + 4 + 2 N)."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("bench_mod", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    traffic = bench.measured_traffic()
    algorithmic = bench.gemv_bytes(24576, 4096)
    assert traffic is not None
    assert algorithmic <= traffic <= 1.02 * algorithmic, (traffic, algorithmic)


def _fake(n, dtype):
    """A DeviceBuffer-shaped object for host-side validation only: a fake
    aligned address that no call reaches, since the checks raise first."""
    import numpy as np

    from inferrous_amd import DeviceBuffer
    b = DeviceBuffer.__new__(DeviceBuffer)
    b.dtype, b.n = np.dtype(dtype), int(n)
    b.nbytes = b.n * b.dtype.itemsize
    b._p, b._base = A, object()     # a view: never freed
    return b


def test_module_grouped_and_swiglu_check_operand_lengths():
    """Short q or weight buffers raise ValueError before the library is
    called, for every member of a group and both SwiGLU matrices."""
    import numpy as np

    from inferrous_amd import LoadedModule
    mod = LoadedModule(None)
    m, k, n = 2, 64, 8
    q, asc = _fake(m * k, np.int8), _fake(m, np.float32)
    ws, out = _fake(n, np.float32), _fake(m * n, np.float32)
    good, short = _fake(n * k, np.int8), _fake(n * k - 1, np.int8)
    with pytest.raises(ValueError, match="q"):
        mod.linear_grouped(None, _fake(m * k - 16, np.int8), asc, k, [(good, ws, out)])
    with pytest.raises(ValueError, match=r"w\[2\]"):
        mod.linear_triple(None, None, q, asc, k, good, ws, out, good, ws, out, short, ws, out)
    with pytest.raises(ValueError, match="w_up"):
        mod.linear_swiglu(None, None, q, asc, k, good, ws, out, short, ws, out, out, None)
    with pytest.raises(ValueError, match="w_gate"):
        mod.linear_swiglu(None, None, q, asc, k, short, ws, out, good, ws, out, out, None)
    with pytest.raises(ValueError, match="q"):
        mod.linear_swiglu(None, None, _fake(k, np.int8), asc, k, good, ws, out, good, ws, out, out, None)
    mx, qo, so = _fake(m, np.uint32), _fake(m * n, np.int8), _fake(m, np.float32)
    with pytest.raises(ValueError, match="w_up"):
        mod.linear_swiglu_quantize(None, None, q, asc, k, good, ws, out, short, ws, out, out, mx, qo, so)
    with pytest.raises(ValueError, match="q_out"):
        mod.linear_swiglu_quantize(None, None, q, asc, k, good, ws, out, good, ws, out, out, mx,
                                   _fake(m * n - 1, np.int8), so)


def test_module_argmax_and_quantize_with_max_check_operand_lengths():
    """linear_argmax and linear_quantize_with_max refuse a weight matrix
    shorter than N*K and an activation row shorter than K with ValueError,
    before the library is called (a short buffer must never reach the
    device as an out-of-bounds read)."""
    import numpy as np

    from inferrous_amd import LoadedModule
    mod = LoadedModule(None)
    k, n = 64, 8
    asc, ws, tok = _fake(1, np.float32), _fake(n, np.float32), _fake(1, np.uint32)
    good_w, short_w = _fake(n * k, np.int8), _fake(n * k - 1, np.int8)
    with pytest.raises(ValueError, match="w has"):
        mod.linear_argmax(None, _fake(k, np.int8), asc, short_w, ws, k, tok)
    with pytest.raises(ValueError, match="q has"):
        mod.linear_argmax(None, _fake(k - 16, np.int8), asc, good_w, ws, k, tok)
    m = 2
    x, q, sc = _fake(m * k, np.float32), _fake(m * k, np.int8), _fake(m, np.float32)
    out = _fake(m * n, np.float32)
    with pytest.raises(ValueError, match="w has"):
        mod.linear_quantize_with_max(None, None, x, k, _fake(m, np.uint32), q, sc, short_w, ws, out)
    with pytest.raises(ValueError, match="maxima has"):
        mod.linear_quantize_with_max(None, None, x, k, _fake(m - 1, np.uint32), q, sc, good_w, ws, out)
    with pytest.raises(ValueError, match="sizes do not match"):
        mod.linear_quantize_with_max(None, None, x, k, _fake(m, np.uint32), _fake(m * k - 4, np.int8), sc,
                                     good_w, ws, out)


@pytest.mark.skipif(no_device_status() > 0, reason="validation-order test assumes no GPU")
def test_noalloc_argmax_validation():
    """Rows beyond the fixed key array are refused with ESHAPE before any
    device call; the other checks are w8a8_linear_argmax's."""
    L = _lib.lib()
    top = _lib.NOALLOC_MAX_ROWS
    assert L.w8a8_linear_argmax_noalloc(None, A, A, A, A, top + 1, 4096, A, None, 0) == _lib.ESHAPE
    assert L.w8a8_linear_argmax_noalloc(None, A, A, A, A, top, 4096, A, None, 0) == _lib.EINIT
    assert L.w8a8_linear_argmax_noalloc(None, A, A, A, A, top, 4096, None, None, 0) == _lib.ENULL
    assert L.w8a8_linear_argmax_noalloc(None, A, A, A, A, top, 4096, A + 2, None, 0) == _lib.EALIGN
    assert L.w8a8_linear_argmax_noalloc(None, A, A, A, A, top, 4096, A, A, 7) == _lib.EARG
    assert L.w8a8_linear_argmax_noalloc(None, A, A, A, A, 33, 4004, A, None, 0) == _lib.ESHAPE


def test_workspace_queries_by_route_and_batch_range():
    """The split-K workspace need depends on the route and is not monotone
    in M: the narrow kernel (M <= 16 on down) needs none, the one-M-tile
    split-K route above it does, AUTO at M = 1 runs the dot4 GEMV, DOT4
    never needs any, MFMA keeps the shape's need; the largest need over
    M = 1..512 for qkv (6144 x 4096) sits at M = 256, where M = 512 needs
    none."""
    L = _lib.lib()
    down = (4096, 12288)
    assert all(L.w8a8_linear_workspace_bytes(m, *down) == 0 for m in range(1, 17))
    assert L.w8a8_linear_workspace_bytes(17, *down) > 0
    assert L.w8a8_linear_workspace_bytes_path(24, *down, _lib.PATH_AUTO) == L.w8a8_linear_workspace_bytes(24, *down)
    assert L.w8a8_linear_workspace_bytes_path(24, *down, _lib.PATH_MFMA) == L.w8a8_linear_workspace_bytes(24, *down)
    assert L.w8a8_linear_workspace_bytes_path(2, *down, _lib.PATH_AUTO) == 0
    assert L.w8a8_linear_workspace_bytes_path(64, *down, _lib.PATH_DOT4) == 0
    assert L.w8a8_linear_workspace_bytes_path(64, *down, 7) == 0
    qkv = (6144, 4096)
    at256 = L.w8a8_linear_workspace_bytes(256, *qkv)
    assert at256 == 4 * 256 * 6144 * 4 and L.w8a8_linear_workspace_bytes(512, *qkv) == 0
    assert L.w8a8_linear_workspace_bytes_upto(512, *qkv) == at256
    assert L.w8a8_linear_workspace_bytes_upto(512, *down) == max(
        L.w8a8_linear_workspace_bytes(m, *down) for m in range(1, 513))
    assert L.w8a8_linear_workspace_bytes_upto(0, *down) == 0


@pytest.mark.skipif(no_device_status() > 0, reason="validation-order test assumes no GPU")
def test_sequence_prepare_validation_precedes_device():
    """w8a8_linear_sequence_prepare checks every entry on the host before
    any device call; a well-formed table stops at the init check."""
    L = _lib.lib()
    S = _lib.SeqEntry

    def ent(**kw):
        a = dict(w=A, ws=A, q=A, asc=A, out=A, residual=None, combined=None, n=4096, k=4096,
                 out_dtype=_lib.OUT_BF16, flags=0)
        a.update(kw)
        return S(a["w"], a["ws"], a["q"], a["asc"], a["out"], a["residual"], a["combined"], a["n"], a["k"],
                 a["out_dtype"], a["flags"])

    def prep(*entries, table=A, nbytes=None, count=None):
        arr = (S * len(entries))(*entries)
        count = len(entries) if count is None else count
        nbytes = 64 * len(entries) if nbytes is None else nbytes
        return L.w8a8_linear_sequence_prepare(arr, count, table, nbytes)

    assert L.w8a8_linear_sequence_table_bytes(145) == 145 * 64
    good = ent()
    assert prep(good, good) == _lib.EINIT
    assert prep(good, ent(out=None, flags=_lib.SEQ_SELECT, out_dtype=_lib.OUT_F32, n=151936)) == _lib.EINIT
    assert prep(good, ent(k=12288, residual=A, combined=A)) == _lib.EINIT
    assert prep(good, count=0) == _lib.ESHAPE
    assert L.w8a8_linear_sequence_prepare(None, 1, A, 64) == _lib.ENULL
    assert prep(good, table=None) == _lib.ENULL
    assert prep(good, good, nbytes=127) == _lib.EWORKSPACE
    assert prep(good, table=A + 8) == _lib.EALIGN
    assert prep(ent(k=1024)) == _lib.ESHAPE
    assert prep(ent(k=4100)) == _lib.ESHAPE
    assert prep(ent(n=0)) == _lib.ESHAPE
    assert prep(ent(n=1 << 33)) == _lib.ESHAPE
    assert prep(ent(out_dtype=_lib.OUT_I32)) == _lib.EARG
    assert prep(ent(flags=2)) == _lib.EARG
    assert prep(ent(flags=_lib.SEQ_SELECT), good) == _lib.EARG      # only the last entry selects
    assert prep(ent(flags=_lib.SEQ_SELECT, residual=A, combined=A)) == _lib.EARG
    assert prep(ent(out=None)) == _lib.ENULL
    assert prep(ent(w=None)) == _lib.ENULL and prep(ent(q=None)) == _lib.ENULL
    assert prep(ent(residual=A)) == _lib.ENULL and prep(ent(combined=A)) == _lib.ENULL
    assert prep(ent(w=A + 4)) == _lib.EALIGN and prep(ent(q=A + 8)) == _lib.EALIGN
    assert prep(ent(out=A + 1)) == _lib.EALIGN and prep(ent(ws=A + 2)) == _lib.EALIGN
    assert prep(ent(out=A + 2, out_dtype=_lib.OUT_F32)) == _lib.EALIGN
    assert L.w8a8_linear_sequence(None, None, 1, None, None, 0, 0) == _lib.ENULL
    assert L.w8a8_linear_sequence(None, A, 1, None, None, 0, 0) == _lib.EINIT
    assert L.w8a8_linear_sequence_status(None) == _lib.ENULL
    st = ctypes.c_uint32()
    assert L.w8a8_linear_sequence_status(ctypes.byref(st)) == _lib.EINIT
    assert L.w8a8_linear_sequence_reset() == _lib.EINIT
    assert L.w8a8_linear_sequence_workspace_bytes() == 0


def test_module_sequence_checks_entries():
    """The Python mirror refuses malformed sequence entries with
    ValueError / TypeError before the library is called."""
    import numpy as np

    from inferrous_amd import LoadedModule
    mod = LoadedModule(None)
    k, n = 4096, 64
    e = dict(q=_fake(k, np.int8), asc=_fake(1, np.float32), w=_fake(n * k, np.int8), ws=_fake(n, np.float32),
             out=_fake(n, np.uint16))
    with pytest.raises(ValueError, match="at least one"):
        mod.prepare_sequence([])
    with pytest.raises(ValueError, match="w has"):
        mod.prepare_sequence([dict(e, w=_fake(n * k - 1, np.int8))])
    with pytest.raises(ValueError, match="one activation row"):
        mod.prepare_sequence([dict(e, asc=_fake(2, np.float32))])
    with pytest.raises(ValueError, match="only the last"):
        mod.prepare_sequence([dict(e, select=True), e])
    with pytest.raises(ValueError, match="out is required"):
        mod.prepare_sequence([dict(e, out=None)])
    with pytest.raises(TypeError, match="float32 or uint16"):
        mod.prepare_sequence([dict(e, out=_fake(n, np.int32))])
    with pytest.raises(ValueError, match="go together"):
        mod.prepare_sequence([dict(e, residual=_fake(n, np.float32))])
    with pytest.raises(ValueError, match="N values"):
        mod.prepare_sequence([dict(e, residual=_fake(n, np.float32), combined=_fake(n, np.float32))])
