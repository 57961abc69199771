"""CPU oracle for the W8A8 linear-layer path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference's arithmetic (bitemyapp/inferrous,
``crates/inferrous-qwen3/src/kernels.rs`` and friends) in plain C
(``w8a8_oracle.c``) and exposes it to Python through ctypes.  Only the test
suite, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import it, as the checker (or as the timed CPU baseline).  The product
package ``inferrous_amd`` never imports it; its ops fail loudly when the HIP
library is missing instead of falling back to anything here.

Every wrapped function cites the reference file:line it follows in the C
header (``w8a8_oracle.h``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liborc_w8a8.so"
_lib = None

SENTINEL = 0xFFFFFFFF


def build(force: bool = False) -> Path:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(_HERE), "-B" if force else "all"],
                       check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        P = ctypes.c_void_p
        S = ctypes.c_size_t
        U64 = ctypes.c_uint64
        sig = {
            "orc_bf16_rne": (ctypes.c_float, [ctypes.c_float]),
            "orc_round_many": (None, [P, S, P]),
            "orc_absmax_bits": (ctypes.c_uint32, [P, S]),
            "orc_quantize_rows": (None, [P, S, S, P, P]),
            "orc_quantize_rows_bf16": (None, [P, S, S, P, P]),
            "orc_quantize_rows_with_max": (None, [P, S, S, P, P, P]),
            "orc_linear_i32": (None, [P, S, P, S, S, P, ctypes.c_int]),
            "orc_epilogue": (None, [P, P, S, P, S, P, P]),
            "orc_linear": (None, [P, P, S, P, P, S, S, P, P, P, ctypes.c_int]),
            "orc_residual": (None, [P, P, S, P]),
            "orc_silu_mul": (ctypes.c_float, [ctypes.c_float, ctypes.c_float]),
            "orc_swiglu": (ctypes.c_uint32, [P, P, S, P]),
            "orc_norm_sum_sq": (ctypes.c_float, [P]),
            "orc_bf16_pack": (S, [P, S, P, P, P]),
            "orc_bf16_unpack_at": (ctypes.c_uint16, [P, P, P, S]),
            "orc_head_bf16": (None, [P, P, S, P]),
            "orc_norm_rows": (None, [P, P, S, P]),
            "orc_norm_quantize": (None, [P, P, S, P, P, P, P]),
            "orc_argmax": (ctypes.c_uint32, [P, S]),
            "orc_linear_argmax": (ctypes.c_uint32, [P, P, P, P, S, S, P, ctypes.c_int]),
            "orc_mix64": (U64, [U64]),
            "orc_synth_hash": (U64, [U64, U64, U64]),
            "orc_synth_i8": (None, [U64, U64, U64, S, P]),
            "orc_synth_f32": (None, [U64, U64, U64, S, ctypes.c_float, ctypes.c_float, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def default_threads() -> int:
    return max(1, min(os.cpu_count() or 1, 16))


# ---------------------------------------------------------------- scalars
def bf16_rne(x: np.ndarray) -> np.ndarray:
    """src/kernels.rs:11-15, vectorised on the bit pattern (same formula)."""
    u = _c(x, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000) & 0xFFFFFFFF
    return u.astype(np.uint32).view(np.float32)


def round_i8(x: np.ndarray) -> np.ndarray:
    """src/kernels.rs:24-34 via the C oracle."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.int8)
    lib().orc_round_many(_p(x), x.size, _p(out))
    return out


# ---------------------------------------------------------------- quantize
def quantize(x: np.ndarray, width: int):
    """src/kernels.rs:414-452. x: f32 [rows*width] -> (q i8, scales f32)."""
    x = _c(x, np.float32).reshape(-1)
    rows = x.size // width
    q = np.empty(rows * width, np.int8)
    s = np.empty(rows, np.float32)
    lib().orc_quantize_rows(_p(x), rows, width, _p(q), _p(s))
    return q, s


def quantize_bf16(x_bits: np.ndarray, width: int):
    x = _c(x_bits, np.uint16).reshape(-1)
    rows = x.size // width
    q = np.empty(rows * width, np.int8)
    s = np.empty(rows, np.float32)
    lib().orc_quantize_rows_bf16(_p(x), rows, width, _p(q), _p(s))
    return q, s


def quantize_with_max(x: np.ndarray, width: int, maxima: np.ndarray):
    """src/kernels.rs:453-475."""
    x = _c(x, np.float32).reshape(-1)
    maxima = _c(maxima, np.uint32)
    rows = x.size // width
    q = np.empty(rows * width, np.int8)
    s = np.empty(rows, np.float32)
    lib().orc_quantize_rows_with_max(_p(x), rows, width, _p(maxima), _p(q), _p(s))
    return q, s


def absmax_bits(x: np.ndarray) -> int:
    x = _c(x, np.float32).reshape(-1)
    return int(lib().orc_absmax_bits(_p(x), x.size))


# ---------------------------------------------------------------- linear
def linear_i32(q: np.ndarray, w: np.ndarray, m: int, n: int, k: int,
               threads: int | None = None) -> np.ndarray:
    q = _c(q, np.int8)
    w = _c(w, np.int8)
    acc = np.empty(m * n, np.int32)
    lib().orc_linear_i32(_p(q), m, _p(w), n, k, _p(acc), threads or default_threads())
    return acc


def linear(q, asc, w, ws, k: int, threads: int | None = None):
    """(acc i32 [m*n], out f32 [m*n] holding BF16 values, out bf16 bits)."""
    q = _c(q, np.int8)
    asc = _c(asc, np.float32)
    w = _c(w, np.int8)
    ws = _c(ws, np.float32)
    m, n = asc.size, ws.size
    acc = np.empty(m * n, np.int32)
    out = np.empty(m * n, np.float32)
    outb = np.empty(m * n, np.uint16)
    lib().orc_linear(_p(q), _p(asc), m, _p(w), _p(ws), n, k, _p(acc), _p(out),
                     _p(outb), threads or default_threads())
    return acc, out, outb


def epilogue(acc, asc, ws):
    acc = _c(acc, np.int32)
    asc = _c(asc, np.float32)
    ws = _c(ws, np.float32)
    m, n = asc.size, ws.size
    out = np.empty(m * n, np.float32)
    outb = np.empty(m * n, np.uint16)
    lib().orc_epilogue(_p(acc), _p(asc), m, _p(ws), n, _p(out), _p(outb))
    return out, outb


def residual(res, out):
    res = _c(res, np.float32)
    out = _c(out, np.float32)
    comb = np.empty(res.size, np.float32)
    lib().orc_residual(_p(res), _p(out), res.size, _p(comb))
    return comb


def swiglu(gate, up):
    """(act f32[n], published maximum bits) -- src/kernels.rs:2172-2190."""
    g = _c(gate, np.float32).reshape(-1)
    u = _c(up, np.float32).reshape(-1)
    act = np.empty(g.size, np.float32)
    mx = int(lib().orc_swiglu(_p(g), _p(u), g.size, _p(act)))
    return act, mx


def norm_sum_sq(x) -> float:
    """The reference's sum-of-squares tree for one 4096-wide row
    (src/kernels.rs:354-392)."""
    x = _c(x, np.float32).reshape(-1)
    assert x.size == 4096
    return float(lib().orc_norm_sum_sq(_p(x)))


def norm_rows(x, gain):
    """`norm` at width 4096 (src/kernels.rs:347-402); rsqrt in binary64."""
    x = _c(x, np.float32).reshape(-1, 4096)
    g = _c(gain, np.float32).reshape(4096)
    out = np.empty_like(x)
    lib().orc_norm_rows(_p(x), _p(g), x.shape[0], _p(out))
    return out


def norm_quantize(x, gain):
    """(out, q, scales, maxima) of `norm_quantize` (src/kernels.rs:476-575)."""
    x = _c(x, np.float32).reshape(-1, 4096)
    g = _c(gain, np.float32).reshape(4096)
    rows = x.shape[0]
    out = np.empty_like(x)
    q = np.empty((rows, 4096), np.int8)
    s = np.empty(rows, np.float32)
    mx = np.empty(rows, np.uint32)
    lib().orc_norm_quantize(_p(x), _p(g), rows, _p(out), _p(q), _p(s), _p(mx))
    return out, q, s, mx


def bf16_pack(values):
    """src/packing.rs:8-46: (words u32, offsets u32, exceptions u16)."""
    v = _c(values, np.uint16).reshape(-1)
    assert v.size % 256 == 0
    words = np.empty(v.size // 8 * 3, np.uint32)
    offsets = np.empty(v.size // 256, np.uint32)
    exc = np.empty(max(v.size, 1), np.uint16)
    n = int(lib().orc_bf16_pack(_p(v), v.size, _p(words), _p(offsets), _p(exc)))
    return words, offsets, exc[:n].copy()


def bf16_unpack_at(words, offsets, exceptions, i: int) -> int:
    words = _c(words, np.uint32)
    offsets = _c(offsets, np.uint32)
    exceptions = _c(exceptions, np.uint16)
    return int(lib().orc_bf16_unpack_at(_p(words), _p(offsets), _p(exceptions), i))


def head_bf16(x, w_bits):
    """`head` (src/kernels.rs:2233-2257): x's last 4096 values against BF16
    rows [rows, 4096]; f32 logits holding BF16 values."""
    x = _c(x, np.float32).reshape(-1)[-4096:].copy()
    w = _c(w_bits, np.uint16).reshape(-1, 4096)
    out = np.empty(w.shape[0], np.float32)
    lib().orc_head_bf16(_p(x), _p(w), w.shape[0], _p(out))
    return out


def argmax(x) -> int:
    x = _c(x, np.float32).reshape(-1)
    return int(lib().orc_argmax(_p(x), x.size))


def linear_argmax(q, asc, w, ws, k: int, threads: int | None = None):
    q = _c(q, np.int8)
    asc = _c(asc, np.float32)
    w = _c(w, np.int8)
    ws = _c(ws, np.float32)
    n = ws.size
    logits = np.empty(n, np.float32)
    tok = lib().orc_linear_argmax(_p(q), _p(asc), _p(w), _p(ws), n, k, _p(logits),
                                  threads or default_threads())
    return int(tok), logits


# ---------------------------------------------------------------- synthetic
def mix64(x: int) -> int:
    return int(lib().orc_mix64(x))


def synth_i8(seed: int, stream: int, first: int, n: int) -> np.ndarray:
    out = np.empty(n, np.int8)
    lib().orc_synth_i8(seed, stream, first, n, _p(out))
    return out


def synth_f32(seed: int, stream: int, first: int, n: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_synth_f32(seed, stream, first, n, lo, hi, _p(out))
    return out
