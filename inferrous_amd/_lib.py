"""ctypes binding of the C ABI declared in include/inferrous_w8a8.h.

The HIP library must exist (build it with ``python -m inferrous_amd.build``);
there is no fallback: loading fails loudly with the path it looked for.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libinferrous_w8a8.so"

OK = 0
ENULL, ESHAPE, EALIGN, EINIT, EWORKSPACE, EARG, ENODEV = -1, -2, -3, -4, -5, -6, -7
OUT_F32, OUT_BF16, OUT_I32 = 0, 1, 2
PATH_AUTO, PATH_DOT4, PATH_MFMA = 0, 1, 2
NOALLOC_MAX_ROWS = 262144  # W8A8_NOALLOC_MAX_ROWS
SEQ_SELECT = 1  # W8A8_SEQ_SELECT


class SeqEntry(ctypes.Structure):
    """w8a8_seq_entry (include/inferrous_w8a8.h)."""
    _fields_ = [("w", ctypes.c_void_p), ("ws", ctypes.c_void_p), ("q", ctypes.c_void_p),
                ("asc", ctypes.c_void_p), ("out", ctypes.c_void_p), ("residual", ctypes.c_void_p),
                ("combined", ctypes.c_void_p), ("n", ctypes.c_size_t), ("k", ctypes.c_uint32),
                ("out_dtype", ctypes.c_int), ("flags", ctypes.c_int)]

P = ctypes.c_void_p
S = ctypes.c_size_t
I = ctypes.c_int
U32 = ctypes.c_uint32
U64 = ctypes.c_uint64
F = ctypes.c_float

# name -> (restype, argtypes); every symbol declared in the header.
SIGNATURES: dict[str, tuple] = {
    "w8a8_abi_version": (I, []),
    "w8a8_status_string": (ctypes.c_char_p, [I]),
    "w8a8_init": (I, [I]),
    "w8a8_device_count": (I, [P]),
    "w8a8_device_info": (I, [P, ctypes.c_char_p, S]),
    "w8a8_device_clock_khz": (I, [P]),
    "w8a8_stream_create": (I, [P]),
    "w8a8_stream_destroy": (I, [P]),
    "w8a8_stream_synchronize": (I, [P]),
    "w8a8_malloc": (I, [P, S]),
    "w8a8_free": (I, [P]),
    "w8a8_host_malloc": (I, [P, S]),
    "w8a8_host_free": (I, [P]),
    "w8a8_memcpy_htod": (I, [P, P, S, P]),
    "w8a8_memcpy_dtoh": (I, [P, P, S, P]),
    "w8a8_memcpy_dtod": (I, [P, P, S, P]),
    "w8a8_fill_zero": (I, [P, S, P]),
    "w8a8_event_create": (I, [P]),
    "w8a8_event_destroy": (I, [P]),
    "w8a8_event_record": (I, [P, P]),
    "w8a8_event_synchronize": (I, [P]),
    "w8a8_event_elapsed_ms": (I, [P, P, P]),
    "w8a8_graph_capture_begin": (I, [P]),
    "w8a8_graph_capture_end": (I, [P, P]),
    "w8a8_graph_launch": (I, [P, P]),
    "w8a8_graph_destroy": (I, [P]),
    "w8a8_rounding_probe": (I, [P, P, S, P]),
    "w8a8_quantize": (I, [P, P, U32, S, P, P, P]),
    "w8a8_quantize_bf16": (I, [P, P, U32, S, P, P, P]),
    "w8a8_quantize_with_max": (I, [P, P, U32, S, P, P, P]),
    "w8a8_linear": (I, [P, P, P, S, P, P, S, U32, P, I]),
    "w8a8_linear_path": (I, [P, P, P, S, P, P, S, U32, P, I, I]),
    "w8a8_linear_residual": (I, [P, P, P, S, P, P, S, U32, P, P, P, I]),
    "w8a8_linear_grouped": (I, [P, P, P, S, U32, I, P, P, P, P, I]),
    "w8a8_linear_workspace_bytes": (S, [S, S, U32]),
    "w8a8_linear_workspace_bytes_path": (S, [S, S, U32, I]),
    "w8a8_linear_workspace_bytes_upto": (S, [S, S, U32]),
    "w8a8_norm_quantize": (I, [P, P, P, S, U32, P, P, P, P]),
    "w8a8_bf16_pack": (I, [P, S, P, P, P, S, P]),
    "w8a8_head_packed": (I, [P, P, S, P, P, P, S, S, P]),
    "w8a8_unpack_bf16": (I, [P, P, P, P, S, P]),
    "w8a8_linear_ex": (I, [P, P, P, S, P, P, S, U32, P, P, P, I, I, P, S]),
    "w8a8_linear_quantize_with_max": (I, [P, P, P, S, U32, P, P, P, P, S, P, P, P, I]),
    "w8a8_linear_swiglu": (I, [P, P, P, S, U32, P, P, P, P, S, P, P, P, P, I]),
    "w8a8_linear_swiglu_quantize": (I, [P, P, P, S, U32, P, P, P, P, S, P, P, P, P, P, P, I]),
    "w8a8_norm_quantize_linear": (I, [P, P, P, P, P, P, P, P, P, S, P, P, P, I]),
    "w8a8_quantize_linear": (I, [P, P, U32, P, P, P, P, P, S, P, P, P, I]),
    "w8a8_norm_quantize_linear_swiglu": (I, [P, P, P, P, P, P, P, P, P, P, S, P, P, P, P, P, P, I]),
    "w8a8_norm_quantize_mlp": (I, [P, P, P, P, P, P, P, P, P, P, S, P, P, P, I, P, P, P, P, P, S, P, P, P, I]),
    "w8a8_swiglu": (I, [P, P, P, S, U32, P, P, I]),
    "w8a8_select_workspace_bytes": (S, [S]),
    "w8a8_select_token": (I, [P, P, S, P, P, S]),
    "w8a8_linear_argmax_workspace_bytes": (S, [S]),
    "w8a8_linear_argmax": (I, [P, P, P, P, P, S, U32, P, P, I, P, S]),
    "w8a8_linear_argmax_noalloc": (I, [P, P, P, P, P, S, U32, P, P, I]),
    "w8a8_linear_sequence_table_bytes": (S, [S]),
    "w8a8_linear_sequence_prepare": (I, [P, S, P, S]),
    "w8a8_linear_sequence_workspace_bytes": (S, []),
    "w8a8_linear_sequence": (I, [P, P, S, P, P, S, U32]),
    "w8a8_linear_sequence_status": (I, [P]),
    "w8a8_linear_sequence_reset": (I, []),
    "w8a8_synth_i8": (I, [P, P, S, U64, U64]),
    "w8a8_synth_f32": (I, [P, P, S, U64, U64, F, F]),
}

_lib: ctypes.CDLL | None = None


class W8A8Error(RuntimeError):
    def __init__(self, status: int, what: str = ""):
        self.status = status
        msg = status_string(status) if _lib is not None else str(status)
        super().__init__(f"{what}: status {status} ({msg})" if what else f"status {status} ({msg})")


# Diagnostics declared in include/inferrous_w8a8_diag.h (no reference
# counterpart; used by bench.py --timeline).
DIAG_SIGNATURES: dict[str, tuple] = {
    "w8a8_diag_linear_timeline_stamps": (S, [S, U32]),
    "w8a8_diag_linear_timeline": (I, [P, P, P, P, P, S, U32, P, I, P, S]),
    "w8a8_diag_linear_route": (I, [S, S, U32, I, I, I, S, P, S]),
    "w8a8_diag_gemm_timeline_stamps": (S, [S, S, U32, S]),
    "w8a8_diag_gemm_timeline": (I, [P, P, P, S, P, P, S, U32, P, P, S, P, S]),
    "w8a8_diag_argmax_route": (I, [S, U32, P, S]),
}


def lib() -> ctypes.CDLL:
    """Load the HIP library (once).  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"HIP library not found at {LIB_PATH}; build it with `python -m inferrous_amd.build`")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in {**SIGNATURES, **DIAG_SIGNATURES}.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def status_string(status: int) -> str:
    return lib().w8a8_status_string(status).decode()


def check(status: int, what: str = "") -> None:
    if status != OK:
        raise W8A8Error(status, what)
