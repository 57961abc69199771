"""Lossless packed storage for the BF16 lm_head: the mirror of
``PackedBf16`` (crates/inferrous-qwen3/src/packing.rs:3-46).

The coding runs in the HIP library's host packer (``w8a8_bf16_pack``): BF16
values in 256-value chunks, 12 bits per value whose exponent lies in
[109, 124), the rest escaped to a per-chunk exception list.  It does not
quantize: every BF16 bit pattern round-trips.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from ._lib import check, lib


@dataclass
class PackedBf16:
    words: np.ndarray       # u32 [n / 8 * 3]
    offsets: np.ndarray     # u32 [n / 256], start of each chunk's exceptions
    exceptions: np.ndarray  # u16, at least one entry

    @staticmethod
    def new(values) -> "PackedBf16":
        """``PackedBf16::new`` (src/packing.rs:10-46): values are BF16 bits,
        a multiple of 256 of them."""
        v = np.ascontiguousarray(values, dtype=np.uint16).reshape(-1)
        if v.size % 256:
            raise ValueError("packed BF16 rows must be a multiple of 256 values")
        words = np.zeros(v.size // 8 * 3, np.uint32)
        offsets = np.zeros(v.size // 256, np.uint32)
        exceptions = np.zeros(max(v.size, 1), np.uint16)
        n = ctypes.c_size_t()
        check(lib().w8a8_bf16_pack(v.ctypes.data, v.size, words.ctypes.data, offsets.ctypes.data,
                                   exceptions.ctypes.data, exceptions.size, ctypes.byref(n)),
              "bf16 pack")
        return PackedBf16(words, offsets, exceptions[:n.value].copy())
