"""Seeded synthetic inputs for the benchmark configurations.

Weights and weight scales are generated on the device by the library
(``LoadedModule.synth_i8`` / ``synth_f32``; a pure function of
(seed, stream id, index)).  Activations are small and generated here on the
host with numpy's PCG64, rounded to BF16 (round-to-nearest-even) and held as
the f32 buffers the reference's quantizers read:

* ``normal_rows``      -- BF16 N(0, 1), configs 1-3 and 5;
* ``student_t_rows``   -- Student-t(df=3) as Z / sqrt(chi2_3 / 3) with 8
  seeded outlier channels scaled x50 (config 4).

Stream ids of the decode weight set: ``weight_stream(layer, shape)``.
"""
from __future__ import annotations

import numpy as np

HIDDEN = 4096
INTER = 12288
VOCAB = 151936
LAYERS = 36

# Qwen3-8B decoder projections as (name, n, k); qkv and gate_up are the
# concatenated siblings (per-channel results are independent of grouping).
DECODE_SHAPES = (("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 24576, 4096),
                 ("down", 4096, 12288))
LM_HEAD = ("lm_head", VOCAB, HIDDEN)


def weight_stream(layer: int, shape_index: int) -> int:
    return 1000 * (layer + 1) + shape_index


def scale_stream(layer: int, shape_index: int) -> int:
    return 1000 * (layer + 1) + 100 + shape_index


def bf16_round(x: np.ndarray) -> np.ndarray:
    """f32 -> BF16 RNE kept in f32 (same bit formula as the device epilogue)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000) & 0xFFFFFFFF
    return u.astype(np.uint32).view(np.float32)


def normal_rows(seed: int, m: int, k: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return bf16_round(rng.standard_normal((m, k), dtype=np.float32))


def student_t_rows(seed: int, m: int, k: int, outliers: int = 8, factor: float = 50.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    z = rng.standard_normal((m, k))
    chi = rng.chisquare(3, size=(m, k))
    t = z / np.sqrt(chi / 3.0)
    cols = rng.choice(k, size=outliers, replace=False)
    t[:, cols] *= factor
    return bf16_round(t.astype(np.float32))


def ragged_rows(seeds, k: int) -> np.ndarray:
    """One independent N(0,1) row per sequence seed (config 5)."""
    return np.concatenate([normal_rows(int(s), 1, k) for s in seeds], axis=0)
