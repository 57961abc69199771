"""Shared pytest configuration.

Markers:
  gpu -- needs an MI355X (gfx950) and the built HIP library; run with -m gpu.

Everything else runs on the CPU: oracle pinning against golden vectors and
closed forms, C-ABI load/export checks and host-side argument validation.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: requires an MI355X GPU and the built HIP library")


class Fixtures:
    """Reader for the reference-format operator fixture manifest."""

    def __init__(self, root: Path):
        self.root = root
        self.manifest = json.loads((root / "manifest.json").read_text())

    def cases(self, op: str):
        return [c for c in self.manifest["cases"] if c["op"] == op]

    def tensor(self, case: dict, key: str) -> np.ndarray:
        meta = case["tensors"][key]
        raw = (self.root / meta["file"]).read_bytes()
        assert hashlib.sha256(raw).hexdigest() == meta["sha256"], f"fixture hash: {key}"
        return np.frombuffer(raw, dtype=np.dtype(meta["dtype"])).reshape(meta["shape"]).copy()


@pytest.fixture(scope="session")
def fixtures() -> Fixtures:
    return Fixtures(GOLDEN / "operator")


def rounding_probe_inputs() -> np.ndarray:
    """The deterministic input set of src/conformance.rs:841-856 (1,328,443 f32):
    every BF16 encoding, a dense signed grid in 1/1024 steps over [-128, 128],
    the +-1-ulp neighbours of every half-integer tie in (-127, 127), and one
    million hashed f32 bit patterns (x * 2654435761 mod 2^32)."""
    parts = [(np.arange(65536, dtype=np.uint32) << 16).view(np.float32)]
    parts.append((np.arange(-131072, 131073, dtype=np.float64) / 1024.0).astype(np.float32))
    ties = []
    for i in range(-127, 127):
        b = int(np.float32(i + 0.5).view(np.uint32))
        ties += [b - 1, b, b + 1]
    parts.append(np.array(ties, dtype=np.uint32).view(np.float32))
    x = np.arange(1_000_000, dtype=np.uint64)
    parts.append(((x * 2654435761) & 0xFFFFFFFF).astype(np.uint32).view(np.float32))
    return np.concatenate(parts)


def rounding_expected(x: np.ndarray) -> np.ndarray:
    """Closed form of src/conformance.rs:857-860: f64 clamp to [-127, 127],
    round half to even, NaN -> 0 (Rust's saturating `as i8`)."""
    d = x.astype(np.float64)
    nan = np.isnan(d)
    d = np.clip(np.where(nan, 0.0, d), -127.0, 127.0)
    return np.rint(d).astype(np.int8)


def argmax_cases() -> list[np.ndarray]:
    """src/conformance.rs:684-698: six hand cases plus, for each length in
    {31, 32, 33, 1023, 1024, 1025, 151936}, i % 97 with f32::MAX at the end,
    then additionally at index 7 (repeated maximum, lowest index wins)."""
    f = np.float32
    big = np.finfo(np.float32).max
    cases = [np.array(v, dtype=f) for v in (
        [0.0, -0.0], [-0.0, 0.0], [np.finfo(np.float32).min], [np.nan],
        [0.0, np.inf], [-np.inf, 0.0])]
    for n in (31, 32, 33, 1023, 1024, 1025, 151936):
        x = (np.arange(n) % 97).astype(f)
        x[n - 1] = big
        cases.append(x.copy())
        x[7] = big
        cases.append(x)
    return cases


def argmax_expected(x: np.ndarray) -> int:
    """src/model.rs:206-218 `argmax`, Err mapped to the GPU sentinel u32::MAX
    (src/conformance.rs:707): strict '>' ascending scan."""
    if x.size == 0 or not np.all(np.isfinite(x)):
        return 0xFFFFFFFF
    best = 0
    for i in range(1, x.size):
        if x[i] > x[best]:
            best = i
    return best


def reference_tolerance_ok(got, want) -> bool:
    """The reference's tolerance for non-exact operators
    (src/conformance.rs:660-673): every element finite with
    |a-b| <= 2e-4 + 0.01|b|, and relative L2 error <= 0.005."""
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    elem = bool(np.isfinite(got).all()) and bool(
        np.all(np.abs(got - want) <= 2e-4 + 0.01 * np.abs(want)))
    l2 = np.sqrt(np.sum((got - want) ** 2) / max(float(np.sum(want ** 2)), 1e-20))
    return elem and l2 <= 0.005


def bf16_ulp_distance(a, b) -> np.ndarray:
    """|a - b| in BF16 ulps for BF16-valued f32 arrays of the same sign."""
    ia = (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.int64)
    ib = (np.ascontiguousarray(b, np.float32).view(np.uint32) >> 16).astype(np.int64)
    return np.abs(ia - ib)


def seeded_linear_shapes(count: int = 48, seed: int = 20261202) -> list[tuple[int, int, int]]:
    """Seeded (m, n, k) for the linear sweeps (GPU parity and the indexing
    replay), three kinds in turn, at most 64 Mi weights and 2e9
    multiply-adds each:
      - m log-uniform in [1, 700], n in [1, 30000] (log-uniform);
      - the same with n in [2000, 30000] (the wide tiles);
      - m in [17, 256], n in [2000, 30000], k a multiple of 1024 (the
        one-M-tile plans and their split-K routes).
    Outside the third kind k is a multiple of 1024 (40%: the narrow
    plans), of 128 (30%: the DMA routes) or of 16 (30%: the guarded
    tiles), up to 12800."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        kind = len(out) % 3
        if kind == 2:
            m = int(np.exp(rng.uniform(np.log(17.0), np.log(257.0))))
            k = 1024 * int(rng.integers(1, 13))
        else:
            m = int(np.exp(rng.uniform(0.0, np.log(700.0))))
            u = rng.random()
            k = (1024 * int(rng.integers(1, 13)) if u < 0.4 else 128 * int(rng.integers(1, 101)) if u < 0.7
                 else 16 * int(rng.integers(1, 801)))
        n = int(np.exp(rng.uniform(np.log(2000.0) if kind else 0.0, np.log(30000.0))))
        if n * k <= 64 << 20 and m * n * k <= 2_000_000_000:
            out.append((m, n, k))
    return out
