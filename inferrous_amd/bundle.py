"""Reader (and writer) of the reference's exported model bundle, for the
W8A8 projection weights this library consumes.

Format (crates/inferrous-qwen3/src/model.rs:7-22, tools/prepare.py:47-53,
:79-86, :109-111): a directory with ``manifest.json``

    {"format_version": 1, "profile": ..., "model_revision": ...,
     "max_context": 4096, "config": {...HF config...},
     "tokenizer_sha256": ..., "tensors": {name: {"shape", "dtype", "sha256"}}}

and one raw little-endian ``{name}.bin`` per tensor.  The projections of
layer ``l`` are ``layer.{l}.{p}.w`` (int8 ``[n, k]``, K contiguous, never
-128) and ``layer.{l}.{p}.scale`` (f32 ``[n]``, finite, > 0) for p in q, k,
v, o, gate, up, down.

Validation follows ``Model::load`` (src/model.rs:46-147): manifest identity
and model configuration, then per tensor the declared dtype and shape, the
file size and its SHA-256, and the value invariants of quantized weights and
scales.  Only the W8A8 projections are read here; norm gains, embedding,
head, rope table and tokenizer belong to the rest of the engine.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np

from .runtime import CudaStream, DeviceBuffer

PROFILE = "qwen3-8b-int8-channel-token-bf16-softmax-v1"       # src/lib.rs:15
MODEL_REVISION = "b968826d9c46dd6066d109eabc6255188de91218"   # src/lib.rs:14
CONTEXT = 4096                                                # src/lib.rs:18
LAYERS = 36
# (name, n, k) -- src/model.rs:127-135
PROJECTIONS = (("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
               ("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288))
# src/model.rs:57-78
CONFIG_INTS = (("hidden_size", 4096), ("intermediate_size", 12288), ("num_hidden_layers", 36),
               ("num_attention_heads", 32), ("num_key_value_heads", 8), ("head_dim", 128),
               ("vocab_size", 151936))
_DTYPES = {"|i1": np.int8, "<u2": np.uint16, "<f4": np.float32}


class BundleError(ValueError):
    """A bundle that the reference loader would reject."""


def _sha(data: bytes) -> str:
    return hashlib.sha256(data).hexdigest()


def model_config() -> dict:
    """The model configuration the reference accepts (src/model.rs:57-78)."""
    cfg = {k: v for k, v in CONFIG_INTS}
    cfg.update(rms_norm_eps=1e-6, rope_theta=1_000_000, rope_scaling=None, attention_bias=False,
               use_sliding_window=False, tie_word_embeddings=False, hidden_act="silu")
    return cfg


class Bundle:
    def __init__(self, root: Path, manifest: dict):
        self.root = Path(root)
        self.manifest = manifest

    @classmethod
    def open(cls, root, check_model: bool = True) -> "Bundle":
        """Read and validate ``manifest.json`` (src/model.rs:47-78)."""
        root = Path(root)
        try:
            m = json.loads((root / "manifest.json").read_bytes())
        except (OSError, ValueError) as e:
            raise BundleError(f"manifest: {e}") from None
        if not isinstance(m, dict) or not isinstance(m.get("tensors"), dict):
            raise BundleError("manifest: missing tensor table")
        if check_model:
            if (m.get("format_version") != 1 or m.get("profile") != PROFILE
                    or m.get("model_revision") != MODEL_REVISION or m.get("max_context") != CONTEXT):
                raise BundleError("unsupported clean model profile")
            cfg = m.get("config") if isinstance(m.get("config"), dict) else {}

            def is_uint(v, n):  # serde_json as_u64() == Some(n): an integer literal
                return isinstance(v, int) and not isinstance(v, bool) and v == n

            for key, n in CONFIG_INTS:
                if not is_uint(cfg.get(key), n):
                    raise BundleError(f"unsupported {key}")
            eps = cfg.get("rms_norm_eps")
            if not (isinstance(eps, (int, float)) and not isinstance(eps, bool) and eps == 1e-6
                    and is_uint(cfg.get("rope_theta"), 1_000_000)
                    and cfg.get("rope_scaling") is None
                    and cfg.get("attention_bias") is False and cfg.get("use_sliding_window") is False
                    and cfg.get("tie_word_embeddings") is False and cfg.get("hidden_act") == "silu"):
                raise BundleError("unsupported model operators")
        return cls(root, m)

    def read(self, name: str, dtype: str, shape) -> np.ndarray:
        """One tensor, checked as src/model.rs:79-100: declared dtype and shape,
        file size, SHA-256."""
        t = self.manifest["tensors"].get(name)
        if t is None:
            raise BundleError(f"missing {name}")
        if t.get("dtype") != dtype or list(t.get("shape", [])) != list(shape):
            raise BundleError(f"{name}: wrong type or shape")
        try:
            raw = (self.root / f"{name}.bin").read_bytes()
        except OSError as e:
            raise BundleError(f"{name}: {e}") from None
        np_dtype = _DTYPES[dtype]
        if len(raw) != int(np.prod(shape)) * np.dtype(np_dtype).itemsize or _sha(raw) != t.get("sha256"):
            raise BundleError(f"{name}: size or hash mismatch")
        return np.frombuffer(raw, dtype=np.dtype(np_dtype).newbyteorder("<")).reshape(shape).copy()

    def matrix(self, layer: int, name: str):
        """(w int8 [n, k], scale f32 [n]) of one projection, with the
        invariants of src/model.rs:137-146: no -128 code, finite scales > 0."""
        shapes = {p: (n, k) for p, n, k in PROJECTIONS}
        if name not in shapes or not 0 <= layer < LAYERS:
            raise BundleError(f"no projection layer.{layer}.{name}")
        n, k = shapes[name]
        w = self.read(f"layer.{layer}.{name}.w", "|i1", [n, k])
        if (w == -128).any():
            raise BundleError("invalid quantized weight")
        scale = self.read(f"layer.{layer}.{name}.scale", "<f4", [n])
        if not np.isfinite(scale).all():
            raise BundleError(f"layer.{layer}.{name}.scale: nonfinite float")
        if not (scale > 0).all():
            raise BundleError("invalid weight scale")
        return w, scale

    def upload(self, stream: CudaStream, layer: int, name: str):
        """Device copies (w, scale) of one projection, ready for ``linear``."""
        w, scale = self.matrix(layer, name)
        return (DeviceBuffer.from_host(stream, w.reshape(-1)),
                DeviceBuffer.from_host(stream, scale))


def write_bundle(root, tensors: dict, config: dict | None = None, *, profile: str = PROFILE,
                 model_revision: str = MODEL_REVISION, tokenizer_sha256: str = "") -> None:
    """Write tensors in the bundle format (tools/prepare.py:47-53, :109-111):
    ``{name}.bin`` raw little-endian plus ``manifest.json``.  Accepts int8,
    uint16 (BF16 bits) and float32 arrays."""
    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    codes = {np.dtype(np.int8): "|i1", np.dtype(np.uint16): "<u2", np.dtype(np.float32): "<f4"}
    table = {}
    for name, value in tensors.items():
        a = np.ascontiguousarray(value)
        if a.dtype not in codes:
            raise TypeError(f"{name}: unsupported dtype {a.dtype}")
        code = codes[a.dtype]
        raw = a.astype(np.dtype(_DTYPES[code]).newbyteorder("<"), copy=False).tobytes()
        (root / f"{name}.bin").write_bytes(raw)
        table[name] = {"shape": list(a.shape), "dtype": code, "sha256": _sha(raw)}
    manifest = {"format_version": 1, "profile": profile, "model_revision": model_revision,
                "max_context": CONTEXT, "config": model_config() if config is None else config,
                "tensors": table, "tokenizer_sha256": tokenizer_sha256}
    (root / "manifest.json").write_text(json.dumps(manifest, indent=1))
