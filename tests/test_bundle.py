"""Bundle reader: the reference's exported-model format (src/model.rs:7-147,
tools/prepare.py:47-53, :79-86, :109-111) for the W8A8 projections.  CPU tests
cover the format and every rejection rule of the reference loader; the GPU
test runs a projection read from a bundle through ``linear``."""
from __future__ import annotations

import json

import numpy as np
import pytest

import oracle
from inferrous_amd import bundle as B


def make_layer0(root, names=("k", "v"), seed=3):
    rng = np.random.default_rng(seed)
    shapes = {p: (n, k) for p, n, k in B.PROJECTIONS}
    tensors = {}
    for name in names:
        n, k = shapes[name]
        tensors[f"layer.0.{name}.w"] = rng.integers(-127, 128, (n, k), dtype=np.int8)
        tensors[f"layer.0.{name}.scale"] = (rng.random(n) / 64 + 1e-4).astype(np.float32)
    B.write_bundle(root, tensors)
    return tensors


def test_roundtrip_and_layout(tmp_path):
    t = make_layer0(tmp_path)
    b = B.Bundle.open(tmp_path)
    w, s = b.matrix(0, "k")
    assert w.shape == (1024, 4096) and w.dtype == np.int8
    assert np.array_equal(w, t["layer.0.k.w"]) and np.array_equal(s, t["layer.0.k.scale"])
    # raw little-endian files, K contiguous (src/model.rs:137-141)
    raw = (tmp_path / "layer.0.v.w.bin").read_bytes()
    assert raw == t["layer.0.v.w"].tobytes() and len(raw) == 1024 * 4096
    m = json.loads((tmp_path / "manifest.json").read_text())
    assert m["tensors"]["layer.0.v.scale"]["dtype"] == "<f4"
    assert m["tensors"]["layer.0.v.w"]["shape"] == [1024, 4096]


def edit_manifest(root, fn):
    m = json.loads((root / "manifest.json").read_text())
    fn(m)
    (root / "manifest.json").write_text(json.dumps(m))


@pytest.mark.parametrize("field,value", [("format_version", 2), ("profile", "other"),
                                         ("model_revision", "0" * 40), ("max_context", 8192)])
def test_rejects_other_profiles(tmp_path, field, value):
    make_layer0(tmp_path, names=("k",))
    edit_manifest(tmp_path, lambda m: m.__setitem__(field, value))
    with pytest.raises(B.BundleError, match="profile"):
        B.Bundle.open(tmp_path)
    B.Bundle.open(tmp_path, check_model=False)   # the tensor layer stays usable


@pytest.mark.parametrize("key,value", [("hidden_size", 5120), ("num_hidden_layers", 36.0),
                                       ("vocab_size", True), ("hidden_act", "gelu"),
                                       ("rope_theta", 10000), ("tie_word_embeddings", True),
                                       ("rms_norm_eps", 1e-5)])
def test_rejects_other_configs(tmp_path, key, value):
    make_layer0(tmp_path, names=("k",))
    edit_manifest(tmp_path, lambda m: m["config"].__setitem__(key, value))
    with pytest.raises(B.BundleError, match="unsupported"):
        B.Bundle.open(tmp_path)


def test_rejects_damaged_tensors(tmp_path):
    make_layer0(tmp_path, names=("k", "v"))
    b = B.Bundle.open(tmp_path)
    # hash mismatch
    raw = bytearray((tmp_path / "layer.0.k.w.bin").read_bytes())
    raw[12345] ^= 1
    (tmp_path / "layer.0.k.w.bin").write_bytes(bytes(raw))
    with pytest.raises(B.BundleError, match="hash"):
        b.matrix(0, "k")
    # declared shape differs from the model's
    edit_manifest(tmp_path, lambda m: m["tensors"]["layer.0.v.w"].__setitem__("shape", [4096, 1024]))
    with pytest.raises(B.BundleError, match="wrong type or shape"):
        B.Bundle.open(tmp_path).matrix(0, "v")
    with pytest.raises(B.BundleError, match="missing"):
        b.matrix(0, "q")


@pytest.mark.parametrize("defect", ["minus128", "zero_scale", "nan_scale"])
def test_rejects_invalid_values(tmp_path, defect):
    rng = np.random.default_rng(9)
    w = rng.integers(-127, 128, (1024, 4096), dtype=np.int8)
    s = np.full(1024, 0.01, np.float32)
    if defect == "minus128":
        w[5, 7] = -128
    elif defect == "zero_scale":
        s[3] = 0
    else:
        s[3] = np.nan
    B.write_bundle(tmp_path, {"layer.0.k.w": w, "layer.0.k.scale": s})
    with pytest.raises(B.BundleError):
        B.Bundle.open(tmp_path).matrix(0, "k")


@pytest.mark.gpu
def test_bundle_projection_through_linear(tmp_path):
    from inferrous_amd import CudaContext, DeviceBuffer, load
    t = make_layer0(tmp_path, names=("k",))
    ctx = CudaContext(0)
    s = ctx.new_stream()
    mod = load(ctx)
    w, ws = B.Bundle.open(tmp_path).upload(s, 0, "k")
    rng = np.random.default_rng(4)
    x = oracle.bf16_rne(rng.standard_normal(2 * 4096).astype(np.float32))
    q = DeviceBuffer.zeroed(s, x.size, np.int8)
    sc = DeviceBuffer.zeroed(s, 2, np.float32)
    mod.quantize(s, None, DeviceBuffer.from_host(s, x), 4096, q, sc)
    out = DeviceBuffer.zeroed(s, 2 * 1024, np.float32)
    mod.linear(s, None, q, sc, w, ws, 4096, out)
    oq, osc = oracle.quantize(x, 4096)
    _, want, _ = oracle.linear(oq, osc, t["layer.0.k.w"], t["layer.0.k.scale"], 4096)
    assert np.array_equal(out.to_host_vec(s).view(np.uint32), want.view(np.uint32))
