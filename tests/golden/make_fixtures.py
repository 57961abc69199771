"""Write the committed operator fixtures under tests/golden/operator/.

The cases follow the recipe of the reference's CPU-integer operator fixture
generator (bitemyapp/inferrous, crates/inferrous-qwen3/tools/operator_fixtures.py):

* quantize (tools/operator_fixtures.py:36-45): three rows per width in
  {128, 4096, 12288}; row 0 all zero (scale floor 1e-8); row 1 starts with
  [127, -127, .5, -.5, 1.5, -1.5, 2.5, -2.5] (rounding ties, exact scale 1.0
  when that row's absmax is 127); expected ``scale = max(|x|, 1e-8) / 127``,
  ``q = clamp(round_half_even(x / scale), -127, 127)``.
* linear (tools/operator_fixtures.py:47-55): (width, rows) in
  {(4096,1), (4096,17), (12288,3), (4096,65), (12288,129)}, 33 output
  channels, q and w uniform int8 in [-127, 127], row 0 of q all 127 and
  weight rows 0/1 all +127/-127 (worst accumulator +-198,193,152 at 12288),
  ``asc ~ U[0, 1/64)``, ``ws ~ U[0, 1/64)``,
  expected ``out = bf16((q @ w.T).float() * asc * ws)``.
* swiglu (tools/operator_fixtures.py:75-76): gate = bf16(linspace(-80, 80,
  12288)), up = bf16(randn(12288)), expected ``out = bf16(silu(gate) * up)``
  in torch's float32 (compared within the reference's tolerance,
  src/conformance.rs:663).  The reference draws its rope/attention inputs
  before this case; those draws are not repeated, so ``up`` differs from the
  reference's own file while following the same recipe.
* norm (tools/operator_fixtures.py:36-40) at width 4096, the width of
  `norm_quantize` (src/kernels.rs:476-575): x = bf16(randn(3, 4096)) with
  row 0 zero, gain = bf16(randn(4096)), expected
  ``out = bf16(x * rsqrt(mean(x^2) + 1e-6) * gain)`` in torch's float32
  (compared within the reference's tolerance).  Drawn from its own
  generator (seed 825) after the other cases, so the earlier files keep
  their bytes.
* head (tools/operator_fixtures.py:78-79): x = bf16(randn(3, 4096)),
  w = BF16 randn(33, 4096) (stored as BF16 bits), expected
  ``out = bf16(x[-1:] @ w.T)`` in torch's float32 (compared within the
  reference's tolerance).  Own generator (seed 826), drawn last.
* weight_quantize (tools/prepare.py:79-83, offline weight quantization):
  BF16 weights [33, 4096] (row 0 zero, row 1 with +-127 and .5 ties) as BF16
  bits, expected ``scale = amax(|w|, 1).clamp(min=1e-8) / 127`` and
  ``q = round(w / scale).clamp(-127, 127)`` per output channel.

Expected values are computed here with torch on the CPU -- an implementation
independent of the C oracle in oracle/ -- and stored with the inputs.  The
i32 accumulators are stored too ("acc"), since the reference never
materialises them.  Draw order matches the reference script (including the
RMSNorm gain draws, which are not stored), seed 824.

The output directory is refused if it exists, as in the reference; the
manifest format is the reference's ({generator, torch, seed, cases: [{name,
op, tensors: {key: {file, shape, sha256}}, width}]}).

Run: python tests/golden/make_fixtures.py tests/golden/operator
"""
from __future__ import annotations

import argparse
import hashlib
import json
from pathlib import Path

import torch


def to_bf16_values(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).to(torch.float32)


class Writer:
    def __init__(self, root: Path):
        self.root = root
        self.cases: list[dict] = []

    def add(self, op: str, tensors: dict[str, torch.Tensor], **params) -> None:
        name = f"{len(self.cases):02d}-{op}"
        meta = {}
        for key, value in tensors.items():
            arr = value.contiguous().numpy()
            raw = arr.tobytes()
            fname = f"{name}-{key}.bin"
            (self.root / fname).write_bytes(raw)
            meta[key] = {"file": fname, "shape": list(arr.shape),
                         "dtype": str(arr.dtype),
                         "sha256": hashlib.sha256(raw).hexdigest()}
        self.cases.append({"name": name, "op": op, "tensors": meta, **params})


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("output", type=Path)
    args = ap.parse_args()
    args.output.mkdir(parents=True, exist_ok=False)
    torch.manual_seed(824)
    out = Writer(args.output)

    ties = torch.tensor([127.0, -127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5])
    for width in (128, 4096, 12288):
        x = to_bf16_values(torch.randn(3, width))
        x[0] = 0
        _gain = torch.randn(width)  # consumed to keep the reference draw order
        x[1, :8] = ties
        scale = x.abs().amax(-1, keepdim=True).clamp(min=1e-8) / 127
        q = torch.round(x / scale).clamp(-127, 127).to(torch.int8)
        out.add("quantize", {"x": x, "q": q, "scale": scale}, width=width)

    for width, rows in ((4096, 1), (4096, 17), (12288, 3), (4096, 65), (12288, 129)):
        q = torch.randint(-127, 128, (rows, width), dtype=torch.int8)
        w = torch.randint(-127, 128, (33, width), dtype=torch.int8)
        q[0] = 127
        w[0] = 127
        w[1] = -127
        asc = torch.rand(rows, 1) / 64
        ws = torch.rand(33) / 64
        acc = q.to(torch.int32) @ w.to(torch.int32).T
        res = to_bf16_values(acc.to(torch.float32) * asc * ws)
        out.add("linear", {"q": q, "asc": asc, "w": w, "ws": ws, "acc": acc,
                           "out": res}, width=width)

    gate = to_bf16_values(torch.linspace(-80, 80, 12288))
    up = to_bf16_values(torch.randn(12288))
    act = to_bf16_values(torch.nn.functional.silu(gate) * up)
    out.add("swiglu", {"gate": gate, "up": up, "out": act})

    w = torch.randn(33, 4096).bfloat16()
    w[0] = 0
    w[1, :8] = ties.bfloat16()
    wf = w.float()
    wscale = wf.abs().amax(1, keepdim=True).clamp(min=1e-8) / 127.0
    wq = torch.round(wf / wscale).clamp(-127, 127).to(torch.int8)
    out.add("weight_quantize", {"w": w.view(torch.int16), "q": wq, "scale": wscale.flatten()})

    gen = torch.Generator().manual_seed(825)
    x = to_bf16_values(torch.randn(3, 4096, generator=gen))
    x[0] = 0
    gain = to_bf16_values(torch.randn(4096, generator=gen))
    normed = to_bf16_values(x * torch.rsqrt(x.square().mean(-1, keepdim=True) + 1e-6) * gain)
    out.add("norm", {"x": x, "gain": gain, "out": normed}, width=4096)

    gen = torch.Generator().manual_seed(826)
    x = to_bf16_values(torch.randn(3, 4096, generator=gen))
    w = torch.randn(33, 4096, generator=gen).bfloat16()
    logits = to_bf16_values(x[-1:] @ w.float().T)
    out.add("head", {"x": x, "w": w.view(torch.int16), "out": logits.flatten()})

    manifest = {"generator": "tests/golden/make_fixtures.py", "torch": torch.__version__,
                "seed": 824, "cases": out.cases}
    (args.output / "manifest.json").write_text(json.dumps(manifest, indent=2) + "\n")


if __name__ == "__main__":
    main()
