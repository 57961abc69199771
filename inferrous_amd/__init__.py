"""inferrous_amd -- MI355X (gfx950) W8A8 linear-layer path.

A drop-in for the W8A8 linear-layer operators of bitemyapp/inferrous
(crates/inferrous-qwen3/src/kernels.rs): dynamic per-token INT8 activation
quantization, the M=1 v_dot4 decode GEMV, the INT8 MFMA GEMM for prefill and
small batches, the fused per-token x per-channel dequant epilogue to BF16,
and greedy selection over the lm_head logits (W8A8, or the reference's
losslessly packed BF16 head).

The compute lives in ``libinferrous_w8a8.so`` (hand-written HIP for gfx950,
C ABI in ``include/inferrous_w8a8.h``).  This package is the host-side mirror
of the reference's operator interface over that ABI; it has no fallback
path -- without the built library every op raises.
"""
from ._lib import (EALIGN, EARG, EINIT, ENODEV, ENULL, ESHAPE, EWORKSPACE, OK, OUT_BF16,
                   OUT_F32, OUT_I32, PATH_AUTO, PATH_DOT4, PATH_MFMA, LIB_PATH, W8A8Error)
from .module import LoadedModule, load
from .packing import PackedBf16
from .runtime import (CudaContext, CudaStream, DeviceBuffer, Event, Graph, LaunchConfig,
                      PinnedHostBuffer, cfg, device_count, rows)

__all__ = [
    "CudaContext", "CudaStream", "DeviceBuffer", "Event", "Graph", "LaunchConfig",
    "LoadedModule", "PackedBf16", "PinnedHostBuffer", "W8A8Error", "cfg", "device_count", "load", "rows",
    "LIB_PATH", "OK", "ENULL", "ESHAPE", "EALIGN", "EINIT", "EWORKSPACE", "EARG", "ENODEV",
    "OUT_F32", "OUT_BF16", "OUT_I32", "PATH_AUTO", "PATH_DOT4", "PATH_MFMA",
]
