"""animaxs_amd: MI355X-native (gfx950) attention + quantized-linear hot path of AnimaXS.

The product is ``libanima_hip.so`` (C ABI in ``include/anima_hip.h``, HIP kernels in
``csrc/``).  This package builds it in-tree (``animaxs_amd.build``) and mirrors the
reference's Swift operator surface in Python over that ABI (``executors``).
"""

from ._abi import AnimaError, LIB_PATH, load  # noqa: F401
from .animapk import AnimapkExecutionRange, AnimapkFile, AnimapkTensor, DiTBlockLocator  # noqa: F401
from .executors import (  # noqa: F401
    AttentionExecutor, BlockOps, Context, CrossKVCache, DiTBlockExecutor, DiTFinalLayerExecutor,
    DiTPreparationExecutor, DitRoPE, EulerSampler, LatentOps, LinearExecutor, QKPrologue, QuantDecoders,
    NumericalMonitor, ProbeFlag, ProbeStats, QuantizedLinearWeightBuffers, QwenLayerExecutor, WeightStreamer,
    as_buffer, qwen_rope, read_probe, read_probe_sink_bytes,
)

__all__ = [
    "AnimaError", "LIB_PATH", "load", "AttentionExecutor", "BlockOps", "Context", "CrossKVCache",
    "DiTBlockExecutor", "WeightStreamer", "DiTPreparationExecutor", "DiTFinalLayerExecutor", "EulerSampler",
    "LatentOps", "AnimapkFile", "AnimapkTensor", "AnimapkExecutionRange", "DiTBlockLocator",
    "DitRoPE", "LinearExecutor", "QKPrologue", "QuantDecoders", "QuantizedLinearWeightBuffers",
    "QwenLayerExecutor", "as_buffer", "qwen_rope", "read_probe", "read_probe_sink_bytes", "NumericalMonitor",
    "ProbeStats", "ProbeFlag",
]
