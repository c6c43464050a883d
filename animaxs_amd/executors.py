"""Python mirror of the reference operator surface over the C ABI.

Same names and argument meaning as the Swift executors so callers (and the
tests) read like the reference's own:

  * ``AttentionExecutor``  AnimaXS/Runtime/Metal/AttentionExecutor.swift:77-848
  * ``LinearExecutor`` / ``QuantizedLinearWeightBuffers``
                           AnimaXS/Runtime/Metal/LinearExecutor.swift:18-459
  * ``QuantDecoders``      AnimaXS/Runtime/Animapk/QuantDecoders.swift:17-164
  * ``DitRoPE`` / ``qwen_rope``  Runtime/Text/DitRoPE.swift:58-107,
                           Runtime/Metal/QwenEncoderMetal.swift:126-143
  * ``DiTBlockExecutor``   AnimaXS/Runtime/Metal/DiTBlockExecutor.swift:155-282
  * ``DiTPreparationExecutor`` / ``DiTFinalLayerExecutor``
                           Runtime/Metal/DiTPreparationExecutor.swift:51-135,
                           Runtime/Metal/DiTFinalLayerExecutor.swift:75-186
  * ``EulerSampler`` / ``LatentOps``  Runtime/Sampler/EulerSampler.swift:6-90,
                           Shaders/AnimaKernels.metal:1191-1297

A "buffer" is anything with ``data_ptr()`` plus ``numel()``/``element_size()``
(a device tensor), an ``(address, length)`` tuple, or an ``_abi.Buffer``.  The
executors never allocate device memory for the caller; they never compute on
the CPU (QuantDecoders and the RoPE builders are CPU functions by definition in
the reference as well).
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Any, Optional

import numpy as np

from . import _abi
from ._abi import AnimaError, call

__all__ = [
    "AnimaError", "Context", "AttentionExecutor", "LinearExecutor", "QuantizedLinearWeightBuffers",
    "QKPrologue", "QuantDecoders", "DitRoPE", "qwen_rope", "DiTBlockExecutor", "BlockOps", "as_buffer",
    "CrossKVCache", "WeightStreamer", "QwenLayerExecutor", "LatentOps", "EulerSampler", "DiTPreparationExecutor",
    "DiTFinalLayerExecutor", "NumericalMonitor", "ProbeStats", "ProbeFlag",
]


def as_buffer(x: Any) -> _abi.Buffer:
    """A device buffer for the C ABI.  Tensors must be contiguous and on the GPU: the
    length is ``numel * element_size`` from ``data_ptr``, which is the tensor's real
    extent only for a contiguous layout (an expanded or strided view would claim bytes
    it does not own), and a host pointer must never reach a kernel."""
    if x is None:
        return _abi.Buffer(None, 0)
    if isinstance(x, _abi.Buffer):
        return x
    if isinstance(x, tuple):
        return _abi.Buffer(C.c_void_p(int(x[0])), int(x[1]))
    if hasattr(x, "data_ptr"):
        if getattr(x, "is_cuda", False) is not True:
            raise TypeError("device buffers must be GPU tensors (got a host tensor)")
        if not x.is_contiguous():
            raise TypeError("device buffers must be contiguous tensors (got a strided or expanded view)")
        return _abi.Buffer(C.c_void_p(x.data_ptr()), int(x.numel() * x.element_size()))
    raise TypeError(f"cannot use {type(x)!r} as a device buffer")


def _ptr(x: Any) -> Optional[int]:
    if x is None:
        return None
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    return int(x)


class Context:
    """MetalContext analog: a HIP device and the stream all encodes append to."""

    def __init__(self, device: int = 0, stream: Any = None):
        h = C.c_void_p()
        call("anima_ctx_create", int(device), C.byref(h))
        self._h = h
        self.device = device
        if stream is not None:
            self.set_stream(stream)

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def set_stream(self, stream: Any) -> None:
        """``stream`` is a raw hipStream_t address or an object with ``cuda_stream``."""
        raw = getattr(stream, "cuda_stream", stream)
        call("anima_ctx_set_stream", self._h, C.c_void_p(int(raw) if raw else None))

    def synchronize(self) -> None:
        call("anima_ctx_synchronize", self._h)

    def close(self) -> None:
        if self._h:
            call("anima_ctx_destroy", self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_NUMERICS = {"legacy": _abi.NUMERICS_LEGACY, "fp32ScoresAndSoftmax": _abi.NUMERICS_FP32_SCORES,
             "fp32": _abi.NUMERICS_FP32_SCORES, "bf16_compute": _abi.NUMERICS_BF16_COMPUTE}
_BACKENDS = {"auto": _abi.ATTN_AUTO, "flash": _abi.ATTN_FLASH, "generic": _abi.ATTN_GENERIC,
             "legacyMPS": _abi.ATTN_LEGACY_MPS, "legacyHeadMajorMPS": _abi.ATTN_LEGACY_MPS,
             "stridedTokenMajorMPS": _abi.ATTN_LEGACY_MPS, "metalFlash": _abi.ATTN_FLASH}


@dataclass
class QKPrologue:
    """Fused per-head RMSNorm (+ split-half RoPE) applied to Q and K.  ``k_rope`` is an
    optional separate table for the keys (the LLM adapter's cross attention rotates its
    context keys with the context positions, LLMAdapterMetal.swift:336-340)."""
    q_norm_weight: Any = None
    k_norm_weight: Any = None
    eps: float = 1e-6
    rope: Any = None
    rope_tokens: int = 0
    rope_q: bool = True
    rope_k: bool = True
    k_rope: Any = None
    k_rope_tokens: int = 0

    def to_c(self) -> _abi.QKPrologue:
        return _abi.QKPrologue(as_buffer(self.q_norm_weight), as_buffer(self.k_norm_weight), float(self.eps),
                               as_buffer(self.rope), int(self.rope_tokens), int(bool(self.rope_q)),
                               int(bool(self.rope_k)), as_buffer(self.k_rope), int(self.k_rope_tokens))


class AttentionExecutor:
    """AttentionExecutor (AttentionExecutor.swift:97-110); layout is
    ``"headMajor"`` or ``("tokenMajor", token_stride)``."""

    def __init__(self, context: Context, tile_rows: int = 128, numerics: str = "legacy",
                 layout: Any = "headMajor", backend: str = "auto", flash_rows: int = 0):
        lay, ts = self._layout(layout)
        cfg = _abi.AttentionConfig(int(tile_rows), _NUMERICS[numerics], _BACKENDS[backend], lay, ts, int(flash_rows))
        h = C.c_void_p()
        call("anima_attention_create", context.handle, C.byref(cfg), C.byref(h))
        self._h = h
        self.context = context
        self.tile_rows = tile_rows
        self.numerics = numerics

    @staticmethod
    def _layout(layout):
        if layout is None:
            return -1, 0
        if layout == "headMajor":
            return _abi.LAYOUT_HEAD_MAJOR, 0
        if isinstance(layout, tuple) and layout[0] == "tokenMajor":
            return _abi.LAYOUT_TOKEN_MAJOR, int(layout[1])
        raise ValueError(f"unknown layout {layout!r}")

    def maximum_score_scratch_bytes(self, key_count: int, query_count: Optional[int] = None) -> int:
        out = C.c_int64()
        call("anima_attention_max_score_scratch_bytes", self._h, int(key_count),
             int(query_count) if query_count is not None else 0, C.byref(out))
        return out.value

    def workspace_bytes(self) -> int:
        out = C.c_int64()
        call("anima_attention_workspace_bytes", self._h, C.byref(out))
        return out.value

    def _args(self, query, key, value, output, heads, query_count, key_count, head_dim,
              query_offset=0, key_offset=0, value_offset=0, output_offset=0, key_value_heads=None,
              causal=False, layout=None, batch=1, key_lengths=None, key_lengths_on_device=False,
              scale=0.0, prologue: Optional[QKPrologue] = None, kv_token_stride: int = 0):
        lay, ts = self._layout(layout)
        keep = []
        kl = None
        if key_lengths is not None:
            if key_lengths_on_device:
                kl = C.c_void_p(_ptr(key_lengths))
            else:
                arr = np.ascontiguousarray(np.asarray(key_lengths, dtype=np.int32))
                keep.append(arr)
                kl = C.c_void_p(arr.ctypes.data)
        pro = None
        if prologue is not None:
            pc = prologue.to_c()
            keep.append(pc)
            pro = C.pointer(pc)
        a = _abi.AttentionArgs(
            as_buffer(query), int(query_offset), as_buffer(key), int(key_offset),
            as_buffer(value), int(value_offset), as_buffer(output), int(output_offset),
            int(heads), int(query_count), int(key_count), int(head_dim),
            int(key_value_heads or 0), int(bool(causal)), lay, ts, int(batch), kl,
            int(bool(key_lengths_on_device)), float(scale), pro, int(kv_token_stride))
        return a, keep

    def encode(self, **kw) -> None:
        """AttentionExecutor.encode (AttentionExecutor.swift:122-133); appends to the context stream."""
        a, keep = self._args(**kw)
        call("anima_attention_encode", self._h, C.byref(a))
        del keep

    def encode_noalloc(self, **kw) -> None:
        """encode() with the workspace taken from the library's static per-device scratch
        (at most 64 MiB): makes no device allocation (anima_attention_encode_noalloc)."""
        a, keep = self._args(**kw)
        call("anima_attention_encode_noalloc", self._h, C.byref(a))
        del keep

    def execute(self, **kw) -> None:
        """AttentionExecutor.execute (AttentionExecutor.swift:751-776): encode + wait."""
        a, keep = self._args(**kw)
        call("anima_attention_execute", self._h, C.byref(a))
        del keep

    def close(self):
        if self._h:
            call("anima_attention_destroy", self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class QuantizedLinearWeightBuffers:
    """QuantizedLinearWeightBuffers (LinearExecutor.swift:18-29)."""
    storage: int
    packed: Any
    scale: Any
    zero: Any
    rows: int
    columns: int
    packed_row_stride: int
    packed_offset: int = 0
    scale_offset: int = 0
    zero_offset: int = 0

    def to_c(self) -> _abi.QWeight:
        return _abi.QWeight(int(self.storage), as_buffer(self.packed), int(self.packed_offset),
                            as_buffer(self.scale), int(self.scale_offset), as_buffer(self.zero),
                            int(self.zero_offset), int(self.rows), int(self.columns), int(self.packed_row_stride))


_LBACK = {"auto": _abi.LINEAR_AUTO, "fused": _abi.LINEAR_FUSED, "dequantizedGEMM": _abi.LINEAR_DEQUANT_THEN_GEMM}
_EPILOGUE = {"gelu": 1, "gate_add": 2, "residual_add": 3}
_FAMILY = {"other": _abi.FAMILY_OTHER, "attentionProjection": _abi.FAMILY_ATTENTION_PROJECTION,
           "mlpUp": _abi.FAMILY_MLP_UP, "mlpDown": _abi.FAMILY_MLP_DOWN}


class LinearExecutor:
    """LinearExecutor (LinearExecutor.swift:64-75)."""

    def __init__(self, context: Context, tile_rows: int = 128, backend: str = "auto"):
        cfg = _abi.LinearConfig(int(tile_rows), _LBACK[backend])
        h = C.c_void_p()
        call("anima_linear_create", context.handle, C.byref(cfg), C.byref(h))
        self._h = h
        self.context = context
        self.tile_rows = tile_rows

    def encode(self, input, weight: QuantizedLinearWeightBuffers, output, input_rows: int,
               input_offset: int = 0, output_offset: int = 0, family: str = "other") -> None:
        w = weight.to_c()
        call("anima_linear_encode", self._h, as_buffer(input), int(input_offset), C.byref(w),
             as_buffer(output), int(output_offset), int(input_rows), _FAMILY[family])

    def encode_group(self, input, weights, outputs, input_rows: int, family: str = "other") -> None:
        """1..3 linears of one input, each into its own output (one launch when the tiled
        GEMM takes them all)."""
        n = len(weights)
        if n != len(outputs):
            raise ValueError("weights and outputs differ in length")
        ws = [w.to_c() for w in weights]
        wp = (C.POINTER(_abi.QWeight) * n)(*[C.pointer(w) for w in ws])
        ob = (_abi.Buffer * n)(*[as_buffer(o) for o in outputs])
        call("anima_linear_encode_group", self._h, as_buffer(input), C.cast(wp, C.c_void_p),
             C.cast(ob, C.c_void_p), n, int(input_rows), _FAMILY[family])

    def encode_epilogue(self, input, weight: QuantizedLinearWeightBuffers, output, input_rows: int,
                        epilogue: str, residual=None, gate=None, input_offset: int = 0, output_offset: int = 0,
                        family: str = "other") -> None:
        """encode() followed by the DiT block's next step, fused into the GEMM where it can be:
        epilogue "gelu" (dit_gelu_half_inplace on the output) or "gate_add" (gate_add_half_f32
        of the output into the fp32 residual with the fp32 gate; output is then scratch)."""
        w = weight.to_c()
        call("anima_linear_encode_epilogue", self._h, as_buffer(input), int(input_offset), C.byref(w),
             as_buffer(output), int(output_offset), int(input_rows), _FAMILY[family], _EPILOGUE[epilogue],
             as_buffer(residual), as_buffer(gate))

    def encode_head_rmsnorm(self, input, weight: QuantizedLinearWeightBuffers, output, input_rows: int,
                            norm_weight, head_dim: int = 128, eps: float = 1e-6, input_offset: int = 0,
                            output_offset: int = 0, family: str = "attentionProjection") -> None:
        """encode() followed by rmsnorm_heads_half on the output (the cross-attention Q /
        context-K projections of DiTBlockExecutor.swift:1103-1161)."""
        w = weight.to_c()
        call("anima_linear_encode_head_rmsnorm", self._h, as_buffer(input), int(input_offset), C.byref(w),
             as_buffer(output), int(output_offset), int(input_rows), _FAMILY[family], as_buffer(norm_weight),
             int(head_dim), float(eps))

    def execute(self, input, weight: QuantizedLinearWeightBuffers, output, input_rows: int,
                input_offset: int = 0, output_offset: int = 0, family: str = "other") -> None:
        w = weight.to_c()
        call("anima_linear_execute", self._h, as_buffer(input), int(input_offset), C.byref(w),
             as_buffer(output), int(output_offset), int(input_rows), _FAMILY[family])

    @staticmethod
    def encode_matvec(context: Context, weight: QuantizedLinearWeightBuffers, input_f32, output_f32,
                      input_offset: int = 0, output_offset: int = 0) -> None:
        """w4/w8/fp16_matvec_f32 (AnimaKernels.metal:804-933)."""
        w = weight.to_c()
        call("anima_matvec_encode", context.handle, C.byref(w), as_buffer(input_f32), int(input_offset),
             as_buffer(output_f32), int(output_offset))

    @staticmethod
    def encode_dequant(context: Context, weight: QuantizedLinearWeightBuffers, output,
                       out_row_stride: Optional[int] = None, output_offset: int = 0) -> None:
        """dequant_w4_to_half / dequant_w8_to_half (AnimaKernels.metal:19-66)."""
        w = weight.to_c()
        call("anima_dequant_to_half_encode", context.handle, C.byref(w), as_buffer(output), int(output_offset),
             int(out_row_stride if out_row_stride is not None else weight.columns))

    def close(self):
        if self._h:
            call("anima_linear_destroy", self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(np.frombuffer(bytes(a), np.uint8) if isinstance(a, (bytes, bytearray)) else np.asarray(a, np.uint8))


def _u16(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    return np.ascontiguousarray(a.astype(np.uint16, copy=False))


class QuantDecoders:
    """QuantDecoders (QuantDecoders.swift:17-164) through the library's C decoders."""

    @staticmethod
    def dequant_w4(data, scale, zero, k: int, group_size: int = 64) -> np.ndarray:
        d, s, z = _u8(data), _u16(scale), _u16(zero)
        out = np.zeros(max(k, 0), np.float32)
        call("anima_dequant_w4", d.ctypes.data, s.ctypes.data, z.ctypes.data, int(k), int(group_size), out.ctypes.data)
        return out

    @staticmethod
    def dequant_w4_matrix(data, scale, zero, rows: int, cols: int, group_size: int = 64) -> np.ndarray:
        d, s, z = _u8(data), _u16(scale), _u16(zero)
        out = np.zeros((rows, cols), np.float32)
        call("anima_dequant_w4_matrix", d.ctypes.data, s.ctypes.data, z.ctypes.data, int(rows), int(cols),
             int(group_size), out.ctypes.data)
        return out

    @staticmethod
    def dequant_w8(data, scale, zero, k: int, group_size: int = 64) -> np.ndarray:
        d, s, z = _u8(data), _u16(scale), _u16(zero)
        out = np.zeros(max(k, 0), np.float32)
        call("anima_dequant_w8", d.ctypes.data, s.ctypes.data, z.ctypes.data, int(k), int(group_size), out.ctypes.data)
        return out

    @staticmethod
    def dequant_w8_matrix(data, scale, zero, rows: int, cols: int, group_size: int = 64) -> np.ndarray:
        d, s, z = _u8(data), _u16(scale), _u16(zero)
        out = np.zeros((rows, cols), np.float32)
        call("anima_dequant_w8_matrix", d.ctypes.data, s.ctypes.data, z.ctypes.data, int(rows), int(cols),
             int(group_size), out.ctypes.data)
        return out

    @staticmethod
    def fp16_to_float32(bits, count: int) -> np.ndarray:
        b = _u16(bits)
        out = np.zeros(max(count, 0), np.float32)
        call("anima_fp16_to_float32", b.ctypes.data, int(count), out.ctypes.data)
        return out


class DitRoPE:
    """DitRoPE.generate (DitRoPE.swift:58-107): fp32 [T*H*W, 64, 2, 2]."""

    @staticmethod
    def generate(T: int = 1, H: int = 32, W: int = 32) -> np.ndarray:
        out = np.zeros((T * H * W, 64, 2, 2), np.float32)
        call("anima_rope_dit3d", int(T), int(H), int(W), out.ctypes.data)
        return out


def read_probe_sink_bytes(nbytes: int) -> int:
    """Bytes the read probe writes for a read of ``nbytes``."""
    return int(_abi.load().anima_read_probe_sink_bytes(int(nbytes)))


def read_probe(context: Context, src, nbytes: int, sink, src_offset: int = 0) -> None:
    """A plain streaming read of ``nbytes`` of ``src`` (the measurement probe
    anima_read_probe_encode): the floor for a weight-streaming kernel of that byte count."""
    call("anima_read_probe_encode", context.handle, as_buffer(src), int(src_offset), int(nbytes), as_buffer(sink))


class ProbeFlag:
    """Flag bits of a probe slot (NumericalMonitor.Flag, NumericalMonitor.swift:163-170).
    The standalone passes set the first four; the last two belong to the reference's
    in-kernel gate-add probe and are decoded for completeness."""
    NAN = 1
    POS_INF = 2
    NEG_INF = 4
    HALF_OVERFLOW = 8
    RESULT_NAN = 16
    RESULT_INF = 32


PROBE_NO_INDEX = 0xFFFFFFFF


@dataclass(frozen=True)
class ProbeStats:
    """One slot of the stats buffer (NumericalMonitor.Stats, NumericalMonitor.swift:136-161):
    words [flags, max |v| as fp32 bits, first offending index, reserved]."""

    flags: int = 0
    max_abs: float = 0.0
    first_index: int = PROBE_NO_INDEX

    @classmethod
    def from_words(cls, words) -> "ProbeStats":
        w = np.asarray(words, dtype=np.int64).astype(np.uint32)
        return cls(int(w[0]), float(w[1:2].view(np.float32)[0]), int(w[2]))

    has_issue = property(lambda self: self.flags != 0)
    has_nan = property(lambda self: bool(self.flags & ProbeFlag.NAN))
    has_pos_inf = property(lambda self: bool(self.flags & ProbeFlag.POS_INF))
    has_neg_inf = property(lambda self: bool(self.flags & ProbeFlag.NEG_INF))
    has_half_overflow = property(lambda self: bool(self.flags & ProbeFlag.HALF_OVERFLOW))
    result_nan = property(lambda self: bool(self.flags & ProbeFlag.RESULT_NAN))
    result_inf = property(lambda self: bool(self.flags & ProbeFlag.RESULT_INF))

    @property
    def condition(self) -> str:
        """The reference's short condition text, in its priority order."""
        if self.has_nan:
            return "NaN detected"
        if self.has_pos_inf:
            return "positive Inf detected"
        if self.has_neg_inf:
            return "negative Inf detected"
        if self.result_nan:
            return "residual became NaN"
        if self.result_inf:
            return "residual became non-finite"
        if self.has_half_overflow:
            return "value exceeded FP16 finite range"
        return "non-finite value detected"


class NumericalMonitor:
    """The device side of NumericalMonitor (NumericalMonitor.swift:186-212, 320-358): a
    stats buffer of one uint32 quad per probe slot, reset by ``begin_run`` and filled by
    standalone passes over fp16 / fp32 buffers (anima_numerics_probe_encode), all on the
    context's stream.  ``stats(slot)`` synchronises and decodes a slot.  Slot numbers are
    the caller's (the reference numbers its probes in execution order, ``Probe`` below)."""

    # Probe slots in the reference's execution order (NumericalMonitor.swift:21-53).
    PROBES = ("crossContextToHalf", "patchesToHalf", "selfProjectionInput", "selfQToken", "selfKToken",
              "selfVToken", "selfScores", "selfAttended", "selfBranch", "selfGateAdd", "selfResidual",
              "crossProjectionInput", "crossQToken", "crossKToken", "crossVToken", "crossScores",
              "crossAttended", "crossBranch", "crossGateAdd", "crossResidual", "mlpProjectionInput",
              "mlpHiddenToHalf", "mlpBranch", "mlpGateAdd", "mlpResidual", "finalResidualToHalf",
              "finalNormalizedToHalf", "finalProjectionInput", "finalProjected", "velocity", "denoised",
              "eulerOutput")

    def __init__(self, context: Context, slots: Optional[int] = None):
        import torch
        self.context = context
        self.slots = len(self.PROBES) if slots is None else int(slots)
        self.buffer = torch.zeros(self.slots * 4, dtype=torch.int32, device=f"cuda:{context.device}")
        self.begin_run()

    def slot(self, probe) -> int:
        return self.PROBES.index(probe) if isinstance(probe, str) else int(probe)

    def begin_run(self) -> None:
        call("anima_numerics_probe_reset_encode", self.context.handle, as_buffer(self.buffer), self.slots)

    def encode_probe(self, values, probe, count: Optional[int] = None, offset: int = 0) -> None:
        """One pass over ``count`` values (fp16 or fp32 tensor; default: all after
        ``offset``) into the probe's slot."""
        import torch
        if values.dtype == torch.float16:
            dtype = 0
        elif values.dtype == torch.float32:
            dtype = 1
        else:
            raise TypeError("the probe reads fp16 or fp32 values")
        n = values.numel() - int(offset) if count is None else int(count)
        call("anima_numerics_probe_encode", self.context.handle, as_buffer(values), int(offset), n, dtype,
             as_buffer(self.buffer), self.slot(probe))

    def stats(self, probe) -> ProbeStats:
        import torch
        torch.cuda.synchronize(self.context.device)
        s = self.slot(probe)
        return ProbeStats.from_words(self.buffer[4 * s:4 * s + 4].cpu().numpy())


def qwen_rope(tokens: int, head_dim: int = 128, theta: float = 1.0e6) -> np.ndarray:
    """QwenEncoderMetal.makeRope (QwenEncoderMetal.swift:126-143): fp32 [tokens, hd/2, 2, 2]."""
    out = np.zeros((tokens, head_dim // 2, 2, 2), np.float32)
    call("anima_rope_neox", int(tokens), int(head_dim), float(theta), out.ctypes.data)
    return out


class BlockOps:
    """DiT block support kernels (AnimaKernels.metal)."""

    def __init__(self, context: Context):
        self.context = context

    def layernorm_modulate_to_half(self, residual, modulation, output, n: int, rows: int, eps: float = 1e-6,
                                   modulation_offset: Optional[int] = None) -> None:
        call("anima_layernorm_modulate_to_half_encode", self.context.handle, as_buffer(residual),
             as_buffer(modulation), as_buffer(output), int(n), int(rows), float(eps),
             int(n if modulation_offset is None else modulation_offset))

    def gate_add_half_f32(self, residual, branch, gate, n: int, count: int) -> None:
        call("anima_gate_add_half_f32_encode", self.context.handle, as_buffer(residual), as_buffer(branch),
             as_buffer(gate), int(n), int(count))

    def gelu_half_inplace(self, values, count: int) -> None:
        call("anima_gelu_half_inplace_encode", self.context.handle, as_buffer(values), int(count))

    def silu(self, input, output, count: int) -> None:
        call("anima_silu_f32_encode", self.context.handle, as_buffer(input), as_buffer(output), int(count))

    def rmsnorm_f32_to_half(self, input, weight, output, n: int, rows: int, eps: float = 1e-6) -> None:
        """rmsnorm_f32_to_f32 + float_to_half (AnimaKernels.metal:172-204, :81-88)."""
        call("anima_rmsnorm_f32_to_half_encode", self.context.handle, as_buffer(input), as_buffer(weight),
             as_buffer(output), int(n), int(rows), float(eps))

    def gated_silu_half(self, gate, up, output, count: int) -> None:
        """gated_silu_half (AnimaKernels.metal:401-411)."""
        call("anima_gated_silu_half_encode", self.context.handle, as_buffer(gate), as_buffer(up),
             as_buffer(output), int(count))

    def add_half_into_float(self, residual, branch, count: int) -> None:
        """add_half_into_float (AnimaKernels.metal:639-647)."""
        call("anima_add_half_into_float_encode", self.context.handle, as_buffer(residual), as_buffer(branch),
             int(count))

    def add_f32(self, destination, source, count: int) -> None:
        call("anima_add_f32_encode", self.context.handle, as_buffer(destination), as_buffer(source), int(count))


class CrossKVCache:
    """CrossKVCache (DiTBlockExecutor.swift:19-43): per-block cross-attention K/V of the
    fixed context, reused exactly by every sampler step of one generation."""

    def __init__(self, context: Context, blocks: int, context_tokens: int = 512, dim: int = 2048):
        h = C.c_void_p()
        call("anima_cross_kv_cache_create", context.handle, int(blocks), int(context_tokens), int(dim), C.byref(h))
        self._h = h
        self.blocks = blocks

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def reset(self) -> None:
        call("anima_cross_kv_cache_reset", self._h)

    def is_ready(self, block: int) -> bool:
        r = C.c_int32()
        call("anima_cross_kv_cache_is_ready", self._h, int(block), C.byref(r))
        return bool(r.value)

    def bytes(self) -> int:
        n = C.c_int64()
        call("anima_cross_kv_cache_bytes", self._h, C.byref(n))
        return n.value

    def close(self):
        if self._h:
            call("anima_cross_kv_cache_destroy", self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class WeightStreamer:
    """WeightStreamer (WeightStreamer.swift:87-213): ``slots`` device slots of ``capacity``
    bytes filled from host block ranges on a copy stream."""

    def __init__(self, context: Context, capacity: int, slots: int = 2):
        h = C.c_void_p()
        call("anima_weight_streamer_create", context.handle, int(capacity), int(slots), C.byref(h))
        self._h = h
        self.capacity = capacity
        self.slots = slots

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def close(self):
        if self._h:
            call("anima_weight_streamer_destroy", self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DiTBlockExecutor:
    """One DiT block (DiTBlockExecutor.execute, :155-282); fp32 residual updated in place.
    ``forward`` is DitForward.execute (DitForward.swift:78-112) over a list of blocks."""

    NAMES = ("self_q", "self_k", "self_v", "self_o", "cross_q", "cross_k", "cross_v", "cross_o", "mlp1", "mlp2",
             "mod_self_w1", "mod_self_w2", "mod_cross_w1", "mod_cross_w2", "mod_mlp_w1", "mod_mlp_w2")
    NORMS = ("self_q_norm", "self_k_norm", "cross_q_norm", "cross_k_norm")

    def __init__(self, context: Context):
        h = C.c_void_p()
        call("anima_dit_block_create", context.handle, C.byref(h))
        self._h = h
        self.context = context

    @classmethod
    def weights_struct(cls, weights, norms: Optional[dict] = None) -> _abi.DitBlockWeights:
        """A dict of QuantizedLinearWeightBuffers plus a dict of norm buffers, or a ready
        ``_abi.DitBlockWeights`` (for example a rebased pack template), passed through."""
        if isinstance(weights, _abi.DitBlockWeights):
            return weights
        w = _abi.DitBlockWeights()
        for n in cls.NAMES:
            setattr(w, n, weights[n].to_c())
        for n in cls.NORMS:
            setattr(w, n, as_buffer(norms[n]))
        return w

    @staticmethod
    def args_struct(residual, emb, adaln_lora, context_tokens_buf, rope, tokens: int, dim: int = 2048,
                    heads: int = 16, head_dim: int = 128, context_tokens: int = 512, context_dim: int = 1024,
                    mlp_hidden: int = 8192, eps: float = 1e-6) -> _abi.DitBlockArgs:
        return _abi.DitBlockArgs(as_buffer(residual), as_buffer(emb), as_buffer(adaln_lora),
                                 as_buffer(context_tokens_buf), as_buffer(rope), int(tokens), int(dim), int(heads),
                                 int(head_dim), int(context_tokens), int(context_dim), int(mlp_hidden), float(eps))

    def encode(self, weights: dict, norms: dict, residual, emb, adaln_lora, context_tokens_buf, rope,
               tokens: int, cache: Optional[CrossKVCache] = None, block_index: int = 0, **shape) -> None:
        w = self.weights_struct(weights, norms)
        a = self.args_struct(residual, emb, adaln_lora, context_tokens_buf, rope, tokens, **shape)
        if cache is None:
            call("anima_dit_block_encode", self._h, C.byref(w), C.byref(a))
        else:
            call("anima_dit_block_encode_cached", self._h, C.byref(w), C.byref(a), cache.handle, int(block_index))

    def forward(self, blocks: list, residual, emb, adaln_lora, context_tokens_buf, rope, tokens: int,
                cache: Optional[CrossKVCache] = None, **shape) -> None:
        """``blocks`` is a list of (weights, norms) pairs or of ``_abi.DitBlockWeights``, run in
        order over the residual."""
        structs = [b if isinstance(b, _abi.DitBlockWeights) else self.weights_struct(*b) for b in blocks]
        arr = (_abi.DitBlockWeights * len(blocks))(*structs)
        a = self.args_struct(residual, emb, adaln_lora, context_tokens_buf, rope, tokens, **shape)
        call("anima_dit_forward_encode", self._h, arr, len(blocks), C.byref(a), cache.handle if cache else None)

    def forward_streamed(self, streamer: WeightStreamer, templates: list, host_ranges: list, residual, emb,
                         adaln_lora, context_tokens_buf, rope, tokens: int, cache: Optional[CrossKVCache] = None,
                         **shape) -> None:
        """``templates[i]`` is a DitBlockWeights whose device pointers hold byte offsets into
        ``host_ranges[i]`` (an (address, length) pair of host memory)."""
        n = len(templates)
        arr = (_abi.DitBlockWeights * n)(*templates)
        ptrs = (C.c_void_p * n)(*[C.c_void_p(int(r[0])) for r in host_ranges])
        lens = (C.c_int64 * n)(*[int(r[1]) for r in host_ranges])
        a = self.args_struct(residual, emb, adaln_lora, context_tokens_buf, rope, tokens, **shape)
        call("anima_dit_forward_encode_streamed", self._h, streamer.handle, arr, C.cast(ptrs, C.c_void_p),
             C.cast(lens, C.c_void_p), n, C.byref(a), cache.handle if cache else None)

    def close(self):
        if self._h:
            call("anima_dit_block_destroy", self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class LatentOps:
    """The latent-layout and sampler kernels of AnimaKernels.metal: patchify17 (:1225-1246),
    unpatchify16 (:1251-1268), unpatchify_velocity16 (:1276-1297) and
    flow_velocity_to_denoised_f32 (:1191-1201), fp32 buffers throughout."""

    def __init__(self, context: Context):
        self.context = context

    def patchify17(self, input, tokens, height: int, width: int, channels: int = 17) -> None:
        """[channels, H, W] -> [(H/2)*(W/2), 68]; channels 16 appends the zero mask channel."""
        call("anima_patchify17_encode", self.context.handle, as_buffer(input), int(channels), int(height), int(width),
             as_buffer(tokens))

    def unpatchify16(self, tokens, output, height: int, width: int) -> None:
        call("anima_unpatchify16_encode", self.context.handle, as_buffer(tokens), int(height), int(width),
             as_buffer(output))

    def unpatchify_velocity16(self, tokens, output, height: int, width: int) -> None:
        call("anima_unpatchify_velocity16_encode", self.context.handle, as_buffer(tokens), int(height), int(width),
             as_buffer(output))

    def flow_velocity_to_denoised(self, x, velocity, denoised, sigma: float, count: int) -> None:
        """DiffusionSampler.convertVelocity (DiffusionSampler.swift:380-402)."""
        call("anima_flow_velocity_to_denoised_encode", self.context.handle, as_buffer(x), as_buffer(velocity),
             as_buffer(denoised), float(sigma), int(count))


class EulerSampler:
    """EulerSampler (EulerSampler.swift:6-90): the Anima-Turbo 8-step schedule and the fp32
    Euler update ``x_next = x + (next_sigma - sigma) * (x - denoised) / sigma``."""

    SIGMAS = (1.0, 0.9546938, 0.90035903, 0.8339981, 0.7511211, 0.64468634, 0.50298506, 0.30500895, 0.0)

    def __init__(self, context: Context):
        self.context = context

    @staticmethod
    def cpu_step(latent, denoised, sigma: float, next_sigma: float) -> np.ndarray:
        """EulerSampler.cpuStep (:29-40), a CPU function in the reference as well."""
        x = np.asarray(latent, np.float32)
        d = np.asarray(denoised, np.float32)
        if x.size == 0 or x.shape != d.shape or not np.isfinite(sigma) or not sigma > 0 or not np.isfinite(next_sigma):
            raise AnimaError(_abi.E_INVALID_ARGUMENT, "invalid Euler sampler input")
        delta = np.float32(next_sigma) - np.float32(sigma)
        return x + (x - d) / np.float32(sigma) * delta

    def encode_step(self, latent, denoised, output, sigma: float, next_sigma: float, count: int) -> None:
        call("anima_euler_step_encode", self.context.handle, as_buffer(latent), as_buffer(denoised),
             as_buffer(output), float(sigma), float(next_sigma), int(count))


class DiTPreparationExecutor:
    """DiTPreparationExecutor.execute (DiTPreparationExecutor.swift:51-135): latent
    ``[16, H, W]`` fp32 and sigma -> fp32 residual ``[(H/2)*(W/2), dim]``, timestep
    embedding ``[dim]`` and AdaLN-LoRA base ``[3*dim]``.  ``weights`` holds
    ``x_embed`` [dim, 68], ``t_embed1`` [dim, dim], ``t_embed2`` [3*dim, dim]
    (QuantizedLinearWeightBuffers) and ``t_norm`` (fp16 [dim] device buffer)."""

    def __init__(self, context: Context):
        h = C.c_void_p()
        call("anima_dit_prepare_create", context.handle, C.byref(h))
        self._h = h
        self.context = context

    def execute(self, weights: dict, latent, sigma: float, residual, embedding, adaln_lora, height: int = 64,
                width: int = 64, dim: int = 2048, eps: float = 1e-6) -> None:
        if isinstance(weights, _abi.DitPrepareWeights):
            w = weights
        else:
            w = _abi.DitPrepareWeights(weights["x_embed"].to_c(), weights["t_embed1"].to_c(),
                                       weights["t_embed2"].to_c(), as_buffer(weights["t_norm"]))
        a = _abi.DitPrepareArgs(as_buffer(latent), int(height), int(width), float(sigma), as_buffer(residual),
                                as_buffer(embedding), as_buffer(adaln_lora), int(dim), float(eps))
        call("anima_dit_prepare_encode", self._h, C.byref(w), C.byref(a))

    def close(self):
        if self._h:
            call("anima_dit_prepare_destroy", self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DiTFinalLayerExecutor:
    """DiTFinalLayerExecutor.execute (DiTFinalLayerExecutor.swift:75-186, fp16Legacy
    residual boundary): fp32 residual, embedding and AdaLN-LoRA -> fp32 velocity
    ``[16, H, W]``.  ``weights`` holds ``mod_w1`` [lora, dim], ``mod_w2`` [2*dim, lora]
    and ``proj`` [64, dim]."""

    def __init__(self, context: Context):
        h = C.c_void_p()
        call("anima_dit_final_create", context.handle, C.byref(h))
        self._h = h
        self.context = context

    def execute(self, weights: dict, residual, emb, adaln_lora, velocity, height: int = 64, width: int = 64,
                dim: int = 2048, eps: float = 1e-6) -> None:
        if isinstance(weights, _abi.DitFinalWeights):
            w = weights
        else:
            w = _abi.DitFinalWeights(weights["mod_w1"].to_c(), weights["mod_w2"].to_c(), weights["proj"].to_c())
        a = _abi.DitFinalArgs(as_buffer(residual), as_buffer(emb), as_buffer(adaln_lora), as_buffer(velocity),
                              int(height), int(width), int(dim), float(eps))
        call("anima_dit_final_encode", self._h, C.byref(w), C.byref(a))

    def close(self):
        if self._h:
            call("anima_dit_final_destroy", self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class QwenLayerExecutor:
    """QwenLayerExecutor.execute (QwenEncoderMetal.swift:232-304) for a batch of right-padded
    sequences; the fp32 residual ``[batch, tokens, hidden]`` is updated in place."""

    NAMES = ("q", "k", "v", "o", "gate", "up", "down")

    def __init__(self, context: Context):
        h = C.c_void_p()
        call("anima_qwen_layer_create", context.handle, C.byref(h))
        self._h = h
        self.context = context

    def encode(self, weights: dict, norms: dict, residual, rope, batch: int, tokens: int,
               key_lengths=None, hidden: int = 1024, heads: int = 16, kv_heads: int = 8, head_dim: int = 128,
               intermediate: int = 3072, eps: float = 1e-6) -> None:
        w = _abi.QwenLayerWeights()
        for n in self.NAMES:
            setattr(w, n, weights[n].to_c())
        for n in ("input_norm", "post_attention_norm", "q_norm", "k_norm"):
            setattr(w, n, as_buffer(norms[n]))
        keep = None
        kl = None
        if key_lengths is not None:
            keep = np.ascontiguousarray(np.asarray(key_lengths, dtype=np.int32))
            kl = C.c_void_p(keep.ctypes.data)
        a = _abi.QwenLayerArgs(as_buffer(residual), as_buffer(rope), kl, int(batch), int(tokens), int(hidden),
                               int(heads), int(kv_heads), int(head_dim), int(intermediate), float(eps))
        call("anima_qwen_layer_encode", self._h, C.byref(w), C.byref(a))
        del keep

    def close(self):
        if self._h:
            call("anima_qwen_layer_destroy", self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
