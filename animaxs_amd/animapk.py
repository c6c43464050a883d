"""``.animapk`` (ANMA v1) packs over the C ABI: the reference's AnimapkFile
(AnimaXS/Runtime/Animapk/AnimapkFile.swift:15-185), AnimapkTensor
(AnimapkTensor.swift:90-153), AnimapkExecutionRange and the DiT locators
(AnimapkRangeLocator.swift:21-261).

The library maps the file and validates it (header, JSON, tensor ranges, table
cross-match); this module only marshals.  Weight templates returned by
``dit_block`` / ``dit_prepare`` / ``dit_final`` hold offsets into their execution
range: ``DiTBlockExecutor.forward_streamed`` takes block templates with the ranges'
host addresses as they are, and ``rebase_*`` turns a template into device weights
once the range has been copied to the GPU.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional

from . import _abi
from ._abi import call

STORAGE_NAMES = {0: "w4", 1: "w8", 2: "fp16", 3: "fp32"}


@dataclass(frozen=True)
class AnimapkTensor:
    name: str
    shape: tuple
    logical_dtype: str
    storage: int
    blob_offset: int
    blob_size: int
    data_offset: int
    data_size: int
    scale_offset: Optional[int]
    scale_size: Optional[int]
    zero_offset: Optional[int]
    zero_size: Optional[int]
    crc32: Optional[int]
    block_index: Optional[int]
    quantization_format: Optional[str]

    @property
    def storage_dtype(self) -> str:
        return STORAGE_NAMES[self.storage]

    @staticmethod
    def from_c(t: _abi.PackTensor) -> "AnimapkTensor":
        opt = lambda v: None if v < 0 else int(v)
        return AnimapkTensor(
            name=t.name.decode(), shape=tuple(int(t.shape[i]) for i in range(t.rank)),
            logical_dtype=t.logical_dtype.decode(), storage=int(t.storage), blob_offset=int(t.blob_offset),
            blob_size=int(t.blob_size), data_offset=int(t.data_offset), data_size=int(t.data_size),
            scale_offset=opt(t.scale_offset), scale_size=opt(t.scale_size), zero_offset=opt(t.zero_offset),
            zero_size=opt(t.zero_size), crc32=int(t.crc32) if t.has_crc32 else None,
            block_index=opt(t.block_index),
            quantization_format=t.quantization_format.decode() if t.quantization_format else None)


@dataclass(frozen=True)
class AnimapkExecutionRange:
    logical_index: int
    file_offset: int
    length: int
    tensor_count: int
    host: int            # address of the mapped bytes (valid while the pack is open)

    @property
    def file_range(self) -> range:
        return range(self.file_offset, self.file_offset + self.length)

    @staticmethod
    def from_c(r: _abi.PackRange) -> "AnimapkExecutionRange":
        return AnimapkExecutionRange(int(r.logical_index), int(r.file_offset), int(r.length), int(r.tensor_count),
                                     int(r.host or 0))


class AnimapkFile:
    """An open pack (read-only mapping).  ``header`` holds the fixed 256-byte header's
    fields; ``tensors`` the JSON tensor_meta in file order."""

    def __init__(self, path):
        h = C.c_void_p()
        call("anima_pack_open", str(path).encode(), C.byref(h))
        self._h = h
        info = _abi.PackInfo()
        call("anima_pack_get_info", h, C.byref(info))
        self.header = {n: getattr(info, n) for n, _ in _abi.PackInfo._fields_
                       if n not in ("quant_scheme", "component_name", "quant_group")}
        self.component = info.component_name.decode()
        self.quant_scheme = info.quant_scheme.decode() if info.quant_scheme else None
        self.quant_group = None if info.quant_group < 0 else int(info.quant_group)
        self.tensors = []
        for i in range(int(info.tensor_count)):
            t = _abi.PackTensor()
            call("anima_pack_tensor_at", h, i, C.byref(t))
            self.tensors.append(AnimapkTensor.from_c(t))

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def tensor(self, name: str) -> Optional[AnimapkTensor]:
        t = _abi.PackTensor()
        st = _abi.load().anima_pack_find(self._h, name.encode(), C.byref(t))
        return AnimapkTensor.from_c(t) if st == _abi.OK else None

    def crc32_mismatch_count(self) -> int:
        n = C.c_int64()
        call("anima_pack_crc32_mismatch_count", self._h, C.byref(n))
        return n.value

    def bytes(self, start: int, end: int) -> bytes:
        """AnimapkFile.bytes(in:) (copied out of the mapping)."""
        p = C.c_void_p()
        call("anima_pack_bytes", self._h, int(start), int(end) - int(start), C.byref(p))
        return C.string_at(p.value, int(end) - int(start)) if end > start else b""

    def execution_ranges(self, prefix: str, count: int) -> list:
        arr = (_abi.PackRange * max(1, count))()
        call("anima_pack_execution_ranges", self._h, prefix.encode(), int(count), arr)
        return [AnimapkExecutionRange.from_c(arr[i]) for i in range(count)]

    def dit_block(self, block: int):
        """(DitBlockWeights template, AnimapkExecutionRange) of DiT block ``block``."""
        w, r = _abi.DitBlockWeights(), _abi.PackRange()
        call("anima_pack_dit_block", self._h, int(block), C.byref(w), C.byref(r))
        return w, AnimapkExecutionRange.from_c(r)

    def dit_prepare(self, dim: int = 2048):
        w, r = _abi.DitPrepareWeights(), _abi.PackRange()
        call("anima_pack_dit_prepare", self._h, int(dim), C.byref(w), C.byref(r))
        return w, AnimapkExecutionRange.from_c(r)

    def dit_final(self, dim: int = 2048):
        w, r = _abi.DitFinalWeights(), _abi.PackRange()
        call("anima_pack_dit_final", self._h, int(dim), C.byref(w), C.byref(r))
        return w, AnimapkExecutionRange.from_c(r)

    def close(self):
        if self._h:
            call("anima_pack_close", self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DiTBlockLocator:
    """DiTBlockLocator (AnimapkRangeLocator.swift:156-174): the 28 block ranges in logical order."""

    block_count = 28

    def __init__(self, file: AnimapkFile, count: int = 28):
        self.blocks = file.execution_ranges("model.diffusion_model.blocks.", count)

    def block(self, index: int) -> AnimapkExecutionRange:
        if not 0 <= index < len(self.blocks):
            raise _abi.AnimaError(_abi.E_INVALID_ARGUMENT, f"DiT block index {index} is out of range")
        return self.blocks[index]


def rebase_block(tmpl: _abi.DitBlockWeights, base: int, range_bytes: int) -> _abi.DitBlockWeights:
    out = _abi.DitBlockWeights()
    call("anima_dit_block_weights_rebase", C.byref(tmpl), C.c_void_p(int(base)), int(range_bytes), C.byref(out))
    return out


def rebase_prepare(tmpl: _abi.DitPrepareWeights, base: int, range_bytes: int) -> _abi.DitPrepareWeights:
    out = _abi.DitPrepareWeights()
    call("anima_dit_prepare_weights_rebase", C.byref(tmpl), C.c_void_p(int(base)), int(range_bytes), C.byref(out))
    return out


def rebase_final(tmpl: _abi.DitFinalWeights, base: int, range_bytes: int) -> _abi.DitFinalWeights:
    out = _abi.DitFinalWeights()
    call("anima_dit_final_weights_rebase", C.byref(tmpl), C.c_void_p(int(base)), int(range_bytes), C.byref(out))
    return out
