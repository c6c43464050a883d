"""W4 / W8 group-64 dequantization oracle (numpy, byte-exact).

Restates:
  * ``QuantDecoders.dequantW4``        AnimaXS/Runtime/Animapk/QuantDecoders.swift:23-48
  * ``QuantDecoders.dequantW4Matrix``  QuantDecoders.swift:54-87 (groups reset per row)
  * ``QuantDecoders.dequantW8``        QuantDecoders.swift:90-114
  * ``QuantDecoders.dequantW8Matrix``  QuantDecoders.swift:117-147
  * ``QuantDecoders.fp16ToFloat32``    QuantDecoders.swift:150-163
  * ``dequant_w4_to_half`` / ``dequant_w8_to_half``
                                       AnimaXS/Shaders/AnimaKernels.metal:19-66
  * ``decode_w4_matrix`` / ``decode_w8_matrix``
                                       scripts/animapk_cuda/quant.py:32-76

Value definition: ``v = fl32(q * scale + zero)``.  ``q*scale`` is exact in fp32
(q has at most 8 significant bits, an fp16 scale 11), so the single fp32
rounding happens in the add whether or not the arithmetic is contracted to an
FMA.  The fp16 weight the GEMM consumes is ``RNE16(v)`` (numpy's cast).

Test infrastructure only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import numpy as np

GROUP = 64

# Storage dtype codes of AnimaXS/Runtime/Animapk/AnimapkTensor.swift:4-9.
STORAGE_W4 = 0
STORAGE_W8 = 1
STORAGE_FP16 = 2
STORAGE_FP32 = 3


def fp16_bits_to_f32(bits) -> np.ndarray:
    """QuantDecoders.fp16ToFloat32 (QuantDecoders.swift:150-163): raw little-endian
    binary16 payloads -> float32 (subnormals preserved, as the W8 matvec requires,
    AnimaKernels.metal:845-867)."""
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def _u8(data) -> np.ndarray:
    """Byte payload (bytes-like or array) as a flat uint8 array."""
    if isinstance(data, (bytes, bytearray, memoryview)):
        return np.frombuffer(bytes(data), dtype=np.uint8)
    return np.asarray(data, dtype=np.uint8).reshape(-1)


def _w4_nibbles(packed_rows: np.ndarray, cols: int) -> np.ndarray:
    """Even K index -> low nibble, odd K index -> high nibble
    (QuantDecoders.swift:7-8, :36, :74)."""
    lo = packed_rows & 0x0F
    hi = packed_rows >> 4
    q = np.stack([lo, hi], axis=-1).reshape(packed_rows.shape[0], -1)
    return q[:, :cols]


def dequant_w4(data, scale_bits, zero_bits, k: int, group: int = GROUP) -> np.ndarray:
    """Flat W4 decode (QuantDecoders.swift:23-48): group = i / group (no row reset)."""
    d = _u8(data)
    if k == 0:
        return np.zeros(0, np.float32)
    i = np.arange(k)
    b = d[i >> 1]
    q = np.where((i & 1) == 0, b & 0x0F, b >> 4).astype(np.float32)
    s = fp16_bits_to_f32(scale_bits)[i // group]
    z = fp16_bits_to_f32(zero_bits)[i // group]
    return (q * s + z).astype(np.float32)


def dequant_w8(data, scale_bits, zero_bits, k: int, group: int = GROUP) -> np.ndarray:
    """Flat W8 decode (QuantDecoders.swift:90-114)."""
    d = _u8(data)
    if k == 0:
        return np.zeros(0, np.float32)
    i = np.arange(k)
    q = d[i].astype(np.float32)
    s = fp16_bits_to_f32(scale_bits)[i // group]
    z = fp16_bits_to_f32(zero_bits)[i // group]
    return (q * s + z).astype(np.float32)


def _params(bits, rows: int, groups: int) -> np.ndarray:
    return fp16_bits_to_f32(np.asarray(bits, dtype=np.uint16).reshape(-1)[: rows * groups]).reshape(rows, groups)


def dequant_w4_matrix(packed, scale_bits, zero_bits, rows: int, cols: int,
                      row_stride: int | None = None, group: int = GROUP) -> np.ndarray:
    """Row-aware W4 decode (QuantDecoders.swift:54-87; quant.py:32-52).

    ``packed`` is ``[rows, row_stride]`` bytes; ``row_stride`` defaults to the tight
    ``(cols+1)//2`` and may be padded (LinearExecutor.swift:423-425 allows
    ``packedRowStride >= (K+1)/2``).  Groups index ``r*ceil(cols/64) + c/64``."""
    stride = (cols + 1) // 2 if row_stride is None else row_stride
    p = _u8(packed)[: rows * stride].reshape(rows, stride)
    groups = (cols + group - 1) // group
    q = _w4_nibbles(p[:, : (cols + 1) // 2], cols).astype(np.float32)
    gidx = np.arange(cols) // group
    s = _params(scale_bits, rows, groups)[:, gidx]
    z = _params(zero_bits, rows, groups)[:, gidx]
    return (q * s + z).astype(np.float32)


def dequant_w8_matrix(packed, scale_bits, zero_bits, rows: int, cols: int,
                      row_stride: int | None = None, group: int = GROUP) -> np.ndarray:
    """Row-aware W8 decode (QuantDecoders.swift:117-147; quant.py:55-76)."""
    stride = cols if row_stride is None else row_stride
    p = _u8(packed)[: rows * stride].reshape(rows, stride)
    groups = (cols + group - 1) // group
    q = p[:, :cols].astype(np.float32)
    gidx = np.arange(cols) // group
    s = _params(scale_bits, rows, groups)[:, gidx]
    z = _params(zero_bits, rows, groups)[:, gidx]
    return (q * s + z).astype(np.float32)


def dequant_to_half(storage: int, packed, scale_bits, zero_bits, rows: int, cols: int,
                    row_stride: int | None = None) -> np.ndarray:
    """``dequant_w4_to_half`` / ``dequant_w8_to_half`` (AnimaKernels.metal:19-66):
    ``half(float(q)*float(s)+float(z))`` -> fp16 bit patterns ``uint16[rows, cols]``.
    FP16 storage (LinearExecutor.swift:481-491 reuses the struct) passes through."""
    if storage == STORAGE_W4:
        v = dequant_w4_matrix(packed, scale_bits, zero_bits, rows, cols, row_stride)
    elif storage == STORAGE_W8:
        v = dequant_w8_matrix(packed, scale_bits, zero_bits, rows, cols, row_stride)
    elif storage == STORAGE_FP16:
        stride = cols if row_stride is None else row_stride
        raw = np.asarray(packed).reshape(-1).view(np.uint8)
        return raw[: rows * stride * 2].view(np.uint16).reshape(rows, stride)[:, :cols].copy()
    else:
        raise ValueError(f"unsupported storage {storage}")
    return v.astype(np.float16).view(np.uint16)


def dequant_matrix_f32(storage: int, packed, scale_bits, zero_bits, rows: int, cols: int,
                       row_stride: int | None = None) -> np.ndarray:
    """fp32 dequantized weight ``[rows, cols]`` for any storage code."""
    if storage == STORAGE_W4:
        return dequant_w4_matrix(packed, scale_bits, zero_bits, rows, cols, row_stride)
    if storage == STORAGE_W8:
        return dequant_w8_matrix(packed, scale_bits, zero_bits, rows, cols, row_stride)
    if storage == STORAGE_FP16:
        return dequant_to_half(storage, packed, scale_bits, zero_bits, rows, cols, row_stride).view(np.float16).astype(np.float32)
    raise ValueError(f"unsupported storage {storage}")


# ---------------------------------------------------------------------------
# Packing helpers used by the seeded generators and tests.
# ---------------------------------------------------------------------------
def pack_w4(q: np.ndarray, row_stride: int | None = None, pad_value: int = 0) -> np.ndarray:
    """Pack ``q[rows, cols]`` (0..15) into ``[rows, row_stride]`` bytes with the even
    index in the low nibble (scripts/pack_anima.py:283-293 packing order)."""
    q = np.asarray(q, dtype=np.uint8)
    rows, cols = q.shape
    tight = (cols + 1) // 2
    stride = tight if row_stride is None else row_stride
    assert stride >= tight
    qq = np.zeros((rows, tight * 2), np.uint8)
    qq[:, :cols] = q & 0x0F
    packed = (qq[:, 0::2] | (qq[:, 1::2] << 4)).astype(np.uint8)
    out = np.full((rows, stride), pad_value, np.uint8)
    out[:, :tight] = packed
    return out


def quantize_affine_w4(w: np.ndarray, group: int = GROUP):
    """Affine W4 quantizer in the packer's convention (scripts/pack_anima.py:229-252):
    per (row, group) ``zero = min``, ``scale = span/15``, ``q = round((w-zero)/scale)``.
    Returns (q uint8 [rows, cols], scale_bits, zero_bits uint16 [rows, groups])."""
    w = np.asarray(w, np.float32)
    rows, cols = w.shape
    groups = (cols + group - 1) // group
    q = np.zeros((rows, cols), np.uint8)
    s16 = np.zeros((rows, groups), np.float16)
    z16 = np.zeros((rows, groups), np.float16)
    for g in range(groups):
        blk = w[:, g * group:(g + 1) * group]
        lo = blk.min(axis=1)
        hi = blk.max(axis=1)
        span = np.maximum(hi - lo, 1e-8)
        s = (span / 15.0).astype(np.float16)
        z = lo.astype(np.float16)
        sf = np.maximum(s.astype(np.float32), 1e-8)
        q[:, g * group:(g + 1) * group] = np.clip(np.rint((blk - z.astype(np.float32)[:, None]) / sf[:, None]), 0, 15)
        s16[:, g] = s
        z16[:, g] = z
    return q, s16.view(np.uint16), z16.view(np.uint16)
