"""Writes small synthetic ANMA v1 ``.animapk`` files for the pack-reader tests, in the
layout of the reference's test factory (AnimaXSTests/Support/TestPackFactory.swift:12-150)
and of the real packs (AnimapkHeader.swift:5-69, AnimapkFile.swift:72-135):

  header (256 B)   magic "ANMA", u16 version 1, u16 component code, u32 alignment 16384,
                   u64 tensor_count @0x0C, json offset/size @0x14/0x1C, table offset/bytes
                   @0x24/0x2C, payload offset @0x34, file size @0x3C, u32 record size 128
                   @0x44, little-endian
  JSON             at 256: {"component", "quant": {"scheme", "group"}, "tensor_meta": [...]}
  table            at the next 16 KiB boundary: one 128-byte record per tensor (name[64],
                   rank, dims, storage codes, numel, u64 blob_offset @96, blob size, region
                   offsets)
  blobs            each 16 KiB aligned: data | fp16 scale | fp16 zero

Test infrastructure: nothing in the library imports it.
"""

from __future__ import annotations

import json
import struct
import zlib

import numpy as np

ALIGN = 16384
STORAGE = {"w4": 0, "w8": 1, "fp16": 2, "fp32": 3}
COMPONENT = {1: "dit", 2: "te", 3: "vae"}


def _up(x: int, a: int = ALIGN) -> int:
    return (x + a - 1) // a * a


def blob(name, shape, storage, data, scale=b"", zero=b"", crc32=True, quantization_format=None, blob_sha256=None,
         logical_dtype=None):
    """One tensor: raw little-endian data / scale / zero bytes.  crc32 True computes it (zlib),
    an int stores that value, None omits the key."""
    data, scale, zero = bytes(data), bytes(scale), bytes(zero)
    return {"name": name, "shape": list(shape), "storage": storage, "data": data, "scale": scale, "zero": zero,
            "crc32": zlib.crc32(data) & 0xFFFFFFFF if crc32 is True else crc32,
            "quantization_format": quantization_format, "blob_sha256": blob_sha256,
            "logical_dtype": logical_dtype or storage}


def qweight_blob(name, w: dict):
    """An oracle weight dict (``oracle.inputs.symmetric_w4``/``_w8``) as a W4/W8 tensor."""
    storage = {0: "w4", 1: "w8"}[w["storage"]]
    packed = np.asarray(w["packed"], np.uint8).reshape(-1)
    return blob(name, (w["rows"], w["cols"]), storage, packed.tobytes(),
                np.asarray(w["scale_bits"], np.uint16).tobytes(), np.asarray(w["zero_bits"], np.uint16).tobytes())


def fp16_blob(name, values):
    a = np.ascontiguousarray(np.asarray(values, np.float16))
    return blob(name, a.shape, "fp16", a.tobytes())


def layout(blobs, component_code=1, quant_scheme="w4", quant_group=64, order=None):
    """Plan the file: returns (header fields, json bytes, table bytes, [(offset, blob)]).
    ``order`` gives the physical order of the blobs (default: as listed)."""
    order = list(range(len(blobs))) if order is None else list(order)
    # JSON size depends on the offsets' digits only weakly; reserve generously and fix up.
    meta_guess = _json(blobs, [0] * len(blobs), component_code, quant_scheme, quant_group)
    json_offset = 256
    table_offset = _up(json_offset + len(meta_guess) + 4096)
    table_bytes = 128 * len(blobs)
    payload = _up(table_offset + table_bytes)
    offsets = [0] * len(blobs)
    cur = payload
    for i in order:
        offsets[i] = cur
        b = blobs[i]
        cur = _up(cur + len(b["data"]) + len(b["scale"]) + len(b["zero"]))
    js = _json(blobs, offsets, component_code, quant_scheme, quant_group)
    assert json_offset + len(js) <= table_offset
    table = bytearray()
    for b, off in zip(blobs, offsets):
        rec = bytearray(128)
        nm = b["name"].encode()[:64]
        rec[0:len(nm)] = nm
        shape = b["shape"]
        struct.pack_into("<I", rec, 64, len(shape))
        for d in range(4):
            struct.pack_into("<I", rec, 68 + 4 * d, shape[d] if d < len(shape) else 0)
        rec[84] = rec[85] = STORAGE[b["storage"]]
        struct.pack_into("<Q", rec, 88, int(np.prod(shape)) if shape else 1)
        struct.pack_into("<QQ", rec, 96, off, len(b["data"]) + len(b["scale"]) + len(b["zero"]))
        struct.pack_into("<IIII", rec, 112, 0, len(b["data"]), len(b["data"]), len(b["data"]) + len(b["scale"]))
        table += rec
    end = max([off + len(b["data"]) + len(b["scale"]) + len(b["zero"]) for b, off in zip(blobs, offsets)] or [payload])
    header = {"version": 1, "component": component_code, "alignment": ALIGN, "tensor_count": len(blobs),
              "json_offset": json_offset, "json_size": len(js), "table_offset": table_offset,
              "table_bytes": table_bytes, "payload_offset": payload, "file_size": end, "record_size": 128}
    return header, js, bytes(table), list(zip(offsets, blobs))


def _json(blobs, offsets, component_code, quant_scheme, quant_group) -> bytes:
    meta = []
    for b, off in zip(blobs, offsets):
        e = {"name": b["name"], "shape": b["shape"], "logical_dtype": b["logical_dtype"],
             "storage_dtype": b["storage"], "blob_offset": off,
             "blob_size": len(b["data"]) + len(b["scale"]) + len(b["zero"]), "data_offset": 0,
             "data_size": len(b["data"])}
        if b["storage"] in ("w4", "w8") or b["scale"]:
            e.update(scale_offset=len(b["data"]), scale_size=len(b["scale"]),
                     zero_offset=len(b["data"]) + len(b["scale"]), zero_size=len(b["zero"]))
        if b["crc32"] is not None:
            e["crc32"] = b["crc32"]
        if b["quantization_format"]:
            e["quantization_format"] = b["quantization_format"]
        if b["blob_sha256"]:
            e["blob_sha256"] = b["blob_sha256"]
        meta.append(e)
    meta.sort(key=lambda e: e["name"])   # tensor_meta is alphabetical in real packs
    env = {"component": COMPONENT[component_code], "quant": {"scheme": quant_scheme, "group": quant_group},
           "tensor_meta": meta}
    return json.dumps(env, separators=(",", ":")).encode()


def header_bytes(h: dict) -> bytes:
    out = bytearray(256)
    out[0:4] = b"ANMA"
    struct.pack_into("<HHI", out, 4, h["version"], h["component"], h["alignment"])
    struct.pack_into("<QQQQQQQ", out, 0x0C, h["tensor_count"], h["json_offset"], h["json_size"], h["table_offset"],
                     h["table_bytes"], h["payload_offset"], h["file_size"])
    struct.pack_into("<I", out, 0x44, h["record_size"])
    return bytes(out)


def write_pack(path, blobs, component_code=1, quant_scheme="w4", quant_group=64, order=None, json_bytes=None,
               header_override=None):
    """Write the pack; returns (header fields, [(blob offset, blob)])."""
    h, js, table, placed = layout(blobs, component_code, quant_scheme, quant_group, order)
    real_size = h["file_size"]
    table_offset = h["table_offset"]
    if json_bytes is not None:
        js = json_bytes
        h["json_size"] = len(js)
        assert h["json_offset"] + len(js) <= table_offset
    if header_override:
        h.update(header_override)
    with open(path, "wb") as f:
        f.write(header_bytes(h))
        f.write(js)
        f.seek(table_offset)
        f.write(table)
        for off, b in placed:
            f.seek(off)
            f.write(b["data"])
            f.write(b["scale"])
            f.write(b["zero"])
        f.truncate(real_size)
    return h, placed


BLOCK_MATRICES = [
    # suffix, rows, cols
    ("adaln_modulation_self_attn.1.weight", 256, 2048), ("adaln_modulation_self_attn.2.weight", 6144, 256),
    ("adaln_modulation_cross_attn.1.weight", 256, 2048), ("adaln_modulation_cross_attn.2.weight", 6144, 256),
    ("adaln_modulation_mlp.1.weight", 256, 2048), ("adaln_modulation_mlp.2.weight", 6144, 256),
    ("self_attn.q_proj.weight", 2048, 2048), ("self_attn.k_proj.weight", 2048, 2048),
    ("self_attn.v_proj.weight", 2048, 2048), ("self_attn.output_proj.weight", 2048, 2048),
    ("cross_attn.q_proj.weight", 2048, 2048), ("cross_attn.k_proj.weight", 2048, 1024),
    ("cross_attn.v_proj.weight", 2048, 1024), ("cross_attn.output_proj.weight", 2048, 2048),
    ("mlp.layer1.weight", 8192, 2048), ("mlp.layer2.weight", 2048, 8192),
]
BLOCK_NORMS = ["self_attn.q_norm.weight", "self_attn.k_norm.weight", "cross_attn.q_norm.weight",
               "cross_attn.k_norm.weight"]

# pack suffix -> DitBlockWeights field
BLOCK_FIELDS = {
    "adaln_modulation_self_attn.1.weight": "mod_self_w1", "adaln_modulation_self_attn.2.weight": "mod_self_w2",
    "adaln_modulation_cross_attn.1.weight": "mod_cross_w1", "adaln_modulation_cross_attn.2.weight": "mod_cross_w2",
    "adaln_modulation_mlp.1.weight": "mod_mlp_w1", "adaln_modulation_mlp.2.weight": "mod_mlp_w2",
    "self_attn.q_proj.weight": "self_q", "self_attn.k_proj.weight": "self_k", "self_attn.v_proj.weight": "self_v",
    "self_attn.output_proj.weight": "self_o", "cross_attn.q_proj.weight": "cross_q",
    "cross_attn.k_proj.weight": "cross_k", "cross_attn.v_proj.weight": "cross_v",
    "cross_attn.output_proj.weight": "cross_o", "mlp.layer1.weight": "mlp1", "mlp.layer2.weight": "mlp2",
    "self_attn.q_norm.weight": "self_q_norm", "self_attn.k_norm.weight": "self_k_norm",
    "cross_attn.q_norm.weight": "cross_q_norm", "cross_attn.k_norm.weight": "cross_k_norm",
}


def zero_block_blobs(index: int, storage: str = "w4"):
    """A DiT block's 20 tensors with zero payloads (layout tests)."""
    p = f"model.diffusion_model.blocks.{index}."
    out = []
    for suffix, rows, cols in BLOCK_MATRICES:
        if suffix.startswith("adaln"):
            out.append(blob(p + suffix, (rows, cols), "fp16", bytes(rows * cols * 2)))
        else:
            stride = (cols + 1) // 2 if storage == "w4" else cols
            groups = (cols + 63) // 64
            out.append(blob(p + suffix, (rows, cols), storage, bytes(rows * stride), bytes(rows * groups * 2),
                            bytes(rows * groups * 2)))
    for suffix in BLOCK_NORMS:
        out.append(blob(p + suffix, (128,), "fp16", bytes(256)))
    return out
