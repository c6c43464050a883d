"""CPU: the .animapk (ANMA v1) reader of libanima_hip against synthetic packs written by
tests/pack_writer.py, mirroring AnimapkParsingTests.swift, AnimapkRangeLocatorTests.swift and
the validation of AnimapkFile.swift:72-135, AnimapkRangeLocator.swift:38-261 and
DiTQuantizedWeightFactory.makeMatrix (LinearExecutor.swift:467-518).  No device work: the
pack is mapped on the host and the weight templates hold offsets."""

from __future__ import annotations

import ctypes as C
import json
import struct
import zlib

import numpy as np
import pytest

from animaxs_amd import AnimaError, AnimapkFile, DiTBlockLocator, _abi
from animaxs_amd import animapk as AP
from tests import pack_writer as PW


def expect(fn, status, fragment):
    with pytest.raises(AnimaError) as ei:
        fn()
    assert ei.value.status == status, ei.value
    assert fragment in ei.value.message, ei.value.message


def _w4_pack(path, crc=True):
    """AnimapkParsingTests.makeW4Pack: shape [8192, 2048], documented first data bytes and scales."""
    k = 2048
    data = bytes([110, 135, 69, 55, 138, 137, 37, 98]) + bytes(k // 2 - 8)
    scales = np.zeros(32, np.float16)
    scales[:4] = [0.0004537, 0.0004232, 0.0004251, 0.0004313]
    b = PW.blob("model.diffusion_model.blocks.0.mlp.layer1.weight", (8192, 2048), "w4", data, scales.tobytes(),
                bytes(64), crc32=crc)
    return PW.write_pack(path, [b], component_code=1, quant_scheme="w4", quant_group=64)


def test_header_parse_and_validation(tmp_path):
    p = tmp_path / "dit.animapk"
    _w4_pack(p)
    with AnimapkFile(p) as f:
        assert f.header["version"] == 1 and f.header["component"] == 1
        assert f.header["alignment"] == 16384 and f.header["tensor_count"] == 1 and f.header["record_size"] == 128
        assert f.quant_scheme == "w4" and f.quant_group == 64 and f.component == "dit"
        t = f.tensor("model.diffusion_model.blocks.0.mlp.layer1.weight")
        assert t.shape == (8192, 2048) and t.storage_dtype == "w4" and t.data_size == 1024
        assert t.blob_offset % 16384 == 0 and t.scale_offset == 1024 and t.zero_offset == 1024 + 64
        assert f.tensor("missing") is None
        assert f.crc32_mismatch_count() == 0
        # the mapped data region holds the documented bytes
        assert f.bytes(t.blob_offset, t.blob_offset + 8) == bytes([110, 135, 69, 55, 138, 137, 37, 98])


def test_crc32_matches_zlib_and_detects_corruption(tmp_path):
    p = tmp_path / "dit.animapk"
    h, placed = _w4_pack(p)
    raw = bytearray(p.read_bytes())
    off = placed[0][0]
    raw[off + 3] ^= 0x01   # corrupt one data byte; the JSON keeps the zlib CRC of the original
    p.write_bytes(bytes(raw))
    with AnimapkFile(p) as f:
        assert f.crc32_mismatch_count() == 1
    # a tensor without a CRC counts as matching
    q = tmp_path / "nocrc.animapk"
    _w4_pack(q, crc=None)
    with AnimapkFile(q) as f:
        assert f.tensors[0].crc32 is None and f.crc32_mismatch_count() == 0
    # known answers of the zlib CRC-32 (the check value of the ISO-HDLC CRC)
    r = tmp_path / "check.animapk"
    PW.write_pack(r, [PW.blob("t", (9,), "fp32", b"123456789", crc32=0xCBF43926)])
    with AnimapkFile(r) as f:
        assert f.crc32_mismatch_count() == 0 and zlib.crc32(b"123456789") == 0xCBF43926


def _patch(path, offset, fmt, value):
    raw = bytearray(path.read_bytes())
    struct.pack_into(fmt, raw, offset, value)
    path.write_bytes(bytes(raw))


def test_header_rejections(tmp_path):
    p = tmp_path / "x.animapk"
    cases = [
        (lambda: _patch(p, 0, "<B", 0x58), "bad magic (expected 'ANMA')"),
        (lambda: _patch(p, 4, "<H", 2), "unsupported ANMA version 2 (expected 1)"),
        (lambda: _patch(p, 8, "<I", 4096), "unexpected alignment 4096 (expected 16384)"),
        (lambda: _patch(p, 0x44, "<I", 64), "unexpected record size 64 (expected 128)"),
        (lambda: p.write_bytes(p.read_bytes() + bytes(100)), "declared file size"),
        (lambda: _patch(p, 0x1C, "<Q", 1 << 40), "JSON section out of file bounds"),
        (lambda: _patch(p, 0x2C, "<Q", 1 << 40), "table section out of file bounds"),
        (lambda: _patch(p, 0x34, "<Q", 1 << 40), "payload offset out of file bounds"),
        (lambda: _patch(p, 0x0C, "<Q", 2), "JSON tensor_meta count 1 != header tensor_count 2"),
        (lambda: p.write_bytes(p.read_bytes()[:200]), "file smaller than 256-byte header (200 bytes)"),
    ]
    for mutate, message in cases:
        _w4_pack(p)
        mutate()
        expect(lambda: AnimapkFile(p), _abi.E_FORMAT, message)
    expect(lambda: AnimapkFile(tmp_path / "absent.animapk"), _abi.E_IO, "cannot open")


def _meta_pack(tmp_path, edit, blobs=None, name="m.animapk"):
    """A pack whose JSON is rewritten by edit(env) after layout (same size class)."""
    blobs = blobs or [PW.blob("a", (4,), "fp16", bytes(8)), PW.blob("b", (4,), "fp16", bytes(8))]
    h, js, table, placed = PW.layout(blobs)
    env = json.loads(js)
    edit(env)
    p = tmp_path / name
    PW.write_pack(p, blobs, json_bytes=json.dumps(env).encode())
    return p


def test_tensor_and_table_rejections(tmp_path):
    def field(i, k, v):
        def e(env):
            env["tensor_meta"][i][k] = v
        return e
    expect(lambda: AnimapkFile(_meta_pack(tmp_path, field(0, "blob_offset", 1 << 40))), _abi.E_FORMAT,
           "blob a out of file bounds")
    expect(lambda: AnimapkFile(_meta_pack(tmp_path, field(1, "blob_offset", 16384 * 2 + 512))), _abi.E_FORMAT,
           "not 16 KB aligned")
    expect(lambda: AnimapkFile(_meta_pack(tmp_path, field(0, "data_size", 9))), _abi.E_FORMAT,
           "blob a data region out of blob bounds")

    def scale(env):
        env["tensor_meta"][0].update(scale_offset=4, scale_size=8)
    expect(lambda: AnimapkFile(_meta_pack(tmp_path, scale)), _abi.E_FORMAT, "blob a scale region out of blob bounds")

    def moved(env):   # both JSON offsets valid, but b no longer where the table says
        env["tensor_meta"][1]["blob_offset"] += 16384
    p = _meta_pack(tmp_path, moved, blobs=[PW.blob("a", (4,), "fp16", bytes(8)),
                                           PW.blob("b", (4,), "fp16", bytes(8)),
                                           PW.blob("c", (4,), "fp16", bytes(8))])
    expect(lambda: AnimapkFile(p), _abi.E_FORMAT, "JSON blob_offsets")
    expect(lambda: AnimapkFile(_meta_pack(tmp_path, lambda env: env.pop("tensor_meta"))), _abi.E_FORMAT,
           "failed to decode architecture JSON")
    expect(lambda: AnimapkFile(_meta_pack(tmp_path, field(0, "blob_size", -1))), _abi.E_FORMAT,
           "failed to decode architecture JSON")
    expect(lambda: AnimapkFile(_meta_pack(tmp_path, field(0, "shape", "4"))), _abi.E_FORMAT,
           "shape of a is not an array")
    # the C record holds 8 dimensions: a 9-dimensional shape is refused, never cut off
    expect(lambda: AnimapkFile(_meta_pack(tmp_path, field(0, "shape", [1] * 8 + [4]))), _abi.E_FORMAT,
           "shape of a has more than 8 dimensions")


def test_malformed_json_text(tmp_path):
    blobs = [PW.blob("a", (4,), "fp16", bytes(8))]
    _, js, _, _ = PW.layout(blobs)
    for bad in (js[:-1], js + b"x", js.replace(b'"component"', b'component')):
        p = tmp_path / "bad.animapk"
        PW.write_pack(p, blobs, json_bytes=bad)
        expect(lambda: AnimapkFile(p), _abi.E_FORMAT, "failed to decode architecture JSON")
    # escapes and unicode in a name round-trip through the parser
    p = tmp_path / "esc.animapk"
    PW.write_pack(p, [PW.blob('q"\\é中\U0001F600', (4,), "fp16", bytes(8))])
    with AnimapkFile(p) as f:
        assert f.tensors[0].name == 'q"\\é中\U0001F600'


def test_optional_quantization_metadata(tmp_path):
    """AnimapkParsingTests.testOptionalANEQuantizationMetadataDecodesWithoutBreakingLegacy."""
    digest = "a" * 64
    b = PW.blob("model.diffusion_model.blocks.0.self_attn.q_proj.weight", (2, 2), "w8", bytes([0, 127, 255, 64]),
                np.array([0.01, 0.02], np.float32).tobytes(), np.array([-1.0, 2.0], np.float32).tobytes(),
                quantization_format="ane_u8_per_row_fp32_v1", blob_sha256=digest)
    p = tmp_path / "ane.animapk"
    PW.write_pack(p, [b], quant_scheme="w8-ane-hybrid-v1")
    with AnimapkFile(p) as f:
        assert f.tensors[0].quantization_format == "ane_u8_per_row_fp32_v1"
        assert f.quant_scheme == "w8-ane-hybrid-v1"
    q = tmp_path / "legacy.animapk"
    _w4_pack(q)
    with AnimapkFile(q) as f:
        assert f.tensors[0].quantization_format is None


def test_dit_logical_order_and_relative_spans(tmp_path):
    """AnimapkRangeLocatorTests.testDiTLogicalOrderAndRelativeSpans: blobs in lexicographic
    physical order (10 before 2) come back in numerical execution order."""
    idx = sorted(range(28), key=str)
    blobs = [PW.blob(f"model.diffusion_model.blocks.{i}.weight", (4,), "w4", bytes([i, 0]), bytes(2), bytes(2))
             for i in idx]
    p = tmp_path / "dit-ranges.animapk"
    PW.write_pack(p, blobs)
    with AnimapkFile(p) as f:
        loc = DiTBlockLocator(f)
        assert [b.logical_index for b in loc.blocks] == list(range(28))
        assert len({b.file_offset for b in loc.blocks}) == 28
        for b in loc.blocks:
            assert b.tensor_count == 1 and b.file_offset % 16384 == 0 and b.length == 6
            assert C.string_at(b.host, 1)[0] == b.logical_index
            assert f.bytes(b.file_offset, b.file_offset + 1)[0] == b.logical_index
        assert loc.block(10).file_offset < loc.block(2).file_offset
        phys = sorted(loc.blocks, key=lambda r: r.file_offset)
        assert all(a.file_offset + a.length <= c.file_offset for a, c in zip(phys, phys[1:]))
        with pytest.raises(AnimaError, match="out of range"):
            loc.block(28)
        expect(lambda: f.execution_ranges("model.diffusion_model.blocks.", 29), _abi.E_FORMAT,
               "no tensors found for model.diffusion_model.blocks.28.")


def test_overlapping_ranges_and_incomplete_metadata(tmp_path):
    # block 0 = tensors at physical slots 0 and 2, block 1 at slot 1: the ranges overlap
    blobs = [PW.blob("blk.0.a", (4,), "fp16", bytes(8)), PW.blob("blk.1.a", (4,), "fp16", bytes(8)),
             PW.blob("blk.0.b", (4,), "fp16", bytes(8))]
    p = tmp_path / "ov.animapk"
    PW.write_pack(p, blobs)
    with AnimapkFile(p) as f:
        expect(lambda: f.execution_ranges("blk.", 2), _abi.E_FORMAT, "execution ranges 0 and 1 overlap")

    def incomplete(env):
        env["tensor_meta"][0]["scale_offset"] = 8
    q = _meta_pack(tmp_path, incomplete, blobs=[PW.blob("blk.0.a", (4,), "fp16", bytes(8))])
    with AnimapkFile(q) as f:
        expect(lambda: f.execution_ranges("blk.", 1), _abi.E_FORMAT, "blk.0.a has incomplete scale metadata")


@pytest.fixture(scope="module")
def dit_pack(tmp_path_factory):
    """Two zero-filled DiT blocks (W4 projections, fp16 modulation and norms) plus the
    preparation and final-layer tensors, physically interleaved with an unrelated tensor."""
    p = tmp_path_factory.mktemp("pack") / "dit.animapk"
    pre = "model.diffusion_model."
    blobs = PW.zero_block_blobs(0) + [PW.blob(pre + "pos_embedder.weight", (4,), "fp16", bytes(8))] + \
        PW.zero_block_blobs(1)
    w4 = lambda n, r, c: PW.blob(n, (r, c), "w4", bytes(r * ((c + 1) // 2)), bytes(r * ((c + 63) // 64) * 2),
                                 bytes(r * ((c + 63) // 64) * 2))
    blobs += [w4(pre + "x_embedder.proj.1.weight", 2048, 68), w4(pre + "t_embedder.1.linear_1.weight", 2048, 2048),
              w4(pre + "t_embedder.1.linear_2.weight", 6144, 2048),
              PW.blob(pre + "t_embedding_norm.weight", (2048,), "fp16", bytes(4096)),
              w4(pre + "final_layer.adaln_modulation.1.weight", 256, 2048),
              w4(pre + "final_layer.adaln_modulation.2.weight", 4096, 256),
              w4(pre + "final_layer.linear.weight", 64, 2048)]
    PW.write_pack(p, blobs)
    return p


def test_dit_block_templates(dit_pack):
    with AnimapkFile(dit_pack) as f:
        for b in (0, 1):
            w, r = f.dit_block(b)
            assert r.tensor_count == 20 and r.logical_index == b and r.file_offset % 16384 == 0
            prefix = f"model.diffusion_model.blocks.{b}."
            for suffix, rows, cols in PW.BLOCK_MATRICES:
                q = getattr(w, PW.BLOCK_FIELDS[suffix])
                t = f.tensor(prefix + suffix)
                assert (q.rows, q.columns) == (rows, cols)
                assert q.packed.ptr is None and q.packed.length == r.length
                assert q.packed_offset == t.blob_offset + t.data_offset - r.file_offset
                if t.storage_dtype == "w4":
                    assert q.storage == 0 and q.packed_row_stride == (cols + 1) // 2
                    assert q.scale_offset == t.blob_offset + t.scale_offset - r.file_offset
                    assert q.zero_offset == t.blob_offset + t.zero_offset - r.file_offset
                else:
                    assert q.storage == 2 and q.packed_row_stride == cols and q.scale_offset == q.packed_offset
            for suffix in PW.BLOCK_NORMS:
                nb = getattr(w, PW.BLOCK_FIELDS[suffix])
                t = f.tensor(prefix + suffix)
                assert nb.ptr == t.blob_offset - r.file_offset and nb.length == 256
            # rebase onto a device copy of the range at `base`
            base = 1 << 40
            dw = AP.rebase_block(w, base, r.length)
            assert dw.self_q.packed.ptr == base and dw.self_q.packed.length == r.length
            assert dw.self_q_norm.ptr == base + w.self_q_norm.ptr
            with pytest.raises(AnimaError, match="outside its block range"):
                AP.rebase_block(w, base, w.self_q_norm.ptr - 1)
        expect(lambda: f.dit_block(2), _abi.E_FORMAT, "no tensors found for model.diffusion_model.blocks.2.")


def test_prepare_and_final_templates(dit_pack):
    with AnimapkFile(dit_pack) as f:
        w, r = f.dit_prepare(2048)
        assert r.tensor_count == 4 and r.logical_index == -2
        assert (w.x_embed.rows, w.x_embed.columns, w.x_embed.packed_row_stride) == (2048, 68, 34)
        assert (w.t_embed2.rows, w.t_embed2.columns) == (6144, 2048) and w.t_norm.length == 4096
        fw, fr = f.dit_final(2048)
        assert fr.tensor_count == 3 and fr.logical_index == -1
        assert (fw.mod_w1.rows, fw.mod_w2.rows, fw.mod_w2.columns, fw.proj.rows) == (256, 4096, 256, 64)
        expect(lambda: f.dit_prepare(1024), _abi.E_INVALID_SHAPE, "x_embedder.proj.1.weight shape mismatch")
        expect(lambda: f.dit_final(1024), _abi.E_INVALID_SHAPE, "adaln_modulation.1.weight shape mismatch")
        pw = AP.rebase_prepare(w, 4096, r.length)
        assert pw.t_norm.ptr == 4096 + w.t_norm.ptr and pw.x_embed.packed.ptr == 4096
        fw2 = AP.rebase_final(fw, 4096, fr.length)
        assert fw2.proj.packed.ptr == 4096


def test_block_layout_rejections(tmp_path):
    def pack_with(edit):
        blobs = PW.zero_block_blobs(0)
        edit(blobs)
        p = tmp_path / "bad-block.animapk"
        PW.write_pack(p, blobs)
        return AnimapkFile(p)

    def drop(blobs):
        del blobs[[b["name"] for b in blobs].index("model.diffusion_model.blocks.0.mlp.layer2.weight")]
    with pack_with(drop) as f:
        expect(lambda: f.dit_block(0), _abi.E_FORMAT, "missing DiT matrix model.diffusion_model.blocks.0.mlp.layer2")

    def shape(blobs):
        b = blobs[[x["name"] for x in blobs].index("model.diffusion_model.blocks.0.cross_attn.k_proj.weight")]
        b["shape"] = [2048, 2048]
    with pack_with(shape) as f:
        expect(lambda: f.dit_block(0), _abi.E_INVALID_SHAPE, "cross_attn.k_proj.weight shape mismatch")

    def short(blobs):
        i = [x["name"] for x in blobs].index("model.diffusion_model.blocks.0.self_attn.q_proj.weight")
        blobs[i] = dict(blobs[i], scale=blobs[i]["scale"][:-2])
    with pack_with(short) as f:
        expect(lambda: f.dit_block(0), _abi.E_FORMAT, "quantized layout mismatch")

    def norm(blobs):
        i = [x["name"] for x in blobs].index("model.diffusion_model.blocks.0.cross_attn.q_norm.weight")
        blobs[i] = PW.blob(blobs[i]["name"], (64,), "fp16", bytes(128))
    with pack_with(norm) as f:
        expect(lambda: f.dit_block(0), _abi.E_FORMAT, "invalid DiT norm model.diffusion_model.blocks.0.cross_attn.q_norm")

    def extra(blobs):
        blobs.append(PW.blob("model.diffusion_model.blocks.0.extra.weight", (4,), "fp16", bytes(8)))
    with pack_with(extra) as f:
        expect(lambda: f.dit_block(0), _abi.E_FORMAT, "exactly 20 tensors")

    def fp32(blobs):
        i = [x["name"] for x in blobs].index("model.diffusion_model.blocks.0.mlp.layer1.weight")
        blobs[i] = PW.blob(blobs[i]["name"], (8192, 2048), "fp32", bytes(16))
    with pack_with(fp32) as f:
        expect(lambda: f.dit_block(0), _abi.E_FORMAT, "must be W4, W8, or FP16")
