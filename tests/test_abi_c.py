"""CPU: a C program compiled against include/anima_hip.h (tests/c/abi_layout.c) checks the
boundary the way a Swift or C binding sees it: every struct's field offsets and sizes as the
C compiler lays them out must equal the ctypes mirror in animaxs_amd/_abi.py, and requests
that fail validation return the reference's status and message through the C entry points
(AttentionExecutor.swift:778-825, LinearExecutor.swift:412-438)."""

from __future__ import annotations

import ctypes as C
import json
import os
import shutil
import subprocess

import pytest

from animaxs_amd import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "c", "abi_layout.c")

STRUCTS = {
    "anima_buffer": _abi.Buffer,
    "anima_attention_config": _abi.AttentionConfig,
    "anima_qk_prologue": _abi.QKPrologue,
    "anima_attention_args": _abi.AttentionArgs,
    "anima_qweight": _abi.QWeight,
    "anima_linear_config": _abi.LinearConfig,
    "anima_dit_block_weights": _abi.DitBlockWeights,
    "anima_dit_block_args": _abi.DitBlockArgs,
    "anima_qwen_layer_weights": _abi.QwenLayerWeights,
    "anima_qwen_layer_args": _abi.QwenLayerArgs,
    "anima_dit_prepare_weights": _abi.DitPrepareWeights,
    "anima_dit_prepare_args": _abi.DitPrepareArgs,
    "anima_dit_final_weights": _abi.DitFinalWeights,
    "anima_dit_final_args": _abi.DitFinalArgs,
    "anima_pack_info": _abi.PackInfo,
    "anima_pack_tensor": _abi.PackTensor,
    "anima_pack_range": _abi.PackRange,
}


@pytest.fixture(scope="module")
def report(tmp_path_factory):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no host C compiler")
    out = tmp_path_factory.mktemp("abi") / "abi_layout"
    libdir = os.path.dirname(str(_abi.LIB_PATH))
    subprocess.run([cc, "-std=c11", "-Wall", "-Werror", "-O1", SRC, "-o", str(out), f"-I{ROOT}/include",
                    f"-L{libdir}", "-lanima_hip", f"-Wl,-rpath,{libdir}"], check=True)
    r = subprocess.run([str(out)], check=True, capture_output=True, text=True)
    return json.loads(r.stdout)


def test_abi_version(report):
    assert report["abi_version"] == _abi.load().anima_abi_version() == 4


def test_every_struct_field_matches_ctypes(report):
    layout = report["layout"]
    seen = set()
    for key, (off, size) in layout.items():
        if "." not in key:
            assert C.sizeof(STRUCTS[key]) == size, f"sizeof({key}) C={size} ctypes={C.sizeof(STRUCTS[key])}"
            continue
        sname, field = key.split(".")
        f = getattr(STRUCTS[sname], field)
        assert (f.offset, f.size) == (off, size), f"{key}: C ({off}, {size}) ctypes ({f.offset}, {f.size})"
        seen.add(key)
    # and the C side lists every ctypes field (no field the C caller does not know of)
    for sname, cls in STRUCTS.items():
        for name, _ in cls._fields_:
            assert f"{sname}.{name}" in seen, f"{sname}.{name} is not checked by the C caller"


def test_rejections_through_the_c_entry_points(report):
    got = {name: (status, msg) for name, status, msg in report["rejections"]}
    ok = {"ctx_create", "attention_create", "linear_create", "prepare_create"}
    for name in ok:
        assert got[name][0] == _abi.OK, (name, got[name])
    want = {
        "ctx_create_negative": (_abi.E_INVALID_ARGUMENT, "handle is null"),
        "attention_causal_counts": (_abi.E_INVALID_SHAPE, "invalid attention shape, offset, or causal dimensions"),
        "attention_token_major_stride": (_abi.E_INVALID_SHAPE,
                                         "P4 token-major attention requires tokenStride == heads * headDim"),
        "attention_short_q_norm": (_abi.E_OUT_OF_BOUNDS, "Q RMSNorm weight holds fewer than head_dim"),
        "attention_short_rope": (_abi.E_OUT_OF_BOUNDS, "RoPE table buffer is shorter than rope_tokens rows"),
        "attention_output_range": (_abi.E_OUT_OF_BOUNDS, "attention buffer range is out of bounds"),
        "attention_null_handle": (_abi.E_INVALID_ARGUMENT, "attention handle is null"),
        "linear_stride": (_abi.E_INVALID_SHAPE, "packed linear row stride is too small"),
        "linear_storage": (_abi.E_UNSUPPORTED, "LinearExecutor requires W4, W8, or FP16 weights"),
        "linear_scale_range": (_abi.E_OUT_OF_BOUNDS, "LinearExecutor buffer range is out of bounds"),
        "cache_shape": (_abi.E_INVALID_SHAPE, "invalid cross K/V cache shape"),
        "streamer_slots": (_abi.E_INVALID_ARGUMENT, "weight slot count must be in 1...4"),
        "rope_dit3d_shape": (_abi.E_INVALID_SHAPE, ""),
        "euler_sigma": (_abi.E_INVALID_ARGUMENT, "invalid Euler sampler buffer or sigma"),
        "patchify_odd": (_abi.E_INVALID_SHAPE, "even height and width"),
        "prepare_sigma": (_abi.E_INVALID_ARGUMENT, "invalid DiT preparation input"),
        "pack_missing": (_abi.E_IO, "cannot open /nonexistent/dir/x.animapk"),
    }
    for name, (status, fragment) in want.items():
        st, msg = got[name]
        assert st == status, (name, st, msg)
        assert fragment in msg, (name, msg)
