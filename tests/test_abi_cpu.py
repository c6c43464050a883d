"""CPU: the C-ABI library loads, exports every function include/anima_hip.h declares, and
its host-side validation rejects bad requests with the reference's messages before any
device work (AttentionExecutor.swift:778-825, LinearExecutor.swift:410-440).  Every case
here fails validation, so no kernel is launched and no device memory is touched; the
buffer pointers are placeholders that are never dereferenced."""

from __future__ import annotations

import ctypes as C
import os
import re

import pytest

import animaxs_amd
from animaxs_amd import _abi
from animaxs_amd._abi import AnimaError

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "anima_hip.h")

FAKE = 0x10000  # placeholder device address; validation fails before it is used


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s+(anima_[a-z0-9_]+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("anima_attention_encode", "anima_linear_encode", "anima_dequant_w4_matrix",
                 "anima_rope_dit3d", "anima_last_error", "anima_ctx_create"):
        assert must in names
    assert len(names) >= 30


def test_library_exports_every_declared_symbol():
    # RTLD_NOW: every symbol the library references must resolve at load time
    # (a kernel whose host stub was not emitted shows up here, not on the GPU).
    lib = C.CDLL(str(_abi.LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_declares_every_symbol():
    missing = [n for n in declared_functions() if n not in _abi.SIGNATURES]
    assert not missing, missing


def test_context_is_lazy_on_cpu():
    ctx = animaxs_amd.Context(0)
    ctx.close()


@pytest.fixture(scope="module")
def ctx():
    c = animaxs_amd.Context(0)
    yield c
    c.close()


def buf(n):
    return (FAKE, int(n))


def attn_kw(**over):
    kw = dict(query=buf(1 << 20), key=buf(1 << 20), value=buf(1 << 20), output=buf(1 << 20),
              heads=2, query_count=4, key_count=4, head_dim=64)
    kw.update(over)
    return kw


def expect(fn, status, fragment):
    with pytest.raises(AnimaError) as ei:
        fn()
    assert ei.value.status == status, ei.value
    assert fragment in ei.value.message, ei.value.message


SHAPE = "invalid attention shape, offset, or causal dimensions"


@pytest.mark.parametrize("over", [dict(heads=0), dict(query_count=0), dict(key_count=-1), dict(head_dim=0),
                                  dict(key_value_heads=3), dict(causal=True, key_count=5),
                                  dict(query_offset=-2)])
def test_attention_shape_validation(ctx, over):
    ex = animaxs_amd.AttentionExecutor(ctx)
    expect(lambda: ex.encode(**attn_kw(**over)), _abi.E_INVALID_SHAPE, SHAPE)


def test_attention_token_major_contract(ctx):
    ex = animaxs_amd.AttentionExecutor(ctx)
    expect(lambda: ex.encode(**attn_kw(layout=("tokenMajor", 100))), _abi.E_INVALID_SHAPE,
           "P4 token-major attention requires tokenStride == heads * headDim and keyValueHeads == heads")
    expect(lambda: ex.encode(**attn_kw(layout=("tokenMajor", 128), key_value_heads=1)), _abi.E_INVALID_SHAPE,
           "P4 token-major attention requires tokenStride == heads * headDim")
    expect(lambda: ex.encode(**attn_kw(layout=("tokenMajor", 128), query_offset=8)), _abi.E_MISALIGNED,
           "P4 token-major attention requires 16-byte-aligned offsets and row stride")


def test_attention_range_and_pointer_checks(ctx):
    ex = animaxs_amd.AttentionExecutor(ctx)
    need = 2 * 4 * 64 * 2
    expect(lambda: ex.encode(**attn_kw(output=buf(need - 2))), _abi.E_OUT_OF_BOUNDS,
           "attention buffer range is out of bounds")
    expect(lambda: ex.encode(**attn_kw(key=buf(need), key_offset=2)), _abi.E_OUT_OF_BOUNDS,
           "attention buffer range is out of bounds")
    expect(lambda: ex.encode(**attn_kw(value=(0, need))), _abi.E_INVALID_ARGUMENT, "pointer is null")
    expect(lambda: ex.encode(**attn_kw(heads=1 << 40, head_dim=1 << 40)), _abi.E_OVERFLOW, "")


def test_attention_numerics_and_lengths(ctx):
    bf16 = animaxs_amd.AttentionExecutor(ctx, numerics="bf16_compute")
    expect(lambda: bf16.encode(**attn_kw()), _abi.E_UNSUPPORTED, "bf16")
    ex = animaxs_amd.AttentionExecutor(ctx)
    expect(lambda: ex.encode(**attn_kw(key_lengths=[0])), _abi.E_INVALID_SHAPE, "key length out of range")
    expect(lambda: ex.encode(**attn_kw(key_lengths=[5])), _abi.E_INVALID_SHAPE, "key length out of range")


def test_flash_backend_rejects_unsupported_head_dim(ctx):
    # the reference's metalFlash backend refuses non-DiT head dims loudly
    # (AttentionExecutorTests.swift testMetalFlashRejectsNonDiTHeadDim)
    ex = animaxs_amd.AttentionExecutor(ctx, layout=("tokenMajor", 128), backend="flash")
    expect(lambda: ex.encode(**attn_kw(head_dim=32, heads=4, layout=("tokenMajor", 128))), _abi.E_UNSUPPORTED,
           "head_dim")


def test_score_scratch_sizing(ctx):
    # AttentionExecutor.swift:112-120 and AttentionExecutorTests.swift:42, :145-148
    legacy = animaxs_amd.AttentionExecutor(ctx)
    assert legacy.maximum_score_scratch_bytes(1024) == 128 * 1024 * 2
    fp32 = animaxs_amd.AttentionExecutor(ctx, numerics="fp32ScoresAndSoftmax")
    assert fp32.maximum_score_scratch_bytes(37, 19) == 19 * 37 * 4
    expect(lambda: legacy.maximum_score_scratch_bytes(0), _abi.E_INVALID_SHAPE, "key count must be positive")


def w4(rows=8, cols=64, stride=None, packed=None, scale=None, zero=None, storage=0):
    stride = (cols + 1) // 2 if stride is None else stride
    groups = (cols + 63) // 64
    return animaxs_amd.QuantizedLinearWeightBuffers(
        storage=storage, packed=buf(rows * stride if packed is None else packed),
        scale=buf(rows * groups * 2 if scale is None else scale),
        zero=buf(rows * groups * 2 if zero is None else zero),
        rows=rows, columns=cols, packed_row_stride=stride)


def test_linear_validation(ctx):
    lin = animaxs_amd.LinearExecutor(ctx)
    x, y = buf(4 * 64 * 2), buf(4 * 8 * 2)
    expect(lambda: lin.encode(x, w4(storage=3), y, 4), _abi.E_UNSUPPORTED,
           "LinearExecutor requires W4, W8, or FP16 weights")
    expect(lambda: lin.encode(x, w4(stride=31), y, 4), _abi.E_INVALID_SHAPE, "packed linear row stride is too small")
    expect(lambda: lin.encode(x, w4(packed=8 * 32 - 1), y, 4), _abi.E_OUT_OF_BOUNDS,
           "LinearExecutor buffer range is out of bounds")
    expect(lambda: lin.encode(x, w4(scale=15), y, 4), _abi.E_OUT_OF_BOUNDS,
           "LinearExecutor buffer range is out of bounds")
    expect(lambda: lin.encode(buf(4 * 64 * 2 - 2), w4(), y, 4), _abi.E_OUT_OF_BOUNDS,
           "LinearExecutor buffer range is out of bounds")
    expect(lambda: lin.encode(x, w4(), y, 0), _abi.E_INVALID_SHAPE, "invalid LinearExecutor shape or offset")
    expect(lambda: lin.encode(x, w4(rows=0), y, 4), _abi.E_INVALID_SHAPE, "invalid LinearExecutor shape or offset")


def test_w8_stride_uses_full_columns(ctx):
    lin = animaxs_amd.LinearExecutor(ctx)
    x, y = buf(4 * 65 * 2), buf(4 * 8 * 2)
    expect(lambda: lin.encode(x, w4(cols=65, stride=33, storage=1), y, 4), _abi.E_INVALID_SHAPE,
           "packed linear row stride is too small")


def test_last_error_is_thread_local_and_set():
    import gc
    import threading
    lib = _abi.load()
    # Any successful call on this thread clears its message, including the destroy calls
    # that finalizers of earlier tests' executors make: collect them first, then keep the
    # collector off while the message must survive.
    gc.collect()
    gc.disable()
    try:
        st = lib.anima_rope_dit3d(0, 1, 1, None)
        assert st != 0
        msg = lib.anima_last_error()
        assert msg and len(msg) > 0
        # a successful call on another thread does not clear this thread's message
        t = threading.Thread(target=lambda: lib.anima_fp16_to_float32(None, 0, None))
        t.start()
        t.join()
        assert lib.anima_last_error() == msg
    finally:
        gc.enable()


def test_grouped_token_major_contract(ctx):
    """kv_token_stride (extension): token-major Q/O rows of heads*D with K/V rows of
    kv_heads*D; any other K/V stride is refused before launch."""
    ex = animaxs_amd.AttentionExecutor(ctx)
    expect(lambda: ex.encode(**attn_kw(layout=("tokenMajor", 128), key_value_heads=1, kv_token_stride=32)),
           _abi.E_INVALID_SHAPE, "kvTokenStride == keyValueHeads * headDim")
    expect(lambda: ex.encode(**attn_kw(layout=("tokenMajor", 128), key_value_heads=1, kv_token_stride=-64)),
           _abi.E_INVALID_SHAPE, "kv_token_stride must be >= 0")
    # K/V ranges use the K/V stride: [4 tokens x 64] halfs is 512 bytes, one short fails.
    expect(lambda: ex.encode(**attn_kw(layout=("tokenMajor", 128), key_value_heads=1, kv_token_stride=64,
                                       key=buf(4 * 64 * 2 - 2))),
           _abi.E_OUT_OF_BOUNDS, "attention buffer range is out of bounds")


def _qwen_weights(hidden=64, qdim=128, kvdim=64, inter=96, bad=None):
    shapes = {"q": (qdim, hidden), "k": (kvdim, hidden), "v": (kvdim, hidden), "o": (hidden, qdim),
              "gate": (inter, hidden), "up": (inter, hidden), "down": (hidden, inter)}
    if bad:
        shapes[bad] = (shapes[bad][0] + 1, shapes[bad][1])
    return {n: w4(rows=r, cols=c, storage=1, stride=c) for n, (r, c) in shapes.items()}


def test_qwen_layer_validation(ctx):
    layer = animaxs_amd.QwenLayerExecutor(ctx)
    norms_ = {n: FAKE for n in ("input_norm", "post_attention_norm", "q_norm", "k_norm")}
    kw = dict(batch=2, tokens=4, hidden=64, heads=2, kv_heads=1, head_dim=64, intermediate=96)
    expect(lambda: layer.encode(_qwen_weights(), norms_, buf(2 * 4 * 64 * 4 - 4), FAKE, **kw),
           _abi.E_OUT_OF_BOUNDS, "invalid Qwen layer input buffers")
    expect(lambda: layer.encode(_qwen_weights(bad="down"), norms_, buf(2 * 4 * 64 * 4), FAKE, **kw),
           _abi.E_INVALID_SHAPE, "invalid Qwen matrix down")
    expect(lambda: layer.encode(_qwen_weights(), norms_, buf(2 * 4 * 64 * 4), FAKE, **dict(kw, kv_heads=3)),
           _abi.E_INVALID_SHAPE, "invalid Qwen layer shape")
    expect(lambda: layer.encode(_qwen_weights(), norms_, buf(2 * 4 * 64 * 4), None, **kw),
           _abi.E_INVALID_ARGUMENT, "requires a RoPE table")
