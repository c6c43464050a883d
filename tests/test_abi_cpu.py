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
    norms_ = {"input_norm": buf(64 * 2), "post_attention_norm": buf(64 * 2), "q_norm": buf(64 * 2),
              "k_norm": buf(64 * 2)}
    rope = buf(4 * 64 * 8)
    kw = dict(batch=2, tokens=4, hidden=64, heads=2, kv_heads=1, head_dim=64, intermediate=96)
    expect(lambda: layer.encode(_qwen_weights(), norms_, buf(2 * 4 * 64 * 4 - 4), rope, **kw),
           _abi.E_OUT_OF_BOUNDS, "invalid Qwen layer input buffers")
    expect(lambda: layer.encode(_qwen_weights(bad="down"), norms_, buf(2 * 4 * 64 * 4), rope, **kw),
           _abi.E_INVALID_SHAPE, "invalid Qwen matrix down")
    expect(lambda: layer.encode(_qwen_weights(), norms_, buf(2 * 4 * 64 * 4), rope, **dict(kw, kv_heads=3)),
           _abi.E_INVALID_SHAPE, "invalid Qwen layer shape")
    expect(lambda: layer.encode(_qwen_weights(), norms_, buf(2 * 4 * 64 * 4), None, **kw),
           _abi.E_INVALID_ARGUMENT, "requires a RoPE table")
    expect(lambda: layer.encode(_qwen_weights(), norms_, buf(2 * 4 * 64 * 4), buf(4 * 64 * 8 - 4), **kw),
           _abi.E_OUT_OF_BOUNDS, "RoPE table is shorter")
    for n in norms_:
        short = dict(norms_, **{n: buf(norms_[n][1] - 2)})
        expect(lambda: layer.encode(_qwen_weights(), short, buf(2 * 4 * 64 * 4), rope, **kw),
               _abi.E_OUT_OF_BOUNDS, "norm weight buffer is too short")
        null = dict(norms_, **{n: None})
        expect(lambda: layer.encode(_qwen_weights(), null, buf(2 * 4 * 64 * 4), rope, **kw),
               _abi.E_INVALID_ARGUMENT, "norm weight pointer is null")


# --------------------------------------------------------------------------------------
# Q/K prologue buffers (lengths checked before launch).
# --------------------------------------------------------------------------------------

def test_prologue_buffer_lengths(ctx):
    ex = animaxs_amd.AttentionExecutor(ctx)
    P = animaxs_amd.QKPrologue
    D = 64
    expect(lambda: ex.encode(**attn_kw(prologue=P(q_norm_weight=buf(D * 2 - 2)))), _abi.E_OUT_OF_BOUNDS,
           "Q RMSNorm weight holds fewer than head_dim")
    expect(lambda: ex.encode(**attn_kw(prologue=P(k_norm_weight=buf(D * 2 - 2)))), _abi.E_OUT_OF_BOUNDS,
           "K RMSNorm weight holds fewer than head_dim")
    # 4 tokens of [32][2][2] fp32 = 4 * 64 * 8 bytes
    expect(lambda: ex.encode(**attn_kw(prologue=P(rope=buf(4 * D * 8 - 4), rope_tokens=4))), _abi.E_OUT_OF_BOUNDS,
           "RoPE table buffer is shorter than rope_tokens rows")
    expect(lambda: ex.encode(**attn_kw(prologue=P(rope=buf(3 * D * 8), rope_tokens=3))), _abi.E_OUT_OF_BOUNDS,
           "RoPE table has fewer rows than query_count")
    expect(lambda: ex.encode(**attn_kw(key_count=6, prologue=P(rope=buf(4 * D * 8), rope_tokens=4, rope_q=False))),
           _abi.E_OUT_OF_BOUNDS, "RoPE table has fewer rows than key_count")
    # separate K table (the adapter's cross attention): its own row count and length
    expect(lambda: ex.encode(**attn_kw(key_count=6, prologue=P(rope=buf(4 * D * 8), rope_tokens=4,
                                                              k_rope=buf(5 * D * 8), k_rope_tokens=5))),
           _abi.E_OUT_OF_BOUNDS, "K RoPE table has fewer rows than key_count")
    expect(lambda: ex.encode(**attn_kw(key_count=6, prologue=P(rope=buf(4 * D * 8), rope_tokens=4,
                                                              k_rope=buf(6 * D * 8 - 4), k_rope_tokens=6))),
           _abi.E_OUT_OF_BOUNDS, "K RoPE table buffer is shorter")
    expect(lambda: ex.encode(**attn_kw(prologue=P(eps=float("nan")))), _abi.E_INVALID_ARGUMENT, "epsilon")


def test_linear_head_rmsnorm_validation(ctx):
    lin = animaxs_amd.LinearExecutor(ctx)
    x, y = buf(4 * 64 * 2), buf(4 * 256 * 2)
    w = w4(rows=256, cols=64)
    expect(lambda: lin.encode_head_rmsnorm(x, w, y, 4, buf(128 * 2 - 2), head_dim=128), _abi.E_OUT_OF_BOUNDS,
           "per-head RMSNorm weight buffer range is out of bounds")
    expect(lambda: lin.encode_head_rmsnorm(x, w, y, 4, None, head_dim=128), _abi.E_INVALID_ARGUMENT,
           "pointer is null")
    expect(lambda: lin.encode_head_rmsnorm(x, w4(rows=200, cols=64), y, 4, buf(256), head_dim=128),
           _abi.E_INVALID_SHAPE, "multiple of head_dim")
    expect(lambda: lin.encode_head_rmsnorm(x, w, y, 4, buf(256), head_dim=0), _abi.E_INVALID_SHAPE,
           "head_dim must be positive")
    expect(lambda: lin.encode_head_rmsnorm(x, w, y, 4, buf(256), head_dim=128, eps=-1.0),
           _abi.E_INVALID_ARGUMENT, "epsilon")


# --------------------------------------------------------------------------------------
# DiT block: every pointer and range is checked before any launch.
# --------------------------------------------------------------------------------------

def _block_case(S=4, dim=256, heads=2, hd=128, T=3, C=128, hidden=512, lora=16):
    shapes = {"self_q": (dim, dim), "self_k": (dim, dim), "self_v": (dim, dim), "self_o": (dim, dim),
              "cross_q": (dim, dim), "cross_k": (dim, C), "cross_v": (dim, C), "cross_o": (dim, dim),
              "mlp1": (hidden, dim), "mlp2": (dim, hidden),
              "mod_self_w1": (lora, dim), "mod_cross_w1": (lora, dim), "mod_mlp_w1": (lora, dim),
              "mod_self_w2": (3 * dim, lora), "mod_cross_w2": (3 * dim, lora), "mod_mlp_w2": (3 * dim, lora)}
    weights = {n: w4(rows=r, cols=c) for n, (r, c) in shapes.items()}
    norms_ = {n: buf(hd * 2) for n in ("self_q_norm", "self_k_norm", "cross_q_norm", "cross_k_norm")}
    args = dict(residual=buf(S * dim * 4), emb=buf(dim * 4), adaln_lora=buf(3 * dim * 4),
                context_tokens_buf=buf(T * C * 2), rope=buf(S * hd * 8))
    shape = dict(tokens=S, dim=dim, heads=heads, head_dim=hd, context_tokens=T, context_dim=C, mlp_hidden=hidden)
    return weights, norms_, args, shape


def test_dit_block_rejects_null_and_short_buffers(ctx):
    blk = animaxs_amd.DiTBlockExecutor(ctx)
    weights, norms_, args, shape = _block_case()

    def run(w=weights, n=norms_, a=args, **over):
        return lambda: blk.encode(w, n, a["residual"], a["emb"], a["adaln_lora"], a["context_tokens_buf"],
                                  a["rope"], **dict(shape, **over))

    for name in norms_:
        expect(run(n=dict(norms_, **{name: None})), _abi.E_INVALID_ARGUMENT, "norm pointer is null")
        expect(run(n=dict(norms_, **{name: buf(128 * 2 - 2)})), _abi.E_OUT_OF_BOUNDS,
               "norm buffer range is out of bounds")
    for name, what in (("residual", "residual"), ("emb", "emb"), ("adaln_lora", "adaln_lora"),
                       ("context_tokens_buf", "context"), ("rope", "RoPE table")):
        expect(run(a=dict(args, **{name: (0, args[name][1])})), _abi.E_INVALID_ARGUMENT,
               f"DiT block {what} pointer is null")
        expect(run(a=dict(args, **{name: buf(args[name][1] - 4)})), _abi.E_OUT_OF_BOUNDS,
               f"DiT block {what} buffer range is out of bounds")
    expect(run(w=dict(weights, mlp2=w4(rows=256, cols=448))), _abi.E_INVALID_SHAPE, "mlp2 shape mismatch")
    expect(run(w=dict(weights, self_v=w4(rows=256, cols=256, packed=100))), _abi.E_OUT_OF_BOUNDS,
           "buffer range is out of bounds")
    expect(run(heads=3), _abi.E_INVALID_SHAPE, "heads * head_dim == dim")


def test_dit_forward_validates_every_block_before_launch(ctx):
    blk = animaxs_amd.DiTBlockExecutor(ctx)
    weights, norms_, args, shape = _block_case()
    bad = dict(weights, cross_o=w4(rows=256, cols=256, scale=2))
    a = args
    expect(lambda: blk.forward([(weights, norms_), (weights, norms_), (bad, norms_)], a["residual"], a["emb"],
                               a["adaln_lora"], a["context_tokens_buf"], a["rope"], **shape),
           _abi.E_OUT_OF_BOUNDS, "buffer range is out of bounds")
    expect(lambda: blk.forward([], a["residual"], a["emb"], a["adaln_lora"], a["context_tokens_buf"], a["rope"],
                               **shape), _abi.E_INVALID_SHAPE, "at least one block")


def test_cache_and_streamer_argument_checks(ctx):
    expect(lambda: animaxs_amd.CrossKVCache(ctx, 0, 512, 2048), _abi.E_INVALID_SHAPE, "invalid cross K/V cache shape")
    expect(lambda: animaxs_amd.WeightStreamer(ctx, 1 << 20, 5), _abi.E_INVALID_ARGUMENT,
           "weight slot count must be in 1...4")
    expect(lambda: animaxs_amd.WeightStreamer(ctx, 0, 2), _abi.E_INVALID_SHAPE, "capacity must be positive")


def test_as_buffer_rejects_host_and_strided_tensors():
    import torch
    with pytest.raises(TypeError, match="GPU tensors"):
        animaxs_amd.as_buffer(torch.zeros(4))
    # a stride-0 expanded view claims more bytes than it owns; checked after the device test,
    # so use a fake object that reports a CUDA tensor which is not contiguous
    class View:
        is_cuda = True

        def data_ptr(self):
            return FAKE

        def is_contiguous(self):
            return False

        def numel(self):
            return 1 << 20

        def element_size(self):
            return 2
    with pytest.raises(TypeError, match="contiguous"):
        animaxs_amd.as_buffer(View())


def test_latent_and_sampler_kernel_checks(ctx):
    """patchify/unpatchify shapes and ranges; EulerSampler.encodeStep / convertVelocity
    rejections (EulerSampler.swift:47-51, DiffusionSampler.swift:380-385)."""
    ops, eu = animaxs_amd.LatentOps(ctx), animaxs_amd.EulerSampler(ctx)
    expect(lambda: ops.patchify17(buf(17 * 16 * 4), buf(4 * 68 * 4), 3, 4), _abi.E_INVALID_SHAPE, "even height")
    expect(lambda: ops.patchify17(buf(15 * 16 * 4), buf(4 * 68 * 4), 4, 4, channels=15), _abi.E_INVALID_SHAPE,
           "16 or 17 channels")
    expect(lambda: ops.patchify17(buf(17 * 16 * 4 - 4), buf(4 * 68 * 4), 4, 4), _abi.E_OUT_OF_BOUNDS,
           "patchify17 input buffer range")
    expect(lambda: ops.patchify17(buf(16 * 16 * 4), buf(4 * 68 * 4 - 4), 4, 4, channels=16), _abi.E_OUT_OF_BOUNDS,
           "patchify17 tokens buffer range")
    expect(lambda: ops.unpatchify16(buf(4 * 68 * 4), buf(16 * 16 * 4 - 4), 4, 4), _abi.E_OUT_OF_BOUNDS,
           "unpatchify16 output")
    expect(lambda: ops.unpatchify_velocity16(buf(4 * 64 * 4 - 4), buf(16 * 16 * 4), 4, 4), _abi.E_OUT_OF_BOUNDS,
           "unpatchify_velocity16 tokens")
    expect(lambda: ops.patchify17(buf(1 << 40), buf(1 << 40), 1 << 20, 1 << 20), _abi.E_INVALID_SHAPE, "too large")
    msg = "invalid Euler sampler buffer or sigma"
    for s, ns, n in ((0.0, 0.5, 8), (-1.0, 0.5, 8), (float("nan"), 0.5, 8), (1.0, float("inf"), 8), (1.0, 0.5, 0)):
        expect(lambda: eu.encode_step(buf(32), buf(32), buf(32), s, ns, n), _abi.E_INVALID_ARGUMENT, msg)
    expect(lambda: eu.encode_step(buf(32), buf(28), buf(32), 1.0, 0.5, 8), _abi.E_OUT_OF_BOUNDS, msg)
    expect(lambda: eu.encode_step(buf(32), buf(32), (0, 32), 1.0, 0.5, 8), _abi.E_INVALID_ARGUMENT, msg)
    fmsg = "invalid FLOW conversion input"
    expect(lambda: ops.flow_velocity_to_denoised(buf(32), buf(32), buf(32), float("nan"), 8), _abi.E_INVALID_ARGUMENT,
           fmsg)
    expect(lambda: ops.flow_velocity_to_denoised(buf(32), buf(31), buf(32), 0.5, 8), _abi.E_OUT_OF_BOUNDS, fmsg)


def _io_weights(dim=256, lora=32):
    return {"x_embed": w4(rows=dim, cols=68), "t_embed1": w4(rows=dim, cols=dim), "t_embed2": w4(rows=3 * dim, cols=dim),
            "t_norm": buf(dim * 2), "mod_w1": w4(rows=lora, cols=dim), "mod_w2": w4(rows=2 * dim, cols=lora),
            "proj": w4(rows=64, cols=dim)}


def test_dit_preparation_validation(ctx):
    """DiTPreparationExecutor.execute guards (DiTPreparationExecutor.swift:55-61, :297-323)."""
    prep = animaxs_amd.DiTPreparationExecutor(ctx)
    w = _io_weights()
    H = W = 8
    a = dict(latent=buf(16 * H * W * 4), residual=buf(16 * 256 * 4), embedding=buf(256 * 4), adaln_lora=buf(768 * 4))

    def run(w=w, sigma=0.5, **over):
        kw = dict(a, height=H, width=W, dim=256)
        kw.update(over)
        return lambda: prep.execute(w, kw.pop("latent"), sigma, kw.pop("residual"), kw.pop("embedding"),
                                    kw.pop("adaln_lora"), **kw)

    for s in (float("nan"), float("inf")):
        expect(run(sigma=s), _abi.E_INVALID_ARGUMENT, "invalid DiT preparation input")
    expect(run(height=6, width=7), _abi.E_INVALID_SHAPE, "even height and width")
    expect(run(dim=255), _abi.E_INVALID_SHAPE, "hidden width must be even")
    expect(run(dim=8194), _abi.E_INVALID_SHAPE, "at most 8192")
    expect(run(w=dict(w, x_embed=w4(rows=256, cols=64))), _abi.E_INVALID_SHAPE, "x_embedder must be [256, 68]")
    expect(run(w=dict(w, t_embed2=w4(rows=512, cols=256))), _abi.E_INVALID_SHAPE, "linear_2 must be [768, 256]")
    expect(run(w=dict(w, t_norm=buf(510))), _abi.E_OUT_OF_BOUNDS, "t_embedding_norm buffer is too small")
    expect(run(w=dict(w, t_norm=None)), _abi.E_INVALID_ARGUMENT, "t_embedding_norm pointer is null")
    for name, what in (("latent", "latent"), ("residual", "residual"), ("embedding", "embedding"),
                       ("adaln_lora", "adaln_lora")):
        expect(run(**{name: buf(a[name][1] - 4)}), _abi.E_OUT_OF_BOUNDS, f"DiT preparation {what} buffer is too small")
        expect(run(**{name: (0, a[name][1])}), _abi.E_INVALID_ARGUMENT, f"DiT preparation {what} pointer is null")


def test_dit_final_layer_validation(ctx):
    """DiTFinalLayerExecutor.validate / FinalWeights (DiTFinalLayerExecutor.swift:382-420)."""
    fin = animaxs_amd.DiTFinalLayerExecutor(ctx)
    w = _io_weights()
    H = W = 8
    a = dict(residual=buf(16 * 256 * 4), emb=buf(256 * 4), adaln_lora=buf(512 * 4), velocity=buf(16 * H * W * 4))

    def run(w=w, **over):
        kw = dict(a, height=H, width=W, dim=256)
        kw.update(over)
        return lambda: fin.execute(w, kw.pop("residual"), kw.pop("emb"), kw.pop("adaln_lora"), kw.pop("velocity"),
                                   **kw)

    expect(run(w=dict(w, mod_w1=w4(rows=32, cols=128))), _abi.E_INVALID_SHAPE, "must have dim columns")
    expect(run(w=dict(w, mod_w2=w4(rows=512, cols=16))), _abi.E_INVALID_SHAPE, "adaln_modulation.2 must be [512, 32]")
    expect(run(w=dict(w, proj=w4(rows=16, cols=256))), _abi.E_INVALID_SHAPE, "linear must be [64, 256]")
    expect(run(height=9), _abi.E_INVALID_SHAPE, "even height and width")
    expect(run(eps=float("nan")), _abi.E_INVALID_ARGUMENT, "epsilon")
    for name in a:
        expect(run(**{name: buf(a[name][1] - 4)}), _abi.E_OUT_OF_BOUNDS, "buffer is too small")
