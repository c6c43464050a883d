"""GPU: anima_attention_encode_noalloc (the allocation-free variant of anima_attention_encode)
against anima_attention_encode, through the C ABI.

Both run the same plan and kernels; only the workspace differs (the library's static
per-device array instead of the executor's allocations), so the outputs must be identical
bit for bit.  Two calls in a row share the static array, the second with a smaller input
and a different workspace use (K prologue rows, then key-split partial rows), so stale
contents from the first call must not leak into the second.  A request whose workspace
exceeds the array is refused before launch.
"""

import pytest
import torch

from animaxs_amd import AnimaError, AttentionExecutor, QKPrologue
from animaxs_amd import _abi
from oracle import inputs
from tests.helpers import dev

pytestmark = pytest.mark.gpu


def _pair(ctx, label, **kw):
    """(output of encode, output of encode_noalloc) for the same arguments."""
    out_shape = kw.pop("out_shape")
    layout = kw.pop("layout")
    ref = torch.full(out_shape, float("nan"), dtype=torch.float16, device="cuda")
    got = torch.full(out_shape, float("nan"), dtype=torch.float16, device="cuda")
    ex = AttentionExecutor(ctx, layout=layout)
    ex.encode(output=ref, **kw)
    na = AttentionExecutor(ctx, layout=layout)
    print(f"NOALLOC {label}", flush=True)
    na.encode_noalloc(output=got, **kw)
    torch.cuda.synchronize()
    assert na.workspace_bytes() == 0, "the allocation-free call grew the executor's own workspace"
    return ref, got


def test_noalloc_equals_encode_on_consecutive_calls(ctx):
    # 1) S=4096 self attention with Q/K RMSNorm + DiT RoPE: the K prologue rows (16 MiB) live
    #    in the static workspace.
    d = inputs.self_attention(2)
    q, k, v = (dev(d[n]) for n in "qkv")
    pro = QKPrologue(dev(d["q_norm_w"]), dev(d["k_norm_w"]), d["eps"], dev(d["rope"]), 4096, True, True)
    ref, got = _pair(ctx, "S4096 norm+rope", query=q, key=k, value=v, heads=16, query_count=4096, key_count=4096,
                     head_dim=128, prologue=pro, out_shape=(1, 4096, 16, 128), layout=("tokenMajor", 2048))
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))

    # 2) smaller: S=1024 without a prologue takes two key splits; their partial rows now
    #    occupy the same static array from offset 0.
    d1 = inputs.self_attention(1)
    q1, k1, v1 = (dev(d1[n]) for n in "qkv")
    ref1, got1 = _pair(ctx, "S1024 key splits", query=q1, key=k1, value=v1, heads=16, query_count=1024,
                       key_count=1024, head_dim=128, out_shape=(1, 1024, 16, 128), layout=("tokenMajor", 2048))
    assert torch.isfinite(got1.float()).all()
    assert torch.equal(got1.view(torch.int16), ref1.view(torch.int16))

    # 3) smaller again: Qwen-shaped causal GQA with right padding and a K prologue (4 MiB).
    d4 = inputs.qwen_attention()
    q4, k4, v4 = (dev(d4[n]) for n in "qkv")
    pro4 = QKPrologue(dev(d4["q_norm_w"]), dev(d4["k_norm_w"]), d4["eps"], dev(d4["rope"]), 512, True, True)
    ref4, got4 = _pair(ctx, "qwen causal gqa", query=q4, key=k4, value=v4, heads=16, query_count=512, key_count=512,
                       head_dim=128, key_value_heads=8, kv_token_stride=1024, causal=True, batch=4,
                       key_lengths=d4["key_lengths"].numpy(), prologue=pro4, out_shape=(4, 512, 16, 128),
                       layout=("tokenMajor", 2048))
    assert torch.equal(got4.view(torch.int16), ref4.view(torch.int16))

    # 4) the head-dim-384 kernel (VAE mid-block shape): 8 key splits, whose fp16 partial rows
    #    (24 MiB) and (max, sum) pairs take the static array.
    g = torch.Generator().manual_seed(384)
    q8, k8, v8 = (dev(torch.randn(4096, 384, generator=g).half()) for _ in range(3))
    ref8, got8 = _pair(ctx, "D384 key splits", query=q8, key=k8, value=v8, heads=1, query_count=4096,
                       key_count=4096, head_dim=384, out_shape=(4096, 384), layout="headMajor")
    assert torch.isfinite(got8.float()).all()
    assert torch.equal(got8.view(torch.int16), ref8.view(torch.int16))


def test_noalloc_refuses_a_workspace_beyond_its_array(ctx):
    """K prologue rows of 16448 tokens x 16 heads x 128 = 64.25 MiB > 64 MiB."""
    S = 16384 + 64
    q = torch.zeros(S, 2048, dtype=torch.float16, device="cuda")
    w = torch.ones(128, dtype=torch.float16, device="cuda")
    o = torch.zeros_like(q)
    ex = AttentionExecutor(ctx, layout=("tokenMajor", 2048))
    with pytest.raises(AnimaError) as ei:
        ex.encode_noalloc(query=q, key=q, value=q, output=o, heads=16, query_count=S, key_count=S, head_dim=128,
                          prologue=QKPrologue(w, w, 1e-6))
    assert ei.value.status == _abi.E_UNSUPPORTED
    assert "allocation-free entry point holds at most" in ei.value.message
