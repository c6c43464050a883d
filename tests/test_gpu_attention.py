"""GPU parity of the attention path against the CPU oracle (through the C ABI).

Bar: max-abs <= 1e-2 and mean-rel (sum|y-ref|/sum|ref|) <= 1e-3 against the fp32
oracle for every workload; the reference's own special-case answers
(AttentionExecutorTests.swift) at their own tolerances.
"""

import math

import numpy as np
import pytest
import torch

import animaxs_amd
from animaxs_amd import AnimaError, AttentionExecutor, QKPrologue
from oracle import attention as oatt
from oracle import inputs, rope as orope
from tests.helpers import assert_attention_close, dev

pytestmark = pytest.mark.gpu


def _run(ctx, q, k, v, *, layout, heads, Sq, Sk, D, out_shape, backend="auto", flash_rows=0, **kw):
    o = torch.full(out_shape, float("nan"), dtype=torch.float16, device="cuda")
    ex = AttentionExecutor(ctx, layout=layout, backend=backend, flash_rows=flash_rows)
    ex.execute(query=q, key=k, value=v, output=o, heads=heads, query_count=Sq, key_count=Sk, head_dim=D, **kw)
    torch.cuda.synchronize()
    return o


def test_workload1_self_attention_s1024(ctx):
    d = inputs.self_attention(1)
    q, k, v = (dev(d[n]) for n in "qkv")
    o = _run(ctx, q, k, v, layout=("tokenMajor", 2048), heads=16, Sq=1024, Sk=1024, D=128, out_shape=(1, 1024, 16, 128))
    ref = oatt.sdpa(d["q"], d["k"], d["v"])
    assert_attention_close(o, ref, label="workload1 S1024")


def test_workload2_self_attention_s4096_norm_rope(ctx):
    d = inputs.self_attention(2)
    q, k, v = (dev(d[n]) for n in "qkv")
    rope = dev(d["rope"])
    pro = QKPrologue(dev(d["q_norm_w"]), dev(d["k_norm_w"]), d["eps"], rope, 4096, True, True)
    o = _run(ctx, q, k, v, layout=("tokenMajor", 2048), heads=16, Sq=4096, Sk=4096, D=128,
             out_shape=(1, 4096, 16, 128), prologue=pro)
    qq = oatt.qk_prologue(d["q"], d["q_norm_w"], d["eps"], d["rope"])
    kk = oatt.qk_prologue(d["k"], d["k_norm_w"], d["eps"], d["rope"])
    ref = oatt.sdpa(qq, kk, d["v"])
    assert_attention_close(o, ref, label="workload2 S4096 norm+rope")


@pytest.mark.parametrize("device_lengths", [False, True])
def test_workload3_cross_attention_masked(ctx, device_lengths):
    d = inputs.cross_attention()
    q, k, v = (dev(d[n]) for n in "qkv")
    L = d["key_lengths"]
    lengths = dev(L) if device_lengths else L.numpy()
    pro = QKPrologue(dev(d["q_norm_w"]), dev(d["k_norm_w"]), d["eps"], None, 0, False, False)
    o = _run(ctx, q, k, v, layout=("tokenMajor", 2048), heads=16, Sq=4096, Sk=512, D=128,
             out_shape=(4, 4096, 16, 128), batch=4, key_lengths=lengths, key_lengths_on_device=device_lengths,
             prologue=pro)
    qq = oatt.qk_prologue(d["q"], d["q_norm_w"], d["eps"], None)
    kk = oatt.qk_prologue(d["k"], d["k_norm_w"], d["eps"], None)
    ref = oatt.sdpa(qq, kk, d["v"], key_lengths=L.tolist())
    assert_attention_close(o, ref, label=f"workload3 cross masked dev={device_lengths}")


def test_workload3_reference_faithful_unmasked_zero_context(ctx):
    """Reference behaviour: no mask; context rows >= L_b are zero
    (scripts/animapk_cuda/comfy_stub/comfy/ldm/anima/model.py:204-205)."""
    d = inputs.cross_attention(B=2, Sq=512)
    L = d["key_lengths"][:2]
    k, v = d["k"].clone(), d["v"].clone()
    for b in range(2):
        k[b, int(L[b]):] = 0
        v[b, int(L[b]):] = 0
    pro = QKPrologue(dev(d["q_norm_w"]), dev(d["k_norm_w"]), d["eps"], None, 0, False, False)
    o = _run(ctx, dev(d["q"]), dev(k), dev(v), layout=("tokenMajor", 2048), heads=16, Sq=512, Sk=512, D=128,
             out_shape=(2, 512, 16, 128), batch=2, prologue=pro)
    qq = oatt.qk_prologue(d["q"], d["q_norm_w"], d["eps"], None)
    kk = oatt.qk_prologue(k, d["k_norm_w"], d["eps"], None)
    ref = oatt.sdpa(qq, kk, v)
    assert_attention_close(o, ref, label="workload3 unmasked zero-padded")


def test_workload4_qwen_causal_gqa(ctx):
    d = inputs.qwen_attention()
    # head-major [B, H, S, D] like the reference's Qwen path (QwenEncoderMetal.swift:269-279)
    qh = d["q"].permute(0, 2, 1, 3).contiguous()
    kh = d["k"].permute(0, 2, 1, 3).contiguous()
    vh = d["v"].permute(0, 2, 1, 3).contiguous()
    L = d["key_lengths"]
    pro = QKPrologue(dev(d["q_norm_w"]), dev(d["k_norm_w"]), d["eps"], dev(d["rope"]), 512, True, True)
    o = _run(ctx, dev(qh), dev(kh), dev(vh), layout="headMajor", heads=16, Sq=512, Sk=512, D=128,
             out_shape=(4, 16, 512, 128), batch=4, key_value_heads=8, causal=True, key_lengths=L.numpy(),
             prologue=pro)
    qq = oatt.qk_prologue(d["q"], d["q_norm_w"], d["eps"], d["rope"])
    kk = oatt.qk_prologue(d["k"], d["k_norm_w"], d["eps"], d["rope"])
    ref = oatt.sdpa(qq, kk, d["v"], causal=True, key_lengths=L.tolist())
    assert_attention_close(o.permute(0, 2, 1, 3), ref, label="workload4 qwen causal gqa")


@pytest.mark.parametrize("flash_rows", [128, 256])
def test_workload4_token_major_grouped_kv_stride(ctx, flash_rows):
    """Workload 4 on the projections' own token-major rows: Q/O [B, S, 16*128], K/V
    [B, S, 8*128] (kv_token_stride extension), both flash variants."""
    d = inputs.qwen_attention()
    L = d["key_lengths"]
    pro = QKPrologue(dev(d["q_norm_w"]), dev(d["k_norm_w"]), d["eps"], dev(d["rope"]), 512, True, True)
    o = _run(ctx, dev(d["q"]), dev(d["k"]), dev(d["v"]), layout=("tokenMajor", 2048), heads=16, Sq=512, Sk=512,
             D=128, out_shape=(4, 512, 16, 128), backend="flash", flash_rows=flash_rows, batch=4,
             key_value_heads=8, kv_token_stride=1024, causal=True, key_lengths=L.numpy(), prologue=pro)
    qq = oatt.qk_prologue(d["q"], d["q_norm_w"], d["eps"], d["rope"])
    kk = oatt.qk_prologue(d["k"], d["k_norm_w"], d["eps"], d["rope"])
    ref = oatt.sdpa(qq, kk, d["v"], causal=True, key_lengths=L.tolist())
    assert_attention_close(o, ref, label=f"workload4 token-major grouped flash{flash_rows}")


# ---------------------------------------------------------------------------
# Reference special cases (AnimaXSTests/AttentionExecutorTests.swift)
# ---------------------------------------------------------------------------
def test_cross_attention_last_value_row_tail_tile(ctx):
    """AttentionExecutorTests.swift:64-88: Q=K=0, only the last V row nonzero ->
    every output row equals (c+1)/512 (129 queries exercise a tail tile)."""
    Sq, Sk, D = 129, 512, 64
    q = torch.zeros(Sq * D, dtype=torch.float16)
    k = torch.zeros(Sk * D, dtype=torch.float16)
    v = torch.zeros(Sk, D, dtype=torch.float16)
    v[-1] = torch.arange(1, D + 1, dtype=torch.float16)
    o = _run(ctx, dev(q), dev(k), dev(v), layout="headMajor", heads=1, Sq=Sq, Sk=Sk, D=D, out_shape=(Sq, D))
    expect = (torch.arange(1, D + 1, dtype=torch.float32) / 512).expand(Sq, D)
    assert float((o.float().cpu() - expect).abs().max()) <= 1e-4


def test_grouped_query_attention_contiguous_kv_heads(ctx):
    """AttentionExecutorTests.swift:90-111: heads 4, kv heads 2 -> mapping 0,0,1,1."""
    q = torch.zeros(4 * 4, dtype=torch.float16)
    k = torch.zeros(2 * 4, dtype=torch.float16)
    v = torch.tensor([2.0] * 4 + [9.0] * 4, dtype=torch.float16)
    o = _run(ctx, dev(q), dev(k), dev(v), layout="headMajor", heads=4, Sq=1, Sk=1, D=4, out_shape=(16,),
             key_value_heads=2)
    assert o.float().cpu().tolist() == [2.0] * 8 + [9.0] * 8


def test_token_major_no_head_mixing(ctx):
    """AttentionExecutorTests.swift:460-504: Q=K=0 -> per-head mean of V rows."""
    heads, D, rows = 2, 4, 3
    model = heads * D
    vals = torch.zeros(rows, model)
    for t in range(rows):
        for h in range(heads):
            for c in range(D):
                vals[t, h * D + c] = t * 10 + h + c / 10
    vals = vals.half()
    zeros = torch.zeros(rows, model, dtype=torch.float16)
    o = _run(ctx, dev(zeros), dev(zeros), dev(vals), layout=("tokenMajor", model), heads=heads, Sq=rows, Sk=rows,
             D=D, out_shape=(rows, model))
    expect = vals.float().mean(0, keepdim=True).expand(rows, model)
    assert float((o.float().cpu() - expect).abs().max()) <= 0.05


def test_query_tiled_self_attention_hd64(ctx):
    """AttentionExecutorTests.swift:28-62 generator (Q=K=1024, hd=64), tol 0.012."""
    count, dim = 1024, 64
    idx = torch.arange(count * dim, dtype=torch.float64)
    q = (torch.sin(((idx * 13) % 997) * 0.017) * 0.25).half()
    k = (torch.cos(((idx * 7) % 991) * 0.019) * 0.25).half()
    v = ((((idx * 17) % 101) - 50) / 50).half()
    o = _run(ctx, dev(q), dev(k), dev(v), layout="headMajor", heads=1, Sq=count, Sk=count, D=dim,
             out_shape=(count, dim))
    ref = oatt.sdpa(q.view(1, count, 1, dim), k.view(1, count, 1, dim), v.view(1, count, 1, dim))[0, :, 0]
    err = float((o.float().cpu() - ref).abs().max())
    assert err <= 0.012, err


def test_flash_backend_rejects_non_dit_head_dim(ctx):
    """AttentionExecutorTests.swift:404-423: the flash backend refuses loudly."""
    heads, D, n = 4, 32, 4
    buf = torch.zeros(n * heads * D, dtype=torch.float16, device="cuda")
    ex = AttentionExecutor(ctx, layout=("tokenMajor", heads * D), backend="flash")
    with pytest.raises(AnimaError) as e:
        ex.execute(query=buf, key=buf, value=buf, output=buf, heads=heads, query_count=n, key_count=n, head_dim=D)
    assert e.value.status == animaxs_amd._abi.E_UNSUPPORTED


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("Sq,Sk,causal", [(200, 77, False), (1, 1, False), (130, 130, True), (257, 700, False),
                                          (600, 600, True), (513, 33, False)])
def test_flash_matches_oracle_ragged(ctx, D, Sq, Sk, causal):
    g = torch.Generator().manual_seed(Sq * 1000 + Sk + D)
    H = 3
    q = torch.randn(1, H, Sq, D, generator=g).half()
    k = torch.randn(1, H, Sk, D, generator=g).half()
    v = torch.randn(1, H, Sk, D, generator=g).half()
    outs = {}
    for name, backend, rows in (("flash128", "flash", 128), ("flash256", "flash", 256), ("flashauto", "flash", 0),
                                ("generic", "generic", 0)):
        outs[name] = _run(ctx, dev(q), dev(k), dev(v), layout="headMajor", heads=H, Sq=Sq, Sk=Sk, D=D,
                          out_shape=(1, H, Sq, D), backend=backend, flash_rows=rows, causal=causal)
    ref = oatt.sdpa(q.permute(0, 2, 1, 3), k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3), causal=causal)
    for name, o in outs.items():
        assert_attention_close(o.permute(0, 2, 1, 3), ref, label=f"{name} D{D} Sq{Sq} Sk{Sk} causal={causal}")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("B,Sq,Sk", [(2, 300, 2056), (1, 1024, 1024), (3, 64, 1040), (1, 1, 4096)])
def test_flash_key_splits(ctx, D, B, Sq, Sk):
    """Short query sequences over long key sequences: the 256-row kernel splits the keys across
    workgroups (2 to 8 splits of at least 512 keys, the last one ragged: 2056 keys in 4 splits of
    576, 1040 in 2 of 576) and a second kernel merges the fp16 normalised partial rows by their fp32
    (max, sum) pairs; token-major layout, batch > 1."""
    g = torch.Generator().manual_seed(B * Sq + Sk + D)
    H = 4
    q = torch.randn(B, Sq, H, D, generator=g).half()
    k = torch.randn(B, Sk, H, D, generator=g).half()
    v = torch.randn(B, Sk, H, D, generator=g).half()
    print(f"SPLITS D={D} B={B} Sq={Sq} Sk={Sk}", flush=True)
    o = _run(ctx, dev(q), dev(k), dev(v), layout=("tokenMajor", H * D), heads=H, Sq=Sq, Sk=Sk, D=D,
             out_shape=(B, Sq, H, D), batch=B)
    ref = oatt.sdpa(q, k, v)
    assert_attention_close(o, ref, label=f"splits D{D} B{B} Sq{Sq} Sk{Sk}")


@pytest.mark.parametrize("H,Sq,Sk,lengths,D", [
    (24, 2048, 2048, None, 128),   # 8 query tiles x 24 heads x 2 key splits = 384 workgroups
    (8, 4096, 1200, [1117], 128),  # host key length (no splits): 16 query tiles x 8 heads = 128
    (16, 2048, 1024, None, 64),    # head_dim 64: 8 query tiles x 16 heads x 2 key splits = 256
])
def test_flash_head_grouped_block_order(ctx, H, Sq, Sk, lengths, D):
    """Single-image launches of at least 128 workgroups over at least 1024 keys whose head count
    8 divides decode 8 heads of one query tile on consecutive workgroups (three groups of 8 at H=24, the only group at H=8),
    with and without key splits: every (query tile, head) is still computed exactly once."""
    g = torch.Generator().manual_seed(H * Sq + Sk + D)
    q = torch.randn(1, Sq, H, D, generator=g).half()
    k = torch.randn(1, Sk, H, D, generator=g).half()
    v = torch.randn(1, Sk, H, D, generator=g).half()
    lens = None if lengths is None else np.array(lengths, dtype=np.int32)
    print(f"HEADGROUP H={H} Sq={Sq} Sk={Sk} D={D} lengths={lengths}", flush=True)
    o = _run(ctx, dev(q), dev(k), dev(v), layout=("tokenMajor", H * D), heads=H, Sq=Sq, Sk=Sk, D=D,
             out_shape=(1, Sq, H, D), key_lengths=lens)
    ref = oatt.sdpa(q, k, v, key_lengths=lengths)
    assert_attention_close(o, ref, label=f"head-grouped H{H} Sq{Sq} Sk{Sk} D{D}")


@pytest.mark.parametrize("B,H,Hkv,Sq,Sk,D,lengths,on_device,norm", [
    (3, 16, 16, 4000, 600, 128, [600, 1, 130], False, True),   # one-tile entry, partial query tile
    (2, 32, 8, 2048, 64, 64, None, False, True),               # head_dim 64, grouped K/V heads, one tile
    (2, 16, 4, 4096, 1000, 128, [1000, 65], True, True),       # device key lengths
    (4, 64, 64, 1000, 128, 128, None, False, True),            # four entries over a partial query tile
    (5, 32, 32, 2048, 300, 128, [300, 2, 299, 64, 65], False, False),   # no Q/K norm, five entries
])
def test_flash_persistent_batch_matches_per_entry_calls(ctx, B, H, Hkv, Sq, Sk, D, lengths, on_device, norm):
    """Batched non-causal calls whose query tiles x heads fill whole rounds of the chip (a
    multiple of 256) run one workgroup per (query tile, head) over every batch entry, with the
    next entry's Q rows and first tiles loaded during the current one.  Each entry must equal
    the same entry computed alone (batch 1, one workgroup per tile) bit for bit, and the oracle
    within the attention bar; the fused Q norm (when given) runs on every entry."""
    g = torch.Generator().manual_seed(7 * B + H + Sq + Sk + D)
    q = torch.randn(B, Sq, H, D, generator=g).half()
    k = torch.randn(B, Sk, Hkv, D, generator=g).half()
    v = torch.randn(B, Sk, Hkv, D, generator=g).half()
    w = (0.8 + 0.4 * torch.rand(D, generator=g)).half()
    pro = QKPrologue(dev(w), dev(w), 1e-6, None, 0, False, False) if norm else None
    kw = dict(layout=("tokenMajor", H * D), heads=H, Sq=Sq, Sk=Sk, D=D, key_value_heads=Hkv,
              kv_token_stride=Hkv * D, prologue=pro)
    lens = None if lengths is None else (dev(torch.tensor(lengths, dtype=torch.int32)) if on_device
                                         else np.array(lengths, dtype=np.int32))
    print(f"PERSIST B={B} H={H} Hkv={Hkv} Sq={Sq} Sk={Sk} D={D} lengths={lengths} dev={on_device}", flush=True)
    o = _run(ctx, dev(q), dev(k), dev(v), out_shape=(B, Sq, H, D), batch=B, key_lengths=lens,
             key_lengths_on_device=on_device, **kw)
    for b in range(B):
        lb = None if lengths is None else (dev(torch.tensor(lengths[b:b + 1], dtype=torch.int32)) if on_device
                                           else np.array(lengths[b:b + 1], dtype=np.int32))
        ob = _run(ctx, dev(q[b:b + 1]), dev(k[b:b + 1]), dev(v[b:b + 1]), out_shape=(1, Sq, H, D), batch=1,
                  key_lengths=lb, key_lengths_on_device=on_device, **kw)
        assert torch.equal(o[b:b + 1], ob), f"entry {b} differs from its batch-1 call"
    qq = oatt.qk_prologue(q, w, 1e-6, None) if norm else q
    kk = oatt.qk_prologue(k, w, 1e-6, None) if norm else k
    ref = oatt.sdpa(qq, kk, v, key_lengths=lengths)
    assert_attention_close(o, ref, label=f"persistent B{B} H{H} Sq{Sq} Sk{Sk} D{D} norm={norm}")


@pytest.mark.parametrize("flash_rows", [128, 256])
def test_flash_variants_masked_batch_gqa(ctx, flash_rows):
    """Both flash variants on batch + GQA + causal + right-padding key lengths + prologue."""
    g = torch.Generator().manual_seed(99)
    B, S, H, Hkv, D = 3, 700, 4, 2, 128
    q = torch.randn(B, H, S, D, generator=g).half()
    k = torch.randn(B, Hkv, S, D, generator=g).half()
    v = torch.randn(B, Hkv, S, D, generator=g).half()
    w = (0.8 + 0.4 * torch.rand(D, generator=g)).half()
    rope = orope.neox_rope_table(S, 1.0e6, D)
    L = [700, 301, 64]
    pro = QKPrologue(dev(w), dev(w), 1e-6, dev(rope), S, True, True)
    o = _run(ctx, dev(q), dev(k), dev(v), layout="headMajor", heads=H, Sq=S, Sk=S, D=D, out_shape=(B, H, S, D),
             backend="flash", flash_rows=flash_rows, batch=B, key_value_heads=Hkv, causal=True, key_lengths=L,
             prologue=pro)
    qq = oatt.qk_prologue(q.permute(0, 2, 1, 3), w, 1e-6, rope)
    kk = oatt.qk_prologue(k.permute(0, 2, 1, 3), w, 1e-6, rope)
    ref = oatt.sdpa(qq, kk, v.permute(0, 2, 1, 3), causal=True, key_lengths=L)
    assert_attention_close(o.permute(0, 2, 1, 3), ref, label=f"flash{flash_rows} batch gqa causal masked")


def test_generic_odd_head_dim_with_prologue(ctx):
    """Generic path, head_dim 6 (even, not 64/128) with norm + RoPE prologue."""
    g = torch.Generator().manual_seed(7)
    B, S, H, D = 2, 37, 4, 6
    q = torch.randn(B, S, H, D, generator=g).half()
    k = torch.randn(B, S, H, D, generator=g).half()
    v = torch.randn(B, S, H, D, generator=g).half()
    w = (0.8 + 0.4 * torch.rand(D, generator=g)).half()
    rope = orope.neox_rope_table(S, 1.0e4, D)
    pro = QKPrologue(dev(w), dev(w), 1e-6, dev(rope), S, True, True)
    o = _run(ctx, dev(q), dev(k), dev(v), layout=("tokenMajor", H * D), heads=H, Sq=S, Sk=S, D=D,
             out_shape=(B, S, H, D), batch=B, prologue=pro)
    qq = oatt.qk_prologue(q, w, 1e-6, rope)
    kk = oatt.qk_prologue(k, w, 1e-6, rope)
    ref = oatt.sdpa(qq, kk, v)
    assert_attention_close(o, ref, label="generic D6 prologue")


def test_validation_errors_do_not_launch(ctx):
    """AttentionExecutor.validate (AttentionExecutor.swift:778-825) error contract."""
    buf = torch.zeros(64, dtype=torch.float16, device="cuda")
    ex = AttentionExecutor(ctx)
    with pytest.raises(AnimaError) as e:
        ex.execute(query=buf, key=buf, value=buf, output=buf, heads=2, query_count=4, key_count=3, head_dim=4,
                   causal=True)
    assert "invalid attention shape" in e.value.message
    with pytest.raises(AnimaError) as e:
        ex.execute(query=buf, key=buf, value=buf, output=buf, heads=4, query_count=8, key_count=8, head_dim=8)
    assert e.value.status == animaxs_amd._abi.E_OUT_OF_BOUNDS


@pytest.mark.parametrize("Tq,Tk", [(300, 512), (77, 200), (256, 256)])
def test_llm_adapter_attention_head_dim_64_separate_key_rope(ctx, Tq, Tk):
    """LLM-adapter attention (LLMAdapterMetal.swift:360-405, rms_rope_adapter64
    AnimaKernels.metal:733-763): 16 heads x head_dim 64 over hidden 1024, per-head RMSNorm with
    weights per side, and RoPE theta 1e4 over 32 pairs where the queries (target tokens) use the
    target table and the keys (context tokens, a different count) their own context table --
    the K-side table of the prologue.  Token-major [tokens, 1024] rows, no transposes."""
    H, D = 16, 64
    g = torch.Generator().manual_seed(Tq * 1000 + Tk)
    q = (torch.randn(1, Tq, H, D, generator=g) * 2).half()
    k = (torch.randn(1, Tk, H, D, generator=g) * 2).half()
    v = torch.randn(1, Tk, H, D, generator=g).half()
    qw = (torch.rand(D, generator=g) * 0.4 + 0.8).half()
    kw = (torch.rand(D, generator=g) * 0.4 + 0.8).half()
    rq = orope.neox_rope_table(Tq, 1.0e4, head_dim=D)
    rk = orope.neox_rope_table(Tk, 1.0e4, head_dim=D)
    lib_rq = animaxs_amd.qwen_rope(Tq, head_dim=D, theta=1.0e4)   # the library's own table builder
    assert np.abs(lib_rq - rq.numpy()).max() < 2e-6
    pro = QKPrologue(dev(qw), dev(kw), 1e-6, dev(rq), Tq, True, True, k_rope=dev(rk), k_rope_tokens=Tk)
    print(f"ADAPTER Tq={Tq} Tk={Tk}", flush=True)
    o = _run(ctx, dev(q), dev(k), dev(v), layout=("tokenMajor", H * D), heads=H, Sq=Tq, Sk=Tk, D=D,
             out_shape=(1, Tq, H, D), prologue=pro)
    ref = oatt.sdpa(oatt.qk_prologue(q, qw, 1e-6, rq).half().float(), oatt.qk_prologue(k, kw, 1e-6, rk).half().float(), v)
    assert_attention_close(o, ref, label=f"adapter D64 Tq{Tq} Tk{Tk}")


# ---------------------------------------------------------------------------
# Head dim 384: the VAE decoder's mid-block attention (VAEDecoder.swift:396-404): one head,
# Q/K/V contiguous [positions, 384] blocks, 4096 positions at the 64x64 latent.
# ---------------------------------------------------------------------------
def test_vae_attention_head_dim_384_matches_oracle(ctx):
    S, D = 4096, 384
    g = torch.Generator().manual_seed(384)
    q = torch.randn(S, D, generator=g).half()
    k = torch.randn(S, D, generator=g).half()
    v = torch.randn(S, D, generator=g).half()
    print("VAE attention D384 S4096", flush=True)
    o = _run(ctx, dev(q), dev(k), dev(v), layout="headMajor", heads=1, Sq=S, Sk=S, D=D, out_shape=(S, D))
    ref = oatt.sdpa(q[None, :, None, :], k[None, :, None, :], v[None, :, None, :])[0, :, 0, :]
    assert_attention_close(o, ref, label="VAE D384 S4096 (wide flash, 8 key splits)")
    # the generic kernel, which the reference's shape used before, agrees to the same bar
    og = _run(ctx, dev(q), dev(k), dev(v), layout="headMajor", heads=1, Sq=S, Sk=S, D=D, out_shape=(S, D),
              backend="generic")
    assert_attention_close(og, ref, label="VAE D384 S4096 generic")


@pytest.mark.parametrize("B,H,Sq,Sk,causal,lengths", [(1, 1, 300, 777, False, None), (2, 2, 129, 64, False, None),
                                                      (1, 3, 260, 260, True, None), (2, 1, 200, 450, False, [37, 450]),
                                                      (1, 1, 1, 33, False, None), (1, 2, 5000, 40, False, None),
                                                      (1, 1, 128, 2049, False, None)])
def test_wide_flash_head_dim_384_ragged(ctx, B, H, Sq, Sk, causal, lengths):
    """Ragged tiles, batch and heads, causal rows, per-sequence key lengths (no key splits) and the
    split path (128 x 2049: 4 splits of 576 keys, the last one ragged; 300 x 777 is too short to
    split); large logits so the lazy running max must rescale."""
    D = 384
    g = torch.Generator().manual_seed(B * 100000 + H * 10000 + Sq + Sk)
    q = (torch.randn(B, Sq, H, D, generator=g) * 4.0).half()    # logits ~N(0, 16^2): the running max
    k = (torch.randn(B, Sk, H, D, generator=g) * 4.0).half()    # grows past the lazy bound
    v = torch.randn(B, Sk, H, D, generator=g).half()
    kw = {}
    if lengths is not None:
        kw["key_lengths"] = np.array(lengths, np.int32)
    print(f"WIDE D384 B{B} H{H} Sq{Sq} Sk{Sk} causal={causal} lengths={lengths}", flush=True)
    o = _run(ctx, dev(q), dev(k), dev(v), layout=("tokenMajor", H * D), heads=H, Sq=Sq, Sk=Sk, D=D,
             out_shape=(B, Sq, H, D), batch=B, causal=causal, backend="flash", **kw)
    ref = oatt.sdpa(q, k, v, causal=causal, key_lengths=lengths)
    assert_attention_close(o, ref, label=f"wide D384 B{B} H{H} Sq{Sq} Sk{Sk} causal={causal}")


@pytest.mark.parametrize("B,H,Hkv,Sq,Sk,causal,lengths", [(1, 4, 2, 256, 1100, False, None),
                                                          (2, 4, 1, 130, 300, False, [300, 77]),
                                                          (1, 2, 1, 200, 200, True, None)])
def test_wide_flash_head_dim_384_grouped_kv_heads(ctx, B, H, Hkv, Sq, Sk, causal, lengths):
    """Head dim 384 with fewer K/V heads than query heads (head h reads K/V head h / (H / Hkv)):
    K/V in their own token-major rows of Hkv * 384 halfs.  1 x 4/2 x 256 x 1100 splits the keys
    (2 splits, the last one ragged); the others run unsplit with key lengths or causal rows."""
    D = 384
    g = torch.Generator().manual_seed(B * 1000 + H * 100 + Hkv * 10 + Sq + Sk)
    q = (torch.randn(B, Sq, H, D, generator=g) * 2.0).half()
    k = (torch.randn(B, Sk, Hkv, D, generator=g) * 2.0).half()
    v = torch.randn(B, Sk, Hkv, D, generator=g).half()
    kw = {}
    if lengths is not None:
        kw["key_lengths"] = np.array(lengths, np.int32)
    print(f"WIDE GQA D384 B{B} H{H}/{Hkv} Sq{Sq} Sk{Sk} causal={causal} lengths={lengths}", flush=True)
    o = _run(ctx, dev(q), dev(k), dev(v), layout=("tokenMajor", H * D), heads=H, Sq=Sq, Sk=Sk, D=D,
             out_shape=(B, Sq, H, D), batch=B, causal=causal, backend="flash", key_value_heads=Hkv,
             kv_token_stride=Hkv * D, **kw)
    ref = oatt.sdpa(q, k, v, causal=causal, key_lengths=lengths)
    assert_attention_close(o, ref, label=f"wide GQA D384 B{B} H{H}/{Hkv} Sq{Sq} Sk{Sk} causal={causal}")


# ---------------------------------------------------------------------------
# The MPS-rounding backend (legacyHeadMajorMPS / stridedTokenMajorMPS under legacy numerics,
# AttentionExecutor.swift:221-301, 412-496): fp16 scaled scores and fp16 normalised
# probabilities, against the oracle's legacy mode (scripts/dit_block0_oracle.py:135-141).
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("case", ["head_major_gqa_causal_lengths", "token_major_norm_rope", "hd64"])
def test_legacy_mps_backend_matches_legacy_oracle(ctx, case):
    g = torch.Generator().manual_seed({"head_major_gqa_causal_lengths": 41, "token_major_norm_rope": 42, "hd64": 43}[case])
    kw = {}
    if case == "head_major_gqa_causal_lengths":
        B, H, Hkv, S, D = 2, 4, 2, 200, 128
        q = (torch.randn(B, H, S, D, generator=g) * 2).half()
        k = (torch.randn(B, Hkv, S, D, generator=g) * 2).half()
        v = torch.randn(B, Hkv, S, D, generator=g).half()
        L = [200, 71]
        o = _run(ctx, dev(q), dev(k), dev(v), layout="headMajor", heads=H, Sq=S, Sk=S, D=D,
                 out_shape=(B, H, S, D), backend="legacyMPS", batch=B, key_value_heads=Hkv, causal=True,
                 key_lengths=L).permute(0, 2, 1, 3)
        qq, kk, vv = (t.permute(0, 2, 1, 3) for t in (q, k, v))
        kw = dict(causal=True, key_lengths=L)
    elif case == "token_major_norm_rope":
        d = inputs.self_attention(2, S=256)
        pro = QKPrologue(dev(d["q_norm_w"]), dev(d["k_norm_w"]), d["eps"], dev(d["rope"]), 256, True, True)
        o = _run(ctx, dev(d["q"]), dev(d["k"]), dev(d["v"]), layout=("tokenMajor", 2048), heads=16, Sq=256,
                 Sk=256, D=128, out_shape=(1, 256, 16, 128), backend="stridedTokenMajorMPS", prologue=pro)
        qq = oatt.qk_prologue(d["q"], d["q_norm_w"], d["eps"], d["rope"]).half()
        kk = oatt.qk_prologue(d["k"], d["k_norm_w"], d["eps"], d["rope"]).half()
        vv = d["v"]
    else:
        B, H, Sq, Sk, D = 1, 3, 77, 300, 64
        q = (torch.randn(B, Sq, H, D, generator=g) * 2).half()
        k = (torch.randn(B, Sk, H, D, generator=g) * 2).half()
        v = torch.randn(B, Sk, H, D, generator=g).half()
        o = _run(ctx, dev(q), dev(k), dev(v), layout=("tokenMajor", H * D), heads=H, Sq=Sq, Sk=Sk, D=D,
                 out_shape=(B, Sq, H, D), backend="legacyHeadMajorMPS", batch=B)
        qq, kk, vv = q, k, v
    print(f"LEGACY MPS {case}", flush=True)
    ref_legacy = oatt.sdpa(qq, kk, vv, legacy=True, **kw)
    ref_fp32 = oatt.sdpa(qq, kk, vv, **kw)
    # Legacy numerics are by design less accurate than fp32 scores: against the fp32 oracle the
    # kernel may be as far as the legacy oracle is, plus its fp16 output rounding.
    gap = float((ref_legacy - ref_fp32).abs().sum() / ref_fp32.abs().sum())
    assert_attention_close(o, ref_fp32, mean_rel_tol=gap + 3e-4, label=f"legacy MPS {case} vs fp32 oracle")
    # The same rounding points as the legacy oracle (whose output, like the kernel's, is
    # stored as fp16): far closer to it than the two oracles are to each other (they differ
    # only by those roundings).
    assert_attention_close(o, ref_legacy.half(), max_abs_tol=2e-3, mean_rel_tol=min(1e-4, 0.25 * gap),
                           label=f"legacy MPS {case} vs fp16 legacy oracle (oracle gap {gap:.2e})")
