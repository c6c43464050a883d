"""CPU: the attention oracle against fp64 brute force, the special cases of the
reference's tests (AttentionExecutorTests.swift, GqaHeadMappingTests.swift,
DiTBlockTests.swift) and the masked-mode equivalence of scripts/qwen_comfy_oracle.py.
No GPU needed."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import inputs


def brute_force(q, k, v, scale=None, causal=False, key_lengths=None):
    """Plain fp64 loops over (b, h, i): scores, masked keys removed, softmax, weighted sum."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    B, Sq, H, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    rep = H // Hkv
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    out = np.zeros((B, Sq, H, D))
    for b in range(B):
        L = Sk if key_lengths is None else int(key_lengths[b])
        for h in range(H):
            kh = h // rep
            for i in range(Sq):
                keys = [j for j in range(L) if not (causal and j > i)]
                s = np.array([scale * float(q[b, i, h] @ k[b, j, kh]) for j in keys])
                p = np.exp(s - s.max())
                p /= p.sum()
                out[b, i, h] = sum(p[n] * v[b, j, kh] for n, j in enumerate(keys))
    return out


def rnd(g, *shape, std=1.0):
    return (torch.randn(*shape, generator=g) * std).half()


@pytest.mark.parametrize("B,Sq,Sk,H,Hkv,D", [(1, 5, 7, 2, 2, 8), (2, 9, 4, 4, 2, 16), (1, 3, 11, 6, 1, 4)])
def test_sdpa_brute_force(B, Sq, Sk, H, Hkv, D):
    g = torch.Generator().manual_seed(B * 100 + Sq)
    q, k, v = rnd(g, B, Sq, H, D, std=2.0), rnd(g, B, Sk, Hkv, D, std=2.0), rnd(g, B, Sk, Hkv, D)
    want = brute_force(q.numpy(), k.numpy(), v.numpy())
    got = A.sdpa(q, k, v).numpy()
    assert np.max(np.abs(got - want)) <= 2e-6


def test_sdpa_brute_force_masked_and_causal():
    g = torch.Generator().manual_seed(5)
    B, S, H, Hkv, D = 3, 12, 4, 2, 8
    q, k, v = rnd(g, B, S, H, D, std=3.0), rnd(g, B, S, Hkv, D, std=3.0), rnd(g, B, S, Hkv, D)
    L = [12, 5, 1]
    for causal in (False, True):
        want = brute_force(q.numpy(), k.numpy(), v.numpy(), causal=causal, key_lengths=L)
        got = A.sdpa(q, k, v, causal=causal, key_lengths=L).numpy()
        assert np.max(np.abs(got - want)) <= 2e-6, causal


def test_scale_argument():
    g = torch.Generator().manual_seed(6)
    q, k, v = rnd(g, 1, 4, 1, 8), rnd(g, 1, 6, 1, 8), rnd(g, 1, 6, 1, 8)
    want = brute_force(q.numpy(), k.numpy(), v.numpy(), scale=0.37)
    assert np.max(np.abs(A.sdpa(q, k, v, scale=0.37).numpy() - want)) <= 2e-6


def test_zero_qk_gives_mean_of_v():
    # AttentionExecutorTests.swift:460-504: zero Q and K -> uniform weights -> mean of V
    g = torch.Generator().manual_seed(7)
    q = torch.zeros(1, 130, 2, 8, dtype=torch.half)
    k = torch.zeros(1, 64, 1, 8, dtype=torch.half)
    v = rnd(g, 1, 64, 1, 8)
    out = A.sdpa(q, k, v)
    mean = v.float().mean(dim=1, keepdim=True)      # [1, 1, 1, 8]
    assert torch.allclose(out, mean.expand_as(out), atol=1e-6)


def test_last_value_row_case():
    # AttentionExecutorTests.swift:64-88: Q=129, K=512, only the last V row is nonzero
    # (column c holds c+1) -> every output row is (c+1)/512
    q = torch.zeros(1, 129, 1, 64, dtype=torch.half)
    k = torch.zeros(1, 512, 1, 64, dtype=torch.half)
    v = torch.zeros(1, 512, 1, 64, dtype=torch.half)
    v[0, 511, 0] = torch.arange(1, 65, dtype=torch.half)
    out = A.sdpa(q, k, v)
    want = (torch.arange(1, 65, dtype=torch.float32) / 512)
    assert torch.allclose(out[0, :, 0], want.expand(129, 64), atol=1e-6)


def test_gqa_contiguous_kv_heads():
    # AttentionExecutorTests.swift:90-111 and GqaHeadMappingTests.swift:23-89:
    # 4 query heads over 2 kv heads map 0,0,1,1
    q = torch.zeros(1, 1, 4, 4, dtype=torch.half)
    k = torch.zeros(1, 1, 2, 4, dtype=torch.half)
    v = torch.stack([torch.full((4,), 2.0), torch.full((4,), 9.0)]).half().reshape(1, 1, 2, 4)
    out = A.sdpa(q, k, v)[0, 0]
    assert out.tolist() == [[2.0] * 4, [2.0] * 4, [9.0] * 4, [9.0] * 4]
    # a distinguishable case: head h must read kv head h // 2, never h % 2
    g = torch.Generator().manual_seed(8)
    q, k, v = rnd(g, 1, 3, 4, 8), rnd(g, 1, 5, 2, 8), rnd(g, 1, 5, 2, 8)
    out = A.sdpa(q, k, v)
    for h in range(4):
        one = A.sdpa(q[:, :, h:h + 1], k[:, :, h // 2:h // 2 + 1], v[:, :, h // 2:h // 2 + 1])
        assert torch.allclose(out[:, :, h:h + 1], one, atol=1e-7)


def test_tiny_scale_and_softmax_case():
    # DiTBlockTests.swift:117-147: 2 queries x 3 keys, head_dim 4
    q = torch.tensor([[1, 0, 0, 0], [0, 1, 0, 0]], dtype=torch.float32).reshape(1, 2, 1, 4)
    k = torch.tensor([[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0]], dtype=torch.float32).reshape(1, 3, 1, 4)
    v = torch.tensor([[10, 20, 30, 40], [50, 60, 70, 80], [90, 100, 110, 120]],
                     dtype=torch.float32).reshape(1, 3, 1, 4)
    out = A.sdpa(q, k, v)[0, :, 0]
    e = math.exp(0.5)
    w_hit, w_miss = e / (e + 2), 1 / (e + 2)
    vv = v[0, :, 0].double()
    want0 = w_hit * vv[0] + w_miss * (vv[1] + vv[2])
    want1 = w_hit * vv[1] + w_miss * (vv[0] + vv[2])
    assert torch.allclose(out[0].double(), want0, atol=1e-4)
    assert torch.allclose(out[1].double(), want1, atol=1e-4)


def test_additive_mask_equals_dropping_keys():
    """scripts/qwen_comfy_oracle.py:233-248 adds finfo.min/4; with at least one valid key
    per row this equals removing the masked keys (exp underflows to exactly 0; only the
    summation order of the library matmul differs)."""
    g = torch.Generator().manual_seed(9)
    q, k, v = rnd(g, 1, 6, 2, 8, std=4.0), rnd(g, 1, 10, 2, 8, std=4.0), rnd(g, 1, 10, 2, 8)
    masked = A.sdpa(q, k, v, key_lengths=[4])
    dropped = A.sdpa(q, k[:, :4], v[:, :4])
    assert torch.allclose(masked, dropped, atol=1e-6, rtol=0)


def test_qk_prologue_matches_parts():
    from oracle import norms, rope
    g = torch.Generator().manual_seed(10)
    x = rnd(g, 1, 16, 2, 128)
    w = rnd(g, 128)
    t = rope.dit_rope_table(1, 4, 4)
    got = A.qk_prologue(x, w, 1e-6, t)
    want = rope.apply_split_half(norms.rms_norm(x, w, 1e-6), t)
    assert torch.equal(got, want)


def test_attention_flops_counts():
    assert A.attention_flops(1, 16, 4096, 4096, 128) == 4.0 * 128 * 16 * 4096 * 4096
    # causal with key mask: row i sees min(i+1, L) keys
    assert A.attention_flops(1, 1, 4, 4, 2, causal=True, key_lengths=[2]) == 4.0 * 2 * (1 + 2 + 2 + 2)


def test_generators_are_seeded_and_shaped():
    a = inputs.self_attention(1, S=64)
    b = inputs.self_attention(1, S=64)
    for key in a:
        if isinstance(a[key], torch.Tensor):
            assert torch.equal(a[key], b[key]), key
    assert a["q"].shape == (1, 64, 16, 128) and a["q"].dtype == torch.float16


# --------------------------------------------------------------------------------------
# Legacy rounding (scripts/dit_block0_oracle.py:135-141; the MPS backends' fp16 score and
# probability matrices, AnimaKernels.metal:1051-1100).
# --------------------------------------------------------------------------------------

def test_legacy_uniform_weights_round_to_fp16():
    """Q = K = 0 over 3 keys: every score is 0 and every probability 1/3, stored as the fp16
    0.333251953125 (= 1365 / 4096), so the output is 1365/4096 * (v0 + v1 + v2) rather than
    the mean.  Over 64 keys 1/64 is exact and legacy equals the mean of V."""
    g = torch.Generator().manual_seed(21)
    q = torch.zeros(1, 2, 1, 8, dtype=torch.half)
    k = torch.zeros(1, 3, 1, 8, dtype=torch.half)
    v = rnd(g, 1, 3, 1, 8, std=4.0)
    got = A.sdpa(q, k, v, legacy=True)[0, :, 0].double()
    want = (1365.0 / 4096.0) * v[0, :, 0].double().sum(0)
    assert torch.allclose(got, want.expand_as(got), rtol=0, atol=1e-5)
    assert not torch.allclose(got, v[0, :, 0].double().mean(0).expand_as(got), rtol=0, atol=1e-4)
    k64 = torch.zeros(1, 64, 1, 8, dtype=torch.half)
    v64 = rnd(g, 1, 64, 1, 8)
    mean = v64.float().mean(dim=1, keepdim=True)
    assert torch.allclose(A.sdpa(q, k64, v64, legacy=True), mean.expand(1, 2, 1, 8), atol=1e-6)


def test_legacy_two_key_closed_form():
    """One query, two keys, scale 1.  Scores 1 + 2^-12 and 0: fp16 stores the first as 1
    (spacing 2^-10 at 1), so the weights are fp16(sigmoid(1)) = 0.73095703125 and
    fp16(sigmoid(-1)) = 0.26904296875, against the fp32 oracle's sigmoid(1 + 2^-12)."""
    D = 8
    q = torch.zeros(1, 1, 1, D)
    q[0, 0, 0, 0] = 1.0
    k = torch.zeros(1, 2, 1, D)
    k[0, 0, 0, 0] = 1.0 + 2.0 ** -12
    v = torch.zeros(1, 2, 1, D)
    v[0, 0, 0, :] = 1.0
    v[0, 1, 0, :] = -3.0
    p0 = float(np.float16(1.0 / (1.0 + math.exp(-1.0))))
    p1 = float(np.float16(1.0 / (1.0 + math.exp(1.0))))
    assert (p0, p1) == (0.73095703125, 0.26904296875)
    got = A.sdpa(q, k, v, scale=1.0, legacy=True)[0, 0, 0].double()
    assert torch.allclose(got, torch.full((D,), p0 * 1.0 + p1 * -3.0, dtype=torch.float64), rtol=0, atol=1e-6)
    s = 1.0 + 2.0 ** -12
    w = 1.0 / (1.0 + math.exp(-s))
    fp32 = A.sdpa(q, k, v, scale=1.0)[0, 0, 0].double()
    assert torch.allclose(fp32, torch.full((D,), w - 3.0 * (1 - w), dtype=torch.float64), rtol=0, atol=1e-6)
    assert float((got - fp32).abs().max()) > 1e-4


def test_legacy_stays_near_fp32_and_keeps_masks():
    """On random inputs legacy differs from fp32 only by the fp16 roundings (a few 1e-4
    relative), and causal / key-length masking behaves as in fp32 (masked keys get weight 0)."""
    g = torch.Generator().manual_seed(22)
    B, S, H, Hkv, D = 2, 9, 4, 2, 16
    q, k, v = rnd(g, B, S, H, D, std=2.0), rnd(g, B, S, Hkv, D, std=2.0), rnd(g, B, S, Hkv, D)
    for causal, L in ((False, None), (True, [9, 4])):
        lg = A.sdpa(q, k, v, causal=causal, key_lengths=L, legacy=True)
        fp = A.sdpa(q, k, v, causal=causal, key_lengths=L)
        rel = float((lg - fp).abs().sum() / fp.abs().sum())
        assert 1e-6 < rel < 3e-3, rel
    lg = A.sdpa(q, k, v, key_lengths=[4, 4], legacy=True)
    assert torch.equal(lg, A.sdpa(q, k[:, :4], v[:, :4], legacy=True))
