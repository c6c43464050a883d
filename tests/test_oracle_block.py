"""CPU: wiring invariants of the DiT block and Qwen layer composition oracles (oracle.blocks.dit_block,
following scripts/dit_block0_oracle.py:327-391) on a 16-token grid.  Each part it composes
is pinned in test_oracle_attention.py / test_oracle_rope.py / test_oracle_quant.py."""

from __future__ import annotations

import pytest
import torch

from oracle import blocks, inputs


@pytest.fixture(scope="module")
def small_block():
    d = inputs.dit_block(S=16, ctx_tokens=8)
    return d, blocks.dequant_weights(d)


def _with(d, **over):
    e = dict(d)
    e.update(over)
    return e


def test_zero_gates_leave_the_residual_unchanged(small_block):
    d, W = small_block
    dim = d["x"].shape[1]
    # modulation = SiLU(emb) W1^T W2^T + adaln: zero W2 and adaln -> shift = scale = gate = 0
    zero = {f"mod_{br}_w2": torch.zeros_like(d[f"mod_{br}_w2"]) for br in ("self", "cross", "mlp")}
    e = _with(d, adaln=torch.zeros(3 * dim), **zero)
    out = blocks.dit_block(e, weights=W)
    assert torch.equal(out, d["x"].float())


def test_branches_add_in_order(small_block):
    """x1 = x + g_self * self_branch; zeroing self_o removes exactly that branch."""
    d, W = small_block
    out, inter = blocks.dit_block(d, weights=W, return_intermediates=True)
    W0 = dict(W)
    W0["self_o"] = torch.zeros_like(W["self_o"])
    _, inter0 = blocks.dit_block(d, weights=W0, return_intermediates=True)
    assert torch.equal(inter0["x1"], d["x"].float())
    assert not torch.equal(inter["x1"], d["x"].float())
    assert torch.isfinite(out).all()


def test_modulation_chunks_shift_scale_gate(small_block):
    d, _ = small_block
    dim = d["x"].shape[1]
    adaln = torch.arange(3 * dim, dtype=torch.float32)
    z1 = torch.zeros_like(d["mod_self_w1"])
    sh, sc, ga = blocks.modulation(d["emb"], z1, d["mod_self_w2"], adaln)
    assert torch.equal(sh, adaln[:dim]) and torch.equal(sc, adaln[dim:2 * dim]) and torch.equal(ga, adaln[2 * dim:])


# --------------------------------------------------------------------------------------
# Qwen layer composition oracle (oracle.blocks.qwen_layer, QwenEncoderMetal.swift:244-303).
# --------------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def small_qwen():
    d = inputs.qwen_layer(B=2, S=12, hidden=256, heads=4, kv_heads=2, intermediate=384)
    d["key_lengths"] = torch.tensor([12, 7], dtype=torch.int32)
    return d, blocks.dequant_weights(d)


def test_qwen_zero_output_projections_leave_the_residual_unchanged(small_qwen):
    d, W = small_qwen
    W0 = dict(W)
    W0["o"] = torch.zeros_like(W["o"])
    W0["down"] = torch.zeros_like(W["down"])
    assert torch.equal(blocks.qwen_layer(d, weights=W0), d["x"].float())
    W1 = dict(W)
    W1["down"] = torch.zeros_like(W["down"])
    out1, inter1 = blocks.qwen_layer(d, weights=W1, return_intermediates=True)
    assert torch.equal(out1, inter1["x1"]) and not torch.equal(out1, d["x"].float())


def test_qwen_first_token_attends_only_to_itself_through_the_gqa_map(small_qwen):
    """Causal: query 0 sees key 0 only, so its attention output is V of token 0, and head h
    reads kv head h // (heads / kv_heads) (GqaHeadMappingTests.swift:17-36)."""
    d, W = small_qwen
    _, inter = blocks.qwen_layer(d, weights=W, return_intermediates=True)
    n = blocks.rms_norm(d["x"].float(), d["input_norm"], d["eps"]).half().float()
    v = (n @ W["v"].T).half().float()                     # [B, S, kv_heads * 128]
    H, Hkv = d["heads"], d["kv_heads"]
    for b in range(d["x"].shape[0]):
        for h in range(H):
            kv = h // (H // Hkv)
            got = inter["attention"][b, 0, h * 128:(h + 1) * 128]
            assert torch.equal(got, v[b, 0, kv * 128:(kv + 1) * 128].half().float())


def test_qwen_causality_and_padding_mask(small_qwen):
    """Changing tokens after t leaves rows <= t unchanged; changing padded tokens (>= L_b)
    leaves every valid row unchanged."""
    d, W = small_qwen
    base = blocks.qwen_layer(d, weights=W)
    x2 = d["x"].clone()
    x2[:, 5:] += 3.0
    e = dict(d); e["x"] = x2
    out = blocks.qwen_layer(e, weights=W)
    assert torch.equal(out[:, :5], base[:, :5]) and not torch.equal(out[:, 5:], base[:, 5:])
    L = int(d["key_lengths"][1])
    x3 = d["x"].clone()
    x3[1, L:] = -2.0
    e = dict(d); e["x"] = x3
    out = blocks.qwen_layer(e, weights=W)
    assert torch.equal(out[1, :L], base[1, :L]) and torch.equal(out[0], base[0])


def test_qwen_sequences_are_independent(small_qwen):
    d, W = small_qwen
    base = blocks.qwen_layer(d, weights=W)
    e = dict(d)
    e["x"] = d["x"].flip(0).contiguous()
    e["key_lengths"] = d["key_lengths"].flip(0).contiguous()
    assert torch.equal(blocks.qwen_layer(e, weights=W), base.flip(0))
