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


# --------------------------------------------------------------------------------------
# Closed-form DiT block cases.  W4 code 8 decodes to 0 and code 9 to `scale` when
# zero = -8*scale (AnimaKernels.metal:19-41), so with scale 1 a code matrix of 8s with 9s
# on a diagonal is an exact identity projection and all 8s an exact zero projection.
# With those projections the block reduces to closed forms that are written out below
# independently of oracle.blocks; each case is built so that a plausible wiring mistake
# (shift/scale swapped at the LN-modulate call, a branch reading another branch's gate
# row, the branches in the wrong order, cross K/V projected from x, RoPE missing on Q or
# on K) changes the result by far more than the tolerance.
# --------------------------------------------------------------------------------------

import math  # noqa: E402

import numpy as np  # noqa: E402

from oracle.quant import pack_w4  # noqa: E402

DIM, HD, NH = 2048, 128, 16


def _w4_from_codes(q: np.ndarray, scale: float = 1.0) -> dict:
    rows, cols = q.shape
    groups = (cols + 63) // 64
    s = np.full((rows, groups), scale, np.float16)
    z = (s.astype(np.float32) * -8.0).astype(np.float16)
    return {"storage": 0, "rows": rows, "cols": cols, "row_stride": (cols + 1) // 2,
            "packed": pack_w4(q.astype(np.uint8)), "scale_bits": s.view(np.uint16), "zero_bits": z.view(np.uint16)}


def _identity(rows: int, cols: int, col_of_row=None) -> dict:
    q = np.full((rows, cols), 8, np.uint8)
    r = np.arange(rows)
    c = r if col_of_row is None else col_of_row(r)
    keep = c < cols
    q[r[keep], c[keep]] = 9
    return _w4_from_codes(q)


def _zero(rows: int, cols: int) -> dict:
    return _w4_from_codes(np.full((rows, cols), 8, np.uint8))


def _h(a):
    """fp16 boundary (where the block stores fp16 activations)."""
    return torch.as_tensor(a).float().half().float()


def _ln_mod(x, scale, shift, eps=1e-6):
    x = x.double()
    mu = x.mean(-1, keepdim=True)
    var = ((x - mu) ** 2).mean(-1, keepdim=True)
    return ((x - mu) / torch.sqrt(var + eps) * (1 + scale.double()) + shift.double()).float()


def _gelu(x):
    x = x.double()
    return (0.5 * x * (1 + torch.erf(x / math.sqrt(2.0)))).float()


def _identity_block(S: int, T: int, **w_over):
    d = inputs.dit_block(S=S, ctx_tokens=T, hidden=DIM)
    w = {n: _zero(*((DIM, 1024) if n in ("cross_k", "cross_v") else (DIM, DIM)))
         for n in ("self_q", "self_k", "cross_q", "cross_k")}
    w.update(self_v=_identity(DIM, DIM), self_o=_identity(DIM, DIM), cross_v=_identity(DIM, 1024),
             cross_o=_identity(DIM, DIM), mlp1=_identity(DIM, DIM), mlp2=_identity(DIM, DIM))
    w.update(w_over)
    d["w"] = w
    return d


def _mods(d):
    out = {}
    for br in ("self", "cross", "mlp"):
        out[br] = blocks.modulation(d["emb"], d[f"mod_{br}_w1"], d[f"mod_{br}_w2"], d["adaln"])
    return out


def test_block_closed_form_identity_projections():
    """Q = K = 0 makes every attention uniform, so with identity V/O/MLP projections:
        n1 = h(LN(x)(1+sc1)+sh1);  x1 = x  + g1 * h(mean_t n1)
        n2 = h(LN(x1)(1+sc2)+sh2); x2 = x1 + g2 * h(mean_j [ctx_j, 0])   (V from the context)
        n3 = h(LN(x2)(1+sc3)+sh3); x3 = x2 + g3 * h(gelu(n3))
    with (sh_b, sc_b, g_b) the three chunks of branch b's modulation (chunk order pinned by
    test_modulation_chunks_shift_scale_gate)."""
    S, T = 16, 8
    d = _identity_block(S, T)
    # give the branches clearly different modulations
    g = torch.Generator().manual_seed(77)
    for br, amp in (("self", 1.0), ("cross", 2.0), ("mlp", 3.0)):
        d[f"mod_{br}_w2"] = (torch.randn(3 * DIM, 256, generator=g) * 0.05 * amp).half()
    m = _mods(d)
    x = d["x"].float()
    ctx = d["ctx"].float()
    (sh1, sc1, g1), (sh2, sc2, g2), (sh3, sc3, g3) = m["self"], m["cross"], m["mlp"]
    n1 = _h(_ln_mod(x, sc1, sh1))
    x1 = x + g1 * _h(n1.double().mean(0).float())
    n2 = _h(_ln_mod(x1, sc2, sh2))
    vpad = torch.cat([ctx, torch.zeros(T, DIM - 1024)], 1)
    x2 = x1 + g2 * _h(vpad.double().mean(0).float())
    n3 = _h(_ln_mod(x2, sc3, sh3))
    x3 = x2 + g3 * _h(_gelu(n3))

    out, inter = blocks.dit_block(d, return_intermediates=True)
    tol = lambda ref: 2e-3 * float(ref.abs().max()) + 1e-4  # noqa: E731  (fp16 boundary ties)
    assert float((inter["x1"] - x1).abs().max()) <= tol(x1)
    assert float((inter["x2"] - x2).abs().max()) <= tol(x2)
    assert float((out - x3).abs().max()) <= tol(x3)

    # The closed form separates the mistakes it is meant to catch.
    def far(a, b):
        return float((a - b).abs().max()) > 50 * tol(b)
    assert far(x + g1 * _h(_h(_ln_mod(x, sh1, sc1)).double().mean(0).float()), x1)   # shift/scale swapped
    assert far(x + g2 * _h(n1.double().mean(0).float()), x1)                          # self uses cross's gate
    assert far(x2 + g1 * _h(_gelu(n3)), x3)                                           # MLP uses self's gate
    assert far(x1 + g2 * _h(n2.double().mean(0).float()), x2)                        # cross V from x, not context
    assert far(x + g2 * _h(vpad.double().mean(0).float()), x2)                        # cross reads x, not x1


def _rope_rotate(v, rope_row):
    """Split-half rotation of one head vector with one table row, fp64, by hand:
    out[p] = c*a - s*b, out[p+64] = s*a + c*b (rope_row[p] = [[c, -s], [s, c]])."""
    out = np.empty_like(v)
    for p in range(64):
        c, s = float(rope_row[p, 0, 0]), float(rope_row[p, 1, 0])
        a, b = v[p], v[p + 64]
        out[p] = c * a - s * b
        out[p + 64] = s * a + c * b
    return out


def test_block_closed_form_rope_changes_the_softmax():
    """2x2 grid.  Token rows share their first 1024 columns and permute their last 1024, so
    LayerNorm statistics (hence the first half of n1) are the same for every token.  Q and K
    both read the first half (heads 0-7 and 8-15 alike) through identity blocks, so Q = K is
    one vector for every token; V = n1 differs per token in heads 8-15.  Without RoPE every
    score is equal (uniform attention); with RoPE on Q only, a query row's scores are still
    equal; with RoPE on K only they differ from RoPE on both.  The expected self branch is an
    fp64 brute force with those roundings; cross and MLP gates are zeroed."""
    S, T = 4, 2
    first_half = lambda r: np.where(r < 1024, r, r - 1024)  # noqa: E731
    d = _identity_block(S, T, self_q=_identity(DIM, DIM, first_half), self_k=_identity(DIM, DIM, first_half))
    g = torch.Generator().manual_seed(5)
    A = torch.randn(1024, generator=g) * 2
    B = torch.randn(1024, generator=g) * 2
    x = torch.stack([torch.cat([A, B[torch.randperm(1024, generator=g)]]) for _ in range(S)])
    d["x"] = x
    d["self_q_norm"] = torch.ones(HD).half()
    d["self_k_norm"] = torch.ones(HD).half()
    for br in ("cross", "mlp"):
        w2 = d[f"mod_{br}_w2"].clone()
        w2[2 * DIM:] = 0
        d[f"mod_{br}_w2"] = w2
    d["adaln"] = torch.cat([d["adaln"][:2 * DIM], torch.zeros(DIM)])
    m = _mods(d)
    sh1, sc1, g1 = m["self"]
    assert float(m["cross"][2].abs().max()) == 0 and float(m["mlp"][2].abs().max()) == 0

    n1 = _h(_ln_mod(x, sc1, sh1)).double().numpy()              # [S, 2048]
    rope = d["rope"].double().numpy()                          # [4, 64, 2, 2]
    eps = d["eps"]

    def branch(rope_q: bool, rope_k: bool):
        out = np.zeros((S, DIM))
        for h in range(NH):
            src = n1[:, (h % 8) * HD:(h % 8 + 1) * HD]            # Q/K projection: first half
            qn = np.stack([_h(src[t] / np.sqrt((src[t] ** 2).mean() + eps)).double().numpy() for t in range(S)])
            q = np.stack([_h(_rope_rotate(qn[t], rope[t])).double().numpy() if rope_q else qn[t] for t in range(S)])
            k = np.stack([_h(_rope_rotate(qn[t], rope[t])).double().numpy() if rope_k else qn[t] for t in range(S)])
            v = n1[:, h * HD:(h + 1) * HD]
            for t in range(S):
                sc = np.array([q[t] @ k[j] for j in range(S)]) / math.sqrt(HD)
                p = np.exp(sc - sc.max())
                p /= p.sum()
                out[t, h * HD:(h + 1) * HD] = p @ v
        return x + g1 * _h(_h(torch.from_numpy(out).float()))      # attention output and O boundary

    want = branch(True, True) - x                                   # the self branch's contribution
    got = blocks.dit_block(d) - x
    tol = 2e-3 * float(want.abs().max())
    err = float((got - want).abs().max())
    assert err <= tol, (err, tol)
    for mistake in (branch(False, False), branch(True, False), branch(False, True)):
        gap = float((mistake - x - want).abs().max())
        assert gap > 10 * tol, (gap, tol)
