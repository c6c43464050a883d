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
    one vector for every token before the norms; V = n1 differs per token in heads 8-15.  The
    Q and K norm weights differ, so a self-attention Q normalised with the K weight (or the
    other way round) changes every score.  Without RoPE every score of a query row is equal
    (uniform attention); with RoPE on one side only they differ from RoPE on both.  The
    expected self branch is an fp64 brute force with those roundings; cross and MLP gates
    are zeroed."""
    S, T = 4, 2
    first_half = lambda r: np.where(r < 1024, r, r - 1024)  # noqa: E731
    d = _identity_block(S, T, self_q=_identity(DIM, DIM, first_half), self_k=_identity(DIM, DIM, first_half))
    g = torch.Generator().manual_seed(5)
    A = torch.randn(1024, generator=g) * 2
    B = torch.randn(1024, generator=g) * 2
    x = torch.stack([torch.cat([A, B[torch.randperm(1024, generator=g)]]) for _ in range(S)])
    d["x"] = x
    d["self_q_norm"] = (0.5 + torch.rand(HD, generator=g)).half()
    d["self_k_norm"] = (0.5 + torch.rand(HD, generator=g)).half()
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

    wq = d["self_q_norm"].double().numpy()
    wk = d["self_k_norm"].double().numpy()

    def branch(rope_q: bool, rope_k: bool, q_w=wq, k_w=wk):
        out = np.zeros((S, DIM))
        for h in range(NH):
            src = n1[:, (h % 8) * HD:(h % 8 + 1) * HD]            # Q/K projection: first half
            qn = np.stack([src[t] / np.sqrt((src[t] ** 2).mean() + eps) * q_w for t in range(S)])
            kn = np.stack([src[t] / np.sqrt((src[t] ** 2).mean() + eps) * k_w for t in range(S)])
            q = np.stack([_hv(_rope_rotate(qn[t], rope[t]) if rope_q else qn[t]) for t in range(S)])
            k = np.stack([_hv(_rope_rotate(kn[t], rope[t]) if rope_k else kn[t]) for t in range(S)])
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
    for mistake in (branch(False, False), branch(True, False), branch(False, True),
                    branch(True, True, q_w=wk), branch(True, True, k_w=wq)):
        gap = float((mistake - x - want).abs().max())
        assert gap > 10 * tol, (gap, tol)


# --------------------------------------------------------------------------------------
# Closed forms that pin the Q/K norm wiring of both blocks and the Qwen layer's SwiGLU and
# norm weights.  W8 codes with zero = -128*scale decode to (code - 128)*scale
# (AnimaKernels.metal:43-66), so with scale 1 code 128 is an exact 0, 129 an exact 1 and
# 130 an exact 2: diagonal code matrices are exact identity / doubling projections.  The
# expected values are fp64 brute force over plain loops with the fp16 roundings at the
# places the reference stores fp16 (QwenEncoderMetal.swift:244-303,
# DiTBlockExecutor.swift:1035-1242).
# --------------------------------------------------------------------------------------

def _w8_diag(rows: int, cols: int, code: int = 129, col_of_row=None) -> dict:
    q = np.full((rows, cols), 128, np.uint8)
    r = np.arange(rows)
    c = r if col_of_row is None else col_of_row(r)
    keep = c < cols
    q[r[keep], c[keep]] = code
    groups = (cols + 63) // 64
    s = np.ones((rows, groups), np.float16)
    z = np.full((rows, groups), -128.0, np.float16)
    return {"storage": 1, "rows": rows, "cols": cols, "row_stride": cols,
            "packed": q.reshape(-1), "scale_bits": s.view(np.uint16), "zero_bits": z.view(np.uint16)}


def _hv(a):
    """fp16 rounding of an fp64 numpy array, back to fp64."""
    return np.asarray(a, np.float64).astype(np.float16).astype(np.float64)


def _rms64(v, w, eps):
    v = np.asarray(v, np.float64)
    return v / math.sqrt(float((v * v).mean()) + eps) * np.asarray(w, np.float64)


def _softmax_rows(scores):
    p = np.exp(scores - scores.max())
    return p / p.sum()


def test_qwen_closed_form_norm_weights_rope_and_swiglu():
    """B1 S5 (key length 4), hidden 256, 2 query heads on 1 KV head, W8 identity projections:
        n1 = h(rms(x) * 3);  q_h = n1[128h:128h+128], k = n1[0:128], v = n1[128:256]
        q_h' = h(rope_t(rms(q_h) * wq)), k' = h(rope_t(rms(k) * wk))    (distinct wq, wk)
        a_h(t) = h(sum_{j<=t, j<4} softmax_j(q_h'(t).k'(j)/sqrt(128)) v(j))
        x1 = x + h(a);  n2 = h(rms(x1) * 0.5);  x2 = x1 + h(h(silu(n2) * h(2 n2)))
    (gate = identity, up = 2 x identity, down = identity).  A dropped Q or K norm, a Q/K
    norm weight swap, RoPE missing on Q or K, the input-norm weight in the post-attention
    norm, gate and up swapped in the SwiGLU and a missing causal mask each move the result
    by far more than the tolerance."""
    B, S, hidden, H, Hkv, I, L = 1, 5, 256, 2, 1, 256, 4
    d = inputs.qwen_layer(B=B, S=S, hidden=hidden, heads=H, kv_heads=Hkv, intermediate=I)
    g = torch.Generator().manual_seed(31)
    d["key_lengths"] = torch.tensor([L], dtype=torch.int32)
    d["input_norm"] = torch.full((hidden,), 3.0).half()
    d["post_attention_norm"] = torch.full((hidden,), 0.5).half()
    d["q_norm"] = (0.5 + torch.rand(HD, generator=g)).half()
    d["k_norm"] = (0.5 + torch.rand(HD, generator=g)).half()
    d["w"] = {"q": _w8_diag(H * HD, hidden), "k": _w8_diag(Hkv * HD, hidden),
              "v": _w8_diag(Hkv * HD, hidden, col_of_row=lambda r: r + 128),
              "o": _w8_diag(hidden, H * HD), "gate": _w8_diag(I, hidden),
              "up": _w8_diag(I, hidden, code=130), "down": _w8_diag(hidden, I)}
    eps = d["eps"]
    x = d["x"][0].double().numpy()
    rope = d["rope"].double().numpy()
    wq = d["q_norm"].double().numpy()
    wk = d["k_norm"].double().numpy()
    w_in = d["input_norm"].double().numpy()
    w_post = d["post_attention_norm"].double().numpy()

    def layer(q_norm=True, k_norm=True, q_w=wq, k_w=wk, rope_q=True, rope_k=True,
              post_w=w_post, swap_gate_up=False, causal=True):
        n1 = np.stack([_hv(_rms64(x[t], w_in, eps)) for t in range(S)])

        def qk(vec, t, norm, w, rot):
            y = _rms64(vec, w, eps) if norm else vec
            return _hv(_rope_rotate(y, rope[t]) if rot else y)
        k = np.stack([qk(n1[t, 0:HD], t, k_norm, k_w, rope_k) for t in range(S)])
        v = n1[:, HD:2 * HD]
        a = np.zeros((S, H * HD))
        for h in range(H):
            for t in range(S):
                qv = qk(n1[t, h * HD:(h + 1) * HD], t, q_norm, q_w, rope_q)
                keys = [j for j in range(S) if (j <= t or not causal) and j < L]
                p = _softmax_rows(np.array([qv @ k[j] for j in keys]) / math.sqrt(HD))
                a[t, h * HD:(h + 1) * HD] = _hv(sum(p[i] * v[j] for i, j in enumerate(keys)))
        x1 = x + a
        n2 = np.stack([_hv(_rms64(x1[t], post_w, eps)) for t in range(S)])
        gate, up = n2, _hv(2 * n2)
        if swap_gate_up:
            gate, up = up, gate
        m = _hv(gate / (1 + np.exp(-gate)) * up)
        return x1, x1 + m

    x1_ref, x2_ref = layer()
    out, inter = blocks.qwen_layer(d, return_intermediates=True)
    got1, got2 = inter["x1"][0].double().numpy(), out[0].double().numpy()
    tol1 = 2e-3 * np.abs(x1_ref - x).max()
    tol2 = 2e-3 * np.abs(x2_ref - x1_ref).max()
    assert np.abs(got1 - x1_ref).max() <= tol1, (np.abs(got1 - x1_ref).max(), tol1)
    assert np.abs(got2 - x2_ref).max() <= tol1 + tol2, (np.abs(got2 - x2_ref).max(), tol2)

    attention_mistakes = {
        "no Q norm": dict(q_norm=False), "no K norm": dict(k_norm=False),
        "Q uses the K weight": dict(q_w=wk), "K uses the Q weight": dict(k_w=wq),
        "no RoPE on Q": dict(rope_q=False), "no RoPE on K": dict(rope_k=False),
        "no causal mask": dict(causal=False),
    }
    for name, kw in attention_mistakes.items():
        gap = np.abs(layer(**kw)[0] - x1_ref).max()
        assert gap > 10 * tol1, (name, gap, tol1)
    mlp_mistakes = {"post norm with the input weight": dict(post_w=w_in),
                    "gate and up swapped": dict(swap_gate_up=True)}
    for name, kw in mlp_mistakes.items():
        gap = np.abs(layer(**kw)[1] - x2_ref).max()
        assert gap > 10 * (tol1 + tol2), (name, gap, tol2)


def test_block_closed_form_cross_attention_norms():
    """Cross branch with non-zero Q and K.  adaLN (shared by the branches) is shift 0,
    scale 2 (so LN(x) * 3), gate 0; W2 is zero except the cross gate rows, so only the cross
    branch has a gate g2.  Q = n2 through an
    identity projection; K = ctx[:, r % 1024] and V = ctx[:, r % 1024] for output column r;
    identity O.  Per head: q' = h(rms(q_h) * wq), k' = h(rms(k_h) * wk) (distinct weights, no
    RoPE), x2 = x + g2 * h(h(softmax(q'k'^T / sqrt(128)) v)).  A dropped cross Q or K norm, one
    side normalised with the other's weight, the self-attention weights used, or RoPE applied
    to the cross Q/K each move the result by far more than the tolerance.  (Exchanging the two
    weights is not among them: q'.k' depends only on their per-column product.)"""
    S, T = 4, 3
    wrap = lambda r: r % 1024  # noqa: E731
    d = _identity_block(S, T, cross_q=_identity(DIM, DIM), cross_k=_identity(DIM, 1024, wrap),
                        cross_v=_identity(DIM, 1024, wrap))
    g = torch.Generator().manual_seed(12)
    d["cross_q_norm"] = (0.5 + torch.rand(HD, generator=g)).half()
    d["cross_k_norm"] = (0.5 + torch.rand(HD, generator=g)).half()
    d["self_q_norm"] = (0.5 + torch.rand(HD, generator=g)).half()
    d["self_k_norm"] = (0.5 + torch.rand(HD, generator=g)).half()
    d["ctx"] = (torch.randn(T, 1024, generator=g) * 2).half()
    for br in ("self", "cross", "mlp"):
        d[f"mod_{br}_w2"] = torch.zeros_like(d[f"mod_{br}_w2"])
    d["mod_cross_w2"][2 * DIM:] = (torch.randn(DIM, 256, generator=g) * 0.05).half()
    d["adaln"] = torch.cat([torch.zeros(DIM), torch.full((DIM,), 2.0), torch.zeros(DIM)])
    m = _mods(d)
    assert float(m["self"][2].abs().max()) == 0 and float(m["mlp"][2].abs().max()) == 0
    assert float(m["cross"][0].abs().max()) == 0 and float(m["cross"][1].min()) == 2.0
    g2 = m["cross"][2].double().numpy()
    assert np.abs(g2).min() > 0

    eps = d["eps"]
    x = d["x"].double().numpy()
    ctx = d["ctx"].double().numpy()
    rope = d["rope"].double().numpy()
    cq, ck = d["cross_q_norm"].double().numpy(), d["cross_k_norm"].double().numpy()
    sq, sk = d["self_q_norm"].double().numpy(), d["self_k_norm"].double().numpy()
    n2 = _h(_ln_mod(d["x"].float(), m["cross"][1], m["cross"][0])).double().numpy()
    kv = np.stack([ctx[j, np.arange(DIM) % 1024] for j in range(T)])

    def branch(q_norm=True, k_norm=True, q_w=cq, k_w=ck, rope_qk=False):
        out = np.zeros((S, DIM))
        for h in range(NH):
            cols = slice(h * HD, (h + 1) * HD)

            def pro(vec, t, norm, w):
                y = _rms64(vec, w, eps) if norm else vec
                return _hv(_rope_rotate(y, rope[t]) if rope_qk else y)
            keys = np.stack([pro(kv[j, cols], j, k_norm, k_w) for j in range(T)])
            for t in range(S):
                qv = pro(n2[t, cols], t, q_norm, q_w)
                p = _softmax_rows(keys @ qv / math.sqrt(HD))
                out[t, cols] = _hv(p @ kv[:, cols])
        return x + g2 * out

    want = branch()
    got = blocks.dit_block(d).double().numpy()
    tol = 2e-3 * np.abs(want - x).max()
    assert np.abs(got - want).max() <= tol, (np.abs(got - want).max(), tol)
    mistakes = {"no cross Q norm": dict(q_norm=False), "no cross K norm": dict(k_norm=False),
                "cross Q with the K weight": dict(q_w=ck), "cross K with the Q weight": dict(k_w=cq),
                "self-attention weights": dict(q_w=sq, k_w=sk), "RoPE on cross Q/K": dict(rope_qk=True)}
    for name, kw in mistakes.items():
        gap = np.abs(branch(**kw) - want).max()
        assert gap > 10 * tol, (name, gap, tol)
