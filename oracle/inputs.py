"""Seeded synthetic inputs for the five measured workloads (CPU torch.Generator).

Seed ``1000 + c`` for workload c in 1..5.  Values are generated in fp32 on the CPU,
rounded to fp16 where the hot path consumes fp16, and the SAME fp16 bits feed both
the HIP library and the oracle (upcast to fp32).  Shapes and distributions:

  1. DiT self-attention 512x512: B1 H16 D128 S1024, Q/K/V ~N(0,1).
  2. DiT self-attention 1024x1024: B1 H16 D128 S4096, Q/K/V ~N(0,1), per-head RMSNorm
     weights ~U(0.8,1.2) (eps 1e-6), DiT 3-D RoPE for a 1x64x64 grid.
  3. DiT cross-attention: B4, 4096 image queries, 512 context keys, H16 D128,
     Q/K/V ~N(0,1) before the per-head RMSNorm (weights ~U(0.8,1.2)), key-padding
     valid length L_b ~U{77..512}.
  4. Qwen3-0.6B-shaped causal GQA: B4 S512, 16 query / 8 KV heads, D128, hidden 1024,
     right padding L_b ~U{8..512}, token ids ~U{0..151935} through a random fp16
     embedding, pre-RMSNorm, fp16 projections ~N(0,0.02^2), QK-RMSNorm + RoPE 1e6.
  5. Full DiT block 1024x1024: S4096 hidden 2048, context [512,1024], 10 W4 linears
     (q ~U{0..15}, fp16 scale ~U(0.005,0.02), zero = -8*scale, group 64), fp16
     modulation weights ~N(0,0.02^2), fp32 emb / adaln_lora / residual ~N(0,1).

The symmetric W4 data of workload 5 is expressed in the reference's affine format
(``value = q*scale + zero``, AnimaKernels.metal:19-41) with ``zero = -8*scale``,
exact in fp16 because multiplying by 8 only shifts the exponent.

Test infrastructure only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import numpy as np
import torch

from . import rope as rope_mod
from .quant import pack_w4

HEADS, HEAD_DIM, DIM = 16, 128, 2048


def _gen(config: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(1000 + config)
    return g


def _randn16(g, *shape, std: float = 1.0) -> torch.Tensor:
    return (torch.randn(*shape, generator=g, dtype=torch.float32) * std).half()


def _uniform(g, lo: float, hi: float, *shape) -> torch.Tensor:
    return lo + (hi - lo) * torch.rand(*shape, generator=g, dtype=torch.float32)


def self_attention(config: int = 1, S: int | None = None, B: int = 1, heads: int = HEADS) -> dict:
    """Workloads 1 and 2 (``S`` overrides the sequence length for reduced tests)."""
    g = _gen(config)
    if S is None:
        S = 1024 if config == 1 else 4096
    d = {
        "q": _randn16(g, B, S, heads, HEAD_DIM),
        "k": _randn16(g, B, S, heads, HEAD_DIM),
        "v": _randn16(g, B, S, heads, HEAD_DIM),
    }
    if config == 2:
        d["q_norm_w"] = _uniform(g, 0.8, 1.2, HEAD_DIM).half()
        d["k_norm_w"] = _uniform(g, 0.8, 1.2, HEAD_DIM).half()
        side = int(round(S ** 0.5))
        assert side * side == S, "workload 2 uses a square 1 x side x side grid"
        d["rope"] = rope_mod.dit_rope_table(1, side, side)
        d["eps"] = 1e-6
    return d


def cross_attention(B: int = 4, Sq: int = 4096, Sk: int = 512, heads: int = HEADS) -> dict:
    """Workload 3."""
    g = _gen(3)
    d = {
        "q": _randn16(g, B, Sq, heads, HEAD_DIM),
        "k": _randn16(g, B, Sk, heads, HEAD_DIM),
        "v": _randn16(g, B, Sk, heads, HEAD_DIM),
        "q_norm_w": _uniform(g, 0.8, 1.2, HEAD_DIM).half(),
        "k_norm_w": _uniform(g, 0.8, 1.2, HEAD_DIM).half(),
        "eps": 1e-6,
    }
    lo = min(77, Sk)
    d["key_lengths"] = torch.randint(lo, Sk + 1, (B,), generator=g, dtype=torch.int32)
    return d


def qwen_attention(B: int = 4, S: int = 512, heads: int = 16, kv_heads: int = 8,
                   hidden: int = 1024, vocab: int = 151936) -> dict:
    """Workload 4: attention inputs of one Qwen3-0.6B-shaped layer.

    Follows scripts/qwen_comfy_oracle.py:268-285 up to the projections: embedding
    gather -> RMSNorm(input_layernorm) -> fp16 q/k/v projections.  Only the gathered
    embedding rows are materialised: row ``id`` is drawn from its own generator
    seeded ``1004 * 1_000_003 + id`` so the table is implicit but fixed."""
    g = _gen(4)
    lengths = torch.randint(min(8, S), S + 1, (B,), generator=g, dtype=torch.int32)
    ids = torch.randint(0, vocab, (B, S), generator=g, dtype=torch.int64)
    in_norm = _uniform(g, 0.8, 1.2, hidden).half()
    wq = _randn16(g, heads * HEAD_DIM, hidden, std=0.02)
    wk = _randn16(g, kv_heads * HEAD_DIM, hidden, std=0.02)
    wv = _randn16(g, kv_heads * HEAD_DIM, hidden, std=0.02)
    q_norm_w = _uniform(g, 0.8, 1.2, HEAD_DIM).half()
    k_norm_w = _uniform(g, 0.8, 1.2, HEAD_DIM).half()
    rows = {}
    for t in torch.unique(ids).tolist():
        rg = torch.Generator(device="cpu")
        rg.manual_seed(1004 * 1_000_003 + int(t))
        rows[t] = torch.randn(hidden, generator=rg, dtype=torch.float32).half()
    x = torch.stack([torch.stack([rows[int(t)] for t in ids[b]]) for b in range(B)])  # [B,S,hidden] fp16
    xf = x.float()
    h = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * in_norm.float()).half()
    q = (h.float() @ wq.float().T).half().reshape(B, S, heads, HEAD_DIM)
    k = (h.float() @ wk.float().T).half().reshape(B, S, kv_heads, HEAD_DIM)
    v = (h.float() @ wv.float().T).half().reshape(B, S, kv_heads, HEAD_DIM)
    return {
        "q": q, "k": k, "v": v, "q_norm_w": q_norm_w, "k_norm_w": k_norm_w,
        "rope": rope_mod.neox_rope_table(S, 1.0e6), "eps": 1e-6, "key_lengths": lengths,
        "ids": ids,
    }


def symmetric_w4(g: torch.Generator, rows: int, cols: int) -> dict:
    """Symmetric int4 weight in the reference's affine W4 layout (see module doc)."""
    q = torch.randint(0, 16, (rows, cols), generator=g, dtype=torch.int64).numpy().astype(np.uint8)
    groups = (cols + 63) // 64
    scale = _uniform(g, 0.005, 0.02, rows, groups).half()
    zero = (scale.float() * -8.0).half()
    assert torch.equal(zero.float(), scale.float() * -8.0)
    return {
        "storage": 0, "rows": rows, "cols": cols, "row_stride": (cols + 1) // 2,
        "packed": pack_w4(q), "scale_bits": scale.numpy().view(np.uint16),
        "zero_bits": zero.numpy().view(np.uint16),
    }


BLOCK_LINEARS = [
    # name, rows (N), cols (K)
    ("self_q", 2048, 2048), ("self_k", 2048, 2048), ("self_v", 2048, 2048), ("self_o", 2048, 2048),
    ("cross_q", 2048, 2048), ("cross_k", 2048, 1024), ("cross_v", 2048, 1024), ("cross_o", 2048, 2048),
    ("mlp1", 8192, 2048), ("mlp2", 2048, 8192),
]


def dit_block(S: int = 4096, ctx_tokens: int = 512, ctx_dim: int = 1024,
              hidden: int = 8192, dim: int = DIM, seed: int | None = None) -> dict:
    """Workload 5 (``S`` may be reduced for fast tests; it must be a square grid).
    ``seed`` replaces the workload seed (other blocks of a multi-block forward)."""
    g = _gen(5)
    if seed is not None:
        g.manual_seed(seed)
    side = int(round(S ** 0.5))
    assert side * side == S
    d = {
        "x": torch.randn(S, dim, generator=g, dtype=torch.float32),
        "emb": torch.randn(dim, generator=g, dtype=torch.float32),
        "adaln": torch.randn(3 * dim, generator=g, dtype=torch.float32),
        "ctx": _randn16(g, ctx_tokens, ctx_dim),
        "rope": rope_mod.dit_rope_table(1, side, side),
        "eps": 1e-6,
    }
    shapes = {"self_q": (dim, dim), "self_k": (dim, dim), "self_v": (dim, dim), "self_o": (dim, dim),
              "cross_q": (dim, dim), "cross_k": (dim, ctx_dim), "cross_v": (dim, ctx_dim),
              "cross_o": (dim, dim), "mlp1": (hidden, dim), "mlp2": (dim, hidden)}
    d["w"] = {name: symmetric_w4(g, *shapes[name]) for name, _, _ in BLOCK_LINEARS}
    for br in ("self", "cross", "mlp"):
        d[f"mod_{br}_w1"] = _randn16(g, 256, dim, std=0.02)
        d[f"mod_{br}_w2"] = _randn16(g, 3 * dim, 256, std=0.02)
    for nm in ("self_q_norm", "self_k_norm", "cross_q_norm", "cross_k_norm"):
        d[nm] = _uniform(g, 0.8, 1.2, HEAD_DIM).half()
    return d


def symmetric_w8(g: torch.Generator, rows: int, cols: int, lo: float = 1e-4, hi: float = 3e-4) -> dict:
    """Symmetric int8 weight in the reference's affine W8 layout: q ~U{0..255},
    scale ~U(lo, hi) stored as fp16 per (row, 64-wide group), zero = -128 * scale
    (exact in fp16)."""
    q = torch.randint(0, 256, (rows, cols), generator=g, dtype=torch.int64).numpy().astype(np.uint8)
    groups = (cols + 63) // 64
    scale = _uniform(g, lo, hi, rows, groups).half()
    zero = (scale.float() * -128.0).half()
    assert torch.equal(zero.float(), scale.float() * -128.0)
    return {
        "storage": 1, "rows": rows, "cols": cols, "row_stride": cols,
        "packed": q.reshape(-1), "scale_bits": scale.numpy().view(np.uint16),
        "zero_bits": zero.numpy().view(np.uint16),
    }


QWEN_LINEARS = ("q", "k", "v", "o", "gate", "up", "down")


def qwen_layer(B: int = 4, S: int = 512, hidden: int = 1024, heads: int = 16, kv_heads: int = 8,
               intermediate: int = 3072) -> dict:
    """One Qwen3-0.6B-shaped encoder layer (QwenEncoderMetal.swift:202-304): W8 projections,
    fp16 norm weights, fp32 residual [B, S, hidden], right padding with L_b ~U{min(8,S)..S}."""
    g = _gen(4)
    qdim, kvdim = heads * HEAD_DIM, kv_heads * HEAD_DIM
    shapes = {"q": (qdim, hidden), "k": (kvdim, hidden), "v": (kvdim, hidden), "o": (hidden, qdim),
              "gate": (intermediate, hidden), "up": (intermediate, hidden), "down": (hidden, intermediate)}
    d = {
        "x": torch.randn(B, S, hidden, generator=g, dtype=torch.float32),
        "key_lengths": torch.randint(min(8, S), S + 1, (B,), generator=g, dtype=torch.int32),
        "input_norm": _uniform(g, 0.8, 1.2, hidden).half(),
        "post_attention_norm": _uniform(g, 0.8, 1.2, hidden).half(),
        "q_norm": _uniform(g, 0.8, 1.2, HEAD_DIM).half(),
        "k_norm": _uniform(g, 0.8, 1.2, HEAD_DIM).half(),
        "rope": rope_mod.neox_rope_table(S, 1.0e6),
        "eps": 1e-6, "heads": heads, "kv_heads": kv_heads,
    }
    d["w"] = {name: symmetric_w8(g, *shapes[name]) for name in QWEN_LINEARS}
    return d


def dit_io(H: int = 64, W: int = 64, dim: int = DIM, lora: int = 256, seed: int = 1007,
           storage: str = "w4") -> dict:
    """The DiT preparation and final-layer inputs at a [16, H, W] latent: W4 (or W8 for
    ``storage="w8"``) x_embedder [dim, 68], t_embedder linears [dim, dim] / [3*dim, dim],
    final modulation [lora, dim] / [2*dim, lora] and projection [64, dim]; fp16 t_norm
    ~U(0.8, 1.2); fp32 latent ~N(0, 1), residual ~N(0, 4), emb / adaln ~N(0, 1)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    T = (H // 2) * (W // 2)
    mk = symmetric_w4 if storage == "w4" else symmetric_w8
    return {
        "latent": torch.randn(16, H, W, generator=g, dtype=torch.float32),
        "residual": torch.randn(T, dim, generator=g, dtype=torch.float32) * 2.0,
        "emb": torch.randn(dim, generator=g, dtype=torch.float32),
        "adaln": torch.randn(3 * dim, generator=g, dtype=torch.float32),
        "t_norm": _uniform(g, 0.8, 1.2, dim).half(),
        "w": {"x_embed": mk(g, dim, 68), "t_embed1": mk(g, dim, dim), "t_embed2": mk(g, 3 * dim, dim),
              "mod_w1": mk(g, lora, dim), "mod_w2": mk(g, 2 * dim, lora), "proj": mk(g, 64, dim)},
        "H": H, "W": W, "dim": dim, "eps": 1e-6,
    }


def small_m_gemm(M: int, N: int, K: int, seed: int = 1006) -> dict:
    """Small-M W4 GEMM sweep inputs: X ~N(0,1) fp16 [M,K], symmetric W4 [N,K]."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed * 100003 + M * 7 + N * 13 + K)
    return {"x": _randn16(g, M, K), "w": symmetric_w4(g, N, K)}
