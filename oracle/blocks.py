"""DiT block and Qwen layer composition oracles (torch-CPU fp32, optional fp16 boundaries).

Restates ``scripts/dit_block0_oracle.py:327-391`` (the MiniTrainDIT block of
ComfyUI predict2.py as transcribed there):

  modulation  (dit_block0_oracle.py:330-338): SiLU(emb) @ W1^T @ W2^T + adaln_lora,
              chunk(3) -> shift, scale, gate
  self-attn   (:345-360): LN-mod -> q,k,v projections -> per-head RMSNorm + split-half
              RoPE on q,k -> SDPA -> O projection -> x += gate * out
  cross-attn  (:366-381): LN-mod -> q from x, k,v from the context -> per-head RMSNorm
              (no RoPE) -> SDPA -> O -> x += gate * out
  MLP         (:387-391): LN-mod -> mlp1 -> exact GELU -> mlp2 -> x += gate * y

``boundary="fp16"`` rounds the branch inputs, projection outputs, normalised Q/K,
attention output and GELU output through fp16 at the same places as
``boundary_quantize`` (dit_block0_oracle.py:164-182, ``--boundary-dtype fp16``); the
residual stays fp32.  That is where the HIP block stores fp16 activations.

Test infrastructure only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import torch

from . import attention as attn
from .norms import gelu_erf, layer_norm_modulated, rms_norm, silu
from .quant import dequant_matrix_f32


def _bq(x: torch.Tensor, boundary: str) -> torch.Tensor:
    if boundary == "none":
        return x.float()
    if boundary == "fp16":
        return x.half().float()
    raise ValueError(boundary)


def dequant_weights(d: dict) -> dict:
    """fp32 dequantized ``[N, K]`` weights for every W4 linear of the block."""
    out = {}
    for name, w in d["w"].items():
        out[name] = torch.from_numpy(dequant_matrix_f32(
            w["storage"], w["packed"], w["scale_bits"], w["zero_bits"], w["rows"], w["cols"], w["row_stride"]))
    return out


def modulation(emb: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, adaln: torch.Tensor):
    """dit_block0_oracle.py:330-335: returns (shift, scale, gate) fp32 [dim] each."""
    h1 = silu(emb) @ w1.float().T
    mod = h1 @ w2.float().T + adaln.float()
    return mod.chunk(3)


def dit_block(d: dict, boundary: str = "fp16", weights: dict | None = None,
              return_intermediates: bool = False):
    """One DiT block on ``d`` (``oracle.inputs.dit_block``) -> fp32 residual [S, dim]."""
    W = weights if weights is not None else dequant_weights(d)
    x = d["x"].float()
    S, dim = x.shape
    heads, hd = 16, 128
    eps = d["eps"]
    mods = {br: modulation(d["emb"], d[f"mod_{br}_w1"], d[f"mod_{br}_w2"], d["adaln"])
            for br in ("self", "cross", "mlp")}
    inter = {}

    def proj(a, name):
        return _bq(a @ W[name].T, boundary)

    # self attention
    sh, sc, ga = mods["self"]
    n = _bq(layer_norm_modulated(x, sc, sh, eps), boundary)
    q = proj(n, "self_q").reshape(1, S, heads, hd)
    k = proj(n, "self_k").reshape(1, S, heads, hd)
    v = proj(n, "self_v").reshape(1, S, heads, hd)
    q = _bq(attn.qk_prologue(q, d["self_q_norm"], eps, d["rope"]), boundary)
    k = _bq(attn.qk_prologue(k, d["self_k_norm"], eps, d["rope"]), boundary)
    a = _bq(attn.sdpa(q, k, v).reshape(S, dim), boundary)
    o = proj(a, "self_o")
    x = x + ga * o
    inter["x1"] = x.clone()

    # cross attention
    sh, sc, ga = mods["cross"]
    ctx = d["ctx"].float()
    T = ctx.shape[0]
    n = _bq(layer_norm_modulated(x, sc, sh, eps), boundary)
    q = proj(n, "cross_q").reshape(1, S, heads, hd)
    k = proj(ctx, "cross_k").reshape(1, T, heads, hd)
    v = proj(ctx, "cross_v").reshape(1, T, heads, hd)
    q = _bq(attn.qk_prologue(q, d["cross_q_norm"], eps, None), boundary)
    k = _bq(attn.qk_prologue(k, d["cross_k_norm"], eps, None), boundary)
    a = _bq(attn.sdpa(q, k, v).reshape(S, dim), boundary)
    o = proj(a, "cross_o")
    x = x + ga * o
    inter["x2"] = x.clone()

    # MLP
    sh, sc, ga = mods["mlp"]
    n = _bq(layer_norm_modulated(x, sc, sh, eps), boundary)
    h = proj(n, "mlp1")
    h = _bq(gelu_erf(h), boundary)
    y = proj(h, "mlp2")
    x = x + ga * y
    if return_intermediates:
        return x, inter
    return x


def block_flops(S: int = 4096, ctx_tokens: int = 512, dim: int = 2048, ctx_dim: int = 1024,
                hidden: int = 8192, heads: int = 16, hd: int = 128) -> float:
    """Algorithmic FLOPs of one block: 10 linears + self and cross attention."""
    lin = 2 * S * dim * dim * 4                      # self q,k,v,o
    lin += 2 * S * dim * dim * 2                     # cross q,o
    lin += 2 * ctx_tokens * dim * ctx_dim * 2        # cross k,v
    lin += 2 * S * dim * hidden * 2                  # mlp1, mlp2
    att = 4 * heads * hd * S * S + 4 * heads * hd * S * ctx_tokens
    return float(lin + att)


def qwen_layer(d: dict, boundary: str = "fp16", weights: dict | None = None,
               return_intermediates: bool = False):
    """One Qwen encoder layer on ``d`` (``oracle.inputs.qwen_layer``) -> fp32 residual [B, S, hidden].

    Restates QwenLayerExecutor.execute (QwenEncoderMetal.swift:244-303) and the layer of
    scripts/qwen_comfy_oracle.py:268-300: RMSNorm(input_layernorm) -> fp16 -> q/k/v
    projections -> per-head RMSNorm + split-half RoPE on q,k -> causal GQA attention with
    the right-padding key mask -> o projection -> x += o -> RMSNorm(post_attention_layernorm)
    -> fp16 -> gate/up -> SiLU(gate)*up (fp32, one rounding, gated_silu_half
    AnimaKernels.metal:401-411) -> down -> x += down.  The residual is fp32; with
    ``boundary="fp16"`` every activation the reference stores as fp16 is rounded there."""
    W = weights if weights is not None else dequant_weights(d)
    x = d["x"].float()
    B, S, hidden = x.shape
    H, Hkv, hd = d["heads"], d["kv_heads"], 128
    eps = d["eps"]
    lengths = d.get("key_lengths")
    inter = {}

    def proj(a, name):
        return _bq(a @ W[name].T, boundary)

    n = _bq(rms_norm(x, d["input_norm"], eps), boundary)
    q = proj(n, "q").reshape(B, S, H, hd)
    k = proj(n, "k").reshape(B, S, Hkv, hd)
    v = proj(n, "v").reshape(B, S, Hkv, hd)
    q = _bq(attn.qk_prologue(q, d["q_norm"], eps, d["rope"]), boundary)
    k = _bq(attn.qk_prologue(k, d["k_norm"], eps, d["rope"]), boundary)
    a = _bq(attn.sdpa(q, k, v, causal=True, key_lengths=lengths).reshape(B, S, H * hd), boundary)
    inter["attention"] = a.clone()
    x = x + proj(a, "o")
    inter["x1"] = x.clone()
    n = _bq(rms_norm(x, d["post_attention_norm"], eps), boundary)
    g = proj(n, "gate")
    u = proj(n, "up")
    h = _bq(silu(g) * u, boundary)
    x = x + proj(h, "down")
    if return_intermediates:
        return x, inter
    return x
