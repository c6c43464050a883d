"""Scaled dot-product attention oracle (torch-CPU fp32).

Restates:
  * the attention of ``scripts/dit_block0_oracle.py:124-143`` (softmax(scale*QK^T) V,
    fp32 scores / probabilities; with ``legacy=True`` the ``LEGACY_ATTENTION`` rounding of
    :135-141: the scaled scores and the normalised probabilities pass through fp16, the
    rounding points of the reference's MPS backends and ``attention_softmax_rows``,
    AnimaKernels.metal:1051-1100),
  * ``DiTBlockCPU.attentionHead`` (AnimaXS/Runtime/Text/DiTBlockCPU.swift:151-186) and
    ``QwenNumerics.scaledDotAttention`` (AnimaXS/Runtime/Text/QwenNumerics.swift:89-115),
  * GQA head map ``kvHead = h / (H / Hkv)`` (AnimaXS/Runtime/Metal/AttentionExecutor.swift:222;
    ComfyUI ``repeat_interleave`` in scripts/qwen_comfy_oracle.py:79-92),
  * the masked mode of ``scripts/qwen_comfy_oracle.py:233-248``: an additive
    ``finfo.min/4`` key-padding mask plus a causal ``triu_(1)`` of the same value,
    used by ``attention_pytorch`` / ``attention_basic`` (:146-187),
  * the per-head Q/K prologue: ``rms_norm`` then split-half RoPE
    (``rms_rope_split_half``, scripts/dit_block0_oracle.py:98-121; cross attention
    without RoPE, :374-375; Qwen ``rms_norm`` + ``apply_rope``, qwen_comfy_oracle.py:283-285).

Tensors are token-major ``[B, S, H, D]``.

Test infrastructure only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import math

import torch

from .norms import rms_norm
from .rope import apply_split_half


def qk_prologue(x: torch.Tensor, norm_w: torch.Tensor | None, eps: float,
                rope: torch.Tensor | None) -> torch.Tensor:
    """Per-head RMSNorm (shared [D] weight) then optional split-half RoPE; fp32 out.
    ``x`` is ``[B, S, H, D]``; ``rope`` is ``[>=S, D/2, 2, 2]`` indexed by token."""
    y = x.float()
    if norm_w is not None:
        y = rms_norm(y, norm_w, eps)
    if rope is not None:
        S = y.shape[1]
        y = apply_split_half(y, rope[:S])
    return y


def sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: float | None = None,
         causal: bool = False, key_lengths=None, legacy: bool = False) -> torch.Tensor:
    """Attention over ``q[B,Sq,H,D]``, ``k,v[B,Sk,Hkv,D]`` -> ``[B,Sq,H,D]`` fp32.

    ``key_lengths[b]`` keys ``j >= L_b`` receive the additive ``finfo(fp32).min/4``
    mask; ``causal`` adds the same value above the diagonal (requires Sq == Sk).
    ``legacy`` rounds the scaled scores (before the mask) and the normalised
    probabilities to fp16."""
    B, Sq, H, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    assert H % Hkv == 0
    rep = H // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    neg = torch.finfo(torch.float32).min / 4
    out = torch.empty((B, Sq, H, D), dtype=torch.float32)
    qf, kf, vf = q.float(), k.float(), v.float()
    for b in range(B):
        mask = None
        if key_lengths is not None:
            L = int(key_lengths[b])
            m = torch.zeros(Sk, dtype=torch.float32)
            m[L:] = neg
            mask = m[None, :].expand(Sq, Sk)
        if causal:
            assert Sq == Sk, "causal attention requires queryCount == keyCount"
            cm = torch.full((Sq, Sk), neg, dtype=torch.float32).triu_(1)
            mask = cm if mask is None else mask + cm
        for h in range(H):
            kh = h // rep
            s = (qf[b, :, h, :] @ kf[b, :, kh, :].T) * scale
            if legacy:
                s = s.half().float()
            if mask is not None:
                s = s + mask
            p = torch.softmax(s, dim=-1)
            if legacy:
                p = p.half().float()
            out[b, :, h, :] = p @ vf[b, :, kh, :]
    return out


def attention_flops(B: int, H: int, Sq: int, Sk: int, D: int, causal: bool = False,
                    key_lengths=None) -> float:
    """Algorithmic FLOPs (two GEMMs) counting only unmasked (query, key) pairs:
    ``4*D`` per pair; causal with key mask L_b counts ``sum_i min(i+1, L_b)``."""
    total = 0
    for b in range(B):
        L = Sk if key_lengths is None else int(key_lengths[b])
        if causal:
            pairs = sum(min(i + 1, L) for i in range(Sq))
        else:
            pairs = Sq * L
        total += pairs
    return 4.0 * D * H * total
