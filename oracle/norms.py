"""Normalisations and activations of the DiT block / Qwen layer (torch-CPU fp32).

Restates:
  * ``rms_norm``          scripts/dit_block0_oracle.py:77-82 (per-head RMSNorm with a
                          shared [head_dim] weight; AnimaKernels.metal:660-689, :696-718)
  * ``layer_norm``        scripts/dit_block0_oracle.py:85-90 (mean-centred, no affine)
  * ``layer_norm_modulated``  dit_block0_oracle.py:93-95 / AnimaKernels.metal:477-524
                          (scale read at offset N, shift at offset 0 of the modulation)
  * ``gelu_erf``          exact-erf GELU, dit_block0_oracle.py:153-157, AnimaKernels.metal:252-283
  * ``silu``              AnimaKernels.metal:388-397

Test infrastructure only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import torch

EPS = 1e-6


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """``x * rsqrt(mean(x^2) + eps) * w`` over the last dim, fp32."""
    xf = x.float()
    inv = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return xf * inv * w.float()


def layer_norm(x: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    xf = x.float()
    mu = xf.mean(-1, keepdim=True)
    var = (xf - mu).pow(2).mean(-1, keepdim=True)
    return (xf - mu) / torch.sqrt(var + eps)


def layer_norm_modulated(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                         eps: float = EPS) -> torch.Tensor:
    return layer_norm(x, eps) * (1.0 + scale.float()) + shift.float()


def gelu_erf(x: torch.Tensor) -> torch.Tensor:
    xf = x.float()
    return 0.5 * xf * (1.0 + torch.erf(xf * 0.7071067811865475))


def silu(x: torch.Tensor) -> torch.Tensor:
    xf = x.float()
    return xf / (1.0 + torch.exp(-xf))
