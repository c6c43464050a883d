"""DiT input / output stages and the sampler update (torch-CPU fp32 with the fp16 boundaries).

Restates:
  * ``timestep_sinusoid``  scripts/dit_source_oracle.py:225-236 (Timesteps(2048): cos half
                           then sin half of sigma * exp(-ln(10000) * i / half)), the same
                           arithmetic as DiTPreparationExecutor.makeTimestep
                           (AnimaXS/Runtime/Metal/DiTPreparationExecutor.swift:137-147)
  * ``patchify17`` / ``unpatchify16`` / ``unpatchify_velocity16``
                           AnimaKernels.metal:1225-1297 as per-element loops (the index
                           maps of the kernels, not the reshape/permute of the source model)
  * ``prepare``            DiTPreparationExecutor.execute (DiTPreparationExecutor.swift:51-135,
                           legacy numerics): zero mask channel, patchify, fp16 patches,
                           x_embedder linear with an fp16 output, fp32 residual;
                           emb = RMSNorm(raw) * t_norm; adaln = W2 . SiLU(W1 . raw)
  * ``final_layer``        DiTFinalLayerExecutor.execute (DiTFinalLayerExecutor.swift:75-186,
                           fp16Legacy): modulation = W2 . (W1 . SiLU(emb)) + adaln[:2*dim],
                           shift then scale; half(residual) -> fp32-stat LayerNorm -> half ->
                           n * (1 + scale) + shift -> half -> linear (fp16 out) -> unpatchify
  * ``flow_to_denoised``   AnimaKernels.metal:1191-1201 / DiffusionSampler.cpuDenoised
                           (DiffusionSampler.swift:380-385)
  * ``euler_step``         EulerSampler.cpuStep (EulerSampler.swift:29-40)
  * ``SIGMAS``             EulerSampler.sigmas (EulerSampler.swift:7-17)

Test infrastructure only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import numpy as np
import torch

from .norms import layer_norm, rms_norm, silu

SIGMAS = (1.0, 0.9546938, 0.90035903, 0.8339981, 0.7511211, 0.64468634, 0.50298506, 0.30500895, 0.0)


def timestep_sinusoid(sigma: float, dim: int = 2048) -> torch.Tensor:
    """fp32 [dim]: [cos(sigma * f_i) for i < dim/2] + [sin(sigma * f_i)], f_i = exp(-ln(1e4) * i / (dim/2))."""
    half = dim // 2
    exponent = torch.tensor(-np.log(10000.0), dtype=torch.float32) * torch.arange(half, dtype=torch.float32) / half
    angle = torch.tensor(sigma, dtype=torch.float32) * torch.exp(exponent)
    return torch.cat([torch.cos(angle), torch.sin(angle)])


def patchify17(x: np.ndarray) -> np.ndarray:
    """[C <= 17, H, W] fp32 -> [(H/2)*(W/2), 68]; channels past C are zero (the mask channel)."""
    C, H, W = x.shape
    pw, ph = W // 2, H // 2
    out = np.zeros((ph * pw, 68), np.float32)
    for t in range(ph * pw):
        i, j = divmod(t, pw)
        for c in range(C):
            for di in range(2):
                for dj in range(2):
                    out[t, c * 4 + di * 2 + dj] = x[c, 2 * i + di, 2 * j + dj]
    return out


def unpatchify16(tokens: np.ndarray, H: int, W: int) -> np.ndarray:
    """[(H/2)*(W/2), 68] -> [16, H, W] (the first 16 channels)."""
    pw = W // 2
    out = np.zeros((16, H, W), np.float32)
    for t in range(tokens.shape[0]):
        i, j = divmod(t, pw)
        for c in range(16):
            for di in range(2):
                for dj in range(2):
                    out[c, 2 * i + di, 2 * j + dj] = tokens[t, c * 4 + di * 2 + dj]
    return out


def unpatchify_velocity16(tokens: np.ndarray, H: int, W: int) -> np.ndarray:
    """FinalLayer [(H/2)*(W/2), 64] with element (di*2 + dj)*16 + c -> [16, H, W]."""
    pw = W // 2
    out = np.zeros((16, H, W), np.float32)
    for t in range(tokens.shape[0]):
        i, j = divmod(t, pw)
        for c in range(16):
            for di in range(2):
                for dj in range(2):
                    out[c, 2 * i + di, 2 * j + dj] = tokens[t, (di * 2 + dj) * 16 + c]
    return out


def _patchify_fast(x: torch.Tensor) -> torch.Tensor:
    """patchify17 by reshapes, for sizes where the loops are slow; equal to ``patchify17``
    (checked in tests/test_oracle_dit_io.py)."""
    C, H, W = x.shape
    x17 = torch.zeros(17, H, W, dtype=torch.float32)
    x17[:C] = x.float()
    t = x17.reshape(17, H // 2, 2, W // 2, 2).permute(1, 3, 0, 2, 4)
    return t.reshape((H // 2) * (W // 2), 68)


def _unpatchify_velocity_fast(tokens: torch.Tensor, H: int, W: int) -> torch.Tensor:
    t = tokens.float().reshape(H // 2, W // 2, 2, 2, 16).permute(4, 0, 2, 1, 3)
    return t.reshape(16, H, W)


def prepare(latent: torch.Tensor, sigma: float, x_embed: torch.Tensor, t1: torch.Tensor, t2: torch.Tensor,
            t_norm: torch.Tensor, eps: float = 1e-6):
    """-> (residual fp32 [T, dim], emb fp32 [dim], adaln fp32 [3*dim]); weights fp32 [N, K]."""
    _, H, W = latent.shape
    dim = x_embed.shape[0]
    patches = _patchify_fast(latent).half().float()
    residual = (patches @ x_embed.float().T).half().float()
    raw = timestep_sinusoid(sigma, dim)
    emb = rms_norm(raw, t_norm, eps)
    hidden = raw @ t1.float().T
    adaln = silu(hidden) @ t2.float().T
    return residual, emb, adaln


def final_layer(residual: torch.Tensor, emb: torch.Tensor, adaln: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                proj: torch.Tensor, H: int, W: int, eps: float = 1e-6) -> torch.Tensor:
    """-> fp32 velocity [16, H, W]."""
    dim = residual.shape[1]
    mod = (silu(emb) @ w1.float().T) @ w2.float().T + adaln.float()[: 2 * dim]
    shift, scale = mod[:dim], mod[dim: 2 * dim]
    x = residual.float().half().float()
    n = layer_norm(x, eps).half().float()
    y = (n * (1.0 + scale) + shift).half().float()
    out = (y @ proj.float().T).half().float()
    return _unpatchify_velocity_fast(out, H, W)


def flow_to_denoised(x: torch.Tensor, velocity: torch.Tensor, sigma: float) -> torch.Tensor:
    return x.float() - sigma * velocity.float()


def euler_step(x: torch.Tensor, denoised: torch.Tensor, sigma: float, next_sigma: float) -> torch.Tensor:
    """x + (x - denoised) / sigma * (next_sigma - sigma), fp32 (EulerSampler.cpuStep)."""
    xf = x.float()
    delta = torch.tensor(next_sigma, dtype=torch.float32) - torch.tensor(sigma, dtype=torch.float32)
    return xf + (xf - denoised.float()) / torch.tensor(sigma, dtype=torch.float32) * delta
