"""RoPE tables and the split-half rotation (torch-CPU fp32).

Restates:
  * DiT 3-D RoPE ``DitRoPE.generate``  AnimaXS/Runtime/Text/DitRoPE.swift:58-107,
    ``dit_rope``                       scripts/dit_source_oracle.py:126-171
    (64 frequency slots: [0,22) temporal theta 1e4 over dim 44, [22,43) height and
    [43,64) width with theta 1e4*4^(42/40) over dim 42; angle = pos * theta^(-2i/dim);
    thetas narrowed to fp32 as DitRoPE.swift:37-39).
  * Qwen NeoX RoPE table ``QwenEncoderMetal.makeRope``
                                       AnimaXS/Runtime/Metal/QwenEncoderMetal.swift:126-143
    (``inv_j = 1 / 1e6^(2j/128)``, angle = pos * inv_j, fp32).
  * Split-half rotation ``rms_rope_split_half`` (rotation part)
                                       AnimaXS/Shaders/AnimaKernels.metal:696-729,
    ``apply_split_half_rope``          scripts/dit_source_oracle.py:174-194
    (pairs (p, p+64): out[p] = c*a - s*b, out[p+64] = s*a + c*b).

Tables are ``[tokens, head_dim/2, 2, 2]`` fp32 with blocks ``[cos, -sin, sin, cos]``.

Test infrastructure only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import torch

HEAD_DIM = 128


def dit_thetas(head_dim: int = HEAD_DIM):
    """(dim_t, dim_h, dim_w, t_theta, h_theta) for the DiT 3-D RoPE
    (DitRoPE.swift:27-39; position_embedding h/w NTK ratio 4.0, t ratio 1.0)."""
    dim_h = head_dim // 6 * 2
    dim_w = dim_h
    dim_t = head_dim - 2 * dim_h
    h_theta = torch.tensor(10000.0 * 4.0 ** (dim_h / (dim_h - 2)), dtype=torch.float32)
    t_theta = torch.tensor(10000.0 * 1.0 ** (dim_t / (dim_t - 2)), dtype=torch.float32)
    return dim_t, dim_h, dim_w, t_theta, h_theta


def dit_rope_table(T: int = 1, H: int = 32, W: int = 32, head_dim: int = HEAD_DIM) -> torch.Tensor:
    """DiT 3-D RoPE ``[T*H*W, head_dim/2, 2, 2]`` fp32 (DitRoPE.swift:58-107).
    Token order is t-major, then h, then w (DitRoPE.swift:71-96)."""
    dim_t, dim_h, dim_w, t_theta, h_theta = dit_thetas(head_dim)
    w_theta = h_theta

    def freqs(theta, dim):
        rng = torch.arange(0, dim, 2)[: dim // 2].float() / dim  # DitRoPE.swift:41-45
        return 1.0 / (theta ** rng)                               # DitRoPE.swift:47-50

    f_t, f_h, f_w = freqs(t_theta, dim_t), freqs(h_theta, dim_h), freqs(w_theta, dim_w)
    seq = torch.arange(max(T, H, W), dtype=torch.float32)        # DitRoPE.swift:64
    a_t = torch.outer(seq[:T], f_t)
    a_h = torch.outer(seq[:H], f_h)
    a_w = torch.outer(seq[:W], f_w)

    def blocks(a):
        return torch.stack([torch.cos(a), -torch.sin(a), torch.sin(a), torch.cos(a)], dim=-1)

    nt, nh, nw = dim_t // 2, dim_h // 2, dim_w // 2
    em = torch.cat([
        blocks(a_t)[:, None, None].expand(T, H, W, nt, 4),
        blocks(a_h)[None, :, None].expand(T, H, W, nh, 4),
        blocks(a_w)[None, None, :].expand(T, H, W, nw, 4),
    ], dim=-2)
    return em.reshape(T * H * W, nt + nh + nw, 2, 2).contiguous()


def neox_rope_table(tokens: int, theta: float = 1.0e6, head_dim: int = HEAD_DIM) -> torch.Tensor:
    """Qwen RoPE ``[tokens, head_dim/2, 2, 2]`` (QwenEncoderMetal.swift:126-143)."""
    half = head_dim // 2
    j = torch.arange(half, dtype=torch.float32)
    inv = 1.0 / torch.pow(torch.tensor(theta, dtype=torch.float32), (2.0 * j) / head_dim)
    pos = torch.arange(tokens, dtype=torch.float32)
    ang = pos[:, None] * inv[None, :]
    c, s = torch.cos(ang), torch.sin(ang)
    return torch.stack([c, -s, s, c], dim=-1).reshape(tokens, half, 2, 2).contiguous()


def apply_split_half(x: torch.Tensor, rope: torch.Tensor) -> torch.Tensor:
    """Rotate pairs (p, p+half) of ``x[..., S, H, D]`` with ``rope[S, D/2, 2, 2]``
    (AnimaKernels.metal:720-728; DiTBlockCPU.applySplitHalfRoPE)."""
    half = x.shape[-1] // 2
    x = x.float()
    c = rope[:, :, 0, 0].float()[:, None, :]
    s = rope[:, :, 1, 0].float()[:, None, :]
    a, b = x[..., :half], x[..., half:]
    return torch.cat([c * a - s * b, s * a + c * b], dim=-1)
