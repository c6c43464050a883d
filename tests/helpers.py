"""Shared helpers for the parity tests (device upload, metrics, weight wrappers)."""

from __future__ import annotations

import numpy as np
import torch

import animaxs_amd

# Attention parity bar (stated in the measured workload definition): against the
# fp32 oracle, max |y - ref| <= 1e-2 and sum|y - ref| / sum|ref| <= 1e-3.
ATTN_MAX_ABS = 1e-2
ATTN_MEAN_REL = 1e-3


def max_abs(y, ref) -> float:
    return float((y.float() - ref.float()).abs().max())


def mean_rel(y, ref) -> float:
    y, ref = y.float(), ref.float()
    return float((y - ref).abs().sum() / ref.abs().sum().clamp_min(1e-30))


def assert_attention_close(y, ref, max_abs_tol=ATTN_MAX_ABS, mean_rel_tol=ATTN_MEAN_REL, label=""):
    y = y.float().cpu()
    ref = ref.float().cpu()
    assert torch.isfinite(y).all(), f"{label}: non-finite output"
    ma, mr = max_abs(y, ref), mean_rel(y, ref)
    print(f"PARITY {label}: max_abs={ma:.3e} mean_rel={mr:.3e}", flush=True)
    assert ma <= max_abs_tol, f"{label}: max_abs {ma} > {max_abs_tol}"
    assert mr <= mean_rel_tol, f"{label}: mean_rel {mr} > {mean_rel_tol}"


def dev(t, dtype=None):
    if isinstance(t, np.ndarray):
        t = torch.from_numpy(np.ascontiguousarray(t))
    t = t.contiguous()
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def device_weight(w: dict, pad_bytes: int = 0) -> tuple:
    """oracle weight dict -> (QuantizedLinearWeightBuffers, keepalive tensors)."""
    packed = np.asarray(w["packed"]).reshape(-1).view(np.uint8)
    if pad_bytes:
        packed = np.concatenate([packed, np.zeros(pad_bytes, np.uint8)])
    p = dev(torch.from_numpy(packed.copy()))
    s = dev(torch.from_numpy(np.asarray(w["scale_bits"], np.uint16).reshape(-1).view(np.int16).copy()))
    z = dev(torch.from_numpy(np.asarray(w["zero_bits"], np.uint16).reshape(-1).view(np.int16).copy()))
    q = animaxs_amd.QuantizedLinearWeightBuffers(
        storage=w["storage"], packed=p, scale=s, zero=z, rows=w["rows"], columns=w["cols"],
        packed_row_stride=w["row_stride"])
    return q, (p, s, z)


def fp16_weight(w16: torch.Tensor) -> tuple:
    """fp16 [N, K] -> FP16-storage QuantizedLinearWeightBuffers."""
    d = dev(w16.half())
    q = animaxs_amd.QuantizedLinearWeightBuffers(
        storage=2, packed=d, scale=d, zero=d, rows=w16.shape[0], columns=w16.shape[1],
        packed_row_stride=w16.shape[1])
    return q, (d,)
