"""GPU: the DiT input / output stages and the sampler update through the C ABI, against the
oracle (oracle/dit_io.py).

  * patchify17 / unpatchify16 / unpatchify_velocity16 are copies: bit-exact, and nothing past
    the logical output is written (the guard tails of MetalExecutionTests.swift:594-678);
  * flow -> denoised and the Euler step: within 1e-6 of the oracle (the bar of
    MetalExecutionTests.swift:680-710; the kernels fuse each product into one FMA);
  * DiTPreparationExecutor / DiTFinalLayerExecutor: residual, embedding, AdaLN-LoRA and velocity
    against the oracle at the 64x64 and 128x128 latents (1024 / 4096 tokens), with the bars
    written in each test;
  * one whole sampler step (prepare -> blocks -> final layer -> denoised -> Euler) against the
    oracle composing the same stages.
"""

import numpy as np
import pytest
import torch

import animaxs_amd
from animaxs_amd import (DiTBlockExecutor, DiTFinalLayerExecutor, DiTPreparationExecutor, EulerSampler,
                         LatentOps)
from oracle import blocks, dit_io, inputs
from oracle.quant import dequant_matrix_f32, dequant_to_half
from tests.helpers import dev, device_weight, fp16_weight, max_abs, mean_rel

pytestmark = pytest.mark.gpu

SENTINEL = 1234567.0


def _guarded(n, extra):
    return torch.full((n + extra,), SENTINEL, dtype=torch.float32, device="cuda")


def _wf32(w):
    """The fp32 weight a matvec multiplies by (w4/w8_matvec_f32 dequantize in fp32)."""
    return torch.from_numpy(dequant_matrix_f32(w["storage"], w["packed"], w["scale_bits"], w["zero_bits"], w["rows"],
                                               w["cols"], w["row_stride"]))


def _wh(w):
    """The fp16 weight a linear multiplies by (dequant_w4/w8_to_half then the fp16 GEMM)."""
    bits = dequant_to_half(w["storage"], w["packed"], w["scale_bits"], w["zero_bits"], w["rows"], w["cols"],
                           w["row_stride"])
    return torch.from_numpy(bits.view(np.float16).astype(np.float32))


@pytest.mark.parametrize("H,W", [(4, 6), (64, 64), (128, 96)])
@pytest.mark.parametrize("channels", [17, 16])
def test_patchify_round_trip_bit_exact(ctx, H, W, channels):
    print(f"PATCHIFY H={H} W={W} channels={channels}", flush=True)
    x = torch.randn(channels, H, W, generator=torch.Generator().manual_seed(H * W + channels))
    if (H, W) == (4, 6):
        idx = torch.arange(channels * H * W)
        x = (((idx * 17) % 101).float() / 10 - 5).reshape(channels, H, W)
    T = (H // 2) * (W // 2)
    ops = LatentOps(ctx)
    tok = _guarded(T * 68, 68)
    ops.patchify17(dev(x), tok[: T * 68], H, W, channels=channels)
    back = _guarded(16 * H * W, H * W)
    ops.unpatchify16(tok[: T * 68], back[: 16 * H * W], H, W)
    torch.cuda.synchronize()
    t = tok.cpu()
    assert torch.all(t[T * 68:] == SENTINEL) and torch.all(back.cpu()[16 * H * W:] == SENTINEL)
    ref = dit_io._patchify_fast(x).numpy()
    if H * W <= 64:
        ref_loop = dit_io.patchify17(x.numpy())
        assert np.array_equal(ref_loop, ref)
    assert np.array_equal(t[: T * 68].numpy().reshape(T, 68), ref)
    assert torch.equal(back.cpu()[: 16 * H * W].reshape(16, H, W), x[:16])


@pytest.mark.parametrize("H,W", [(4, 6), (64, 64), (128, 128)])
def test_unpatchify_velocity_bit_exact(ctx, H, W):
    print(f"UNPATCHIFY velocity H={H} W={W}", flush=True)
    T = (H // 2) * (W // 2)
    tok = torch.arange(T * 64, dtype=torch.float32) if T * 64 < 2 ** 24 else torch.randn(T * 64)
    out = _guarded(16 * H * W, H * W)
    LatentOps(ctx).unpatchify_velocity16(dev(tok), out[: 16 * H * W], H, W)
    torch.cuda.synchronize()
    o = out.cpu()
    assert torch.all(o[16 * H * W:] == SENTINEL)
    ref = dit_io._unpatchify_velocity_fast(tok, H, W)
    if T <= 16:
        assert np.array_equal(dit_io.unpatchify_velocity16(tok.numpy().reshape(T, 64), H, W), ref.numpy())
    assert torch.equal(o[: 16 * H * W].reshape(16, H, W), ref)


def test_euler_known_values_and_guard(ctx):
    """MetalExecutionTests.swift:680-710: five values, eight guard elements left untouched."""
    x = dev(torch.tensor([-2, -0.5, 0, 1, 3], dtype=torch.float32))
    d = dev(torch.tensor([1, -1, 2, 0.25, -4], dtype=torch.float32))
    out = _guarded(5, 8)
    EulerSampler(ctx).encode_step(x, d, out[:5], 0.75, 0.625, 5)
    torch.cuda.synchronize()
    o = out.cpu()
    np.testing.assert_allclose(o[:5].numpy(), [-1.5, -0.5 - 1 / 12, 1 / 3, 0.875, 3 - 7 / 6], atol=1e-6, rtol=0)
    assert torch.all(o[5:] == SENTINEL)


@pytest.mark.parametrize("count", [1, 7, 16 * 64 * 64, 16 * 128 * 128 + 3])
def test_flow_and_euler_match_oracle(ctx, count):
    print(f"FLOW+EULER count={count}", flush=True)
    g = torch.Generator().manual_seed(count)
    x, v = torch.randn(count, generator=g), torch.randn(count, generator=g)
    ops, eu = LatentOps(ctx), EulerSampler(ctx)
    dx, dv = dev(x), dev(v)
    den, nxt = torch.empty_like(dx), torch.empty_like(dx)
    for s, ns in zip(EulerSampler.SIGMAS[:-1], EulerSampler.SIGMAS[1:]):
        ops.flow_velocity_to_denoised(dx, dv, den, s, count)
        eu.encode_step(dx, den, nxt, s, ns, count)
        torch.cuda.synchronize()
        rd = dit_io.flow_to_denoised(x, v, s)
        np.testing.assert_allclose(den.cpu().numpy(), rd.numpy(), atol=1e-6, rtol=1e-6)
        rn = dit_io.euler_step(x, den.cpu(), s, ns)
        np.testing.assert_allclose(nxt.cpu().numpy(), rn.numpy(), atol=1e-6, rtol=1e-6)
    # the last transition (next sigma 0) returns the denoised latent
    s = EulerSampler.SIGMAS[-2]
    ops.flow_velocity_to_denoised(dx, dv, den, s, count)
    eu.encode_step(dx, den, nxt, s, 0.0, count)
    torch.cuda.synchronize()
    np.testing.assert_allclose(nxt.cpu().numpy(), den.cpu().numpy(), atol=1e-6, rtol=1e-6)


def _device_weights(d, names):
    keep, out = [], {}
    for n in names:
        q, k = device_weight(d["w"][n])
        out[n] = q
        keep.append(k)
    return out, keep


@pytest.mark.parametrize("H,W,storage", [(64, 64, "w4"), (128, 128, "w4"), (64, 64, "w8"), (20, 36, "w4")])
def test_preparation_matches_oracle(ctx, H, W, storage):
    d = inputs.dit_io(H, W, storage=storage)
    dim, T = d["dim"], (H // 2) * (W // 2)
    print(f"PREPARE H={H} W={W} {storage}", flush=True)
    w, keep = _device_weights(d, ("x_embed", "t_embed1", "t_embed2"))
    w["t_norm"] = dev(d["t_norm"])
    prep = DiTPreparationExecutor(ctx)
    res = torch.empty(T, dim, device="cuda")
    emb = torch.empty(dim, device="cuda")
    adaln = torch.empty(3 * dim, device="cuda")
    sigma = 0.8339981
    prep.execute(w, dev(d["latent"]), sigma, res, emb, adaln, height=H, width=W, dim=dim)
    torch.cuda.synchronize()
    r_res, r_emb, r_adaln = dit_io.prepare(d["latent"], sigma, _wh(d["w"]["x_embed"]), _wf32(d["w"]["t_embed1"]),
                                           _wf32(d["w"]["t_embed2"]), d["t_norm"].float())
    # residual: fp16 outputs of a K=68 GEMM over the same fp16 operands.  The fp32 sums differ
    # only in order, by at most 68 * 2^-24 * sum|x_k w_k| on each side, and the result may then
    # round to a neighbouring fp16 value: |y - ref| <= ulp16(ref) + 2 * 68 * 2^-24 * sum|x_k w_k|.
    y = res.cpu()
    patches = dit_io._patchify_fast(d["latent"]).half().float()
    sum_abs = patches.abs() @ _wh(d["w"]["x_embed"]).abs().T
    bound = torch.clamp(r_res.abs(), min=2 ** -14) * 2 ** -10 + 2 * 68 * 2 ** -24 * sum_abs
    excess = ((y - r_res).abs() / bound).max()
    print(f"PARITY prepare residual: max |y - ref| / bound = {float(excess):.3f}", flush=True)
    assert excess <= 1.0
    # emb: fp32 sinusoid (device exp/cos/sin within a few ulp) times the RMSNorm scale
    ma = max_abs(emb.cpu(), r_emb)
    print(f"PARITY prepare emb max_abs={ma:.3e}", flush=True)
    assert ma <= 2e-6
    # adaln: two fp32 matvecs over K = dim (sum order differs)
    mr = mean_rel(adaln.cpu(), r_adaln)
    print(f"PARITY prepare adaln mean_rel={mr:.3e} max_abs={max_abs(adaln.cpu(), r_adaln):.3e}", flush=True)
    assert mr <= 1e-5 and max_abs(adaln.cpu(), r_adaln) <= 1e-4 * float(r_adaln.abs().max())


@pytest.mark.parametrize("H,W,storage", [(64, 64, "w4"), (128, 128, "w4"), (64, 64, "w8"), (20, 36, "w4")])
def test_final_layer_matches_oracle(ctx, H, W, storage):
    d = inputs.dit_io(H, W, storage=storage)
    dim = d["dim"]
    print(f"FINAL H={H} W={W} {storage}", flush=True)
    w, keep = _device_weights(d, ("mod_w1", "mod_w2", "proj"))
    fin = DiTFinalLayerExecutor(ctx)
    vel = _guarded(16 * H * W, 64)
    fin.execute(w, dev(d["residual"]), dev(d["emb"]), dev(d["adaln"]), vel[: 16 * H * W], height=H, width=W,
                dim=dim)
    torch.cuda.synchronize()
    v = vel.cpu()
    assert torch.all(v[16 * H * W:] == SENTINEL)
    ref = dit_io.final_layer(d["residual"], d["emb"], d["adaln"], _wf32(d["w"]["mod_w1"]), _wf32(d["w"]["mod_w2"]),
                             _wh(d["w"]["proj"]), H, W)
    y = v[: 16 * H * W].reshape(16, H, W)
    assert torch.isfinite(y).all()
    ma, mr = max_abs(y, ref), mean_rel(y, ref)
    print(f"PARITY final velocity max_abs={ma:.3e} mean_rel={mr:.3e} (|ref|max {float(ref.abs().max()):.2f})",
          flush=True)
    # fp16 boundaries on both sides: a value may land on the other side of an fp16 rounding
    # (the modulation matvecs sum in another order), so allow a few fp16 ulps at the output
    assert mr <= 1e-3
    assert ma <= 4e-3 * float(ref.abs().max())


def test_preparation_and_final_validation(ctx):
    d = inputs.dit_io(8, 8, dim=256, lora=32)
    w, keep = _device_weights(d, ("x_embed", "t_embed1", "t_embed2", "mod_w1", "mod_w2", "proj"))
    w["t_norm"] = dev(d["t_norm"])
    prep, fin = DiTPreparationExecutor(ctx), DiTFinalLayerExecutor(ctx)
    res, emb, adaln = (torch.empty(16, 256, device="cuda"), torch.empty(256, device="cuda"),
                       torch.empty(768, device="cuda"))
    lat = dev(d["latent"][:, :8, :8])
    with pytest.raises(animaxs_amd.AnimaError, match="invalid DiT preparation input"):
        prep.execute(w, lat, float("nan"), res, emb, adaln, height=8, width=8, dim=256)
    with pytest.raises(animaxs_amd.AnimaError, match="even height and width"):
        prep.execute(w, lat, 1.0, res, emb, adaln, height=7, width=8, dim=256)
    with pytest.raises(animaxs_amd.AnimaError, match="residual buffer is too small"):
        prep.execute(w, lat, 1.0, res[:15], emb, adaln, height=8, width=8, dim=256)
    with pytest.raises(animaxs_amd.AnimaError, match=r"x_embedder must be \[128, 68\]"):
        prep.execute(w, lat, 1.0, res, emb, adaln, height=8, width=8, dim=128)
    vel = torch.empty(16 * 64, device="cuda")
    with pytest.raises(animaxs_amd.AnimaError, match="velocity buffer is too small"):
        fin.execute(w, res, emb, adaln, vel[:-1], height=8, width=8, dim=256)
    bad = dict(w)
    bad["mod_w2"] = w["proj"]
    with pytest.raises(animaxs_amd.AnimaError, match="adaln_modulation.2 must be"):
        fin.execute(bad, res, emb, adaln, vel, height=8, width=8, dim=256)


# --------------------------------------------------------------------------------------
# One whole sampler step: DiffusionSampler.swift:212-250 at a 32x32 latent (256 tokens)
# over two DiT blocks.
# --------------------------------------------------------------------------------------

def test_sampler_step_matches_oracle(ctx):
    H = W = 32
    T, dim, nblk = 256, 2048, 2
    io = inputs.dit_io(H, W)
    ds = [inputs.dit_block(S=T, seed=9100 + i) for i in range(nblk)]
    for d in ds[1:]:  # one generation: every block attends to the same context
        d["ctx"] = ds[0]["ctx"]
    print(f"SAMPLER step H={H} W={W} blocks={nblk}", flush=True)
    keep = []
    pw, k1 = _device_weights(io, ("x_embed", "t_embed1", "t_embed2"))
    fw, k2 = _device_weights(io, ("mod_w1", "mod_w2", "proj"))
    keep += [k1, k2]
    pw["t_norm"] = dev(io["t_norm"])
    dev_blocks = []
    for d in ds:
        bw = {}
        for name, w in d["w"].items():
            q, k = device_weight(w)
            bw[name] = q
            keep.append(k)
        for br in ("self", "cross", "mlp"):
            for i in (1, 2):
                q, k = fp16_weight(d[f"mod_{br}_w{i}"])
                bw[f"mod_{br}_w{i}"] = q
                keep.append(k)
        dev_blocks.append((bw, {n: dev(d[n]) for n in DiTBlockExecutor.NORMS}))
    ctx_tokens, rope = dev(ds[0]["ctx"]), dev(ds[0]["rope"])

    step, sigma, nsigma = 3, EulerSampler.SIGMAS[3], EulerSampler.SIGMAS[4]
    latent = dev(io["latent"][:, :H, :W].contiguous())
    res = torch.empty(T, dim, device="cuda")
    emb = torch.empty(dim, device="cuda")
    adaln = torch.empty(3 * dim, device="cuda")
    vel = torch.empty(16, H, W, device="cuda")
    den = torch.empty_like(vel)
    nxt = torch.empty_like(vel)
    DiTPreparationExecutor(ctx).execute(pw, latent, sigma, res, emb, adaln, height=H, width=W)
    DiTBlockExecutor(ctx).forward(dev_blocks, res, emb, adaln, ctx_tokens, rope, tokens=T)
    DiTFinalLayerExecutor(ctx).execute(fw, res, emb, adaln, vel, height=H, width=W)
    LatentOps(ctx).flow_velocity_to_denoised(latent, vel, den, sigma, vel.numel())
    EulerSampler(ctx).encode_step(latent, den, nxt, sigma, nsigma, vel.numel())
    torch.cuda.synchronize()

    lat = io["latent"][:, :H, :W].contiguous()
    r_res, r_emb, r_adaln = dit_io.prepare(lat, sigma, _wh(io["w"]["x_embed"]), _wf32(io["w"]["t_embed1"]),
                                           _wf32(io["w"]["t_embed2"]), io["t_norm"].float())
    x = r_res
    for d in ds:
        e = dict(d)
        e.update(x=x, emb=r_emb, adaln=r_adaln)
        x = blocks.dit_block(e, boundary="fp16")
    r_vel = dit_io.final_layer(x, r_emb, r_adaln, _wf32(io["w"]["mod_w1"]), _wf32(io["w"]["mod_w2"]),
                               _wh(io["w"]["proj"]), H, W)
    r_den = dit_io.flow_to_denoised(lat, r_vel, sigma)
    r_nxt = dit_io.euler_step(lat, r_den, sigma, nsigma)
    for name, y, r in (("velocity", vel, r_vel), ("x_next", nxt, r_nxt)):
        y = y.cpu()
        assert torch.isfinite(y).all()
        ma, mr = max_abs(y, r), mean_rel(y, r)
        print(f"PARITY sampler step {step} {name}: max_abs={ma:.3e} mean_rel={mr:.3e}", flush=True)
        assert mr <= 1e-3
        assert ma <= 1e-2 * float(r.abs().max())
