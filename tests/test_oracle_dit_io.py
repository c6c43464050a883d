"""CPU: pin the DiT input / output and sampler oracle (oracle/dit_io.py).

Known answers come from the reference's own tests (TimestepEmbedderTests.swift,
DiTInputTests.swift, MetalExecutionTests.swift checkPatchRoundTrip / checkEuler) with the
expected values worked out by hand here; the prepare and final-layer compositions are pinned
by closed forms in which a swapped shift/scale, a wrong half of the sinusoid or a transposed
patch index changes the result by far more than the tolerance.
"""

import math

import numpy as np
import pytest
import torch

from oracle import dit_io


# ------------------------------------------------------------------ timestep sinusoid

def test_sinusoid_known_answers():
    """TimestepEmbedderTests.swift:18-34 (torch fp32 values at sigma = 1)."""
    s = dit_io.timestep_sinusoid(1.0, 2048)
    assert s.shape == (2048,) and s.dtype == torch.float32
    cos_ref = [0.54030234, 0.5478152, 0.5552175, 0.56251031, 0.56969506, 0.57677263, 0.58374441, 0.59061158]
    sin_ref = [0.84147096, 0.83659935, 0.83170521, 0.82679027, 0.8218562, 0.81690472, 0.81193745, 0.80695599]
    np.testing.assert_allclose(s[:8].numpy(), cos_ref, atol=1e-6, rtol=0)
    np.testing.assert_allclose(s[1024:1032].numpy(), sin_ref, atol=1e-6, rtol=0)
    assert abs(float(s[1]) - math.cos(0.99104583)) <= 1e-6
    # DiTInputTests.swift:67-73: angle 0 is sigma itself
    assert abs(float(s[0]) - math.cos(1.0)) <= 1e-6 and abs(float(s[1024]) - math.sin(1.0)) <= 1e-6


@pytest.mark.parametrize("sigma", dit_io.SIGMAS)
def test_sinusoid_fp64_closed_form(sigma):
    for dim in (2048, 64):
        half = dim // 2
        i = np.arange(half, dtype=np.float64)
        ang = sigma * np.exp(-math.log(10000.0) * i / half)
        ref = np.concatenate([np.cos(ang), np.sin(ang)])
        np.testing.assert_allclose(dit_io.timestep_sinusoid(sigma, dim).double().numpy(), ref, atol=2e-6, rtol=0)


# ------------------------------------------------------------------ patch layouts

def test_patchify_markers():
    """DiTInputTests.swift:14-52: channel-0 pixel markers land at features 0..3 of token 0."""
    x = np.zeros((17, 64, 64), np.float32)
    x[0, 0, 0], x[0, 0, 1], x[0, 1, 0], x[0, 1, 1] = 1, 2, 3, 4
    t = dit_io._patchify_fast(torch.from_numpy(x)).numpy()
    assert t.shape == (1024, 68)
    assert list(t[0, :5]) == [1, 2, 3, 4, 0]
    x[1, 0, 0] = 7  # channel 1 starts at feature 4
    assert dit_io._patchify_fast(torch.from_numpy(x)).numpy()[0, 4] == 7


def _round_trip_input(C=17, H=4, W=6):
    """MetalExecutionTests.swift:548-552: value i -> (i*17 % 101)/10 - 5."""
    idx = np.arange(C * H * W)
    return (((idx * 17) % 101) / 10.0 - 5.0).astype(np.float32).reshape(C, H, W)


def test_patchify_hand_values_and_round_trip():
    x = _round_trip_input()
    t = dit_io.patchify17(x)
    assert t.shape == (6, 68)
    # token 1 = patch row 0, column 1: channel 0 pixels (0,2) (0,3) (1,2) (1,3) = inputs 2, 3, 8, 9
    np.testing.assert_allclose(t[1, 0:4], [-1.6, 0.1, -1.5, 0.2], atol=1e-6)
    # token 3 = patch row 1, column 0: channel 1 pixels (2,0) (2,1) (3,0) (3,1) = inputs 36, 37, 42, 43
    np.testing.assert_allclose(t[3, 4:8], [(36 * 17 % 101) / 10 - 5, (37 * 17 % 101) / 10 - 5,
                                           (42 * 17 % 101) / 10 - 5, (43 * 17 % 101) / 10 - 5], atol=1e-6)
    # the mask channel is channel 16 at features 64..67
    np.testing.assert_allclose(t[0, 64:68], x[16, 0:2, 0:2].reshape(-1))
    assert np.array_equal(dit_io.unpatchify16(t, 4, 6), x[:16])
    # the loop form equals the reshape/permute form of the source model (dit_source_oracle.py:367-373)
    assert np.array_equal(dit_io._patchify_fast(torch.from_numpy(x)).numpy(), t)
    # 16 input channels: the zero mask channel is appended
    t16 = dit_io.patchify17(x[:16])
    assert np.array_equal(t16[:, :64], t[:, :64]) and not t16[:, 64:].any()


def test_unpatchify_velocity_layout():
    """MetalExecutionTests.swift:573-591 with tokens 0, 1, 2, ...: the FinalLayer token stride is 64."""
    H, W = 4, 6
    tok = np.arange(6 * 64, dtype=np.float32).reshape(6, 64)
    v = dit_io.unpatchify_velocity16(tok, H, W)
    assert v[0, 0, 0] == 0 and v[0, 0, 1] == 16 and v[0, 1, 0] == 32 and v[0, 1, 1] == 48
    assert v[1, 0, 0] == 1 and v[15, 0, 0] == 15
    assert v[0, 0, 2] == 64 and v[0, 2, 0] == 3 * 64          # token 1 and token 3 (patch row 1)
    assert v[5, 3, 5] == 5 * 64 + 3 * 16 + 5                  # token 5, di = dj = 1, channel 5
    # the source model's unpatchify (dit_source_oracle.py:375-382) as reshapes
    assert np.array_equal(dit_io._unpatchify_velocity_fast(torch.from_numpy(tok), H, W).numpy(), v)


# ------------------------------------------------------------------ sampler update

def test_euler_hand_values():
    """MetalExecutionTests.swift:680-710 vectors; x + (x - d) * (-0.125 / 0.75) worked by hand."""
    x = torch.tensor([-2, -0.5, 0, 1, 3], dtype=torch.float32)
    d = torch.tensor([1, -1, 2, 0.25, -4], dtype=torch.float32)
    y = dit_io.euler_step(x, d, 0.75, 0.625)
    np.testing.assert_allclose(y.numpy(), [-1.5, -0.5 - 1 / 12, 1 / 3, 0.875, 3 - 7 / 6], atol=1e-6, rtol=0)


def test_euler_last_step_returns_denoised_and_flow_composition():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(4096, generator=g)
    v = torch.randn(4096, generator=g)
    for s, ns in zip(dit_io.SIGMAS[:-1], dit_io.SIGMAS[1:]):
        d = dit_io.flow_to_denoised(x, v, s)
        y = dit_io.euler_step(x, d, s, ns)
        # (x - d) / s == v, so the step is x + (ns - s) * v
        np.testing.assert_allclose(y.numpy(), (x + (ns - s) * v).numpy(), atol=2e-6, rtol=1e-6)
    d = dit_io.flow_to_denoised(x, v, dit_io.SIGMAS[-2])
    np.testing.assert_allclose(dit_io.euler_step(x, d, dit_io.SIGMAS[-2], 0.0).numpy(), d.numpy(), atol=1e-6)


def test_schedule():
    """EulerSampler.sigmas (EulerSampler.swift:7-17): 8 steps from 1 to 0, strictly decreasing."""
    s = dit_io.SIGMAS
    assert len(s) == 9 and s[0] == 1.0 and s[-1] == 0.0
    assert all(a > b for a, b in zip(s, s[1:]))


# ------------------------------------------------------------------ compositions (closed forms)

def test_prepare_closed_form_identity_weights():
    H, W, dim = 8, 6, 128
    latent = torch.randn(16, H, W, generator=torch.Generator().manual_seed(5))
    xe = torch.zeros(dim, 68)
    xe[:68, :68] = torch.eye(68)
    t2 = torch.zeros(3 * dim, dim)
    t2[:dim] = torch.eye(dim)
    sigma = 0.64468634
    res, emb, adaln = dit_io.prepare(latent, sigma, xe, torch.eye(dim), t2, torch.ones(dim), eps=1e-6)
    T = (H // 2) * (W // 2)
    assert res.shape == (T, dim)
    # residual[:, :68] = fp16(patches): token 2 of a 6-wide latent is patch (0, 2)
    assert torch.equal(res[2, 0:4], latent[0, 0:2, 4:6].reshape(-1).half().float())
    assert not res[:, 64:].any()                 # mask channel and unused rows are zero
    raw = dit_io.timestep_sinusoid(sigma, dim)
    np.testing.assert_allclose(emb.numpy(), (raw / math.sqrt(0.5 + 1e-6)).numpy(), rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(adaln[:dim].numpy(), (raw / (1 + torch.exp(-raw))).numpy(), rtol=1e-6)
    assert not adaln[dim:].any()


def test_final_layer_closed_form():
    """Rows a_t * (+1, -1, +1, ...): mean 0, LayerNorm +-1 (exact after the fp16 boundary), so
    with emb = 0 the modulation is adaln[:2*dim] and y = +-(1 + scale) + shift exactly."""
    H, W, dim = 4, 6, 128
    T = 6
    sign = torch.tensor([1.0 if k % 2 == 0 else -1.0 for k in range(dim)])
    residual = torch.stack([(1.0 + t) * sign for t in range(T)])
    adaln = torch.zeros(3 * dim)
    adaln[:dim] = 0.25          # shift
    adaln[dim:2 * dim] = 0.5    # scale
    adaln[2 * dim:] = 100.0     # the gate third is not read
    proj = torch.zeros(64, dim)
    proj[:, :64] = torch.eye(64)
    v = dit_io.final_layer(residual, torch.zeros(dim), adaln, torch.randn(32, dim), torch.randn(2 * dim, 32), proj,
                           H, W)
    y = torch.where(sign[:64] > 0, torch.tensor(1.75), torch.tensor(-1.25))
    # token t, element q = (di*2 + dj)*16 + c -> velocity[c, 2i+di, 2j+dj]
    for t in range(T):
        i, j = divmod(t, W // 2)
        for q in range(64):
            c, p = q % 16, q // 16
            assert float(v[c, 2 * i + p // 2, 2 * j + p % 2]) == float(y[q])
