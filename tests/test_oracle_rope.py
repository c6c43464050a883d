"""CPU: RoPE tables, split-half rotation and the normalisations, against the reference's
recorded RoPE table (tests/golden/dit_rope_subset.npz, taken from
scripts/oracle_out/dit_rope_oracle.npz), the anchors of AnimaXSTests/DitRoPETests.swift,
the hand values of DiTBlockTests.swift and fp64 closed forms.  No GPU needed."""

from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from oracle import norms, rope

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "dit_rope_subset.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


@pytest.fixture(scope="module")
def table32():
    return rope.dit_rope_table(1, 32, 32).numpy()


@pytest.fixture(scope="module")
def lib_table32():
    import animaxs_amd
    return animaxs_amd.DitRoPE.generate(1, 32, 32)


# --- configuration (DitRoPETests.swift:13-31) ------------------------------------------

def test_config_and_thetas(golden):
    dim_t, dim_h, dim_w, t_theta, h_theta = rope.dit_thetas()
    assert (dim_t, dim_h, dim_w) == (44, 42, 42)
    assert dim_t // 2 + dim_h // 2 + dim_w // 2 == 64
    assert tuple(golden["dims"]) == (44, 42, 42)
    assert float(h_theta) == pytest.approx(42870.938, abs=0.01)
    assert float(h_theta) == float(np.float32(10000.0 * 4.0 ** (42.0 / 40.0)))
    assert float(h_theta) == float(golden["h_theta"])
    assert float(t_theta) == 10000.0


# --- golden table ------------------------------------------------------------------------

@pytest.mark.parametrize("who", ["oracle", "lib"])
def test_matches_recorded_table(who, golden, table32, lib_table32):
    t = table32 if who == "oracle" else lib_table32
    tokens = golden["tokens"]
    ref = golden["rope"]
    got = t[tokens]
    # the recorded table comes from float32 numpy cos/sin of fp32 angles; allow a few ulp
    assert np.max(np.abs(got - ref)) <= 2e-6, np.max(np.abs(got - ref))


def test_grid_size_invariance(table32, lib_table32):
    """Angles depend only on (t, h, w): token (h, w) of the 32x32 table equals token
    h*64 + w of the 64x64 table."""
    t64 = rope.dit_rope_table(1, 64, 64).numpy()
    import animaxs_amd
    l64 = animaxs_amd.DitRoPE.generate(1, 64, 64)
    idx = np.array([h * 64 + w for h in range(32) for w in range(32)])
    assert np.array_equal(t64[idx], table32)
    assert np.array_equal(l64[idx], lib_table32)


def test_lib_equals_oracle_fp64_bound(lib_table32):
    """The library's table against an fp64 evaluation of the same angles."""
    dim_t, dim_h, dim_w, t_theta, h_theta = rope.dit_thetas()
    th = float(h_theta)

    def f(theta, dim):
        i = np.arange(0, dim, 2)[: dim // 2].astype(np.float32) / np.float32(dim)
        return 1.0 / np.power(float(theta), i.astype(np.float64))

    ft, fh, fw = f(10000.0, dim_t), f(th, dim_h), f(th, dim_w)
    H = W = 32
    ang = np.zeros((H * W, 64))
    for h in range(H):
        for w in range(W):
            tok = h * W + w
            ang[tok, :22] = 0.0 * ft
            ang[tok, 22:43] = h * fh
            ang[tok, 43:] = w * fw
    want = np.stack([np.cos(ang), -np.sin(ang), np.sin(ang), np.cos(ang)], -1).reshape(H * W, 64, 2, 2)
    assert np.max(np.abs(lib_table32 - want)) <= 5e-6


# --- DitRoPETests.swift anchors ---------------------------------------------------------

def _blk(t, tok, f):
    return t[tok, f].reshape(4)


@pytest.mark.parametrize("who", ["oracle", "lib"])
def test_anchors(who, table32, lib_table32):
    t = table32 if who == "oracle" else lib_table32
    assert t.shape == (1024, 64, 2, 2) and np.isfinite(t).all()
    assert abs(t.min() + 1.0) < 1e-3 and abs(t.max() - 1.0) < 1e-3
    for f in range(64):                                         # :45-56 token 0 identity
        assert np.allclose(_blk(t, 0, f), [1, 0, 0, 1], atol=1e-6)
    np.testing.assert_allclose(_blk(t, 1, 43), [0.5403023, -0.8414710, 0.8414710, 0.5403023], atol=1e-5)
    np.testing.assert_allclose(_blk(t, 17, 43), [-0.27516335, 0.96139747, -0.96139747, -0.27516335], atol=1e-5)
    np.testing.assert_allclose(_blk(t, 31, 43), [0.91474235, 0.40403765, -0.40403765, 0.91474235], atol=1e-5)
    np.testing.assert_allclose(_blk(t, 1, 22), [1, 0, 0, 1], atol=1e-6)
    np.testing.assert_allclose(_blk(t, 32, 22), [0.5403023, -0.8414710, 0.8414710, 0.5403023], atol=1e-5)
    tok = 32 + 5                                                 # :80-88 t,h,w ordering
    np.testing.assert_allclose(_blk(t, tok, 22), [0.5403023, -0.8414710, 0.8414710, 0.5403023], atol=1e-5)
    np.testing.assert_allclose(_blk(t, tok, 43), [math.cos(5), -math.sin(5), math.sin(5), math.cos(5)], atol=1e-5)
    np.testing.assert_allclose(_blk(t, tok, 0), [1, 0, 0, 1], atol=1e-6)


# --- NeoX (Qwen) table --------------------------------------------------------------------

@pytest.mark.parametrize("theta", [1.0e6, 1.0e4])
def test_neox_table_closed_form(theta):
    import animaxs_amd
    tokens, hd = 300, 128
    j = np.arange(hd // 2, dtype=np.float64)
    inv = 1.0 / np.power(theta, 2.0 * j / hd)
    ang = np.arange(tokens)[:, None] * inv[None, :]
    want = np.stack([np.cos(ang), -np.sin(ang), np.sin(ang), np.cos(ang)], -1).reshape(tokens, hd // 2, 2, 2)
    ora = rope.neox_rope_table(tokens, theta).numpy()
    lib = animaxs_amd.qwen_rope(tokens, hd, theta)
    # fp32 angle (pos * inv rounded) -> error grows like pos * ulp(inv)
    assert np.max(np.abs(ora - want)) <= 1e-4
    assert np.max(np.abs(lib - want)) <= 1e-4
    assert np.max(np.abs(lib - ora)) <= 1e-4


def test_neox_equals_rotate_half_form():
    """QwenNumerics' rotate-half RoPE: x*cos + rotate_half(x)*sin equals the split-half
    rotation with the NeoX table."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, 40, 2, 128, generator=g)
    t = rope.neox_rope_table(40)
    c = t[:, :, 0, 0]
    s = t[:, :, 1, 0]
    cos = torch.cat([c, c], -1)[None, :, None, :]
    sin = torch.cat([s, s], -1)[None, :, None, :]
    rot = torch.cat([-x[..., 64:], x[..., :64]], -1)
    want = x * cos + rot * sin
    assert torch.allclose(rope.apply_split_half(x, t), want, atol=1e-6)


# --- split-half rotation (DiTBlockTests.swift:18-63) --------------------------------------

def _tbl(blocks):
    return torch.tensor(blocks, dtype=torch.float32).reshape(1, len(blocks), 2, 2)


def test_split_half_identity():
    x = torch.tensor([1, 2, 3, 4, 10, 20, 30, 40], dtype=torch.float32).reshape(1, 1, 1, 8)
    out = rope.apply_split_half(x, _tbl([[1, 0, 0, 1]] * 4))
    assert torch.equal(out, x)


def test_split_half_rotation_hand_values():
    x = torch.tensor([1, 2, 3, 4], dtype=torch.float32).reshape(1, 1, 1, 4)
    out = rope.apply_split_half(x, _tbl([[0, -1, 1, 0], [-1, 0, 0, -1]])).reshape(-1)
    assert out.tolist() == [-3.0, -2.0, 1.0, -4.0]   # adjacent pairing would give -2, -3


# --- normalisations (DiTBlockTests.swift:66-114, :168-172) --------------------------------

def test_layer_norm_hand_values():
    x = torch.tensor([0.0, 1.0, 2.0, 3.0])
    std = math.sqrt(1.25)
    want = torch.tensor([(v - 1.5) / std for v in [0, 1, 2, 3]])
    assert torch.allclose(norms.layer_norm(x, eps=0.0), want, atol=1e-6)
    assert torch.allclose(norms.layer_norm(x), want, atol=1e-5)
    scale = torch.tensor([0.0, 1, 0, -1])
    shift = torch.tensor([1.0, 2, 3, 4])
    assert torch.allclose(norms.layer_norm_modulated(x, scale, shift), want * (1 + scale) + shift, atol=1e-5)
    assert torch.allclose(norms.layer_norm(x), torch.nn.functional.layer_norm(x, (4,), eps=1e-6), atol=1e-6)


def test_rms_norm_heads_shared_weight():
    w = torch.tensor([1.0, 2, 3, 4])
    x = torch.tensor([[[(t + 1) * 10 + (h + 1) + d for d in range(4)] for h in range(2)] for t in range(2)],
                     dtype=torch.float32)
    out = norms.rms_norm(x, w)
    for t in range(2):
        for h in range(2):
            v = x[t, h].double()
            inv = 1.0 / math.sqrt(float((v * v).sum()) / 4 + 1e-6)
            assert torch.allclose(out[t, h].double(), v * inv * w.double(), atol=1e-5)
    assert torch.allclose(out, torch.nn.functional.rms_norm(x, (4,), w, eps=1e-6), atol=1e-6)


def test_gelu_exact_values():
    out = norms.gelu_erf(torch.tensor([0.0, 1.0, -1.0]))
    np.testing.assert_allclose(out.numpy(), [0.0, 0.84134474, -0.15865526], atol=1e-6)
    x = torch.linspace(-6, 6, 97)
    want = torch.tensor([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x.double().tolist()], dtype=torch.float64)
    assert torch.allclose(norms.gelu_erf(x).double(), want, atol=1e-6)


def test_silu_closed_form():
    x = torch.linspace(-10, 10, 101)
    want = torch.tensor([v / (1 + math.exp(-v)) for v in x.double().tolist()], dtype=torch.float64)
    assert torch.allclose(norms.silu(x).double(), want, atol=1e-6)
