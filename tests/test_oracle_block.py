"""CPU: wiring invariants of the DiT block composition oracle (oracle.blocks.dit_block,
following scripts/dit_block0_oracle.py:327-391) on a 16-token grid.  Each part it composes
is pinned in test_oracle_attention.py / test_oracle_rope.py / test_oracle_quant.py."""

from __future__ import annotations

import pytest
import torch

from oracle import blocks, inputs


@pytest.fixture(scope="module")
def small_block():
    d = inputs.dit_block(S=16, ctx_tokens=8)
    return d, blocks.dequant_weights(d)


def _with(d, **over):
    e = dict(d)
    e.update(over)
    return e


def test_zero_gates_leave_the_residual_unchanged(small_block):
    d, W = small_block
    dim = d["x"].shape[1]
    # modulation = SiLU(emb) W1^T W2^T + adaln: zero W2 and adaln -> shift = scale = gate = 0
    zero = {f"mod_{br}_w2": torch.zeros_like(d[f"mod_{br}_w2"]) for br in ("self", "cross", "mlp")}
    e = _with(d, adaln=torch.zeros(3 * dim), **zero)
    out = blocks.dit_block(e, weights=W)
    assert torch.equal(out, d["x"].float())


def test_branches_add_in_order(small_block):
    """x1 = x + g_self * self_branch; zeroing self_o removes exactly that branch."""
    d, W = small_block
    out, inter = blocks.dit_block(d, weights=W, return_intermediates=True)
    W0 = dict(W)
    W0["self_o"] = torch.zeros_like(W["self_o"])
    _, inter0 = blocks.dit_block(d, weights=W0, return_intermediates=True)
    assert torch.equal(inter0["x1"], d["x"].float())
    assert not torch.equal(inter["x1"], d["x"].float())
    assert torch.isfinite(out).all()


def test_modulation_chunks_shift_scale_gate(small_block):
    d, _ = small_block
    dim = d["x"].shape[1]
    adaln = torch.arange(3 * dim, dtype=torch.float32)
    z1 = torch.zeros_like(d["mod_self_w1"])
    sh, sc, ga = blocks.modulation(d["emb"], z1, d["mod_self_w2"], adaln)
    assert torch.equal(sh, adaln[:dim]) and torch.equal(sc, adaln[dim:2 * dim]) and torch.equal(ga, adaln[2 * dim:])
