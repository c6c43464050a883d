"""GPU: the DiT forward loop (DitForward.execute, DitForward.swift:78-112), the cross-attention
K/V cache (CrossKVCache, DiTBlockExecutor.swift:19-43, :1110-1161) and the streamed-weight
forward (WeightStreamer.swift:87-213), through the C ABI.

  * a multi-block forward matches the oracle applying the same blocks in turn;
  * a cache hit gives the same bits as a cache miss and as the uncached block (the reference's
    cache is exact by construction: it holds the attention's post-norm K and V);
  * the forward equals the blocks encoded one by one, and the streamed forward (host ranges
    copied through 1 or 2 device slots) equals the resident one, bit for bit.
"""

import ctypes as C

import numpy as np
import pytest
import torch

import animaxs_amd
from animaxs_amd import CrossKVCache, DiTBlockExecutor, WeightStreamer, _abi
from oracle import blocks, inputs
from tests.helpers import dev, device_weight, fp16_weight, max_abs, mean_rel

pytestmark = pytest.mark.gpu

NORMS = ("self_q_norm", "self_k_norm", "cross_q_norm", "cross_k_norm")


def _device_block(d):
    keep = []
    weights = {}
    for name, w in d["w"].items():
        qw, k = device_weight(w)
        weights[name] = qw
        keep.append(k)
    for br in ("self", "cross", "mlp"):
        for i in (1, 2):
            qw, k = fp16_weight(d[f"mod_{br}_w{i}"])
            weights[f"mod_{br}_w{i}"] = qw
            keep.append(k)
    norms_d = {n: dev(d[n]) for n in NORMS}
    return weights, norms_d, keep


def _shared(d):
    """The per-step inputs every block shares (one emb / adaln / context / rope)."""
    return dict(emb=dev(d["emb"]), adaln_lora=dev(d["adaln"]), context_tokens_buf=dev(d["ctx"]), rope=dev(d["rope"]))


def _blocks(S, n, hidden=8192):
    ds = [inputs.dit_block(S=S, hidden=hidden, seed=9000 + i) for i in range(n)]
    base = ds[0]
    for d in ds[1:]:  # one step's shared inputs: emb, adaln_lora, context, rope, residual
        for k in ("x", "emb", "adaln", "ctx", "rope"):
            d[k] = base[k]
    return ds


def test_cache_hit_equals_miss_and_uncached(ctx):
    S = 1024
    d = inputs.dit_block(S=S)
    weights, norms_d, keep = _device_block(d)
    sh = _shared(d)
    blk = DiTBlockExecutor(ctx)
    print("CACHE hit/miss S=1024", flush=True)

    r0 = dev(d["x"].clone())
    blk.encode(weights, norms_d, r0, tokens=S, **sh)
    cache = CrossKVCache(ctx, blocks=4, context_tokens=512, dim=2048)
    assert cache.bytes() == 4 * 2 * 512 * 2048 * 2
    assert not cache.is_ready(2)
    r1 = dev(d["x"].clone())
    blk.encode(weights, norms_d, r1, tokens=S, cache=cache, block_index=2, **sh)   # miss: fills slot 2
    assert cache.is_ready(2) and not cache.is_ready(1)
    r2 = dev(d["x"].clone())
    blk.encode(weights, norms_d, r2, tokens=S, cache=cache, block_index=2, **sh)   # hit
    torch.cuda.synchronize()
    assert torch.equal(r1.view(torch.int32), r0.view(torch.int32))
    assert torch.equal(r2.view(torch.int32), r1.view(torch.int32))
    # a reset forgets every block; the context is projected again
    cache.reset()
    assert not cache.is_ready(2)


def test_forward_matches_oracle_over_three_blocks(ctx):
    S, n = 256, 3
    ds = _blocks(S, n)
    dev_blocks = [_device_block(d) for d in ds]
    sh = _shared(ds[0])
    residual = dev(ds[0]["x"].clone())
    cache = CrossKVCache(ctx, blocks=n)
    print(f"FORWARD S={S} blocks={n}", flush=True)
    DiTBlockExecutor(ctx).forward([(w, nm) for w, nm, _ in dev_blocks], residual, tokens=S, cache=cache, **sh)
    torch.cuda.synchronize()
    x = ds[0]["x"].float()
    for d in ds:
        e = dict(d)
        e["x"] = x
        x = blocks.dit_block(e, boundary="fp16")
    y = residual.cpu()
    assert torch.isfinite(y).all()
    ma, mr = max_abs(y, x), mean_rel(y, x)
    print(f"PARITY dit_forward {n} blocks S{S}: max_abs={ma:.3e} mean_rel={mr:.3e}", flush=True)
    assert mr <= 1e-3
    assert ma <= 5e-3 * float(x.abs().max())
    assert all(cache.is_ready(i) for i in range(n))


def test_forward_equals_blocks_and_second_step_hits_cache(ctx):
    S, n = 256, 3
    ds = _blocks(S, n)
    dev_blocks = [_device_block(d) for d in ds]
    sh = _shared(ds[0])
    blk = DiTBlockExecutor(ctx)
    x0 = ds[0]["x"]
    print(f"FORWARD equals blocks S={S} blocks={n}", flush=True)

    seq = dev(x0.clone())
    for w, nm, _ in dev_blocks:
        blk.encode(w, nm, seq, tokens=S, **sh)
    cache = CrossKVCache(ctx, blocks=n)
    step1 = dev(x0.clone())
    blk.forward([(w, nm) for w, nm, _ in dev_blocks], step1, tokens=S, cache=cache, **sh)
    step2 = dev(x0.clone())   # the next sampler step with the same context: every block hits
    blk.forward([(w, nm) for w, nm, _ in dev_blocks], step2, tokens=S, cache=cache, **sh)
    torch.cuda.synchronize()
    assert torch.equal(step1.view(torch.int32), seq.view(torch.int32))
    assert torch.equal(step2.view(torch.int32), step1.view(torch.int32))


def test_forward_of_nine_blocks_equals_blocks(ctx):
    """The forward computes every block's modulation rows before the first block, up to 24
    matvecs per launch: 9 blocks make 27 matvecs per stage, so one launch of 24 and one of 3.
    The rows, and so the output, keep the bits of the blocks encoded one by one."""
    S, n = 256, 9
    ds = _blocks(S, n)
    dev_blocks = [_device_block(d) for d in ds]
    sh = _shared(ds[0])
    blk = DiTBlockExecutor(ctx)
    print(f"FORWARD equals blocks S={S} blocks={n}", flush=True)
    seq = dev(ds[0]["x"].clone())
    for w, nm, _ in dev_blocks:
        blk.encode(w, nm, seq, tokens=S, **sh)
    fwd = dev(ds[0]["x"].clone())
    blk.forward([(w, nm) for w, nm, _ in dev_blocks], fwd, tokens=S, **sh)
    torch.cuda.synchronize()
    assert torch.isfinite(fwd).all()
    assert torch.equal(fwd.view(torch.int32), seq.view(torch.int32))


# --------------------------------------------------------------------------------------
# Streamed weights: every block's tensors packed into one contiguous host range (the pack's
# execution range), with a template whose pointers are offsets into that range.
# --------------------------------------------------------------------------------------

def _host_range(d):
    """(pinned uint8 tensor, template DitBlockWeights) for one block."""
    parts = []
    off = 0

    def put(arr) -> int:
        nonlocal off
        b = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
        at = (off + 255) // 256 * 256
        parts.append((at, b))
        off = at + b.size
        return at

    t = _abi.DitBlockWeights()
    for name, w in d["w"].items():
        p = put(np.asarray(w["packed"], np.uint8))
        s = put(np.asarray(w["scale_bits"], np.uint16))
        z = put(np.asarray(w["zero_bits"], np.uint16))
        setattr(t, name, _abi.QWeight(w["storage"], _abi.Buffer(C.c_void_p(p), 0), 0, _abi.Buffer(C.c_void_p(s), 0), 0,
                                      _abi.Buffer(C.c_void_p(z), 0), 0, w["rows"], w["cols"], w["row_stride"]))
    for br in ("self", "cross", "mlp"):
        for i in (1, 2):
            m = d[f"mod_{br}_w{i}"].numpy().view(np.uint16)
            p = put(m)
            setattr(t, f"mod_{br}_w{i}", _abi.QWeight(2, _abi.Buffer(C.c_void_p(p), 0), 0, _abi.Buffer(C.c_void_p(p), 0), 0,
                                                      _abi.Buffer(C.c_void_p(p), 0), 0, m.shape[0], m.shape[1],
                                                      m.shape[1]))
    for nm in NORMS:
        setattr(t, nm, _abi.Buffer(C.c_void_p(put(d[nm].numpy().view(np.uint16))), 0))
    host = torch.empty(off, dtype=torch.uint8, pin_memory=True)
    hv = host.numpy()
    for at, b in parts:
        hv[at:at + b.size] = b
    return host, t


@pytest.mark.parametrize("slots", [1, 2])
def test_streamed_forward_equals_resident(ctx, slots):
    S, n = 256, 3
    ds = _blocks(S, n, hidden=4096)
    dev_blocks = [_device_block(d) for d in ds]
    sh = _shared(ds[0])
    shape = dict(mlp_hidden=4096)
    blk = DiTBlockExecutor(ctx)
    x0 = ds[0]["x"]
    print(f"STREAMED forward slots={slots} S={S} blocks={n}", flush=True)
    resident = dev(x0.clone())
    blk.forward([(w, nm) for w, nm, _ in dev_blocks], resident, tokens=S, **sh, **shape)
    ranges = [_host_range(d) for d in ds]
    cap = max(h.numel() for h, _ in ranges)
    st = WeightStreamer(ctx, capacity=cap, slots=slots)
    streamed = dev(x0.clone())
    blk.forward_streamed(st, [t for _, t in ranges], [(h.data_ptr(), h.numel()) for h, _ in ranges], streamed,
                         tokens=S, **sh, **shape)
    torch.cuda.synchronize()
    assert torch.equal(streamed.view(torch.int32), resident.view(torch.int32))
    # a range larger than the slot is refused before anything is queued
    small = WeightStreamer(ctx, capacity=cap // 2, slots=slots)
    with pytest.raises(animaxs_amd.AnimaError, match="does not fit the weight slot"):
        blk.forward_streamed(small, [t for _, t in ranges], [(h.data_ptr(), h.numel()) for h, _ in ranges],
                             streamed, tokens=S, **sh, **shape)
