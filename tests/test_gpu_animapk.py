"""GPU: weights read out of a .animapk pack run through the executors exactly like weights
uploaded tensor by tensor.  A synthetic pack holds two DiT blocks (W4 projections, fp16
modulation and norms), the preparation and the final-layer tensors; the test compares, bit
for bit:

  * the forward over the blocks' execution ranges copied to the device and rebased
    (resident), streamed from the mapped pack through a 2-slot WeightStreamer
    (DitForward + WeightStreamer.swift:94-213), and built from per-tensor device buffers;
  * DiTPreparation / DiTFinalLayer from rebased pack ranges against per-tensor buffers.
"""

import ctypes as C

import numpy as np
import pytest
import torch

from animaxs_amd import (AnimapkFile, CrossKVCache, DiTBlockExecutor, DiTFinalLayerExecutor, DiTPreparationExecutor,
                         WeightStreamer)
from animaxs_amd import animapk as AP
from oracle import inputs
from tests import pack_writer as PW
from tests.helpers import dev, device_weight, fp16_weight

pytestmark = pytest.mark.gpu

PRE = "model.diffusion_model."
# oracle linear name -> pack suffix
LINEARS = {"self_q": "self_attn.q_proj.weight", "self_k": "self_attn.k_proj.weight",
           "self_v": "self_attn.v_proj.weight", "self_o": "self_attn.output_proj.weight",
           "cross_q": "cross_attn.q_proj.weight", "cross_k": "cross_attn.k_proj.weight",
           "cross_v": "cross_attn.v_proj.weight", "cross_o": "cross_attn.output_proj.weight",
           "mlp1": "mlp.layer1.weight", "mlp2": "mlp.layer2.weight"}
MODS = {"self": "adaln_modulation_self_attn", "cross": "adaln_modulation_cross_attn", "mlp": "adaln_modulation_mlp"}
NORMS = {"self_q_norm": "self_attn.q_norm.weight", "self_k_norm": "self_attn.k_norm.weight",
         "cross_q_norm": "cross_attn.q_norm.weight", "cross_k_norm": "cross_attn.k_norm.weight"}


def _block_blobs(i, d):
    p = f"{PRE}blocks.{i}."
    out = [PW.qweight_blob(p + LINEARS[n], d["w"][n]) for n in LINEARS]
    for br, stem in MODS.items():
        out += [PW.fp16_blob(p + stem + ".1.weight", d[f"mod_{br}_w1"].numpy()),
                PW.fp16_blob(p + stem + ".2.weight", d[f"mod_{br}_w2"].numpy())]
    out += [PW.fp16_blob(p + NORMS[n], d[n].numpy()) for n in NORMS]
    return out


def _device_block(d):
    keep, w = [], {}
    for name, qw in d["w"].items():
        q, k = device_weight(qw)
        w[name] = q
        keep.append(k)
    for br in MODS:
        for j in (1, 2):
            q, k = fp16_weight(d[f"mod_{br}_w{j}"])
            w[f"mod_{br}_w{j}"] = q
            keep.append(k)
    return w, {n: dev(d[n]) for n in NORMS}, keep


def _upload(r):
    host = np.frombuffer((C.c_uint8 * r.length).from_address(r.host), dtype=np.uint8)
    return torch.from_numpy(host.copy()).cuda()


@pytest.fixture(scope="module")
def pack(tmp_path_factory):
    S = 256
    ds = [inputs.dit_block(S=S, seed=9200 + i) for i in range(2)]
    for d in ds[1:]:
        for k in ("x", "emb", "adaln", "ctx", "rope"):
            d[k] = ds[0][k]
    io = inputs.dit_io(32, 32)
    blobs = _block_blobs(1, ds[1]) + _block_blobs(0, ds[0])   # block 1 stored first
    blobs += [PW.qweight_blob(PRE + "x_embedder.proj.1.weight", io["w"]["x_embed"]),
              PW.qweight_blob(PRE + "t_embedder.1.linear_1.weight", io["w"]["t_embed1"]),
              PW.qweight_blob(PRE + "t_embedder.1.linear_2.weight", io["w"]["t_embed2"]),
              PW.fp16_blob(PRE + "t_embedding_norm.weight", io["t_norm"].numpy()),
              PW.qweight_blob(PRE + "final_layer.adaln_modulation.1.weight", io["w"]["mod_w1"]),
              PW.qweight_blob(PRE + "final_layer.adaln_modulation.2.weight", io["w"]["mod_w2"]),
              PW.qweight_blob(PRE + "final_layer.linear.weight", io["w"]["proj"])]
    path = tmp_path_factory.mktemp("packs") / "dit.animapk"
    PW.write_pack(path, blobs)
    return path, ds, io


def test_forward_from_pack_resident_streamed_and_per_tensor(ctx, pack):
    path, ds, _ = pack
    S = 256
    print("PACK forward 2 blocks S=256", flush=True)
    f = AnimapkFile(path)
    assert f.crc32_mismatch_count() == 0
    templates, ranges, dev_ranges, resident = [], [], [], []
    for b in range(2):
        t, r = f.dit_block(b)
        templates.append(t)
        ranges.append(r)
        buf = _upload(r)
        dev_ranges.append(buf)
        resident.append(AP.rebase_block(t, buf.data_ptr(), r.length))
    assert ranges[1].file_offset < ranges[0].file_offset
    sh = dict(emb=dev(ds[0]["emb"]), adaln_lora=dev(ds[0]["adaln"]), context_tokens_buf=dev(ds[0]["ctx"]),
              rope=dev(ds[0]["rope"]))
    blk = DiTBlockExecutor(ctx)
    x0 = ds[0]["x"]

    per_tensor = [_device_block(d) for d in ds]
    ref = dev(x0.clone())
    blk.forward([(w, n) for w, n, _ in per_tensor], ref, tokens=S, **sh)
    out_res = dev(x0.clone())
    blk.forward(resident, out_res, tokens=S, cache=CrossKVCache(ctx, blocks=2), **sh)
    st = WeightStreamer(ctx, capacity=max(r.length for r in ranges), slots=2)
    out_st = dev(x0.clone())
    blk.forward_streamed(st, templates, [(r.host, r.length) for r in ranges], out_st, tokens=S, **sh)
    torch.cuda.synchronize()
    assert torch.isfinite(ref).all()
    assert torch.equal(out_res.view(torch.int32), ref.view(torch.int32))
    assert torch.equal(out_st.view(torch.int32), ref.view(torch.int32))
    f.close()


def test_prepare_and_final_from_pack(ctx, pack):
    path, _, io = pack
    H = W = 32
    T, dim = 256, 2048
    print("PACK preparation + final layer 32x32", flush=True)
    f = AnimapkFile(path)
    pt, pr = f.dit_prepare(dim)
    ft, fr = f.dit_final(dim)
    pbuf, fbuf = _upload(pr), _upload(fr)
    pw = AP.rebase_prepare(pt, pbuf.data_ptr(), pr.length)
    fw = AP.rebase_final(ft, fbuf.data_ptr(), fr.length)
    keep = []
    dw = {}
    for n in ("x_embed", "t_embed1", "t_embed2", "mod_w1", "mod_w2", "proj"):
        q, k = device_weight(io["w"][n])
        dw[n] = q
        keep.append(k)
    dw["t_norm"] = dev(io["t_norm"])
    latent = dev(io["latent"])
    outs = []
    for w_prep, w_fin in ((pw, fw), (dw, dw)):
        res = torch.empty(T, dim, device="cuda")
        emb = torch.empty(dim, device="cuda")
        adaln = torch.empty(3 * dim, device="cuda")
        vel = torch.empty(16, H, W, device="cuda")
        DiTPreparationExecutor(ctx).execute(w_prep, latent, 0.7511211, res, emb, adaln, height=H, width=W)
        DiTFinalLayerExecutor(ctx).execute(w_fin, res, emb, adaln, vel, height=H, width=W)
        outs.append((res, emb, adaln, vel))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    assert torch.isfinite(outs[0][3]).all()
    f.close()
