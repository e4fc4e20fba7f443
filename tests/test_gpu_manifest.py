"""Layers bound from the reference's packs and banks (axk.manifest) run on the GPU exactly as the same weights passed as
loose tensors: the 9B group's MXFP4 layers (banks, column strips) and the 35B group's MXFP8 GDN layer (column blocks),
through axk_gdn_layer_decode / axk_attn_layer_decode. Bit-identical outputs, states and caches."""
import os

import pytest
import torch

from axk import configs, layer
from axk import manifest as mf
from oracle import layer as olayer

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "manifests")


def _bound(m, role, layer_idx, w, dev):
    k = m.kernel(role)
    kind = k.kinds()[layer_idx]
    names = set(k.packs) | {f"k_b{layer_idx % 4}_{b}" for b in mf.BANKS[kind]}
    bufs = {e.name: torch.zeros(e.bytes, dtype=torch.uint8, device=dev) for e in k.inputs if e.name in names}
    for e in k.inputs:
        if any(e.name == f"{b}{layer_idx}" for b in mf.EXPERT_IO):
            bufs[e.name] = torch.zeros(e.bytes, dtype=torch.uint8, device=dev)
    m.store_layer(role, bufs, layer_idx, w)
    return m.bind_layer(role, bufs, layer_idx), bufs


def _gdn_run(x, w, st, cv, nk, nv, fmt):
    o, so, co = layer.gdn_layer_decode(x, w, st.clone(), cv.clone(), nk, nv, proj_fmt=fmt[0], mlp_fmt=fmt[1])
    torch.cuda.synchronize()
    return o, so, co


@pytest.mark.parametrize("path,layer_idx,h,f,fmt", [
    ("qwen35_9b_c131072.manifest.json", 0, 4096, 12288, "mxfp4"),
    ("qwen35_35b_a3b.manifest.json", 1, 2048, 512, "mxfp8"),
])
def test_bound_gdn_layer_runs_like_loose_tensors(dev, path, layer_idx, h, f, fmt):
    m = mf.Manifest.load(os.path.join(HERE, path))
    g = torch.Generator().manual_seed(layer_idx + h)
    w = configs.gdn_layer_weights(g, h, f, 16, 32, proj_fmt=fmt, mlp_fmt=fmt)
    if m.model == "qwen35_moe":
        w["w_router"] = (torch.randn(256, h, generator=g) * 0.02).bfloat16()
        w["w_shg"] = (torch.randn(h, generator=g) * 0.02).bfloat16()
    wd = {n: t.to(dev) for n, t in w.items()}
    b, bufs = _bound(m, "decode.group", layer_idx, wd, dev)
    print(f"{m.model} layer {layer_idx}: {b.kind} {b.proj_fmt}/{b.mlp_fmt}", flush=True)
    assert (b.proj_fmt, b.mlp_fmt) == (fmt, fmt)
    x = torch.randn(2, h, generator=g).bfloat16().to(dev)
    st = (torch.randn(2, 32, 128, 128, generator=g) * 0.02).to(dev)
    cv = torch.randn(2, 3, 8192, generator=g).bfloat16().to(dev)
    ref = _gdn_run(x, wd, st, cv, 16, 32, (fmt, fmt))
    got = _gdn_run(x, b.weights, st, cv, 16, 32, (b.proj_fmt, b.mlp_fmt))
    for r, t in zip(ref, got):
        assert torch.equal(r.view(torch.uint8), t.view(torch.uint8))


def test_bound_9b_attention_layer_runs_like_loose_tensors(dev):
    m = mf.Manifest.load(os.path.join(HERE, "qwen35_9b_c131072.manifest.json"))
    g = torch.Generator().manual_seed(3)
    hq, hkv, d, page = 16, 4, 256, 256
    w = configs.attn_layer_weights(g, 4096, 12288, hq, hkv, d, proj_fmt="mxfp4", mlp_fmt="mxfp4")
    wd = {n: t.to(dev) for n, t in w.items()}
    b, _ = _bound(m, "decode.group", 3, wd, dev)
    assert b.kind == "attn" and (b.proj_fmt, b.mlp_fmt) == ("mxfp4", "mxfp4")
    c = configs.append_token_case([300, 1000, 256], hq, hkv, d, page, g)
    x = torch.randn(3, 4096, generator=g).bfloat16().to(dev)
    cos, sin = olayer.rope_cos_sin(c["pos"], 64, 10_000_000.0)
    args = [cos.to(dev), sin.to(dev)]
    meta = [c["indptr"].to(dev), c["indices"].to(dev), c["last_page_len"].to(dev), c["loc"].to(dev)]
    outs = []
    for weights in (wd, b.weights):
        cache = c["cache"].to(dev)
        o = layer.attn_layer_decode(x, weights, *args, cache, *meta, hq, 64, proj_fmt="mxfp4", mlp_fmt="mxfp4")
        torch.cuda.synchronize()
        outs.append((o, cache))
    assert torch.equal(outs[0][0].view(torch.int16), outs[1][0].view(torch.int16))
    assert torch.equal(outs[0][1].view(torch.int16), outs[1][1].view(torch.int16))


def test_bound_35b_moe_layer_runs_like_loose_tensors(dev):
    """The 35B group's GDN layer as the reference binds it, MoE block included (the router and shared gate from its
    packs, the routed experts e_gw<j> .. as their own IO): axk_gdn_layer_decode_moe on the bound tensors equals the
    call on the same weights as loose tensors, bit for bit."""
    m = mf.Manifest.load(os.path.join(HERE, "qwen35_35b_a3b.manifest.json"))
    g = torch.Generator().manual_seed(35)
    h, f = 2048, 512
    w = configs.gdn_layer_weights(g, h, f, 16, 32, proj_fmt="mxfp8", mlp_fmt="mxfp8")
    blk = configs.moe_block(g, h, 256, 512, 8)
    w["w_router"], w["w_shg"] = blk["w_router"], blk["w_shg"]
    wd = {n: t.to(dev) for n, t in w.items()}
    b, bufs = _bound(m, "decode.group", 1, wd, dev)
    for n in mf.EXPERT_IO:
        bufs[f"{n}1"].copy_(blk[n].reshape(-1).to(dev))
    print(f"{m.model} layer 1: {b.kind} {b.proj_fmt}/{b.mlp_fmt}", flush=True)
    names = ("w_router", "w_shg") + mf.EXPERT_IO
    bound = dict({n: b.weights[n] for n in names}, top_k=8)
    loose = dict({n: (blk[n] if n in mf.EXPERT_IO else w[n]).to(dev) for n in names}, top_k=8)
    x = torch.randn(2, h, generator=g).bfloat16().to(dev)
    st = (torch.randn(2, 32, 128, 128, generator=g) * 0.02).to(dev)
    cv = torch.randn(2, 3, 8192, generator=g).bfloat16().to(dev)
    outs = []
    for weights, moe in ((wd, loose), (b.weights, bound)):
        o = layer.gdn_layer_decode(x, weights, st.clone(), cv.clone(), 16, 32, proj_fmt=b.proj_fmt,
                                   mlp_fmt=b.mlp_fmt, moe=moe)
        torch.cuda.synchronize()
        outs.append(o)
    for r, t in zip(*outs):
        assert torch.equal(r.view(torch.uint8), t.view(torch.uint8))
