"""Config 4 (the 16-layer hybrid decode group, (GDN, GDN, GDN, attention) x 4) on the GPU at its full widths:
hidden 4096, MLP 12288, batch 8, HQ 32 / HKV 4 / D 256, GDN 16 / 32 heads, FP8 projections, MXFP4 MLP.

  * one GDN layer and one attention layer of the group against the oracle, at a 4,096-token context (the size the
    oracle finishes in seconds). Both layer outputs are held to the reference's bar for fused layer outputs,
    rel 5e-2 / abs 0.0625 (models/qwen35_35b_a3b/sgl/tests/test_gdn_attn.py:348-354, 537): at these widths the MLP's
    down output reaches |d| of 4 to 8 before the residual add, so one bf16 rounding flip of d (both sides round it,
    from fp32 sums taken in different orders) moves an output that the residual has cancelled to near 0 by
    ulp(d) = 0.03125. The GDN state keeps the reference's temporal bar and the conv state the per-op bar;
  * the whole group at its full 131,072-token context, by properties that hold at any size: a HIP-graph replay of
    the 16-layer step equals the eager step bit for bit (outputs, GDN states, conv states, KV caches); the states
    and conv states advance in place; no KV byte outside the new token's slot changes; every output is finite; and
    the attention layer's output for sequence 0 over its full context matches the oracle.
The reference checks its group the same way, per-layer goldens plus a whole-group run
(models/qwen38_27b/decode/q35_group.py:413-437, 575-637).
"""
import pytest
import torch

from axk import configs, layer
from oracle import layer as olayer

pytestmark = pytest.mark.gpu
TOL = dict(rtol=2e-2, atol=1e-2)
FUSED_TOL = dict(rtol=5e-2, atol=0.0625)
STATE_TOL = dict(rtol=5e-2, atol=3e-3)


def _cpu(w):
    return {k: v.cpu() for k, v in w.items()}


def _attn_args(c):
    return c["cos"], c["sin"], c["indptr"], c["indices"], c["last_page_len"], c["loc"]


def _written_mask(cache, loc):
    m = torch.zeros(cache.shape[0], cache.shape[2], dtype=torch.bool, device=cache.device)
    m[loc[:, 0].long(), loc[:, 1].long()] = True
    return m


def test_config4_layers_at_4096_context(dev):
    c = configs.config4_group(dev, ctx=4096)
    c4 = c["cfg"]
    print(f"config4 widths, ctx {c4['ctx']}, batch {c4['batch']}", flush=True)
    x = c["x"]
    gl = c["layers"][0]
    out, so, co = layer.gdn_layer_decode(x, gl["w"], gl["state"], gl["conv"], c4["nk"], c4["nv"], c4["eps"])
    ro, rs, rc = olayer.gdn_layer_decode(x.cpu(), _cpu(gl["w"]), gl["state"].cpu(), gl["conv"].cpu(), c4["nk"],
                                         c4["nv"], c4["eps"])
    torch.testing.assert_close(out.float().cpu(), ro.float(), **FUSED_TOL)
    torch.testing.assert_close(so.cpu(), rs, **STATE_TOL)
    assert torch.equal(co[:, :-1].cpu(), rc[:, :-1])
    torch.testing.assert_close(co[:, -1].float().cpu(), rc[:, -1].float(), **TOL)

    al = c["layers"][3]
    cos, sin, indptr, indices, last, loc = _attn_args(c)
    before = al["cache"].cpu()
    out = layer.attn_layer_decode(x, al["w"], cos, sin, al["cache"], indptr, indices, last, loc, c4["hq"], c4["rot"],
                                  c4["eps"])
    ro, rcache = olayer.attn_layer_decode(x.cpu(), _cpu(al["w"]), cos.cpu(), sin.cpu(), before, indptr.cpu(),
                                          indices.cpu(), last.cpu(), loc.cpu(), c4["hq"], c4["rot"], c4["eps"])
    torch.testing.assert_close(out.float().cpu(), ro.float(), **FUSED_TOL)
    got = al["cache"].cpu()
    wm = _written_mask(got, loc.cpu())
    torch.testing.assert_close(got.permute(0, 2, 1, 3, 4)[wm].float(), rcache.permute(0, 2, 1, 3, 4)[wm].float(),
                               **TOL)
    assert torch.equal(got.permute(0, 2, 1, 3, 4)[~wm].view(torch.int16),
                       before.permute(0, 2, 1, 3, 4)[~wm].view(torch.int16))


def _step(c, x, y, ws_g, ws_a, inputs=None):
    """The group's 16 layers for one new token per sequence, states and caches in place; returns the last output
    buffer. inputs (optional) collects each layer's input."""
    c4 = c["cfg"]
    cos, sin, indptr, indices, last, loc = _attn_args(c)
    for L in c["layers"]:
        if inputs is not None:
            inputs.append(x.clone())
        if L["kind"] == "g":
            layer.gdn_layer_decode(x, L["w"], L["state"], L["conv"], c4["nk"], c4["nv"], c4["eps"], workspace=ws_g,
                                   out=y, state_out=L["state"], conv_out=L["conv"])
        else:
            layer.attn_layer_decode(x, L["w"], cos, sin, L["cache"], indptr, indices, last, loc, c4["hq"],
                                    c4["rot"], c4["eps"], workspace=ws_a, out=y)
        x, y = y, x
    return x


def test_config4_group_full_context(dev):
    c = configs.config4_group(dev)
    c4 = c["cfg"]
    b, h, f = c4["batch"], c4["hidden"], c4["inter"]
    print(f"config4 group, ctx {c4['ctx']}, batch {b}, {len(c['layers'])} layers", flush=True)
    ws_g = layer.gdn_workspace(b, h, c4["nk"], c4["nv"], f, dev)
    ws_a = layer.attn_workspace(b, h, c4["hq"], c4["hkv"], c4["d"], f, dev)
    gdn = [L for L in c["layers"] if L["kind"] == "g"]
    attn = [L for L in c["layers"] if L["kind"] == "a"]
    st0 = [L["state"].clone() for L in gdn]
    cv0 = [L["conv"].clone() for L in gdn]
    kv0 = [L["cache"].clone() for L in attn]
    loc = c["loc"]
    wm = _written_mask(kv0[0], loc)

    # eager step
    x0 = c["x"].clone()
    bufs = [x0.clone(), torch.empty_like(x0)]
    inputs = []
    out_e = _step(c, bufs[0], bufs[1], ws_g, ws_a, inputs).clone()
    torch.cuda.synchronize()
    assert torch.isfinite(out_e.float()).all()
    for xi in inputs:
        assert torch.isfinite(xi.float()).all()
    st_e = [L["state"].clone() for L in gdn]
    cv_e = [L["conv"].clone() for L in gdn]
    for s0, s1, c0, c1 in zip(st0, st_e, cv0, cv_e):
        assert torch.isfinite(s1).all() and not torch.equal(s0, s1)
        assert torch.equal(c1[:, :-1], c0[:, 1:])  # the conv state shifted in place by one token
    for k0, L in zip(kv0, attn):
        got = L["cache"].permute(0, 2, 1, 3, 4)
        ref = k0.permute(0, 2, 1, 3, 4)
        assert torch.equal(got[~wm].view(torch.int16), ref[~wm].view(torch.int16))  # only the new slots change
        assert torch.isfinite(got[wm].float()).all()
    kv_e = [L["cache"].permute(0, 2, 1, 3, 4)[wm].clone() for L in attn]

    # the attention layer at the full context, sequence 0, against the oracle: its pages gathered into a compact
    # host cache holding the state before the step
    al, xi = attn[0], inputs[3]
    cos, sin, indptr, indices, last, _ = _attn_args(c)
    n0 = int(indptr[1].item())
    pages = indices[:n0].long()
    cache0 = kv0[0][pages].cpu()
    loc0 = torch.tensor([[n0 - 1, int(loc[0, 1].item())]], dtype=torch.int32)
    ro, _ = olayer.attn_layer_decode(xi[:1].cpu(), _cpu(al["w"]), cos[:1].cpu(), sin[:1].cpu(), cache0,
                                     torch.tensor([0, n0], dtype=torch.int32), torch.arange(n0, dtype=torch.int32),
                                     last[:1].cpu(), loc0, c4["hq"], c4["rot"], c4["eps"])
    del cache0
    torch.testing.assert_close(inputs[4][:1].float().cpu(), ro.float(), **FUSED_TOL)

    # the same step as one HIP graph, from the same starting states: bit for bit the eager step
    for L, s0, c0 in zip(gdn, st0, cv0):
        L["state"].copy_(s0)
        L["conv"].copy_(c0)
    for L, k0 in zip(attn, kv0):
        L["cache"].copy_(k0)
    del kv0
    bufs = [torch.empty_like(x0), torch.empty_like(x0)]
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            out_g = _step(c, bufs[0], bufs[1], ws_g, ws_a)
    bufs[0].copy_(x0)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out_g.view(torch.int16), out_e.view(torch.int16))
    for L, s1, c1 in zip(gdn, st_e, cv_e):
        assert torch.equal(L["state"], s1)
        assert torch.equal(L["conv"].view(torch.int16), c1.view(torch.int16))
    for L, k1 in zip(attn, kv_e):
        assert torch.equal(L["cache"].permute(0, 2, 1, 3, 4)[wm].view(torch.int16), k1.view(torch.int16))
