"""GPU parity of the MoE decode layers (axk_gdn_layer_decode_moe / axk_attn_layer_decode_moe through the C-ABI): the
decode layers with the 35B's MoE block as their MLP (moe_full, models/qwen35_35b_a3b/src/70b0fbc/q35_layer_mc.py:
797-853): the shared expert in the layer's MLP format (MXFP8 in the 35B manifest), router, top-K and the MXFP4 routed
experts.

Bars (those of tests/test_gpu_layer.py and tests/test_gpu_moe.py together):
  * the routing from the kernel's own logits: ids bit-exact against a stable descending sort of them, weights at
    fp32 tolerance; the logits within the per-op bar of the oracle's (h2 is a bf16 result of the layer's first half);
  * the output within the reference's fused-layer bar rel 5e-2 / abs 0.0625 (test_gdn_attn.py:348-354, 537) of the
    oracle on the kernel's routing, plus the derived slack for one-ulp flips of the bf16 expert activations
    (oracle.moe.moe_parts);
  * GDN state / conv state and the KV rows as the dense layers.
"""
import pytest
import torch

from axk import _lib, configs, layer
from oracle import layer as olayer
from oracle import moe as omoe

pytestmark = pytest.mark.gpu
TOL = dict(rtol=2e-2, atol=1e-2)
FUSED_TOL = dict(rtol=5e-2, atol=0.0625)
STATE_TOL = dict(rtol=5e-2, atol=3e-3)


def _dev(w, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in w.items()}


def _routing_outputs(b, blk, dev):
    e, k = blk["w_router"].shape[0], blk["top_k"]
    return dict(logits=torch.empty(b, e, device=dev), topk_ids=torch.empty(b, k, dtype=torch.int32, device=dev),
                topk_weights=torch.empty(b, k, device=dev))


def _check_moe(out, r, x, y, w, blk, fmt):
    """out [B, H] of the kernel, r its routing outputs; x the layer input, y the oracle's first half."""
    logits, ids, wts = r["logits"].cpu(), r["topk_ids"].cpu(), r["topk_weights"].cpu()
    sids, swts = omoe.route(logits, blk["top_k"], True)
    assert torch.equal(ids, sids), "top-K ids differ from the stable sort of the kernel's logits"
    torch.testing.assert_close(wts, swts, rtol=1e-5, atol=1e-6)
    base, routed, slack, ref_logits, _, _ = olayer.moe_block_parts(x, y, w, blk, fmt=fmt, ids=ids.long(), wts=wts)
    torch.testing.assert_close(logits, ref_logits, **TOL)
    ref = (base + routed).bfloat16().float()
    d = (out.float().cpu() - ref).abs()
    tol = FUSED_TOL["atol"] + FUSED_TOL["rtol"] * ref.abs()
    assert (d <= tol + slack).all(), f"max excess {(d - tol - slack).max().item()}"


@pytest.mark.parametrize("b,h,f,nk,nv,e,fe,k,fmt", [
    (3, 256, 256, 2, 4, 16, 256, 4, "mxfp8"),
    (5, 256, 512, 2, 4, 40, 256, 8, "mxfp4"),
    (3, 256, 256, 2, 4, 16, 256, 4, "nvfp4"),  # an NVFP4 shared expert
    (2, 2048, 512, 16, 32, 256, 512, 8, "mxfp8"),  # the 35B's widths (hidden 2048, 256 experts of 512, top-8)
    (32, 2048, 512, 16, 32, 256, 512, 8, "mxfp8"),  # the bench's moe_layer_decode: the 35B's widths at 32 sequences
])
def test_gdn_layer_decode_moe(dev, b, h, f, nk, nv, e, fe, k, fmt):
    g = torch.Generator().manual_seed(b * 100 + e)
    print(f"gdn moe b={b} h={h} e={e} fe={fe} k={k} {fmt}", flush=True)
    w = configs.gdn_layer_weights(g, h, f, nk, nv, proj_fmt="mxfp8", mlp_fmt=fmt)
    blk = configs.moe_block(g, h, e, fe, k)
    x = torch.randn(b, h, generator=g).bfloat16()
    st = torch.randn(b, nv, 128, 128, generator=g) * 0.02
    cv = torch.randn(b, 3, 2 * nk * 128 + nv * 128, generator=g).bfloat16()
    r = _routing_outputs(b, blk, dev)
    out, so, co = layer.gdn_layer_decode(x.to(dev), _dev(w, dev), st.to(dev), cv.to(dev), nk, nv, proj_fmt="mxfp8",
                                         mlp_fmt=fmt, moe=dict(_dev(blk, dev), **r))
    y, rs, rc = olayer.gdn_layer_half(x, w, st, cv, nk, nv, proj_fmt="mxfp8")
    _check_moe(out, r, x, y, w, blk, fmt)
    torch.testing.assert_close(so.cpu(), rs, **STATE_TOL)
    assert torch.equal(co[:, :-1].cpu(), rc[:, :-1])


@pytest.mark.parametrize("lens,hq,hkv,e,fe,k,fmt", [([100, 64, 300], 4, 2, 16, 256, 4, "mxfp8"),
                                                    ([17 + 9 * i for i in range(20)], 4, 2, 64, 256, 8, "mxfp4")])
def test_attn_layer_decode_moe(dev, lens, hq, hkv, e, fe, k, fmt):
    g = torch.Generator().manual_seed(len(lens) * 11 + e)
    h, f, d = 256, 256, 256
    print(f"attn moe lens={len(lens)} e={e} {fmt}", flush=True)
    w = configs.attn_layer_weights(g, h, f, hq, hkv, d, proj_fmt="mxfp8", mlp_fmt=fmt)
    blk = configs.moe_block(g, h, e, fe, k)
    c = configs.append_token_case(lens, hq, hkv, d, 64, g)
    x = torch.randn(len(lens), h, generator=g).bfloat16()
    cos, sin = olayer.rope_cos_sin(c["pos"], 64, 10_000_000.0)
    cache = c["cache"].to(dev)
    r = _routing_outputs(len(lens), blk, dev)
    out = layer.attn_layer_decode(x.to(dev), _dev(w, dev), cos.to(dev), sin.to(dev), cache, c["indptr"].to(dev),
                                  c["indices"].to(dev), c["last_page_len"].to(dev), c["loc"].to(dev), hq, 64,
                                  proj_fmt="mxfp8", mlp_fmt=fmt, moe=dict(_dev(blk, dev), **r))
    y, rcache = olayer.attn_layer_half(x, w, cos, sin, c["cache"], c["indptr"], c["indices"], c["last_page_len"],
                                       c["loc"], hq, 64, proj_fmt="mxfp8")
    _check_moe(out, r, x, y, w, blk, fmt)
    got = cache.cpu()
    written = torch.zeros(got.shape[0], got.shape[2], dtype=torch.bool)
    for p, o in c["loc"].tolist():
        written[p, o] = True
    torch.testing.assert_close(got.permute(0, 2, 1, 3, 4)[written].float(),
                               rcache.permute(0, 2, 1, 3, 4)[written].float(), **TOL)
    assert torch.equal(got.permute(0, 2, 1, 3, 4)[~written].view(torch.int16),
                       c["cache"].permute(0, 2, 1, 3, 4)[~written].view(torch.int16))


def test_moe_layer_routing_stays_in_the_workspace_without_outputs(dev):
    """Without routing outputs the call gives the same layer output (the routing lives in the workspace)."""
    g = torch.Generator().manual_seed(9)
    w = configs.gdn_layer_weights(g, 256, 256, 2, 4, proj_fmt="mxfp8", mlp_fmt="mxfp8")
    blk = configs.moe_block(g, 256, 16, 256, 4)
    x = torch.randn(3, 256, generator=g).bfloat16().to(dev)
    st = (torch.randn(3, 4, 128, 128, generator=g) * 0.02).to(dev)
    cv = torch.randn(3, 3, 1024, generator=g).bfloat16().to(dev)
    wd, bd = _dev(w, dev), _dev(blk, dev)
    a, _, _ = layer.gdn_layer_decode(x, wd, st, cv, 2, 4, proj_fmt="mxfp8", mlp_fmt="mxfp8", moe=bd)
    r = _routing_outputs(3, blk, dev)
    b, _, _ = layer.gdn_layer_decode(x, wd, st, cv, 2, 4, proj_fmt="mxfp8", mlp_fmt="mxfp8", moe=dict(bd, **r))
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_moe_layer_late_contract_error_enqueues_nothing(dev):
    """A misaligned routed-expert weight (checked in the MoE block, the layer's last step) returns AXK_E_ALIGN before
    anything is launched: the recurrent and conv states are unchanged."""
    g = torch.Generator().manual_seed(23)
    w = configs.gdn_layer_weights(g, 256, 256, 2, 4, proj_fmt="mxfp8", mlp_fmt="mxfp8")
    blk = _dev(configs.moe_block(g, 256, 16, 256, 4), dev)
    raw = torch.zeros(blk["e_dw"].numel() + 16, dtype=torch.uint8, device=dev)
    raw[1:1 + blk["e_dw"].numel()] = blk["e_dw"].reshape(-1)
    blk["e_dw"] = raw[1:1 + blk["e_dw"].numel()].view(blk["e_dw"].shape)  # one byte off a 16-byte boundary
    x = torch.randn(3, 256, generator=g).bfloat16()
    st = torch.randn(3, 4, 128, 128, generator=g) * 0.02
    cv = torch.randn(3, 3, 1024, generator=g).bfloat16()
    sd, cd = st.to(dev), cv.to(dev)
    with pytest.raises(_lib.AxkError) as e:
        layer.gdn_layer_decode(x.to(dev), _dev(w, dev), sd, cd, 2, 4, state_out=sd, conv_out=cd, proj_fmt="mxfp8",
                               mlp_fmt="mxfp8", moe=blk)
    assert e.value.status == 3  # AXK_E_ALIGN
    torch.cuda.synchronize()
    assert torch.equal(sd.cpu(), st) and torch.equal(cd.cpu(), cv)
