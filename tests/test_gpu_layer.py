"""GPU parity of whole hybrid decode layers (axk_gdn_layer_decode / axk_attn_layer_decode through the C-ABI)
against the oracle composed of the per-op restatements.

Bars:
  * GDN layer output within the per-op bar rel 2e-2 / abs 1e-2 of the oracle;
  * attention layer output within the reference's bar for fused (composed) layer outputs, rel 5e-2 / abs 0.0625
    (models/qwen35_35b_a3b/sgl/tests/test_gdn_attn.py:354, 517, 537): the attention kernel multiplies P in bf16
    (as the reference's own attention does) against an fp32 SDPA golden, and that difference passes through the
    o projection, the residual, the RMSNorm and the MLP (each of those ops meets the per-op bar in its own test);
  * the GDN state within the reference's temporal tolerance rel 5e-2 / abs 3e-3 (test_gdn_attn.py:711-712); the
    conv state's shifted entries exact (moved inputs), its newest entry (this token's qkv projection output, a bf16
    result of an fp32 sum) within the per-op bar; the KV rows written within the per-op bar, every other cache byte
    untouched.
"""
import pytest
import torch

from axk import configs, layer
from oracle import layer as olayer

pytestmark = pytest.mark.gpu
TOL = dict(rtol=2e-2, atol=1e-2)
FUSED_TOL = dict(rtol=5e-2, atol=0.0625)
STATE_TOL = dict(rtol=5e-2, atol=3e-3)
H, F = 256, 512


def _dev(w, dev):
    return {k: v.to(dev) for k, v in w.items()}


def _check_conv(got, ref):
    # [B, K-1, C]: entries 0 .. K-3 are the previous state shifted (exact); entry K-2 is the new token's projection
    assert torch.equal(got[:, :-1].cpu(), ref[:, :-1])
    torch.testing.assert_close(got[:, -1].float().cpu(), ref[:, -1].float(), **TOL)


def _gdn_case(seed, b=3, nk=2, nv=4):
    g = torch.Generator().manual_seed(seed)
    w = configs.gdn_layer_weights(g, H, F, nk, nv)
    x = torch.randn(b, H, generator=g).bfloat16()
    st = torch.randn(b, nv, 128, 128, generator=g) * 0.02
    cv = torch.randn(b, 3, 2 * nk * 128 + nv * 128, generator=g).bfloat16()
    return w, x, st, cv


# (2, 16, 32): config 4's heads, so the qkv | z | b | a projection group has 772 tiles and runs two tiles per
# workgroup (with the conv epilogue); (20, 2, 4): more than 16 sequences, two 16-row M tiles per workgroup
@pytest.mark.parametrize("b,nk,nv", [(3, 2, 4), (1, 1, 2), (8, 2, 2), (2, 16, 32), (20, 2, 4)])
def test_gdn_layer_decode(dev, b, nk, nv):
    w, x, st, cv = _gdn_case(b + nk + nv, b, nk, nv)
    out, so, co = layer.gdn_layer_decode(x.to(dev), _dev(w, dev), st.to(dev), cv.to(dev), nk, nv)
    ro, rs, rc = olayer.gdn_layer_decode(x, w, st, cv, nk, nv)
    torch.testing.assert_close(out.float().cpu(), ro.float(), **TOL)
    torch.testing.assert_close(so.cpu(), rs, **STATE_TOL)
    _check_conv(co, rc)


@pytest.mark.parametrize("entry", ["decode", "verify", "prefill"])
def test_gdn_layers_value_head_orders(dev, entry):
    """Both value-head orders against the oracle (grouped: value head vh reads key head vh / (NV / NK); tiled, the
    reference layers' default: vh % NK), and the tiled order on weights converted by tile_value_heads computes the
    grouped layer: the state and conv state bit-identical up to the value-head permutation (each head's arithmetic
    is the same), the output within the per-op bar (the output projection sums the heads in another order)."""
    nk, nv, b, t = 2, 6, 3, {"decode": 1, "verify": 3, "prefill": 70}[entry]
    g = torch.Generator().manual_seed(606 + t)
    w = configs.gdn_layer_weights(g, H, F, nk, nv)
    x = torch.randn(b, t, H, generator=g).bfloat16()
    st = torch.randn(b, nv, 128, 128, generator=g) * 0.02
    cv = torch.randn(b, 3, (2 * nk + nv) * 128, generator=g).bfloat16()
    kd = 2 * nk * 128
    wt = layer.tile_value_heads(w, nk, nv)
    stt = layer.v_tiled(st, 1, nk, nv, 1)
    cvt = torch.cat((cv[..., :kd], layer.v_tiled(cv[..., kd:], 2, nk, nv, 128)), -1)
    print(f"gdn v_order {entry} t={t}", flush=True)

    def run(weights, s0, c0, order):
        wd = _dev(weights, dev)
        if entry == "decode":
            o, so, co = layer.gdn_layer_decode(x[:, 0].contiguous().to(dev), wd, s0.to(dev), c0.to(dev), nk, nv,
                                               v_order=order)
            return o[:, None], so, co
        fn = layer.gdn_layer_verify if entry == "verify" else layer.gdn_layer_prefill
        return fn(x.to(dev), wd, s0.to(dev), c0.to(dev), nk, nv, v_order=order)

    def oracle(order):
        if entry == "prefill":
            return olayer.gdn_layer_prefill(x, w, st, cv, nk, nv, v_order=order)
        r = olayer.gdn_layer_verify(x, w, st, cv, nk, nv, v_order=order)
        return r[0], r[1], r[2]

    res = {}
    for order in ("grouped", "tiled"):
        out, so, co = res[order] = run(w, st, cv, order)
        ro, rs, rc = oracle(order)
        torch.testing.assert_close(out.float().cpu(), ro.float(), **FUSED_TOL)
        torch.testing.assert_close(so.cpu(), rs, **STATE_TOL)
    assert not torch.allclose(res["grouped"][1], res["tiled"][1])  # the orders pair other heads
    out_t, so_t, co_t = run(wt, stt, cvt, "tiled")
    out_g, so_g, co_g = res["grouped"]
    assert torch.equal(so_t, layer.v_tiled(so_g, 1, nk, nv, 1))
    assert torch.equal(co_t, torch.cat((co_g[..., :kd], layer.v_tiled(co_g[..., kd:], 2, nk, nv, 128)), -1))
    torch.testing.assert_close(out_t.float(), out_g.float(), **TOL)


def test_gdn_layer_two_steps_in_place(dev):
    w, x, st, cv = _gdn_case(11)
    x2 = torch.randn(3, H, generator=torch.Generator().manual_seed(12)).bfloat16()
    wd, sd, cd = _dev(w, dev), st.to(dev), cv.to(dev)
    ws = layer.gdn_workspace(3, H, 2, 4, F, dev)
    o1, _, _ = layer.gdn_layer_decode(x.to(dev), wd, sd, cd, 2, 4, workspace=ws, state_out=sd, conv_out=cd)
    o2, _, _ = layer.gdn_layer_decode(x2.to(dev), wd, sd, cd, 2, 4, workspace=ws, state_out=sd, conv_out=cd)
    r1, rs, rc = olayer.gdn_layer_decode(x, w, st, cv, 2, 4)
    r2, rs, rc = olayer.gdn_layer_decode(x2, w, rs, rc, 2, 4)
    torch.testing.assert_close(o1.float().cpu(), r1.float(), **TOL)
    torch.testing.assert_close(o2.float().cpu(), r2.float(), **TOL)
    torch.testing.assert_close(sd.cpu(), rs, **STATE_TOL)
    _check_conv(cd, rc)


# hq = 32, hkv = 4: config 4's heads (the q | k | v group has 1152 tiles: two per workgroup); 20 sequences: two
# 16-row M tiles per workgroup in every projection
@pytest.mark.parametrize("lens,hq,hkv,rot", [([100, 64, 300], 4, 2, 64), ([1, 127], 8, 2, 64), ([640], 4, 4, 0),
                                             ([70, 200], 32, 4, 64), ([17 + 9 * i for i in range(20)], 4, 2, 64)])
def test_attn_layer_decode(dev, lens, hq, hkv, rot):
    g = torch.Generator().manual_seed(len(lens) * 7 + hq)
    d = 256
    w = configs.attn_layer_weights(g, H, F, hq, hkv, d)
    c = configs.append_token_case(lens, hq, hkv, d, 64, g)
    x = torch.randn(len(lens), H, generator=g).bfloat16()
    cos, sin = olayer.rope_cos_sin(c["pos"], max(rot, 2), 10_000_000.0)
    cos, sin = cos[:, : rot // 2].contiguous(), sin[:, : rot // 2].contiguous()
    cache = c["cache"].to(dev)
    out = layer.attn_layer_decode(x.to(dev), _dev(w, dev), cos.to(dev), sin.to(dev), cache, c["indptr"].to(dev),
                                  c["indices"].to(dev), c["last_page_len"].to(dev), c["loc"].to(dev), hq, rot)
    ro, rcache = olayer.attn_layer_decode(x, w, cos, sin, c["cache"], c["indptr"], c["indices"], c["last_page_len"],
                                          c["loc"], hq, rot)
    torch.testing.assert_close(out.float().cpu(), ro.float(), **FUSED_TOL)
    got = cache.cpu()
    written = torch.zeros(got.shape[0], got.shape[2], dtype=torch.bool)
    for p, o in c["loc"].tolist():
        written[p, o] = True
    torch.testing.assert_close(got.permute(0, 2, 1, 3, 4)[written].float(),
                               rcache.permute(0, 2, 1, 3, 4)[written].float(), **TOL)
    assert torch.equal(got.permute(0, 2, 1, 3, 4)[~written].view(torch.int16),
                       c["cache"].permute(0, 2, 1, 3, 4)[~written].view(torch.int16))


def test_layer_contract_errors(dev):
    from axk import _lib

    w, x, st, cv = _gdn_case(3)
    wd = _dev(w, dev)
    with pytest.raises(_lib.AxkError):  # workspace too small
        layer.gdn_layer_decode(x.to(dev), wd, st.to(dev), cv.to(dev), 2, 4,
                               workspace=torch.empty(256, dtype=torch.uint8, device=dev))
    with pytest.raises(ValueError):
        bad = dict(wd)
        bad.pop("norm_w")
        layer.gdn_layer_decode(x.to(dev), bad, st.to(dev), cv.to(dev), 2, 4)


def test_layer_late_contract_error_enqueues_nothing(dev):
    """A contract error in a late sub-call (the GDN out projection's weight misaligned; a page size the paged decode
    rejects) returns its status before anything is launched: the recurrent state, the conv state and the KV cache
    are unchanged, so a caller's retry cannot advance them twice."""
    from axk import _lib

    w, x, st, cv = _gdn_case(21)
    wd = _dev(w, dev)
    raw = torch.zeros(wd["w_out"].numel() + 16, dtype=torch.uint8, device=dev)
    raw[1:1 + wd["w_out"].numel()] = wd["w_out"].reshape(-1)
    wd["w_out"] = raw[1:1 + wd["w_out"].numel()].view(wd["w_out"].shape)  # one byte off a 16-byte boundary
    sd, cd = st.to(dev), cv.to(dev)
    with pytest.raises(_lib.AxkError) as e:
        layer.gdn_layer_decode(x.to(dev), wd, sd, cd, 2, 4, state_out=sd, conv_out=cd)
    assert e.value.status == 3  # AXK_E_ALIGN
    torch.cuda.synchronize()
    assert torch.equal(sd.cpu(), st) and torch.equal(cd.cpu(), cv)

    g = torch.Generator().manual_seed(22)
    hq, hkv, d, page = 4, 2, 256, 24  # 24-token pages: the q / k / v preparation accepts them, the decode does not
    wa = configs.attn_layer_weights(g, H, F, hq, hkv, d)
    c = configs.append_token_case([30, 50], hq, hkv, d, page, g)
    xa = torch.randn(2, H, generator=g).bfloat16()
    cos, sin = olayer.rope_cos_sin(c["pos"], 64, 10_000_000.0)
    cache = c["cache"].to(dev)
    with pytest.raises(_lib.AxkError) as e:
        layer.attn_layer_decode(xa.to(dev), _dev(wa, dev), cos.to(dev), sin.to(dev), cache, c["indptr"].to(dev),
                                c["indices"].to(dev), c["last_page_len"].to(dev), c["loc"].to(dev), hq, 64)
    assert e.value.status == 2  # AXK_E_SHAPE
    torch.cuda.synchronize()
    assert torch.equal(cache.cpu().view(torch.int16), c["cache"].view(torch.int16))


# ---- the manifests' weight formats: MXFP8 layer weights (the 35B manifest, q35_mx_build.py:60-72) and MXFP4 layer
# weights (the 9B / 27B manifests), for the projections and the MLP ----
@pytest.mark.parametrize("proj_fmt,mlp_fmt", [("mxfp8", "mxfp8"), ("mxfp4", "mxfp4"), ("mxfp8", "mxfp4"),
                                              ("nvfp4", "nvfp4"), ("mxfp8", "nvfp4")])
def test_gdn_layer_decode_weight_formats(dev, proj_fmt, mlp_fmt):
    b, nk, nv = 3, 2, 4
    g = torch.Generator().manual_seed(31)
    w = configs.gdn_layer_weights(g, H, F, nk, nv, proj_fmt=proj_fmt, mlp_fmt=mlp_fmt)
    x = torch.randn(b, H, generator=g).bfloat16()
    st = torch.randn(b, nv, 128, 128, generator=g) * 0.02
    cv = torch.randn(b, 3, 2 * nk * 128 + nv * 128, generator=g).bfloat16()
    print(f"gdn layer proj={proj_fmt} mlp={mlp_fmt}", flush=True)
    out, so, co = layer.gdn_layer_decode(x.to(dev), _dev(w, dev), st.to(dev), cv.to(dev), nk, nv, proj_fmt=proj_fmt,
                                         mlp_fmt=mlp_fmt)
    ro, rs, rc = olayer.gdn_layer_decode(x, w, st, cv, nk, nv, proj_fmt=proj_fmt, mlp_fmt=mlp_fmt)
    torch.testing.assert_close(out.float().cpu(), ro.float(), **TOL)
    torch.testing.assert_close(so.cpu(), rs, **STATE_TOL)
    _check_conv(co, rc)


@pytest.mark.parametrize("proj_fmt,mlp_fmt", [("mxfp8", "mxfp8"), ("mxfp4", "mxfp4"), ("nvfp4", "nvfp4")])
def test_attn_layer_decode_weight_formats(dev, proj_fmt, mlp_fmt):
    lens, hq, hkv, rot, d = [100, 64, 300], 4, 2, 64, 256
    g = torch.Generator().manual_seed(37)
    w = configs.attn_layer_weights(g, H, F, hq, hkv, d, proj_fmt=proj_fmt, mlp_fmt=mlp_fmt)
    c = configs.append_token_case(lens, hq, hkv, d, 64, g)
    x = torch.randn(len(lens), H, generator=g).bfloat16()
    cos, sin = olayer.rope_cos_sin(c["pos"], rot, 10_000_000.0)
    cache = c["cache"].to(dev)
    print(f"attn layer proj={proj_fmt} mlp={mlp_fmt}", flush=True)
    out = layer.attn_layer_decode(x.to(dev), _dev(w, dev), cos.to(dev), sin.to(dev), cache, c["indptr"].to(dev),
                                  c["indices"].to(dev), c["last_page_len"].to(dev), c["loc"].to(dev), hq, rot,
                                  proj_fmt=proj_fmt, mlp_fmt=mlp_fmt)
    ro, _ = olayer.attn_layer_decode(x, w, cos, sin, c["cache"], c["indptr"], c["indices"], c["last_page_len"],
                                     c["loc"], hq, rot, proj_fmt=proj_fmt, mlp_fmt=mlp_fmt)
    torch.testing.assert_close(out.float().cpu(), ro.float(), **FUSED_TOL)
