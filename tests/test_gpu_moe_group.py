"""The 35B's MoE decode group on the GPU: axk.DecodeGroup over the MoE decode layers (axk_gdn_layer_decode_moe /
axk_attn_layer_decode_moe through the C-ABI), in the role of the 35B manifest's qwen35moe_group8_gggaggga_mx8_kvc_c16384
(models/qwen35_35b_a3b/src/70b0fbc/q35_moe_group.py): 8 layers ((GDN, GDN, GDN, attention) x 2) at the 35B's widths
(hidden 2048, MXFP8 projections and shared expert of 512, 256 MXFP4 experts of 512, top-8, GDN 16 / 32 heads,
attention HQ 16 / HKV 2 / D 256), 32 sequences at 16,383 cached tokens each.

  * the group against its layers one by one, as the reference checks its group (q35_moe_group.py:168-183, there
    bitwise on the output): the step captured as one HIP graph equals the layers called eagerly one after another bit
    for bit (the output, every GDN state and conv state, the new KV rows), on three replays with eager steps, state
    restores and synchronisations between them, the second from another input;
  * the group bound from the 35B manifest's decode.group (its packs filled by Manifest.store_layer, the routed
    experts in e_gw<j> .. e_ds<j>) through group.manifest_layers runs like the same weights as loose tensors, bit for
    bit (a small batch and context);
  * the group carrying the LM head (final norm + the 35B's MXFP4 output projection) gives the separate calls'
    logits bit for bit, eager and replayed, and the oracle's on a slice;
  * the first GDN layer (4 sequences) and the first attention layer (sequence 0 over its full context) of the eager
    step against the oracle at the MoE layer bars: the routing from the kernel's own logits (ids bit-exact against a
    stable descending sort of them, weights at fp32 tolerance), the output within the reference's fused-layer bar
    rel 5e-2 / abs 0.0625 (test_gdn_attn.py:348-354, 537) plus the derived slack for one-ulp flips of the bf16 expert
    activations, the GDN state at the temporal bar, the conv state shifted exactly, the new KV row at the per-op bar;
    every layer's output finite; no KV byte outside the new slots changed.
"""
import os

import pytest
import torch

from axk import configs, group
from axk import gemm as axk_gemm
from axk import manifest as mf
from oracle import layer as olayer
from oracle import moe as omoe

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(__file__), "golden", "manifests")
TOL = dict(rtol=2e-2, atol=1e-2)
FUSED_TOL = dict(rtol=5e-2, atol=0.0625)
STATE_TOL = dict(rtol=5e-2, atol=3e-3)


def _cpu(d):
    return {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in d.items()}


def _check_moe(out, r, x, y, w, blk):
    """out [n, H] of the kernel and r its routing outputs (rows 0..n-1); x the layer input, y the oracle's first
    half, all on the host."""
    logits, ids, wts = r["logits"], r["topk_ids"], r["topk_weights"]
    sids, swts = omoe.route(logits, blk["top_k"], True)
    assert torch.equal(ids, sids), "top-K ids differ from the stable sort of the kernel's logits"
    torch.testing.assert_close(wts, swts, rtol=1e-5, atol=1e-6)
    base, routed, slack, ref_logits, _, _ = olayer.moe_block_parts(x, y, w, blk, fmt="mxfp8", ids=ids.long(), wts=wts)
    torch.testing.assert_close(logits, ref_logits, **TOL)
    ref = (base + routed).bfloat16().float()
    d = (out.float() - ref).abs()
    tol = FUSED_TOL["atol"] + FUSED_TOL["rtol"] * ref.abs()
    assert (d <= tol + slack).all(), f"max excess {(d - tol - slack).max().item()}"


def _snapshot(c, wm):
    """The step's state: every GDN state and conv state, every attention layer's new KV rows."""
    out = []
    for L in c["layers"]:
        if L["kind"] == "g":
            out += [L["state"].clone(), L["conv"].clone()]
        else:
            out.append(L["cache"].permute(0, 2, 1, 3, 4)[wm].clone())
    return out


def _restore(c, snap, wm):
    it = iter(snap)
    for L in c["layers"]:
        if L["kind"] == "g":
            L["state"].copy_(next(it))
            L["conv"].copy_(next(it))
        else:
            L["cache"].permute(0, 2, 1, 3, 4)[wm] = next(it)


def _same(a, b):
    return a.dtype == b.dtype and torch.equal(a.view(torch.uint8), b.view(torch.uint8))


def test_moe_group_35b_graph_equals_layers(dev):
    c = configs.moe_group(dev)
    cg = c["cfg"]
    b, h = cg["batch"], cg["hidden"]
    print(f"35B MoE group {cg['pattern']}, batch {b}, ctx {cg['ctx']}", flush=True)
    grp = group.DecodeGroup(c["layers"], b, h, dev, cg["nk"], cg["nv"], cg["hq"], cg["rot"], cg["eps"], "mxfp8",
                            "mxfp8", attn=c["attn"], routing=True)
    a = c["attn"]
    loc = a["loc"]
    attn = [L for L in c["layers"] if L["kind"] == "a"]
    wm = torch.zeros(attn[0]["cache"].shape[0], attn[0]["cache"].shape[2], dtype=torch.bool, device=dev)
    wm[loc[:, 0].long(), loc[:, 1].long()] = True
    kv0 = [L["cache"].clone() for L in attn]
    s0 = _snapshot(c, wm)
    x0 = c["x"].clone()

    # eager step 1: the layers one after another
    out1 = grp.step(x0, record=True).clone()
    rt1 = [None if r is None else {k: v.clone() for k, v in r.items()} for r in grp.routing]
    torch.cuda.synchronize()
    ins = grp.inputs
    for xi in ins[1:] + [out1]:
        assert torch.isfinite(xi.float()).all()
    gi = 0
    for L in c["layers"]:  # the GDN states advanced in place, the conv states shifted by one token
        if L["kind"] == "g":
            st0, cv0 = s0[gi], s0[gi + 1]
            assert torch.isfinite(L["state"]).all() and not torch.equal(L["state"], st0)
            assert torch.equal(L["conv"][:, :-1], cv0[:, 1:])
            gi += 2
        else:
            gi += 1
    for k0, L in zip(kv0, attn):  # only the new slots change
        got, ref = L["cache"].permute(0, 2, 1, 3, 4), k0.permute(0, 2, 1, 3, 4)
        assert torch.equal(got[~wm].view(torch.int16), ref[~wm].view(torch.int16))
        assert torch.isfinite(got[wm].float()).all()
    s1 = _snapshot(c, wm)

    # the first GDN layer against the oracle, sequences 0..3
    n = 4
    L0 = c["layers"][0]
    w0, m0 = _cpu(L0["w"]), _cpu(L0["moe"])
    y, rs, rc = olayer.gdn_layer_half(ins[0][:n].cpu(), w0, s0[0][:n].cpu(), s0[1][:n].cpu(), cg["nk"], cg["nv"],
                                      cg["eps"], proj_fmt="mxfp8")
    _check_moe(ins[1][:n].cpu(), {k: v[:n].cpu() for k, v in rt1[0].items()}, ins[0][:n].cpu(), y, w0, m0)
    torch.testing.assert_close(s1[0][:n].cpu(), rs, **STATE_TOL)
    assert torch.equal(s1[1][:n, :-1].cpu(), rc[:, :-1])
    del w0, m0

    # the first attention layer against the oracle: sequence 0 over its full context, its pages gathered into a
    # compact host cache holding the state before the step
    ja = next(j for j, L in enumerate(c["layers"]) if L["kind"] == "a")
    La = c["layers"][ja]
    n0 = int(a["indptr"][1].item())
    cache0 = kv0[0][a["indices"][:n0].long()].cpu()
    loc0 = torch.tensor([[n0 - 1, int(loc[0, 1].item())]], dtype=torch.int32)
    wa, ma = _cpu(La["w"]), _cpu(La["moe"])
    y, rcache = olayer.attn_layer_half(ins[ja][:1].cpu(), wa, a["cos"][:1].cpu(), a["sin"][:1].cpu(), cache0,
                                       torch.tensor([0, n0], dtype=torch.int32), torch.arange(n0, dtype=torch.int32),
                                       a["last_page_len"][:1].cpu(), loc0, cg["hq"], cg["rot"], cg["eps"],
                                       proj_fmt="mxfp8")
    _check_moe(ins[ja + 1][:1].cpu(), {k: v[:1].cpu() for k, v in rt1[ja].items()}, ins[ja][:1].cpu(), y, wa, ma)
    p0, o0 = int(loc[0, 0].item()), int(loc[0, 1].item())
    torch.testing.assert_close(La["cache"][p0, :, o0].float().cpu(), rcache[n0 - 1, :, o0].float(), **TOL)
    del cache0, rcache, wa, ma, kv0

    # eager step 2 from the state after step 1, another input
    gx = torch.Generator(device=dev).manual_seed(5)
    x2 = torch.randn(b, h, generator=gx, device=dev).bfloat16()
    out2 = grp.step(x2).clone()
    torch.cuda.synchronize()
    s2 = _snapshot(c, wm)

    # the step as one HIP graph: three replays, each from restored states, each bit for bit the eager step
    grp.capture()
    for x, start, want_out, want in ((x0, s0, out1, s1), (x2, s1, out2, s2), (x0, s0, out1, s1)):
        _restore(c, start, wm)
        torch.cuda.synchronize()
        got = grp.replay(x).clone()
        torch.cuda.synchronize()
        assert _same(got, want_out), "graph replay output differs from the eager step"
        for g_, w_ in zip(_snapshot(c, wm), want):
            assert _same(g_, w_), "graph replay state differs from the eager step"
        for r, r1 in zip(grp.routing, rt1 if x is x0 else [None] * len(rt1)):
            if r is not None and r1 is not None:
                assert torch.equal(r["topk_ids"], r1["topk_ids"])


def test_moe_group_bound_from_the_manifest_runs_like_loose_tensors(dev):
    m = mf.Manifest.load(os.path.join(HERE, "qwen35_35b_a3b.manifest.json"))
    role = "decode.group"
    k = m.kernel(role)
    c = configs.moe_group(dev, batch=2, ctx=100, seed=3)
    cg = c["cfg"]
    print(f"{m.model} {k.file}: bound vs loose, batch 2, ctx 100", flush=True)
    names = set(k.packs) | {f"{n}{j}" for j in range(len(c["layers"])) for n in mf.EXPERT_IO}
    bufs = {e.name: torch.zeros(e.bytes, dtype=torch.uint8, device=dev) for e in k.inputs if e.name in names}
    for j, L in enumerate(c["layers"]):
        m.store_layer(role, bufs, j, dict(L["w"], w_router=L["moe"]["w_router"], w_shg=L["moe"]["w_shg"]))
        for n in mf.EXPERT_IO:
            bufs[f"{n}{j}"].copy_(L["moe"][n].reshape(-1))
    layers, proj_fmt, mlp_fmt = group.manifest_layers(m, role, bufs, top_k=cg["top_k"])
    assert (proj_fmt, mlp_fmt) == ("mxfp8", "mxfp8")
    assert "".join(L["kind"] for L in layers) == cg["pattern"]
    for Lb, L in zip(layers, c["layers"]):  # the bound group's own copies of the starting states
        for n in ("state", "conv", "cache"):
            if n in L:
                Lb[n] = L[n].clone()
    args = (cg["batch"], cg["hidden"], dev, cg["nk"], cg["nv"], cg["hq"], cg["rot"], cg["eps"])
    loose = group.DecodeGroup(c["layers"], *args, "mxfp8", "mxfp8", attn=c["attn"])
    bound = group.DecodeGroup(layers, *args, proj_fmt, mlp_fmt, attn=c["attn"])
    out_l = loose.step(c["x"]).clone()
    out_b = bound.step(c["x"]).clone()
    torch.cuda.synchronize()
    assert torch.isfinite(out_l.float()).all()
    assert _same(out_b, out_l)
    for Lb, L in zip(layers, c["layers"]):
        for n in ("state", "conv", "cache"):
            if n in L:
                assert _same(Lb[n], L[n])


@pytest.mark.parametrize("fmt", ["mxfp4", "nvfp4"])
def test_moe_group_with_lm_head(dev, fmt):
    """The group that ends the model carries the LM head (q35_group.py:442-452 with LMHEAD=1): the final norm and
    the 35B's output projection (248320 x 2048: MXFP4 as mul_mat_mx4_n248320_k2048, or NVFP4 as the reference's
    NVFP4 head) inside the step. The logits equal the separate norm and GEMM calls on the step's output bit for bit,
    eager and graph-replayed; the normalised rows and a slice of the logits against the oracle at the per-op bar."""
    from axk import glue
    from oracle import mx

    c = configs.moe_group(dev, batch=4, ctx=100, seed=7)
    cg = c["cfg"]
    lm = configs.lm_head_case(dev, seed=8) if fmt == "mxfp4" else configs.lm_head_nvfp4_case(dev, seed=8)
    norm = 1.0 + 0.1 * torch.randn(cg["hidden"], generator=torch.Generator(device=dev).manual_seed(9), device=dev)
    print(f"35B MoE group + {fmt} LM head {lm['w'].shape[0]} x {cg['hidden']}, batch 4", flush=True)
    grp = group.DecodeGroup(c["layers"], cg["batch"], cg["hidden"], dev, cg["nk"], cg["nv"], cg["hq"], cg["rot"],
                            cg["eps"], "mxfp8", "mxfp8", attn=c["attn"],
                            lm_head=dict(norm=norm, w=lm["w"], s=lm["s"], s2=lm.get("s2"), fmt=fmt))
    wm = torch.zeros(c["layers"][3]["cache"].shape[0], c["layers"][3]["cache"].shape[2], dtype=torch.bool,
                     device=dev)
    wm[c["attn"]["loc"][:, 0].long(), c["attn"]["loc"][:, 1].long()] = True
    s0 = _snapshot(c, wm)
    out = grp.step(c["x"]).clone()
    logits = grp.logits.clone()
    hn = glue.rmsnorm(out, norm, cg["eps"])
    if fmt == "mxfp4":
        sep = axk_gemm.mxfp4_gemm(hn, lm["w"], lm["s"], out_dtype=torch.float32)
    else:
        sep = axk_gemm.nvfp4_gemm(hn, lm["w"], lm["s"], lm["s2"], out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert _same(grp.hn, hn) and _same(logits, sep)
    assert torch.isfinite(logits).all()
    ref_h = olayer.rmsnorm(out.cpu(), norm.cpu(), cg["eps"])
    torch.testing.assert_close(hn.float().cpu(), ref_h.float(), **TOL)
    rows = 3000
    if fmt == "mxfp4":
        ref = mx.mx_linear(hn.cpu(), lm["w"][:rows].cpu().numpy(), lm["s"][:rows].cpu().numpy())
    else:
        ref = mx.nvfp4_linear(hn.cpu(), lm["w"][:rows].cpu().numpy(), lm["s"][:rows].cpu().numpy(), lm["s2"].item())
    torch.testing.assert_close(logits[:, :rows].cpu(), ref.float(), **TOL)
    # graph-replayed from the same states: the same logits bit for bit
    grp.capture()
    _restore(c, s0, wm)
    torch.cuda.synchronize()
    grp.replay(c["x"])
    torch.cuda.synchronize()
    assert _same(grp.out, out) and _same(grp.logits, logits)
