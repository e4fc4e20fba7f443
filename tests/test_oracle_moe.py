"""Pins the MoE oracle (CPU only)."""
import numpy as np
import torch

from axk import configs
from oracle import moe, mx


def _small(seed=0, t=6, h=64, e=8, f=32, fs=32, k=3):
    g = torch.Generator().manual_seed(seed)
    w = configs.moe_weights(g, hidden=h, experts=e, inter=f, shared_inter=fs, router_std=0.5)
    h2 = torch.randn(t, h, generator=g).to(torch.bfloat16)
    x = torch.randn(t, h, generator=g).to(torch.bfloat16)
    return h2, x, w, k


def test_route_matches_topk_and_tie_rule():
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(50, 64, generator=g)
    ids, w = moe.route(logits, 8)
    tv, ti = torch.topk(torch.softmax(logits, -1), 8)  # no ties in continuous random logits
    assert torch.equal(ids.long(), ti)
    torch.testing.assert_close(w, tv / tv.sum(-1, keepdim=True))
    tied = torch.zeros(2, 16)
    tied[0, [3, 7, 11]] = 1.0
    ids2, w2 = moe.route(tied, 4)
    assert ids2[0].tolist() == [3, 7, 11, 0] and ids2[1].tolist() == [0, 1, 2, 3]
    torch.testing.assert_close(w2.sum(-1), torch.ones(2))


def test_layer_matches_dense_all_experts_formulation():
    h2, x, w, k = _small()
    out, logits, ids, wts = moe.moe_layer(h2, w, k, x_res=x)
    # dense: every token through every expert, combined with a [T, E] routing matrix
    t, h = h2.shape
    e, two_f, _ = w["e_gw"].shape
    dense = torch.stack([moe.swiglu_expert(h2, w["e_gw"][j].numpy(), w["e_gs"][j].numpy(), w["e_dw"][j].numpy(),
                                           w["e_ds"][j].numpy(), split=two_f // 2) for j in range(e)], 1)
    route = torch.zeros(t, e).scatter_(1, ids.long(), wts)
    wg = torch.from_numpy(mx.dequant_mxfp4(w["w_gate"].numpy(), w["s_gate"].numpy()))
    wu = torch.from_numpy(mx.dequant_mxfp4(w["w_up"].numpy(), w["s_up"].numpy()))
    wd = torch.from_numpy(mx.dequant_mxfp4(w["w_down"].numpy(), w["s_down"].numpy()))
    act = (torch.nn.functional.silu((h2.float() @ wg.T).bfloat16().float()) * (h2.float() @ wu.T).bfloat16().float())
    sh = act.bfloat16().float() @ wd.T
    gate = torch.sigmoid(h2.float() @ w["w_shg"].float())
    base = (x.float() + gate[:, None] * sh).bfloat16().float()
    ref = (base + torch.einsum("te,teh->th", route, dense)).bfloat16()
    torch.testing.assert_close(out.float(), ref.float(), rtol=1e-2, atol=1e-2)
    # a swapped gate / up order must not pass
    swapped = dict(w)
    f = two_f // 2
    swapped["e_gw"] = torch.cat([w["e_gw"][:, f:], w["e_gw"][:, :f]], 1)
    swapped["e_gs"] = torch.cat([w["e_gs"][:, f:], w["e_gs"][:, :f]], 1)
    bad, *_ = moe.moe_layer(h2, swapped, k, x_res=x, ids=ids, wts=wts)
    assert not torch.allclose(bad.float(), out.float(), rtol=2e-2, atol=1e-2)


def test_single_expert_weight_one_and_zero_router():
    h2, x, w, _ = _small(seed=2)
    w1 = {n: v for n, v in w.items() if not n.startswith(("w_gate", "s_gate", "w_up", "s_up", "w_down", "s_down"))}
    w1["w_router"] = torch.zeros_like(w["w_router"])  # uniform softmax: ties -> experts 0..K-1, weight 1/K
    out, logits, ids, wts = moe.moe_layer(h2, w1, 1, x_res=None)
    assert (ids == 0).all() and torch.equal(wts, torch.ones_like(wts))
    e_gw = w["e_gw"][0].numpy()
    y = moe.swiglu_expert(h2, e_gw, w["e_gs"][0].numpy(), w["e_dw"][0].numpy(), w["e_ds"][0].numpy(),
                          split=e_gw.shape[0] // 2)
    torch.testing.assert_close(out.float(), y.bfloat16().float(), rtol=1e-2, atol=1e-2)


def test_flip_slack_bounds_flipped_activations():
    # flip two activations of every (token, expert) row by one bf16 ulp, recompute the routed sum by hand: the
    # change stays inside the slack moe_parts reports
    h2, x, w, k = _small(seed=7, t=9, h=64, e=6, f=32, fs=32, k=3)
    _, _, ids, wts = moe.moe_layer(h2, w, k, x_res=x)
    base, routed, slack = moe.moe_parts(h2, w, ids, wts, x)
    g = torch.Generator().manual_seed(3)
    e_gw, e_gs, e_dw, e_ds = (w[n] for n in ("e_gw", "e_gs", "e_dw", "e_ds"))
    inter = e_gw.shape[1] // 2
    moved = torch.zeros_like(routed)
    for t in range(h2.shape[0]):
        for j in range(k):
            e = int(ids[t, j])
            act = moe.swiglu_act(h2[t:t + 1], e_gw[e], e_gs[e], split=inter)[0]
            cols = torch.randperm(inter, generator=g)[:2]
            sign = torch.where(torch.rand(2, generator=g) < 0.5, -1.0, 1.0)
            act[cols] += sign * moe.ulp_bf16(act[cols])
            wd = moe._deq(e_dw[e], e_ds[e])
            moved[t] += wts[t, j] * (act @ wd.T)
    diff = (moved - routed).abs()
    assert diff.max() > 0
    assert (diff <= slack + 1e-5).all()
