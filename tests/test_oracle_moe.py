"""Pins the MoE oracle (CPU only)."""
import numpy as np
import pytest
import torch

from axk import configs
from oracle import moe, mx, rounding


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


def test_bf16_slots_schedule():
    """The prefill schedule (each routed slot bf16(rw y) before the fp32 sum): with every slot exactly
    representable in bf16 (dyadic routing weights on an expert whose outputs are bf16 values) it equals the fp32
    schedule; in general each slot moves by at most half a bf16 ulp of itself, and the reported slack covers that
    rounding on top of the activation flips."""
    h2, x, w, k = _small(seed=11, t=12, h=64, e=4, f=32, fs=32, k=2)
    _, _, ids, wts = moe.moe_layer(h2, w, k, x_res=x)
    base, r32, s32 = moe.moe_parts(h2, w, ids, wts, x)
    _, r16, s16 = moe.moe_parts(h2, w, ids, wts, x, slot_bf16=True)
    assert not torch.equal(r16, r32)
    # bound: |sum bf16(y_k) - sum y_k| <= sum_k ulp(y_k) / 2 <= the added slack
    assert ((r16 - r32).abs() <= (s16 - s32) / 2 + 1e-6).all()
    assert (s16 >= s32).all()
    # exactness: an expert whose down weight has one 1.0 per row (so each output is one bf16 activation) and dyadic
    # routing weights make every slot exact in bf16: both schedules agree bit for bit
    ids2 = torch.tensor([[1, 2]], dtype=torch.int32).repeat(h2.shape[0], 1)
    wts2 = torch.tensor([[0.5, 0.25]]).repeat(h2.shape[0], 1)
    w2 = dict(w)
    dw, ds = w["e_dw"].clone(), w["e_ds"].clone()
    hid, f2 = dw.shape[1], dw.shape[2] * 2
    for e in (1, 2):
        dw[e] = 0
        ds[e] = 127
        for r in range(hid):
            col = (3 * r + e) % f2
            dw[e, r, col // 2] = 2 if col % 2 == 0 else 2 << 4  # E2M1 code 2 = 1.0
    w2["e_dw"], w2["e_ds"] = dw, ds
    _, b32, _ = moe.moe_parts(h2, w2, ids2, wts2, x)
    _, b16, _ = moe.moe_parts(h2, w2, ids2, wts2, x, slot_bf16=True)
    assert torch.equal(b32, b16) and b32.abs().max() > 0


def _hf_moe_block(w, top_k):
    """transformers' Qwen3_5MoeSparseMoeBlock (fp32, eager experts) holding the exactly dequantised weights."""
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeSparseMoeBlock

    e, two_f, h = w["e_gw"].shape[0], w["e_gw"].shape[1], w["w_router"].shape[1]
    cfg = Qwen3_5MoeTextConfig(hidden_size=h, num_experts=e, moe_intermediate_size=two_f // 2,
                               shared_expert_intermediate_size=w["w_gate"].shape[0], num_experts_per_tok=top_k,
                               num_hidden_layers=1, layer_types=["full_attention"], hidden_act="silu")
    cfg._experts_implementation = "eager"
    blk = Qwen3_5MoeSparseMoeBlock(cfg).float().eval()

    def deq(c, s):
        return torch.from_numpy(mx.dequant_mxfp4(np.asarray(c), np.asarray(s)))

    with torch.no_grad():
        blk.gate.weight.copy_(w["w_router"].float())
        blk.experts.gate_up_proj.copy_(torch.stack([deq(w["e_gw"][j], w["e_gs"][j]) for j in range(e)]))
        blk.experts.down_proj.copy_(torch.stack([deq(w["e_dw"][j], w["e_ds"][j]) for j in range(e)]))
        blk.shared_expert.gate_proj.weight.copy_(deq(w["w_gate"], w["s_gate"]))
        blk.shared_expert.up_proj.weight.copy_(deq(w["w_up"], w["s_up"]))
        blk.shared_expert.down_proj.weight.copy_(deq(w["w_down"], w["s_down"]))
        blk.shared_expert_gate.weight.copy_(w["w_shg"].float().reshape(1, -1))
    return blk


@pytest.mark.parametrize("seed,t,h,e,f,fs,k", [(0, 6, 64, 8, 32, 32, 3), (4, 17, 128, 16, 64, 96, 8),
                                                (5, 3, 64, 32, 32, 64, 4)])
def test_moe_layer_matches_transformers_sparse_moe_block(seed, t, h, e, f, fs, k):
    """The reference's own oracle family (q35_moe.py:300-312): transformers' Qwen3_5MoeSparseMoeBlock with the
    dequantised MXFP4 experts, shared expert and sigmoid gate. Pins the router (softmax -> top-K -> renormalise),
    the [gate | up] split of the gate-up matrix, silu(gate) * up, the sigmoid-gated shared expert and the sum."""
    h2, x, w, _ = _small(seed=seed, t=t, h=h, e=e, f=f, fs=fs, k=k)
    blk = _hf_moe_block(w, k)
    with torch.no_grad():
        ref = blk(h2.float()[None])[0]
        _, hf_w, hf_ids = blk.gate(h2.float())
    logits = h2.float() @ w["w_router"].float().T
    ids, wts = moe.route(logits, k)
    assert torch.equal(ids.long(), hf_ids)
    torch.testing.assert_close(wts, hf_w, rtol=1e-6, atol=1e-7)
    with rounding.fp32():
        out, *_ = moe.moe_layer(h2, w, k, x_res=x, ids=ids, wts=wts, round_base=False)
    assert out.dtype == torch.float32
    torch.testing.assert_close(out, x.float() + ref, rtol=1e-5, atol=1e-5)
    # the bf16 rounding points (q35_moe.py:96-137) stay within the north-star bar of the fp32 composition
    out_bf, *_ = moe.moe_layer(h2, w, k, x_res=x, ids=ids, wts=wts)
    torch.testing.assert_close(out_bf.float(), x.float() + ref, rtol=2e-2, atol=1e-2)


def test_transformers_pin_detects_plausible_slips():
    """Each slip a restatement could make moves the output far outside the fp32 bar of the pin above."""
    h2, x, w, k = _small(seed=9, t=8, h=64, e=8, f=32, fs=32, k=3)
    blk = _hf_moe_block(w, k)
    with torch.no_grad():
        ref = x.float() + blk(h2.float()[None])[0]
    ids, wts = moe.route(h2.float() @ w["w_router"].float().T, k)

    def run(wd, **kw):
        with rounding.fp32():
            return moe.moe_layer(h2, wd, k, x_res=x, ids=ids, wts=wts, round_base=False)[0]

    f = w["e_gw"].shape[1] // 2
    swapped = dict(w, e_gw=torch.cat([w["e_gw"][:, f:], w["e_gw"][:, :f]], 1),
                   e_gs=torch.cat([w["e_gs"][:, f:], w["e_gs"][:, :f]], 1))
    no_gate = {n: v for n, v in w.items() if n != "w_shg"}  # shared expert ungated
    for bad in (run(swapped), run(no_gate)):
        assert not torch.allclose(bad, ref, rtol=1e-3, atol=1e-3)
    with rounding.fp32():
        unnorm = moe.moe_layer(h2, w, k, x_res=x, norm=False, round_base=False)[0]  # weights not renormalised
    assert not torch.allclose(unnorm, ref, rtol=1e-3, atol=1e-3)
