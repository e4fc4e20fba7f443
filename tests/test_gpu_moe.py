"""GPU parity of the MoE layer (router, top-K, shared + routed MXFP4 SwiGLU experts) against the oracle.

Bar: top-K ids bit-exact against a stable descending sort of the kernel's own logits; routing weights and
logits at fp32 tolerance; bf16 outputs within rel 2e-2 / abs 1e-2 of the oracle on the same routing. The prefill
path (tokens > 256) is checked against the reference's delivered prefill schedule, each routed slot rounded to
bf16 before the slot-order sum (q35_moe_prefill.py:41, 100, 165, 196-213); decode against fp32 slots.
"""
import pytest
import torch

from axk import configs, moe
from oracle import moe as omoe

pytestmark = pytest.mark.gpu
TOL = dict(rtol=2e-2, atol=1e-2)


def _dev_w(w, dev):
    return {n: v.to(dev) for n, v in w.items()}


def _check_layer(c, dev, norm=True):
    h2, x, w, k = c["h2"], c["x_res"], c["weights"], c["top_k"]
    out, logits, ids, wts = moe.moe_decode(h2.to(dev), _dev_w(w, dev), top_k=k,
                                           x_res=None if x is None else x.to(dev), norm_topk_prob=norm)
    out, logits, ids, wts = out.cpu(), logits.cpu(), ids.cpu(), wts.cpu()
    ref_logits = h2.float() @ w["w_router"].float().T
    torch.testing.assert_close(logits, ref_logits, rtol=1e-4, atol=1e-4)
    sids, swts = omoe.route(logits, k, norm)  # the host rule on the kernel's own logits
    assert torch.equal(ids, sids), "top-K ids differ from the stable sort of the kernel's logits"
    torch.testing.assert_close(wts, swts, rtol=1e-5, atol=1e-6)
    prefill = h2.shape[0] > 256
    base, routed, slack = omoe.moe_parts(h2, w, ids, wts, x, slot_bf16=prefill)
    ref = (base + routed).to(torch.bfloat16).float()  # base kept fp32, one final rounding (the kernel's schedule)
    tol = TOL["atol"] + TOL["rtol"] * ref.abs()
    d = (out.float() - ref).abs()
    # Elementwise at the stated tolerance, except where a one-ulp flip of a bf16 activation (g, u, act are rounded
    # at the reference's points; which way a value at a rounding midpoint goes depends on the fp32 summation
    # order) moves an output that cancels to near zero: such elements are rare and stay inside the derived slack.
    assert (d <= tol + slack).all(), f"max excess {(d - tol - slack).max().item()}"
    # The prefill schedule rounds each of the K routed slots to bf16 as well: K more order-dependent roundings per
    # element, so more of the (rare, slack-bounded) flips reach the plain bar (config 3b: about 1.6e-5 of elements)
    frac = 5e-5 if prefill else 1e-5
    assert (d > tol).float().mean().item() <= frac, f"{int((d > tol).sum())} elements outside the plain tolerance"
    # the reference's rounding schedule (base rounded to bf16 first) differs by at most one ulp of |base| more
    sched = (base.to(torch.bfloat16).float() + routed).to(torch.bfloat16).float()
    assert ((out.float() - sched).abs() <= omoe.ulp_bf16(base) + tol + slack).all()
    return out


# e spans the router's 64 / 256 / 1024-expert register layouts; t = 130 and 256 span several 64-token words
# of the grouping bitmask (256 is the largest token count of the decode path); the last three take the staged-weight
# streaming kernels (t <= 64) or just miss them (t = 65)
@pytest.mark.parametrize("t,h,e,f,fs,k", [(1, 64, 8, 32, 32, 2), (5, 256, 16, 64, 96, 4), (33, 128, 64, 32, 64, 8),
                                          (7, 192, 40, 160, 0, 6), (3, 128, 200, 32, 32, 8),
                                          (2, 64, 1000, 32, 0, 32), (130, 64, 16, 32, 32, 4),
                                          (256, 64, 8, 32, 0, 2),
                                          # K multiples of 256 with <= 64 tokens: the staged-weight streaming kernels
                                          (20, 512, 32, 256, 256, 4), (64, 256, 64, 256, 0, 8), (65, 256, 16, 256, 256, 2),
                                          # the staged-weight kernels at H 1024 / 2048: one token; experts over several
                                          # 8-row passes with F != Fs; no shared expert and 2-tile slots; E > 256;
                                          # 6-tile routed and 2-tile shared slots
                                          (1, 1024, 16, 64, 64, 4), (64, 1024, 8, 96, 160, 2), (33, 2048, 128, 32, 0, 8),
                                          (40, 1024, 300, 32, 32, 6), (9, 1024, 64, 96, 32, 3)])
def test_moe_small_shapes(dev, t, h, e, f, fs, k):
    g = torch.Generator().manual_seed(t + h + e)
    w = configs.moe_weights(g, hidden=h, experts=e, inter=f, shared_inter=max(fs, 32), router_std=0.5)
    if fs == 0:  # no shared expert
        for n in ("w_gate", "s_gate", "w_up", "s_up", "w_down", "s_down", "w_shg"):
            w.pop(n)
    c = {"h2": torch.randn(t, h, generator=g).to(torch.bfloat16), "x_res": torch.randn(t, h, generator=g).to(torch.bfloat16),
         "weights": w, "top_k": k}
    print(f"case t={t} h={h} e={e} f={f} fs={fs} k={k}", flush=True)
    _check_layer(c, dev)


def test_moe_config3_decode_and_determinism(dev):
    c = configs.config3(32)
    out = _check_layer(c, dev)
    again, *_ = moe.moe_decode(c["h2"].to(dev), _dev_w(c["weights"], dev), top_k=8, x_res=c["x_res"].to(dev))
    assert torch.equal(out.view(torch.int16), again.cpu().view(torch.int16))


def test_moe_route_ties_and_experts_given_routing(dev):
    logits = torch.zeros(3, 32)
    logits[0, [5, 9, 30]] = 2.0
    logits[1] = torch.arange(32).float() % 4  # many ties at the top
    ids, wts = moe.moe_route(logits.to(dev), 6)
    sids, swts = omoe.route(logits, 6)
    assert torch.equal(ids.cpu(), sids)
    torch.testing.assert_close(wts.cpu(), swts)
    # ties in every register column of the 256- and 1024-expert layouts, and -inf logits (chosen last)
    for e, k in [(200, 8), (1000, 32)]:
        lg = (torch.arange(e) % 7).float().repeat(2, 1)
        lg[1, ::3] = float("-inf")
        ids, wts = moe.moe_route(lg.to(dev), k)
        sids, swts = omoe.route(lg, k)
        assert torch.equal(ids.cpu(), sids)
        torch.testing.assert_close(wts.cpu(), swts)
    ids, wts = moe.moe_route(logits.to(dev), 6)
    # experts with host-given routing (the reference's two-call path: host route(), experts kernel)
    g = torch.Generator().manual_seed(4)
    w = configs.moe_weights(g, hidden=128, experts=32, inter=64, shared_inter=64, router_std=0.5)
    h2 = torch.randn(3, 128, generator=g).to(torch.bfloat16)
    out = moe.moe_experts(h2.cuda(), _dev_w(w, dev), ids, wts).cpu()
    ref, *_ = omoe.moe_layer(h2, w, 6, ids=ids.cpu(), wts=wts.cpu(), round_base=False)
    torch.testing.assert_close(out.float(), ref.float(), **TOL)


def test_moe_experts_out_of_range_ids_select_nothing(dev):
    g = torch.Generator().manual_seed(9)
    w = configs.moe_weights(g, hidden=64, experts=8, inter=32, shared_inter=32, router_std=0.5)
    h2 = torch.randn(4, 64, generator=g).to(torch.bfloat16)
    ids = torch.tensor([[1, 2], [3, -1], [8, 0], [5, 6]], dtype=torch.int32)
    wts = torch.rand(4, 2, generator=g)
    out = moe.moe_experts(h2.to(dev), _dev_w(w, dev), ids.to(dev), wts.to(dev)).cpu()
    # the reference computation with each invalid pair replaced by a zero-weight valid expert
    ids_ref, wts_ref = ids.clone(), wts.clone()
    ids_ref[1, 1], ids_ref[2, 0] = 7, 7
    wts_ref[1, 1], wts_ref[2, 0] = 0.0, 0.0
    ref, *_ = omoe.moe_layer(h2, w, 2, ids=ids_ref, wts=wts_ref, round_base=False)
    torch.testing.assert_close(out.float(), ref.float(), **TOL)



# the prefill path (tokens > 256: blocked grouping, tile list, grouped MFMA GEMMs)
@pytest.mark.parametrize("t,h,e,f,fs,k", [(300, 128, 16, 64, 64, 4), (513, 256, 300, 64, 0, 8),
                                          (1000, 256, 64, 128, 192, 8), (257, 64, 8, 64, 64, 2)])
def test_moe_prefill_shapes(dev, t, h, e, f, fs, k):
    g = torch.Generator().manual_seed(t + e)
    w = configs.moe_weights(g, hidden=h, experts=e, inter=f, shared_inter=max(fs, 64), router_std=0.5)
    if fs == 0:
        for n in ("w_gate", "s_gate", "w_up", "s_up", "w_down", "s_down", "w_shg"):
            w.pop(n)
    c = {"h2": torch.randn(t, h, generator=g).to(torch.bfloat16), "x_res": torch.randn(t, h, generator=g).to(torch.bfloat16),
         "weights": w, "top_k": k}
    print(f"case t={t} h={h} e={e} f={f} fs={fs} k={k}", flush=True)
    _check_layer(c, dev)


def test_moe_prefill_config3b_and_determinism(dev):
    c = configs.config3(4096)
    out = _check_layer(c, dev)
    again, *_ = moe.moe_decode(c["h2"].to(dev), _dev_w(c["weights"], dev), top_k=8, x_res=c["x_res"].to(dev))
    assert torch.equal(out.view(torch.int16), again.cpu().view(torch.int16))


def test_moe_prefill_out_of_range_ids(dev):
    g = torch.Generator().manual_seed(21)
    w = configs.moe_weights(g, hidden=64, experts=8, inter=64, shared_inter=64, router_std=0.5)
    t = 400
    h2 = torch.randn(t, 64, generator=g).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(8, generator=g)[:2] for _ in range(t)]).to(torch.int32)
    ids[5, 1], ids[300, 0] = -3, 8
    wts = torch.rand(t, 2, generator=g)
    out = moe.moe_experts(h2.to(dev), _dev_w(w, dev), ids.to(dev), wts.to(dev)).cpu()
    ids_ref, wts_ref = ids.clone(), wts.clone()
    for r, c_ in ((5, 1), (300, 0)):
        other = int(ids[r, 1 - c_])
        ids_ref[r, c_] = (other + 1) % 8
        wts_ref[r, c_] = 0.0
    ref, *_ = omoe.moe_layer(h2, w, 2, ids=ids_ref, wts=wts_ref, round_base=False, slot_bf16=True)
    torch.testing.assert_close(out.float(), ref.float(), **TOL)
