"""GPU parity of the prefill layers (axk_gdn_layer_prefill / axk_attn_layer_prefill through the C-ABI): T new tokens
per sequence in one call (models/qwen35_35b_a3b/src/70b0fbc/q35_prefill.py: gdn_layer_prefill 57-141,
attn_layer_prefill 172-336).

Oracles: the GDN layer against oracle.layer.gdn_layer_prefill (the chunked delta rule with the reference's bf16
rounding points, 64-token chunks, the conv over the tokens from the conv state), and at small T also against T decode
steps (oracle.layer.gdn_layer_verify); the attention layer against T decode steps (oracle.layer.attn_layer_verify:
token t attends the history and tokens 0 .. t). Ragged T (not a multiple of the 64-token chunk), T = 1, sequences
with and without history, and rows >= 128 (the dense GEMM path of every projection).

Bars: layer outputs the fused-layer bar rel 5e-2 / abs 0.0625 (models/qwen35_35b_a3b/sgl/tests/test_gdn_attn.py:
348-354, 537); recurrent states the temporal bar rel 5e-2 / abs 3e-3; conv states: entries moved from the input
state exact, entries from this call's projection rows within the per-op bar rel 2e-2 / abs 1e-2; KV rows written
within the per-op bar and every other cache byte untouched.
"""
import pytest
import torch

from axk import _lib, configs, layer
from oracle import layer as olayer

pytestmark = pytest.mark.gpu
TOL = dict(rtol=2e-2, atol=1e-2)
FUSED_TOL = dict(rtol=5e-2, atol=0.0625)
STATE_TOL = dict(rtol=5e-2, atol=3e-3)
H, F = 256, 512


def _dev(w, dev):
    return {k: v.to(dev) for k, v in w.items()}


def _gdn_case(seed, b, t, nk=2, nv=4, proj_fmt="fp8", mlp_fmt="mxfp4"):
    g = torch.Generator().manual_seed(seed)
    w = configs.gdn_layer_weights(g, H, F, nk, nv, proj_fmt=proj_fmt, mlp_fmt=mlp_fmt)
    x = torch.randn(b, t, H, generator=g).bfloat16()
    st = torch.randn(b, nv, 128, 128, generator=g) * 0.02
    cv = torch.randn(b, 3, 2 * nk * 128 + nv * 128, generator=g).bfloat16()
    return w, x, st, cv


def _conv_close(got, ref, fresh):
    keep = got.shape[-2] - fresh
    if keep > 0:
        assert torch.equal(got[..., :keep, :].cpu(), ref[..., :keep, :])
    if fresh > 0:
        torch.testing.assert_close(got[..., keep:, :].float().cpu(), ref[..., keep:, :].float(), **TOL)


def _fused_close(got, ref, slack):
    """The fused bar plus the slack of one-ulp flips of the gated output rows (oracle.layer.gdn_layer_prefill_parts):
    with MXFP4 projections the gate raises that bf16 intermediate to tens, where one ulp times a large weight is
    above the bar's absolute term."""
    ref = ref.float()
    d = (got.float().cpu() - ref).abs()
    tol = FUSED_TOL["atol"] + FUSED_TOL["rtol"] * ref.abs()
    assert (d <= tol + slack).all(), f"max excess {(d - tol - slack).max().item()}"


# ragged chunks (100 = 64 + 36), one token, exactly one chunk, rows >= 128 in the dense GEMM path, the 35B's heads,
# NVFP4 weights
@pytest.mark.parametrize("b,t,nk,nv,proj_fmt,mlp_fmt", [(2, 100, 2, 4, "fp8", "mxfp4"), (3, 1, 2, 4, "fp8", "mxfp4"),
                                                       (1, 64, 2, 2, "mxfp8", "mxfp8"),
                                                       (2, 130, 1, 2, "mxfp4", "mxfp8"),
                                                       (1, 40, 16, 32, "mxfp8", "mxfp4"),
                                                       # NVFP4 projections and MLP, rows >= 128 (the prefill GEMM)
                                                       (2, 100, 2, 4, "nvfp4", "nvfp4")])
def test_gdn_layer_prefill_matches_oracle(dev, b, t, nk, nv, proj_fmt, mlp_fmt):
    w, x, st, cv = _gdn_case(b * 1000 + t + nk, b, t, nk, nv, proj_fmt, mlp_fmt)
    print(f"gdn prefill b={b} t={t} nk={nk} nv={nv} {proj_fmt}/{mlp_fmt}", flush=True)
    out, so, co = layer.gdn_layer_prefill(x.to(dev), _dev(w, dev), st.to(dev), cv.to(dev), nk, nv,
                                          proj_fmt=proj_fmt, mlp_fmt=mlp_fmt)
    ro, rs, rc, slack = olayer.gdn_layer_prefill_parts(x, w, st, cv, nk, nv, proj_fmt=proj_fmt, mlp_fmt=mlp_fmt)
    _fused_close(out, ro, slack)
    torch.testing.assert_close(so.cpu(), rs, **STATE_TOL)
    _conv_close(co, rc, min(t, 3))


def test_gdn_layer_prefill_state_matches_decode_steps(dev):
    """At small T the prefill's states equal those of T decode steps (the recurrent form) within the temporal bar.
    (Its outputs are held to the chunked oracle above, which equals the recurrent form in fp32 arithmetic,
    tests/test_oracle_layer.py; against the recurrent form's own bf16 points the chunk products' rounding moves the
    core by up to the per-op bar, which the gate and the output projection amplify past the fused bar.)"""
    b, t = 2, 12
    w, x, st, cv = _gdn_case(12, b, t)
    out, so, co = layer.gdn_layer_prefill(x.to(dev), _dev(w, dev), st.to(dev), cv.to(dev), 2, 4)
    _, rs, rc, _, _ = olayer.gdn_layer_verify(x, w, st, cv, 2, 4)
    torch.testing.assert_close(so.cpu(), rs, **STATE_TOL)
    _conv_close(co, rc, 3)


def test_gdn_layer_prefill_in_two_halves_continues(dev):
    """A prefill of 90 tokens then one of 60 from its state and conv rows, in place (the reference's two-half
    prefill, q35_prefill.py:60-68), against the oracle run the same way; the states equal those of one prefill
    of all 150 tokens within the temporal bar."""
    b, t, t1 = 2, 150, 90
    w, x, st, cv = _gdn_case(150, b, t)
    wd = _dev(w, dev)
    _, sf, cf = layer.gdn_layer_prefill(x.to(dev), wd, st.to(dev), cv.to(dev), 2, 4)
    sd, cd = st.to(dev), cv.to(dev)
    o1, _, _ = layer.gdn_layer_prefill(x[:, :t1].contiguous().to(dev), wd, sd, cd, 2, 4, state_out=sd, conv_out=cd)
    o2, _, _ = layer.gdn_layer_prefill(x[:, t1:].contiguous().to(dev), wd, sd, cd, 2, 4, state_out=sd, conv_out=cd)
    r1, rs1, rc1, sl1 = olayer.gdn_layer_prefill_parts(x[:, :t1], w, st, cv, 2, 4)
    r2, rs2, rc2, sl2 = olayer.gdn_layer_prefill_parts(x[:, t1:], w, rs1, rc1, 2, 4)
    _fused_close(o1, r1, sl1)
    _fused_close(o2, r2, sl2)
    torch.testing.assert_close(sd.cpu(), rs2, **STATE_TOL)
    _conv_close(cd, rc2, 3)
    torch.testing.assert_close(sd, sf, **STATE_TOL)
    torch.testing.assert_close(cd.float(), cf.float(), **TOL)


def _attn_case(lens, rows, hq, hkv, seed, page=64):
    g = torch.Generator().manual_seed(seed)
    d = 256
    w = configs.attn_layer_weights(g, H, F, hq, hkv, d)
    c = configs.verify_rows_case(lens, rows, hq, hkv, d, page, g)
    x = torch.randn(len(lens), rows, H, generator=g).bfloat16()
    cos, sin = olayer.rope_cos_sin(c["pos"].reshape(-1), 64, 10_000_000.0)
    cos = cos.reshape(len(lens), rows, -1).contiguous()
    sin = sin.reshape(len(lens), rows, -1).contiguous()
    return w, c, x, cos, sin


# a fresh prompt (no history), history + new tokens across page boundaries, rows >= 128, config 4's heads
@pytest.mark.parametrize("lens,rows,hq,hkv", [([0, 0], 70, 4, 2), ([100, 5, 300], 48, 4, 2), ([37], 150, 8, 2),
                                              ([64, 200], 20, 32, 4)])
def test_attn_layer_prefill_matches_decode_steps(dev, lens, rows, hq, hkv):
    w, c, x, cos, sin = _attn_case(lens, rows, hq, hkv, len(lens) * 7 + rows)
    print(f"attn prefill lens={lens} rows={rows} hq={hq} hkv={hkv}", flush=True)
    cache = c["cache"].to(dev)
    out = layer.attn_layer_prefill(x.to(dev), _dev(w, dev), cos.to(dev), sin.to(dev), cache, c["indptr"].to(dev),
                                   c["indices"].to(dev), c["last_page_len"].to(dev), c["loc"].to(dev), hq, 64)
    ro, rcache = olayer.attn_layer_verify(x, w, cos, sin, c["cache"], c["indptr"], c["indices"], c["last_page_len"],
                                          c["loc"], hq, 64)
    torch.testing.assert_close(out.float().cpu(), ro.float(), **FUSED_TOL)
    got = cache.cpu()
    written = torch.zeros(got.shape[0], got.shape[2], dtype=torch.bool)
    for p, o in c["loc"].reshape(-1, 2).tolist():
        written[p, o] = True
    torch.testing.assert_close(got.permute(0, 2, 1, 3, 4)[written].float(),
                               rcache.permute(0, 2, 1, 3, 4)[written].float(), **TOL)
    assert torch.equal(got.permute(0, 2, 1, 3, 4)[~written].view(torch.int16),
                       c["cache"].permute(0, 2, 1, 3, 4)[~written].view(torch.int16))


def test_attn_layer_prefill_equals_verify_layer(dev):
    """At T <= 16 the prefill and the verify entries run the same kernels: bit-identical outputs and caches."""
    w, c, x, cos, sin = _attn_case([90, 10], 8, 4, 2, 3)
    wd = _dev(w, dev)
    outs, caches = [], []
    for fn in (layer.attn_layer_prefill, layer.attn_layer_verify):
        cache = c["cache"].to(dev)
        outs.append(fn(x.to(dev), wd, cos.to(dev), sin.to(dev), cache, c["indptr"].to(dev), c["indices"].to(dev),
                       c["last_page_len"].to(dev), c["loc"].to(dev), 4, 64))
        caches.append(cache)
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert torch.equal(caches[0].view(torch.int16), caches[1].view(torch.int16))


def test_prefill_contract_errors_enqueue_nothing(dev):
    w, x, st, cv = _gdn_case(4, 2, 20)
    wd = _dev(w, dev)
    sd, cd = st.to(dev), cv.to(dev)
    ws = layer.gdn_prefill_workspace(2, 20, H, 2, 4, F, dev)
    with pytest.raises(_lib.AxkError) as e:  # a workspace one byte short
        layer.gdn_layer_prefill(x.to(dev), wd, sd, cd, 2, 4, workspace=ws[:-1], state_out=sd, conv_out=cd)
    assert e.value.status == 6  # AXK_E_WORKSPACE
    bad = dict(wd)
    bad["w_out"] = torch.zeros(wd["w_out"].numel() + 16, dtype=torch.uint8, device=dev)[1:1 + wd["w_out"].numel()] \
        .view(wd["w_out"].shape)  # one byte off a 16-byte boundary
    with pytest.raises(_lib.AxkError) as e:
        layer.gdn_layer_prefill(x.to(dev), bad, sd, cd, 2, 4, state_out=sd, conv_out=cd)
    assert e.value.status == 3  # AXK_E_ALIGN, found by the validate pass before the conv / state launches
    torch.cuda.synchronize()
    assert torch.equal(sd.cpu(), st) and torch.equal(cd.cpu(), cv)


# ---- the MoE prefill layers (qwen35moe_gdn_prefill / qwen35moe_attn_prefill, q35_moe_prefill.py:47-77) ----
def _routing_outputs(rows, blk, dev):
    e, k = blk["w_router"].shape[0], blk["top_k"]
    return dict(logits=torch.empty(rows, e, device=dev), topk_ids=torch.empty(rows, k, dtype=torch.int32, device=dev),
                topk_weights=torch.empty(rows, k, device=dev))


def _check_moe(out, r, x, y, w, blk, fmt, extra_slack):
    """out [B, T, H]; r the kernel's routing outputs over the B T rows; y [B T, H] the oracle's first half; more
    than 256 rows take the grouped prefill experts, whose slots are bf16 (oracle slot_bf16)."""
    from oracle import moe as omoe

    rows = y.shape[0]
    logits, ids, wts = r["logits"].cpu(), r["topk_ids"].cpu(), r["topk_weights"].cpu()
    sids, swts = omoe.route(logits, blk["top_k"], True)
    assert torch.equal(ids, sids), "top-K ids differ from the stable sort of the kernel's logits"
    torch.testing.assert_close(wts, swts, rtol=1e-5, atol=1e-6)
    base, routed, slack, ref_logits, _, _ = olayer.moe_block_parts(x.reshape(rows, -1), y, w, blk, fmt=fmt,
                                                                   ids=ids.long(), wts=wts, slot_bf16=rows > 256)
    torch.testing.assert_close(logits, ref_logits, **TOL)
    ref = (base + routed).bfloat16().float()
    d = (out.reshape(rows, -1).float().cpu() - ref).abs()
    tol = FUSED_TOL["atol"] + FUSED_TOL["rtol"] * ref.abs()
    assert (d <= tol + slack + extra_slack).all(), f"max excess {(d - tol - slack - extra_slack).max().item()}"


def _dev_any(w, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in w.items()}


# 40 rows (the decode experts), 300 rows (the grouped prefill experts with bf16 slots), the 35B's widths
@pytest.mark.parametrize("b,t,h,nk,nv,e,fe,k,fmt", [(2, 20, 256, 2, 4, 16, 256, 4, "mxfp8"),
                                                    (2, 150, 256, 2, 4, 40, 256, 8, "mxfp4"),
                                                    (1, 300, 2048, 16, 32, 256, 512, 8, "mxfp8")])
def test_gdn_layer_prefill_moe(dev, b, t, h, nk, nv, e, fe, k, fmt):
    g = torch.Generator().manual_seed(b * t + e)
    print(f"gdn prefill moe b={b} t={t} h={h} e={e} {fmt}", flush=True)
    w = configs.gdn_layer_weights(g, h, 256, nk, nv, proj_fmt="mxfp8", mlp_fmt=fmt)
    blk = configs.moe_block(g, h, e, fe, k)
    x = torch.randn(b, t, h, generator=g).bfloat16()
    st = torch.randn(b, nv, 128, 128, generator=g) * 0.02
    cv = torch.randn(b, 3, (2 * nk + nv) * 128, generator=g).bfloat16()
    r = _routing_outputs(b * t, blk, dev)
    out, so, co = layer.gdn_layer_prefill(x.to(dev), _dev(w, dev), st.to(dev), cv.to(dev), nk, nv, proj_fmt="mxfp8",
                                          mlp_fmt=fmt, moe=dict(_dev_any(blk, dev), **r))
    y, rs, rc, yslack = olayer.gdn_prefill_half(x, w, st, cv, nk, nv, proj_fmt="mxfp8")
    _check_moe(out, r, x, y, w, blk, fmt, yslack)
    torch.testing.assert_close(so.cpu(), rs, **STATE_TOL)
    _conv_close(co, rc, 3)


def test_gdn_layer_prefill_moe_bench_shape(dev):
    """The bench's moe_layer_prefill itself: the 35B GDN MoE layer (hidden 2048, 16 / 32 heads, MXFP8 projections and
    shared expert of 512, 256 MXFP4 experts of 512, top-8) over one 4096-token chunk from a random state."""
    g = torch.Generator().manual_seed(4096)
    b, t, h, nk, nv, e, fe, k, fmt = 1, 4096, 2048, 16, 32, 256, 512, 8, "mxfp8"
    print("gdn prefill moe at the bench shape: t=4096 h=2048 e=256", flush=True)
    w = configs.gdn_layer_weights(g, h, 512, nk, nv, proj_fmt="mxfp8", mlp_fmt=fmt)
    blk = configs.moe_block(g, h, e, fe, k)
    x = torch.randn(b, t, h, generator=g).bfloat16()
    st = torch.randn(b, nv, 128, 128, generator=g) * 0.02
    cv = torch.randn(b, 3, (2 * nk + nv) * 128, generator=g).bfloat16()
    r = _routing_outputs(b * t, blk, dev)
    out, so, co = layer.gdn_layer_prefill(x.to(dev), _dev(w, dev), st.to(dev), cv.to(dev), nk, nv, proj_fmt="mxfp8",
                                          mlp_fmt=fmt, moe=dict(_dev_any(blk, dev), **r))
    y, rs, rc, yslack = olayer.gdn_prefill_half(x, w, st, cv, nk, nv, proj_fmt="mxfp8")
    _check_moe(out, r, x, y, w, blk, fmt, yslack)
    torch.testing.assert_close(so.cpu(), rs, **STATE_TOL)
    _conv_close(co, rc, 3)


def test_attn_layer_prefill_moe(dev):
    """140 new tokens for each of 2 sequences (280 rows: the grouped prefill experts) over histories of 100 and 5."""
    g = torch.Generator().manual_seed(280)
    hq, hkv, rows = 4, 2, 140
    w = configs.attn_layer_weights(g, H, 256, hq, hkv, 256, proj_fmt="mxfp8", mlp_fmt="mxfp8")
    blk = configs.moe_block(g, H, 16, 256, 4)
    c = configs.verify_rows_case([100, 5], rows, hq, hkv, 256, 64, g)
    x = torch.randn(2, rows, H, generator=g).bfloat16()
    cos, sin = olayer.rope_cos_sin(c["pos"].reshape(-1), 64, 10_000_000.0)
    cos, sin = cos.reshape(2, rows, -1).contiguous(), sin.reshape(2, rows, -1).contiguous()
    r = _routing_outputs(2 * rows, blk, dev)
    cache = c["cache"].to(dev)
    out = layer.attn_layer_prefill(x.to(dev), _dev(w, dev), cos.to(dev), sin.to(dev), cache, c["indptr"].to(dev),
                                   c["indices"].to(dev), c["last_page_len"].to(dev), c["loc"].to(dev), hq, 64,
                                   proj_fmt="mxfp8", mlp_fmt="mxfp8", moe=dict(_dev_any(blk, dev), **r))
    y, rcache = olayer.attn_rows_half(x, w, cos, sin, c["cache"], c["indptr"], c["indices"], c["last_page_len"],
                                      c["loc"], hq, 64, proj_fmt="mxfp8")
    _check_moe(out, r, x, y, w, blk, "mxfp8", 0.0)
    got = cache.cpu()
    written = torch.zeros(got.shape[0], got.shape[2], dtype=torch.bool)
    for p, o in c["loc"].reshape(-1, 2).tolist():
        written[p, o] = True
    torch.testing.assert_close(got.permute(0, 2, 1, 3, 4)[written].float(),
                               rcache.permute(0, 2, 1, 3, 4)[written].float(), **TOL)

