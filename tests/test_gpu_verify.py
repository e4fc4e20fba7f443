"""GPU parity of the speculative-verification layers (axk_gdn_layer_verify / axk_attn_layer_verify through the C-ABI):
T new rows per sequence in one call against T decode steps of the oracle (the verify group's defining property,
models/qwen38_27b/verify/verify_group_m4.py:1-9) and against T calls of the GPU decode layers.

Bars: layer outputs the reference's bar for fused (composed) layer outputs, rel 5e-2 / abs 0.0625
(models/qwen35_35b_a3b/sgl/tests/test_gdn_attn.py:348-354, 537: a one-ulp flip of a bf16 intermediate, such as the
MLP's down output before the residual add, moves an output the residual has cancelled by up to that ulp); states
(and every per-row state snapshot) the temporal bar rel 5e-2 / abs 3e-3; conv states and snapshots: entries moved from the previous state exact, entries from this call's projections within the per-op
bar; KV rows written within the per-op bar, every other cache byte untouched.
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


def _gdn_case(seed, b, t, nk=2, nv=4):
    g = torch.Generator().manual_seed(seed)
    w = configs.gdn_layer_weights(g, H, F, nk, nv)
    x = torch.randn(b, t, H, generator=g).bfloat16()
    st = torch.randn(b, nv, 128, 128, generator=g) * 0.02
    cv = torch.randn(b, 3, 2 * nk * 128 + nv * 128, generator=g).bfloat16()
    return w, x, st, cv


def _conv_close(got, ref, fresh):
    """Conv state(s) [.., K-1, C]: the first K-1-fresh entries are moved inputs (exact), the last `fresh` are this
    call's projection rows (per-op bar)."""
    keep = got.shape[-2] - fresh
    if keep > 0:
        assert torch.equal(got[..., :keep, :].cpu(), ref[..., :keep, :])
    if fresh > 0:
        torch.testing.assert_close(got[..., keep:, :].float().cpu(), ref[..., keep:, :].float(), **TOL)


@pytest.mark.parametrize("b,t,nk,nv", [(2, 4, 2, 4), (5, 3, 1, 2), (1, 1, 2, 4), (3, 2, 16, 32)])
def test_gdn_layer_verify_matches_decode_steps(dev, b, t, nk, nv):
    w, x, st, cv = _gdn_case(b * 10 + t, b, t, nk, nv)
    print(f"gdn verify b={b} t={t} nk={nk} nv={nv}", flush=True)
    snap = torch.empty(t, *st.shape, device=dev)
    csnap = torch.empty(t, *cv.shape, dtype=torch.bfloat16, device=dev)
    out, so, co = layer.gdn_layer_verify(x.to(dev), _dev(w, dev), st.to(dev), cv.to(dev), nk, nv, state_snap=snap,
                                         conv_snap=csnap)
    ro, rs, rc, rsnap, rcsnap = olayer.gdn_layer_verify(x, w, st, cv, nk, nv)
    torch.testing.assert_close(out.float().cpu(), ro.float(), **FUSED_TOL)
    torch.testing.assert_close(so.cpu(), rs, **STATE_TOL)
    torch.testing.assert_close(snap.cpu(), rsnap, **STATE_TOL)
    assert torch.equal(snap[-1], so)  # the last row's snapshot is the state left in place
    _conv_close(co, rc, min(t, 3))
    for r in range(t):
        _conv_close(csnap[r], rcsnap[r], min(r + 1, 3))
    assert torch.equal(csnap[-1], co)


def test_gdn_layer_verify_equals_decode_layer_calls(dev):
    """One verify call == T GPU decode-layer calls (the same kernels' math per row; projections over B T rows)."""
    b, t = 4, 4
    w, x, st, cv = _gdn_case(77, b, t)
    wd = _dev(w, dev)
    out, so, co = layer.gdn_layer_verify(x.to(dev), wd, st.to(dev), cv.to(dev), 2, 4)
    s, c = st.to(dev), cv.to(dev)
    rows = []
    for r in range(t):
        o, s, c = layer.gdn_layer_decode(x[:, r].contiguous().to(dev), wd, s, c, 2, 4)
        rows.append(o)
    torch.testing.assert_close(out.float(), torch.stack(rows, 1).float(), **FUSED_TOL)
    torch.testing.assert_close(so, s, **STATE_TOL)
    _conv_close(co, c.cpu(), 3)


def test_gdn_layer_verify_in_place_and_rollback(dev):
    """States advanced in place; a host that accepts 2 of 4 draft rows restores the row-1 snapshots and continues
    with a decode step, which then equals decoding rows 0, 1 and the new row."""
    b, t = 2, 4
    w, x, st, cv = _gdn_case(5, b, t)
    wd = _dev(w, dev)
    sd, cd = st.to(dev), cv.to(dev)
    snap = torch.empty(t, *st.shape, device=dev)
    csnap = torch.empty(t, *cv.shape, dtype=torch.bfloat16, device=dev)
    layer.gdn_layer_verify(x.to(dev), wd, sd, cd, 2, 4, state_out=sd, conv_out=cd, state_snap=snap, conv_snap=csnap)
    torch.cuda.synchronize()
    assert torch.equal(sd, snap[-1]) and torch.equal(cd, csnap[-1])
    sd.copy_(snap[1])
    cd.copy_(csnap[1])
    xn = torch.randn(b, H, generator=torch.Generator().manual_seed(6)).bfloat16()
    o_new, _, _ = layer.gdn_layer_decode(xn.to(dev), wd, sd, cd, 2, 4)
    _, rs, rc, _, _ = olayer.gdn_layer_verify(x[:, :2], w, st, cv, 2, 4)
    ro, _, _ = olayer.gdn_layer_decode(xn, w, rs, rc, 2, 4)
    torch.testing.assert_close(o_new.float().cpu(), ro.float(), **FUSED_TOL)


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


# a draft crossing a page boundary (63 + 4 rows), sequences with little or no history, config 4's heads
@pytest.mark.parametrize("lens,rows,hq,hkv", [([100, 63, 300], 4, 4, 2), ([0, 1, 127], 3, 8, 2), ([640], 1, 4, 4),
                                              ([70, 200], 4, 32, 4), ([17 + 9 * i for i in range(6)], 2, 4, 2)])
def test_attn_layer_verify_matches_decode_steps(dev, lens, rows, hq, hkv):
    w, c, x, cos, sin = _attn_case(lens, rows, hq, hkv, len(lens) * 3 + rows)
    print(f"attn verify lens={lens} rows={rows} hq={hq} hkv={hkv}", flush=True)
    cache = c["cache"].to(dev)
    out = layer.attn_layer_verify(x.to(dev), _dev(w, dev), cos.to(dev), sin.to(dev), cache, c["indptr"].to(dev),
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


def test_verify_contract_errors(dev):
    w, x, st, cv = _gdn_case(3, 2, 4)
    wd = _dev(w, dev)
    with pytest.raises(ValueError):  # 17 rows: more than the verify entries take
        layer.gdn_verify_workspace(2, 17, H, 2, 4, F, dev)
    ws = layer.gdn_verify_workspace(2, 4, H, 2, 4, F, dev)
    sd, cd = st.to(dev), cv.to(dev)
    # a conv snapshot that overlaps the conv state it is taken from
    raw = torch.empty(4 * cv.numel(), dtype=torch.bfloat16, device=dev)
    cd_alias = raw[:cv.numel()].view(cv.shape)
    cd_alias.copy_(cd)
    with pytest.raises(_lib.AxkError) as e:
        layer.gdn_layer_verify(x.to(dev), wd, sd, cd_alias, 2, 4, workspace=ws, conv_out=cd_alias,
                               conv_snap=raw.view(4, *cv.shape))
    assert e.value.status == 5  # AXK_E_ALIAS
    torch.cuda.synchronize()
    assert torch.equal(cd_alias.cpu(), cv)  # nothing ran
