"""GPU parity of the GDN recurrent / decode kernel against the oracle (bf16 outputs rel 2e-2 / abs 1e-2;
the fp32 state against the fp32 recurrence at rel 1e-3 / abs 1e-4, and against the reference golden, whose
bf16 rounding points it does not share, at the output tolerance)."""
import pytest
import torch

from axk import configs, gdn
from oracle import gdn as ogdn

pytestmark = pytest.mark.gpu
TOL = dict(rtol=2e-2, atol=1e-2)


def _dev(c, dev):
    return {k: v.to(dev) for k, v in c.items()}


def _run(c, dev, inplace=False):
    d = _dev(c, dev)
    out, st = gdn.gdn_recurrent(d["q"], d["k"], d["v"], d["a"], d["b"], d["a_log"], d["dt_bias"], d["state"],
                                state_out=d["state"] if inplace else None)
    return out.cpu(), st.cpu()


def _args(c):
    return c["q"], c["k"], c["v"], c["a"], c["b"], c["a_log"], c["dt_bias"], c["state"]


def test_gdn_decode_config2(dev):
    c = configs.config2_decode()
    out, st = _run(c, dev)
    o32, s32 = ogdn.gdn_fp32(*_args(c))
    torch.testing.assert_close(out.float(), o32.to(torch.bfloat16).float(), **TOL)
    torch.testing.assert_close(st, s32, rtol=1e-3, atol=1e-4)
    o_ref, s_ref = ogdn.gdn_reference(*_args(c))
    torch.testing.assert_close(out.float(), o_ref.float(), **TOL)
    torch.testing.assert_close(st, s_ref, **TOL)


@pytest.mark.parametrize("bsz,t,nk,nv", [(1, 1, 1, 1), (2, 7, 4, 8), (3, 33, 16, 32)])
def test_gdn_multi_token_and_gates(dev, bsz, t, nk, nv):
    g = torch.Generator().manual_seed(bsz * 100 + t)
    c = configs.gdn_inputs(bsz, t, g, nk=nk, nv=nv, state_std=0.05)
    c["a_log"] = torch.randn(nv, generator=g) * 0.5
    c["dt_bias"] = torch.randn(nv, generator=g) * 0.5
    print(f"case bsz={bsz} t={t} nk={nk} nv={nv}", flush=True)
    out, st = _run(c, dev)
    o32, s32 = ogdn.gdn_fp32(*_args(c))
    torch.testing.assert_close(out.float(), o32.to(torch.bfloat16).float(), **TOL)
    torch.testing.assert_close(st, s32, rtol=1e-3, atol=1e-4)


def test_gdn_in_place_equals_out_of_place_and_decode_chain(dev):
    c = configs.gdn_inputs(2, 6, torch.Generator().manual_seed(9), nk=4, nv=8)
    out_a, st_a = _run(c, dev)
    out_b, st_b = _run(c, dev, inplace=True)
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16)) and torch.equal(st_a, st_b)
    # six single-token decode steps chained through the state == one 6-token call (same kernel math)
    d = _dev(c, dev)
    state = d["state"].clone()
    outs = []
    for t in range(6):
        sl = lambda x: x[:, t : t + 1].contiguous()
        o, state = gdn.gdn_recurrent(sl(d["q"]), sl(d["k"]), sl(d["v"]), sl(d["a"]), sl(d["b"]), d["a_log"],
                                     d["dt_bias"], state, state_out=state)
        outs.append(o)
    assert torch.equal(torch.cat(outs, 1).cpu().view(torch.int16), out_a.view(torch.int16))
    assert torch.equal(state.cpu(), st_a)
