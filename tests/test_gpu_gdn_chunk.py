"""GPU parity of the GDN chunked prefill (axk_gdn_chunk_prefill) against the oracle.

Bars: bf16 outputs within rel 2e-2 / abs 1e-2 of the oracle's chunked form with the reference's rounding
points (oracle.gdn.gdn_chunk) and of the fp32 recurrence; the fp32 final state within the reference's own
temporal tolerance, rel 5e-2 / abs 3e-3 (test_gdn_attn.py:711-712), of both. Invariants: chunked == recurrent
(the decode kernel over the same tokens), prefill then decode == recurrence over all tokens, in-place state.
"""
import pytest
import torch

from axk import configs, gdn
from oracle import gdn as ogdn

pytestmark = pytest.mark.gpu
TOL = dict(rtol=2e-2, atol=1e-2)
STATE_TOL = dict(rtol=5e-2, atol=3e-3)
ARGS = ("q", "k", "v", "a", "b", "a_log", "dt_bias", "state")


def _case(bsz, t, nk, nv, seed, state_std=0.02, gates=True):
    g = torch.Generator().manual_seed(seed)
    c = configs.gdn_inputs(bsz, t, g, nk=nk, nv=nv, state_std=state_std)
    if gates:  # non-trivial A_log / dt_bias (the config-2 draws use zeros)
        c["a_log"] = torch.randn(nv, generator=g) * 0.5
        c["dt_bias"] = torch.randn(nv, generator=g) * 0.5
    return c


def _chunk(c, dev, inplace=False, workspace=None):
    d = {k: v.to(dev) for k, v in c.items()}
    out, st = gdn.gdn_chunk_prefill(*(d[n] for n in ARGS), state_out=d["state"] if inplace else None,
                                    workspace=workspace)
    return out.cpu(), st.cpu()


def _check(c, out, st):
    args = [c[n] for n in ARGS]
    o_ref, s_ref = ogdn.gdn_chunk(*args, chunk=64, round_bf16=True)
    torch.testing.assert_close(out.float(), o_ref.float(), **TOL)
    torch.testing.assert_close(st, s_ref, **STATE_TOL)
    o32, s32 = ogdn.gdn_fp32(*args)
    torch.testing.assert_close(out.float(), o32.to(torch.bfloat16).float(), **TOL)
    torch.testing.assert_close(st, s32, **STATE_TOL)


@pytest.mark.parametrize("bsz,t,nk,nv,std", [(1, 64, 1, 1, 0.02), (1, 1, 1, 2, 0.02), (2, 100, 2, 4, 0.0),
                                             (3, 130, 1, 3, 0.02), (1, 257, 4, 8, 0.02), (2, 640, 2, 2, 0.0)])
def test_chunk_prefill_shapes(dev, bsz, t, nk, nv, std):
    print(f"case bsz={bsz} t={t} nk={nk} nv={nv} std={std}", flush=True)
    c = _case(bsz, t, nk, nv, seed=t + nv, state_std=std)
    out, st = _chunk(c, dev)
    _check(c, out, st)


def test_chunk_prefill_config2b(dev):
    c = configs.config2_prefill()
    out, st = _chunk(c, dev)
    _check(c, out, st)
    # the decode kernel over the same 4096 tokens (the recurrent form) agrees with the chunked form
    d = {k: v.to(dev) for k, v in c.items()}
    r_out, r_st = gdn.gdn_recurrent(*(d[n] for n in ARGS))
    torch.testing.assert_close(out.float(), r_out.cpu().float(), **TOL)
    torch.testing.assert_close(st, r_st.cpu(), **STATE_TOL)


def test_prefill_then_decode_continuation(dev):
    c = _case(2, 200, 2, 4, seed=11)
    head = {k: (v[:, :199].contiguous() if v.dim() >= 3 and k != "state" else v) for k, v in c.items()}
    out, st = _chunk(head, dev)
    d = {k: v.to(dev) for k, v in c.items()}
    step = {n: d[n][:, 199:200].contiguous() for n in ("q", "k", "v", "a", "b")}
    o1, s1 = gdn.gdn_recurrent(step["q"], step["k"], step["v"], step["a"], step["b"], d["a_log"], d["dt_bias"],
                               st.to(dev))
    o_all, s_all = ogdn.gdn_fp32(*(c[n] for n in ARGS))
    torch.testing.assert_close(out.float(), o_all[:, :199].to(torch.bfloat16).float(), **TOL)
    torch.testing.assert_close(o1.cpu().float(), o_all[:, 199:200].to(torch.bfloat16).float(), **TOL)
    torch.testing.assert_close(s1.cpu(), s_all, **STATE_TOL)


def test_chunk_prefill_in_place_and_workspace_reuse(dev):
    c = _case(1, 150, 2, 4, seed=5)
    ws = gdn.gdn_chunk_workspace(1, 150, 2, 4, dev)
    ref_out, ref_st = _chunk(c, dev, workspace=ws)
    out, st = _chunk(c, dev, inplace=True, workspace=ws)
    assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
    assert torch.equal(st, ref_st)


def test_chunk_prefill_contract_errors(dev):
    c = _case(1, 70, 1, 2, seed=1)
    d = {k: v.to(dev) for k, v in c.items()}
    with pytest.raises(ValueError):
        gdn.gdn_chunk_workspace(1, 70, 1, 2, dev, chunk_size=32)  # chunk 64 only
    small = torch.empty(1024, dtype=torch.uint8, device=dev)
    from axk import _lib

    with pytest.raises(_lib.AxkError):
        gdn.gdn_chunk_prefill(*(d[n] for n in ARGS), workspace=small)
