"""Pins the GDN oracle (CPU only)."""
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn


def _case(B=2, T=5, NK=2, NV=4, D=16, seed=0, zero_state=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, NK, D, generator=g).bfloat16()
    k = torch.randn(B, T, NK, D, generator=g).bfloat16()
    v = torch.randn(B, T, NV, D, generator=g).bfloat16()
    a = torch.randn(B, T, NV, generator=g).bfloat16()
    b = torch.randn(B, T, NV, generator=g).bfloat16()
    a_log = torch.randn(NV, generator=g) * 0.5
    dt_bias = torch.randn(NV, generator=g) * 0.5
    s = torch.zeros(B, NV, D, D) if zero_state else torch.randn(B, NV, D, D, generator=g) * 0.02
    return q, k, v, a, b, a_log, dt_bias, s


def test_fp32_matches_transformers_recurrent_rule():
    from transformers.models.qwen3_5.modeling_qwen3_5 import torch_recurrent_gated_delta_rule

    q, k, v, a, b, a_log, dt_bias, s = _case()
    out, st = gdn.gdn_fp32(q, k, v, a, b, a_log, dt_bias, s)
    g, beta = gdn.gates(a, b, a_log, dt_bias)
    rep = v.shape[2] // q.shape[2]
    ref_out, ref_st = torch_recurrent_gated_delta_rule(
        q.float().repeat_interleave(rep, 2), k.float().repeat_interleave(rep, 2), v.float(), g, beta, s.clone(),
        True, use_qk_l2norm_in_kernel=True)
    torch.testing.assert_close(out, ref_out.float(), rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(st, ref_st.float(), rtol=1e-4, atol=1e-4)


def test_single_step_from_zero_state_closed_form():
    # S1 = beta k v^T (the decay multiplies a zero state); o = (q.k) beta v with unit q, k and q scaled
    q, k, v, a, b, a_log, dt_bias, s = _case(B=1, T=1, NK=1, NV=1, zero_state=True)
    out, st = gdn.gdn_fp32(q, k, v, a, b, a_log, dt_bias, s)
    qn = F.normalize(q[0, 0, 0].double(), dim=0, eps=0) * 16 ** -0.5
    kn = F.normalize(k[0, 0, 0].double(), dim=0, eps=0)
    beta = torch.sigmoid(b[0, 0, 0].double())
    torch.testing.assert_close(st[0, 0].double(), beta * torch.outer(kn, v[0, 0, 0].double()), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(out[0, 0, 0].double(), (qn @ kn) * beta * v[0, 0, 0].double(), rtol=1e-5, atol=1e-6)


def test_gate_formula_and_gqa_head_order():
    q, k, v, a, b, a_log, dt_bias, s = _case(B=1, T=1, NK=2, NV=4)
    g, beta = gdn.gates(a, b, a_log, dt_bias)
    h = 3
    want = -torch.exp(a_log[h]) * torch.log1p(torch.exp(a[0, 0, h].float() + dt_bias[h]))
    torch.testing.assert_close(g[0, 0, h], want)
    # value head h reads key head h // (NV / NK): perturbing key head 0 leaves heads 2, 3 unchanged
    k2 = k.clone()
    k2[:, :, 0] = torch.randn_like(k2[:, :, 0].float()).bfloat16()
    o1, _ = gdn.gdn_fp32(q, k, v, a, b, a_log, dt_bias, s)
    o2, _ = gdn.gdn_fp32(q, k2, v, a, b, a_log, dt_bias, s)
    assert torch.equal(o1[:, :, 2:], o2[:, :, 2:]) and not torch.equal(o1[:, :, :2], o2[:, :, :2])


def test_reference_golden_close_to_fp32():
    # the reference golden differs from exact arithmetic only by its bf16 rounding points
    q, k, v, a, b, a_log, dt_bias, s = _case(T=8, D=32, seed=3)
    o_ref, s_ref = gdn.gdn_reference(q, k, v, a, b, a_log, dt_bias, s)
    o32, s32 = gdn.gdn_fp32(q, k, v, a, b, a_log, dt_bias, s)
    torch.testing.assert_close(o_ref.float(), o32, rtol=2e-2, atol=1e-2)
    torch.testing.assert_close(s_ref, s32, rtol=2e-2, atol=1e-2)


def test_chunk_fp32_matches_transformers_chunk_rule():
    from transformers.models.qwen3_5.modeling_qwen3_5 import torch_chunk_gated_delta_rule

    q, k, v, a, b, a_log, dt_bias, s = _case(B=2, T=150, NK=2, NV=4, D=32, seed=3)
    g, beta = gdn.gates(a, b, a_log, dt_bias)
    rep = v.shape[2] // q.shape[2]
    for chunk in (16, 64):
        out, st = gdn.gdn_chunk(q, k, v, a, b, a_log, dt_bias, s, chunk=chunk, round_bf16=False)
        ref_out, ref_st = torch_chunk_gated_delta_rule(
            q.float().repeat_interleave(rep, 2), k.float().repeat_interleave(rep, 2), v.float(), g, beta, chunk,
            s.clone(), True, use_qk_l2norm_in_kernel=True)
        torch.testing.assert_close(out, ref_out.float(), rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(st, ref_st.float(), rtol=1e-5, atol=1e-5)


def test_chunked_equals_recurrent():
    # the chunked form is an exact rewrite of the recurrence (q35_prefill.py:439-463 checks the same)
    q, k, v, a, b, a_log, dt_bias, s = _case(B=1, T=97, NK=1, NV=2, D=32, seed=4)
    out, st = gdn.gdn_chunk(q, k, v, a, b, a_log, dt_bias, s, chunk=32, round_bf16=False)
    ref_out, ref_st = gdn.gdn_fp32(q, k, v, a, b, a_log, dt_bias, s)
    torch.testing.assert_close(out, ref_out, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(st, ref_st, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("size,batch", [(1, 1), (2, 2), (17, 1), (32, 2), (64, 1), (256, 2)])
def test_unit_lower_inverse_reference_cases(size, batch):
    # the correlated strictly-lower matrices of test_gdn_attn.py:738-768, against a triangular solve
    pos = torch.arange(size)
    dist = pos[:, None] - pos[None, :]
    neg = torch.tril(-0.96 * torch.exp(-0.012 * dist.float()), diagonal=-1)
    if batch > 1:
        neg = torch.stack((neg, neg * 0.7))
    eye = torch.eye(size, dtype=torch.float64).expand(neg.shape)
    expected = torch.linalg.solve_triangular(eye - neg.double(), eye, upper=False)
    got = gdn.unit_lower_inverse(neg)
    torch.testing.assert_close(got.double(), expected, rtol=2e-5, atol=2e-6)
    torch.testing.assert_close((eye - neg.double()) @ got.double(), eye, rtol=0, atol=3e-6)


def test_chunk_bf16_schedule_close_to_fp32():
    q, k, v, a, b, a_log, dt_bias, s = _case(B=1, T=130, NK=2, NV=4, D=128, seed=5)
    out, st = gdn.gdn_chunk(q, k, v, a, b, a_log, dt_bias, s, chunk=64, round_bf16=True)
    ref_out, ref_st = gdn.gdn_fp32(q, k, v, a, b, a_log, dt_bias, s)
    torch.testing.assert_close(out.float(), ref_out, rtol=2e-2, atol=1e-2)
    torch.testing.assert_close(st, ref_st, rtol=5e-2, atol=3e-3)  # test_gdn_attn.py temporal tolerance
