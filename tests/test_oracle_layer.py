"""Pins the per-layer glue oracle (CPU only) against transformers' Qwen3.5 modules and torch's conv1d."""
import pytest
import torch
import torch.nn.functional as F

from oracle import layer


def _g(seed):
    return torch.Generator().manual_seed(seed)


def test_rmsnorm_matches_transformers_one_plus_rmsnorm():
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5RMSNorm

    g = _g(0)
    x = torch.randn(6, 256, generator=g).bfloat16()
    w_raw = (torch.randn(256, generator=g) * 0.1).bfloat16()
    m = Qwen3_5RMSNorm(256, eps=1e-6)
    m.weight.data = w_raw.float()
    ref = m(x)
    got = layer.rmsnorm(x, 1.0 + w_raw.float(), 1e-6)  # the reference passes one_plus(w) at run time
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_gated_norm_against_transformers_rmsnorm_gated():
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5RMSNormGated

    g = _g(1)
    x = torch.randn(8, 128, generator=g).bfloat16()
    z = torch.randn(8, 128, generator=g).bfloat16()
    m = Qwen3_5RMSNormGated(128, eps=1e-6)
    # unit weight: both round the normalised row to bf16 before the gate -> identical
    assert torch.equal(layer.gated_rmsnorm_silu(x, torch.ones(128), z).view(torch.int16), m(x, z).view(torch.int16))
    # a general weight: the reference multiplies before its bf16 rounding, transformers after -> one rounding apart
    w = torch.rand(128, generator=g) + 0.5
    m.weight.data = w
    torch.testing.assert_close(layer.gated_rmsnorm_silu(x, w, z).float(), m(x, z).float(), rtol=1e-2, atol=1e-2)


def _conv_fp32(x, w, state):
    """Independent formulation: torch depthwise conv1d over [state; x] (PyTorch tap order: last tap = now)."""
    b, t, c = x.shape
    k = w.shape[1]
    seq = torch.cat((state, x), 1).float().transpose(1, 2)  # [B, C, K-1+T]
    w_pt = w.float().flip(-1).reshape(c, 1, k)
    return F.silu(F.conv1d(seq, w_pt, groups=c)).transpose(1, 2)


@pytest.mark.parametrize("b,t,c,k", [(2, 1, 64, 4), (3, 7, 40, 4), (1, 5, 16, 2), (2, 3, 24, 1)])
def test_conv1d_silu_against_torch_conv1d(b, t, c, k):
    g = _g(b * 100 + t)
    x = torch.randn(b, t, c, generator=g).bfloat16()
    w = (torch.randn(c, k, generator=g) * 0.5).bfloat16()
    st = torch.randn(b, k - 1, c, generator=g).bfloat16()
    out, st_out = layer.causal_conv1d_silu(x, w, st)
    torch.testing.assert_close(out.float(), _conv_fp32(x, w, st), rtol=3e-2, atol=2e-2)
    seq = torch.cat((st, x), 1)
    assert torch.equal(st_out, seq[:, seq.shape[1] - (k - 1):])


def test_conv1d_single_tap_is_exact_and_state_carries():
    # only tap 2 nonzero: out_t = silu(bf16(x_{t-2} w)); two calls of 3 tokens == one call of 6
    g = _g(7)
    x = torch.randn(1, 6, 8, generator=g).bfloat16()
    w = torch.zeros(8, 4).bfloat16()
    w[:, 2] = 0.75
    st = torch.randn(1, 3, 8, generator=g).bfloat16()
    out, st6 = layer.causal_conv1d_silu(x, w, st)
    seq = torch.cat((st, x), 1).float()
    want = F.silu((seq[:, 1:7] * 0.75).bfloat16().float()).bfloat16()
    assert torch.equal(out, want)
    o1, s1 = layer.causal_conv1d_silu(x[:, :3], w, st)
    o2, s2 = layer.causal_conv1d_silu(x[:, 3:], w, s1)
    assert torch.equal(torch.cat((o1, o2), 1), out) and torch.equal(s2, st6)


def test_rope_matches_transformers_partial_rotary():
    from transformers.models.qwen3_5.modeling_qwen3_5 import apply_rotary_pos_emb

    g = _g(3)
    b, h, d, rot = 3, 4, 256, 64
    q = torch.randn(b, h, d, generator=g).bfloat16()
    pos = torch.tensor([0, 17, 130000])
    cos, sin = layer.rope_cos_sin(pos, rot, 10_000_000.0)
    got = layer.rope(q, cos, sin, rot)
    # transformers: cos / sin over the full rotary width (both halves), q [B, heads, seq, D]
    cf = torch.cat((cos, cos), -1).float()[:, None, :]
    sf = torch.cat((sin, sin), -1).float()[:, None, :]
    ref, _ = apply_rotary_pos_emb(q.float()[:, :, None, :], q.float()[:, :, None, :], cf, sf, unsqueeze_dim=1)
    assert torch.equal(got.view(torch.int16), ref[:, :, 0, :].bfloat16().view(torch.int16))
    # position 0 is the identity; channels past rot pass through; each rotated pair keeps its length
    assert torch.equal(got[0], q[0])
    assert torch.equal(got[..., rot:], q[..., rot:])
    half = rot // 2
    n_in = q.float()[..., :half] ** 2 + q.float()[..., half:rot] ** 2
    n_out = got.float()[..., :half] ** 2 + got.float()[..., half:rot] ** 2
    torch.testing.assert_close(n_out, n_in, rtol=2e-2, atol=2e-2)


def test_elementwise_gates_special_values():
    x = torch.tensor([[1.5, -2.0, 3.0, 0.25]]).bfloat16()
    zero = torch.zeros_like(x)
    assert torch.equal(layer.sigmoid_mul(x, zero), (x.float() * 0.5).bfloat16())  # sigmoid(0) = 1/2
    assert torch.equal(layer.silu_mul(zero, x), zero)  # silu(0) = 0
    assert torch.equal(layer.add(x, zero), x)
    s, n = layer.add_rmsnorm(x, x, torch.ones(4))
    assert torch.equal(s, (2 * x.float()).bfloat16())
    assert torch.equal(n, layer.rmsnorm(s, torch.ones(4)))
