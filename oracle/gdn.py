"""Oracle: Gated DeltaNet gate, q/k L2 norm and the delta-rule state update (CPU, test infrastructure only).

Restates
  * gdn_reference   models/qwen35_35b_a3b/sgl/tests/test_gdn_attn.py:259-296 — the reference's torch golden,
                    with its bf16 rounding points (normalised q/k, beta, prediction, error, output)
  * gdn_fp32        the same recurrence in fp32 without intermediate rounding: l2norm_lastdim and gdn_gate of
                    sgl_kernel_axera/attention/gdn.py:919-949, gdn_recurrent_step 952-989
Pinned by tests/test_oracle_gdn.py against transformers' torch_recurrent_gated_delta_rule (an independent
fp32 implementation: Qwen3.5's modeling code, third-party, installed), against a closed form for a
single step from a zero state, and against the reference golden's rounding schedule.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def gates(a, b, a_log, dt_bias):
    """g = -exp(A_log) * softplus(a + dt_bias) (log decay, fp32); beta = sigmoid(b)  (gdn.py:934-949)."""
    nv = a.shape[-1]
    g = -torch.exp(a_log.float()).reshape(*([1] * (a.dim() - 1)), nv) * F.softplus(
        a.float() + dt_bias.float().reshape(*([1] * (a.dim() - 1)), nv))
    return g, torch.sigmoid(b.float())


def _l2n(x):
    x = x.float()
    return x / torch.sqrt(x.square().sum(dim=-1, keepdim=True) + 1e-6)


def gdn_reference(q, k, v, a, b, a_log, dt_bias, state_in):
    """test_gdn_attn.py:259-296: q, k [B, T, NK, DK]; v [B, T, NV, DV]; a, b [B, T, NV];
    state [B, NV, DK, DV] fp32. Returns (bf16 output [B, T, NV, DV], fp32 final state)."""
    key_dim = q.shape[-1]
    value_heads = v.shape[2]
    per_key = value_heads // q.shape[2]
    q_norm = _l2n(q).to(torch.bfloat16)
    k_norm = _l2n(k).to(torch.bfloat16)
    q_norm = (q_norm.float() * (key_dim ** -0.5)).to(torch.bfloat16)
    g, beta = gates(a, b, a_log, dt_bias)
    beta = beta.to(torch.bfloat16)
    state = state_in.clone().float()
    output = torch.empty(v.shape, dtype=torch.bfloat16)
    for t in range(q.shape[1]):
        for h in range(value_heads):
            kh = h // per_key
            state[:, h] *= torch.exp(g[:, t, h]).reshape(-1, 1, 1)
            pred = torch.einsum("bk,bkv->bv", k_norm[:, t, kh].float(), state[:, h]).to(torch.bfloat16)
            err = ((v[:, t, h].float() - pred.float()).to(torch.bfloat16).float()
                   * beta[:, t, h].float().reshape(-1, 1)).to(torch.bfloat16)
            state[:, h] += torch.einsum("bk,bv->bkv", k_norm[:, t, kh].float(), err.float())
            output[:, t, h] = torch.einsum("bk,bkv->bv", q_norm[:, t, kh].float(), state[:, h]).to(torch.bfloat16)
    return output, state


def gdn_fp32(q, k, v, a, b, a_log, dt_bias, state_in):
    """The same recurrence without intermediate rounding; returns (fp32 output, fp32 final state)."""
    key_dim = q.shape[-1]
    per_key = v.shape[2] // q.shape[2]
    qn = _l2n(q).repeat_interleave(per_key, dim=2) * key_dim ** -0.5  # [B, T, NV, DK]
    kn = _l2n(k).repeat_interleave(per_key, dim=2)
    g, beta = gates(a, b, a_log, dt_bias)
    s = state_in.clone().double()
    out = torch.empty(v.shape, dtype=torch.float64)
    for t in range(q.shape[1]):
        s = s * torch.exp(g[:, t].double())[..., None, None]
        pred = torch.einsum("bhk,bhkv->bhv", kn[:, t].double(), s)
        err = (v[:, t].double() - pred) * beta[:, t].double()[..., None]
        s = s + kn[:, t].double()[..., :, None] * err[..., None, :]
        out[:, t] = torch.einsum("bhk,bhkv->bhv", qn[:, t].double(), s)
    return out.float(), s.float()
