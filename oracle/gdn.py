"""Oracle: Gated DeltaNet gate, q/k L2 norm and the delta-rule state update (CPU, test infrastructure only).

Restates
  * gdn_reference   models/qwen35_35b_a3b/sgl/tests/test_gdn_attn.py:259-296 — the reference's torch golden,
                    with its bf16 rounding points (normalised q/k, beta, prediction, error, output)
  * gdn_fp32        the same recurrence in fp32 without intermediate rounding: l2norm_lastdim and gdn_gate of
                    sgl_kernel_axera/attention/gdn.py:919-949, gdn_recurrent_step 952-989
  * unit_lower_inverse  inverse_unit_lower_recursive / inverse_unit_lower_blocks (gdn.py:1048-1119): (I - N)^-1
                    of strictly lower N by recursive halving, zero-padded to a power of two
  * gdn_chunk       the chunked (WY) form: gdn_stable_chunk (gdn.py:1122-1212) driven as gdn_prefill_impl does
                    (gdn.py:1628-1790: l2norm, gates, chunk_prefix_sum_fp32 992-1009, per-chunk solve), with the
                    reference's bf16 rounding points (round_bf16=True) or none (False)
Pinned by tests/test_oracle_gdn.py against transformers' torch_recurrent_gated_delta_rule and
torch_chunk_gated_delta_rule (independent fp32 implementations: Qwen3.5's modeling code, third-party,
installed), against a closed form for a single step from a zero state, against the reference golden's rounding
schedule, chunked == recurrent, and the triangular inverse against torch.linalg.solve_triangular on the
reference's correlated-matrix cases (test_gdn_attn.py:738-768).
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


def unit_lower_inverse(neg_lower):
    """(I - N)^-1 for strictly lower-triangular N [..., n, n] (fp32): pad to a power of two, then
    [[A, 0], [C, B]]^-1 = [[A^-1, 0], [B^-1 C A^-1, B^-1]] recursively; a block of size <= 2 is I + N."""
    n = neg_lower.shape[-1]
    size = 1 << max(0, (n - 1).bit_length())
    m = torch.zeros(*neg_lower.shape[:-2], size, size, dtype=torch.float32)
    m[..., :n, :n] = neg_lower.float()

    def inv(x):
        s = x.shape[-1]
        if s <= 2:
            return x + torch.eye(s, dtype=x.dtype)
        h = s // 2
        top, bottom = inv(x[..., :h, :h]), inv(x[..., h:, h:])
        out = torch.zeros_like(x)
        out[..., :h, :h] = top
        out[..., h:, h:] = bottom
        out[..., h:, :h] = bottom @ (x[..., h:, :h] @ top)
        return out

    return inv(m)[..., :n, :n]


def gdn_chunk(q, k, v, a, b, a_log, dt_bias, state_in, chunk=64, round_bf16=True):
    """Chunked gated delta rule. q, k [B, T, NK, DK]; v [B, T, NV, DV]; a, b [B, T, NV]; state [B, NV, DK, DV].
    Returns (output [B, T, NV, DV] (bf16 if round_bf16 else fp32), final state fp32).

    Per chunk (C tokens, gate prefix G = cumsum g, Gamma = exp G, decay_ij = exp(G_i - G_j) for i >= j):
      L = beta_i (k_i . k_j) decay_ij (i > j);  Tinv = (I + L)^-1
      u = Tinv (beta v);  w = Tinv (beta Gamma k);  v_new = u - w S
      o = Gamma (q S) + ((q k^T) * decay) v_new;  S <- Gamma_C S + k^T (v_new * decay_C,:)."""
    r = (lambda x: x.to(torch.bfloat16).float()) if round_bf16 else (lambda x: x.float())
    bsz, t, nk, dk = q.shape
    nv, dv = v.shape[2], v.shape[3]
    per_key = nv // nk
    qn = r(r(_l2n(q)) * dk ** -0.5).repeat_interleave(per_key, dim=2)  # gdn.py:1631-1632
    kn = r(_l2n(k)).repeat_interleave(per_key, dim=2)
    g, beta = gates(a, b, a_log, dt_bias)
    beta = r(beta)  # gdn_gate returns beta in bf16
    s = state_in.clone().float()
    out = torch.empty(bsz, t, nv, dv, dtype=torch.float32)
    for c0 in range(0, t, chunk):
        c1 = min(c0 + chunk, t)
        n = c1 - c0
        qc, kc = qn[:, c0:c1].transpose(1, 2), kn[:, c0:c1].transpose(1, 2)  # [B, NV, n, DK]
        vc = v[:, c0:c1].float().transpose(1, 2)
        bc = beta[:, c0:c1].transpose(1, 2)[..., None]  # [B, NV, n, 1]
        gp = torch.cumsum(g[:, c0:c1].transpose(1, 2), dim=-1)  # chunk_prefix_sum_fp32
        gam = torch.exp(gp)[..., None]
        lower = torch.tril(torch.ones(n, n))
        decay = torch.exp((gp[..., :, None] - gp[..., None, :]) * lower) * lower
        neg = -(kc @ kc.transpose(-1, -2) * bc * decay) * torch.tril(torch.ones(n, n), -1)
        tinv = r(unit_lower_inverse(neg))
        u = r(tinv @ r(vc * bc))
        w = r(tinv @ r(kc * bc * gam))
        sb = r(s)
        v_new = u - w @ sb
        read = r((qc @ kc.transpose(-1, -2)) * decay)
        o = (qc @ sb) * gam + read @ r(v_new)
        out[:, c0:c1] = r(o).transpose(1, 2)
        upd = r(v_new * decay[..., n - 1, :][..., None])
        s = gam[..., n - 1:n, :] * s + kc.transpose(-1, -2) @ upd
    return (out.to(torch.bfloat16) if round_bf16 else out), s
