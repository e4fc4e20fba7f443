"""Oracle: MoE layer with MXFP4 experts — router top-K, shared expert, routed SwiGLU experts, combine
(CPU, test infrastructure only).

Restates
  * route         models/qwen35_35b_a3b/src/70b0fbc/q35_moe.py:293-297 (softmax fp32 -> top-K -> / sum) with the
                  tie rule of q35_layer_mc.py:1461-1466 (stable descending sort: ties to the lower expert id)
  * shared expert q35_moe.py:123-137 (moe_pre): act = bf16(silu(bf16 g) * bf16 u), sh = act Wd^T (fp32),
                  gate = sigmoid(h2 . w_shg), base = bf16(x1 + gate * sh)
  * experts       q35_moe.py:96-113 (moe_experts_gu) and q35_layer_mc.py:830-853 (moe_full): gate-up rows
                  [gate | up] of one [2F, H] matrix, y = act Wd^T (fp32) * rw, out = bf16(base + sum_k y_k)
Pinned by tests/test_oracle_moe.py: torch.topk / stable sort agreement, a dense all-experts formulation
(every token through every expert, masked by the routing) and closed-form special cases (one expert with
weight 1, zero router).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import mx


def route(logits: torch.Tensor, top_k: int, norm: bool = True):
    """Ids by a stable descending sort of the logits (ties: lower id); weights from the fp32 softmax."""
    p = torch.softmax(logits.float(), dim=-1)
    _, order = torch.sort(logits.float(), dim=-1, descending=True, stable=True)
    ids = order[:, :top_k]
    w = torch.gather(p, 1, ids)
    if norm:
        w = w / w.sum(-1, keepdim=True)
    return ids.to(torch.int32), w


def _deq(codes, scales) -> torch.Tensor:
    return torch.from_numpy(mx.dequant_mxfp4(np.asarray(codes), np.asarray(scales)))


def swiglu_expert(h: torch.Tensor, gw, gs, dw, ds, split: int | None = None, uw=None, us=None) -> torch.Tensor:
    """h [n, H] bf16 -> fp32 [n, H]: gate/up projections rounded to bf16, act = bf16(silu(g) * u), act Wd^T."""
    if uw is None:  # one [2F, H] gate-up matrix: gate rows first
        wgu = _deq(gw, gs)
        wg, wu = wgu[:split], wgu[split:]
    else:
        wg, wu = _deq(gw, gs), _deq(uw, us)
    g = (h.float() @ wg.T).to(torch.bfloat16).float()
    u = (h.float() @ wu.T).to(torch.bfloat16).float()
    act = (F.silu(g) * u).to(torch.bfloat16).float()
    return act @ _deq(dw, ds).T


def moe_layer(h2, weights, top_k=8, x_res=None, norm=True, ids=None, wts=None, round_base=True):
    """Returns (out bf16 [T, H], logits f32 [T, E], ids i32 [T, K], weights f32 [T, K]).
    round_base: round base = x1 + gate * sh to bf16 before the expert sum, as the reference's layer kernel
    stores it (q35_layer_mc.py:845-846); False keeps it fp32 (a single final rounding)."""
    w = weights
    logits = h2.float() @ w["w_router"].float().T
    if ids is None:
        ids, wts = route(logits, top_k, norm)
    t, hidden = h2.shape
    e_gw, e_gs, e_dw, e_ds = (np.asarray(w[n]) for n in ("e_gw", "e_gs", "e_dw", "e_ds"))
    inter = e_gw.shape[1] // 2
    base = x_res.float() if x_res is not None else torch.zeros(t, hidden)
    if w.get("w_gate") is not None:
        sh = swiglu_expert(h2, w["w_gate"], w["s_gate"], w["w_down"], w["s_down"], uw=w["w_up"], us=w["s_up"])
        gate = torch.sigmoid(h2.float() @ w["w_shg"].float()) if w.get("w_shg") is not None else torch.ones(t)
        base = base + gate[:, None] * sh
    if round_base:
        base = base.to(torch.bfloat16).float()
    acc = base.clone()
    ids_np = ids.numpy()
    for e in np.unique(ids_np):
        rows, slots = np.nonzero(ids_np == e)
        y = swiglu_expert(h2[rows], e_gw[e], e_gs[e], e_dw[e], e_ds[e], split=inter)
        y = y * wts[rows, slots][:, None]
        acc.index_add_(0, torch.from_numpy(rows), y)
    return acc.to(torch.bfloat16), logits, ids, wts


def base_ulp(h2, weights, x_res):
    """One bf16 ulp of |x1 + gate * sh| per element: the most the reference's intermediate rounding of base
    can move the output."""
    w = weights
    t, hidden = h2.shape
    base = x_res.float() if x_res is not None else torch.zeros(t, hidden)
    if w.get("w_gate") is not None:
        sh = swiglu_expert(h2, w["w_gate"], w["s_gate"], w["w_down"], w["s_down"], uw=w["w_up"], us=w["s_up"])
        gate = torch.sigmoid(h2.float() @ w["w_shg"].float()) if w.get("w_shg") is not None else torch.ones(t)
        base = base + gate[:, None] * sh
    e = torch.floor(torch.log2(base.abs().clamp_min(1e-30)))
    return torch.exp2(e - 7)
