"""Oracle: MoE layer with MXFP4 experts — router top-K, shared expert, routed SwiGLU experts, combine
(CPU, test infrastructure only).

Restates
  * route         models/qwen35_35b_a3b/src/70b0fbc/q35_moe.py:293-297 (softmax fp32 -> top-K -> / sum) with the
                  tie rule of q35_layer_mc.py:1461-1466 (stable descending sort: ties to the lower expert id)
  * shared expert q35_moe.py:123-137 (moe_pre): act = bf16(silu(bf16 g) * bf16 u), sh = act Wd^T (fp32),
                  gate = sigmoid(h2 . w_shg), base = bf16(x1 + gate * sh)
  * experts       q35_moe.py:96-113 (moe_experts_gu) and q35_layer_mc.py:830-853 (moe_full): gate-up rows
                  [gate | up] of one [2F, H] matrix, y = act Wd^T (fp32) * rw, out = bf16(base + sum_k y_k)
  * moe_parts     base, routed sum and the bound on one-ulp flips of the bf16 activations (see its docstring)
Pinned by tests/test_oracle_moe.py: against transformers' Qwen3_5MoeSparseMoeBlock (third-party, installed; the
reference's own oracle family, q35_moe.py:300-312) holding the exactly dequantised weights: router ids and
weights equal, and the layer equal at fp32 tolerance with the bf16 points switched off (oracle.rounding.fp32());
the bf16 schedule within tolerance of that; torch.topk / stable sort agreement, a dense all-experts formulation
(every token through every expert, masked by the routing) and closed-form special cases (one expert with
weight 1, zero router); the flip bound by flipping activations on purpose.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import mx
from .rounding import bf as _bf


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


def swiglu_act(h: torch.Tensor, gw, gs, split: int | None = None, uw=None, us=None) -> torch.Tensor:
    """h [n, H] bf16 -> act [n, F] (bf16 values in fp32): gate/up projections rounded to bf16,
    act = bf16(silu(g) * u)."""
    if uw is None:  # one [2F, H] gate-up matrix: gate rows first
        wgu = _deq(gw, gs)
        wg, wu = wgu[:split], wgu[split:]
    else:
        wg, wu = _deq(gw, gs), _deq(uw, us)
    g = _bf(h.float() @ wg.T).float()
    u = _bf(h.float() @ wu.T).float()
    return _bf(F.silu(g) * u).float()


def swiglu_expert(h: torch.Tensor, gw, gs, dw, ds, split: int | None = None, uw=None, us=None) -> torch.Tensor:
    """h [n, H] bf16 -> fp32 [n, H]: act Wd^T."""
    return swiglu_act(h, gw, gs, split, uw, us) @ _deq(dw, ds).T


def ulp_bf16(x: torch.Tensor) -> torch.Tensor:
    """One bf16 ulp (7 stored mantissa bits) of |x|."""
    return torch.exp2(torch.floor(torch.log2(x.abs().clamp_min(1e-30))) - 7)


def moe_parts(h2, weights, ids, wts, x_res=None, flips: int = 2, slot_bf16: bool = False):
    """(base, routed, slack), all fp32 [T, H]: base = x1 + gate * shared expert, routed = sum_k rw_k y_k, and
    a bound on how far `flips` one-ulp changes of the bf16 activations of each (token, expert) row can move the
    output. g, u and act are rounded to bf16 at the reference's points, but a value that lies within the fp32
    accumulation error of a rounding midpoint goes either way depending on the summation order, so two correct
    implementations may hold neighbouring bf16 values there; the slack charges every row `flips` times its
    largest activation ulp against the largest |Wd| of each output column.
    slot_bf16: each routed slot is bf16(rw_k y_k) before the fp32 sum, as the reference's delivered prefill slot
    kernels store it (qwen35moe_slots*_bo, SLOT_OUT=bf16: q35_moe_prefill.py:41, 100, 165; the combine's bf16 sout,
    moe_combine 196-213); the slack then also takes one ulp of each slot (its rounding, like the activations', can
    go either way between two summation orders)."""
    w = weights
    t, hidden = h2.shape
    base = x_res.float() if x_res is not None else torch.zeros(t, hidden)
    slack = torch.zeros(t, hidden)
    if w.get("w_gate") is not None:
        act = swiglu_act(h2, w["w_gate"], w["s_gate"], uw=w["w_up"], us=w["s_up"])
        wd = _deq(w["w_down"], w["s_down"])
        gate = torch.sigmoid(h2.float() @ w["w_shg"].float()) if w.get("w_shg") is not None else torch.ones(t)
        base = base + gate[:, None] * (act @ wd.T)
        slack += flips * (gate * ulp_bf16(act).amax(dim=1))[:, None] * wd.abs().amax(dim=1)[None, :]
    e_gw, e_gs, e_dw, e_ds = (np.asarray(w[n]) for n in ("e_gw", "e_gs", "e_dw", "e_ds"))
    inter = e_gw.shape[1] // 2
    routed = torch.zeros(t, hidden)
    ids_np = ids.numpy()
    for e in np.unique(ids_np):
        rows, slots = np.nonzero(ids_np == e)
        act = swiglu_act(h2[rows], e_gw[e], e_gs[e], split=inter)
        wd = _deq(e_dw[e], e_ds[e])
        rw = wts[rows, slots][:, None]
        r = torch.from_numpy(rows)
        y = (act @ wd.T) * rw
        if slot_bf16:
            y = _bf(y).float()
            slack.index_add_(0, r, ulp_bf16(y))
        routed.index_add_(0, r, y)
        slack.index_add_(0, r, flips * rw * ulp_bf16(act).amax(dim=1)[:, None] * wd.abs().amax(dim=1)[None, :])
    return base, routed, slack


def moe_layer(h2, weights, top_k=8, x_res=None, norm=True, ids=None, wts=None, round_base=True, slot_bf16=False):
    """Returns (out bf16 [T, H], logits f32 [T, E], ids i32 [T, K], weights f32 [T, K]).
    round_base: round base = x1 + gate * sh to bf16 before the expert sum, as the reference's layer kernel
    stores it (q35_layer_mc.py:845-846); False keeps it fp32 (a single final rounding). slot_bf16: as moe_parts."""
    w = weights
    logits = h2.float() @ w["w_router"].float().T
    if ids is None:
        ids, wts = route(logits, top_k, norm)
    base, routed, _ = moe_parts(h2, w, ids, wts, x_res, slot_bf16=slot_bf16)
    if round_base:
        base = _bf(base).float()
    return _bf(base + routed), logits, ids, wts


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
    return ulp_bf16(base)
