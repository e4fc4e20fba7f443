"""MoE layer with MXFP4 experts on gfx950 (router top-K, shared expert, routed SwiGLU experts).

Mirrors the MoE decode of the reference: moe_full (models/qwen35_35b_a3b/src/70b0fbc/q35_layer_mc.py:797-853),
route() (q35_moe.py:293-297) and moe_experts_gu (q35_moe.py:96-113). Weights are runtime inputs named as in
the model manifest: router ``w_router`` bf16 [E, H]; shared-expert gate ``w_shg`` bf16 [H]; shared expert
``w_gate``/``s_gate``, ``w_up``/``s_up``, ``w_down``/``s_down`` (MXFP4 codes / E8M0 scales); routed experts
``e_gw``, ``e_gs``, ``e_dw``, ``e_ds`` (planar [E, ...] MXFP4).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _u8(t: Optional[torch.Tensor], name: str) -> Optional[torch.Tensor]:
    if t is None:
        return None
    if t.dtype in (torch.float4_e2m1fn_x2, torch.float8_e8m0fnu):
        t = t.view(torch.uint8)
    _check(t.dtype == torch.uint8 and t.is_contiguous(), f"{name} must be contiguous uint8")
    return t


def moe_workspace(tokens: int, hidden: int, num_experts: int, top_k: int, inter: int, shared_inter: int,
                  device) -> torch.Tensor:
    n = _lib.load().axk_moe_workspace_size(tokens, hidden, num_experts, top_k, inter, shared_inter)
    _check(n > 0, "unsupported MoE shape")
    return torch.empty(n, dtype=torch.uint8, device=device)


def moe_route(logits: torch.Tensor, top_k: int, norm_topk_prob: bool = True):
    """softmax -> top_k (ties: lower id) -> renormalised weights. Returns (ids i32 [T, K], weights f32 [T, K])."""
    _check(logits.dim() == 2 and logits.dtype == torch.float32 and logits.is_contiguous(), "logits: f32 [T, E]")
    t, e = logits.shape
    ids = torch.empty(t, top_k, dtype=torch.int32, device=logits.device)
    w = torch.empty(t, top_k, dtype=torch.float32, device=logits.device)
    _lib.require_device(logits)
    _lib.call("axk_moe_route", logits.data_ptr(), ids.data_ptr(), w.data_ptr(), t, e, top_k, int(norm_topk_prob),
              _lib.stream_of(logits))
    return ids, w


def _dims(h2, weights):
    _check(h2.dim() == 2 and h2.dtype == torch.bfloat16 and h2.is_contiguous(), "h2 must be contiguous bf16 [T, H]")
    t, hidden = h2.shape
    e_gw = _u8(weights["e_gw"], "e_gw")
    e, two_f, hh = e_gw.shape
    _check(hh * 2 == hidden and two_f % 2 == 0, f"e_gw shape {tuple(e_gw.shape)} does not match hidden {hidden}")
    inter = two_f // 2
    shared = weights.get("w_gate")
    fs = _u8(shared, "w_gate").shape[0] if shared is not None else 0
    return t, hidden, e, inter, fs


def _ptrs(weights):
    names = ("w_gate", "s_gate", "w_up", "s_up", "w_down", "s_down", "e_gw", "e_gs", "e_dw", "e_ds")
    return [_lib.ptr(_u8(weights.get(n), n)) for n in names]


def moe_experts(h2, weights, topk_ids, topk_weights, x_res=None, output=None, workspace=None):
    """Shared expert + routed experts for the given routing; returns bf16 [T, H]."""
    t, hidden, e, inter, fs = _dims(h2, weights)
    k = topk_ids.shape[1]
    if output is None:
        output = torch.empty_like(h2)
    if workspace is None:
        workspace = moe_workspace(t, hidden, e, k, inter, fs, h2.device)
    w_shg = weights.get("w_shg")
    _lib.require_device(h2, x_res, topk_ids, topk_weights, output, workspace)
    _lib.call("axk_moe_experts", h2.data_ptr(), _lib.ptr(x_res), _lib.ptr(w_shg), *_ptrs(weights),
              topk_ids.data_ptr(), topk_weights.data_ptr(), output.data_ptr(), t, hidden, e, k, inter, fs,
              workspace.data_ptr(), workspace.numel(), _lib.stream_of(h2))
    return output


def moe_decode(h2, weights, top_k: int = 8, x_res=None, norm_topk_prob: bool = True, output=None, workspace=None):
    """The MoE layer: returns (out bf16 [T, H], logits f32 [T, E], topk_ids i32 [T, K], topk_weights f32 [T, K])."""
    t, hidden, e, inter, fs = _dims(h2, weights)
    w_router = weights["w_router"]
    _check(w_router.shape == (e, hidden) and w_router.dtype == torch.bfloat16, "w_router must be bf16 [E, H]")
    if output is None:
        output = torch.empty_like(h2)
    if workspace is None:
        workspace = moe_workspace(t, hidden, e, top_k, inter, fs, h2.device)
    logits = torch.empty(t, e, dtype=torch.float32, device=h2.device)
    ids = torch.empty(t, top_k, dtype=torch.int32, device=h2.device)
    wts = torch.empty(t, top_k, dtype=torch.float32, device=h2.device)
    w_shg = weights.get("w_shg")
    _lib.require_device(h2, x_res, w_router, output, workspace)
    _lib.call("axk_moe_decode", h2.data_ptr(), _lib.ptr(x_res), w_router.data_ptr(), _lib.ptr(w_shg),
              *_ptrs(weights), output.data_ptr(), logits.data_ptr(), ids.data_ptr(), wts.data_ptr(), t, hidden, e,
              top_k, inter, fs, int(norm_topk_prob), workspace.data_ptr(), workspace.numel(), _lib.stream_of(h2))
    return output, logits, ids, wts
