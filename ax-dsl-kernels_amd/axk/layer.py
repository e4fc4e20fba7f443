"""Hybrid decode layers (one token per sequence) over libaxk.so: the GDN layer and the attention layer of
models/qwen35_35b_a3b/src/70b0fbc/q35_step.py (gdn_layer 149-183, attn_block 186-293), each with its MLP.

Weights travel in dicts keyed by the reference's names (q35_step.py gdn_args / attn_args / mlp_args 361-406, the
manifest params of tools/manifest/mkmanifest.py:23-35): each projection and MLP weight as w_<name> with its scales
s_<name>, in the format given by proj_fmt / mlp_fmt:
  "fp8"   (w u8 E4M3 [N, K], s f32 [N] per output channel)  - config 4's projections (sgl gemm.py:119-181)
  "mxfp8" (w u8 E4M3 [N, K], s u8 E8M0 [N, K/32])            - the 35B manifest (q35_mx_build.py:60-72)
  "mxfp4" (w u8 E2M1 pairs [N, K/2], s u8 E8M0 [N, K/32])    - the 9B / 27B manifests and config 4's MLP
  "nvfp4" (w u8 E2M1 pairs [N, K/2], s u8 E4M3 [N, K/16], t_<name> f32 [1] scale2) - the WFMT=nv4 projections
          (q35_mx_build.py:168-200; sgl quantize_nvfp4), passed to the C-ABI as an axk_nvfp4_scales per weight
norms f32 (ln1, ln2, q_norm, k_norm as 1 + weight; norm_w raw). The workspace is allocated once by the caller
(layer_workspace) and reused; a layer call allocates nothing.

GDN value-head order (v_order, q35_step.py:82-85): "tiled" (value head vh reads key head vh % NK; the order the
reference's layer kernels are built with by default, its exported weights permuted to it by v_tiled, 351-358) or
"grouped" (vh / (NV / NK), the checkpoint's). tile_value_heads converts a grouped weight dict to the tiled order.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib

GDN_WEIGHTS = ("ln1", "w_qkv", "s_qkv", "w_z", "s_z", "w_b", "s_b", "w_a", "s_a", "conv_w", "a_log", "dt_bias",
               "norm_w", "w_out", "s_out", "ln2")
ATTN_WEIGHTS = ("ln1", "w_q", "s_q", "w_k", "s_k", "w_v", "s_v", "q_norm", "k_norm", "w_o", "s_o", "ln2")
MLP_WEIGHTS = ("w_gate", "s_gate", "w_up", "s_up", "w_down", "s_down")
WFMT = {"fp8": 0, "mxfp8": 1, "mxfp4": 2, "nvfp4": 3}  # AXK_WFMT_FP8_CHANNEL, _MXFP8, _MXFP4, _NVFP4
_PROJ_SCALES = {"s_qkv", "s_z", "s_b", "s_a", "s_out", "s_q", "s_k", "s_v", "s_o"}
_MLP_SCALES = {"s_gate", "s_up", "s_down"}
VORDER = {"grouped": 0, "tiled": 1}  # AXK_VORDER_GROUPED, AXK_VORDER_TILED


def _vorder(name: str) -> int:
    _check(name in VORDER, f"v_order must be one of {sorted(VORDER)}, got {name!r}")
    return VORDER[name]


def v_tiled(t: torch.Tensor, dim: int, num_k_heads: int, num_v_heads: int, unit: int) -> torch.Tensor:
    """The value heads along `dim` (each `unit` entries wide) from the grouped order to the tiled one: entry
    (vo, kh) of the result is entry (kh, vo) of t (q35_step.py v_tiled 351-358)."""
    if num_v_heads == num_k_heads:
        return t
    sh = list(t.shape)
    _check(sh[dim] == num_v_heads * unit, f"dim {dim} of {sh} is not {num_v_heads} heads of {unit}")
    t = t.reshape(sh[:dim] + [num_k_heads, num_v_heads // num_k_heads, unit] + sh[dim + 1:]).transpose(dim, dim + 1)
    return t.contiguous().reshape(sh)


def tile_value_heads(w: dict, num_k_heads: int, num_v_heads: int, proj_fmt: str = "fp8") -> dict:
    """A GDN layer's weight dict in the grouped value-head order -> the tiled one (the reference's gdn_args,
    q35_step.py:361-377): the v rows of w_qkv / conv_w, the rows of w_z, w_b, w_a and their scales, a_log, dt_bias,
    and the input columns of w_out (with its MX scale columns). Other entries are passed through. States of that
    layer convert with v_tiled (the recurrent state along dim 1, unit 1; the conv state's v channels, unit 128)."""
    nk, nv = num_k_heads, num_v_heads
    kd = 2 * nk * 128
    out = dict(w)

    def rows(name, unit, start=0):
        t = w[name]
        out[name] = torch.cat((t[:start], v_tiled(t[start:], 0, nk, nv, unit))) if start else v_tiled(t, 0, nk, nv,
                                                                                                      unit)

    rows("w_qkv", 128, kd)
    rows("conv_w", 128, kd)
    rows("w_z", 128)
    rows("w_b", 1)
    rows("w_a", 1)
    rows("a_log", 1)
    rows("dt_bias", 1)
    for name, unit, start in (("s_qkv", 128, kd), ("s_z", 128, 0), ("s_b", 1, 0), ("s_a", 1, 0)):
        rows(name, unit, start)  # per-row scales: f32 [N] or E8M0 [N, K/32], rows as their weight's
    out["w_out"] = v_tiled(w["w_out"], 1, nk, nv, 64 if proj_fmt in ("mxfp4", "nvfp4") else 128)
    if proj_fmt != "fp8":  # E8M0 [H, VD / 32]: 4 scale columns per value head (NVFP4's E4M3 [H, VD / 16]: 8)
        out["s_out"] = v_tiled(w["s_out"], 1, nk, nv, 8 if proj_fmt == "nvfp4" else 4)
    return out


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


class _Nvfp4Scales:
    """An NVFP4 weight's scales as the C-ABI takes them: an axk_nvfp4_scales (host memory) naming the E4M3 block scales
    s_<name> [N, K/16] and the fp32 scale2 t_<name> [1]; it stands in the weight lists for the tensor s_<name>."""

    def __init__(self, name: str, s: torch.Tensor, t: torch.Tensor):
        _check(s.dtype in (torch.uint8, torch.float8_e4m3fn) and s.is_contiguous(),
               f"{name} must be contiguous E4M3 bytes [N, K/16]")
        _check(t.dtype == torch.float32 and t.numel() == 1 and t.device == s.device,
               f"t_{name[2:]} must be one float32 on {s.device}")
        self.s, self.t, self.device = s, t, s.device
        self.st = _lib.Nvfp4Scales(s.data_ptr(), t.data_ptr())

    def data_ptr(self) -> int:
        return ctypes.addressof(self.st)

    def is_contiguous(self) -> bool:
        return True


def _nv_weights(w: dict, proj_fmt: str, mlp_fmt: str) -> dict:
    """w with each NVFP4 weight's s_<name> replaced by its _Nvfp4Scales (s_<name> and t_<name> together)."""
    if "nvfp4" not in (proj_fmt, mlp_fmt):
        return w
    out = dict(w)
    for n in w:
        fmt = proj_fmt if n in _PROJ_SCALES else mlp_fmt if n in _MLP_SCALES else None
        if fmt == "nvfp4":
            t = w.get("t_" + n[2:])
            _check(t is not None, f"the NVFP4 weight w_{n[2:]} needs its scale2 t_{n[2:]}")
            out[n] = _Nvfp4Scales(n, w[n], t)
    return out


def _weights(w: dict, names) -> list:
    missing = [n for n in names if n not in w]
    _check(not missing, f"missing weights: {missing}")
    for n in names:
        _check(w[n].is_contiguous(), f"{n} must be contiguous")
    return [w[n] for n in names]


MOE_WEIGHTS = ("w_router", "e_gw", "e_gs", "e_dw", "e_ds")


def moe_block(moe: dict, rows: Optional[int] = None) -> _lib.MoeBlock:
    """The axk_moe_block of a MoE block (moe_full, q35_layer_mc.py:797-853) given as a dict: w_router bf16 [E, H],
    w_shg bf16 [H] (optional: the shared expert's sigmoid gate), the routed experts e_gw / e_gs [E, 2 F, H/2 | H/32]
    and e_dw / e_ds [E, H, F/2 | F/32] (MXFP4, the manifest's planar layout), top_k, norm_topk_prob (default True),
    and optional routing outputs logits f32 [B, E], topk_ids int32 [B, K], topk_weights f32 [B, K] (B = rows when
    given: the layer's token rows). The shared expert is the layer's MLP weights (w_gate .. s_down) in mlp_fmt."""
    _weights(moe, MOE_WEIGHTS)
    shg = moe.get("w_shg")
    _check(shg is None or shg.is_contiguous(), "w_shg must be contiguous")
    e, two_f = moe["e_gw"].shape[0], moe["e_gw"].shape[1]
    _check("top_k" in moe, "the MoE block needs top_k")
    m = _lib.MoeBlock()
    m.w_router, m.e_gw, m.e_gs, m.e_dw, m.e_ds = (moe[n].data_ptr() for n in MOE_WEIGHTS)
    m.w_shg = _lib.ptr(shg)
    m.num_experts, m.top_k, m.expert_inter = e, int(moe["top_k"]), two_f // 2
    m.norm_topk_prob = 1 if moe.get("norm_topk_prob", True) else 0
    for n, dt, cols in (("logits", torch.float32, e), ("topk_ids", torch.int32, m.top_k),
                        ("topk_weights", torch.float32, m.top_k)):
        t = moe.get(n)
        _check(t is None or (t.dtype == dt and t.dim() == 2 and t.shape[1] == cols and t.is_contiguous() and
                             (rows is None or t.shape[0] == rows)),
               f"{n} must be contiguous {dt} [{'B' if rows is None else rows}, {cols}]")
        setattr(m, n, _lib.ptr(t))
    return m


def _moe_tensors(moe: Optional[dict]) -> list:
    """The MoE block's tensors (for the device check)."""
    if moe is None:
        return []
    return [moe[n] for n in MOE_WEIGHTS] + [moe[n] for n in ("w_shg", "logits", "topk_ids", "topk_weights")
                                            if moe.get(n) is not None]


def gdn_workspace(batch: int, hidden: int, num_k_heads: int, num_v_heads: int, inter: int,
                  device, head_dim: int = 128, moe: Optional[dict] = None) -> torch.Tensor:
    """The workspace of gdn_layer_decode (with moe: of its MoE form)."""
    lib = _lib.load()
    if moe is None:
        n = lib.axk_gdn_layer_workspace_size(batch, hidden, num_k_heads, num_v_heads, head_dim, inter)
    else:
        m = moe_block(moe)
        n = lib.axk_gdn_layer_moe_workspace_size(batch, hidden, num_k_heads, num_v_heads, head_dim, inter,
                                                 ctypes.addressof(m))
    _check(n > 0, "unsupported GDN layer shape")
    return torch.empty(n, dtype=torch.uint8, device=device)


def attn_workspace(batch: int, hidden: int, num_qo_heads: int, num_kv_heads: int, head_dim: int, inter: int,
                   device, moe: Optional[dict] = None) -> torch.Tensor:
    """The workspace of attn_layer_decode (with moe: of its MoE form)."""
    lib = _lib.load()
    if moe is None:
        n = lib.axk_attn_layer_workspace_size(batch, hidden, num_qo_heads, num_kv_heads, head_dim, inter)
    else:
        m = moe_block(moe)
        n = lib.axk_attn_layer_moe_workspace_size(batch, hidden, num_qo_heads, num_kv_heads, head_dim, inter,
                                                  ctypes.addressof(m))
    _check(n > 0, "unsupported attention layer shape")
    return torch.empty(n, dtype=torch.uint8, device=device)


def _fmt(name: str) -> int:
    _check(name in WFMT, f"weight format must be one of {sorted(WFMT)}, got {name!r}")
    return WFMT[name]


def gdn_layer_decode(x: torch.Tensor, w: dict, state_in: torch.Tensor, conv_in: torch.Tensor,
                     num_k_heads: int, num_v_heads: int, eps: float = 1e-6, workspace: Optional[torch.Tensor] = None,
                     out: Optional[torch.Tensor] = None, state_out: Optional[torch.Tensor] = None,
                     conv_out: Optional[torch.Tensor] = None, proj_fmt: str = "fp8", mlp_fmt: str = "mxfp4",
                     moe: Optional[dict] = None, v_order: str = "tiled"):
    """x bf16 [B, hidden]; state f32 [B, NV, 128, 128]; conv state bf16 [B, K-1, 2 KD + VD].
    Returns (out, state_out, conv_out); state_out / conv_out may be the inputs (in place).
    moe (optional, see moe_block): the MLP is the MoE block, whose shared expert is the MLP weights
    (gdn_layer_full_mx, q35_layer_mc.py:855-866)."""
    _check(x.dtype == torch.bfloat16 and x.dim() == 2 and x.is_contiguous(), "x must be contiguous bf16 [B, H]")
    w = _nv_weights(w, proj_fmt, mlp_fmt)
    b, h = x.shape
    inter = w["w_gate"].shape[0]
    kconv = w["conv_w"].shape[1]
    ws = workspace if workspace is not None else gdn_workspace(b, h, num_k_heads, num_v_heads, inter, x.device,
                                                               moe=moe)
    o = torch.empty_like(x) if out is None else out
    so = torch.empty_like(state_in) if state_out is None else state_out
    co = torch.empty_like(conv_in) if conv_out is None else conv_out
    args = _weights(w, GDN_WEIGHTS) + _weights(w, MLP_WEIGHTS)
    extra = _moe_tensors(moe)
    _lib.require_device(x, ws, o, so, co, state_in, conv_in, *args, *extra)
    ptrs = [t.data_ptr() for t in args]
    tail = (state_in.data_ptr(), conv_in.data_ptr(), o.data_ptr(), so.data_ptr(), co.data_ptr(), b, h, num_k_heads,
            num_v_heads, 128, kconv, inter, eps, _fmt(proj_fmt), _fmt(mlp_fmt), _vorder(v_order), ws.data_ptr(),
            ws.numel(), _lib.stream_of(x))
    # the C order: x, ln1 .. s_out, ln2, MLP, [moe], state_in, conv_in, out, state_out, conv_out
    if moe is None:
        _lib.call("axk_gdn_layer_decode", x.data_ptr(), *ptrs, *tail)
    else:
        m = moe_block(moe, b)
        _lib.call("axk_gdn_layer_decode_moe", x.data_ptr(), *ptrs, ctypes.addressof(m), *tail)
    return o, so, co


def attn_layer_decode(x: torch.Tensor, w: dict, cos: torch.Tensor, sin: torch.Tensor, kv_cache: torch.Tensor,
                      indptr: torch.Tensor, indices: torch.Tensor, last_page_len: torch.Tensor,
                      cache_location: torch.Tensor, num_qo_heads: int, rot: int, eps: float = 1e-6,
                      sm_scale: Optional[float] = None, workspace: Optional[torch.Tensor] = None,
                      out: Optional[torch.Tensor] = None, proj_fmt: str = "fp8", mlp_fmt: str = "mxfp4",
                      moe: Optional[dict] = None) -> torch.Tensor:
    """x bf16 [B, hidden]; kv_cache bf16 [P, 2, page, HKV, D] written in place at cache_location (int32 [B, 2]);
    the page table describes each sequence including the new token; cos, sin bf16 [B, rot/2].
    moe (optional, see moe_block): the MLP is the MoE block (attn_layer_full_mx, q35_layer_mc.py:867-880)."""
    _check(x.dtype == torch.bfloat16 and x.dim() == 2 and x.is_contiguous(), "x must be contiguous bf16 [B, H]")
    w = _nv_weights(w, proj_fmt, mlp_fmt)
    b, h = x.shape
    pages, two, page, hkv, d = kv_cache.shape
    inter = w["w_gate"].shape[0]
    ws = workspace if workspace is not None else attn_workspace(b, h, num_qo_heads, hkv, d, inter, x.device, moe=moe)
    o = torch.empty_like(x) if out is None else out
    scale = d ** -0.5 if sm_scale is None else sm_scale
    wa = _weights(w, ATTN_WEIGHTS)
    mlp = _weights(w, MLP_WEIGHTS)
    extra = _moe_tensors(moe)
    _lib.require_device(x, ws, o, kv_cache, indptr, indices, last_page_len, cache_location, cos, sin, *wa, *mlp,
                        *extra)
    (ln1, w_q, s_q, w_k, s_k, w_v, s_v, q_norm, k_norm, w_o, s_o, ln2) = wa
    head = (x.data_ptr(), ln1.data_ptr(), w_q.data_ptr(), s_q.data_ptr(), w_k.data_ptr(), s_k.data_ptr(),
            w_v.data_ptr(), s_v.data_ptr(), q_norm.data_ptr(), k_norm.data_ptr(), _lib.ptr(cos), _lib.ptr(sin),
            kv_cache.data_ptr(), indptr.data_ptr(), indices.data_ptr(), last_page_len.data_ptr(),
            cache_location.data_ptr(), w_o.data_ptr(), s_o.data_ptr(), ln2.data_ptr(), *[t.data_ptr() for t in mlp])
    tail = (o.data_ptr(), b, h, num_qo_heads, hkv, d, rot, page, pages, inter, eps, scale, _fmt(proj_fmt),
            _fmt(mlp_fmt), ws.data_ptr(), ws.numel(), _lib.stream_of(x))
    if moe is None:
        _lib.call("axk_attn_layer_decode", *head, *tail)
    else:
        m = moe_block(moe, b)
        _lib.call("axk_attn_layer_decode_moe", *head, ctypes.addressof(m), *tail)
    return o


# ---- speculative verification: T consecutive rows per sequence through one layer call (models/qwen38_27b/verify/
# verify_group_m4.py:1-9; the decode.verify role of models/qwen38_27b/README.md:11) ----
def gdn_verify_workspace(batch: int, tokens: int, hidden: int, num_k_heads: int, num_v_heads: int, inter: int,
                         device, head_dim: int = 128) -> torch.Tensor:
    n = _lib.load().axk_gdn_layer_verify_workspace_size(batch, tokens, hidden, num_k_heads, num_v_heads, head_dim,
                                                        inter)
    _check(n > 0, "unsupported GDN verify shape")
    return torch.empty(n, dtype=torch.uint8, device=device)


def attn_verify_workspace(batch: int, tokens: int, hidden: int, num_qo_heads: int, num_kv_heads: int,
                          head_dim: int, inter: int, device) -> torch.Tensor:
    n = _lib.load().axk_attn_layer_verify_workspace_size(batch, tokens, hidden, num_qo_heads, num_kv_heads, head_dim,
                                                         inter)
    _check(n > 0, "unsupported attention verify shape")
    return torch.empty(n, dtype=torch.uint8, device=device)


def gdn_layer_verify(x: torch.Tensor, w: dict, state_in: torch.Tensor, conv_in: torch.Tensor, num_k_heads: int,
                     num_v_heads: int, eps: float = 1e-6, workspace: Optional[torch.Tensor] = None,
                     out: Optional[torch.Tensor] = None, state_out: Optional[torch.Tensor] = None,
                     conv_out: Optional[torch.Tensor] = None, state_snap: Optional[torch.Tensor] = None,
                     conv_snap: Optional[torch.Tensor] = None, proj_fmt: str = "fp8", mlp_fmt: str = "mxfp4",
                     v_order: str = "tiled"):
    """x bf16 [B, T, hidden]: T new rows per sequence. state f32 [B, NV, 128, 128]; conv state bf16
    [B, K-1, 2 KD + VD]. Returns (out [B, T, hidden], state_out, conv_out) after the last row; the optional
    snapshots state_snap f32 [T, B, NV, 128, 128] and conv_snap bf16 [T, B, K-1, C] receive the states after
    each row."""
    _check(x.dtype == torch.bfloat16 and x.dim() == 3 and x.is_contiguous(), "x must be contiguous bf16 [B, T, H]")
    w = _nv_weights(w, proj_fmt, mlp_fmt)
    b, t, h = x.shape
    inter = w["w_gate"].shape[0]
    kconv = w["conv_w"].shape[1]
    ws = workspace if workspace is not None else gdn_verify_workspace(b, t, h, num_k_heads, num_v_heads, inter,
                                                                      x.device)
    o = torch.empty_like(x) if out is None else out
    so = torch.empty_like(state_in) if state_out is None else state_out
    co = torch.empty_like(conv_in) if conv_out is None else conv_out
    for name, snap, shape, dt in (("state_snap", state_snap, (t,) + tuple(state_in.shape), torch.float32),
                                  ("conv_snap", conv_snap, (t,) + tuple(conv_in.shape), torch.bfloat16)):
        _check(snap is None or (snap.shape == shape and snap.dtype == dt and snap.is_contiguous()),
               f"{name} must be contiguous {dt} {list(shape)}")
    args = _weights(w, GDN_WEIGHTS) + _weights(w, MLP_WEIGHTS)
    _lib.require_device(x, ws, o, so, co, state_in, conv_in, state_snap, conv_snap, *args)
    ptrs = [t_.data_ptr() for t_ in args]
    _lib.call("axk_gdn_layer_verify", x.data_ptr(), *ptrs, state_in.data_ptr(), conv_in.data_ptr(), o.data_ptr(),
              so.data_ptr(), co.data_ptr(), _lib.ptr(state_snap), _lib.ptr(conv_snap), b, t, h, num_k_heads,
              num_v_heads, 128, kconv, inter, eps, _fmt(proj_fmt), _fmt(mlp_fmt), _vorder(v_order), ws.data_ptr(),
              ws.numel(), _lib.stream_of(x))
    return o, so, co


def attn_layer_verify(x: torch.Tensor, w: dict, cos: torch.Tensor, sin: torch.Tensor, kv_cache: torch.Tensor,
                      indptr: torch.Tensor, indices: torch.Tensor, last_page_len: torch.Tensor,
                      cache_location: torch.Tensor, num_qo_heads: int, rot: int, eps: float = 1e-6,
                      sm_scale: Optional[float] = None, workspace: Optional[torch.Tensor] = None,
                      out: Optional[torch.Tensor] = None, proj_fmt: str = "fp8", mlp_fmt: str = "mxfp4") -> torch.Tensor:
    """x bf16 [B, T, hidden]; the page table covers each sequence's history and its T new rows; cache_location int32
    [B, T, 2] (page, slot) of each new row; cos, sin bf16 [B, T, rot / 2]. kv_cache bf16 [P, 2, page, HKV, D] is
    written in place. Returns out bf16 [B, T, hidden]."""
    _check(x.dtype == torch.bfloat16 and x.dim() == 3 and x.is_contiguous(), "x must be contiguous bf16 [B, T, H]")
    w = _nv_weights(w, proj_fmt, mlp_fmt)
    b, t, h = x.shape
    pages, two, page, hkv, d = kv_cache.shape
    inter = w["w_gate"].shape[0]
    _check(cache_location.dtype == torch.int32 and cache_location.numel() == 2 * b * t and
           cache_location.is_contiguous(), "cache_location must be contiguous int32 [B, T, 2]")
    ws = workspace if workspace is not None else attn_verify_workspace(b, t, h, num_qo_heads, hkv, d, inter, x.device)
    o = torch.empty_like(x) if out is None else out
    scale = d ** -0.5 if sm_scale is None else sm_scale
    wa = _weights(w, ATTN_WEIGHTS)
    mlp = _weights(w, MLP_WEIGHTS)
    _lib.require_device(x, ws, o, kv_cache, indptr, indices, last_page_len, cache_location, cos, sin, *wa, *mlp)
    (ln1, w_q, s_q, w_k, s_k, w_v, s_v, q_norm, k_norm, w_o, s_o, ln2) = wa
    _lib.call("axk_attn_layer_verify", x.data_ptr(), ln1.data_ptr(), w_q.data_ptr(), s_q.data_ptr(), w_k.data_ptr(),
              s_k.data_ptr(), w_v.data_ptr(), s_v.data_ptr(), q_norm.data_ptr(), k_norm.data_ptr(),
              _lib.ptr(cos), _lib.ptr(sin), kv_cache.data_ptr(), indptr.data_ptr(), indices.data_ptr(),
              last_page_len.data_ptr(), cache_location.data_ptr(), w_o.data_ptr(), s_o.data_ptr(), ln2.data_ptr(),
              *[t_.data_ptr() for t_ in mlp], o.data_ptr(), b, t, h, num_qo_heads, hkv, d, rot, page, pages, inter,
              eps, scale, _fmt(proj_fmt), _fmt(mlp_fmt), ws.data_ptr(), ws.numel(), _lib.stream_of(x))
    return o


# ---- prefill: T new tokens per sequence through one layer call (models/qwen35_35b_a3b/src/70b0fbc/q35_prefill.py:
# gdn_layer_prefill 57-141, attn_layer_prefill 172-336) ----
def gdn_prefill_workspace(batch: int, tokens: int, hidden: int, num_k_heads: int, num_v_heads: int, inter: int,
                          device, head_dim: int = 128, moe: Optional[dict] = None) -> torch.Tensor:
    """The workspace of gdn_layer_prefill (with moe: of its MoE form)."""
    lib = _lib.load()
    if moe is None:
        n = lib.axk_gdn_layer_prefill_workspace_size(batch, tokens, hidden, num_k_heads, num_v_heads, head_dim, inter)
    else:
        m = moe_block(moe)
        n = lib.axk_gdn_layer_prefill_moe_workspace_size(batch, tokens, hidden, num_k_heads, num_v_heads, head_dim,
                                                         inter, ctypes.addressof(m))
    _check(n > 0, "unsupported GDN prefill shape")
    return torch.empty(n, dtype=torch.uint8, device=device)


def attn_prefill_workspace(batch: int, tokens: int, hidden: int, num_qo_heads: int, num_kv_heads: int,
                           head_dim: int, inter: int, device, moe: Optional[dict] = None) -> torch.Tensor:
    """The workspace of attn_layer_prefill (with moe: of its MoE form)."""
    lib = _lib.load()
    if moe is None:
        n = lib.axk_attn_layer_prefill_workspace_size(batch, tokens, hidden, num_qo_heads, num_kv_heads, head_dim,
                                                      inter)
    else:
        m = moe_block(moe)
        n = lib.axk_attn_layer_prefill_moe_workspace_size(batch, tokens, hidden, num_qo_heads, num_kv_heads,
                                                          head_dim, inter, ctypes.addressof(m))
    _check(n > 0, "unsupported attention prefill shape")
    return torch.empty(n, dtype=torch.uint8, device=device)


def gdn_layer_prefill(x: torch.Tensor, w: dict, state_in: torch.Tensor, conv_in: torch.Tensor, num_k_heads: int,
                      num_v_heads: int, eps: float = 1e-6, workspace: Optional[torch.Tensor] = None,
                      out: Optional[torch.Tensor] = None, state_out: Optional[torch.Tensor] = None,
                      conv_out: Optional[torch.Tensor] = None, proj_fmt: str = "fp8", mlp_fmt: str = "mxfp4",
                      v_order: str = "tiled", moe: Optional[dict] = None):
    """x bf16 [B, T, hidden]: T new tokens per sequence. state f32 [B, NV, 128, 128]; conv state bf16
    [B, K-1, 2 KD + VD]. Returns (out [B, T, hidden], state_out, conv_out) after the last token. moe (optional, see
    moe_block; routing outputs [B T, ...]): the MLP is the MoE block (qwen35moe_gdn_prefill,
    q35_moe_prefill.py:47-52)."""
    _check(x.dtype == torch.bfloat16 and x.dim() == 3 and x.is_contiguous(), "x must be contiguous bf16 [B, T, H]")
    w = _nv_weights(w, proj_fmt, mlp_fmt)
    b, t, h = x.shape
    inter = w["w_gate"].shape[0]
    kconv = w["conv_w"].shape[1]
    ws = workspace if workspace is not None else gdn_prefill_workspace(b, t, h, num_k_heads, num_v_heads, inter,
                                                                       x.device, moe=moe)
    o = torch.empty_like(x) if out is None else out
    so = torch.empty_like(state_in) if state_out is None else state_out
    co = torch.empty_like(conv_in) if conv_out is None else conv_out
    args = _weights(w, GDN_WEIGHTS) + _weights(w, MLP_WEIGHTS)
    _lib.require_device(x, ws, o, so, co, state_in, conv_in, *args, *_moe_tensors(moe))
    ptrs = [t_.data_ptr() for t_ in args]
    tail = (state_in.data_ptr(), conv_in.data_ptr(), o.data_ptr(), so.data_ptr(), co.data_ptr(), b, t, h,
            num_k_heads, num_v_heads, 128, kconv, inter, eps, _fmt(proj_fmt), _fmt(mlp_fmt), _vorder(v_order),
            ws.data_ptr(), ws.numel(), _lib.stream_of(x))
    if moe is None:
        _lib.call("axk_gdn_layer_prefill", x.data_ptr(), *ptrs, *tail)
    else:
        m = moe_block(moe, b * t)
        _lib.call("axk_gdn_layer_prefill_moe", x.data_ptr(), *ptrs, ctypes.addressof(m), *tail)
    return o, so, co


def attn_layer_prefill(x: torch.Tensor, w: dict, cos: torch.Tensor, sin: torch.Tensor, kv_cache: torch.Tensor,
                       indptr: torch.Tensor, indices: torch.Tensor, last_page_len: torch.Tensor,
                       cache_location: torch.Tensor, num_qo_heads: int, rot: int, eps: float = 1e-6,
                       sm_scale: Optional[float] = None, workspace: Optional[torch.Tensor] = None,
                       out: Optional[torch.Tensor] = None, proj_fmt: str = "fp8", mlp_fmt: str = "mxfp4",
                       moe: Optional[dict] = None) -> torch.Tensor:
    """x bf16 [B, T, hidden]; the page table covers each sequence's history and its T new tokens; cache_location
    int32 [B, T, 2] (page, slot) of each new token; cos, sin bf16 [B, T, rot / 2]. kv_cache bf16
    [P, 2, page, HKV, D] is written in place. Returns out bf16 [B, T, hidden]. moe (optional): the MLP is the MoE
    block (qwen35moe_attn_prefill, q35_moe_prefill.py:55-60)."""
    _check(x.dtype == torch.bfloat16 and x.dim() == 3 and x.is_contiguous(), "x must be contiguous bf16 [B, T, H]")
    w = _nv_weights(w, proj_fmt, mlp_fmt)
    b, t, h = x.shape
    pages, two, page, hkv, d = kv_cache.shape
    inter = w["w_gate"].shape[0]
    _check(cache_location.dtype == torch.int32 and cache_location.numel() == 2 * b * t and
           cache_location.is_contiguous(), "cache_location must be contiguous int32 [B, T, 2]")
    ws = workspace if workspace is not None else attn_prefill_workspace(b, t, h, num_qo_heads, hkv, d, inter,
                                                                        x.device, moe=moe)
    o = torch.empty_like(x) if out is None else out
    scale = d ** -0.5 if sm_scale is None else sm_scale
    wa = _weights(w, ATTN_WEIGHTS)
    mlp = _weights(w, MLP_WEIGHTS)
    _lib.require_device(x, ws, o, kv_cache, indptr, indices, last_page_len, cache_location, cos, sin, *wa, *mlp,
                        *_moe_tensors(moe))
    (ln1, w_q, s_q, w_k, s_k, w_v, s_v, q_norm, k_norm, w_o, s_o, ln2) = wa
    head = (x.data_ptr(), ln1.data_ptr(), w_q.data_ptr(), s_q.data_ptr(), w_k.data_ptr(), s_k.data_ptr(),
            w_v.data_ptr(), s_v.data_ptr(), q_norm.data_ptr(), k_norm.data_ptr(), _lib.ptr(cos), _lib.ptr(sin),
            kv_cache.data_ptr(), indptr.data_ptr(), indices.data_ptr(), last_page_len.data_ptr(),
            cache_location.data_ptr(), w_o.data_ptr(), s_o.data_ptr(), ln2.data_ptr(), *[t_.data_ptr() for t_ in mlp])
    tail = (o.data_ptr(), b, t, h, num_qo_heads, hkv, d, rot, page, pages, inter, eps, scale, _fmt(proj_fmt),
            _fmt(mlp_fmt), ws.data_ptr(), ws.numel(), _lib.stream_of(x))
    if moe is None:
        _lib.call("axk_attn_layer_prefill", *head, *tail)
    else:
        m = moe_block(moe, b * t)
        _lib.call("axk_attn_layer_prefill_moe", *head, ctypes.addressof(m), *tail)
    return o
