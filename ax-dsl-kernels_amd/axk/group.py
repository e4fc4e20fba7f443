"""A decode group: G consecutive decode layers run as one step, captured once as a HIP graph and replayed per token.

Layer j's output is layer j+1's input; GDN recurrent / conv states and the attention layers' paged KV caches advance
in place. Each layer runs through its own decode entry (layer.gdn_layer_decode / layer.attn_layer_decode, the MoE
form where the layer carries a MoE block), so the group computes exactly what the layers compute one by one; the
graph takes the host out of the step (one replay per token instead of about 15 launches per layer).

The role of the reference's group kernels, one call per group of G layers instead of G:
  * models/qwen35_35b_a3b/src/70b0fbc/q35_moe_group.py:90-123 (the 35B's MoE group: every layer's MLP the MoE block,
    the layer kinds g / a per the model's layer list, 47), checked against the whole-layer kernels called one after
    another (168-183);
  * models/qwen38_27b/decode/q35_group.py:413-437 (the dense group of config 4).
The attention layers of a group share the step's rope rows and page table (cos / sin / pos / nblk / mask of
q35_moe_group.py:97-99, 155-156: the same token positions in every attention layer of the step).
A group that ends the model also carries the LM head (LMHEAD=1 of models/qwen38_27b/decode/q35_group.py:55-57,
442-452): the final RMSNorm of the last layer's output and the output projection into fp32 logits, inside the step.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import gemm, glue, layer

_ATTN_KEYS = ("cos", "sin", "indptr", "indices", "last_page_len", "loc")


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


class DecodeGroup:
    """layers: list of dicts, in order, each {"kind": "g" | "a", "w": the layer's weights (layer.py names),
    "moe": the MoE block (layer.moe_block's dict) or absent for a dense MLP} plus, for "g", "state" f32
    [B, NV, 128, 128] and "conv" bf16 [B, K-1, 2 KD + VD] and, for "a", "cache" bf16 [P, 2, page, HKV, D] (all
    updated in place by every step). attn: the page table of the step shared by the attention layers, {"cos", "sin"
    bf16 [B, rot/2], "indptr", "indices", "last_page_len" int32, "loc" int32 [B, 2]} (layer.attn_layer_decode's
    arguments). routing=True gives every MoE layer its routing outputs (logits, topk_ids, topk_weights) in
    self.routing[j]. lm_head (optional): {"norm": f32 [H] (the final norm's 1 + weight), "w", "s": the output
    projection [V, H] in "fmt" ("mxfp4": E2M1 pairs [V, H/2] with E8M0 scales [V, H/32]; "mxfp8": E4M3 bytes
    [V, H] with E8M0 scales [V, H/32]; "nvfp4": E2M1 pairs [V, H/2] with E4M3 scales [V, H/16] and "s2", the fp32
    scale2 [1] on the device)};
    every step then also writes self.logits f32 [B, V] = rmsnorm(out, norm) W^T (self.hn holds the normalised rows).

    Workspaces are allocated here, once per layer kind, and shared by the layers of that kind (the layers run one
    after another on one stream); a step allocates nothing. step() runs the layers eagerly; capture() records one
    step as a HIP graph reading self.x; replay(x) copies x into self.x (when given) and replays. Both return
    self.out, which the next step overwrites."""

    def __init__(self, layers: list, batch: int, hidden: int, device, num_k_heads: int = 16, num_v_heads: int = 32,
                 num_qo_heads: int = 0, rot: int = 0, eps: float = 1e-6, proj_fmt: str = "fp8",
                 mlp_fmt: str = "mxfp4", attn: Optional[dict] = None, routing: bool = False,
                 lm_head: Optional[dict] = None):
        _check(len(layers) > 0, "a decode group needs at least one layer")
        self.layers, self.b, self.h = layers, batch, hidden
        self.nk, self.nv, self.hq, self.rot, self.eps = num_k_heads, num_v_heads, num_qo_heads, rot, eps
        self.proj_fmt, self.mlp_fmt = proj_fmt, mlp_fmt
        kinds = {L["kind"] for L in layers}
        _check(kinds <= {"g", "a"}, f"layer kinds must be 'g' or 'a', got {sorted(kinds)}")
        if "a" in kinds:
            _check(attn is not None and all(k in attn for k in _ATTN_KEYS),
                   f"attention layers need the step's page table ({', '.join(_ATTN_KEYS)})")
            _check(num_qo_heads > 0 and rot > 0, "attention layers need num_qo_heads and rot")
        self.attn = attn
        self.ws = {}
        for kind in sorted(kinds):
            group = [L for L in layers if L["kind"] == kind]
            first = group[0]
            for L in group[1:]:  # one workspace per kind: the layers of a kind share its shape
                _check(L["w"]["w_gate"].shape == first["w"]["w_gate"].shape and
                       (L.get("moe") is None) == (first.get("moe") is None) and
                       (L.get("moe") is None or (L["moe"]["e_gw"].shape == first["moe"]["e_gw"].shape and
                                                 L["moe"]["top_k"] == first["moe"]["top_k"])),
                       "the layers of one kind must share their MLP / MoE shapes")
            inter = first["w"]["w_gate"].shape[0]
            if kind == "g":
                self.ws[kind] = layer.gdn_workspace(batch, hidden, num_k_heads, num_v_heads, inter, device,
                                                    moe=first.get("moe"))
            else:
                _, _, _, hkv, d = first["cache"].shape
                self.ws[kind] = layer.attn_workspace(batch, hidden, num_qo_heads, hkv, d, inter, device,
                                                     moe=first.get("moe"))
        self.routing = []
        self._moe = []
        for L in layers:
            m = L.get("moe")
            r = None
            if m is not None and routing:
                e, k = m["w_router"].shape[0], int(m["top_k"])
                r = dict(logits=torch.empty(batch, e, device=device),
                         topk_ids=torch.empty(batch, k, dtype=torch.int32, device=device),
                         topk_weights=torch.empty(batch, k, device=device))
                m = dict(m, **r)
            self.routing.append(r)
            self._moe.append(m)
        self.x = torch.zeros(batch, hidden, dtype=torch.bfloat16, device=device)
        self.out = torch.empty_like(self.x)
        self._bufs = [torch.empty_like(self.x), torch.empty_like(self.x)]
        self.inputs = None  # set by step(record=True): each layer's input, cloned
        self.lm_head, self.hn, self.logits = None, None, None
        if lm_head is not None:
            fmt = lm_head.get("fmt", "mxfp4")
            _check(fmt in ("mxfp4", "mxfp8", "nvfp4"), f"the LM head's fmt must be mxfp4, mxfp8 or nvfp4, got {fmt!r}")
            nw, w, sc = lm_head["norm"], lm_head["w"], lm_head["s"]
            _check(nw.dtype == torch.float32 and nw.numel() == hidden, f"the LM head's norm must be float32 [{hidden}]")
            kw = hidden if fmt == "mxfp8" else hidden // 2
            ks = hidden // (16 if fmt == "nvfp4" else 32)
            _check(w.dim() == 2 and w.shape[1] == kw and tuple(sc.shape) == (w.shape[0], ks),
                   f"the LM head's w / s must be [V, {kw}] / [V, {ks}]")
            _check(fmt != "nvfp4" or lm_head.get("s2") is not None, "an NVFP4 LM head needs its scale2 s2")
            self.lm_head = dict(norm=nw, w=w, s=sc, fmt=fmt, s2=lm_head.get("s2"))
            self.hn = torch.empty_like(self.x)
            self.logits = torch.empty(batch, w.shape[0], dtype=torch.float32, device=device)
        self.graph = None
        self._stream = None

    def _layer(self, j: int, x: torch.Tensor, y: torch.Tensor) -> None:
        L = self.layers[j]
        if L["kind"] == "g":
            layer.gdn_layer_decode(x, L["w"], L["state"], L["conv"], self.nk, self.nv, self.eps,
                                   workspace=self.ws["g"], out=y, state_out=L["state"], conv_out=L["conv"],
                                   proj_fmt=self.proj_fmt, mlp_fmt=self.mlp_fmt, moe=self._moe[j])
        else:
            a = self.attn
            layer.attn_layer_decode(x, L["w"], a["cos"], a["sin"], L["cache"], a["indptr"], a["indices"],
                                    a["last_page_len"], a["loc"], self.hq, self.rot, self.eps,
                                    workspace=self.ws["a"], out=y, proj_fmt=self.proj_fmt, mlp_fmt=self.mlp_fmt,
                                    moe=self._moe[j])

    def step(self, x: Optional[torch.Tensor] = None, record: bool = False) -> torch.Tensor:
        """One token per sequence through every layer (x bf16 [B, H], default self.x). record=True keeps a clone of
        each layer's input in self.inputs (eager use only)."""
        src = self.x if x is None else x
        _check(src.dtype == torch.bfloat16 and tuple(src.shape) == (self.b, self.h) and src.is_contiguous(),
               f"x must be contiguous bf16 [{self.b}, {self.h}]")
        if record:
            self.inputs = []
        n = len(self.layers)
        for j in range(n):
            dst = self.out if j == n - 1 else self._bufs[j % 2]
            if record:
                self.inputs.append(src.clone())
            self._layer(j, src, dst)
            src = dst
        if self.lm_head is not None:
            lm = self.lm_head
            glue.rmsnorm(self.out, lm["norm"], self.eps, out=self.hn)
            if lm["fmt"] == "mxfp4":
                gemm.mxfp4_gemm(self.hn, lm["w"], lm["s"], out_dtype=torch.float32, output=self.logits)
            elif lm["fmt"] == "nvfp4":
                gemm.nvfp4_gemm(self.hn, lm["w"], lm["s"], lm["s2"], out_dtype=torch.float32, output=self.logits)
            else:
                gemm.mxfp8_gemm(self.hn, lm["w"], lm["s"], out_dtype=torch.float32, output=self.logits, fmt="e4m3")
        return self.out

    def capture(self) -> None:
        """Record one step (reading self.x) as a HIP graph on a side stream of default priority."""
        self.graph = torch.cuda.CUDAGraph()
        self._stream = torch.cuda.Stream()
        self._stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(self._stream):
            with torch.cuda.graph(self.graph, stream=self._stream):
                self.step()
        torch.cuda.current_stream().wait_stream(self._stream)

    def replay(self, x: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Replay the captured step on the current stream's order (x, when given, is copied into self.x first)."""
        _check(self.graph is not None, "capture() the group first")
        if x is not None:
            self.x.copy_(x)
        self._stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(self._stream):
            self.graph.replay()
        torch.cuda.current_stream().wait_stream(self._stream)
        return self.out


def manifest_layers(manifest, role: str, buffers: dict, top_k: Optional[int] = None,
                    norm_topk_prob: bool = True) -> tuple:
    """Every layer of the packed group kernel `role` of a manifest (axk.manifest.Manifest) bound to the caller's
    buffers (the packs and banks, and a MoE group's routed experts e_gw<j> .. e_ds<j>, by IO name), as DecodeGroup
    layer dicts without their states: {"kind": "g" | "a", "w": the layer's weights, "moe": its MoE block} (a MoE
    layer is one whose bound weights carry the router; its block takes the router, the shared-expert gate and the
    routed experts, with top_k). The caller adds each layer's "state" / "conv" or "cache". Returns
    (layers, proj_fmt, mlp_fmt): the group's one projection format and one MLP format."""
    kinds = manifest.kernel(role).kinds()
    layers, fmts = [], set()
    for j, kind in enumerate(kinds):
        b = manifest.bind_layer(role, buffers, j)
        fmts.add((b.proj_fmt, b.mlp_fmt))
        w = dict(b.weights)
        moe = None
        if "w_router" in w:
            _check(top_k is not None and top_k > 0, f"{role}: a MoE layer needs top_k")
            moe = {n: w.pop(n) for n in ("w_router", "w_shg", "e_gw", "e_gs", "e_dw", "e_ds") if n in w}
            moe.update(top_k=int(top_k), norm_topk_prob=norm_topk_prob)
        layers.append({"kind": "g" if kind == "gdn" else "a", "w": w, "moe": moe})
    _check(len(fmts) == 1, f"{role}: the layers mix weight formats {sorted(fmts)}")
    proj_fmt, mlp_fmt = fmts.pop()
    return layers, proj_fmt, mlp_fmt
