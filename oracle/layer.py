"""Oracle: per-layer glue of the Qwen3.5 hybrid decode layer (CPU, test infrastructure only).

Restates, with the reference's rounding points (bf16 tensors between ops, fp32 inside each op):
  * rmsnorm            q35_step.py rmsnorm(x, w, eps) with w = 1 + weight for layer / q / k norms (one_plus,
                       models/qwen35_35b_a3b/src/70b0fbc/q35_step.py:346-348); models/qwen38_27b/mtp/mtp_ref.py:172-174
  * gated_rmsnorm_silu the GDN output norm, rmsnorm(core, norm_w) then silu_gate(normed, z) (q35_step.py:179-180)
  * causal_conv1d_silu causal_conv1d_silu_reference (models/qwen35_35b_a3b/sgl/tests/test_gdn_attn.py:241-256) in
                       the kernel's weight layout (column 0 multiplies the current token, gdn_args q35_step.py:365-368)
  * rope               NeoX halves of the first rot channels (models/qwen38_27b/mtp/mtp_ref.py:176-187), cos / sin
                       given as bf16 (rope_cos_sin, q35_step.py:408-411)
  * qk_norm_rope, sigmoid_mul, silu_mul, add: attn_block / mlp_block (q35_step.py:136-139, 191-197, 276-279)
Pinned by tests/test_oracle_layer.py against transformers' Qwen3_5RMSNorm, Qwen3_5RMSNormGated and
apply_rotary_pos_emb (third-party, installed), torch.nn.functional.conv1d, and closed forms; the whole decode
layers (gdn_layer_decode, attn_layer_decode) token by token against transformers' Qwen3_5DecoderLayer run over
the same tokens in fp32 (oracle.rounding.fp32() switches the bf16 points off), and the bf16 schedule within
tolerance of that fp32 composition.
"""
from __future__ import annotations

import torch

from .rounding import bf as _bf
from .rounding import rounding


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """bf16(x * rsqrt(mean(x^2) + eps) * w) over the last dim, fp32 inside."""
    xf = x.float()
    return _bf(xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float())


def add_rmsnorm(x: torch.Tensor, y: torch.Tensor, w: torch.Tensor, eps: float = 1e-6):
    s = _bf(x.float() + y.float())
    return s, rmsnorm(s, w, eps)


def gated_rmsnorm_silu(x: torch.Tensor, w: torch.Tensor, z: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    normed = rmsnorm(x, w, eps)
    return _bf(normed.float() * torch.nn.functional.silu(z.float()))


def causal_conv1d_silu(x: torch.Tensor, w: torch.Tensor, state_in: torch.Tensor):
    """x [B, T, C] bf16; w [C, K] bf16 (column j multiplies x_{t-j}); state [B, K-1, C] bf16 (oldest first).
    Returns (out [B, T, C] bf16, state_out [B, K-1, C] bf16)."""
    k = w.shape[1]
    seq = torch.cat((state_in, x), dim=1)  # [B, K-1+T, C]
    t = x.shape[1]
    out = torch.zeros_like(x)
    for j in range(k):  # the current token first, then back through the window (test_gdn_attn.py:249-253)
        src = seq[:, k - 1 - j: k - 1 - j + t, :]
        out = _bf(out.float() + src.float() * w[:, j].float().reshape(1, 1, -1))
    state_out = seq[:, seq.shape[1] - (k - 1):, :] if k > 1 else seq[:, :0, :]
    return _bf(torch.nn.functional.silu(out.float())), state_out.contiguous()


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, rot: int) -> torch.Tensor:
    """x [B, heads, D] (bf16 values); cos, sin [B, rot/2]. fp32 rotation, bf16 out."""
    half = rot // 2
    xf = x.float()
    y = xf.clone()
    c, s = cos.float()[:, None, :], sin.float()[:, None, :]
    x1, x2 = xf[..., :half], xf[..., half:rot]
    y[..., :half] = x1 * c - x2 * s
    y[..., half:rot] = x2 * c + x1 * s
    return _bf(y)


def qk_norm_rope(x: torch.Tensor, w: torch.Tensor, cos, sin, rot: int, eps: float = 1e-6) -> torch.Tensor:
    r = rmsnorm(x, w, eps)
    return rope(r, cos, sin, rot) if rot else r


def rope_cos_sin(pos: torch.Tensor, rot: int, theta: float) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 cos / sin [B, rot/2] of each sequence's position (q35_step.py:408-411)."""
    inv = 1.0 / (theta ** (torch.arange(0, rot, 2, dtype=torch.int64).float() / rot))
    f = pos.float().reshape(-1, 1) * inv.reshape(1, -1)
    return _bf(f.cos()), _bf(f.sin())


def sigmoid_mul(x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    return _bf(x.float() * torch.sigmoid(gate.float()))


def silu_mul(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    return _bf(torch.nn.functional.silu(g.float()) * u.float())


def add(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    return _bf(x.float() + y.float())


# ---------------------------------------------------------------------------------------------
# Whole decode layers, composed from the restatements above and the other oracles
# (gdn_layer q35_step.py:149-183, attn_block 186-293, mlp_block 118-142)
# ---------------------------------------------------------------------------------------------
def proj(a: torch.Tensor, w: dict, name: str, fmt: str = "fp8") -> torch.Tensor:
    """bf16(a @ W_name^T) in fp32 for the weight w_<name> / s_<name> in format fmt: "fp8" (E4M3 with a per-channel
    scale, gemm.py:119-181), "mxfp8" (E4M3 + E8M0 per 32, q35_mx_build.py:60-72), "mxfp4" (q35_moe.py:46-63) or
    "nvfp4" (E2M1 + E4M3 per 16 + the scale2 t_<name>, q35_mx_build.py:168-200)."""
    from oracle import mx

    wt, s = w["w_" + name], w["s_" + name]
    if fmt == "fp8":
        y = mx.fp8_linear(a, wt.numpy(), None, s)
    elif fmt == "mxfp8":
        y = mx.mxfp8_linear(a, wt.numpy(), s.numpy(), "e4m3")
    elif fmt == "nvfp4":  # E2M1 + E4M3 per 16 + scale2 t_<name> (q35_mx_build.py:168-200)
        y = mx.nvfp4_linear(a, wt.numpy(), s.view(torch.uint8).numpy(), float(w["t_" + name].reshape(-1)[0]))
    else:
        y = mx.mx_linear(a, wt.numpy(), s.numpy())
    return _bf(y)


def mlp_residual(x: torch.Tensor, y: torch.Tensor, w: dict, eps: float, fmt: str = "mxfp4") -> torch.Tensor:
    """x1 = bf16(x + y); out = bf16(x1 + down(bf16(silu(gate h2) * up h2))), h2 = rmsnorm(x1, ln2)."""
    x1, h2 = add_rmsnorm(x, y, w["ln2"], eps)
    g = proj(h2, w, "gate", fmt)
    u = proj(h2, w, "up", fmt)
    d = proj(silu_mul(g, u), w, "down", fmt)
    return add(x1, d)


def dequant_weight(w: dict, name: str, fmt: str) -> torch.Tensor:
    """The fp32 weight w_<name> [N, K] of format fmt, exactly dequantised (as proj multiplies it)."""
    from oracle import mx

    wt, s = w["w_" + name].numpy(), w["s_" + name]
    if fmt == "fp8":
        return torch.from_numpy(mx.e4m3_table()[wt]) * s.float().reshape(-1, 1)
    if fmt == "mxfp8":
        return torch.from_numpy(mx.dequant_mxfp8(wt, s.numpy(), "e4m3"))
    if fmt == "nvfp4":
        return torch.from_numpy(mx.dequant_nvfp4(wt, s.view(torch.uint8).numpy(), float(w["t_" + name].reshape(-1)[0])))
    return torch.from_numpy(mx.dequant_mxfp4(wt, s.numpy()))


def moe_block_parts(x, y, w: dict, moe: dict, eps: float = 1e-6, fmt: str = "mxfp8", ids=None, wts=None,
                    flips: int = 2, slot_bf16: bool = False):
    """moe_full (models/qwen35_35b_a3b/src/70b0fbc/q35_layer_mc.py:797-853) after the layer's first half:
    x1 = bf16(x + y), h2 = rmsnorm(x1, ln2); the shared expert sh = bf16(silu(bf16 h2 Wg^T) * bf16 h2 Wu^T) Wd^T in
    fp32, its weights the layer's MLP (w_gate .. s_down) in fmt; logits = h2 w_router^T; the routing (ids, wts)
    given or the top-K of the logits (oracle.moe.route); base = x1 + sigmoid(h2 . w_shg) sh; the routed MXFP4 experts
    as oracle.moe.moe_parts (fp32 slots; slot_bf16: bf16 slots, the prefill form). Returns (base, routed, slack,
    logits, ids, wts), fp32; slack bounds `flips` one-ulp changes of each bf16 activation row, the shared expert's
    included (oracle.moe.moe_parts)."""
    from oracle import moe as omoe

    x1, h2 = add_rmsnorm(x, y, w["ln2"], eps)
    logits = h2.float() @ moe["w_router"].float().T
    if ids is None:
        ids, wts = omoe.route(logits, int(moe["top_k"]), moe.get("norm_topk_prob", True))
    act = silu_mul(proj(h2, w, "gate", fmt), proj(h2, w, "up", fmt)).float()
    wd = dequant_weight(w, "down", fmt)
    sh = act @ wd.T
    shg = moe.get("w_shg")
    gate = torch.sigmoid(h2.float() @ shg.float()) if shg is not None else torch.ones(x.shape[0])
    routed_w = {n: moe[n] for n in ("e_gw", "e_gs", "e_dw", "e_ds")}
    base0, routed, slack = omoe.moe_parts(h2, routed_w, ids, wts, x1, flips=flips, slot_bf16=slot_bf16)
    base = base0 + gate[:, None] * sh
    slack = slack + flips * (gate * omoe.ulp_bf16(act).amax(dim=1))[:, None] * wd.abs().amax(dim=1)[None, :]
    return base, routed, slack, logits, ids, wts


def value_head_keys(x, num_v_heads: int, v_order: str):
    """q or k [B, T, NK, D] -> [B, T, NV, D]: the key head each value head reads. "grouped": value head vh reads key
    head vh / (NV / NK) (the checkpoint's order and the GDN operators', test_gdn_attn.py:268-277); "tiled": vh % NK,
    the order the reference's layer kernels are built with by default (models/qwen35_35b_a3b/src/70b0fbc/
    q35_step.py:82-85 VORDER; 171: vh = vo * NK + kh)."""
    rep = num_v_heads // x.shape[2]
    if v_order == "grouped":
        return x.repeat_interleave(rep, dim=2)
    assert v_order == "tiled", v_order
    return x.repeat(1, 1, rep, 1)


def gdn_layer_decode(x, w: dict, state_in, conv_in, num_k_heads: int, num_v_heads: int, eps: float = 1e-6,
                     proj_fmt: str = "fp8", mlp_fmt: str = "mxfp4", v_order: str = "tiled"):
    """One token per sequence. Returns (out bf16 [B, H], state_out f32, conv_out bf16)."""
    y, state_out, conv_out = gdn_layer_half(x, w, state_in, conv_in, num_k_heads, num_v_heads, eps, proj_fmt,
                                            v_order)
    return mlp_residual(x, y, w, eps, mlp_fmt), state_out, conv_out


def gdn_layer_half(x, w: dict, state_in, conv_in, num_k_heads: int, num_v_heads: int, eps: float = 1e-6,
                   proj_fmt: str = "fp8", v_order: str = "tiled"):
    """The GDN layer up to its output projection y (bf16, before the residual and the MLP / MoE block).
    Returns (y, state_out, conv_out)."""
    from oracle import gdn

    b = x.shape[0]
    kd, vd = num_k_heads * 128, num_v_heads * 128
    h = rmsnorm(x, w["ln1"], eps)
    qkv, z, bb, aa = (proj(h, w, n, proj_fmt) for n in ("qkv", "z", "b", "a"))
    mixed, conv_out = causal_conv1d_silu(qkv[:, None, :], w["conv_w"], conv_in)
    m = mixed[:, 0]
    q = m[:, :kd].reshape(b, 1, num_k_heads, 128)
    k = m[:, kd:2 * kd].reshape(b, 1, num_k_heads, 128)
    v = m[:, 2 * kd:].reshape(b, 1, num_v_heads, 128)
    q, k = value_head_keys(q, num_v_heads, v_order), value_head_keys(k, num_v_heads, v_order)
    core, state_out = gdn.gdn_fp32(q, k, v, aa[:, None], bb[:, None], w["a_log"], w["dt_bias"], state_in)
    core = _bf(core).reshape(b * num_v_heads, 128)
    gated = gated_rmsnorm_silu(core, w["norm_w"], z.reshape(b * num_v_heads, 128), eps).reshape(b, vd)
    return proj(gated, w, "out", proj_fmt), state_out, conv_out


def attn_layer_decode(x, w: dict, cos, sin, cache, indptr, indices, last_page_len, cache_location,
                      num_qo_heads: int, rot: int, eps: float = 1e-6, sm_scale=None, proj_fmt: str = "fp8",
                      mlp_fmt: str = "mxfp4"):
    """One token per sequence over the paged cache (the page table includes the new token).
    Returns (out bf16 [B, H], the cache with the new K / V rows written)."""
    y, cache2 = attn_layer_half(x, w, cos, sin, cache, indptr, indices, last_page_len, cache_location, num_qo_heads,
                                rot, eps, sm_scale, proj_fmt)
    return mlp_residual(x, y, w, eps, mlp_fmt), cache2


def attn_layer_half(x, w: dict, cos, sin, cache, indptr, indices, last_page_len, cache_location,
                    num_qo_heads: int, rot: int, eps: float = 1e-6, sm_scale=None, proj_fmt: str = "fp8"):
    """The attention layer up to its output projection y (bf16, before the residual and the MLP / MoE block).
    Returns (y, the cache with the new K / V rows written)."""
    from oracle import paged_attn

    b = x.shape[0]
    hkv, d = cache.shape[3], cache.shape[4]
    scale = d ** -0.5 if sm_scale is None else sm_scale
    h = rmsnorm(x, w["ln1"], eps)
    qg = proj(h, w, "q", proj_fmt).reshape(b, num_qo_heads, 2 * d)
    kk = proj(h, w, "k", proj_fmt).reshape(b, hkv, d)
    vv = proj(h, w, "v", proj_fmt).reshape(b, hkv, d)
    q = qk_norm_rope(qg[..., :d], w["q_norm"], cos, sin, rot, eps)
    k = qk_norm_rope(kk, w["k_norm"], cos, sin, rot, eps)
    cache2 = paged_attn.store_paged_kv(cache, k, vv, cache_location.numpy())
    attn = _bf(paged_attn.paged_decode(q, cache2, indptr, indices, last_page_len, scale))
    gated = sigmoid_mul(attn, qg[..., d:]).reshape(b, num_qo_heads * d)
    return proj(gated, w, "o", proj_fmt), cache2


# ---------------------------------------------------------------------------------------------
# Speculative verification (models/qwen38_27b/verify/verify_group_m4.py:1-9): T rows per sequence through a layer in
# one call is, by definition, T decode steps one row each; the per-row snapshots are the states after each step.
# ---------------------------------------------------------------------------------------------
def gdn_layer_verify(x, w: dict, state_in, conv_in, num_k_heads: int, num_v_heads: int, eps: float = 1e-6,
                     proj_fmt: str = "fp8", mlp_fmt: str = "mxfp4", v_order: str = "tiled"):
    """x bf16 [B, T, H]. Returns (out [B, T, H], state_out, conv_out, state_snaps [T, ...], conv_snaps [T, ...])."""
    outs, snaps, csnaps = [], [], []
    st, cv = state_in, conv_in
    for t in range(x.shape[1]):
        o, st, cv = gdn_layer_decode(x[:, t], w, st, cv, num_k_heads, num_v_heads, eps, proj_fmt, mlp_fmt, v_order)
        outs.append(o)
        snaps.append(st)
        csnaps.append(cv)
    return torch.stack(outs, 1), st, cv, torch.stack(snaps), torch.stack(csnaps)


def attn_layer_verify(x, w: dict, cos, sin, cache, indptr, indices, last_page_len, cache_location,
                      num_qo_heads: int, rot: int, eps: float = 1e-6, sm_scale=None, proj_fmt: str = "fp8",
                      mlp_fmt: str = "mxfp4"):
    """x bf16 [B, T, H]; the page table (indptr / indices / last_page_len) covers each sequence's history and its T
    new rows; cache_location [B, T, 2]; cos, sin [B, T, rot / 2]. Row t runs as a decode step over the table's
    prefix of length history + t + 1. Returns (out [B, T, H], the cache with every new row written)."""
    import numpy as np

    from oracle import paged_attn

    b, t_rows = x.shape[:2]
    page = cache.shape[2]
    ip = np.asarray(indptr)
    idx = np.asarray(indices)
    full = paged_attn.seq_lens(indptr, last_page_len, page)
    outs = []
    for t in range(t_rows):
        ptr, ind, last = [0], [], []
        for s in range(b):
            n_tok = full[s] - (t_rows - 1 - t)
            pages = (n_tok + page - 1) // page
            ind += idx[ip[s]:ip[s] + pages].tolist()
            ptr.append(len(ind))
            last.append(n_tok - (pages - 1) * page)
        o, cache = attn_layer_decode(x[:, t], w, cos[:, t], sin[:, t], cache, torch.tensor(ptr, dtype=torch.int32),
                                     torch.tensor(ind, dtype=torch.int32), torch.tensor(last, dtype=torch.int32),
                                     cache_location[:, t], num_qo_heads, rot, eps, sm_scale, proj_fmt, mlp_fmt)
        outs.append(o)
    return torch.stack(outs, 1), cache


# ---------------------------------------------------------------------------------------------
# Prefill (models/qwen35_35b_a3b/src/70b0fbc/q35_prefill.py): T new tokens per sequence through a layer; the
# projections and the MLP row by row as in decode, the GDN conv over the T tokens and the delta rule in the chunked
# form the reference's prefill uses (gdn_chunked, q35_prefill.py:144-169).
# ---------------------------------------------------------------------------------------------
def gdn_layer_prefill(x, w: dict, state_in, conv_in, num_k_heads: int, num_v_heads: int, eps: float = 1e-6,
                      proj_fmt: str = "fp8", mlp_fmt: str = "mxfp4", chunk: int = 64, v_order: str = "tiled"):
    """gdn_layer_prefill, q35_prefill.py:57-141: x bf16 [B, T, H]. rmsnorm and the qkv / z / b / a projections over
    the B T rows (69-74), the causal conv1d + SiLU over each sequence's tokens from its conv state (75-101), the
    chunked delta rule from state_in (gdn.gdn_chunk with the reference's bf16 rounding points, none when the layer's
    points are switched off; 103-109, gdn_chunked 144-169), the gated norm (125-138), the output projection and the
    MLP (139-140). Returns (out [B, T, H], state_out, conv_out)."""
    return gdn_layer_prefill_parts(x, w, state_in, conv_in, num_k_heads, num_v_heads, eps, proj_fmt, mlp_fmt,
                                   chunk, v_order=v_order)[:3]


def gdn_layer_prefill_parts(x, w: dict, state_in, conv_in, num_k_heads: int, num_v_heads: int, eps: float = 1e-6,
                            proj_fmt: str = "fp8", mlp_fmt: str = "mxfp4", chunk: int = 64, flips: int = 2,
                            v_order: str = "tiled"):
    """gdn_layer_prefill and the slack of gdn_prefill_half. Returns (out, state_out, conv_out, slack fp32
    [B, T, H])."""
    b, t, hd = x.shape
    y, state_out, conv_out, slack = gdn_prefill_half(x, w, state_in, conv_in, num_k_heads, num_v_heads, eps, proj_fmt,
                                                     chunk, flips, v_order)
    out = mlp_residual(x.reshape(b * t, hd), y, w, eps, mlp_fmt).reshape(b, t, hd)
    return out, state_out, conv_out, slack.reshape(b, t, hd)


def gdn_prefill_half(x, w: dict, state_in, conv_in, num_k_heads: int, num_v_heads: int, eps: float = 1e-6,
                     proj_fmt: str = "fp8", chunk: int = 64, flips: int = 2, v_order: str = "tiled"):
    """The GDN prefill layer up to its output projection (q35_prefill.py:69-139 before the residual), over the B T
    rows, and a bound on how far `flips` one-ulp changes of each row's bf16 gated output (the input of the output
    projection, rmsnorm(core) * silu(z), whose magnitude the gate can raise well above the core's) move y: per row,
    flips times the row's largest gated ulp against the largest |W_out| of each output column, the model of
    oracle.moe.moe_parts. Returns (y bf16 [B T, H], state_out, conv_out, slack fp32 [B T, H])."""
    from oracle import gdn
    from oracle import moe as omoe

    b, t, hd = x.shape
    r = b * t
    kd, vd = num_k_heads * 128, num_v_heads * 128
    xr = x.reshape(r, hd)
    h = rmsnorm(xr, w["ln1"], eps)
    qkv, z, bb, aa = (proj(h, w, n, proj_fmt) for n in ("qkv", "z", "b", "a"))
    mixed, conv_out = causal_conv1d_silu(qkv.reshape(b, t, -1), w["conv_w"], conv_in)
    q = mixed[..., :kd].reshape(b, t, num_k_heads, 128)
    k = mixed[..., kd:2 * kd].reshape(b, t, num_k_heads, 128)
    v = mixed[..., 2 * kd:].reshape(b, t, num_v_heads, 128)
    q, k = value_head_keys(q, num_v_heads, v_order), value_head_keys(k, num_v_heads, v_order)
    core, state_out = gdn.gdn_chunk(q, k, v, aa.reshape(b, t, num_v_heads), bb.reshape(b, t, num_v_heads),
                                    w["a_log"], w["dt_bias"], state_in, chunk=chunk, round_bf16=rounding())
    core = _bf(core).reshape(r * num_v_heads, 128)
    gated = gated_rmsnorm_silu(core, w["norm_w"], z.reshape(r * num_v_heads, 128), eps).reshape(r, vd)
    y = proj(gated, w, "out", proj_fmt)
    wo = dequant_weight(w, "out", proj_fmt)
    slack = flips * omoe.ulp_bf16(gated.float()).amax(dim=1)[:, None] * wo.abs().amax(dim=1)[None, :]
    return y, state_out, conv_out, slack


def attn_rows_half(x, w: dict, cos, sin, cache, indptr, indices, last_page_len, cache_location, num_qo_heads: int,
                   rot: int, eps: float = 1e-6, sm_scale=None, proj_fmt: str = "fp8"):
    """The attention layer over T new rows per sequence up to its output projection: row t as a decode step over
    the page table's prefix of history + t + 1 tokens (as attn_layer_verify). Returns (y bf16 [B T, H], the cache
    with every new row written)."""
    import numpy as np

    from oracle import paged_attn

    b, t_rows = x.shape[:2]
    page = cache.shape[2]
    ip = np.asarray(indptr)
    idx = np.asarray(indices)
    full = paged_attn.seq_lens(indptr, last_page_len, page)
    ys = []
    for t in range(t_rows):
        ptr, ind, last = [0], [], []
        for s_ in range(b):
            n_tok = full[s_] - (t_rows - 1 - t)
            pages = (n_tok + page - 1) // page
            ind += idx[ip[s_]:ip[s_] + pages].tolist()
            ptr.append(len(ind))
            last.append(n_tok - (pages - 1) * page)
        y, cache = attn_layer_half(x[:, t], w, cos[:, t], sin[:, t], cache, torch.tensor(ptr, dtype=torch.int32),
                                   torch.tensor(ind, dtype=torch.int32), torch.tensor(last, dtype=torch.int32),
                                   cache_location[:, t], num_qo_heads, rot, eps, sm_scale, proj_fmt)
        ys.append(y)
    return torch.stack(ys, 1).reshape(b * t_rows, -1), cache
