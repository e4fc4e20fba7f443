"""Seeded synthetic inputs for the BASELINE configs (CPU torch.Generator, fixed draw order).

Each generator returns host tensors; callers move them to the device. Draw order is part of the
contract (tests, smoke and bench all regenerate the same inputs from the seed).
"""
from __future__ import annotations

import torch


def pack_codes(codes: torch.Tensor) -> torch.Tensor:
    """Logical E2M1 codes [..., K] -> packed u8 [..., K/2], even column in the low nibble."""
    codes = codes.to(torch.uint8)
    return (codes[..., 0::2] & 15) | ((codes[..., 1::2] & 15) << 4)


def mxfp4_weight(n: int, k: int, g: torch.Generator, lo: int = 119, hi: int = 123, lead=()):
    """Uniform random nibbles and E8M0 exponent bytes uniform in [lo, hi]: (codes [.., n, k/2], scales [.., n, k/32])."""
    codes = torch.randint(0, 16, (*lead, n, k), generator=g, dtype=torch.uint8)
    scales = torch.randint(lo, hi + 1, (*lead, n, k // 32), generator=g, dtype=torch.uint8)
    return pack_codes(codes).contiguous(), scales.contiguous()


def config0(seed: int = 0):
    """Config 0: single MXFP4 linear, W N=4096 x K=4096, x bf16 [1, 4096] ~ N(0,1)."""
    g = torch.Generator().manual_seed(seed)
    codes, scales = mxfp4_weight(4096, 4096, g)
    x = torch.randn(1, 4096, generator=g).to(torch.bfloat16)
    return {"x": x, "w": codes, "s": scales}


LM_HEAD = {"vocab": 248320, "hidden": 2048}  # mul_mat_mx4_n248320_k2048 (tools/manifest/mkmanifest.py:42)


def lm_head_case(dev, seed: int = 0, n: int = LM_HEAD["vocab"], k: int = LM_HEAD["hidden"], m: int = 1):
    """The MXFP4 LM head GEMV (decode): W [n, k] as config 0's weight (uniform nibbles, E8M0 bytes in 119..123),
    x bf16 [m, k] ~ N(0,1), fp32 logits. Generated on `dev` (a 270 MB weight at the full vocabulary)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    codes = torch.randint(0, 16, (n, k), generator=g, dtype=torch.uint8, device=dev)
    scales = torch.randint(119, 124, (n, k // 32), generator=g, dtype=torch.uint8, device=dev)
    x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
    return {"x": x, "w": pack_codes(codes).contiguous(), "s": scales.contiguous()}


def lm_head_nvfp4_case(dev, seed: int = 0, n: int = LM_HEAD["vocab"], k: int = LM_HEAD["hidden"], m: int = 1):
    """The LM head in NVFP4 (the reference's NVFP4 head, test_nvfp4_lm_head.py): uniform nibbles, E4M3 block scale
    bytes uniform in 0x28 .. 0x37 (0.25 .. 0.47), scale2 = 0.05 (a weight RMS of about 0.05 as the MXFP4 head's), x
    bf16 [m, k] ~ N(0,1), fp32 logits. Generated on `dev`."""
    g = torch.Generator(device=dev).manual_seed(seed)
    codes = torch.randint(0, 16, (n, k), generator=g, dtype=torch.uint8, device=dev)
    scales = torch.randint(0x28, 0x38, (n, k // 16), generator=g, dtype=torch.uint8, device=dev)
    x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
    return {"x": x, "w": pack_codes(codes).contiguous(), "s": scales.contiguous(),
            "s2": torch.tensor([0.05], dtype=torch.float32, device=dev)}


def paged_case(lens, hq: int, hkv: int, d: int, page: int, g: torch.Generator, extra_pages: int = 0):
    """A paged KV pool holding sequences of the given lengths, pages placed by a random permutation."""
    npages = [(L + page - 1) // page for L in lens]
    pool = sum(npages) + extra_pages
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    indptr = torch.zeros(len(lens) + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(torch.tensor(npages, dtype=torch.int32), 0)
    indices = perm[: int(indptr[-1])].contiguous()
    last = torch.tensor([L - page * (n - 1) if n else 0 for L, n in zip(lens, npages)], dtype=torch.int32)
    q = torch.randn(len(lens), hq, d, generator=g).to(torch.bfloat16)
    cache = torch.randn(pool, 2, page, hkv, d, generator=g).to(torch.bfloat16)
    return {"q": q, "cache": cache, "indptr": indptr, "indices": indices, "last_page_len": last,
            "lens": list(lens), "scale": d ** -0.5}


def prefill_case(qlens, kv_lens, hq: int, hkv: int, d: int, page: int, g: torch.Generator, extra_pages: int = 0):
    """paged_case over kv_lens plus q bf16 [sum(qlens), HQ, D] and qo_indptr: sequence b's qlens[b] new tokens are
    the last of its kv_lens[b] cached tokens."""
    c = paged_case(kv_lens, hq, hkv, d, page, g, extra_pages)
    c["q"] = torch.randn(sum(qlens), hq, d, generator=g).to(torch.bfloat16)
    qo = torch.zeros(len(qlens) + 1, dtype=torch.int32)
    qo[1:] = torch.cumsum(torch.tensor(qlens, dtype=torch.int32), 0)
    c["qo_indptr"] = qo
    c["qlens"] = list(qlens)
    return c


def config1(seed: int = 0):
    """Config 1: paged decode, batch 16, 16 q heads / 2 KV heads, D 256, page 64, L_b ~ U[1024, 16384]."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(1024, 16385, (16,), generator=g).tolist()
    return paged_case(lens, 16, 2, 256, 64, g)


def gdn_inputs(bsz: int, t: int, g: torch.Generator, nk: int = 16, nv: int = 32, d: int = 128,
               state_std: float = 0.02):
    """Config 2 distributions: q, k, v ~ N(0,1) (the kernel L2-normalises q and k); a, b ~ N(0,1) with
    A_log = dt_bias = 0, so g = -softplus(a) and beta = sigmoid(b); state ~ N(0, state_std) (0: zero state)."""
    q = torch.randn(bsz, t, nk, d, generator=g).to(torch.bfloat16)
    k = torch.randn(bsz, t, nk, d, generator=g).to(torch.bfloat16)
    v = torch.randn(bsz, t, nv, d, generator=g).to(torch.bfloat16)
    a = torch.randn(bsz, t, nv, generator=g).to(torch.bfloat16)
    b = torch.randn(bsz, t, nv, generator=g).to(torch.bfloat16)
    a_log = torch.zeros(nv)
    dt_bias = torch.zeros(nv)
    state = (torch.randn(bsz, nv, d, d, generator=g) * state_std) if state_std else torch.zeros(bsz, nv, d, d)
    return {"q": q, "k": k, "v": v, "a": a, "b": b, "a_log": a_log, "dt_bias": dt_bias, "state": state}


def config2_decode(seed: int = 0):
    """Config 2 decode: B = 32, one token, 32 value / 16 key heads, d = 128, state ~ N(0, 0.02)."""
    return gdn_inputs(32, 1, torch.Generator().manual_seed(seed))


def config2_prefill(seed: int = 0):
    """Config 2 prefill: B = 1, T = 4096 from a zero state (chunk 64)."""
    return gdn_inputs(1, 4096, torch.Generator().manual_seed(seed), state_std=0.0)


def moe_weights(g: torch.Generator, hidden: int = 2048, experts: int = 256, inter: int = 512,
                shared_inter: int = 512, router_std: float = 0.02):
    """Config 3 weights: MXFP4 experts as config 0 (nibbles uniform, scale bytes 119..123), bf16 router and
    shared-expert gate ~ N(0, router_std). Draw order: router, w_shg, shared gate / up / down, e_gw/e_gs,
    e_dw/e_ds."""
    w = {}
    w["w_router"] = (torch.randn(experts, hidden, generator=g) * router_std).to(torch.bfloat16)
    w["w_shg"] = (torch.randn(hidden, generator=g) * router_std).to(torch.bfloat16)
    w["w_gate"], w["s_gate"] = mxfp4_weight(shared_inter, hidden, g)
    w["w_up"], w["s_up"] = mxfp4_weight(shared_inter, hidden, g)
    w["w_down"], w["s_down"] = mxfp4_weight(hidden, shared_inter, g)
    w["e_gw"], w["e_gs"] = mxfp4_weight(2 * inter, hidden, g, lead=(experts,))
    w["e_dw"], w["e_ds"] = mxfp4_weight(hidden, inter, g, lead=(experts,))
    return w


def moe_block(g: torch.Generator, hidden: int, experts: int = 256, inter: int = 512, top_k: int = 8,
              router_std: float = 0.02) -> dict:
    """The MoE block of a MoE decode layer beside the layer's MLP weights (its shared expert): bf16 router and
    shared-expert gate ~ N(0, router_std), MXFP4 routed experts as config 3 (nibbles uniform, scale bytes 119..123),
    top_k. Draw order: router, w_shg, e_gw/e_gs, e_dw/e_ds."""
    w = {"w_router": (torch.randn(experts, hidden, generator=g) * router_std).to(torch.bfloat16),
         "w_shg": (torch.randn(hidden, generator=g) * router_std).to(torch.bfloat16)}
    w["e_gw"], w["e_gs"] = mxfp4_weight(2 * inter, hidden, g, lead=(experts,))
    w["e_dw"], w["e_ds"] = mxfp4_weight(hidden, inter, g, lead=(experts,))
    w["top_k"] = top_k
    return w


def config3(tokens: int = 32, seed: int = 0):
    """Config 3: MoE layer, hidden 2048, 256 routed experts (inter 512) + 1 shared expert (inter 512), top-8,
    activations ~ N(0,1) at `tokens` (32 = decode, 4096 = prefill); x_res ~ N(0,1) residual."""
    g = torch.Generator().manual_seed(seed)
    w = moe_weights(g)
    h2 = torch.randn(tokens, 2048, generator=g).to(torch.bfloat16)
    x_res = torch.randn(tokens, 2048, generator=g).to(torch.bfloat16)
    return {"h2": h2, "x_res": x_res, "weights": w, "top_k": 8}


def config4_fp8_proj(seed: int = 0, n: int = 16384, k: int = 4096, m: int = 8):
    """Config 4's largest FP8 projection (attention q + gate, [16384, 4096]) at the group's decode batch of 8:
    weight = N(0, 0.5) rounded to E4M3 (u8 codes), per-output-channel scale_b ~ U(0.01, 0.03) f32,
    x bf16 [m, k] ~ N(0,1). Draw order: weight, scale_b, x."""
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=g) * 0.5).to(torch.float8_e4m3fn).view(torch.uint8).contiguous()
    scale_b = torch.rand(n, generator=g) * 0.02 + 0.01
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    return {"x": x, "w": w, "scale_b": scale_b}


def config1_kv_write(seed: int = 0):
    """The current token's K and V rows of config 1 (bf16 [16, 2, 256] ~ N(0,1)), written into the config-1
    cache at each sequence's last page, offset last_page_len - 1 (in bounds of the pool)."""
    c = config1(seed)
    g = torch.Generator().manual_seed(seed + 1)
    b, hkv, d = c["q"].shape[0], c["cache"].shape[3], c["cache"].shape[4]
    k = torch.randn(b, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(b, hkv, d, generator=g).to(torch.bfloat16)
    ends = c["indptr"][1:].long() - 1
    loc = torch.stack([c["indices"][ends], c["last_page_len"] - 1], dim=1).to(torch.int32).contiguous()
    return {"cache": c["cache"], "k": k, "v": v, "loc": loc}


def fp8_proj_weight(n: int, k: int, g: torch.Generator):
    """FP8 E4M3 projection [n, k] (N(0, 0.5) rounded to E4M3) and per-output-channel scale ~ U(1, 3) / sqrt(k)."""
    w = (torch.randn(n, k, generator=g) * 0.5).to(torch.float8_e4m3fn).view(torch.uint8).contiguous()
    s = (torch.rand(n, generator=g) * 2 + 1) / (k ** 0.5)
    return w, s


def proj_weight(fmt: str, n: int, k: int, g: torch.Generator):
    """A weight [n, k] in format fmt with its scales: "fp8" as fp8_proj_weight; "mxfp4" as mxfp4_weight (config 0's
    draws); "mxfp8" E4M3 codes of N(0, 3^2) (torch's float8_e4m3fn cast) with E8M0 scale bytes uniform in 119..123,
    the same weight RMS (about 0.05) as the MXFP4 draws."""
    if fmt == "fp8":
        return fp8_proj_weight(n, k, g)
    if fmt == "mxfp4":
        return mxfp4_weight(n, k, g)
    codes = (torch.randn(n, k, generator=g) * 3).to(torch.float8_e4m3fn).view(torch.uint8).contiguous()
    return codes, torch.randint(119, 124, (n, k // 32), generator=g, dtype=torch.uint8)


def _put(w: dict, name: str, fmt: str, n: int, k: int, g: torch.Generator) -> None:
    """w_<name>, s_<name> (and t_<name> for "nvfp4") of an [n, k] weight in format fmt: proj_weight's draws, or for
    NVFP4 uniform nibbles with E4M3 scale bytes uniform in 0x28 .. 0x37 (0.25 .. 0.47) and scale2 0.05, a weight RMS
    of about 0.05 as the MXFP8 draws."""
    if fmt == "nvfp4":
        codes = torch.randint(0, 16, (n, k), generator=g, dtype=torch.uint8)
        w["w_" + name] = pack_codes(codes).contiguous()
        w["s_" + name] = torch.randint(0x28, 0x38, (n, k // 16), generator=g, dtype=torch.uint8)
        w["t_" + name] = torch.tensor([0.05], dtype=torch.float32)
    else:
        w["w_" + name], w["s_" + name] = proj_weight(fmt, n, k, g)


def _norm_w(n: int, g: torch.Generator):
    """A norm's run-time weight as the reference passes it: 1 + N(0, 0.1) (f32)."""
    return 1.0 + 0.1 * torch.randn(n, generator=g)


def mlp_weights(g: torch.Generator, hidden: int, inter: int, fmt: str = "mxfp4") -> dict:
    """The dense MLP of a layer: gate / up [inter, hidden], down [hidden, inter] (MXFP4 by default, as config 0's
    draws)."""
    w = {}
    _put(w, "gate", fmt, inter, hidden, g)
    _put(w, "up", fmt, inter, hidden, g)
    _put(w, "down", fmt, hidden, inter, g)
    return w


def gdn_layer_weights(g: torch.Generator, hidden: int, inter: int, nk: int, nv: int, conv_kernel: int = 4,
                      proj_fmt: str = "fp8", mlp_fmt: str = "mxfp4") -> dict:
    """A GDN decode layer's weights (names of q35_step.py gdn_args): projections in proj_fmt (FP8 by default), bf16
    conv taps, f32 norms (ln1 / ln2 = 1 + N(0, 0.1); norm_w = 1 + N(0, 0.1)), A_log, dt_bias ~ N(0, 0.5), the MLP in
    mlp_fmt (MXFP4 by default)."""
    kd, vd = nk * 128, nv * 128
    w = {"ln1": _norm_w(hidden, g)}
    _put(w, "qkv", proj_fmt, 2 * kd + vd, hidden, g)
    _put(w, "z", proj_fmt, vd, hidden, g)
    _put(w, "b", proj_fmt, nv, hidden, g)
    _put(w, "a", proj_fmt, nv, hidden, g)
    w["conv_w"] = (torch.randn(2 * kd + vd, conv_kernel, generator=g) * 0.5).to(torch.bfloat16)
    w["a_log"] = torch.randn(nv, generator=g) * 0.5
    w["dt_bias"] = torch.randn(nv, generator=g) * 0.5
    w["norm_w"] = _norm_w(128, g)
    _put(w, "out", proj_fmt, hidden, vd, g)
    w["ln2"] = _norm_w(hidden, g)
    w.update(mlp_weights(g, hidden, inter, mlp_fmt))
    return w


def attn_layer_weights(g: torch.Generator, hidden: int, inter: int, hq: int, hkv: int, d: int,
                       proj_fmt: str = "fp8", mlp_fmt: str = "mxfp4") -> dict:
    """An attention decode layer's weights (names of q35_step.py attn_args): q (per head [q | gate]), k, v, o in
    proj_fmt (FP8 by default); f32 norms 1 + N(0, 0.1); the MLP in mlp_fmt (MXFP4 by default)."""
    w = {"ln1": _norm_w(hidden, g)}
    _put(w, "q", proj_fmt, hq * 2 * d, hidden, g)
    _put(w, "k", proj_fmt, hkv * d, hidden, g)
    _put(w, "v", proj_fmt, hkv * d, hidden, g)
    w["q_norm"] = _norm_w(d, g)
    w["k_norm"] = _norm_w(d, g)
    _put(w, "o", proj_fmt, hidden, hq * d, g)
    w["ln2"] = _norm_w(hidden, g)
    w.update(mlp_weights(g, hidden, inter, mlp_fmt))
    return w


def append_token_case(lens, hq: int, hkv: int, d: int, page: int, g: torch.Generator):
    """A paged cache holding sequences of `lens` tokens plus room for one more each: returns the paged case with
    the page table already covering the new token (lens + 1), its cache locations (int32 [B, 2]) and positions."""
    c = paged_case(lens, hq, hkv, d, page, g, extra_pages=len(lens))
    used = set(c["indices"].tolist())
    spare = [p for p in range(c["cache"].shape[0]) if p not in used]
    loc, new_last, new_indices, new_indptr = [], [], [], [0]
    for b, L in enumerate(lens):
        pages = c["indices"][int(c["indptr"][b]):int(c["indptr"][b + 1])].tolist()
        if L % page == 0:
            pages.append(spare.pop())
        loc.append([pages[-1], L % page])
        new_indices += pages
        new_indptr.append(len(new_indices))
        new_last.append(L % page + 1)
    c.update(indices=torch.tensor(new_indices, dtype=torch.int32), indptr=torch.tensor(new_indptr, dtype=torch.int32),
             last_page_len=torch.tensor(new_last, dtype=torch.int32), lens=[L + 1 for L in lens],
             loc=torch.tensor(loc, dtype=torch.int32), pos=torch.tensor(list(lens)))
    return c


def verify_rows_case(lens, rows: int, hq: int, hkv: int, d: int, page: int, g: torch.Generator):
    """A paged cache holding sequences of `lens` tokens plus room for `rows` more each (a speculative draft): the page
    table already covers the new rows (lens + rows tokens), cache locations int32 [B, rows, 2] and positions
    [B, rows] of the new rows."""
    c = paged_case(lens, hq, hkv, d, page, g, extra_pages=len(lens) * ((rows + page - 1) // page + 1))
    used = set(c["indices"].tolist())
    spare = [p for p in range(c["cache"].shape[0]) if p not in used]
    loc, new_last, new_indices, new_indptr, pos = [], [], [], [0], []
    for b, L in enumerate(lens):
        pages = c["indices"][int(c["indptr"][b]):int(c["indptr"][b + 1])].tolist()
        rl = []
        for r in range(rows):
            tok = L + r
            if tok // page >= len(pages):
                pages.append(spare.pop())
            rl.append([pages[tok // page], tok % page])
        loc.append(rl)
        pos.append([L + r for r in range(rows)])
        new_indices += pages
        new_indptr.append(len(new_indices))
        n = L + rows
        new_last.append(n - (len(pages) - 1) * page)
    c.update(indices=torch.tensor(new_indices, dtype=torch.int32), indptr=torch.tensor(new_indptr, dtype=torch.int32),
             last_page_len=torch.tensor(new_last, dtype=torch.int32), lens=[L + rows for L in lens],
             loc=torch.tensor(loc, dtype=torch.int32), pos=torch.tensor(pos))
    return c


# Config 4: the 16-layer hybrid decode group (GDN, GDN, GDN, attention) x 4 of BASELINE.json configs[4].
CONFIG4 = dict(batch=8, ctx=131072, hidden=4096, inter=12288, hq=32, hkv=4, d=256, rot=64, nk=16, nv=32, conv=4,
               page=64, theta=10_000_000.0, eps=1e-6, pattern="gggagggagggaggga")


def config4_group(dev, seed: int = 0, ctx: int | None = None, batch: int | None = None) -> dict:
    """The group's weights, states, paged KV caches and page table, generated ON THE DEVICE by a seeded device
    generator (about 20 GB: the KV of 4 attention layers at 131,072 tokens per sequence). Distributions as the
    small-shape generators: FP8 projections N(0, 0.5) with scales U(1, 3) / sqrt(K), MXFP4 nibbles uniform with
    exponent bytes 116..120 (weight RMS about 0.012, near 1 / sqrt(K), which keeps the MLP's outputs O(1) at
    K = 4096 and 12288 as the FP8 scales do for the projections), norms 1 + N(0, 0.1), KV ~ N(0, 1) bf16, GDN state ~ N(0, 0.02),
    x ~ N(0, 1).
    Every sequence holds ctx tokens; the step's new token is position ctx (a fresh page per sequence)."""
    c4 = dict(CONFIG4)
    if ctx is not None:
        c4["ctx"] = ctx
    if batch is not None:
        c4["batch"] = batch
    b, h, f, d, hkv, page = c4["batch"], c4["hidden"], c4["inter"], c4["d"], c4["hkv"], c4["page"]
    nk, nv, hq = c4["nk"], c4["nv"], c4["hq"]
    g = torch.Generator(device=dev).manual_seed(seed)

    def fp8(n, k):
        w = (torch.randn(n, k, generator=g, device=dev) * 0.5).to(torch.float8_e4m3fn).view(torch.uint8)
        return w.contiguous(), (torch.rand(n, generator=g, device=dev) * 2 + 1) / (k ** 0.5)

    def mx(n, k):
        codes = torch.randint(0, 256, (n, k // 2), generator=g, device=dev, dtype=torch.uint8)
        scales = torch.randint(116, 121, (n, k // 32), generator=g, device=dev, dtype=torch.uint8)
        return codes, scales

    def norm(n):
        return 1.0 + 0.1 * torch.randn(n, generator=g, device=dev)

    def mlp():
        w = {}
        w["w_gate"], w["s_gate"] = mx(f, h)
        w["w_up"], w["s_up"] = mx(f, h)
        w["w_down"], w["s_down"] = mx(h, f)
        return w

    kd, vd = nk * 128, nv * 128
    pages_per_seq = c4["ctx"] // page + 1  # + the new token's page (ctx is a multiple of the page)
    pool = b * pages_per_seq
    perm = torch.randperm(pool, generator=g, device=dev).to(torch.int32)
    indptr = (torch.arange(b + 1, device=dev, dtype=torch.int32) * pages_per_seq).contiguous()
    last = torch.full((b,), c4["ctx"] % page + 1, dtype=torch.int32, device=dev)
    loc = torch.stack([perm[indptr[1:].long() - 1], torch.full((b,), c4["ctx"] % page, dtype=torch.int32,
                                                               device=dev)], 1).to(torch.int32).contiguous()
    layers = []
    for kind in c4["pattern"]:
        if kind == "g":
            w = {"ln1": norm(h)}
            w["w_qkv"], w["s_qkv"] = fp8(2 * kd + vd, h)
            w["w_z"], w["s_z"] = fp8(vd, h)
            w["w_b"], w["s_b"] = fp8(nv, h)
            w["w_a"], w["s_a"] = fp8(nv, h)
            w["conv_w"] = (torch.randn(2 * kd + vd, c4["conv"], generator=g, device=dev) * 0.5).to(torch.bfloat16)
            w["a_log"] = torch.randn(nv, generator=g, device=dev) * 0.5
            w["dt_bias"] = torch.randn(nv, generator=g, device=dev) * 0.5
            w["norm_w"] = norm(128)
            w["w_out"], w["s_out"] = fp8(h, vd)
            w["ln2"] = norm(h)
            w.update(mlp())
            st = torch.randn(b, nv, 128, 128, generator=g, device=dev) * 0.02
            cv = torch.randn(b, c4["conv"] - 1, 2 * kd + vd, generator=g, device=dev).to(torch.bfloat16)
            layers.append({"kind": "g", "w": w, "state": st, "conv": cv})
        else:
            w = {"ln1": norm(h)}
            w["w_q"], w["s_q"] = fp8(hq * 2 * d, h)
            w["w_k"], w["s_k"] = fp8(hkv * d, h)
            w["w_v"], w["s_v"] = fp8(hkv * d, h)
            w["q_norm"] = norm(d)
            w["k_norm"] = norm(d)
            w["w_o"], w["s_o"] = fp8(h, hq * d)
            w["ln2"] = norm(h)
            w.update(mlp())
            cache = torch.randn(pool, 2, page, hkv, d, generator=g, device=dev, dtype=torch.bfloat16)
            layers.append({"kind": "a", "w": w, "cache": cache})
    inv = 1.0 / (c4["theta"] ** (torch.arange(0, c4["rot"], 2, dtype=torch.int64).float() / c4["rot"]))
    fpos = float(c4["ctx"]) * inv
    cos = fpos.cos().bfloat16().reshape(1, -1).repeat(b, 1).to(dev).contiguous()
    sin = fpos.sin().bfloat16().reshape(1, -1).repeat(b, 1).to(dev).contiguous()
    x = torch.randn(b, h, generator=g, device=dev).to(torch.bfloat16)
    return {"cfg": c4, "layers": layers, "indptr": indptr, "indices": perm, "last_page_len": last, "loc": loc,
            "cos": cos, "sin": sin, "x": x}


# The 35B's MoE decode group (qwen35moe_group8_gggaggga_mx8_kvc_c16384 of the 35B manifest, built by
# models/qwen35_35b_a3b/src/70b0fbc/q35_moe_group.py): 8 layers (GDN, GDN, GDN, attention) x 2, hidden 2048,
# MXFP8 projections and shared expert (inter 512), 256 MXFP4 routed experts of 512, top-8, GDN 16 / 32 heads,
# attention HQ 16 / HKV 2 / D 256 (the manifest's w_q [8192, 2048] = 16 heads of [q | gate], kc [16384, 512]),
# rot 64; the reference's 16,384-token cache, here per sequence at a batch of 32 (config 3a's decode batch).
MOE_GROUP = dict(batch=32, ctx=16383, hidden=2048, inter=512, experts=256, expert_inter=512, top_k=8, hq=16, hkv=2,
                 d=256, rot=64, nk=16, nv=32, conv=4, page=64, theta=10_000_000.0, eps=1e-6, pattern="gggaggga")


def moe_group(dev, seed: int = 0, ctx: int | None = None, batch: int | None = None,
              pattern: str | None = None) -> dict:
    """The MoE group's weights, states, paged KV caches and page table, generated ON THE DEVICE by a seeded device
    generator. Distributions as the small-shape generators: MXFP8 projections and shared expert as proj_weight
    ("mxfp8": E4M3 codes of N(0, 3^2), E8M0 bytes uniform in 119..123), routed experts as moe_block (MXFP4 nibbles
    uniform, E8M0 bytes 119..123), bf16 router and shared-expert gate N(0, 0.02), norms 1 + N(0, 0.1), conv taps
    N(0, 0.5^2) bf16, A_log and dt_bias N(0, 0.5^2), KV ~ N(0, 1) bf16, GDN state ~ N(0, 0.02^2), x ~ N(0, 1).
    Every sequence holds ctx tokens before the step; the step's token is position ctx, in the page that holds it
    (a fresh page when ctx is a multiple of the page size). Returns {"cfg", "layers" (DecodeGroup's layer dicts),
    "attn" (cos, sin, indptr, indices, last_page_len, loc), "x"}."""
    cg = dict(MOE_GROUP)
    for k, v in (("ctx", ctx), ("batch", batch), ("pattern", pattern)):
        if v is not None:
            cg[k] = v
    b, h, f, fe, ne = cg["batch"], cg["hidden"], cg["inter"], cg["expert_inter"], cg["experts"]
    d, hkv, hq, page, nk, nv = cg["d"], cg["hkv"], cg["hq"], cg["page"], cg["nk"], cg["nv"]
    g = torch.Generator(device=dev).manual_seed(seed)

    def mx8(n, k):
        codes = (torch.randn(n, k, generator=g, device=dev) * 3).to(torch.float8_e4m3fn).view(torch.uint8)
        return codes.contiguous(), torch.randint(119, 124, (n, k // 32), generator=g, device=dev, dtype=torch.uint8)

    def mx4(lead, n, k):
        codes = torch.randint(0, 256, (lead, n, k // 2), generator=g, device=dev, dtype=torch.uint8)
        return codes, torch.randint(119, 124, (lead, n, k // 32), generator=g, device=dev, dtype=torch.uint8)

    def norm(n):
        return 1.0 + 0.1 * torch.randn(n, generator=g, device=dev)

    def bf16(*shape, std=1.0):
        return (torch.randn(*shape, generator=g, device=dev) * std).to(torch.bfloat16)

    def mlp_and_moe(w):
        w["w_gate"], w["s_gate"] = mx8(f, h)
        w["w_up"], w["s_up"] = mx8(f, h)
        w["w_down"], w["s_down"] = mx8(h, f)
        m = {"w_router": bf16(ne, h, std=0.02), "w_shg": bf16(h, std=0.02)}
        m["e_gw"], m["e_gs"] = mx4(ne, 2 * fe, h)
        m["e_dw"], m["e_ds"] = mx4(ne, h, fe)
        m["top_k"] = cg["top_k"]
        return m

    kd, vd = nk * 128, nv * 128
    pages_per_seq = cg["ctx"] // page + 1  # the pages up to and including the one holding position ctx
    pool = b * pages_per_seq
    perm = torch.randperm(pool, generator=g, device=dev).to(torch.int32)
    indptr = (torch.arange(b + 1, device=dev, dtype=torch.int32) * pages_per_seq).contiguous()
    last = torch.full((b,), cg["ctx"] % page + 1, dtype=torch.int32, device=dev)
    loc = torch.stack([perm[indptr[1:].long() - 1], torch.full((b,), cg["ctx"] % page, dtype=torch.int32,
                                                               device=dev)], 1).to(torch.int32).contiguous()
    layers = []
    for kind in cg["pattern"]:
        w = {"ln1": norm(h)}
        if kind == "g":
            w["w_qkv"], w["s_qkv"] = mx8(2 * kd + vd, h)
            w["w_z"], w["s_z"] = mx8(vd, h)
            w["w_b"], w["s_b"] = mx8(nv, h)
            w["w_a"], w["s_a"] = mx8(nv, h)
            w["conv_w"] = bf16(2 * kd + vd, cg["conv"], std=0.5)
            w["a_log"] = torch.randn(nv, generator=g, device=dev) * 0.5
            w["dt_bias"] = torch.randn(nv, generator=g, device=dev) * 0.5
            w["norm_w"] = norm(128)
            w["w_out"], w["s_out"] = mx8(h, vd)
            w["ln2"] = norm(h)
            m = mlp_and_moe(w)
            st = torch.randn(b, nv, 128, 128, generator=g, device=dev) * 0.02
            cv = bf16(b, cg["conv"] - 1, 2 * kd + vd)
            layers.append({"kind": "g", "w": w, "moe": m, "state": st, "conv": cv})
        else:
            w["w_q"], w["s_q"] = mx8(hq * 2 * d, h)
            w["w_k"], w["s_k"] = mx8(hkv * d, h)
            w["w_v"], w["s_v"] = mx8(hkv * d, h)
            w["q_norm"] = norm(d)
            w["k_norm"] = norm(d)
            w["w_o"], w["s_o"] = mx8(h, hq * d)
            w["ln2"] = norm(h)
            m = mlp_and_moe(w)
            cache = torch.randn(pool, 2, page, hkv, d, generator=g, device=dev, dtype=torch.bfloat16)
            layers.append({"kind": "a", "w": w, "moe": m, "cache": cache})
    inv = 1.0 / (cg["theta"] ** (torch.arange(0, cg["rot"], 2, dtype=torch.int64).float() / cg["rot"]))
    fpos = float(cg["ctx"]) * inv
    cos = fpos.cos().bfloat16().reshape(1, -1).repeat(b, 1).to(dev).contiguous()
    sin = fpos.sin().bfloat16().reshape(1, -1).repeat(b, 1).to(dev).contiguous()
    x = bf16(b, h)
    attn = {"cos": cos, "sin": sin, "indptr": indptr, "indices": perm, "last_page_len": last, "loc": loc}
    return {"cfg": cg, "layers": layers, "attn": attn, "x": x}
