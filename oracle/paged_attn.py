"""Oracle: paged decode attention and the paged KV write (CPU, test infrastructure only).

Restates
  * the paged SDPA golden of models/qwen35_35b_a3b/sgl/tests/test_qwen35_runtime.py:73-84: gather the
    history rows of the sequence's pages (cache[rows, 0/1].reshape(-1, HKV, D)[:L]) and run fp32
    softmax(q K^T * scale) V with GQA (query head h uses KV head h // (HQ / HKV));
  * the page-table semantics of sgl_kernel_axera/attention/flash_attn.py:1478-1495 (physical page =
    indices[indptr[b] + logical page]) and the tail mask of 87-104 (tokens past the valid length of the
    last page are excluded);
  * store_paged_kv of flash_attn.py:53-84 (row = (page * 2 + plane) * page_size + offset);
  * the 8-bit caches of models/qwen38_27b/decode/q35_group.py: FP8 with a static scale (KV8=2, 244-247) and INT8
    with a bf16 scale per row and head (KV8=1: kv_quant_row 197-205, kv_page 208-221, kv_write_paged 250-255).
Pinned by tests/test_oracle_paged.py: torch SDPA (enable_gqa=True, the reference's golden call) on the
same gathered rows, a brute-force per-token index computation of the gather, invariance under a
consistent permutation of the page pool, and the one-page case against dense attention; the INT8 quantizer by its
error bound (|x - bf16(q s)| <= s / 2 plus the bf16 roundings), the row maximum on +-127 (126 or 128 clipped only by
the bf16 rounding of s and 1 / s), the 1e-5 floor for zero rows, and exactness where x is already a multiple of s.
"""
from __future__ import annotations

import numpy as np
import torch


def seq_lens(indptr, last_page_len, page_size: int) -> list[int]:
    ip = np.asarray(indptr)
    lp = np.asarray(last_page_len)
    out = []
    for b in range(len(lp)):
        n = int(ip[b + 1] - ip[b])
        out.append(0 if n == 0 else (n - 1) * page_size + int(lp[b]))
    return out


def gather_kv(cache: torch.Tensor, indptr, indices, last_page_len, b: int):
    """K, V rows [L, HKV, D] of sequence b, in token order (flash_attn.py:1478-1495)."""
    page_size = cache.shape[2]
    ip = np.asarray(indptr)
    rows = torch.as_tensor(np.asarray(indices)[ip[b]:ip[b + 1]], dtype=torch.long)
    L = seq_lens(indptr, last_page_len, page_size)[b]
    k = cache[rows, 0].reshape(-1, cache.shape[3], cache.shape[4])[:L]
    v = cache[rows, 1].reshape(-1, cache.shape[3], cache.shape[4])[:L]
    return k, v


def paged_decode(q: torch.Tensor, cache: torch.Tensor, indptr, indices, last_page_len, sm_scale: float) -> torch.Tensor:
    """fp32 [B, HQ, D]; a sequence without tokens yields zeros."""
    bsz, hq, d = q.shape
    hkv = cache.shape[3]
    grp = hq // hkv
    out = torch.zeros(bsz, hq, d, dtype=torch.float32)
    for b in range(bsz):
        k, v = gather_kv(cache, indptr, indices, last_page_len, b)
        if k.shape[0] == 0:
            continue
        kf = k.float().repeat_interleave(grp, dim=1)  # [L, HQ, D]
        vf = v.float().repeat_interleave(grp, dim=1)
        s = torch.einsum("hd,lhd->hl", q[b].float(), kf) * sm_scale
        p = torch.softmax(s, dim=-1)
        out[b] = torch.einsum("hl,lhd->hd", p, vf)
    return out


def paged_prefill(q: torch.Tensor, cache: torch.Tensor, qo_indptr, indptr, indices, last_page_len,
                  sm_scale: float) -> torch.Tensor:
    """fp32 [T, HQ, D]: the new tokens of sequence b (rows qo_indptr[b] .. qo_indptr[b+1] of q) are its last qlen
    cached tokens; token t attends cached positions 0 .. L - qlen + t (the causal current block over the history,
    flash_attn.py:484-486; q35_prefill.py:264-300 builds the same additive mask). A row that sees nothing yields 0."""
    t_all, hq, d = q.shape
    hkv = cache.shape[3]
    grp = hq // hkv
    qi = np.asarray(qo_indptr)
    out = torch.zeros(t_all, hq, d, dtype=torch.float32)
    for b in range(len(qi) - 1):
        q0, qlen = int(qi[b]), int(qi[b + 1] - qi[b])
        if qlen <= 0:
            continue
        k, v = gather_kv(cache, indptr, indices, last_page_len, b)
        L = k.shape[0]
        kf = k.float().repeat_interleave(grp, dim=1).permute(1, 0, 2)  # [HQ, L, D]
        vf = v.float().repeat_interleave(grp, dim=1).permute(1, 0, 2)
        qf = q[q0:q0 + qlen].float().permute(1, 0, 2)  # [HQ, qlen, D]
        s = torch.matmul(qf, kf.transpose(1, 2)) * sm_scale  # [HQ, qlen, L]
        pos = torch.arange(qlen).reshape(-1, 1) + (L - qlen)
        s = s.masked_fill(torch.arange(L).reshape(1, -1) > pos, float("-inf"))
        seen = (pos >= 0).reshape(1, -1, 1) & (L > 0)
        p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0) * seen
        out[q0:q0 + qlen] = torch.matmul(p, vf).permute(1, 0, 2)
    return out


def store_paged_kv_(cache: torch.Tensor, k: torch.Tensor, v: torch.Tensor, loc) -> torch.Tensor:
    """Writes k[b] / v[b] at (page, offset) = loc[b] of cache in place and returns it (flash_attn.py:53-84)."""
    loc = np.asarray(loc).reshape(-1, 2)
    for b in range(k.shape[0]):
        page, off = int(loc[b, 0]), int(loc[b, 1])
        cache[page, 0, off] = k[b]
        cache[page, 1, off] = v[b]
    return cache


def store_paged_kv(cache: torch.Tensor, k: torch.Tensor, v: torch.Tensor, loc) -> torch.Tensor:
    """Returns a copy of cache with k[b] / v[b] written at (page, offset) = loc[b] (flash_attn.py:53-84)."""
    return store_paged_kv_(cache.clone(), k, v, loc)


def quant_kv_fp8(x: torch.Tensor, kv_scale: float) -> torch.Tensor:
    """The FP8 cache's stored bytes: e4m3(bf16(x * kv_scale)) as u8 (kv_write_paged with KV8=2,
    models/qwen38_27b/decode/q35_group.py:244-247: a bf16 multiply, then the cast to fp8_e4m3)."""
    return (x.float() * kv_scale).to(torch.bfloat16).float().to(torch.float8_e4m3fn).view(torch.uint8)


def dequant_kv_fp8(codes: torch.Tensor, kv_scale: float) -> torch.Tensor:
    """The values attention reads from an FP8 cache: stored / kv_scale (q35_group.py:48-51: K through a constant
    E8M0 scale of 1 / KV8_SCALE, V with the probabilities carrying it), exact in bf16 for a power-of-two scale."""
    return (codes.view(torch.float8_e4m3fn).float() / kv_scale).to(torch.bfloat16)


# ---- INT8 cache with a bf16 scale per row and KV head (models/qwen38_27b/decode/q35_group.py:44-47, KV8=1) ----
_BF16_1E5 = float(torch.tensor(1e-5).to(torch.bfloat16))        # the floor of amax, a bf16 constant
_BF16_INV127 = float(torch.tensor(1.0 / 127).to(torch.bfloat16))  # bf16(1 / 127)


def quant_kv_i8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """kv_quant_row (q35_group.py:197-205) for rows x bf16 [..., D]: amax = max(max |x|, bf16(1e-5)); s = bf16(amax *
    bf16(1 / 127)); codes = int8(bf16(x * bf16(1 / s))). Each product in fp32 then rounded to bf16 (the DSL's bf16
    outputs); the int8 cast rounds to nearest even and saturates (the AX cast's rounding of ties and its saturation are
    not stated in the reference: parity unpinned there). Returns (codes int8 [..., D], s bf16 [...])."""
    xf = x.float()
    amax = torch.clamp(xf.abs().amax(dim=-1), min=_BF16_1E5)
    s = (amax * _BF16_INV127).to(torch.bfloat16)
    r = (1.0 / s.float()).to(torch.bfloat16)
    y = (xf * r.float()[..., None]).to(torch.bfloat16).float()
    codes = torch.clamp(torch.round(y), -128, 127).to(torch.int8)
    return codes, s


def dequant_kv_i8(codes: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """kv_page's dequantization (q35_group.py:218-220): bf16(q * s) per row and head."""
    return (codes.float() * s.float()[..., None]).to(torch.bfloat16)


def store_paged_kv_i8(cache: torch.Tensor, scales: torch.Tensor, k: torch.Tensor, v: torch.Tensor, loc):
    """kv_write_paged with kvs (q35_group.py:250-255): rows of k / v [B, HKV, D] quantized into cache int8
    [P, 2, page, HKV, D] and scales bf16 [P, 2, page, HKV] at loc [B, 2] = (page, slot). Returns new tensors."""
    cache, scales = cache.clone(), scales.clone()
    for plane, x in ((0, k), (1, v)):
        codes, s = quant_kv_i8(x)
        for b, (pg, off) in enumerate(np.asarray(loc).reshape(-1, 2).tolist()):
            cache[pg, plane, off] = codes[b]
            scales[pg, plane, off] = s[b]
    return cache, scales
