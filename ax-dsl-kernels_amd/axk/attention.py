"""Paged decode attention and the paged KV write on gfx950.

Mirrors the paged-KV part of sgl_kernel_axera.attention.flash_attn
(models/qwen35_35b_a3b/sgl/python/sgl_kernel_axera/attention/flash_attn.py): cache
[pages, 2, page_size, HKV, D] bf16, FlashInfer-style indptr / indices / last_page_len page tables
(flash_attn.py:2549-2665) and store_paged_kv's cache_location = [page, offset] (53-84). Like the
reference, the operator allocates nothing it is not asked to: pass ``workspace`` (see
``paged_decode_workspace``) to keep calls allocation-free.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def paged_decode_workspace(batch: int, num_qo_heads: int, num_kv_heads: int, head_dim: int,
                           device) -> torch.Tensor:
    """A byte buffer large enough for paged_decode with this configuration."""
    n = _lib.load().axk_paged_decode_workspace_size(batch, num_qo_heads, num_kv_heads, head_dim)
    _check(n > 0, "invalid paged decode configuration")
    return torch.empty(n, dtype=torch.uint8, device=device)


def _check_decode(q, kv_cache, indptr, indices, last_page_len, kv_dtype=torch.bfloat16):
    _check(q.dim() == 3 and q.dtype == torch.bfloat16 and q.is_contiguous(), "q must be contiguous bf16 [B, HQ, D]")
    _check(kv_cache.dim() == 5 and kv_cache.dtype == kv_dtype and kv_cache.is_contiguous(),
           f"kv_cache must be contiguous {kv_dtype} [pages, 2, page_size, HKV, D]")
    b, hq, d = q.shape
    p, two, page, hkv, d2 = kv_cache.shape
    _check(two == 2 and d2 == d, f"kv_cache shape {tuple(kv_cache.shape)} does not match q {tuple(q.shape)}")
    _check(hq % hkv == 0 and hq // hkv <= 16, f"num_qo_heads {hq} must be a multiple (<= 16x) of num_kv_heads {hkv}")
    _check(d in (64, 128, 256), f"head_dim {d} not supported (64, 128, 256)")
    _check(page % 16 == 0 and page <= 4096, f"page_size {page} must be a multiple of 16, at most 4096")
    for name, t, n in (("indptr", indptr, b + 1), ("last_page_len", last_page_len, b)):
        _check(t.dtype == torch.int32 and t.dim() == 1 and t.numel() == n and t.is_contiguous(),
               f"{name} must be contiguous int32 [{n}]")
    _check(indices.dtype == torch.int32 and indices.dim() == 1 and indices.is_contiguous(),
           "indices must be contiguous int32 [nnz]")
    return b, hq, hkv, d, page, p


def paged_decode_plan(indptr: torch.Tensor, last_page_len: torch.Tensor, num_qo_heads: int, num_kv_heads: int,
                      head_dim: int, page_size: int, workspace: torch.Tensor) -> None:
    """Compute the split-KV partition for this page-table shape into ``workspace`` (once per decode step)."""
    b = indptr.numel() - 1
    _check(indptr.dtype == torch.int32 and indptr.dim() == 1 and b > 0, "indptr must be int32 [B+1]")
    _check(last_page_len.dtype == torch.int32 and last_page_len.numel() == b, "last_page_len must be int32 [B]")
    _lib.require_device(indptr, last_page_len, workspace)
    _lib.call("axk_paged_decode_plan", indptr.data_ptr(), last_page_len.data_ptr(), b, num_qo_heads, num_kv_heads,
              head_dim, page_size, workspace.data_ptr(), workspace.numel(), _lib.stream_of(indptr))


def paged_decode_run(q, kv_cache, indptr, indices, last_page_len, workspace, sm_scale=None, output=None):
    """Decode attention with a plan already in ``workspace`` (see paged_decode_plan)."""
    b, hq, hkv, d, page, p = _check_decode(q, kv_cache, indptr, indices, last_page_len)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    if output is None:
        output = torch.empty_like(q)
    _check(output.shape == q.shape and output.dtype == q.dtype and output.is_contiguous(), "bad output tensor")
    _lib.require_device(q, kv_cache, indptr, indices, last_page_len, output, workspace)
    _lib.call(
        "axk_paged_decode_run", q.data_ptr(), kv_cache.data_ptr(), indptr.data_ptr(), indices.data_ptr(),
        last_page_len.data_ptr(), output.data_ptr(), b, hq, hkv, d, page, p, float(sm_scale),
        workspace.data_ptr(), workspace.numel(), _lib.stream_of(q),
    )
    return output


def paged_decode(
    q: torch.Tensor,
    kv_cache: torch.Tensor,
    indptr: torch.Tensor,
    indices: torch.Tensor,
    last_page_len: torch.Tensor,
    sm_scale: Optional[float] = None,
    output: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """One decode token per sequence attends all valid tokens of its pages.

    q [B, HQ, D] bf16; kv_cache [P, 2, page, HKV, D] bf16; indptr [B+1], indices [nnz],
    last_page_len [B] int32 (1..page; tokens in the last page). Returns bf16 [B, HQ, D].
    """
    b, hq, hkv, d, page, p = _check_decode(q, kv_cache, indptr, indices, last_page_len)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    if output is None:
        output = torch.empty_like(q)
    _check(output.shape == q.shape and output.dtype == q.dtype and output.is_contiguous(), "bad output tensor")
    if workspace is None:
        workspace = paged_decode_workspace(b, hq, hkv, d, q.device)
    _lib.require_device(q, kv_cache, indptr, indices, last_page_len, output, workspace)
    _lib.call(
        "axk_paged_decode", q.data_ptr(), kv_cache.data_ptr(), indptr.data_ptr(), indices.data_ptr(),
        last_page_len.data_ptr(), output.data_ptr(), b, hq, hkv, d, page, p, float(sm_scale),
        workspace.data_ptr(), workspace.numel(), _lib.stream_of(q),
    )
    return output


def paged_attention_decode(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    kv_cache: torch.Tensor,
    indptr: torch.Tensor,
    indices: torch.Tensor,
    last_page_len: torch.Tensor,
    cache_location: torch.Tensor,
    sm_scale: Optional[float] = None,
    output: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
    status: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Decode attention in the sgl operator's page-table convention (flash_attn.py:2335-2357, 1421-1596): writes the
    current token's k, v ([B, HKV, D] bf16) at cache_location[b] = (page, offset), then q attends the history
    ((pages - 1) * page_size + last_page_len[b] tokens, last_page_len counting history only, 0 .. page - 1) plus the
    current token. The page list already holds the current token's page. Returns bf16 [B, HQ, D]."""
    b, hq, hkv, d, page, p = _check_decode(q, kv_cache, indptr, indices, last_page_len)
    _check(k.shape == (b, hkv, d) and v.shape == k.shape and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16
           and k.is_contiguous() and v.is_contiguous(), f"k and v must be contiguous bf16 [{b}, {hkv}, {d}]")
    loc = cache_location.reshape(-1, 2) if cache_location.numel() == 2 * b else None
    _check(loc is not None and cache_location.dtype == torch.int32 and loc.is_contiguous(),
           "cache_location must be int32 [B, 2] = (page, offset)")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    if output is None:
        output = torch.empty_like(q)
    _check(output.shape == q.shape and output.dtype == q.dtype and output.is_contiguous(), "bad output tensor")
    if workspace is None:
        workspace = paged_decode_workspace(b, hq, hkv, d, q.device)
    _lib.require_device(q, k, v, kv_cache, indptr, indices, last_page_len, loc, output, workspace, status)
    _lib.call(
        "axk_paged_attention_decode", q.data_ptr(), k.data_ptr(), v.data_ptr(), kv_cache.data_ptr(),
        indptr.data_ptr(), indices.data_ptr(), last_page_len.data_ptr(), loc.data_ptr(), output.data_ptr(), b, hq,
        hkv, d, page, p, float(sm_scale), _lib.ptr(status), workspace.data_ptr(), workspace.numel(),
        _lib.stream_of(q),
    )
    return output


def store_paged_kv(k: torch.Tensor, v: torch.Tensor, kv_cache: torch.Tensor, cache_location: torch.Tensor,
                   status: Optional[torch.Tensor] = None) -> None:
    """Write k[b], v[b] ([B, HKV, D] bf16) at cache_location[b] = (page, offset) in place (flash_attn.py:53-84)."""
    _check(k.shape == v.shape and k.dim() == 3 and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16,
           "k and v must be bf16 [B, HKV, D]")
    _check(k.is_contiguous() and v.is_contiguous() and kv_cache.is_contiguous(), "tensors must be contiguous")
    b, hkv, d = k.shape
    p, two, page, hkv2, d2 = kv_cache.shape
    _check(two == 2 and hkv2 == hkv and d2 == d, "kv_cache shape does not match k / v")
    loc = cache_location.reshape(-1, 2) if cache_location.numel() == 2 * b else None
    _check(loc is not None and cache_location.dtype == torch.int32 and loc.is_contiguous(),
           "cache_location must be int32 [B, 2] = (page, offset)")
    _lib.require_device(k, v, kv_cache, loc, status)
    _lib.call(
        "axk_paged_kv_write", k.data_ptr(), v.data_ptr(), kv_cache.data_ptr(), loc.data_ptr(), b, hkv, d, page, p,
        _lib.ptr(status), _lib.stream_of(k),
    )


def _check_kv_scale(kv_scale: float) -> None:
    m, e = math.frexp(kv_scale)
    _check(kv_scale > 0 and m == 0.5, f"kv_scale {kv_scale} must be a power of two")


def paged_decode_fp8(
    q: torch.Tensor,
    kv_cache: torch.Tensor,
    indptr: torch.Tensor,
    indices: torch.Tensor,
    last_page_len: torch.Tensor,
    kv_scale: float,
    sm_scale: Optional[float] = None,
    output: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """paged_decode over an FP8 cache (q35_group.py:44-54, KV8=2): kv_cache u8 (or float8_e4m3fn) [P, 2, page, HKV,
    D] holding e4m3(bf16(x * kv_scale)); attention reads stored / kv_scale. kv_scale: a power of two; D 128 or 256."""
    if kv_cache.dtype == torch.float8_e4m3fn:
        kv_cache = kv_cache.view(torch.uint8)
    _check(kv_cache.dtype == torch.uint8, "kv_cache must be u8 / float8_e4m3fn")
    b, hq, hkv, d, page, p = _check_decode(q, kv_cache, indptr, indices, last_page_len, kv_dtype=torch.uint8)
    _check(d in (128, 256), f"head_dim {d} not supported with an FP8 cache (128, 256)")
    _check_kv_scale(kv_scale)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    if output is None:
        output = torch.empty_like(q)
    _check(output.shape == q.shape and output.dtype == q.dtype and output.is_contiguous(), "bad output tensor")
    if workspace is None:
        workspace = paged_decode_workspace(b, hq, hkv, d, q.device)
    _lib.require_device(q, kv_cache, indptr, indices, last_page_len, output, workspace)
    _lib.call(
        "axk_paged_decode_fp8", q.data_ptr(), kv_cache.data_ptr(), indptr.data_ptr(), indices.data_ptr(),
        last_page_len.data_ptr(), output.data_ptr(), b, hq, hkv, d, page, p, float(sm_scale), float(kv_scale),
        workspace.data_ptr(), workspace.numel(), _lib.stream_of(q),
    )
    return output


def store_paged_kv_fp8(k: torch.Tensor, v: torch.Tensor, kv_cache: torch.Tensor, cache_location: torch.Tensor,
                       kv_scale: float, status: Optional[torch.Tensor] = None) -> None:
    """store_paged_kv into an FP8 cache: the bytes at cache_location[b] become e4m3(bf16(x * kv_scale)) for
    x = k[b] (plane 0) and v[b] (plane 1) (q35_group.py:244-247)."""
    if kv_cache.dtype == torch.float8_e4m3fn:
        kv_cache = kv_cache.view(torch.uint8)
    _check(k.shape == v.shape and k.dim() == 3 and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16,
           "k and v must be bf16 [B, HKV, D]")
    _check(kv_cache.dtype == torch.uint8 and kv_cache.dim() == 5, "kv_cache must be u8 [P, 2, page, HKV, D]")
    _check(k.is_contiguous() and v.is_contiguous() and kv_cache.is_contiguous(), "tensors must be contiguous")
    _check_kv_scale(kv_scale)
    b, hkv, d = k.shape
    p, two, page, hkv2, d2 = kv_cache.shape
    _check(two == 2 and hkv2 == hkv and d2 == d, "kv_cache shape does not match k / v")
    loc = cache_location.reshape(-1, 2) if cache_location.numel() == 2 * b else None
    _check(loc is not None and cache_location.dtype == torch.int32 and loc.is_contiguous(),
           "cache_location must be int32 [B, 2] = (page, offset)")
    _lib.require_device(k, v, kv_cache, loc, status)
    _lib.call(
        "axk_paged_kv_write_fp8", k.data_ptr(), v.data_ptr(), kv_cache.data_ptr(), loc.data_ptr(), b, hkv, d, page,
        p, float(kv_scale), _lib.ptr(status), _lib.stream_of(k),
    )


def paged_decode_i8(
    q: torch.Tensor,
    kv_cache: torch.Tensor,
    kv_scales: torch.Tensor,
    indptr: torch.Tensor,
    indices: torch.Tensor,
    last_page_len: torch.Tensor,
    sm_scale: Optional[float] = None,
    output: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """paged_decode over an INT8 cache (q35_group.py:44-47, 208-221, KV8=1): kv_cache int8 [P, 2, page, HKV, D],
    kv_scales bf16 [P, 2, page, HKV]; attention reads bf16(q * s). D 128 or 256, HKV <= 16."""
    b, hq, hkv, d, page, p = _check_decode(q, kv_cache, indptr, indices, last_page_len, kv_dtype=torch.int8)
    _check(d in (128, 256) and hkv <= 16, f"head_dim {d} / num_kv_heads {hkv} not supported with an INT8 cache")
    _check(kv_scales.dtype == torch.bfloat16 and tuple(kv_scales.shape) == (p, 2, page, hkv) and
           kv_scales.is_contiguous(), "kv_scales must be contiguous bf16 [P, 2, page, HKV]")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    if output is None:
        output = torch.empty_like(q)
    _check(output.shape == q.shape and output.dtype == q.dtype and output.is_contiguous(), "bad output tensor")
    if workspace is None:
        workspace = paged_decode_workspace(b, hq, hkv, d, q.device)
    _lib.require_device(q, kv_cache, kv_scales, indptr, indices, last_page_len, output, workspace)
    _lib.call(
        "axk_paged_decode_i8", q.data_ptr(), kv_cache.data_ptr(), kv_scales.data_ptr(), indptr.data_ptr(),
        indices.data_ptr(), last_page_len.data_ptr(), output.data_ptr(), b, hq, hkv, d, page, p, float(sm_scale),
        workspace.data_ptr(), workspace.numel(), _lib.stream_of(q),
    )
    return output


def store_paged_kv_i8(k: torch.Tensor, v: torch.Tensor, kv_cache: torch.Tensor, kv_scales: torch.Tensor,
                      cache_location: torch.Tensor, status: Optional[torch.Tensor] = None) -> None:
    """store_paged_kv into an INT8 cache (kv_write_paged with kvs, q35_group.py:250-255): each row and head of k[b]
    (plane 0) and v[b] (plane 1) quantized as kv_quant_row (197-205) into kv_cache at cache_location[b], its scale
    into kv_scales."""
    _check(k.shape == v.shape and k.dim() == 3 and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16,
           "k and v must be bf16 [B, HKV, D]")
    _check(kv_cache.dtype == torch.int8 and kv_cache.dim() == 5, "kv_cache must be int8 [P, 2, page, HKV, D]")
    _check(k.is_contiguous() and v.is_contiguous() and kv_cache.is_contiguous() and kv_scales.is_contiguous(),
           "tensors must be contiguous")
    b, hkv, d = k.shape
    p, two, page, hkv2, d2 = kv_cache.shape
    _check(two == 2 and hkv2 == hkv and d2 == d and d in (128, 256), "kv_cache shape does not match k / v")
    _check(kv_scales.dtype == torch.bfloat16 and tuple(kv_scales.shape) == (p, 2, page, hkv),
           "kv_scales must be bf16 [P, 2, page, HKV]")
    loc = cache_location.reshape(-1, 2) if cache_location.numel() == 2 * b else None
    _check(loc is not None and cache_location.dtype == torch.int32 and loc.is_contiguous(),
           "cache_location must be int32 [B, 2] = (page, offset)")
    _lib.require_device(k, v, kv_cache, kv_scales, loc, status)
    _lib.call(
        "axk_paged_kv_write_i8", k.data_ptr(), v.data_ptr(), kv_cache.data_ptr(), kv_scales.data_ptr(),
        loc.data_ptr(), b, hkv, d, page, p, _lib.ptr(status), _lib.stream_of(k),
    )


def paged_prefill(
    q: torch.Tensor,
    kv_cache: torch.Tensor,
    qo_indptr: torch.Tensor,
    indptr: torch.Tensor,
    indices: torch.Tensor,
    last_page_len: torch.Tensor,
    sm_scale: Optional[float] = None,
    output: Optional[torch.Tensor] = None,
    status: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Causal attention of several new tokens per sequence over the paged cache (prefill chunks, speculative verify):
    q bf16 [T, HQ, D] holds sequence b's new tokens in rows qo_indptr[b] .. qo_indptr[b + 1]; their K / V are already
    in the cache as the sequence's last tokens, so new token t of a sequence of kv_len cached tokens sees positions
    0 .. kv_len - qlen + t (flash_attn.py:471-611, q35_prefill.py:264-336). Returns bf16 [T, HQ, D]. A page id
    outside the pool or a query range outside q sets status (device int32 [1], if given) to 1."""
    _check(q.dim() == 3 and q.dtype == torch.bfloat16 and q.is_contiguous(), "q must be contiguous bf16 [T, HQ, D]")
    _check(kv_cache.dim() == 5 and kv_cache.dtype == torch.bfloat16 and kv_cache.is_contiguous(),
           "kv_cache must be contiguous bf16 [pages, 2, page_size, HKV, D]")
    t, hq, d = q.shape
    p, two, page, hkv, d2 = kv_cache.shape
    _check(two == 2 and d2 == d, f"kv_cache shape {tuple(kv_cache.shape)} does not match q {tuple(q.shape)}")
    _check(hq % hkv == 0, f"num_qo_heads {hq} must be a multiple of num_kv_heads {hkv}")
    _check(d in (64, 128, 256), f"head_dim {d} not supported (64, 128, 256)")
    _check(page % 16 == 0, f"page_size {page} must be a multiple of 16")
    b = qo_indptr.numel() - 1
    _check(b > 0, "qo_indptr must hold B + 1 offsets")
    for name, x, n in (("qo_indptr", qo_indptr, b + 1), ("indptr", indptr, b + 1), ("last_page_len", last_page_len, b)):
        _check(x.dtype == torch.int32 and x.dim() == 1 and x.numel() == n and x.is_contiguous(),
               f"{name} must be contiguous int32 [{n}]")
    _check(indices.dtype == torch.int32 and indices.dim() == 1 and indices.is_contiguous(),
           "indices must be contiguous int32 [nnz]")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    if output is None:
        output = torch.empty_like(q)
    _check(output.shape == q.shape and output.dtype == q.dtype and output.is_contiguous(), "bad output tensor")
    tensors = [q, kv_cache, qo_indptr, indptr, indices, last_page_len, output]
    if status is not None:
        _check(status.dtype == torch.int32 and status.numel() >= 1, "status must be int32 [1]")
        tensors.append(status)
    _lib.require_device(*tensors)
    _lib.call(
        "axk_paged_prefill", q.data_ptr(), kv_cache.data_ptr(), qo_indptr.data_ptr(), indptr.data_ptr(),
        indices.data_ptr(), last_page_len.data_ptr(), output.data_ptr(), b, t, hq, hkv, d, page, p, float(sm_scale),
        _lib.ptr(status), _lib.stream_of(q),
    )
    return output
