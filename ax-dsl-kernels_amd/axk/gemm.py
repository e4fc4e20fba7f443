"""Runtime-weight linear operators (MXFP4 / NVFP4 / MXFP8 / FP8 E4M3 / INT8 / INT4 / bf16 weights) on gfx950.

Mirrors the operator API of sgl_kernel_axera.gemm
(models/qwen35_35b_a3b/sgl/python/sgl_kernel_axera/gemm.py): the same names, argument meaning and
``ValueError`` contract checks (_prepare_bias_output 26-46, _normalize_scale 17-23). Every call goes
through libaxk.so; there is no host fallback.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib

_OUT_DT = {torch.bfloat16: _lib.DT_BF16, torch.float32: _lib.DT_F32}


def _as_u8(t: torch.Tensor, name: str) -> torch.Tensor:
    """FP4 codes / E8M0 / E4M3 payloads travel as u8; accept torch's packed views of the same bytes."""
    if t.dtype in (torch.uint8, torch.float4_e2m1fn_x2, torch.float8_e8m0fnu, torch.float8_e4m3fn, torch.float8_e5m2):
        return t.view(torch.uint8)
    raise ValueError(f"{name} must be uint8 (or a float4/float8 view of bytes), got {t.dtype}")


def _prepare_bias_output(n, m, device, out_dtype, bias, output):
    """As gemm.py:26-46: bias defaults to zeros and is rounded to out_dtype; output is [m, n]."""
    if out_dtype not in _OUT_DT:
        raise ValueError(f"out_dtype must be bfloat16 or float32, got {out_dtype}")
    if bias is not None:
        if tuple(bias.shape) != (n,):
            raise ValueError(f"bias shape {tuple(bias.shape)} is incompatible with N={n}")
        bias = bias.to(device=device, dtype=out_dtype).float().contiguous()
    if output is None:
        output = torch.empty((m, n), device=device, dtype=out_dtype)
    elif tuple(output.shape) != (m, n):
        raise ValueError(f"output shape {tuple(output.shape)} is incompatible with {(m, n)}")
    elif output.dtype != out_dtype or not output.is_contiguous():
        raise ValueError("output must be a contiguous tensor of out_dtype")
    return bias, output


def _normalize_scale(scale: torch.Tensor, size: int, name: str, device) -> torch.Tensor:
    """As gemm.py:17-23: a scalar broadcasts, otherwise one fp32 scale per row / channel."""
    scale = scale.reshape(-1)
    if scale.numel() == 1:
        return scale.to(device=device, dtype=torch.float32).expand(size).contiguous()
    if scale.numel() != size:
        raise ValueError(f"{name} shape {tuple(scale.shape)} is incompatible with size={size}")
    return scale.to(device=device, dtype=torch.float32).contiguous()


def _check_a(a: torch.Tensor) -> tuple[int, int]:
    if a.dim() != 2:
        raise ValueError("a must be a 2D tensor")
    if a.dtype != torch.bfloat16:
        raise ValueError(f"a must be bfloat16, got {a.dtype}")
    if a.stride(1) != 1:
        raise ValueError("a must have unit stride along K")
    return a.shape


def mxfp4_dequant(b_fp4: torch.Tensor, b_scale: torch.Tensor, output: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Exact fp32 dequantisation of packed E2M1 codes [N, K/2] and E8M0 scales [N, K/32] (into `output` when
    given: fp32 [N, K], contiguous)."""
    codes, scales = _as_u8(b_fp4, "b_fp4").contiguous(), _as_u8(b_scale, "b_scale").contiguous()
    _lib.require_device(codes, scales)
    n, k = codes.shape[0], codes.shape[1] * 2
    if tuple(scales.shape) != (n, k // 32):
        raise ValueError(f"b_scale shape {tuple(scales.shape)} is incompatible with codes {tuple(codes.shape)}")
    if output is None:
        out = torch.empty((n, k), device=codes.device, dtype=torch.float32)
    else:
        if output.dtype != torch.float32 or tuple(output.shape) != (n, k) or not output.is_contiguous():
            raise ValueError(f"output must be contiguous float32 [{n}, {k}]")
        _lib.require_device(output)
        out = output
    _lib.call("axk_mxfp4_dequant", codes.data_ptr(), scales.data_ptr(), out.data_ptr(), n, k, _lib.stream_of(out))
    return out


def mxfp4_gemm(
    a: torch.Tensor,
    b_fp4: torch.Tensor,
    b_scale: torch.Tensor,
    out_dtype: torch.dtype = torch.bfloat16,
    bias: Optional[torch.Tensor] = None,
    output: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """MXFP4 GEMM: output = a @ dequant(b_fp4, b_scale).T + bias (gemm.py:626-641).

    a       : (m, k) bf16 activation
    b_fp4   : (n, k/2) packed E2M1 codes, low nibble = even column (u8 or float4_e2m1fn_x2 view)
    b_scale : (n, k/32) E8M0 per-32 block scale (u8 or float8_e8m0fnu view)
    """
    m, k = _check_a(a)
    codes, scales = _as_u8(b_fp4, "b_fp4"), _as_u8(b_scale, "b_scale")
    n = codes.shape[0]
    if codes.dim() != 2 or codes.shape[1] * 2 != k:
        raise ValueError(f"b_fp4 shape {tuple(b_fp4.shape)} is incompatible with a having k={k}")
    if tuple(scales.shape) != (n, k // 32):
        raise ValueError(f"b_scale shape {tuple(b_scale.shape)} is incompatible with (n, k/32)={(n, k // 32)}")
    bias, output = _prepare_bias_output(n, m, a.device, out_dtype, bias, output)
    codes, scales = codes.contiguous(), scales.contiguous()
    _lib.require_device(a, codes, scales, output)
    _lib.call(
        "axk_mxfp4_gemm", a.data_ptr(), a.stride(0), codes.data_ptr(), scales.data_ptr(), _lib.ptr(bias),
        output.data_ptr(), _OUT_DT[out_dtype], m, n, k, _lib.stream_of(a),
    )
    return output


def nvfp4_gemm(
    a: torch.Tensor,
    b_fp4: torch.Tensor,
    b_scale: torch.Tensor,
    b_scale2: torch.Tensor,
    out_dtype: torch.dtype = torch.bfloat16,
    bias: Optional[torch.Tensor] = None,
    output: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """NVFP4 GEMM: output = a @ dequant(b_fp4, b_scale, b_scale2).T + bias (gemm.py:495-561).

    a        : (m, k) bf16 activation
    b_fp4    : (n, k/2) packed E2M1 codes, low nibble = even column (u8 or float4_e2m1fn_x2 view), as
               quantize_nvfp4 packs them
    b_scale  : (n, k/16) E4M3 per-16 block scale (u8 or float8_e4m3fn view)
    b_scale2 : (1,) float32 global scale on the device (a runtime input: rescaling it needs no repacking)
    """
    m, k = _check_a(a)
    codes, scales = _as_u8(b_fp4, "b_fp4"), _as_u8(b_scale, "b_scale")
    n = codes.shape[0]
    if codes.dim() != 2 or codes.shape[1] * 2 != k:
        raise ValueError(f"b_fp4 shape {tuple(b_fp4.shape)} is incompatible with a having k={k}")
    if tuple(scales.shape) != (n, k // 16):
        raise ValueError(f"b_scale shape {tuple(b_scale.shape)} is incompatible with (n, k/16)={(n, k // 16)}")
    if b_scale2.dtype != torch.float32 or b_scale2.numel() != 1:
        raise ValueError("b_scale2 must be a float32 tensor of one element")
    bias, output = _prepare_bias_output(n, m, a.device, out_dtype, bias, output)
    codes, scales = codes.contiguous(), scales.contiguous()
    _lib.require_device(a, codes, scales, b_scale2, output)
    _lib.call(
        "axk_nvfp4_gemm", a.data_ptr(), a.stride(0), codes.data_ptr(), scales.data_ptr(), b_scale2.data_ptr(),
        _lib.ptr(bias), output.data_ptr(), _OUT_DT[out_dtype], m, n, k, _lib.stream_of(a),
    )
    return output


def fp8_gemm(
    a: torch.Tensor,
    b_fp8_t: torch.Tensor,
    scale_a: Optional[torch.Tensor],
    scale_b: torch.Tensor,
    out_dtype: torch.dtype = torch.bfloat16,
    bias: Optional[torch.Tensor] = None,
    output: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """FP8 E4M3 weight linear with per-output-channel scales (gemm.py:119-181, 457-466).

    output = (a * scale_a[:, None]) @ (b_fp8_t * scale_b[:, None]).T + bias, fp32 accumulation.
    The activation is bf16 here (the hybrid decode group feeds bf16 hidden states).
    """
    m, k = _check_a(a)
    w = _as_u8(b_fp8_t, "b_fp8_t")
    if w.dim() != 2 or w.shape[1] != k:
        raise ValueError(f"b_t must have shape [N, K], got {tuple(b_fp8_t.shape)} for K={k}")
    n = w.shape[0]
    sa = None if scale_a is None else _normalize_scale(scale_a, m, "scale_a", a.device)
    sb = _normalize_scale(scale_b, n, "scale_b", a.device)
    bias, output = _prepare_bias_output(n, m, a.device, out_dtype, bias, output)
    w = w.contiguous()
    _lib.require_device(a, w, output)
    _lib.call(
        "axk_fp8_gemm", a.data_ptr(), a.stride(0), w.data_ptr(), _lib.ptr(sa), sb.data_ptr(), _lib.ptr(bias),
        output.data_ptr(), _OUT_DT[out_dtype], m, n, k, _lib.stream_of(a),
    )
    return output


_FP8_DT = {"e4m3": _lib.DT_FP8E4M3, "e5m2": _lib.DT_FP8E5M2}


def mxfp8_gemm(
    a: torch.Tensor,
    b_fp8: torch.Tensor,
    b_scale: torch.Tensor,
    out_dtype: torch.dtype = torch.bfloat16,
    bias: Optional[torch.Tensor] = None,
    output: Optional[torch.Tensor] = None,
    fmt: Optional[str] = None,
) -> torch.Tensor:
    """MXFP8 GEMM: output = a @ dequant(b_fp8, b_scale).T + bias (gemm.py:644-659).

    a       : (m, k) bf16 activation
    b_fp8   : (n, k) MXFP8 weight, fp8_e4m3 or fp8_e5m2 (a float8 view, or u8 with fmt = "e4m3" / "e5m2")
    b_scale : (n, k//32) E8M0 per-32 block scale (u8 or float8_e8m0fnu view)
    """
    m, k = _check_a(a)
    if fmt is None:
        if b_fp8.dtype == torch.float8_e4m3fn:
            fmt = "e4m3"
        elif b_fp8.dtype == torch.float8_e5m2:
            fmt = "e5m2"
        else:
            raise ValueError("b_fp8 must be a float8_e4m3fn / float8_e5m2 tensor, or u8 with fmt given")
    if fmt not in _FP8_DT:
        raise ValueError(f"fmt must be 'e4m3' or 'e5m2', got {fmt}")
    if b_fp8.dtype not in (torch.uint8, torch.float8_e4m3fn, torch.float8_e5m2):
        raise ValueError(f"b_fp8 must be uint8 or a float8 view, got {b_fp8.dtype}")
    w = b_fp8.view(torch.uint8)
    scales = _as_u8(b_scale, "b_scale")
    if w.dim() != 2 or w.shape[1] != k:
        raise ValueError(f"b_fp8 shape {tuple(b_fp8.shape)} is incompatible with a having k={k}")
    n = w.shape[0]
    if tuple(scales.shape) != (n, k // 32):
        raise ValueError(f"b_scale shape {tuple(b_scale.shape)} is incompatible with (n, k/32)={(n, k // 32)}")
    bias, output = _prepare_bias_output(n, m, a.device, out_dtype, bias, output)
    w, scales = w.contiguous(), scales.contiguous()
    _lib.require_device(a, w, scales, output)
    _lib.call(
        "axk_mxfp8_gemm", a.data_ptr(), a.stride(0), w.data_ptr(), scales.data_ptr(), _FP8_DT[fmt], _lib.ptr(bias),
        output.data_ptr(), _OUT_DT[out_dtype], m, n, k, _lib.stream_of(a),
    )
    return output


def bf16_gemm(
    a: torch.Tensor,
    b_t: torch.Tensor,
    out_dtype: torch.dtype = torch.bfloat16,
    bias: Optional[torch.Tensor] = None,
    output: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Dense bf16 projection a[M,K] @ b_t[N,K].T + bias with fp32 accumulation (gemm.py:81-116, 469-476)."""
    m, k = _check_a(a)
    if b_t.dim() != 2 or b_t.shape[1] != k or b_t.dtype != torch.bfloat16:
        raise ValueError(f"b_t must be bfloat16 [N, K], got {tuple(b_t.shape)} {b_t.dtype} for K={k}")
    n = b_t.shape[0]
    bias, output = _prepare_bias_output(n, m, a.device, out_dtype, bias, output)
    b_t = b_t.contiguous()
    _lib.require_device(a, b_t, output)
    _lib.call(
        "axk_bf16_gemm", a.data_ptr(), a.stride(0), b_t.data_ptr(), _lib.ptr(bias), output.data_ptr(),
        _OUT_DT[out_dtype], m, n, k, _lib.stream_of(a),
    )
    return output


def int8_gemm(
    a_int8: torch.Tensor,
    b_int8_t: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    out_dtype: torch.dtype = torch.bfloat16,
    bias: Optional[torch.Tensor] = None,
    output: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """INT8 scaled GEMM (gemm.py:479-492 over _scaled_gemm 119-181).

    output = (a_int8 * scale_a[:, None]) @ (b_int8_t * scale_b[:, None]).T + bias
    a_int8 int8 [m, k] (unit stride along K, k % 16 == 0); b_int8_t int8 [n, k]; scale_a [m] or a scalar,
    scale_b [n] or a scalar. The int8 products are summed exactly in int32; each sum is scaled once in fp32.
    """
    if a_int8.dim() != 2 or b_int8_t.dim() != 2:
        raise ValueError("a and b_t must be 2D tensors")
    if a_int8.dtype != torch.int8 or b_int8_t.dtype != torch.int8:
        raise ValueError(f"a_int8 and b_int8_t must be int8, got {a_int8.dtype} / {b_int8_t.dtype}")
    m, k = a_int8.shape
    if b_int8_t.shape[1] != k:
        raise ValueError(f"b_t must have shape [N, K], got {tuple(b_int8_t.shape)} for K={k}")
    n = b_int8_t.shape[0]
    sa = _normalize_scale(scale_a, m, "scale_a", a_int8.device)
    sb = _normalize_scale(scale_b, n, "scale_b", a_int8.device)
    bias, output = _prepare_bias_output(n, m, a_int8.device, out_dtype, bias, output)
    if m == 0 or n == 0:  # nothing to compute (an empty tensor may have no device address)
        return output
    if a_int8.stride(1) != 1 or a_int8.stride(0) % 16:
        a_int8 = a_int8.contiguous()
    w = b_int8_t.contiguous()
    _lib.require_device(a_int8, w, sa, sb, output)
    _lib.call(
        "axk_int8_gemm", a_int8.data_ptr(), a_int8.stride(0), w.data_ptr(), sa.data_ptr(), sb.data_ptr(),
        _lib.ptr(bias), output.data_ptr(), _OUT_DT[out_dtype], m, n, k, _lib.stream_of(a_int8),
    )
    return output


def int4_gemm(
    a: torch.Tensor,
    b_int4: torch.Tensor,
    b_scale: torch.Tensor,
    out_dtype: torch.dtype = torch.bfloat16,
    bias: Optional[torch.Tensor] = None,
    output: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """INT4 GEMM: output = a @ dequant(b_int4, b_scale).T + bias (gemm.py:662-677).

    a       : (m, k) bf16 activation
    b_int4  : (n, k) int8 tensor holding one signed int4 value (-8..7) per byte
    b_scale : (n, k // group) float32 per-group scale; group = k // b_scale.shape[1], a multiple of 32
    """
    m, k = _check_a(a)
    if b_int4.dim() != 2 or b_int4.shape[1] != k:
        raise ValueError(f"b_w shape {tuple(b_int4.shape)} is incompatible with a having k={k}")
    if b_int4.dtype != torch.int8:
        raise ValueError(f"b_int4 must be an int8 tensor (one int4 per byte), got {b_int4.dtype}")
    n = b_int4.shape[0]
    if b_scale.dim() != 2 or b_scale.shape[0] != n or b_scale.shape[1] == 0 or k % b_scale.shape[1]:
        raise ValueError(f"b_scale shape {tuple(b_scale.shape)} is incompatible with (n, k/group) for n={n}, k={k}")
    group = k // b_scale.shape[1]
    if group % 32:
        raise ValueError(f"group size {group} must be a multiple of 32")
    bias, output = _prepare_bias_output(n, m, a.device, out_dtype, bias, output)
    if m == 0 or n == 0:  # nothing to compute (an empty tensor may have no device address)
        return output
    w = b_int4.contiguous()
    scales = b_scale.to(torch.float32).contiguous()
    _lib.require_device(a, w, scales, output)
    _lib.call(
        "axk_int4_gemm", a.data_ptr(), a.stride(0), w.data_ptr(), scales.data_ptr(), group, _lib.ptr(bias),
        output.data_ptr(), _OUT_DT[out_dtype], m, n, k, _lib.stream_of(a),
    )
    return output
