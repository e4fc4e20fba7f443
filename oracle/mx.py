"""Oracle: MXFP4 / E8M0 / E4M3 codecs and the runtime-weight linear (CPU, test infrastructure only).

Restates
  * dequant_mxfp4            models/qwen35_35b_a3b/src/70b0fbc/q35_moe.py:60-63
                             models/qwen38_27b/head/mx4_common.py:37-49
  * quant_mxfp4 (ggml rule)  models/qwen38_27b/head/mx4_common.py:11-34 (== q35_moe.py:46-57 plus the
                             0..254 clamp of the scale byte)
  * pack_fp4_codes           models/qwen35_35b_a3b/sgl/tests/test_gdn_attn.py:160-166
  * MX linear golden         q35_moe.py:222-239 (torch fp32 matmul on exactly dequantised weights),
                             sgl_kernel_axera/gemm.py:564-641 (a @ dequant(w).T + bias, fp32 acc)
  * FP8 per-channel linear   sgl_kernel_axera/gemm.py:119-181
  * quant_mxfp8 / dequant    models/qwen35_35b_a3b/src/70b0fbc/q35_mx_build.py:60-72 (E4M3 codes, one E8M0 per 32
                             along K, e = ceil(log2(amax / 448)) so nothing saturates); E5M2 codes as the other
                             MXFP8 element type sgl's mxfp8_gemm accepts (gemm.py:644-659)
  * quantize_nvfp4 / dequant  models/qwen35_35b_a3b/sgl/python/sgl_kernel_axera/quantization.py:8-37 (scale2 =
                             amax / (448 * 6) or 1; E4M3 block scales per 16 along K = clamp(block amax / (6 scale2),
                             448) rounded to nearest even; codes = E2M1 of value / (scale * scale2), nearest with ties
                             to the even code, saturating at 6, the sign kept for values that round to zero);
                             the decode of models/qwen35_35b_a3b/sgl/tests/test_nvfp4_lm_head.py:11-16
  * NVFP4 linear             sgl_kernel_axera/gemm.py:495-561 (a @ dequant(w).T + bias, fp32 acc)
  * INT8 scaled linear       sgl_kernel_axera/gemm.py:479-492 over 119-181 (each int8 operand times its scale,
                             rounded to the output dtype; fp32 matmul; bias rounded to the output dtype)
  * INT4 dequant / linear    sgl_kernel_axera/gemm.py:662-677 over 564-623 (one int4 per byte times its fp32 group
                             scale, group = K / scale columns; a @ w.T + bias, fp32 acc)
Pinned by tests/test_oracle_mx.py: exhaustive 16 x 256 code/scale table against the closed form and
torch's float8_e8m0fnu / exp2, E4M3 and E5M2 tables against torch.float8_e4m3fn / float8_e5m2, the
MXFP8 dequant against a float64 bit-field decode for every (code, scale) pair, the MXFP8 quantiser's
scale rule and nearest-code choice against a brute-force search over all 256 codes, the C restatement
(oracle/mx_codec.c) against this module, quantiser brute force + round trip, the NVFP4 codec against the reference
test's vectors (its midpoint row, zero blocks, an all-zero matrix) and its E2M1 choice against a brute-force
nearest-value search, the NVFP4 dequant against a float64 decode of every (code, scale) pair, the INT8 linear
against exact int64 dot products under power-of-two scales and against single-element cases of its operand and bias
rounding, the INT4 linear against float64 loops over each group, and the linears against float64 dot products.
"""
from __future__ import annotations

import numpy as np
import torch

GROUP = 32
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)
FP4_LUT = np.concatenate([E2M1, -E2M1]).astype(np.float32)  # code -> value; code 8 -> -0.0


def e8m0_to_f32(scales: np.ndarray) -> np.ndarray:
    """2^(s - 127) in fp32, as torch.exp2(s.float() - 127) of q35_moe.py:63 (0 -> 2^-127, 255 -> inf)."""
    s = np.asarray(scales).astype(np.int32)
    with np.errstate(over="ignore"):
        return np.ldexp(np.float32(1.0), s - 127).astype(np.float32)


def pack_fp4_codes(codes: np.ndarray) -> np.ndarray:
    """Logical codes [..., K] (0..15) -> packed [..., K/2] u8, even column in the low nibble."""
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    return (c[..., 0::2] & 15) | ((c[..., 1::2] & 15) << 4)


def unpack_fp4_codes(packed: np.ndarray) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    return np.stack([p & 15, p >> 4], axis=-1).reshape(*p.shape[:-1], p.shape[-1] * 2)


def dequant_mxfp4(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """[N, K/2] u8 codes + [N, K/32] u8 E8M0 -> [N, K] fp32 (q35_moe.py:60-63)."""
    code = unpack_fp4_codes(packed)
    n, k = code.shape
    mag = E2M1[code & 7]
    v = mag * np.where(code >= 8, np.float32(-1.0), np.float32(1.0))
    f = e8m0_to_f32(scales)
    with np.errstate(invalid="ignore", over="ignore"):
        return (v.reshape(n, k // GROUP, GROUP) * f[..., None]).reshape(n, k).astype(np.float32)


def quant_mxfp4(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """ggml-axera's MXFP4 quantiser (mx4_common.py:11-34): e = floor(log2 amax) - 2 (0 if amax == 0),
    scale byte clamp(e + 127, 0, 254), nearest E2M1 magnitude with ties to the lower code."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    g = w.reshape(n, k // GROUP, GROUP)
    amax = np.abs(g).max(-1)
    with np.errstate(divide="ignore"):
        e = np.where(amax > 0, np.floor(np.log2(np.maximum(amax, np.float32(1e-30)))) - 2, 0).astype(np.float32)
    x = g / np.exp2(e)[..., None]
    dist = np.abs(np.abs(x)[..., None] - E2M1)  # argmin returns the first minimum: ties go low
    best = dist.argmin(-1).astype(np.uint8)
    code = best | ((x < 0).astype(np.uint8) << 3)
    packed = pack_fp4_codes(code.reshape(n, k))
    scale = np.clip(e + 127, 0, 254).astype(np.uint8)
    return packed, scale


def e4m3_table() -> np.ndarray:
    """All 256 OCP E4M3 (fn) values from the format definition: bias 7, subnormal m * 2^-9, 0x7f/0xff NaN."""
    out = np.empty(256, dtype=np.float32)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e, m = (b >> 3) & 15, b & 7
        if e == 15 and m == 7:
            out[b] = np.nan
        elif e == 0:
            out[b] = s * m * 2.0 ** -9
        else:
            out[b] = s * (1 + m / 8.0) * 2.0 ** (e - 7)
    return out


def e5m2_table() -> np.ndarray:
    """All 256 OCP E5M2 values from the format definition: bias 15, subnormal m * 2^-16, exponent 31 = inf / NaN."""
    out = np.empty(256, dtype=np.float32)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e, m = (b >> 2) & 31, b & 3
        if e == 31:
            out[b] = s * np.inf if m == 0 else np.nan
        elif e == 0:
            out[b] = s * m * 2.0 ** -16
        else:
            out[b] = s * (1 + m / 4.0) * 2.0 ** (e - 15)
    return out


FP8_MAX = {"e4m3": 448.0, "e5m2": 57344.0}


def fp8_table(fmt: str) -> np.ndarray:
    return e4m3_table() if fmt == "e4m3" else e5m2_table()


def quant_mxfp8(w, fmt: str = "e4m3") -> tuple[np.ndarray, np.ndarray]:
    """[N, K] -> (codes u8 [N, K], E8M0 scales u8 [N, K/32]) as q35_mx_build.py:60-66: per block of 32 along K,
    amax clamped to >= 2^-126, e = clamp(ceil(log2(amax / FP8_MAX)), -127, 127), codes = FP8(w / 2^e) rounded to
    nearest even by torch's float8 cast, scale byte e + 127."""
    t = torch.as_tensor(np.asarray(w, dtype=np.float32))
    n, k = t.shape
    g = t.reshape(n, k // GROUP, GROUP)
    amax = g.abs().amax(-1, keepdim=True).clamp_min(2.0 ** -126)
    e = torch.ceil(torch.log2(amax / FP8_MAX[fmt])).clamp(-127, 127)
    dt = torch.float8_e4m3fn if fmt == "e4m3" else torch.float8_e5m2
    codes = (g / torch.exp2(e)).to(dt).reshape(n, k).view(torch.uint8)
    scale = (e.squeeze(-1) + 127).to(torch.uint8)
    return codes.numpy(), scale.numpy()


def dequant_mxfp8(codes: np.ndarray, scales: np.ndarray, fmt: str = "e4m3") -> np.ndarray:
    """u8 FP8 codes [N, K] + u8 E8M0 [N, K/32] -> fp32 [N, K] (q35_mx_build.py:69-72)."""
    c = np.asarray(codes, dtype=np.uint8)
    n, k = c.shape
    v = fp8_table(fmt)[c]
    f = e8m0_to_f32(scales)
    with np.errstate(invalid="ignore", over="ignore"):
        return (v.reshape(n, k // GROUP, GROUP) * f[..., None]).reshape(n, k).astype(np.float32)


def mxfp8_linear(a: torch.Tensor, codes: np.ndarray, scales: np.ndarray, fmt: str = "e4m3", bias=None):
    """a[M, K] @ dequant_mxfp8(codes, scales).T (+ bias) in fp32 (sgl mxfp8_gemm, gemm.py:644-659)."""
    w = torch.from_numpy(dequant_mxfp8(codes, scales, fmt))
    out = a.float().cpu() @ w.T
    if bias is not None:
        out = out + bias.float().cpu()
    return out


def bf16_round(x: np.ndarray | torch.Tensor) -> np.ndarray:
    """fp32 -> bf16 (round to nearest even) -> fp32."""
    t = torch.as_tensor(np.asarray(x, dtype=np.float32))
    return t.to(torch.bfloat16).float().numpy()


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def mx_linear(a: torch.Tensor, packed: np.ndarray, scales: np.ndarray, bias=None) -> torch.Tensor:
    """a[M,K] (bf16 / fp32 values) @ dequant(packed, scales).T (+ bias) in fp32: the reference golden
    (q35_moe.py:234-238, gemm.py:564-598). Returns fp32; the caller rounds to its output dtype."""
    w = torch.from_numpy(dequant_mxfp4(packed, scales))
    out = a.float().cpu() @ w.T
    if bias is not None:
        out = out + bias.float().cpu()
    return out


def fp8_linear(a: torch.Tensor, w_fp8: np.ndarray, scale_a, scale_b, bias=None) -> torch.Tensor:
    """(a * scale_a) @ (E4M3(w) * scale_b).T + bias in fp32 (gemm.py:123-153)."""
    w = torch.from_numpy(e4m3_table()[np.asarray(w_fp8, dtype=np.uint8)])
    w = w * torch.as_tensor(scale_b, dtype=torch.float32).reshape(-1, 1)
    x = a.float().cpu()
    if scale_a is not None:
        x = x * torch.as_tensor(scale_a, dtype=torch.float32).reshape(-1, 1)
    out = x @ w.T
    if bias is not None:
        out = out + bias.float().cpu()
    return out


NV_GROUP = 16  # NVFP4 block size along K


def e2m1_code(x: np.ndarray) -> np.ndarray:
    """fp32 values -> E2M1 codes (u8): the magnitude to the nearest of 0, 0.5, 1, 1.5, 2, 3, 4, 6 (beyond 6: 6), a
    tie between two neighbours to the even code; bit 3 the sign of x, kept for values that round to zero (the
    reference's expected codes turn -0.25 into 8, test_nvfp4_lm_head.py:21-31)."""
    x = np.asarray(x, dtype=np.float32)
    mag = np.abs(x).astype(np.float64)
    d = np.abs(mag[..., None] - E2M1.astype(np.float64))
    best = d.min(-1, keepdims=True)
    tied = d == best
    idx = np.arange(8)
    even = np.where(tied & (idx % 2 == 0), idx, 8).min(-1)
    code = np.where(even < 8, even, np.argmax(tied, -1))
    return (code | (np.signbit(x).astype(np.int64) << 3)).astype(np.uint8)


def quantize_nvfp4(w) -> tuple[np.ndarray, np.ndarray, np.float32]:
    """[N, K] (K % 16 == 0) -> (packed E2M1 u8 [N, K/2] (even k in the low nibble), E4M3 scale bytes u8 [N, K/16],
    fp32 scale2) by the rule of quantization.py:8-37: scale2 = fp32(amax / 2688) (1 for an all-zero matrix); each
    block's scale = E4M3(min(fp32(block amax / fp32(6 scale2)), 448)) by torch's round-to-nearest-even cast; the
    values divided by fp32(scale * scale2) (by 1 where that is 0) and coded by e2m1_code."""
    t = torch.as_tensor(np.asarray(w, dtype=np.float32))
    n, k = t.shape
    assert k % NV_GROUP == 0
    amax = float(t.abs().max()) if t.numel() else 0.0
    s2 = np.float32(amax / (448 * 6) if amax else 1.0)
    blocks = t.reshape(n, k // NV_GROUP, NV_GROUP)
    six_s2 = np.float32(6.0) * s2
    sc = torch.clamp(blocks.abs().amax(-1) / torch.tensor(six_s2), max=448.0).to(torch.float8_e4m3fn)
    dec = sc.float() * torch.tensor(s2)
    scaled = blocks / torch.where(dec > 0, dec, torch.ones_like(dec)).unsqueeze(-1)
    codes = e2m1_code(scaled.reshape(n, k).numpy())
    return pack_fp4_codes(codes), sc.view(torch.uint8).numpy(), s2


def dequant_nvfp4(packed: np.ndarray, scales: np.ndarray, scale2) -> np.ndarray:
    """packed u8 [N, K/2] + E4M3 scale bytes u8 [N, K/16] + fp32 scale2 -> fp32 [N, K]: value(code) * scale * scale2
    in that order (test_nvfp4_lm_head.py:11-16)."""
    codes = unpack_fp4_codes(np.asarray(packed, dtype=np.uint8))
    n, k = codes.shape
    v = FP4_LUT[codes].reshape(n, k // NV_GROUP, NV_GROUP)
    s = e4m3_table()[np.asarray(scales, dtype=np.uint8)].reshape(n, k // NV_GROUP, 1)
    with np.errstate(invalid="ignore", over="ignore"):
        return ((v * s) * np.float32(scale2)).reshape(n, k).astype(np.float32)


def nvfp4_linear(a: torch.Tensor, packed: np.ndarray, scales: np.ndarray, scale2, bias=None) -> torch.Tensor:
    """a[M, K] @ dequant_nvfp4(packed, scales, scale2).T (+ bias) in fp32 (sgl nvfp4_gemm, gemm.py:495-561)."""
    w = torch.from_numpy(dequant_nvfp4(packed, scales, scale2))
    out = a.float().cpu() @ w.T
    if bias is not None:
        out = out + bias.float().cpu()
    return out


def int8_linear(a_int8, b_int8, scale_a, scale_b, out_dtype=torch.bfloat16, bias=None) -> torch.Tensor:
    """sgl int8_gemm (gemm.py:479-492 -> scaled_gemm_kernel 123-153): each operand times its per-row / per-channel
    scale (a scalar broadcasts, _normalize_scale 17-23) rounded to out_dtype, an fp32 matmul, plus the bias rounded
    to out_dtype (_prepare_bias_output 34-39). Returns fp32; the caller rounds to out_dtype."""
    a = torch.as_tensor(np.asarray(a_int8, dtype=np.int8)).float()
    b = torch.as_tensor(np.asarray(b_int8, dtype=np.int8)).float()
    sa = torch.as_tensor(np.asarray(scale_a, dtype=np.float32)).reshape(-1)
    sb = torch.as_tensor(np.asarray(scale_b, dtype=np.float32)).reshape(-1)
    sa = sa.expand(a.shape[0]) if sa.numel() == 1 else sa
    sb = sb.expand(b.shape[0]) if sb.numel() == 1 else sb
    x = (a * sa[:, None]).to(out_dtype).float()
    w = (b * sb[:, None]).to(out_dtype).float()
    out = x @ w.T
    if bias is not None:
        out = out + torch.as_tensor(bias).float().to(out_dtype).float()
    return out


def dequant_int4(b_int4, b_scale) -> np.ndarray:
    """int4 values (one signed value per byte) [N, K] times the fp32 scale of their group of K / G along K
    (G = K / b_scale.shape[1]): the hardware dequantisation w = w_int * scale of gemm.py:580-589."""
    w = np.asarray(b_int4, dtype=np.int8).astype(np.float32)
    s = np.asarray(b_scale, dtype=np.float32)
    n, k = w.shape
    g = k // s.shape[1]
    return (w.reshape(n, k // g, g) * s[:, :, None]).reshape(n, k)


def int4_linear(a: torch.Tensor, b_int4, b_scale, bias=None) -> torch.Tensor:
    """a[M, K] @ dequant_int4(b_int4, b_scale).T (+ bias) in fp32 (sgl int4_gemm, gemm.py:662-677 -> _mx_gemm)."""
    w = torch.from_numpy(dequant_int4(b_int4, b_scale))
    out = a.float().cpu() @ w.T
    if bias is not None:
        out = out + bias.float().cpu()
    return out
