"""Host preparation of packed runtime-quantised weights, once at model load (the role of
models/qwen35_35b_a3b/sgl/python/sgl_kernel_axera/quantization.py).

quantize_nvfp4(weight) -> (E2M1 pairs [N, K/2], E4M3 block scales [N, K/16], fp32 scale2 [1]) in the layout
axk_nvfp4_gemm reads: even k in the low nibble, one E4M3 scale per 16 values along K, and
  scale2 = amax(|W|) / (448 * 6) (1 for an all-zero matrix),
  scale[n, b] = E4M3(min(amax(|W[n, 16 b : 16 b + 16]|) / (6 scale2), 448)),
  code = E2M1(W / (scale * scale2)) (divided by 1 where that product is 0),
both casts to the nearest value with ties to even (the E2M1 tie to the even code, magnitudes past 6 to 6, the sign
of a value that rounds to zero kept), as quantization.py:8-37. Rows are processed 1024 at a time, so a large head
never expands to fp32 whole.
"""
from __future__ import annotations

import torch

_BOUNDS = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])  # midpoints between the E2M1 magnitudes


def _e2m1_codes(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> E2M1 codes (uint8): the magnitude's interval between midpoints, a value on a midpoint to the even
    neighbour, bit 3 the sign."""
    mag = x.abs()
    idx = torch.bucketize(mag, _BOUNDS)  # mag on a midpoint b_i lands in i, the lower neighbour
    on_mid = (idx < _BOUNDS.numel()) & (mag == _BOUNDS[idx.clamp(max=_BOUNDS.numel() - 1)])
    idx = torch.where(on_mid & (idx % 2 == 1), idx + 1, idx)
    return (idx | (torch.signbit(x).to(torch.int64) << 3)).to(torch.uint8)


def quantize_nvfp4(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """A floating [N, K] matrix (K % 16 == 0) -> (packed float4_e2m1fn_x2 [N, K/2], float8_e4m3fn [N, K/16],
    float32 [1]) on the host (see the module docstring); move them to the device for axk.nvfp4_gemm."""
    if weight.dim() != 2 or weight.shape[1] % 16:
        raise ValueError("NVFP4 weights require a matrix with K divisible by 16")
    if weight.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError("NVFP4 quantization requires floating-point weights")
    w = weight.detach().cpu()
    n, k = w.shape
    amax = float(w.abs().max()) if w.numel() else 0.0
    scale2 = torch.tensor([amax / (448 * 6) if amax else 1.0], dtype=torch.float32)
    packed = torch.empty((n, k // 2), dtype=torch.uint8)
    scales = torch.empty((n, k // 16), dtype=torch.float8_e4m3fn)
    for r0 in range(0, n, 1024):
        blk = w[r0:r0 + 1024].float().reshape(-1, k // 16, 16)
        sc = (blk.abs().amax(-1) / (6 * scale2)).clamp(max=448).to(torch.float8_e4m3fn)
        scales[r0:r0 + 1024] = sc
        dec = sc.float() * scale2
        codes = _e2m1_codes(blk / torch.where(dec > 0, dec, torch.ones_like(dec)).unsqueeze(-1)).reshape(-1, k)
        packed[r0:r0 + 1024] = codes[:, 0::2] | (codes[:, 1::2] << 4)
    return packed.view(torch.float4_e2m1fn_x2), scales, scale2
