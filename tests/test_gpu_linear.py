"""GPU parity of the MXFP4 codec and the MXFP4 / FP8 / bf16 runtime-weight linear against the oracle.

Bar: dequantised values bit-exact; bf16 outputs within rel 2e-2 / abs 1e-2 of the fp32-accumulating
golden (fp32 outputs: rel 1e-3 / abs 1e-3, the only difference being summation order).
"""
import numpy as np
import pytest
import torch

import axk
from axk import configs
from oracle import mx

pytestmark = pytest.mark.gpu

BF16_TOL = dict(rtol=2e-2, atol=1e-2)
F32_TOL = dict(rtol=1e-3, atol=1e-3)


def _bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return bool(np.all((np.isnan(a) & np.isnan(b)) | (a.view(np.uint32) == b.view(np.uint32))))


def test_dequant_exhaustive_table_bit_exact(dev):
    codes = np.tile(np.arange(16, dtype=np.uint8), (256, 2))
    packed = mx.pack_fp4_codes(codes)
    scales = np.arange(256, dtype=np.uint8)[:, None]
    got = axk.mxfp4_dequant(torch.from_numpy(packed).to(dev), torch.from_numpy(scales).to(dev)).cpu().numpy()
    assert _bits_equal(got, mx.dequant_mxfp4(packed, scales))


@pytest.mark.parametrize("n,k", [(1, 32), (37, 96), (4096, 4096)])
def test_dequant_random_bit_exact(dev, n, k):
    g = torch.Generator().manual_seed(n + k)
    packed = torch.randint(0, 256, (n, k // 2), generator=g, dtype=torch.uint8)
    scales = torch.randint(0, 256, (n, k // 32), generator=g, dtype=torch.uint8)
    got = axk.mxfp4_dequant(packed.to(dev), scales.to(dev)).cpu().numpy()
    assert _bits_equal(got, mx.dequant_mxfp4(packed.numpy(), scales.numpy()))


@pytest.mark.parametrize(
    "m,n,k",
    [(1, 4096, 4096), (1, 16, 32), (1, 100, 96), (3, 2048, 512), (8, 1024, 2048), (16, 256, 4096),
     (17, 300, 1024), (32, 512, 2048), (40, 64, 256)],
)
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_mxfp4_gemm_matches_oracle(dev, m, n, k, out_dtype):
    g = torch.Generator().manual_seed(1000 * m + n + k)
    packed, scales = configs.mxfp4_weight(n, k, g)
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    bias = torch.randn(n, generator=g) / 8
    ref = mx.mx_linear(a, packed.numpy(), scales.numpy(), bias.to(out_dtype))
    got = axk.mxfp4_gemm(a.to(dev), packed.to(dev), scales.to(dev), out_dtype=out_dtype, bias=bias.to(dev))
    assert got.dtype == out_dtype and got.shape == (m, n)
    tol = BF16_TOL if out_dtype == torch.bfloat16 else F32_TOL
    torch.testing.assert_close(got.float().cpu(), ref.to(out_dtype).float(), **tol)


def test_mxfp4_gemm_config0(dev):
    c = configs.config0()
    ref = mx.mx_linear(c["x"], c["w"].numpy(), c["s"].numpy()).to(torch.bfloat16)
    got = axk.mxfp4_gemm(c["x"].to(dev), c["w"].to(dev), c["s"].to(dev))
    torch.testing.assert_close(got.float().cpu(), ref.float(), **BF16_TOL)
    # runtime weights: flipping every sign bit in place negates the output with the same launch
    w = c["w"].to(dev)
    w.bitwise_xor_(0x88)
    neg = axk.mxfp4_gemm(c["x"].to(dev), w, c["s"].to(dev))
    torch.testing.assert_close(neg.float().cpu(), -ref.float(), **BF16_TOL)


def test_mxfp4_gemm_strided_activation_and_output_buffer(dev):
    g = torch.Generator().manual_seed(7)
    packed, scales = configs.mxfp4_weight(64, 128, g)
    big = torch.randn(4, 256, generator=g).to(torch.bfloat16)
    a = big[:, :128]  # row stride 256
    out = torch.empty(4, 64, dtype=torch.float32, device=dev)
    a_dev = big.to(dev)[:, :128]
    assert a_dev.stride(0) == 256
    res = axk.mxfp4_gemm(a_dev, packed.to(dev), scales.to(dev), out_dtype=torch.float32, output=out)
    assert res is out
    ref = mx.mx_linear(a, packed.numpy(), scales.numpy())
    torch.testing.assert_close(out.cpu(), ref, **F32_TOL)


@pytest.mark.parametrize("m,n,k", [(1, 1024, 4096), (8, 4096, 4096), (5, 96, 64), (32, 300, 512)])
def test_fp8_gemm_matches_oracle(dev, m, n, k):
    g = torch.Generator().manual_seed(m * n + k)
    w = (torch.randn(n, k, generator=g) * 0.5).to(torch.float8_e4m3fn)
    sb = torch.rand(n, generator=g) * 0.02 + 0.001
    sa = torch.rand(m, generator=g) + 0.5
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    ref = mx.fp8_linear(a, w.view(torch.uint8).numpy(), sa, sb)
    got = axk.fp8_gemm(a.to(dev), w.to(dev), sa.to(dev), sb.to(dev))
    torch.testing.assert_close(got.float().cpu(), ref.to(torch.bfloat16).float(), **BF16_TOL)
    got32 = axk.fp8_gemm(a.to(dev), w.to(dev), None, sb.to(dev), out_dtype=torch.float32)
    ref32 = mx.fp8_linear(a, w.view(torch.uint8).numpy(), None, sb)
    torch.testing.assert_close(got32.cpu(), ref32, **F32_TOL)


def test_fp8_gemm_config4_q_projection(dev):
    # the measured config-4 shape: E4M3 [16384, 4096] + per-channel scale, decode batch 8
    c = configs.config4_fp8_proj()
    ref = mx.fp8_linear(c["x"], c["w"].numpy(), None, c["scale_b"])
    got = axk.fp8_gemm(c["x"].to(dev), c["w"].to(dev), None, c["scale_b"].to(dev))
    torch.testing.assert_close(got.float().cpu(), ref.to(torch.bfloat16).float(), **BF16_TOL)


def test_dequant_config0_into_output_buffer(dev):
    # the measured codec workload: config 0's weight into a caller-owned fp32 buffer, bit-exact
    c = configs.config0()
    out = torch.full((4096, 4096), float("nan"), dtype=torch.float32, device=dev)
    got = axk.mxfp4_dequant(c["w"].to(dev), c["s"].to(dev), output=out)
    assert got.data_ptr() == out.data_ptr()
    assert _bits_equal(out.cpu().numpy(), mx.dequant_mxfp4(c["w"].numpy(), c["s"].numpy()))


@pytest.mark.parametrize("m,n,k", [(32, 256, 2048), (1, 64, 32), (4096 // 64, 256, 2048)])
def test_bf16_gemm_matches_oracle(dev, m, n, k):
    g = torch.Generator().manual_seed(m + n + k)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    ref = a.float() @ w.float().T
    got = axk.bf16_gemm(a.to(dev), w.to(dev), out_dtype=torch.float32)
    torch.testing.assert_close(got.cpu(), ref, **F32_TOL)


def test_lm_head_vocab_gemv(dev):
    """The MXFP4 LM head at the full vocabulary (248320 x 2048, fp32 logits), M = 1 and the 4 rows of a
    speculative verify: against an fp32 matmul on the GPU over the bit-exact dequantised weight (the oracle's
    formula; the exhaustive codec tests pin the dequant), at the bf16-output bar."""
    from axk import configs

    c = configs.lm_head_case(dev, seed=3, m=4)
    wf = axk.mxfp4_dequant(c["w"], c["s"])  # [N, K] fp32, exact
    for m in (1, 4):
        x = c["x"][:m].contiguous()
        got = axk.mxfp4_gemm(x, c["w"], c["s"], out_dtype=torch.float32)
        ref = (wf @ x.float().t().contiguous()).t()  # contiguous right operand
        torch.testing.assert_close(got, ref, rtol=2e-2, atol=1e-2)
    del wf


def test_lm_head_rows_against_oracle(dev):
    """A slice of LM-head rows (n not a multiple of the 16-row tile) against the CPU oracle, fp32 out."""
    from axk import configs
    from oracle import mx

    c = configs.lm_head_case(dev, seed=4, n=3000, m=1)
    got = axk.mxfp4_gemm(c["x"], c["w"], c["s"], out_dtype=torch.float32).cpu()
    ref = mx.mx_linear(c["x"].cpu(), c["w"].cpu().numpy(), c["s"].cpu().numpy())
    torch.testing.assert_close(got, ref.float(), rtol=2e-2, atol=1e-2)


# ---- MXFP8 (E4M3 / E5M2 codes + E8M0 per 32 along K): sgl mxfp8_gemm (gemm.py:644-659), q35_mx_build.py:60-72 ----
def _mxfp8_weight(n, k, g, fmt, lo=119, hi=124):
    """Finite FP8 codes (uniform over the non-NaN / non-inf bytes) and scale bytes uniform in lo .. hi - 1."""
    table = mx.fp8_table(fmt)
    finite = np.flatnonzero(np.isfinite(table)).astype(np.uint8)
    codes = finite[torch.randint(0, finite.size, (n, k), generator=g).numpy()]
    scales = torch.randint(lo, hi, (n, k // 32), generator=g, dtype=torch.uint8).numpy()
    return codes, scales


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_mxfp8_decode_bit_exact_through_identity(dev, fmt):
    """out = I @ dequant(W)^T = dequant(W)^T exactly (each output is one product, fp32 out): every finite code at
    every scale byte of the bf16-normal range goes through the in-register scaled convert unchanged. A zero weight
    comes out as +0 whatever its sign (1 * -0 + 0 * others rounds to +0 in any linear), so zeros compare by value."""
    table = mx.fp8_table(fmt)
    finite = np.flatnonzero(np.isfinite(table)).astype(np.uint8)
    k = 256
    codes = np.resize(finite, (64, k)).astype(np.uint8)
    codes = np.roll(codes, 7, axis=1)
    lo = 10 if fmt == "e4m3" else 17  # the smallest subnormal code times 2^(lo - 127) is a bf16 normal
    scales = (lo + (np.arange(64 * k // 32).reshape(64, k // 32) * 29) % (239 - lo)).astype(np.uint8)
    eye = torch.eye(k, dtype=torch.bfloat16)
    got = axk.mxfp8_gemm(eye.to(dev), torch.from_numpy(codes).to(dev), torch.from_numpy(scales).to(dev),
                         out_dtype=torch.float32, fmt=fmt).cpu().numpy()
    want = mx.dequant_mxfp8(codes, scales, fmt).T
    zero = want == 0
    assert (got[zero] == 0).all()
    assert _bits_equal(got[~zero], want[~zero])


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize(
    "m,n,k",
    [(1, 16, 32), (1, 100, 96), (3, 2048, 512), (8, 1024, 2048), (17, 300, 1024), (32, 512, 2048), (40, 64, 256)],
)
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_mxfp8_gemm_matches_oracle(dev, fmt, m, n, k, out_dtype):
    g = torch.Generator().manual_seed(7000 * m + n + k)
    codes, scales = _mxfp8_weight(n, k, g, fmt)
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    bias = torch.randn(n, generator=g) / 8
    ref = mx.mxfp8_linear(a, codes, scales, fmt, bias.to(out_dtype))
    got = axk.mxfp8_gemm(a.to(dev), torch.from_numpy(codes).to(dev), torch.from_numpy(scales).to(dev),
                         out_dtype=out_dtype, bias=bias.to(dev), fmt=fmt)
    if out_dtype == torch.bfloat16:
        torch.testing.assert_close(got.float().cpu(), ref.to(out_dtype).float(), **BF16_TOL)
    else:
        # fp32 out: the two fp32 summation orders may differ by a few ulps of the largest partial sums, which with
        # E5M2 codes over their whole range (weights up to ~3600) can exceed a flat 1e-3 on a cancelling sum; bound
        # each element by its terms' magnitude: 1e-3 + 2^-20 * sum_k |a_k w_k|
        w = torch.from_numpy(mx.dequant_mxfp8(codes, scales, fmt))
        mag = a.float().abs() @ w.abs().T
        err = (got.float().cpu() - ref).abs()
        assert (err <= 1e-3 + 1e-3 * ref.abs() + mag * 2.0 ** -20).all(), float((err - mag * 2.0 ** -20).max())


@pytest.mark.parametrize("n,k", [(16384, 4096), (1024, 4096), (4096, 8192), (8192, 4096)])
def test_mxfp8_config4_projections(dev, n, k):
    """Config 4's attention / GDN projection shapes (q, k / v, o, GDN qkv) with MXFP8 weights from the reference's
    own quantiser rule (quant_mxfp8 of an N(0, 0.02) weight), 8 decode rows."""
    g = torch.Generator().manual_seed(n + k)
    w = (torch.randn(n, k, generator=g) * 0.02).numpy()
    codes, scales = mx.quant_mxfp8(w)
    a = torch.randn(8, k, generator=g).to(torch.bfloat16)
    got = axk.mxfp8_gemm(a.to(dev), torch.from_numpy(codes).to(dev), torch.from_numpy(scales).to(dev), fmt="e4m3")
    ref = mx.mxfp8_linear(a, codes, scales, "e4m3")
    torch.testing.assert_close(got.float().cpu(), ref.to(torch.bfloat16).float(), **BF16_TOL)


# ---- NVFP4 (E2M1 pairs + E4M3 per 16 along K + an fp32 scale2): sgl nvfp4_gemm (gemm.py:495-561) ----
def _nvfp4_weight(n, k, g, lo=0x20, hi=0x50):
    """Uniform nibbles and E4M3 scale bytes in lo .. hi - 1 (normal positive scales 2^-3 .. 2^2)."""
    codes = torch.randint(0, 16, (n, k), generator=g, dtype=torch.uint8).numpy()
    scales = torch.randint(lo, hi, (n, k // 16), generator=g, dtype=torch.uint8).numpy()
    return mx.pack_fp4_codes(codes), scales


def test_nvfp4_decode_bit_exact_through_identity(dev):
    """out = I @ dequant(W)^T = dequant(W)^T exactly (one product per output, fp32 out, scale2 1): every code at every
    finite positive E4M3 scale byte (0x01 .. 0x7e) through the decode and the scale multiply, on the staged group
    kernel (k = 256) and the unstaged one (k = 160: rows of 80 bytes); gfx950's scaled converts would apply only the
    scale's exponent, so a non-power-of-two scale exposes that mistake."""
    for k in (256, 160):
        n = 126
        codes = np.resize(np.arange(16, dtype=np.uint8), (n, k))
        codes = np.roll(codes, 5, axis=1)
        scales = (1 + (np.arange(n * k // 16).reshape(n, k // 16) * 37) % 126).astype(np.uint8)
        packed = mx.pack_fp4_codes(codes)
        eye = torch.eye(k, dtype=torch.bfloat16)
        one = torch.ones(1, device=dev)
        got = axk.nvfp4_gemm(eye.to(dev), torch.from_numpy(packed).to(dev), torch.from_numpy(scales).to(dev), one,
                             out_dtype=torch.float32).cpu().numpy()
        want = mx.dequant_nvfp4(packed, scales, np.float32(1)).T
        zero = want == 0
        assert (got[zero] == 0).all()
        assert _bits_equal(got[~zero], want[~zero]), f"k={k}"


# decode shapes on the staged group kernel (k a multiple of 256), rows of 80 / 48 bytes on the unstaged kernel, and
# m >= 128 on the prefill GEMM (k a multiple of 64)
@pytest.mark.parametrize("m,n,k", [(1, 16, 256), (1, 4096, 2048), (4, 1000, 2048), (16, 512, 512), (33, 300, 1024),
                                   (1, 100, 160), (5, 64, 96), (128, 512, 1024), (300, 1000, 2048), (200, 64, 320)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_nvfp4_gemm_matches_oracle(dev, m, n, k, out_dtype):
    g = torch.Generator().manual_seed(9000 * m + n + k)
    packed, scales = _nvfp4_weight(n, k, g)
    s2 = np.float32(0.0371)
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    bias = torch.randn(n, generator=g) / 8
    print(f"nvfp4 m={m} n={n} k={k} {out_dtype}", flush=True)
    got = axk.nvfp4_gemm(a.to(dev), torch.from_numpy(packed).to(dev), torch.from_numpy(scales).to(dev),
                         torch.tensor([s2], device=dev), out_dtype=out_dtype, bias=bias.to(dev)).cpu()
    ref = mx.nvfp4_linear(a, packed, scales, s2, bias=bias.to(out_dtype).float())
    torch.testing.assert_close(got.float(), ref.to(out_dtype).float(), **(BF16_TOL if out_dtype == torch.bfloat16 else F32_TOL))


def test_nvfp4_gemm_runtime_scale2_and_quantized_weights(dev):
    """Weights from the host codec (axk.quantize_nvfp4): the product within the bf16 bar of the oracle on the same
    codes; scale2 is a runtime input: doubling it doubles every fp32 output exactly (as the reference's test rescales
    it without repacking, test_nvfp4_lm_head.py:55-60)."""
    g = torch.Generator().manual_seed(93)
    w = torch.randn(513, 1024, generator=g) * 0.1
    packed, scales, s2 = axk.quantize_nvfp4(w)
    a = torch.randn(17, 1024, generator=g).bfloat16()
    pd, sd, s2d = packed.to(dev), scales.to(dev), s2.to(dev)
    got = axk.nvfp4_gemm(a.to(dev), pd, sd, s2d, out_dtype=torch.float32)
    ref = mx.nvfp4_linear(a, packed.view(torch.uint8).numpy(), scales.view(torch.uint8).numpy(), s2.item())
    torch.testing.assert_close(got.cpu(), ref, **F32_TOL)
    twice = axk.nvfp4_gemm(a.to(dev), pd, sd, s2d * 2, out_dtype=torch.float32)
    assert torch.equal(twice, got * 2)


def test_nvfp4_lm_head_vocab_gemv(dev):
    """The NVFP4 LM head at the full vocabulary (248320 x 2048, fp32 logits), M = 1 and 4, against an fp32 matmul
    on the GPU over the dequantised weight (torch ops on the codes, scales and scale2), and a slice of rows against
    the CPU oracle."""
    c = configs.lm_head_nvfp4_case(dev, seed=5, m=4)
    lut = torch.tensor(mx.FP4_LUT, device=dev)
    p = c["w"]
    codes = torch.stack([p & 15, p >> 4], -1).reshape(p.shape[0], -1).long()
    sc = c["s"].view(torch.float8_e4m3fn).float().repeat_interleave(16, -1)
    wf = (lut[codes] * sc) * c["s2"]
    del codes, sc
    for m in (1, 4):
        x = c["x"][:m].contiguous()
        got = axk.nvfp4_gemm(x, c["w"], c["s"], c["s2"], out_dtype=torch.float32)
        ref = (wf @ x.float().t().contiguous()).t()
        torch.testing.assert_close(got, ref, **BF16_TOL)
    del wf
    rows = 3000
    got = axk.nvfp4_gemm(c["x"][:1].contiguous(), c["w"][:rows], c["s"][:rows], c["s2"], out_dtype=torch.float32)
    ref = mx.nvfp4_linear(c["x"][:1].cpu(), c["w"][:rows].cpu().numpy(), c["s"][:rows].cpu().numpy(),
                          c["s2"].item())
    torch.testing.assert_close(got.cpu(), ref, **F32_TOL)
