"""GPU parity of the integer-weight linears (sgl int8_gemm / int4_gemm) against the oracle.

Bar: bit-exact where the arithmetic is exact (int8 sums under power-of-two scales; int4 weights with integer
activations and power-of-two group scales, fp32 output); otherwise bf16 outputs within rel 2e-2 / abs 1e-2 of the
oracle and fp32 outputs within rel 1e-4 / abs 1e-4 (the kernel scales the exact integer sum once where the reference
scales each operand, so the two differ by fp32 rounding).
"""
import numpy as np
import pytest
import torch

import axk
from oracle import mx

pytestmark = pytest.mark.gpu

BF16_TOL = dict(rtol=2e-2, atol=1e-2)
F32_TOL = dict(rtol=1e-4, atol=1e-4)

# m <= 64 takes the skinny kernels (row tiles 1, 2, 4: m = 1, 20, 33, 64), larger m the 64 x 64 tiles
I8_SHAPES = [(1, 64, 64), (1, 4096, 2048), (20, 1000, 4096), (33, 100, 272), (64, 128, 1024), (65, 96, 128),
             (200, 300, 4096)]


def _i8(shape, seed):
    return torch.randint(-128, 128, shape, generator=torch.Generator().manual_seed(seed), dtype=torch.int8)


@pytest.mark.parametrize("m,n,k", I8_SHAPES)
def test_int8_gemm_exact_under_power_of_two_scales(dev, m, n, k):
    a, b = _i8((m, k), m + k), _i8((n, k), n + 3 * k)
    g = torch.Generator().manual_seed(n)
    sa = torch.exp2(torch.randint(-8, 3, (m,), generator=g).float())
    sb = torch.exp2(torch.randint(-8, 3, (n,), generator=g).float())
    got = axk.int8_gemm(a.to(dev), b.to(dev), sa.to(dev), sb.to(dev), out_dtype=torch.float32).cpu()
    exact = (a.long() @ b.long().T).double() * sa.double()[:, None] * sb.double()[None, :]
    assert torch.equal(got.double(), exact)
    want = mx.int8_linear(a.numpy(), b.numpy(), sa.numpy(), sb.numpy(), torch.float32)
    assert torch.equal(got, want)


@pytest.mark.parametrize("m,n,k", I8_SHAPES)
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_int8_gemm_matches_oracle(dev, m, n, k, out_dtype):
    a, b = _i8((m, k), 7 * m + k), _i8((n, k), 5 * n + k)
    g = torch.Generator().manual_seed(m * n)
    sa = (torch.rand(m, generator=g) + 0.5) / (127 * k ** 0.5)
    sb = (torch.rand(n, generator=g) + 0.5) / 127
    bias = torch.randn(n, generator=g)
    got = axk.int8_gemm(a.to(dev), b.to(dev), sa.to(dev), sb.to(dev), out_dtype=out_dtype, bias=bias.to(dev))
    want = mx.int8_linear(a.numpy(), b.numpy(), sa.numpy(), sb.numpy(), out_dtype, bias)
    assert got.dtype == out_dtype
    torch.testing.assert_close(got.float().cpu(), want, **(BF16_TOL if out_dtype == torch.bfloat16 else F32_TOL))


def test_int8_gemm_scalar_scales_and_strided_activation(dev):
    """Scalar scales broadcast as _normalize_scale does; an activation row stride wider than K is read in place."""
    m, n, k = 48, 200, 512
    base, b = _i8((m, k + 64), 1).to(dev), _i8((n, k), 2).to(dev)
    a = base[:, :k]
    got = axk.int8_gemm(a, b, torch.tensor(0.5, device=dev), torch.tensor([0.25], device=dev),
                        out_dtype=torch.float32)
    exact = (a.cpu().long() @ b.cpu().long().T).double() * 0.125
    assert torch.equal(got.cpu().double(), exact)
    out = torch.full((m, n), 7.0, device=dev, dtype=torch.bfloat16)
    assert axk.int8_gemm(a, b, torch.tensor(0.5, device=dev), torch.tensor([0.25], device=dev), output=out) is out
    assert torch.equal(out.cpu(), exact.float().to(torch.bfloat16))


# skinny (m <= 64) in both step widths (group 32: 32 K a step; group % 64 == 0: 64) and all row tiles; then tiled
I4_SHAPES = [(1, 64, 64, 32), (7, 130, 96, 32), (20, 64, 256, 32), (40, 80, 512, 32), (32, 256, 2048, 128),
             (48, 512, 4096, 64), (1, 4096, 2048, 128), (65, 96, 96, 32), (130, 200, 2048, 256)]


def _i4(n, k, seed):
    return torch.randint(-8, 8, (n, k), generator=torch.Generator().manual_seed(seed), dtype=torch.int8)


@pytest.mark.parametrize("m,n,k,g", I4_SHAPES)
def test_int4_gemm_exact_with_integer_activations(dev, m, n, k, g):
    """Integer activations and power-of-two group scales make every partial exact: the output is bit-exact."""
    gen = torch.Generator().manual_seed(k + g)
    a = torch.randint(-16, 17, (m, k), generator=gen).to(torch.bfloat16)
    w = _i4(n, k, n)
    s = torch.exp2(torch.randint(-6, 2, (n, k // g), generator=gen).float())
    got = axk.int4_gemm(a.to(dev), w.to(dev), s.to(dev), out_dtype=torch.float32).cpu()
    exact = torch.einsum("mgq,ngq,ng->mn", a.double().reshape(m, k // g, g), w.double().reshape(n, k // g, g),
                         s.double())
    assert torch.equal(got.double(), exact)


@pytest.mark.parametrize("m,n,k,g", I4_SHAPES)
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_int4_gemm_matches_oracle(dev, m, n, k, g, out_dtype):
    gen = torch.Generator().manual_seed(m + n + k)
    a = torch.randn(m, k, generator=gen).to(torch.bfloat16)
    w = _i4(n, k, k)
    s = (torch.rand(n, k // g, generator=gen) + 0.5) / (8 * k ** 0.5)
    bias = torch.randn(n, generator=gen).to(out_dtype)
    got = axk.int4_gemm(a.to(dev), w.to(dev), s.to(dev), out_dtype=out_dtype, bias=bias.to(dev))
    want = mx.int4_linear(a, w.numpy(), s.numpy(), bias)
    torch.testing.assert_close(got.float().cpu(), want, **(BF16_TOL if out_dtype == torch.bfloat16 else F32_TOL))
