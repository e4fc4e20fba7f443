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

# m <= 64 takes the skinny kernels (row tiles 1, 2, 4: m = 1, 20, 33, 64); m and n >= 128 the 128 x 128 tiles
# (exact, ragged, a K tail); the rest the 64 x 64 tiles
I8_SHAPES = [(1, 64, 64), (1, 4096, 2048), (20, 1000, 4096), (33, 100, 272), (64, 128, 1024), (65, 96, 128),
             (128, 128, 64), (300, 200, 272), (200, 300, 4096), (130, 100, 512)]


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


# skinny (m <= 64) in both step widths (group 32: 32 K a step; group % 64 == 0: 64) and all row tiles; then the
# 64 x 64 tiles (n < 128) and the 128 x 128 tiles (exact, ragged, a half step of K at the end)
I4_SHAPES = [(1, 64, 64, 32), (7, 130, 96, 32), (20, 64, 256, 32), (40, 80, 512, 32), (32, 256, 2048, 128),
             (48, 512, 4096, 64), (1, 4096, 2048, 128), (65, 96, 96, 32), (130, 200, 2048, 256), (128, 128, 64, 32),
             (256, 300, 96, 32), (200, 512, 1024, 64)]


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


def test_int_gemm_edge_shapes(dev):
    """Empty m returns the empty output; the smallest K (16 for int8, 32 for int4); one output channel; a weight given
    as a transposed view (made contiguous by the wrapper); bias None against an explicit zero bias."""
    a0 = torch.empty(0, 64, dtype=torch.int8, device=dev)
    out = axk.int8_gemm(a0, _i8((8, 64), 1).to(dev), torch.ones(1, device=dev), torch.ones(8, device=dev))
    assert out.shape == (0, 8)
    a, b = _i8((5, 16), 2), _i8((3, 16), 3)
    got = axk.int8_gemm(a.to(dev), b.to(dev), torch.tensor(1.0), torch.tensor(1.0), out_dtype=torch.float32).cpu()
    assert torch.equal(got.double(), (a.long() @ b.long().T).double())
    bt = _i8((96, 1), 4).to(dev).T  # [1, 96] view of a [96, 1] tensor
    a = _i8((4, 96), 5).to(dev)
    got = axk.int8_gemm(a, bt, torch.tensor(0.5), torch.tensor(2.0), out_dtype=torch.float32).cpu()
    assert torch.equal(got.double(), (a.cpu().long() @ bt.cpu().long().T).double())
    x = torch.randn(3, 32, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(dev)
    w, s = _i4(2, 32, 7).to(dev), torch.full((2, 1), 0.25, device=dev)
    z = torch.zeros(2, device=dev)
    assert torch.equal(axk.int4_gemm(x, w, s, out_dtype=torch.float32),
                       axk.int4_gemm(x, w, s, out_dtype=torch.float32, bias=z))


def test_int_gemm_graph_replays(dev):
    """Both entry points captured in one HIP graph: every replay, with eager calls and new inputs copied in between,
    equals the eager result (no memset or allocation inside the calls)."""
    m, n, k = 8, 512, 1024
    a8, b8 = _i8((m, k), 8).to(dev), _i8((n, k), 9).to(dev)
    sa, sb = torch.rand(m, device=dev), torch.rand(n, device=dev)
    xa = torch.randn(m, k, device=dev).to(torch.bfloat16)
    w4, s4 = _i4(n, k, 10).to(dev), torch.rand(n, k // 64, device=dev)
    o8 = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
    o4 = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
    axk.int8_gemm(a8, b8, sa, sb, output=o8)
    axk.int4_gemm(xa, w4, s4, output=o4)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            axk.int8_gemm(a8, b8, sa, sb, output=o8)
            axk.int4_gemm(xa, w4, s4, output=o4)
    torch.cuda.synchronize()
    for rep in range(3):
        a8.copy_(_i8((m, k), 20 + rep).to(dev))
        xa.copy_(torch.randn(m, k, generator=torch.Generator().manual_seed(rep)).to(torch.bfloat16).to(dev))
        want8 = axk.int8_gemm(a8, b8, sa, sb).clone()
        want4 = axk.int4_gemm(xa, w4, s4).clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"int gemm replay {rep}", flush=True)
        assert torch.equal(o8, want8) and torch.equal(o4, want4)
