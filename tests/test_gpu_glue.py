"""GPU parity of the per-layer glue kernels (axk.glue over the C-ABI) against the oracle.

Bar: bf16 outputs within rel 2e-2 / abs 1e-2 of the oracle (which keeps the reference's rounding points);
exact where the operation is exact (the residual sum, the conv state, pass-through channels).
"""
import pytest
import torch

from axk import glue
from oracle import layer

pytestmark = pytest.mark.gpu
TOL = dict(rtol=2e-2, atol=1e-2)


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _close(got, ref):
    torch.testing.assert_close(got.float().cpu(), ref.float(), **TOL)


# rows of 16-lane groups (n <= 128: a partial last workgroup at 5 and 33 rows), 32-lane groups (136, 256), waves,
# workgroups and the looping kernel (n > 8192)
@pytest.mark.parametrize("rows,n", [(8, 4096), (3, 2048), (64, 128), (5, 8), (2, 8192), (4, 6144), (3, 1032),
                                    (2, 16384), (9, 1024), (5, 128), (33, 128), (7, 256), (3, 136)])
def test_rmsnorm(dev, rows, n):
    g = _g(rows + n)
    x = torch.randn(rows, n, generator=g).bfloat16() * 3
    w = torch.rand(n, generator=g) + 0.5
    _close(glue.rmsnorm(x.to(dev), w.to(dev)), layer.rmsnorm(x, w))


def test_rmsnorm_strided_rows_and_output_buffer(dev):
    g = _g(1)
    qg = torch.randn(4, 6, 512, generator=g).bfloat16()  # [B, heads, 2D]: the q half of each row
    w = torch.rand(256, generator=g) + 0.5
    q = qg.to(dev)[..., :256].reshape(24, 256)
    out = torch.empty(24, 256, dtype=torch.bfloat16, device=dev)
    got = glue.rmsnorm(q, w.to(dev), out=out)
    assert got.data_ptr() == out.data_ptr()
    _close(got, layer.rmsnorm(qg[..., :256].reshape(24, 256), w))


@pytest.mark.parametrize("rows,n", [(8, 4096), (3, 512), (2, 16384)])
def test_add_rmsnorm(dev, rows, n):
    g = _g(2 + n)
    x = torch.randn(rows, n, generator=g).bfloat16()
    y = torch.randn(rows, n, generator=g).bfloat16()
    w = torch.rand(n, generator=g) + 0.5
    s, n = glue.add_rmsnorm(x.to(dev), y.to(dev), w.to(dev))
    rs, rn = layer.add_rmsnorm(x, y, w)
    assert torch.equal(s.cpu().view(torch.int16), rs.view(torch.int16))
    _close(n, rn)


@pytest.mark.parametrize("rows", [8 * 32, 13, 4096 * 32])
def test_gated_rmsnorm_silu(dev, rows):
    g = _g(3)
    x = torch.randn(rows, 128, generator=g).bfloat16()
    z = torch.randn(rows, 128, generator=g).bfloat16()
    w = torch.rand(128, generator=g) + 0.5
    _close(glue.gated_rmsnorm_silu(x.to(dev), w.to(dev), z.to(dev)), layer.gated_rmsnorm_silu(x, w, z))


# one token; a channel count that is not a multiple of 8 (the per-channel kernel); fewer tokens than K - 1; several
# 32-token tiles with a one-token tail; eight taps; config 2b's conv width at prefill length
@pytest.mark.parametrize("b,t,c,k", [(8, 1, 8192, 4), (2, 5, 200, 4), (1, 3, 64, 2), (3, 2, 16, 1), (2, 2, 64, 4),
                                     (2, 33, 256, 4), (3, 100, 136, 8), (1, 4096, 8192, 4)])
def test_causal_conv1d_silu(dev, b, t, c, k):
    g = _g(b * 10 + t)
    x = torch.randn(b, t, c, generator=g).bfloat16()
    w = (torch.randn(c, k, generator=g) * 0.5).bfloat16()
    st = torch.randn(b, k - 1, c, generator=g).bfloat16()
    out, so = glue.causal_conv1d_silu(x.to(dev), w.to(dev), st.to(dev))
    ro, rs = layer.causal_conv1d_silu(x, w, st)
    _close(out, ro)
    assert torch.equal(so.cpu(), rs)


def test_causal_conv1d_in_place_state_over_many_tiles(dev):
    """An in-place conv state with several token tiles: the tile that reads the state is the one that rewrites it."""
    g = _g(5)
    x = torch.randn(2, 150, 256, generator=g).bfloat16()
    w = (torch.randn(256, 4, generator=g) * 0.5).bfloat16()
    st = torch.randn(2, 3, 256, generator=g).bfloat16()
    ref_out, ref_st = layer.causal_conv1d_silu(x, w, st)
    sd = st.to(dev)
    o1, _ = glue.causal_conv1d_silu(x[:, :100].contiguous().to(dev), w.to(dev), sd, state_out=sd)
    o2, _ = glue.causal_conv1d_silu(x[:, 100:].contiguous().to(dev), w.to(dev), sd, state_out=sd)
    _close(torch.cat((o1, o2), 1), ref_out)
    assert torch.equal(sd.cpu(), ref_st)


def test_causal_conv1d_in_place_state_and_continuation(dev):
    g = _g(4)
    x = torch.randn(2, 6, 96, generator=g).bfloat16()
    w = (torch.randn(96, 4, generator=g) * 0.5).bfloat16()
    st = torch.randn(2, 3, 96, generator=g).bfloat16()
    ref_out, ref_st = layer.causal_conv1d_silu(x, w, st)
    sd = st.to(dev)
    o1, s1 = glue.causal_conv1d_silu(x[:, :4].contiguous().to(dev), w.to(dev), sd, state_out=sd)
    o2, s2 = glue.causal_conv1d_silu(x[:, 4:].contiguous().to(dev), w.to(dev), sd, state_out=sd)
    assert s1.data_ptr() == sd.data_ptr() and s2.data_ptr() == sd.data_ptr()
    _close(torch.cat((o1, o2), 1), ref_out)
    assert torch.equal(sd.cpu(), ref_st)


@pytest.mark.parametrize("b,h,d,rot", [(8, 32, 256, 64), (3, 4, 256, 64), (2, 5, 128, 32), (4, 2, 256, 0),
                                       (1, 3, 64, 64)])
def test_qk_norm_rope(dev, b, h, d, rot):
    g = _g(b * h + d + rot)
    x = torch.randn(b, h, d, generator=g).bfloat16() * 2
    w = torch.rand(d, generator=g) + 0.5
    pos = torch.randint(0, 131072, (b,), generator=g)
    cos, sin = layer.rope_cos_sin(pos, max(rot, 2), 10_000_000.0)
    cos, sin = cos[:, : rot // 2].contiguous(), sin[:, : rot // 2].contiguous()
    got = glue.qk_norm_rope(x.to(dev), w.to(dev), cos.to(dev), sin.to(dev), rot)
    ref = layer.qk_norm_rope(x, w, cos, sin, rot)
    _close(got, ref)


def test_qk_norm_rope_strided_q_half(dev):
    g = _g(5)
    qg = torch.randn(8, 16, 512, generator=g).bfloat16()  # [B, HQ, q | gate]
    w = torch.rand(256, generator=g) + 0.5
    cos, sin = layer.rope_cos_sin(torch.arange(8) * 1000, 64, 10_000_000.0)
    got = glue.qk_norm_rope(qg.to(dev)[..., :256], w.to(dev), cos.to(dev), sin.to(dev), 64)
    _close(got, layer.qk_norm_rope(qg[..., :256], w, cos, sin, 64))


def test_gates_and_add(dev):
    g = _g(6)
    a = torch.randn(8, 32, 256, generator=g).bfloat16()
    qg = torch.randn(8, 32, 512, generator=g).bfloat16()
    _close(glue.sigmoid_mul(a.to(dev), qg.to(dev)[..., 256:]), layer.sigmoid_mul(a, qg[..., 256:]))
    u = torch.randn(8, 12288, generator=g).bfloat16()
    v = torch.randn(8, 12288, generator=g).bfloat16()
    _close(glue.silu_mul(u.to(dev), v.to(dev)), layer.silu_mul(u, v))
    assert torch.equal(glue.add(u.to(dev), v.to(dev)).cpu().view(torch.int16), layer.add(u, v).view(torch.int16))


def test_contract_errors(dev):
    x = torch.randn(4, 12, dtype=torch.bfloat16, device=dev)
    with pytest.raises(Exception):
        glue.rmsnorm(x, torch.ones(12, device=dev))  # n % 8 != 0
    with pytest.raises(ValueError):
        glue.silu_mul(x, torch.randn(4, 8, dtype=torch.bfloat16, device=dev))
    with pytest.raises(Exception):
        glue.causal_conv1d_silu(torch.randn(1, 1, 8, dtype=torch.bfloat16, device=dev),
                                torch.randn(8, 9, dtype=torch.bfloat16, device=dev),
                                torch.zeros(1, 8, 8, dtype=torch.bfloat16, device=dev))  # kernel > 8
