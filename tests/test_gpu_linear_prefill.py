"""GPU parity of the runtime-weight linears at prefill row counts (m >= 128: the dense LDS-pipelined GEMM path of the
same entry points), against the oracle: MXFP4, FP8 per-channel (with and without the activation row scale), MXFP8
E4M3 / E5M2, ragged m and n, bf16 and fp32 outputs, bias. Bar: bf16 outputs within rel 2e-2 / abs 1e-2 (the per-op
bar); fp32 outputs within the fp32 summation-order bound of their terms' magnitudes. The decode layers at more than
128 sequences take the same path for every grouped projection (SwiGLU, residual, plain, fp32 for the MoE block's
shared expert): they are checked against the oracle at the bars of tests/test_gpu_layer.py and
tests/test_gpu_layer_moe.py."""
import numpy as np
import pytest
import torch

import axk
from axk import configs, layer
from oracle import layer as olayer
from oracle import mx

pytestmark = pytest.mark.gpu
BF16_TOL = dict(rtol=2e-2, atol=1e-2)
FUSED_TOL = dict(rtol=5e-2, atol=0.0625)
STATE_TOL = dict(rtol=5e-2, atol=3e-3)


def _close(got, ref, out_dtype, a, w):
    if out_dtype == torch.bfloat16:
        torch.testing.assert_close(got.float().cpu(), ref.to(out_dtype).float(), **BF16_TOL)
    else:
        mag = a.float().abs() @ w.abs().T
        err = (got.float().cpu() - ref).abs()
        assert (err <= 1e-3 + 1e-3 * ref.abs() + mag * 2.0 ** -20).all(), float((err - mag * 2.0 ** -20).max())


@pytest.mark.parametrize("m,n,k", [(128, 256, 256), (300, 1000, 512), (4096, 512, 2048), (200, 4096, 4096),
                                   (129, 17, 8192)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_mxfp4_gemm_prefill_rows(dev, m, n, k, out_dtype):
    print(f"mxfp4 m={m} n={n} k={k} {out_dtype}", flush=True)
    g = torch.Generator().manual_seed(m * 7 + n + k)
    packed, scales = configs.mxfp4_weight(n, k, g)
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    bias = torch.randn(n, generator=g) / 8
    ref = mx.mx_linear(a, packed.numpy(), scales.numpy(), bias.to(out_dtype))
    got = axk.mxfp4_gemm(a.to(dev), packed.to(dev), scales.to(dev), out_dtype=out_dtype, bias=bias.to(dev))
    _close(got, ref, out_dtype, a, torch.from_numpy(mx.dequant_mxfp4(packed.numpy(), scales.numpy())))


@pytest.mark.parametrize("m,n,k,row_scale", [(256, 384, 1024, False), (333, 1024, 4096, True)])
def test_fp8_gemm_prefill_rows(dev, m, n, k, row_scale):
    g = torch.Generator().manual_seed(m + n + k)
    w = (torch.randn(n, k, generator=g) * 0.5).to(torch.float8_e4m3fn).view(torch.uint8).contiguous()
    scale_b = torch.rand(n, generator=g) * 0.02 + 0.01
    scale_a = torch.rand(m, generator=g) + 0.5 if row_scale else None
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    ref = mx.fp8_linear(a, w.numpy(), scale_a, scale_b)
    got = axk.fp8_gemm(a.to(dev), w.to(dev), None if scale_a is None else scale_a.to(dev), scale_b.to(dev))
    torch.testing.assert_close(got.float().cpu(), ref.to(torch.bfloat16).float(), **BF16_TOL)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("m,n,k", [(192, 512, 1024), (1000, 300, 2048)])
def test_mxfp8_gemm_prefill_rows(dev, fmt, m, n, k):
    g = torch.Generator().manual_seed(m + n + k + (1 if fmt == "e5m2" else 0))
    w = (torch.randn(n, k, generator=g) * 0.02).numpy()
    codes, scales = mx.quant_mxfp8(w, fmt)
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    ref = mx.mxfp8_linear(a, codes, scales, fmt)
    got = axk.mxfp8_gemm(a.to(dev), torch.from_numpy(codes).to(dev), torch.from_numpy(scales).to(dev), fmt=fmt)
    torch.testing.assert_close(got.float().cpu(), ref.to(torch.bfloat16).float(), **BF16_TOL)


@pytest.mark.parametrize("proj_fmt,mlp_fmt", [("fp8", "mxfp4"), ("mxfp8", "mxfp8")])
def test_gdn_layer_decode_at_130_sequences(dev, proj_fmt, mlp_fmt):
    """130 sequences: the qkv | z | b | a group (with the conv epilogue) stays on the group kernel, the output
    projection and the MLP (SwiGLU, residual) take the dense GEMM."""
    g = torch.Generator().manual_seed(130)
    b, h, f, nk, nv = 130, 256, 512, 2, 4
    w = configs.gdn_layer_weights(g, h, f, nk, nv, proj_fmt=proj_fmt, mlp_fmt=mlp_fmt)
    x = torch.randn(b, h, generator=g).bfloat16()
    st = torch.randn(b, nv, 128, 128, generator=g) * 0.02
    cv = torch.randn(b, 3, 2 * nk * 128 + nv * 128, generator=g).bfloat16()
    out, so, co = layer.gdn_layer_decode(x.to(dev), {n: v.to(dev) for n, v in w.items()}, st.to(dev), cv.to(dev),
                                         nk, nv, proj_fmt=proj_fmt, mlp_fmt=mlp_fmt)
    ro, rs, rc = olayer.gdn_layer_decode(x, w, st, cv, nk, nv, proj_fmt=proj_fmt, mlp_fmt=mlp_fmt)
    torch.testing.assert_close(out.float().cpu(), ro.float(), **FUSED_TOL)
    torch.testing.assert_close(so.cpu(), rs, **STATE_TOL)
    assert torch.equal(co[:, :-1].cpu(), rc[:, :-1])


def test_attn_layer_decode_at_160_sequences(dev):
    """160 sequences: q | k | v, the o projection and the MLP all take the dense GEMM."""
    g = torch.Generator().manual_seed(160)
    hq, hkv, d, h, f = 4, 2, 256, 256, 512
    lens = [1 + (37 * i) % 300 for i in range(160)]
    w = configs.attn_layer_weights(g, h, f, hq, hkv, d)
    c = configs.append_token_case(lens, hq, hkv, d, 64, g)
    x = torch.randn(len(lens), h, generator=g).bfloat16()
    cos, sin = olayer.rope_cos_sin(c["pos"], 64, 10_000_000.0)
    cache = c["cache"].to(dev)
    out = layer.attn_layer_decode(x.to(dev), {n: v.to(dev) for n, v in w.items()}, cos.to(dev), sin.to(dev), cache,
                                  c["indptr"].to(dev), c["indices"].to(dev), c["last_page_len"].to(dev),
                                  c["loc"].to(dev), hq, 64)
    ro, _ = olayer.attn_layer_decode(x, w, cos, sin, c["cache"], c["indptr"], c["indices"], c["last_page_len"],
                                     c["loc"], hq, 64)
    torch.testing.assert_close(out.float().cpu(), ro.float(), **FUSED_TOL)


def test_moe_layer_decode_at_144_sequences(dev):
    """The MoE block's shared expert at 144 rows through the dense GEMM (SwiGLU, then fp32 down into the combine)."""
    from oracle import moe as omoe

    g = torch.Generator().manual_seed(144)
    b, h, f, nk, nv, e, fe, k = 144, 256, 256, 2, 4, 16, 256, 4
    w = configs.gdn_layer_weights(g, h, f, nk, nv, proj_fmt="mxfp8", mlp_fmt="mxfp8")
    blk = configs.moe_block(g, h, e, fe, k)
    x = torch.randn(b, h, generator=g).bfloat16()
    st = torch.randn(b, nv, 128, 128, generator=g) * 0.02
    cv = torch.randn(b, 3, 2 * nk * 128 + nv * 128, generator=g).bfloat16()
    r = dict(logits=torch.empty(b, e, device=dev), topk_ids=torch.empty(b, k, dtype=torch.int32, device=dev),
             topk_weights=torch.empty(b, k, device=dev))
    bd = {n: (v.to(dev) if torch.is_tensor(v) else v) for n, v in blk.items()}
    out, _, _ = layer.gdn_layer_decode(x.to(dev), {n: v.to(dev) for n, v in w.items()}, st.to(dev), cv.to(dev), nk,
                                       nv, proj_fmt="mxfp8", mlp_fmt="mxfp8", moe=dict(bd, **r))
    ids, wts = r["topk_ids"].cpu(), r["topk_weights"].cpu()
    assert torch.equal(ids, omoe.route(r["logits"].cpu(), k, True)[0])
    y, _, _ = olayer.gdn_layer_half(x, w, st, cv, nk, nv, proj_fmt="mxfp8")
    base, routed, slack, _, _, _ = olayer.moe_block_parts(x, y, w, blk, fmt="mxfp8", ids=ids.long(), wts=wts)
    ref = (base + routed).bfloat16().float()
    d = (out.float().cpu() - ref).abs()
    assert (d <= FUSED_TOL["atol"] + FUSED_TOL["rtol"] * ref.abs() + slack).all()
