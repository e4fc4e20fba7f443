"""Pins the paged-attention oracle (CPU only)."""
import numpy as np
import torch
import torch.nn.functional as F

from axk import configs
from oracle import paged_attn as pa


def _case(seed=0, lens=(1, 63, 64, 65, 200), hq=8, hkv=2, d=64, page=32):
    g = torch.Generator().manual_seed(seed)
    return configs.paged_case(list(lens), hq, hkv, d, page, g, extra_pages=3)


def test_gather_brute_force_index_math():
    c = _case()
    page = c["cache"].shape[2]
    for b, L in enumerate(c["lens"]):
        k, v = pa.gather_kv(c["cache"], c["indptr"], c["indices"], c["last_page_len"], b)
        assert k.shape[0] == L
        for t in range(L):  # token t lives in logical page t // page at slot t % page
            phys = int(c["indices"][int(c["indptr"][b]) + t // page])
            assert torch.equal(k[t], c["cache"][phys, 0, t % page])
            assert torch.equal(v[t], c["cache"][phys, 1, t % page])


def test_matches_torch_sdpa_gqa():
    # the reference's golden call: F.scaled_dot_product_attention(..., enable_gqa=True)
    # (models/qwen35_35b_a3b/sgl/tests/test_qwen35_runtime.py:79-84)
    c = _case(1)
    got = pa.paged_decode(c["q"], c["cache"], c["indptr"], c["indices"], c["last_page_len"], c["scale"])
    for b in range(len(c["lens"])):
        k, v = pa.gather_kv(c["cache"], c["indptr"], c["indices"], c["last_page_len"], b)
        ref = F.scaled_dot_product_attention(
            c["q"][b : b + 1, :, None].float(), k.float().permute(1, 0, 2)[None], v.float().permute(1, 0, 2)[None],
            enable_gqa=True, scale=c["scale"],
        )[0, :, 0]
        torch.testing.assert_close(got[b], ref, rtol=1e-5, atol=1e-5)


def test_pool_permutation_invariance():
    c = _case(2)
    base = pa.paged_decode(c["q"], c["cache"], c["indptr"], c["indices"], c["last_page_len"], c["scale"])
    pool = c["cache"].shape[0]
    perm = torch.randperm(pool, generator=torch.Generator().manual_seed(9))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(pool)
    cache2 = c["cache"][perm]  # new slot i holds old page perm[i]
    idx2 = inv[c["indices"].long()].to(torch.int32)
    got = pa.paged_decode(c["q"], cache2, c["indptr"], idx2, c["last_page_len"], c["scale"])
    torch.testing.assert_close(got, base, rtol=0, atol=0)


def test_single_page_equals_dense_attention_and_tail_mask():
    g = torch.Generator().manual_seed(3)
    c = configs.paged_case([20], 4, 4, 64, 32, g)
    got = pa.paged_decode(c["q"], c["cache"], c["indptr"], c["indices"], c["last_page_len"], 0.125)
    page = int(c["indices"][0])
    k = c["cache"][page, 0, :20].float()  # slots 20..31 of the page are not part of the sequence
    v = c["cache"][page, 1, :20].float()
    for h in range(4):
        p = torch.softmax(c["q"][0, h].float() @ k[:, h].T * 0.125, -1)
        torch.testing.assert_close(got[0, h], p @ v[:, h], rtol=1e-5, atol=1e-5)


def test_store_paged_kv_row_math():
    c = _case(4)
    k = torch.randn(2, 2, 64).bfloat16()
    v = torch.randn(2, 2, 64).bfloat16()
    loc = np.array([[3, 5], [0, 31]], dtype=np.int32)
    out = pa.store_paged_kv(c["cache"], k, v, loc)
    flat = out.reshape(-1, 2, 64)  # rows (page * 2 + plane) * page_size + offset (flash_attn.py:68-70)
    for b in range(2):
        for plane, src in ((0, k), (1, v)):
            row = (int(loc[b, 0]) * 2 + plane) * 32 + int(loc[b, 1])
            assert torch.equal(flat[row], src[b])
    diff = (out != c["cache"]).reshape(out.shape[0], 2, 32, -1).any(-1)
    assert int(diff.sum()) <= 4



def test_fp8_kv_codec_pinned():
    """The FP8 cache codec against an independent E4M3 decode (OCP e4m3fn: bias 7, no infinities, S.1111.111 = NaN)
    and the round trip of every finite code through bf16(x * S) with S = 8; past 464 after scaling -> NaN."""
    import math

    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    vals = pa.dequant_kv_fp8(codes, 8.0).float()
    for c in range(256):
        s, e, m = c >> 7, (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            assert math.isnan(vals[c])
            continue
        mag = (m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
        assert vals[c].item() == (-mag if s else mag) / 8.0, c
    finite = ~torch.isnan(vals)
    assert torch.equal(pa.quant_kv_fp8(vals[finite].bfloat16(), 8.0), codes[finite])
    big = pa.quant_kv_fp8(torch.tensor([60.0, -61.0, 58.0]).bfloat16(), 8.0)  # 480 -> NaN; 464 ties to 448
    assert big.tolist() == [0x7F, 0xFF, 0x7E]
