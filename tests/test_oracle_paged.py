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


def _pcase(seed, qlens, kv_lens, hq=8, hkv=2, d=64, page=32):
    g = torch.Generator().manual_seed(seed)
    return configs.prefill_case(qlens, kv_lens, hq, hkv, d, page, g, extra_pages=3)


def _prefill(c):
    return pa.paged_prefill(c["q"], c["cache"], c["qo_indptr"], c["indptr"], c["indices"], c["last_page_len"],
                            c["scale"])


def test_prefill_matches_sdpa_lower_right_causal():
    # torch's own bottom-right-aligned causal bias (the new tokens are the last of the sequence) with GQA
    from torch.nn.attention.bias import causal_lower_right

    c = _pcase(11, [5, 40, 1, 33], [5, 100, 70, 33])
    got = _prefill(c)
    for b, (ql, L) in enumerate(zip(c["qlens"], c["lens"])):
        k, v = pa.gather_kv(c["cache"], c["indptr"], c["indices"], c["last_page_len"], b)
        q0 = int(c["qo_indptr"][b])
        ref = F.scaled_dot_product_attention(
            c["q"][q0:q0 + ql].float().permute(1, 0, 2)[None], k.float().permute(1, 0, 2)[None],
            v.float().permute(1, 0, 2)[None], attn_mask=causal_lower_right(ql, L), enable_gqa=True, scale=c["scale"],
        )[0].permute(1, 0, 2)
        torch.testing.assert_close(got[q0:q0 + ql], ref, rtol=1e-5, atol=1e-5)


def test_prefill_brute_force_small():
    # per (token, head): softmax over positions 0 .. L - qlen + t by explicit loops
    c = _pcase(12, [3, 2], [4, 2], hq=4, hkv=2, d=8, page=16)
    got = _prefill(c)
    for b, (ql, L) in enumerate(zip(c["qlens"], c["lens"])):
        k, v = pa.gather_kv(c["cache"], c["indptr"], c["indices"], c["last_page_len"], b)
        q0 = int(c["qo_indptr"][b])
        for t in range(ql):
            for h in range(4):
                kvh = h // 2
                scores = [float((c["q"][q0 + t, h].float() * k[j, kvh].float()).sum()) * c["scale"]
                          for j in range(L - ql + t + 1)]
                m = max(scores)
                w = [np.exp(s - m) for s in scores]
                o = sum(wj * v[j, kvh].double() for j, wj in enumerate(w)) / sum(w)
                torch.testing.assert_close(got[q0 + t, h].double(), o, rtol=1e-5, atol=1e-6)


def test_prefill_one_token_equals_decode_and_causality():
    c = _pcase(13, [1, 1, 1], [1, 65, 200])
    got = _prefill(c)
    dec = pa.paged_decode(c["q"], c["cache"], c["indptr"], c["indices"], c["last_page_len"], c["scale"])
    torch.testing.assert_close(got, dec, rtol=1e-6, atol=1e-6)
    # future rows do not matter: rewriting the cache past token t's position leaves row t unchanged
    c = _pcase(14, [30], [90])
    base = _prefill(c)
    k, _ = pa.gather_kv(c["cache"], c["indptr"], c["indices"], c["last_page_len"], 0)
    page = c["cache"].shape[2]
    pos = 90 - 30 + 9  # token 9 of the block
    for j in range(pos + 1, 90):
        pg = int(c["indices"][j // page])
        c["cache"][pg, :, j % page] = 100.0
    after = _prefill(c)
    torch.testing.assert_close(after[:10], base[:10], rtol=0, atol=0)
    assert not torch.allclose(after[10:], base[10:])


def test_prefill_empty_and_short_cache():
    # a sequence without new tokens contributes no rows; rows before the cache start see nothing (zeros)
    c = _pcase(15, [0, 4, 6], [10, 4, 3])
    got = _prefill(c)
    assert got.shape == (10, 8, 64)
    assert not got[4:7].any()  # sequence 2: qlen 6 > 3 cached tokens, its first 3 rows see nothing
    assert got[7:].abs().sum() > 0


# ---- the INT8 cache's quantizer (kv_quant_row, q35_group.py:197-205; KV8=1) ----
def test_int8_quantizer_error_bound_and_scale():
    """|x - bf16(q s)| stays within s / 2 plus the bf16 roundings of 1 / s, x / s and q s; s tracks
    amax / 127 to the two bf16 roundings (a 1 / 128 divisor or a truncating cast fails one of these); the row
    maximum lands on 127 in magnitude up to those roundings (126, or -128 on the negative side)."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(64, 8, 128, generator=g) * torch.logspace(-3, 2, 64)[:, None, None]
    x[5, 2, 17] = 400.0  # an outlier row
    x = x.bfloat16()
    q, s = pa.quant_kv_i8(x)
    deq = pa.dequant_kv_i8(q, s).float()
    sf = s.float()[..., None]
    err = (x.float() - deq).abs()
    # x / s carries the roundings of 1 / s and of the product (2^-8 relative each) into the code; bf16(q s) adds one
    assert (err <= 0.5 * sf + x.float().abs() * 3 * 2.0 ** -8 + 1e-12).all(), float((err - 0.5 * sf).max())
    amax = x.float().abs().amax(-1)
    assert ((s.float() * 127 - amax).abs() <= amax * 2.0 ** -8 * 1.5).all()
    top = q.int().abs().amax(-1)  # -128 is reachable: bf16(-amax * bf16(1 / s)) can round to -128
    assert ((top >= 126) & (top <= 128)).all()
    assert q.dtype == torch.int8 and s.dtype == torch.bfloat16


def test_int8_quantizer_zero_rows_and_rounding_to_nearest():
    """A zero row keeps the 1e-5 floor (codes 0, s = bf16(bf16(1e-5) / 127)); codes round to nearest (not toward
    zero): x = (k + 0.4) s gives k, x = (k + 0.6) s gives k + 1 away from the row maximum."""
    z = torch.zeros(1, 128).bfloat16()
    q, s = pa.quant_kv_i8(z)
    assert not q.any()
    assert float(s) == float((torch.tensor(1e-5).bfloat16().float() * torch.tensor(1 / 127).bfloat16().float())
                              .bfloat16())
    # a row whose max is exactly 127 s (s a power of two: every product exact)
    s0 = 2.0 ** -4
    vals = torch.tensor([127.0, 10.4, 10.6, -20.4, -20.6, 0.4, 0.6, -3.0]) * s0
    row = torch.zeros(1, 128)
    row[0, :8] = vals
    q, s = pa.quant_kv_i8(row.bfloat16())
    assert q[0, :8].tolist() == [127, 10, 11, -20, -21, 0, 1, -3]


def test_int8_quantizer_ties_and_saturation_choice():
    """The oracle's stated choice where the reference is silent (parity unpinned against the AX cast): on rows whose
    scale is exactly 1, every code equals Python's round-half-to-even of the exact half-integer, clamped to [-128, 127]
    (so 127.5 saturates to 127 and -127.5 lands on -128)."""
    d = 64
    half = torch.arange(d, dtype=torch.float32) - d // 2 + 0.5
    row = half.clone()
    row[0], row[1] = 127.5, -127.5
    q, s = pa.quant_kv_i8(row.bfloat16()[None])
    assert float(s[0]) == 1.0
    want = [max(-128, min(127, round(float(x)))) for x in row]
    assert q[0].tolist() == want
