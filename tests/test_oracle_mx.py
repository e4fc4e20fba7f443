"""Pins the MX codec / linear oracle (CPU only).

Checks chosen so a plausible mistake (nibble order, sign of code 8, scale bias, denormal / inf scale
bytes, transposed weight) fails: exhaustive 16 x 256 table vs closed form and vs torch's own E8M0
dtype, the reference's FP4 table, the C restatement vs numpy, quantiser brute force and round trip.
"""
import numpy as np
import pytest
import torch

from oracle import _c, mx

# models/qwen35_35b_a3b/sgl/tests/test_gdn_attn.py:157 (the reference's FP4 code table, data)
REF_FP4_LUT = [0, 0.5, 1, 1.5, 2, 3, 4, 6, 0, -0.5, -1, -1.5, -2, -3, -4, -6]


def _bits_equal(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    both_nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(both_nan | (a.view(np.uint32) == b.view(np.uint32))))


def test_e2m1_table_matches_reference_and_bit_layout():
    np.testing.assert_array_equal(mx.FP4_LUT, np.array(REF_FP4_LUT, np.float32))
    # independent derivation from the E2M1 layout s|e1 e0|m0, bias 1
    for c in range(16):
        s, e, m = c >> 3, (c >> 1) & 3, c & 1
        v = m * 0.5 if e == 0 else 2.0 ** (e - 1) * (1 + m / 2)
        assert mx.FP4_LUT[c] == (-v if s else v)
    assert np.signbit(mx.FP4_LUT[8]) and mx.FP4_LUT[8] == 0.0  # code 8 is -0


def test_e8m0_matches_torch_exp2_and_e8m0_dtype():
    s = np.arange(256)
    ours = mx.e8m0_to_f32(s)
    ref = torch.exp2(torch.arange(256).float() - 127).numpy()  # q35_moe.py:63
    assert _bits_equal(ours, ref)
    tdt = torch.arange(256, dtype=torch.uint8).view(torch.float8_e8m0fnu).float().numpy()
    assert _bits_equal(ours[:255], tdt[:255])  # 0xFF: torch says NaN (OCP), the reference's exp2 gives inf
    assert np.isinf(ours[255]) and ours[0] == np.float32(2.0 ** -127)


def test_exhaustive_code_scale_table():
    codes = np.repeat(np.arange(16, dtype=np.uint8)[None, :], 256, 0)  # [256 scales, 16 codes]
    codes = np.tile(codes, (1, 2))  # 32 codes per row = one block
    packed = mx.pack_fp4_codes(codes)
    scales = np.arange(256, dtype=np.uint8)[:, None]
    got = mx.dequant_mxfp4(packed, scales)
    expect = np.empty_like(got)
    for s in range(256):
        # closed form in float64, then one rounding to fp32 (exact: E2M1 x 2^e is representable)
        factor = np.float64(2.0) ** (s - 127) if s < 255 else np.inf
        for j in range(32):
            c = j % 16
            v = -0.0 if c == 8 else np.float64(REF_FP4_LUT[c])
            with np.errstate(invalid="ignore", over="ignore"):
                expect[s, j] = np.float32(v * factor)
    assert _bits_equal(got, expect)
    assert _bits_equal(_c.mxfp4_dequant(packed, scales), got)


def test_pack_layout_matches_reference_bit_method():
    rng = np.random.default_rng(0)
    logical = rng.integers(0, 16, size=(7, 64), dtype=np.uint8)
    # test_gdn_attn.py:160-166 packs with numpy bit operations, low nibble = even column
    bits = np.unpackbits(logical.reshape(-1), bitorder="little").reshape(-1, 8)[:, :4]
    ref = np.packbits(bits, bitorder="little").reshape(7, 32)
    np.testing.assert_array_equal(mx.pack_fp4_codes(logical), ref)
    np.testing.assert_array_equal(mx.unpack_fp4_codes(ref), logical)


def test_pack_and_decode_reference_kat():
    # known-answer data of test_nvfp4_lm_head.py:19-30: source values and the codes the reference's quantiser
    # assigns them (its rounding sends ties to the even code); packed low nibble = even column
    source = [0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5, 6, -0.25, -0.75, -1.25, -1.75, -2.5, -3.5, -5]
    codes = np.array([0, 0, 2, 2, 4, 4, 6, 6, 7, 8, 10, 10, 12, 12, 14, 14], np.uint8)
    expect_bytes = codes[::2] | (codes[1::2] << 4)
    np.testing.assert_array_equal(mx.pack_fp4_codes(codes[None, :])[0], expect_bytes)
    # decoding the KAT's bytes at scale 2^0 gives the E2M1 grid points the KAT names, and each one lies
    # within half a grid step of its source value
    dec = mx.dequant_mxfp4(np.concatenate([expect_bytes] * 2)[None, :], np.array([[127]], np.uint8))[0, :16]
    np.testing.assert_array_equal(dec, np.array(REF_FP4_LUT, np.float32)[codes])
    step = np.array([0.5 if abs(v) <= 2 else 1.0 if abs(v) <= 4 else 2.0 for v in source])
    assert np.all(np.abs(dec - np.array(source)) <= step / 2)


def test_c_oracle_matches_numpy_random():
    rng = np.random.default_rng(1)
    packed = rng.integers(0, 256, size=(33, 96), dtype=np.uint8)
    scales = rng.integers(0, 256, size=(33, 6), dtype=np.uint8)
    assert _bits_equal(_c.mxfp4_dequant(packed, scales), mx.dequant_mxfp4(packed, scales))


def test_linear_golden_vs_float64():
    rng = np.random.default_rng(2)
    n, k, m = 40, 256, 3
    packed = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scales = rng.integers(119, 124, size=(n, k // 32), dtype=np.uint8)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).bfloat16()
    w64 = mx.dequant_mxfp4(packed, scales).astype(np.float64)
    ref64 = x.double().numpy() @ w64.T
    got = mx.mx_linear(x, packed, scales).numpy()
    np.testing.assert_allclose(got, ref64, rtol=1e-5, atol=1e-5)
    xb = x.view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_allclose(_c.mxfp4_linear(xb, packed, scales, nthreads=2), ref64, rtol=1e-5, atol=1e-5)
    # a transposed or mis-ordered weight must not pass
    assert not np.allclose(x.double().numpy() @ w64[::-1].T, ref64, rtol=1e-3, atol=1e-3)


def test_quantiser_brute_force_and_round_trip():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((8, 128)) * 0.02).astype(np.float32)
    w[0, :32] = 0.0  # zero block -> e = 0 -> byte 127, codes 0
    packed, scales = mx.quant_mxfp4(w)
    assert scales[0, 0] == 127 and not packed[0, :16].any()
    codes = mx.unpack_fp4_codes(packed)
    for r in range(8):
        for b in range(4):
            blk = w[r, 32 * b : 32 * b + 32].astype(np.float64)
            amax = np.abs(blk).max()
            e = np.floor(np.log2(amax)) - 2 if amax > 0 else 0.0
            assert scales[r, b] == np.clip(e + 127, 0, 254)
            for j in range(32):
                x = blk[j] / 2.0 ** e
                d = np.abs(np.abs(x) - mx.E2M1.astype(np.float64))
                best = int(np.flatnonzero(d == d.min())[0])  # ties to the lower magnitude
                assert codes[r, 32 * b + j] == best | ((x < 0) << 3)
    # round trip: every block holds a magnitude-6 code, so the scale is recovered exactly
    logical = rng.choice([c for c in range(16) if c != 8], size=(4, 64)).astype(np.uint8)
    logical[:, 0] = 7
    logical[:, 32] = 15
    sc = rng.integers(100, 140, size=(4, 2), dtype=np.uint8)
    p2, s2 = mx.quant_mxfp4(mx.dequant_mxfp4(mx.pack_fp4_codes(logical), sc))
    np.testing.assert_array_equal(s2, sc)
    np.testing.assert_array_equal(mx.unpack_fp4_codes(p2), logical)


def test_e4m3_table_matches_torch():
    got = mx.e4m3_table()
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    assert _bits_equal(got, ref)


@pytest.mark.parametrize("shape", [(1, 4096), (3, 77)])
def test_bf16_round_is_rne(shape):
    rng = np.random.default_rng(4)
    x = rng.standard_normal(shape).astype(np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rne = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16).astype(np.uint32).view(np.float32)
    np.testing.assert_array_equal(mx.bf16_round(x), rne)


# ---- MXFP8 (q35_mx_build.py:60-72; sgl mxfp8_gemm, gemm.py:644-659) ----
def _fp8_closed_form(b: int, fmt: str) -> float:
    """float64 decode of one FP8 byte from its bit fields (independent of the oracle's table loop)."""
    ebits, mbits, bias = (4, 3, 7) if fmt == "e4m3" else (5, 2, 15)
    s = -1.0 if b >> 7 else 1.0
    e, m = (b >> mbits) & ((1 << ebits) - 1), b & ((1 << mbits) - 1)
    if fmt == "e4m3" and e == 15 and m == 7:
        return float("nan")
    if fmt == "e5m2" and e == 31:
        return s * float("inf") if m == 0 else float("nan")
    if e == 0:
        return s * m * 2.0 ** (1 - bias - mbits)
    return s * (1.0 + m / 2.0 ** mbits) * 2.0 ** (e - bias)


@pytest.mark.parametrize("fmt,dt", [("e4m3", torch.float8_e4m3fn), ("e5m2", torch.float8_e5m2)])
def test_fp8_tables_against_torch_and_bit_fields(fmt, dt):
    t = mx.fp8_table(fmt)
    ref = torch.arange(256, dtype=torch.uint8).view(dt).float().numpy()
    cf = np.array([_fp8_closed_form(b, fmt) for b in range(256)], dtype=np.float64)
    assert np.array_equal(np.isnan(t), np.isnan(ref)) and np.array_equal(np.isnan(t), np.isnan(cf))
    ok = ~np.isnan(t)
    assert np.array_equal(t[ok], ref[ok]) and np.array_equal(t[ok].astype(np.float64), cf[ok])


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_dequant_mxfp8_every_code_and_scale(fmt):
    # rows: one per scale byte 0..254; columns: the 256 codes in 8 blocks of 32
    codes = np.tile(np.arange(256, dtype=np.uint8), (255, 1))
    scales = np.repeat(np.arange(255, dtype=np.uint8)[:, None], 8, axis=1)
    got = mx.dequant_mxfp8(codes, scales, fmt).astype(np.float64)
    cf = np.array([_fp8_closed_form(b, fmt) for b in range(256)])
    with np.errstate(invalid="ignore", over="ignore"):
        want = cf[None, :] * np.ldexp(1.0, np.arange(255)[:, None] - 127)
    with np.errstate(over="ignore"):
        want32 = want.astype(np.float32).astype(np.float64)  # the fp32 result of the exact product
    both_nan = np.isnan(got) & np.isnan(want32)
    assert np.array_equal(got[~both_nan], want32[~both_nan])


def test_quant_mxfp8_scale_rule_and_nearest_code():
    g = torch.Generator().manual_seed(4)
    w = (torch.randn(6, 256, generator=g) * torch.logspace(-6, 6, 6)[:, None]).numpy()
    w[0, :32] = 0.0  # an all-zero block: amax clamps to 2^-126
    codes, scales = mx.quant_mxfp8(w)
    e = scales.astype(np.int32) - 127
    amax = np.abs(w.reshape(6, 8, 32)).max(-1)
    # the chosen exponent is the smallest with amax / 2^e <= 448 (nothing saturates, no NaN codes)
    nz = amax > 0
    assert (amax[nz] / np.ldexp(1.0, e[nz]) <= 448.0).all()
    assert (amax[nz] / np.ldexp(1.0, e[nz] - 1) > 448.0).all()
    table = mx.e4m3_table()
    assert not np.isnan(table[codes]).any()
    # every code is a nearest E4M3 value of w / 2^e (brute force over the 254 finite codes)
    x = (w.reshape(6, 8, 32) / np.ldexp(1.0, e)[..., None]).reshape(6, 256)
    fin = table[~np.isnan(table)]
    best = np.abs(x[..., None] - fin[None, None, :]).min(-1)
    assert np.allclose(np.abs(x - table[codes]), best, rtol=0, atol=0)
    # round trip within half an E4M3 step (3 mantissa bits) of each element's block scale
    back = mx.dequant_mxfp8(codes, scales)
    step = np.ldexp(1.0, e).repeat(32, axis=1) * 2.0 ** -9  # coarsest step below the subnormal boundary
    assert (np.abs(back - w) <= np.maximum(np.abs(w) * 2.0 ** -4, step)).all()


def test_mxfp8_linear_against_float64():
    g = torch.Generator().manual_seed(5)
    w = torch.randn(48, 128, generator=g).numpy()
    for fmt in ("e4m3", "e5m2"):
        codes, scales = mx.quant_mxfp8(w, fmt)
        a = torch.randn(3, 128, generator=g).bfloat16()
        got = mx.mxfp8_linear(a, codes, scales, fmt)
        ref = a.double() @ torch.from_numpy(mx.dequant_mxfp8(codes, scales, fmt)).double().T
        torch.testing.assert_close(got.double(), ref, rtol=1e-6, atol=1e-6)


def _outside_bar(ref: torch.Tensor, got: torch.Tensor) -> float:
    return float(((got - ref).abs() > 1e-2 + 2e-2 * ref.abs()).float().mean())


def test_narrow_activations_break_the_parity_bar():
    """Why the prefill GEMMs decode the MX weights to bf16 and run bf16 MFMA instead of gfx950's scaled FP8 / FP4 MFMA:
    the scaled forms take both operands narrow, so the bf16 activations would be quantized (MXFP8 / MXFP4 with an E8M0
    scale per 32, as the reference's own quant_mxfp8 / quant_mxfp4 do, q35_mx_build.py:60-72, mx4_common.py:11-49). On
    config 3's draws (one expert's gate-up, activations ~ N(0, 1)) and config 0's linear, the product with quantized
    activations leaves far more than the few-per-million flips the parity bar rel 2e-2 / abs 1e-2 tolerates (measured:
    E4M3 about half of the outputs, E5M2 and E2M1 most of them), while bf16 activations stay inside it."""
    from axk import configs

    g = torch.Generator().manual_seed(0)
    w = configs.moe_weights(g, hidden=2048, experts=2, inter=512, shared_inter=64)
    wq = torch.from_numpy(mx.dequant_mxfp4(w["e_gw"][0].numpy(), w["e_gs"][0].numpy()))  # [1024, 2048] exact
    x = torch.randn(32, 2048, generator=g).bfloat16().float()
    ref = x @ wq.T
    assert _outside_bar(ref, (x @ wq.T).bfloat16().float()) == 0.0  # bf16 outputs of bf16 activations: inside
    fr = {}
    for fmt in ("e4m3", "e5m2"):
        codes, sc = mx.quant_mxfp8(x.numpy(), fmt)
        xq = torch.from_numpy(mx.dequant_mxfp8(codes, sc, fmt))
        fr[fmt] = _outside_bar(ref, (xq @ wq.T).bfloat16().float())
    packed, sc = mx.quant_mxfp4(x.numpy())
    fr["e2m1"] = _outside_bar(ref, (torch.from_numpy(mx.dequant_mxfp4(packed, sc)) @ wq.T).bfloat16().float())
    assert fr["e4m3"] > 0.2 and fr["e5m2"] > 0.4 and fr["e2m1"] > 0.6, fr
    c0 = configs.config0()
    w0 = torch.from_numpy(mx.dequant_mxfp4(c0["w"].numpy(), c0["s"].numpy()))
    x0 = c0["x"].float()
    codes, sc = mx.quant_mxfp8(x0.numpy(), "e4m3")
    got0 = (torch.from_numpy(mx.dequant_mxfp8(codes, sc, "e4m3")) @ w0.T).bfloat16().float()
    assert _outside_bar(x0 @ w0.T, got0) > 0.2


# ---- NVFP4 (E2M1 codes, E4M3 scales per 16 along K, an fp32 scale2): quantization.py:8-37 ----
def _e2m1_by_binade(x):
    """E2M1 rounding restated per binade: the grid spacing is 0.5 below 2, 1 in [2, 4), 2 in [4, 6]; numpy's
    round-half-even on the multiple of the spacing makes a tie go to the even mantissa, which is the even code;
    past 6 the value saturates. Returns (code, value)."""
    x = np.asarray(x, dtype=np.float64)
    mag = np.abs(x)
    step = np.where(mag < 2, 0.5, np.where(mag < 4, 1.0, 2.0))
    val = np.minimum(np.round(mag / step) * step, 6.0)
    code = np.searchsorted(mx.E2M1.astype(np.float64), val)
    return (code | (np.signbit(x) << 3)).astype(np.uint8), np.where(np.signbit(x), -val, val)


def test_nvfp4_reference_vectors():
    """The reference test's own vectors (test_nvfp4_lm_head.py:19-39): a midpoint row, zero blocks, scale2 = 1."""
    src = torch.zeros(3, 32, dtype=torch.bfloat16)
    src[0, 0] = 448 * 6  # makes the global decode scale exactly one
    src[1, :16] = torch.tensor([0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5, 6, -0.25, -0.75, -1.25, -1.75, -2.5, -3.5, -5])
    packed, scales, s2 = mx.quantize_nvfp4(src.float().numpy())
    assert packed.shape == (3, 16) and scales.shape == (3, 2) and s2 == np.float32(1)
    expected = np.array([0, 0, 2, 2, 4, 4, 6, 6, 7, 8, 10, 10, 12, 12, 14, 14], dtype=np.uint8)
    assert np.array_equal(packed[1, :8], expected[::2] | (expected[1::2] << 4))
    assert not packed[2].any()
    assert mx.e4m3_table()[scales[1, 0]] == 1 and not mx.e4m3_table()[scales[2]].any()
    assert np.isfinite(mx.dequant_nvfp4(packed, scales, s2)).all()
    zp, zs, z2 = mx.quantize_nvfp4(np.zeros((2, 16), np.float32))
    assert z2 == np.float32(1) and not mx.dequant_nvfp4(zp, zs, z2).any()


def test_e2m1_code_against_binade_rounding():
    grid = mx.E2M1.astype(np.float64)
    mids = (grid[:-1] + grid[1:]) / 2
    g = np.random.default_rng(5)
    x = np.concatenate([grid, mids, -grid, -mids, mids + 1e-6, mids - 1e-6, [6.5, 7.0, 1e6, -9.0],
                        g.uniform(-7, 7, 4000)]).astype(np.float32)
    code, val = _e2m1_by_binade(x)
    assert np.array_equal(mx.e2m1_code(x), code)
    assert np.array_equal(mx.FP4_LUT[code], val.astype(np.float32))


def test_dequant_nvfp4_every_code_and_scale():
    """Every (code, E4M3 scale byte) pair against a float64 decode of the two fields, times an fp32 scale2."""
    codes = np.tile(np.arange(16, dtype=np.uint8), 256 * 2)  # 32 values per row: two 16-blocks
    codes = np.tile(codes[:32], (256, 1))
    packed = mx.pack_fp4_codes(codes)
    scales = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 2, axis=1)
    for s2 in (np.float32(1.0), np.float32(2.0 ** -9), np.float32(0.0371)):
        got = mx.dequant_nvfp4(packed, scales, s2).astype(np.float64)
        e4 = np.array([_fp8_closed_form(b, "e4m3") for b in range(256)])
        v = np.array(REF_FP4_LUT, dtype=np.float64)[codes]
        with np.errstate(invalid="ignore"):
            want = ((v * e4[:, None]).astype(np.float32).astype(np.float64) * np.float64(s2)).astype(np.float32)
        both_nan = np.isnan(got) & np.isnan(want)
        assert np.array_equal(got[~both_nan], want.astype(np.float64)[~both_nan])


def test_quantize_nvfp4_block_rule():
    """Every block with a normal E4M3 scale codes its largest magnitude to 6 (the scale rounds within E4M3's relative
    step of amax / 6, so the quotient lands above the 4 / 6 midpoint; blocks far below the matrix's amax get
    subnormal or zero scales, the format's range limit), and each code is the nearest E2M1 value of the block's
    quotient."""
    g = torch.Generator().manual_seed(11)
    w = (torch.randn(8, 256, generator=g) * torch.logspace(-4, 2, 8)[:, None]).numpy()
    packed, scales, s2 = mx.quantize_nvfp4(w)
    codes = mx.unpack_fp4_codes(packed).reshape(8, 16, 16)
    blocks = w.reshape(8, 16, 16)
    top = np.abs(blocks).argmax(-1)
    normal = ((scales >> 3) & 15) >= 1
    assert normal.sum() >= 64 and (~normal).sum() >= 8  # both kinds of block occur
    assert np.all((np.take_along_axis(codes, top[..., None], -1)[..., 0] & 7)[normal] == 7)
    dec = (mx.e4m3_table()[scales].astype(np.float32) * s2).astype(np.float32)
    q = (blocks / np.where(dec > 0, dec, np.float32(1))[..., None]).astype(np.float32)  # a zero scale divides by 1
    assert np.array_equal(codes, _e2m1_by_binade(q)[0])


def test_int8_linear_exact_under_power_of_two_scales():
    """With power-of-two scales every scaled operand, product and sum up to 2^24 is exact in fp32 and bf16 holds
    int8 * 2^e exactly, so the linear equals the int64 dot product times 2^(ea[m] + eb[n]) bit for bit; distinct m
    and n sizes and scales make a transposed operand or swapped scale fail."""
    rng = np.random.default_rng(5)
    m, n, k = 5, 7, 96
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    b = rng.integers(-128, 128, (n, k), dtype=np.int8)
    ea, eb = rng.integers(-6, 4, m), rng.integers(-5, 5, n)
    exact = np.zeros((m, n), dtype=np.int64)
    for i in range(m):
        for j in range(n):
            exact[i, j] = sum(int(a[i, t]) * int(b[j, t]) for t in range(k))
    want = exact.astype(np.float64) * np.exp2(ea)[:, None] * np.exp2(eb)[None, :]
    for dt in (torch.float32, torch.bfloat16):
        got = mx.int8_linear(a, b, np.exp2(ea).astype(np.float32), np.exp2(eb).astype(np.float32), dt)
        assert np.array_equal(got.numpy().astype(np.float64), want)
    # a scalar scale broadcasts like a vector of one value
    one = mx.int8_linear(a, b, np.float32(0.25), np.float32(2.0), torch.float32)
    vec = mx.int8_linear(a, b, np.full(m, 0.25, np.float32), np.full(n, 2.0, np.float32), torch.float32)
    assert torch.equal(one, vec) and np.array_equal(one.numpy().astype(np.float64), exact * 0.5)


def test_int8_linear_rounds_operands_and_bias_to_the_output_dtype():
    """1 x 1 x 1 cases: 127 * (1/3) is rounded to bf16 (42.25, not fp32's 42.333332) before the matmul when the
    output is bf16 and kept in fp32 otherwise; a bias of 1 + 2^-10 adds 1 at bf16."""
    a, b = np.array([[127]], np.int8), np.array([[1]], np.int8)
    third = np.float32(1.0 / 3.0)
    assert mx.int8_linear(a, b, third, np.float32(1), torch.bfloat16).item() == 42.25
    assert mx.int8_linear(a, b, third, np.float32(1), torch.float32).item() == float(np.float32(127) * third)
    bias = torch.tensor([1.0 + 2.0 ** -10])
    assert mx.int8_linear(a, b, np.float32(1), np.float32(1), torch.bfloat16, bias).item() == 128.0
    assert mx.int8_linear(a, b, np.float32(1), np.float32(1), torch.float32, bias).item() == 128.0 + 2.0 ** -10


def test_int4_linear_against_group_loops():
    """The int4 linear equals float64 loops that scale each group's partial dot product by its own scale (group = K /
    scale columns): a scale indexed by k % G, by the wrong channel, or a transposed weight fails."""
    rng = np.random.default_rng(6)
    for m, n, k, g in ((3, 5, 128, 32), (2, 4, 192, 64)):
        a = torch.randn(m, k, generator=torch.Generator().manual_seed(k)).to(torch.bfloat16)
        w = rng.integers(-8, 8, (n, k), dtype=np.int8)
        s = (rng.random((n, k // g)) + 0.25).astype(np.float32)
        af = a.double().numpy()
        want = np.zeros((m, n))
        for i in range(m):
            for j in range(n):
                for q in range(k // g):
                    want[i, j] += float(s[j, q]) * sum(af[i, t] * int(w[j, t]) for t in range(q * g, (q + 1) * g))
        got = mx.int4_linear(a, w, s).numpy().astype(np.float64)
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
        # unit scales: the plain integer-weight product
        ones = mx.int4_linear(a, w, np.ones_like(s)).numpy().astype(np.float64)
        np.testing.assert_allclose(ones, af @ w.T.astype(np.float64), rtol=1e-6, atol=1e-5)
