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
