// Device helpers shared by every axk kernel (gfx950 / CDNA4, wave64).
//
// Number formats on the boundary (all passed as raw bytes / bits):
//   bf16  : uint16_t bit pattern, rounded from fp32 with round-to-nearest-even (torch's rule)
//   E2M1  : 4-bit code s|e1 e0|m0, two per byte, LOW nibble = EVEN column
//           (models/qwen35_35b_a3b/src/70b0fbc/q35_moe.py:46-63)
//   E8M0  : one byte per 32 consecutive K values, value 2^(s-127) exactly as torch.exp2(s - 127):
//           s = 0 -> 2^-127 (fp32 denormal), s = 255 -> +inf (q35_moe.py:60-63)
//   E4M3  : OCP fp8 e4m3fn (no inf, 0x7f/0xff = NaN)
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define AXK_DEV __device__ __forceinline__

typedef __bf16 axk_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 axk_bf16x2 __attribute__((ext_vector_type(2)));
typedef float axk_f32x4 __attribute__((ext_vector_type(4)));
typedef float axk_f32x2 __attribute__((ext_vector_type(2)));

AXK_DEV float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// fp32 -> bf16 bits, round to nearest even (gfx950's v_cvt_pk_bf16_f32); NaN stays a quiet NaN.
AXK_DEV uint32_t f32_to_bf16_bits(float f) {
  const __bf16 b = (__bf16)f;
  return (uint32_t)__builtin_bit_cast(uint16_t, b);
}

// Two fp32 -> packed bf16 pair (low half = lo), one conversion instruction.
AXK_DEV uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  const axk_bf16x2 r = __builtin_convertvector((f2){lo, hi}, axk_bf16x2);
  return __builtin_bit_cast(uint32_t, r);
}

AXK_DEV float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// E8M0 byte -> fp32 2^(s-127); bit-identical to torch.exp2(float(s) - 127): s << 23 is the value's bits for s >= 1
// (s = 255: +inf), and for s = 0 the subnormal 2^-127 (0x00400000) is the larger of the two (a max, not a select).
AXK_DEV float e8m0_to_f32(uint32_t s) { return __uint_as_float(max(s << 23, 0x00400000u)); }

// E2M1 code (low 4 bits of c) -> exact fp32 value, code 8 -> -0.0.
AXK_DEV float e2m1_to_f32(uint32_t c) {
  const uint32_t m = c & 7u;
  const uint32_t mag = m < 2u ? (m ? 0x3f000000u : 0u) : ((((m >> 1) + 126u) << 23) | ((m & 1u) << 22));
  return __uint_as_float(mag | ((c & 8u) << 28));
}

// Eight consecutive bf16 values (16 bytes) as an MFMA operand.
AXK_DEV axk_bf16x8 load_bf16x8(const uint16_t* p) {
  return *reinterpret_cast<const axk_bf16x8*>(p);
}

AXK_DEV axk_bf16x8 zero_bf16x8() {
  axk_bf16x8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = (__bf16)0.0f;
  return z;
}

// Eight E2M1 codes (one 32-bit word, low nibble first) -> eight bf16 scaled by `scale`
// (a power of two), using gfx950's scaled FP4 conversion.
AXK_DEV axk_bf16x8 fp4x8_to_bf16x8(uint32_t w, float scale) {
  axk_bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0);
  axk_bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1);
  axk_bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2);
  axk_bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3);
  axk_bf16x8 r;
  r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
  r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
  return r;
}

// E4M3 (OCP) byte -> exact fp32, written from the format definition (bias 7, no inf).
AXK_DEV float e4m3_to_f32(uint32_t b) {
  const uint32_t s = (b & 0x80u) << 24;
  const uint32_t e = (b >> 3) & 0xfu;
  const uint32_t m = b & 7u;
  if (e == 0xfu && m == 7u) return __uint_as_float(s | 0x7fc00000u);
  if (e == 0u) {  // subnormal: m * 2^-9 (m == 0 keeps the sign of zero)
    const float v = (float)m * 0.001953125f;
    return s ? -v : v;
  }
  return __uint_as_float(s | ((e + 120u) << 23) | (m << 20));
}

// Eight E2M1 codes times an arbitrary fp32 scale s (an NVFP4 block's E4M3 scale) -> bf16. gfx950's scaled converts
// apply only the exponent of their scale operand (a power of two, as MX scales are), so the codes are decoded
// exactly at scale 1 and multiplied by s in fp32: the product of an E2M1 value (at most 2 significant bits) and an
// E4M3 value (at most 4) is exact in fp32 and again in bf16.
AXK_DEV axk_bf16x8 fp4x8_to_bf16x8_mul(uint32_t w, float s) {
  const axk_f32x2 f0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
  const axk_f32x2 f1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
  const axk_f32x2 f2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
  const axk_f32x2 f3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
  axk_bf16x8 r;
  r[0] = (__bf16)(f0[0] * s); r[1] = (__bf16)(f0[1] * s); r[2] = (__bf16)(f1[0] * s); r[3] = (__bf16)(f1[1] * s);
  r[4] = (__bf16)(f2[0] * s); r[5] = (__bf16)(f2[1] * s); r[6] = (__bf16)(f3[0] * s); r[7] = (__bf16)(f3[1] * s);
  return r;
}


// Four E4M3 bytes -> four bf16 (exact: E4M3 values fit bf16's 8-bit exponent and 7-bit mantissa).
AXK_DEV void fp8x4_to_bf16(uint32_t w, __bf16* dst) {
#pragma unroll
  for (int i = 0; i < 4; ++i) dst[i] = (__bf16)e4m3_to_f32((w >> (8 * i)) & 0xffu);
}

typedef unsigned int axk_u32x4 __attribute__((ext_vector_type(4)));
typedef short axk_s16x4 __attribute__((ext_vector_type(4)));

// Non-temporal 16-byte load and store (the nt cache policy) for streams touched once per launch: weights, the
// recurrent state tile.
AXK_DEV axk_u32x4 load_nt(const void* p) { return __builtin_nontemporal_load(reinterpret_cast<const axk_u32x4*>(p)); }
AXK_DEV void store_nt(void* p, axk_u32x4 v) { __builtin_nontemporal_store(v, reinterpret_cast<axk_u32x4*>(p)); }

// ds_read_b64_tr_b16: each lane gives the LDS address of 4 consecutive 16-bit values; in every group of 16 lanes,
// lane i receives element i % 4 of the values of lanes i / 4, i / 4 + 4, i / 4 + 8 and i / 4 + 12 (one 64-bit
// read per lane that transposes a 16 x 4 block of the group).
AXK_DEV axk_s16x4 lds_read_tr16(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) axk_s16x4*)(p));
}

// Transposing 8-byte LDS read of 8-bit elements: in each 16-lane group, lane i receives byte i % 8 of the 8-byte rows
// read by source lanes i / 8 + 2j, j = 0 .. 7 (source lane 2j + a pointing at row j, bytes 8a .. 8a + 7 of a 16-column
// block gives lane i column i of the eight rows).
typedef int axk_i32x2 __attribute__((ext_vector_type(2)));
AXK_DEV axk_i32x2 lds_read_tr8(const void* p) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) axk_i32x2*)(p));
}

// LDS byte address of a __shared__ pointer (for M0).
AXK_DEV uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Direct global -> LDS loads: lane l's 16 bytes at gptr land at lds_base + 16 l (lds_base wave-uniform).
// Issued from asm on purpose: the compiler then counts none of these loads, so its own waits can only over-wait,
// and pipeline waits (wait_vmcnt<n>) stay exactly as written. M0 is restored.
// lds_dma16: non-temporal, for bytes read once per launch (they should not displace cached lines);
// lds_dma16_cached: the default policy, for tiles other workgroups re-read through L2.
AXK_DEV void lds_dma16(const void* gptr, uint32_t lds_base_any) {
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(lds_base_any);
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %2, off nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "s"(lds_base), "v"(gptr)
      : "memory");
}
AXK_DEV void lds_dma16_cached(const void* gptr, uint32_t lds_base_any) {
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(lds_base_any);
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "s"(lds_base), "v"(gptr)
      : "memory");
}

// As lds_dma16_cached for 4 bytes a lane: lane l's dword at gptr (4-byte aligned) lands at lds_base + 4 l.
AXK_DEV void lds_dma4_cached(const void* gptr, uint32_t lds_base_any) {
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(lds_base_any);
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dword %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "s"(lds_base), "v"(gptr)
      : "memory");
}

// A wave-uniform pointer in scalar registers (the value of the first active lane).
AXK_DEV const void* uniform_ptr(const void* p) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a), hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  return (const void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// As lds_dma16, addressed as a wave-uniform 64-bit base (scalar registers) plus this lane's 32-bit byte offset: no
// per-lane 64-bit address arithmetic.
AXK_DEV void lds_dma16_so(const void* sbase_any, uint32_t voff, uint32_t lds_base_any) {
  const void* sbase = uniform_ptr(sbase_any);
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(lds_base_any);
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %2, %3 nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "s"(lds_base), "v"(voff), "s"(sbase)
      : "memory");
}

template <int N>
AXK_DEV void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

AXK_DEV axk_f32x4 mfma_bf16_16x16x32(axk_bf16x8 a, axk_bf16x8 b, axk_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Wave-wide reductions (wave64) on DPP lane moves inside rows of 16 lanes, then two row broadcasts that leave
// the total in lane 63, read back as a uniform value. Control codes (GFX9 DPP): quad_perm [1,0,3,2] = 0xB1,
// [2,3,0,1] = 0x4E, row_half_mirror 0x141, row_mirror 0x140, row_bcast15 0x142 (rows 1 and 3 take lane 15 of
// the row below), row_bcast31 0x143 (rows 2 and 3 take lane 31).
template <int CTRL, int ROW_MASK = 0xF>
AXK_DEV float dpp_move(float old, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                               __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF,
                                                               false));
}
AXK_DEV float lane63(float v) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63)); }
// The sum of every lane's v (the same value in every lane).
AXK_DEV float wave_sum(float v) {
  v += dpp_move<0xB1>(v, v);
  v += dpp_move<0x4E>(v, v);
  v += dpp_move<0x141>(v, v);
  v += dpp_move<0x140>(v, v);
  v += dpp_move<0x142, 0xA>(0.f, v);
  v += dpp_move<0x143, 0xC>(0.f, v);
  return lane63(v);
}
// Cross-row exchanges on VALU (gfx950 v_permlane16_swap / v_permlane32_swap, which swap the odd rows of 16 lanes
// (upper 32 lanes) of the first operand with the even rows (lower 32 lanes) of the second): given v twice, the
// pair holds the even-row (lower-half) value and the odd-row (upper-half) value of each row pair (half pair) in
// every lane, hence v op v(l ^ 16) and v op v(l ^ 32) without the LDS pipe. The second copy of v is laundered
// through an empty asm: with two operands it can prove equal, the compiler folds the swap away.
AXK_DEV uint2 row_pair16(float v) {
  unsigned a = __builtin_bit_cast(unsigned, v), b = a;
  asm volatile("" : "+v"(b));
  const auto p = __builtin_amdgcn_permlane16_swap(a, b, false, false);
  return make_uint2(p[0], p[1]);
}
AXK_DEV uint2 half_pair32(float v) {
  unsigned a = __builtin_bit_cast(unsigned, v), b = a;
  asm volatile("" : "+v"(b));
  const auto p = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  return make_uint2(p[0], p[1]);
}
AXK_DEV float xor16_sum(float v) { const uint2 p = row_pair16(v); return __uint_as_float(p.x) + __uint_as_float(p.y); }
AXK_DEV float xor32_sum(float v) { const uint2 p = half_pair32(v); return __uint_as_float(p.x) + __uint_as_float(p.y); }
AXK_DEV float xor16_max(float v) { const uint2 p = row_pair16(v); return fmaxf(__uint_as_float(p.x), __uint_as_float(p.y)); }
AXK_DEV float xor32_max(float v) { const uint2 p = half_pair32(v); return fmaxf(__uint_as_float(p.x), __uint_as_float(p.y)); }

// Two 16x16 MFMA accumulator tiles a (rows 4 g + r) and b (rows 16 + 4 g + r) of one column (lane l16), rounded to
// bf16, as the B operand of one 32-deep k-step (lane (column, g) holds k rows 8 g .. 8 g + 7). permlane32_swap gives
// the lane groups {a@0, a@1, b@0, b@1} and {a@2, a@3, b@2, b@3}; permlane16_swap of those gives each group g the rows
// of groups 2 (g & 1) (first four) and 2 (g & 1) + 1 (last four) of tile a (g < 2) or b (g >= 2).
AXK_DEV axk_bf16x8 acc_pair_to_b(const axk_f32x4& a, const axk_f32x4& b) {
  const unsigned a01 = pack_bf16x2(a[0], a[1]), a23 = pack_bf16x2(a[2], a[3]);
  const unsigned b01 = pack_bf16x2(b[0], b[1]), b23 = pack_bf16x2(b[2], b[3]);
  const auto s01 = __builtin_amdgcn_permlane32_swap(a01, b01, false, false);
  const auto s23 = __builtin_amdgcn_permlane32_swap(a23, b23, false, false);
  const auto t01 = __builtin_amdgcn_permlane16_swap(s01[0], s01[1], false, false);
  const auto t23 = __builtin_amdgcn_permlane16_swap(s23[0], s23[1], false, false);
  const axk_u32x4 f = {t01[0], t23[0], t01[1], t23[1]};
  return __builtin_bit_cast(axk_bf16x8, f);
}

// fp16 operands (the INT8 cache decode)
typedef _Float16 axk_f16x8 __attribute__((ext_vector_type(8)));
AXK_DEV axk_f32x4 mfma_f16_16x16x32(axk_f16x8 a, axk_f16x8 b, axk_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
// Eight int8 codes (two dwords, bytes in order) as the fp16 values 1152 + code, exactly: the byte with its sign bit
// flipped (code + 128, 0 .. 255) is the low mantissa byte under the exponent of 1024 (fp16 bits 0x6400 | byte), one
// byte permute per two values (selector bytes 0 .. 3 take the flipped codes, 4 the 0x64 of the first operand).
AXK_DEV axk_f16x8 i8x8_to_f16x8_off(uint32_t w0, uint32_t w1) {
  const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
  const axk_u32x4 r = {__builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u),
                       __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u),
                       __builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u),
                       __builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u)};
  return __builtin_bit_cast(axk_f16x8, r);
}
// Two floats -> fp16 pair, round to nearest even.
AXK_DEV uint32_t pack_f16x2(float lo, float hi) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
// acc_pair_to_b with fp16 rounding (the same lane swaps).
AXK_DEV axk_f16x8 acc_pair_to_b_f16(const axk_f32x4& a, const axk_f32x4& b) {
  const unsigned a01 = pack_f16x2(a[0], a[1]), a23 = pack_f16x2(a[2], a[3]);
  const unsigned b01 = pack_f16x2(b[0], b[1]), b23 = pack_f16x2(b[2], b[3]);
  const auto s01 = __builtin_amdgcn_permlane32_swap(a01, b01, false, false);
  const auto s23 = __builtin_amdgcn_permlane32_swap(a23, b23, false, false);
  const auto t01 = __builtin_amdgcn_permlane16_swap(s01[0], s01[1], false, false);
  const auto t23 = __builtin_amdgcn_permlane16_swap(s23[0], s23[1], false, false);
  const axk_u32x4 f = {t01[0], t23[0], t01[1], t23[1]};
  return __builtin_bit_cast(axk_f16x8, f);
}

// Sum inside aligned groups of W lanes (W = 2, 4, 8 or 16), the same value in every lane of the group.
template <int W>
AXK_DEV float group_sum(float v) {
  static_assert(W == 2 || W == 4 || W == 8 || W == 16, "group of 2..16 lanes");
  v += dpp_move<0xB1>(v, v);
  if constexpr (W >= 4) v += dpp_move<0x4E>(v, v);
  if constexpr (W >= 8) v += dpp_move<0x141>(v, v);
  if constexpr (W >= 16) v += dpp_move<0x140>(v, v);
  return v;
}
AXK_DEV float wave_max(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v, v));
  v = fmaxf(v, dpp_move<0x4E>(v, v));
  v = fmaxf(v, dpp_move<0x141>(v, v));
  v = fmaxf(v, dpp_move<0x140>(v, v));
  v = fmaxf(v, dpp_move<0x142, 0xA>(v, v));
  v = fmaxf(v, dpp_move<0x143, 0xC>(v, v));
  return lane63(v);
}

AXK_DEV float silu_f32(float x) { return x / (1.0f + __expf(-x)); }

// One token of the causal depthwise conv1d for one channel: taps wk[0 .. K-1] (wk[0] multiplies the current input
// xt, wk[j] the input j tokens back), hist[0 .. K-2] the previous inputs, oldest first (K <= kMaxConvTaps). Each
// tap's partial sum is rounded to bf16, as the reference accumulates in bf16; SiLU is applied by the caller.
constexpr int kMaxConvTaps = 8;
AXK_DEV float conv_taps(float xt, const float (&wk)[kMaxConvTaps], const float (&hist)[kMaxConvTaps], int K) {
  float acc = round_bf16(__fadd_rn(0.f, __fmul_rn(xt, wk[0])));
#pragma unroll
  for (int j = 1; j < kMaxConvTaps; ++j)
    if (j < K) acc = round_bf16(__fadd_rn(acc, __fmul_rn(hist[K - 1 - j], wk[j])));
  return acc;
}
AXK_DEV float sigmoid_f32(float x) { return 1.0f / (1.0f + __expf(-x)); }
AXK_DEV float softplus_f32(float x) { return x > 20.0f ? x : log1pf(__expf(x)); }
