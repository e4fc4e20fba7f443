// Weight-streaming MFMA tile shared by the linear and MoE kernels (gfx950).
//
// A 16-row weight tile (one MFMA N tile) is streamed along K in 16-byte lane units and dequantised in
// registers to bf16; activations are the MFMA A operand. Lane l: N column l % 16, K group g = l / 16. Chunk
// c covers K [c*4V, (c+1)*4V); the lane's unit inside it is [c*4V + g*V, +V). MFMA step s uses
// k = unit + 8s .. +8 for both operands, so any K order works as long as A and B agree.
#pragma once
#include "axk_common.h"

namespace axk {

enum WeightFmt { WF_MXFP4 = 0, WF_FP8 = 1, WF_BF16 = 2, WF_MXFP8 = 3, WF_MXBF8 = 4, WF_NVFP4 = 5 };

// Formats whose E8M0 scales (one per 32 values along K, [N, K/32]) are applied inside the unit decode.
__host__ __device__ constexpr bool is_mx(int F) { return F == WF_MXFP4 || F == WF_MXFP8 || F == WF_MXBF8; }
// NVFP4: E2M1 codes as MXFP4's with E4M3 scales, one per 16 values along K ([N, K/16]), applied inside the unit
// decode; the per-matrix fp32 scale2 multiplies the sums in the epilogue.
__host__ __device__ constexpr bool is_nv(int F) { return F == WF_NVFP4; }
__host__ __device__ constexpr bool has_block_scales(int F) { return is_mx(F) || is_nv(F); }
__host__ __device__ constexpr bool is_fp4(int F) { return F == WF_MXFP4 || F == WF_NVFP4; }

template <int F>
struct WUnit;

// MXFP4: codes [N, K/2] (low nibble = even k), E8M0 scales [N, K/32].
template <>
struct WUnit<WF_MXFP4> {
  static constexpr int V = 32;
  static constexpr int STEPS = 4;
  static AXK_DEV uint4 load(const uint8_t* w, int64_t n, int64_t K, int64_t kb) {
    return *reinterpret_cast<const uint4*>(w + n * (K >> 1) + (kb >> 1));
  }
  static AXK_DEV float scale(const uint8_t* s, int64_t n, int64_t K, int64_t kb) {
    return e8m0_to_f32(s[n * (K >> 5) + (kb >> 5)]);
  }
  static AXK_DEV axk_bf16x8 conv(const uint4& q, int step, float sc) {
    const uint32_t word = step == 0 ? q.x : step == 1 ? q.y : step == 2 ? q.z : q.w;
    return fp4x8_to_bf16x8(word, sc);
  }
};

// NVFP4: codes [N, K/2] (low nibble = even k), E4M3 scales [N, K/16]. A 16-byte unit (32 values) spans two scale
// blocks: steps 0-1 the first, 2-3 the second; its scale is the two E4M3 bytes (first block low).
template <>
struct WUnit<WF_NVFP4> {
  static constexpr int V = 32;
  static constexpr int STEPS = 4;
  static AXK_DEV uint4 load(const uint8_t* w, int64_t n, int64_t K, int64_t kb) {
    return *reinterpret_cast<const uint4*>(w + n * (K >> 1) + (kb >> 1));
  }
  static AXK_DEV uint32_t scale(const uint8_t* s, int64_t n, int64_t K, int64_t kb) {
    const uint8_t* p = s + n * (K >> 4) + (kb >> 4);
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8);
  }
  static AXK_DEV axk_bf16x8 conv(const uint4& q, int step, uint32_t sc2) {
    const uint32_t word = step == 0 ? q.x : step == 1 ? q.y : step == 2 ? q.z : q.w;
    // both E4M3 scales of the unit in one convert (scale 1: exact), shared by the four steps
    const axk_f32x2 s = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(sc2, 1.0f, false);
    return fp4x8_to_bf16x8_mul(word, step >= 2 ? s[1] : s[0]);
  }
};

// FP8 E4M3: [N, K] bytes; the per-channel scale is applied in the epilogue.
template <>
struct WUnit<WF_FP8> {
  static constexpr int V = 16;
  static constexpr int STEPS = 2;
  static AXK_DEV uint4 load(const uint8_t* w, int64_t n, int64_t K, int64_t kb) {
    return *reinterpret_cast<const uint4*>(w + n * K + kb);
  }
  static AXK_DEV float scale(const uint8_t*, int64_t, int64_t, int64_t) { return 1.0f; }
  static AXK_DEV axk_bf16x8 conv(const uint4& q, int step, float) {
    const uint32_t w0 = step == 0 ? q.x : q.z, w1 = step == 0 ? q.y : q.w;
    axk_bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false);
    axk_bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true);
    axk_bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false);
    axk_bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true);
    axk_bf16x8 r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
  }
};

// MXFP8: OCP FP8 codes [N, K] bytes, E4M3 (WF_MXFP8) or E5M2 (WF_MXBF8), with E8M0 scales [N, K/32]; a 16-byte unit
// is half a scale block. gfx950's scaled converts multiply by the block scale on the way to bf16 (exact while the
// scaled value is a bf16 normal).
template <int F>
struct WUnitMx8 {
  static constexpr int V = 16;
  static constexpr int STEPS = 2;
  static AXK_DEV uint4 load(const uint8_t* w, int64_t n, int64_t K, int64_t kb) {
    return *reinterpret_cast<const uint4*>(w + n * K + kb);
  }
  static AXK_DEV float scale(const uint8_t* s, int64_t n, int64_t K, int64_t kb) {
    return e8m0_to_f32(s[n * (K >> 5) + (kb >> 5)]);
  }
  template <bool HI>
  static AXK_DEV axk_bf16x2 cvt(uint32_t w, float sc) {
    if constexpr (F == WF_MXBF8) return __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, sc, HI);
    else return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, sc, HI);
  }
  static AXK_DEV axk_bf16x8 conv(const uint4& q, int step, float sc) {
    const uint32_t w0 = step == 0 ? q.x : q.z, w1 = step == 0 ? q.y : q.w;
    const axk_bf16x2 p0 = cvt<false>(w0, sc), p1 = cvt<true>(w0, sc), p2 = cvt<false>(w1, sc), p3 = cvt<true>(w1, sc);
    axk_bf16x8 r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
  }
};
template <>
struct WUnit<WF_MXFP8> : WUnitMx8<WF_MXFP8> {};
template <>
struct WUnit<WF_MXBF8> : WUnitMx8<WF_MXBF8> {};

// bf16: [N, K] (uint16 bits).
template <>
struct WUnit<WF_BF16> {
  static constexpr int V = 8;
  static constexpr int STEPS = 1;
  static AXK_DEV uint4 load(const uint8_t* w, int64_t n, int64_t K, int64_t kb) {
    return *reinterpret_cast<const uint4*>(w + (n * K + kb) * 2);
  }
  static AXK_DEV float scale(const uint8_t*, int64_t, int64_t, int64_t) { return 1.0f; }
  static AXK_DEV axk_bf16x8 conv(const uint4& q, int, float) {
    return *reinterpret_cast<const axk_bf16x8*>(&q);
  }
};


// Accumulate acc[t] += A_t (16 rows x K) * W (16 rows x K)^T for the chunks c = c_begin, c_begin + c_step, ...
// xrow[t]: this lane's activation row of M tile t (row l % 16 of the tile); mvalid[t]: that row exists.
// w points at weight row n (this lane's N column); nvalid: that row exists.
template <int F, int MT, int UNROLL = 2>
__device__ __forceinline__ void mx_tile_accum(const uint16_t* const (&xrow)[MT], const bool (&mvalid)[MT],
                                              const uint8_t* __restrict__ w, const uint8_t* __restrict__ wscale,
                                              int64_t n, bool nvalid, int64_t K, int64_t c_begin, int64_t c_step,
                                              axk_f32x4 (&acc)[MT]) {
  using U = WUnit<F>;
  constexpr int CH = 4 * U::V;
  const int lane = threadIdx.x & 63, g = lane >> 4;
  const int64_t NC = (K + CH - 1) / CH;
  for (int64_t c0 = c_begin; c0 < NC; c0 += c_step * UNROLL) {
    using S = decltype(U::scale(wscale, n, K, 0));  // float, or NVFP4's pair of E4M3 bytes
    uint4 q[UNROLL];
    S sc[UNROLL];
    int64_t kb[UNROLL];
    bool kv[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int64_t c = c0 + (int64_t)u * c_step;
      kb[u] = c * CH + g * U::V;
      kv[u] = c < NC && kb[u] < K;
      q[u] = make_uint4(0u, 0u, 0u, 0u);
      sc[u] = S(1);
      if (nvalid && kv[u]) {
        q[u] = U::load(w, n, K, kb[u]);
        sc[u] = U::scale(wscale, n, K, kb[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
#pragma unroll
      for (int s = 0; s < U::STEPS; ++s) {
        const axk_bf16x8 b = U::conv(q[u], s, sc[u]);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const axk_bf16x8 a = (mvalid[t] && kv[u]) ? load_bf16x8(xrow[t] + kb[u] + 8 * s) : zero_bf16x8();
          acc[t] = mfma_bf16_16x16x32(a, b, acc[t]);
        }
      }
    }
  }
}

// Staged loads (the linear kernels) read a tile's weights as 128-byte row segments, two instructions of 8 rows x
// 128 bytes each (whole cache lines, which keeps the address path's per-line work low), through an LDS tile of
// [16 rows][kSegLd bytes] (16 bytes of padding per row).
constexpr int kSegBytes = 128;
constexpr int kSegLd = kSegBytes + 16;

template <int F>
__host__ __device__ constexpr int64_t row_bytes(int64_t K) {
  return is_fp4(F) ? K / 2 : (F == WF_BF16 ? 2 * K : K);
}

}  // namespace axk
