// MXFP4 codec and runtime-weight linear (MXFP4 / FP8 E4M3 / bf16 weights) for gfx950.
//
// Decode-shaped projections (m <= 32 rows per launch tile) are pure weight streaming: every weight
// byte is read once, so the kernel is bound by HBM bandwidth. The design:
//   * a workgroup owns 16 output channels (one MFMA N tile) and splits K across its waves;
//   * each lane streams one 16-byte weight unit per chunk with a single 128-bit load
//     (MXFP4: 32 codes = exactly one E8M0 block; FP8: 16 values; bf16: 8 values), so the
//     16 lanes of an N tile x 4 K-groups read 4 x 64 contiguous bytes per row;
//   * the unit is dequantised in registers to bf16 (gfx950 scaled FP4/FP8 converts; exact, since
//     E2M1 x 2^e and E4M3 values are representable in bf16) and fed to
//     v_mfma_f32_16x16x32_bf16 with the activations as the A operand (fp32 accumulation);
//   * per-wave partial tiles are summed through LDS and the epilogue applies row/column scales
//     and bias, rounding once to the output dtype.
// Reference semantics: sgl_kernel_axera/gemm.py:564-641 (mx_gemm_kernel, mxfp4_gemm),
// gemm.py:119-181 (scaled GEMM), q35_mx_build.py:100-115 (proj_mx).
#include "axk_common.h"
#include "axk_host.h"
#include "axk_mx_tile.h"

namespace {

using axk::WF_BF16;
using axk::WF_FP8;
using axk::WF_MXFP4;
using axk::WUnit;

constexpr int kMaxWaves = 16;

// One workgroup: output channels [16*blockIdx.x, +16) x rows [32*blockIdx.y... ) in MT tiles of 16.
// Lane l: N column nl = l % 16, K group g = l / 16. Chunk c covers K [c*4V, (c+1)*4V); the lane's
// unit inside it is [c*4V + g*V, +V). MFMA step s uses k = unit + 8s .. +8 for both operands.
template <int F, int MT>
__global__ __launch_bounds__(1024) void mx_linear_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                          const uint8_t* __restrict__ w,
                                                          const uint8_t* __restrict__ wscale,
                                                          const float* __restrict__ row_scale,
                                                          const float* __restrict__ col_scale,
                                                          const float* __restrict__ bias, void* __restrict__ out,
                                                          int out_f32, int M, int N, int64_t K) {
  __shared__ float red[kMaxWaves * MT * 4 * 64];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int nl = lane & 15;
  const int64_t n = (int64_t)blockIdx.x * 16 + nl;
  const int m0 = blockIdx.y * 16 * MT;
  const bool nvalid = n < N;

  const uint16_t* xrow[MT];
  bool mvalid[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = m0 + t * 16 + nl;
    mvalid[t] = m < M;
    xrow[t] = x + (int64_t)(mvalid[t] ? m : 0) * ldx;
  }

  axk_f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = axk_f32x4{0.f, 0.f, 0.f, 0.f};
  axk::mx_tile_accum<F, MT>(xrow, mvalid, w, wscale, n, nvalid, K, wave, nwaves, acc);

#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[((wave * MT + t) * 4 + r) * 64 + lane] = acc[t][r];
  __syncthreads();

  for (int idx = threadIdx.x; idx < MT * 256; idx += blockDim.x) {
    const int t = idx >> 8, r = (idx >> 6) & 3, l = idx & 63;
    float v = 0.f;
    for (int wv = 0; wv < nwaves; ++wv) v += red[((wv * MT + t) * 4 + r) * 64 + l];
    const int m = m0 + t * 16 + 4 * (l >> 4) + r;
    const int64_t nn = (int64_t)blockIdx.x * 16 + (l & 15);
    if (m < M && nn < N) {
      if (row_scale) v *= row_scale[m];
      if (col_scale) v *= col_scale[nn];
      if (bias) v += bias[nn];
      if (out_f32)
        reinterpret_cast<float*>(out)[(int64_t)m * N + nn] = v;
      else
        reinterpret_cast<uint16_t*>(out)[(int64_t)m * N + nn] = (uint16_t)f32_to_bf16_bits(v);
    }
  }
}

// Exact E2M1 x E8M0 -> fp32, one 32-value block per thread.
__global__ __launch_bounds__(256) void mxfp4_dequant_kernel(const uint8_t* __restrict__ codes,
                                                            const uint8_t* __restrict__ scales,
                                                            float* __restrict__ out, int64_t N, int64_t K) {
  const int64_t nbk = K >> 5;
  const int64_t total = N * nbk;
  for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < total; b += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = b / nbk, kb = b - n * nbk;
    const uint4 q = *reinterpret_cast<const uint4*>(codes + n * (K >> 1) + kb * 16);
    const float sc = e8m0_to_f32(scales[n * nbk + kb]);
    float4* o = reinterpret_cast<float4*>(out + n * K + kb * 32);
    const uint32_t words[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t wd = words[i];
      float4 lo, hi;
      lo.x = e2m1_to_f32(wd) * sc;
      lo.y = e2m1_to_f32(wd >> 4) * sc;
      lo.z = e2m1_to_f32(wd >> 8) * sc;
      lo.w = e2m1_to_f32(wd >> 12) * sc;
      hi.x = e2m1_to_f32(wd >> 16) * sc;
      hi.y = e2m1_to_f32(wd >> 20) * sc;
      hi.z = e2m1_to_f32(wd >> 24) * sc;
      hi.w = e2m1_to_f32(wd >> 28) * sc;
      o[2 * i] = lo;
      o[2 * i + 1] = hi;
    }
  }
}

template <int F>
int launch_linear(const uint16_t* a, int64_t lda, const uint8_t* w, const uint8_t* ws, const float* row_scale,
                  const float* col_scale, const float* bias, void* out, int out_dtype, int64_t m, int64_t n,
                  int64_t k, axk_stream_t stream) {
  AXK_REQUIRE(a && w && out, AXK_E_NULL);
  AXK_REQUIRE(F != WF_MXFP4 || ws, AXK_E_NULL);
  AXK_REQUIRE(m >= 0 && n >= 0 && k > 0 && k % 32 == 0, AXK_E_SHAPE);
  AXK_REQUIRE(m <= INT32_MAX && n <= INT32_MAX, AXK_E_SHAPE);
  AXK_REQUIRE(lda >= k && lda % 8 == 0, AXK_E_ALIGN);
  AXK_REQUIRE(axk_aligned(a, 16) && axk_aligned(w, 16), AXK_E_ALIGN);
  AXK_REQUIRE(out_dtype == AXK_DT_BF16 || out_dtype == AXK_DT_F32, AXK_E_DTYPE);
  if (m == 0 || n == 0) return AXK_OK;
  const size_t out_bytes = (size_t)m * n * (out_dtype == AXK_DT_F32 ? 4 : 2);
  const size_t a_bytes = (size_t)((m - 1) * lda + k) * 2;
  AXK_REQUIRE(!axk_overlap(out, out_bytes, a, a_bytes), AXK_E_ALIAS);

  constexpr int CH = 4 * WUnit<F>::V;
  const int64_t nc = (k + CH - 1) / CH;
  const int waves = (int)(nc < kMaxWaves ? nc : kMaxWaves);
  const int mt = m <= 16 ? 1 : 2;
  dim3 grid((unsigned)((n + 15) / 16), (unsigned)((m + 16 * mt - 1) / (16 * mt)));
  dim3 block(64 * waves);
  const int of32 = out_dtype == AXK_DT_F32;
  if (mt == 1)
    hipLaunchKernelGGL((mx_linear_kernel<F, 1>), grid, block, 0, axk_stream(stream), a, lda, w, ws, row_scale,
                       col_scale, bias, out, of32, (int)m, (int)n, k);
  else
    hipLaunchKernelGGL((mx_linear_kernel<F, 2>), grid, block, 0, axk_stream(stream), a, lda, w, ws, row_scale,
                       col_scale, bias, out, of32, (int)m, (int)n, k);
  return axk_launch_status();
}

}  // namespace

extern "C" int axk_mxfp4_dequant(const uint8_t* codes, const uint8_t* scales, float* out, int64_t n, int64_t k,
                                 axk_stream_t stream) {
  AXK_REQUIRE(codes && scales && out, AXK_E_NULL);
  AXK_REQUIRE(n >= 0 && k > 0 && k % 32 == 0, AXK_E_SHAPE);
  AXK_REQUIRE(axk_aligned(codes, 16) && axk_aligned(out, 16), AXK_E_ALIGN);
  if (n == 0) return AXK_OK;
  AXK_REQUIRE(!axk_overlap(out, (size_t)n * k * 4, codes, (size_t)n * k / 2), AXK_E_ALIAS);
  const int64_t blocks = n * (k / 32);
  int64_t grid = (blocks + 255) / 256;
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(mxfp4_dequant_kernel, dim3((unsigned)grid), dim3(256), 0, axk_stream(stream), codes, scales, out,
                     n, k);
  return axk_launch_status();
}

extern "C" int axk_mxfp4_gemm(const uint16_t* a, int64_t lda, const uint8_t* b_fp4, const uint8_t* b_scale,
                              const float* bias, void* out, int out_dtype, int64_t m, int64_t n, int64_t k,
                              axk_stream_t stream) {
  return launch_linear<WF_MXFP4>(a, lda, b_fp4, b_scale, nullptr, nullptr, bias, out, out_dtype, m, n, k, stream);
}

extern "C" int axk_fp8_gemm(const uint16_t* a, int64_t lda, const uint8_t* b_fp8, const float* scale_a,
                            const float* scale_b, const float* bias, void* out, int out_dtype, int64_t m, int64_t n,
                            int64_t k, axk_stream_t stream) {
  AXK_REQUIRE(scale_b, AXK_E_NULL);
  return launch_linear<WF_FP8>(a, lda, b_fp8, nullptr, scale_a, scale_b, bias, out, out_dtype, m, n, k, stream);
}

extern "C" int axk_bf16_gemm(const uint16_t* a, int64_t lda, const uint16_t* b, const float* bias, void* out,
                             int out_dtype, int64_t m, int64_t n, int64_t k, axk_stream_t stream) {
  return launch_linear<WF_BF16>(a, lda, reinterpret_cast<const uint8_t*>(b), nullptr, nullptr, nullptr, bias, out,
                                out_dtype, m, n, k, stream);
}
