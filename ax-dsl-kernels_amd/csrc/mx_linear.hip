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
// STAGE: the weights are read as whole 128-byte row segments through a wave-private LDS tile
// (axk::mx_tile_accum_staged); wave w takes segments w, w + nwaves, ...
template <int F, int MT, bool STAGE>
__global__ __launch_bounds__(1024) void mx_linear_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                          const uint8_t* __restrict__ w,
                                                          const uint8_t* __restrict__ wscale,
                                                          const float* __restrict__ row_scale,
                                                          const float* __restrict__ col_scale,
                                                          const float* __restrict__ bias, void* __restrict__ out,
                                                          int out_f32, int M, int N, int64_t K) {
  // the waves' staging tiles, then (after a barrier) the cross-wave partial sums
  constexpr int kTileBytes = kMaxWaves * 16 * axk::kSegLd, kRedBytes = kMaxWaves * MT * 4 * 64 * 4;
  __shared__ __align__(16) unsigned char smem[kTileBytes > kRedBytes ? kTileBytes : kRedBytes];
  float* red = reinterpret_cast<float*>(smem);

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
  if (STAGE) {
    axk::mx_tile_accum_staged<F, MT>(xrow, mvalid, w, wscale, (int64_t)blockIdx.x * 16, N, K, wave, nwaves,
                                     smem + wave * 16 * axk::kSegLd, acc);
    __syncthreads();  // the staging tiles become the reduction buffer
  } else {
    axk::mx_tile_accum<F, MT>(xrow, mvalid, w, wscale, n, nvalid, K, wave, nwaves, acc);
  }

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

// Exact E2M1 x E8M0 -> fp32. Lane-consecutive quads of 4 values: a wave's stores cover contiguous 1 KiB
// (64 lanes x 16 bytes) and its code loads contiguous 128 bytes. A thread converts kDqQuads quads, 64 quads
// apart, with every load issued before the first store. Requires K % 32 == 0 (rows are whole quads).
constexpr int kDqQuads = 4;
__global__ __launch_bounds__(256) void mxfp4_dequant_kernel(const uint8_t* __restrict__ codes,
                                                            const uint8_t* __restrict__ scales,
                                                            float* __restrict__ out, int64_t N, int64_t K) {
  const int64_t qpr = K >> 2, total = N * qpr;  // quads per row, quads in all
  const int lane = threadIdx.x & 63;
  const int64_t wave_base = ((int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * (64 * kDqQuads);
  const int64_t wave_step = (int64_t)gridDim.x * (blockDim.x >> 6) * (64 * kDqQuads);
  for (int64_t q0 = wave_base + lane; q0 < total; q0 += wave_step) {
    uint32_t c[kDqQuads];
    float sc[kDqQuads];
#pragma unroll
    for (int j = 0; j < kDqQuads; ++j) {
      const int64_t q = min(q0 + 64 * j, total - 1);  // clamped: in bounds, never stored past total
      const int64_t n = q / qpr, kq = (q - n * qpr) << 2;
      c[j] = *reinterpret_cast<const uint16_t*>(codes + n * (K >> 1) + (kq >> 1));
      sc[j] = e8m0_to_f32(scales[n * (K >> 5) + (kq >> 5)]);
    }
#pragma unroll
    for (int j = 0; j < kDqQuads; ++j) {
      const int64_t q = q0 + 64 * j;
      if (q < total)
        reinterpret_cast<float4*>(out)[q] = make_float4(e2m1_to_f32(c[j]) * sc[j], e2m1_to_f32(c[j] >> 4) * sc[j],
                                                        e2m1_to_f32(c[j] >> 8) * sc[j], e2m1_to_f32(c[j] >> 12) * sc[j]);
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

  // staged weight loads when rows are whole 128-byte segments (and MXFP4 scale rows 8-byte aligned)
  const int64_t rb = axk::row_bytes<F>(k);
  const bool stage = rb % axk::kSegBytes == 0 && (F != WF_MXFP4 || axk_aligned(ws, 8));
  constexpr int CH = 4 * WUnit<F>::V;
  const int64_t nc = stage ? rb / axk::kSegBytes : (k + CH - 1) / CH;  // K work units: segments or chunks
  const int waves = (int)(nc < kMaxWaves ? nc : kMaxWaves);
  const int mt = m <= 16 ? 1 : 2;
  dim3 grid((unsigned)((n + 15) / 16), (unsigned)((m + 16 * mt - 1) / (16 * mt)));
  dim3 block(64 * waves);
  const int of32 = out_dtype == AXK_DT_F32;
  hipStream_t st = axk_stream(stream);
#define AXK_MX_LAUNCH(MT_, ST_)                                                                            \
  hipLaunchKernelGGL((mx_linear_kernel<F, MT_, ST_>), grid, block, 0, st, a, lda, w, ws, row_scale, col_scale, \
                     bias, out, of32, (int)m, (int)n, k)
  if (mt == 1) {
    if (stage) AXK_MX_LAUNCH(1, true); else AXK_MX_LAUNCH(1, false);
  } else {
    if (stage) AXK_MX_LAUNCH(2, true); else AXK_MX_LAUNCH(2, false);
  }
#undef AXK_MX_LAUNCH
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
  const int64_t waves = (n * (k / 4) + 64 * kDqQuads - 1) / (64 * kDqQuads);
  int64_t grid = (waves + 3) / 4;
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
