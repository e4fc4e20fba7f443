// MXFP4 codec and runtime-weight linear (MXFP4 / FP8 E4M3 / bf16 weights) for gfx950.
//
// Decode-shaped projections (m <= 32 rows per launch tile) are pure weight streaming: every weight
// byte is read once, so the kernel is bound by HBM bandwidth. The design:
//   * a 16-row weight tile is one MFMA N tile; a workgroup holds NT tiles (one or two) and splits K across
//     its waves in 128-byte row segments, so each activation fragment a wave loads feeds NT tiles;
//   * a segment of a tile is read as two instructions of 8 rows x 128 bytes (whole cache lines), staged
//     through a wave-private LDS tile and read back in the MFMA layout (rows whose byte length is not a
//     multiple of 128 take an unstaged kernel that loads one 16-byte unit per lane);
//   * the unit is dequantised in registers to bf16 (gfx950 scaled FP4/FP8 converts; exact, since
//     E2M1 x 2^e and E4M3 values are representable in bf16) and fed to
//     v_mfma_f32_16x16x32_bf16 with the activations as the A operand (fp32 accumulation);
//   * per-wave partial tiles are summed through LDS and the epilogue applies row/column scales
//     and bias, rounding once to the output dtype.
// One launch may cover a group of up to four weight matrices that share the activations (the projections of
// one decode layer): their tiles are laid end to end. Two fused epilogues serve the MLP: SwiGLU (a gate and an
// up matrix of one shape, out = bf16(silu(bf16 g) * bf16 u)) and the residual add (out = bf16(res + bf16 y)),
// each rounding exactly where the separate ops round.
// Reference semantics: sgl_kernel_axera/gemm.py:564-641 (mx_gemm_kernel, mxfp4_gemm),
// gemm.py:119-181 (scaled GEMM), q35_mx_build.py:100-115 (proj_mx), q35_step.py:118-142 (mlp_block).
#include "axk_common.h"
#include "axk_host.h"
#include "axk_mx_tile.h"

namespace {

using axk::WF_BF16;
using axk::WF_FP8;
using axk::WF_MXFP4;
using axk::WUnit;

constexpr int kMaxWaves = 16;  // unstaged kernel
constexpr int kGroupWaves = 8;  // group kernel: waves per workgroup (at most)
constexpr int kGroupMaxNT = 2;  // group kernel: N tiles per workgroup (at most)

enum { EPI_PLAIN = 0, EPI_SWIGLU = 1, EPI_RES = 2 };

// Unstaged kernel, for rows whose byte length is not a multiple of 128. One workgroup: output channels
// [16*blockIdx.x, +16) x rows [16*MT*blockIdx.y, ...) in MT tiles of 16. Lane l: N column nl = l % 16, K group
// g = l / 16. Chunk c covers K [c*4V, (c+1)*4V); the lane's unit inside it is [c*4V + g*V, +V).
template <int F, int MT>
__global__ __launch_bounds__(1024) void mx_linear_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                          const uint8_t* __restrict__ w,
                                                          const uint8_t* __restrict__ wscale,
                                                          const float* __restrict__ row_scale,
                                                          const float* __restrict__ col_scale,
                                                          const float* __restrict__ bias,
                                                          const float* __restrict__ gscale, void* __restrict__ out,
                                                          int out_f32, int M, int N, int64_t K) {
  __shared__ __align__(16) float red[kMaxWaves * MT * 4 * 64];

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
      if (gscale) v *= *gscale;
      if (bias) v += bias[nn];
      if (out_f32)
        reinterpret_cast<float*>(out)[(int64_t)m * N + nn] = v;
      else
        reinterpret_cast<uint16_t*>(out)[(int64_t)m * N + nn] = (uint16_t)f32_to_bf16_bits(v);
    }
  }
}

// A group of weight matrices sharing the activations. Matrix i owns the virtual 16-row tiles
// [tile0[i], tile0[i + 1]); for EPI_SWIGLU matrix 0 is the gate and matrix 1 the up projection (one shape) and a
// workgroup's tile slots alternate gate / up over the same channels.
struct MxGroup {
  const uint8_t* w[AXK_MX_GROUP_MAX];
  const uint8_t* ws[AXK_MX_GROUP_MAX];
  const float* col_scale[AXK_MX_GROUP_MAX];
  const float* bias[AXK_MX_GROUP_MAX];
  const float* gscale[AXK_MX_GROUP_MAX];  // NVFP4: the matrix's fp32 scale2 (one value, device memory)
  void* out[AXK_MX_GROUP_MAX];
  int64_t ldo[AXK_MX_GROUP_MAX];
  int n[AXK_MX_GROUP_MAX];
  int tile0[AXK_MX_GROUP_MAX + 1];
  int count;
  const float* row_scale;
  const uint16_t* res;  // EPI_RES: the residual [M, n] (leading dimension ldr)
  int64_t ldr;
  int out_f32;
  // optional on matrix 0 (EPI_PLAIN): causal conv1d + SiLU over its bf16 output, one token per row, with the
  // conv state [M, conv_k - 1, n[0]] (conv_out may be conv_in)
  const uint16_t* conv_w;
  const uint16_t* conv_in;
  uint16_t* conv_out;
  int conv_k;
};

// Matrix and local tile of workgroup slot t.
template <int NT, int EPI>
AXK_DEV void slot_tile(const MxGroup& g, int t, int& mi, int& lt, bool& valid) {
  if (EPI == EPI_SWIGLU) {
    mi = t & 1;
    lt = (int)blockIdx.x * (NT / 2) + (t >> 1);
    valid = lt < g.tile0[1];
    if (!valid) lt = g.tile0[1] - 1;
  } else {
    int v = (int)blockIdx.x * NT + t;
    valid = v < g.tile0[g.count];
    if (!valid) v = g.tile0[g.count] - 1;
    mi = 0;
#pragma unroll
    for (int i = 1; i < AXK_MX_GROUP_MAX; ++i) mi += (i < g.count && v >= g.tile0[i]) ? 1 : 0;
    lt = v - g.tile0[mi];
  }
}

// Staged group kernel: wave w takes the 128-byte row segments d = w, w + nwaves, ... of its NT tiles (rows of
// whole segments; MXFP4 scale rows as 8-byte words). Segment d: the NT tiles' weights are loaded (two
// instructions of 8 rows x 128 bytes per tile: rows past a matrix's end re-read its last row), then the MT
// activation fragments, which every tile reuses; each tile goes through the wave's LDS tile into the MFMA layout
// (lane (nl, g): 16-byte unit g of each 64-byte chunk), so the k mapping is the unstaged kernel's. LDS is
// wave-private and in order: no barrier until the cross-wave sum.
// Occupancy: the 4-wave form (four tiles) is held to at least 4 waves per SIMD, what its LDS allows; left to
// itself the compiler spends enough registers to drop it to 3 (measured on the LM head: 59.5 against 44 us). The
// 8-wave forms keep the compiler's choice (forcing more waves there spills).
template <int F, int MT, int NT, int EPI, int WMAX = kGroupWaves>
__global__ __launch_bounds__(64 * WMAX) __attribute__((amdgpu_waves_per_eu(WMAX == 4 ? 4 : 1))) void mx_group_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const MxGroup g, int M, int64_t K) {
  using U = axk::WUnit<F>;
  constexpr int CH = 4 * U::V, SEGK = 2 * CH;  // values per 64-byte chunk, per 128-byte segment
  constexpr int kTileBytes = WMAX * NT * 16 * axk::kSegLd, kRedBytes = WMAX * NT * MT * 4 * 64 * 4;
  __shared__ __align__(16) unsigned char smem[kTileBytes > kRedBytes ? kTileBytes : kRedBytes];
  float* red = reinterpret_cast<float*>(smem);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int nl = lane & 15, kg = lane >> 4, lr = lane >> 3, lc = lane & 7;
  const int m0 = blockIdx.y * 16 * MT;
  const int64_t rb = axk::row_bytes<F>(K), ND = rb / axk::kSegBytes;
  unsigned char* tile = smem + wave * NT * 16 * axk::kSegLd;

  const uint16_t* xrow[MT];
  bool mvalid[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = m0 + t * 16 + nl;
    mvalid[t] = m < M;
    xrow[t] = x + (int64_t)(mvalid[t] ? m : 0) * ldx;
  }
  const uint8_t* src[NT][2];
  const uint8_t* srow[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int mi, lt;
    bool valid;
    slot_tile<NT, EPI>(g, t, mi, lt, valid);
    const int64_t n0 = (int64_t)lt * 16, nmax = g.n[mi] - 1;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t r = n0 + 8 * h + lr;
      src[t][h] = g.w[mi] + (r < nmax ? r : nmax) * rb + 16 * lc;
    }
    srow[t] = axk::has_block_scales(F) ? g.ws[mi] + (n0 + nl < nmax ? n0 + nl : nmax) * (K / (axk::is_nv(F) ? 16 : 32))
                                       : nullptr;
  }

  axk_f32x4 acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int u = 0; u < MT; ++u) acc[t][u] = axk_f32x4{0.f, 0.f, 0.f, 0.f};

  for (int64_t d = wave; d < ND; d += nwaves) {
    axk_u32x4 q[NT][2];
    uint2 sw[NT];  // the segment's E8M0 scales: 8 bytes (MXFP4: 256 values) or 4 (MXFP8: 128 values)
    uint4 sv[NT];  // NVFP4: the segment's 16 E4M3 scales (256 values)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int h = 0; h < 2; ++h)  // weights are read once: non-temporal
        q[t][h] = __builtin_nontemporal_load(reinterpret_cast<const axk_u32x4*>(src[t][h] + d * axk::kSegBytes));
      if (F == axk::WF_MXFP4) sw[t] = *reinterpret_cast<const uint2*>(srow[t] + 8 * d);
      if (F == axk::WF_NVFP4) sv[t] = *reinterpret_cast<const uint4*>(srow[t] + 16 * d);
      if (F == axk::WF_MXFP8 || F == axk::WF_MXBF8) sw[t].x = *reinterpret_cast<const uint32_t*>(srow[t] + 4 * d);
    }
    axk_bf16x8 a[MT][2][U::STEPS];
#pragma unroll
    for (int u = 0; u < MT; ++u)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int s = 0; s < U::STEPS; ++s)
          a[u][j][s] = mvalid[u] ? load_bf16x8(xrow[u] + d * SEGK + j * CH + kg * U::V + 8 * s) : zero_bf16x8();
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        *reinterpret_cast<axk_u32x4*>(tile + (t * 16 + 8 * h + lr) * axk::kSegLd + 16 * lc) = q[t][h];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint4 unit = __builtin_bit_cast(
            uint4, *reinterpret_cast<const axk_u32x4*>(tile + (t * 16 + nl) * axk::kSegLd + 64 * j + 16 * kg));
        // unit (j, kg) of the segment: values 64 j + V kg .. + V, in scale block (64 j + V kg) / 32 (NVFP4: the two
        // 16-value blocks 4 j + 2 kg and the next, bytes 2 (kg % 2) .. + 1 of dword 2 j + kg / 2)
        decltype(U::scale(nullptr, 0, 0, 0)) sc;
        if constexpr (F == axk::WF_NVFP4) {
          const uint32_t dw = (kg >> 1) ? (j ? sv[t].w : sv[t].y) : (j ? sv[t].z : sv[t].x);
          sc = (dw >> (16 * (kg & 1))) & 0xffffu;
        } else {
          sc = F == axk::WF_MXFP4 ? e8m0_to_f32(((j ? sw[t].y : sw[t].x) >> (8 * kg)) & 0xffu)
               : axk::is_mx(F)    ? e8m0_to_f32((sw[t].x >> (8 * (2 * j + (kg >> 1)))) & 0xffu)
                                  : 1.0f;
        }
#pragma unroll
        for (int s = 0; s < U::STEPS; ++s) {
          const axk_bf16x8 b = U::conv(unit, s, sc);
#pragma unroll
          for (int u = 0; u < MT; ++u) acc[t][u] = mfma_bf16_16x16x32(a[u][j][s], b, acc[t][u]);
        }
      }
    }
  }
  __syncthreads();  // the staging tiles become the reduction buffer
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int u = 0; u < MT; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[(((wave * NT + t) * MT + u) * 4 + r) * 64 + lane] = acc[t][u][r];
  __syncthreads();

  // element (u, r, l) of slot t: row m0 + 16u + 4(l / 16) + r, channel 16 lt + l % 16 of matrix mi
  auto total = [&](int t, int u, int r, int l) {
    float v = 0.f;
    for (int wv = 0; wv < nwaves; ++wv) v += red[(((wv * NT + t) * MT + u) * 4 + r) * 64 + l];
    return v;
  };
  auto emit = [&](int t, int mi, int lt, int e) {
    const int u = e >> 8, r = (e >> 6) & 3, l = e & 63;
    const int m = m0 + u * 16 + 4 * (l >> 4) + r;
    const int64_t nn = (int64_t)lt * 16 + (l & 15), n_i = g.n[mi];
    if (m >= M || nn >= n_i) return;
    float v = total(t, u, r, l);
    if (g.row_scale) v *= g.row_scale[m];
    if (g.col_scale[mi]) v *= g.col_scale[mi][nn];
    if (g.gscale[mi]) v *= *g.gscale[mi];
    if (g.bias[mi]) v += g.bias[mi][nn];
    if (EPI == EPI_SWIGLU) {
      float up = total(t + 1, u, r, l);
      if (g.row_scale) up *= g.row_scale[m];
      if (g.col_scale[1]) up *= g.col_scale[1][nn];
      if (g.gscale[1]) up *= *g.gscale[1];
      if (g.bias[1]) up += g.bias[1][nn];
      v = silu_f32(round_bf16(v)) * round_bf16(up);
    } else if (EPI == EPI_RES) {
      v = bf16_bits_to_f32(g.res[(int64_t)m * g.ldr + nn]) + round_bf16(v);
    } else if (g.conv_w && mi == 0) {  // the token enters the channel's conv window (q35_step.py:164)
      const int kc = g.conv_k;
      const float xt = round_bf16(v);
      float wk[kMaxConvTaps], hist[kMaxConvTaps];
#pragma unroll
      for (int j = 0; j < kMaxConvTaps; ++j) {
        wk[j] = j < kc ? bf16_bits_to_f32(g.conv_w[nn * kc + j]) : 0.f;
        hist[j] = j < kc - 1 ? bf16_bits_to_f32(g.conv_in[((int64_t)m * (kc - 1) + j) * n_i + nn]) : 0.f;
      }
      v = silu_f32(conv_taps(xt, wk, hist, kc));
#pragma unroll
      for (int j = 0; j < kMaxConvTaps - 1; ++j)
        if (j < kc - 1)
          g.conv_out[((int64_t)m * (kc - 1) + j) * n_i + nn] = (uint16_t)f32_to_bf16_bits(j + 1 < kc - 1 ? hist[j + 1] : xt);
    }
    if (g.out_f32)
      reinterpret_cast<float*>(g.out[mi])[(int64_t)m * g.ldo[mi] + nn] = v;
    else
      reinterpret_cast<uint16_t*>(g.out[mi])[(int64_t)m * g.ldo[mi] + nn] = (uint16_t)f32_to_bf16_bits(v);
  };
  constexpr int kOutSlots = EPI == EPI_SWIGLU ? NT / 2 : NT;
  if constexpr (WMAX == 4) {
    // the four-tile form (short-lived workgroups): slots unrolled, each slot's matrix resolved once (measured on
    // the LM head: 58.9 -> 52 us); the eight-wave forms keep the compact loop (smaller code, measured faster there)
#pragma unroll
    for (int o = 0; o < kOutSlots; ++o) {
      const int t = EPI == EPI_SWIGLU ? 2 * o : o;
      int mi, lt;
      bool valid;
      slot_tile<NT, EPI>(g, t, mi, lt, valid);
      if (!valid) continue;  // uniform
      for (int e = threadIdx.x; e < MT * 256; e += blockDim.x) emit(t, mi, lt, e);
    }
  } else {
    for (int idx = threadIdx.x; idx < kOutSlots * MT * 256; idx += blockDim.x) {
      const int o = idx / (MT * 256), t = EPI == EPI_SWIGLU ? 2 * o : o;
      int mi, lt;
      bool valid;
      slot_tile<NT, EPI>(g, t, mi, lt, valid);
      if (valid) emit(t, mi, lt, idx - o * (MT * 256));
    }
  }
}

// Exact E2M1 x E8M0 -> fp32. Lane-consecutive quads of 4 values: a wave's stores cover contiguous 1 KiB
// (64 lanes x 16 bytes) and its code loads contiguous 128 bytes. A thread converts kDqQuads quads, 64 quads
// apart, with every load issued before the first store. Codes and output are streamed once (non-temporal).
// Requires K % 32 == 0 (rows are whole quads).
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
      c[j] = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(codes + n * (K >> 1) + (kq >> 1)));
      sc[j] = e8m0_to_f32(scales[n * (K >> 5) + (kq >> 5)]);
    }
#pragma unroll
    for (int j = 0; j < kDqQuads; ++j) {
      const int64_t q = q0 + 64 * j;
      if (q < total)
        store_nt(out + 4 * q, axk_u32x4{__float_as_uint(e2m1_to_f32(c[j]) * sc[j]), __float_as_uint(e2m1_to_f32(c[j] >> 4) * sc[j]),
                                        __float_as_uint(e2m1_to_f32(c[j] >> 8) * sc[j]),
                                        __float_as_uint(e2m1_to_f32(c[j] >> 12) * sc[j])});
    }
  }
}

template <int F, int MT, int NT, int EPI, int WMAX = kGroupWaves>
void launch_group(const uint16_t* a, int64_t lda, const MxGroup& g, int64_t m, int64_t k, int64_t slots,
                  hipStream_t st) {
  const int64_t nd = axk::row_bytes<F>(k) / axk::kSegBytes;
  const int waves = (int)(nd < WMAX ? nd : WMAX);
  dim3 grid((unsigned)((slots + NT - 1) / NT), (unsigned)((m + 16 * MT - 1) / (16 * MT)));
  hipLaunchKernelGGL((mx_group_kernel<F, MT, NT, EPI, WMAX>), grid, dim3(64 * waves), 0, st, a, lda, g, (int)m, k);
}

template <int F, int EPI>
int group_dispatch(const uint16_t* a, int64_t lda, const MxGroup& g, int64_t m, int64_t k, hipStream_t st) {
  const int tiles = g.tile0[g.count];
  const int64_t slots = EPI == EPI_SWIGLU ? 2 * (int64_t)g.tile0[1] : tiles;
  // short rows (<= 8 segments) of a very wide matrix (the LM head): four tiles and four waves per workgroup, so a
  // wave streams two segments of four tiles (measured on 248320 x 2048 MXFP4: 60 -> 44 us against two tiles and
  // eight waves)
  const int64_t nd = axk::row_bytes<F>(k) / axk::kSegBytes;
  if (EPI == EPI_PLAIN && m <= 16 && nd <= 8 && tiles >= 4096) {
    launch_group<F, 1, 4, EPI, 4>(a, lda, g, m, k, slots, st);
    return axk_launch_status();
  }
  // two tiles per workgroup when that still leaves >= 384 workgroups per M tile (a SwiGLU pair always)
  const bool two = EPI == EPI_SWIGLU || tiles >= 768;
  if (m <= 16) {
    if (two) launch_group<F, 1, 2, EPI>(a, lda, g, m, k, slots, st);
    else launch_group<F, 1, 1, EPI>(a, lda, g, m, k, slots, st);
  } else {
    if (two) launch_group<F, 2, 2, EPI>(a, lda, g, m, k, slots, st);
    else launch_group<F, 2, 1, EPI>(a, lda, g, m, k, slots, st);
  }
  return axk_launch_status();
}

// ---------------------------------------------------------------------------------------------
// The large-M path (prefill): a dense GEMM over the matrices of a group (or a gate / up pair) with an LDS pipeline.
// Workgroup = BM activation rows (dg_bm: 128 for MXFP4, 64 for the 8-bit formats) x 256 weight rows (EPI_SWIGLU: 128
// gate + the same 128 up channels), wave w a BM x 64 block of BM / 16 by four MFMA tiles (every A fragment feeds
// four MFMAs, every decoded B fragment BM / 16). The activation rows and the
// weight rows of each 64-wide K step land in a ring of kDgStages LDS slots by direct loads two steps ahead, one
// barrier per step: A [BM rows][128 B] with 16-byte chunk c of row r at position c ^ (r & 7); B [256 rows][RB bytes]
// (RB = 32 for MXFP4, 64 for the 8-bit formats) with 16-byte chunk c of row r at c ^ ((r >> 3) & 1) (MXFP4) or
// c ^ ((r >> 2) & 3) (8-bit): the fragment reads are free of bank conflicts. The E8M0 bytes of each step come with
// the step's direct loads (one dword per weight row), so LDS holds only the ring (75 KiB for MXFP4, 73.5 KiB for the
// 8-bit formats) and two workgroups share a CU; FP8 per-channel scales, biases, row scales and the SwiGLU / residual epilogues as the group
// kernel's. Consecutive workgroups go round-robin over the 8 XCDs, so each XCD takes a contiguous run of the tile
// order, which walks groups of 8 row blocks across all column blocks: an XCD's L2 keeps its activation rows.
// ---------------------------------------------------------------------------------------------
constexpr int kDgBN = 256, kDgBK = 64, kDgStages = 3, kDgXcds = 8, kDgGroupRows = 8;
// activation rows per workgroup: 128 for MXFP4 (each decoded weight fragment feeds eight MFMAs; a 75 KiB ring, two
// workgroups a CU), 64 for the 8-bit formats (whose 64-byte weight rows would make a 128-row ring 99 KiB: one a CU)
template <int F>
constexpr int dg_bm() { return axk::is_fp4(F) ? 128 : 64; }
template <int F>
constexpr int dg_mt() { return dg_bm<F>() / 16; }  // 16-row MFMA tiles per wave (a wave spans every row of the tile)
template <int F>
constexpr int dg_ai() { return dg_bm<F>() * kDgBK * 2 / 1024 / 4; }  // A direct-load instructions per wave and step
template <int F>
constexpr int dg_astage() { return dg_bm<F>() * kDgBK * 2; }
constexpr int64_t kDgMinRows = 128;  // below this the group kernel (weights streamed once per 16 / 32 rows) is faster
template <int F>
constexpr int dg_row_bytes() { return axk::is_fp4(F) ? kDgBK / 2 : kDgBK; }  // weight bytes per row and step
constexpr int kDgSStage = kDgBN * 4;  // MX formats: one scale dword per weight row and step
template <int F>
constexpr int dg_stage() {
  return dg_astage<F>() + kDgBN * dg_row_bytes<F>() + (axk::has_block_scales(F) ? kDgSStage : 0);
}
template <int F>
size_t dg_lds_bytes(int64_t) {
  return (size_t)kDgStages * dg_stage<F>();
}

struct DgArgs {
  const uint16_t* a;
  int64_t lda;
  const uint8_t* w[AXK_MX_GROUP_MAX];   // EPI_PLAIN: the group's matrices; EPI_SWIGLU: gate, up; EPI_RES: one
  const uint8_t* ws[AXK_MX_GROUP_MAX];  // E8M0 scales [n, k/32] (MX formats)
  const float* col_scale[AXK_MX_GROUP_MAX];
  const float* bias[AXK_MX_GROUP_MAX];
  const float* gscale[AXK_MX_GROUP_MAX];  // NVFP4 scale2
  void* out[AXK_MX_GROUP_MAX];
  int64_t ldo[AXK_MX_GROUP_MAX];
  int n[AXK_MX_GROUP_MAX];
  int cb0[AXK_MX_GROUP_MAX + 1];  // EPI_PLAIN: first column block of each matrix (cb0[count] = all of them)
  int count;
  const float* row_scale;
  const uint16_t* res;  // EPI_RES
  int64_t ldr;
  int out_f32;
  int m, k;
};

template <int F>
AXK_DEV axk_bf16x8 dg_decode(const unsigned char* row, int kh, int g4, int r, float sc) {
  if constexpr (axk::is_fp4(F)) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(row + 16 * (kh ^ ((r >> 3) & 1)) + 4 * g4);
    if constexpr (F == axk::WF_NVFP4) return fp4x8_to_bf16x8_mul(w, sc);
    else return fp4x8_to_bf16x8(w, sc);
  } else {
    // 8 bytes (k = 32 kh + 8 g4 ..) of the 64-byte row: chunk 2 kh + g4 / 2, half g4 % 2
    const int c = (2 * kh + (g4 >> 1)) ^ ((r >> 2) & 3);
    const uint2 w = *reinterpret_cast<const uint2*>(row + 16 * c + 8 * (g4 & 1));
    const uint4 q = make_uint4(w.x, w.y, 0u, 0u);
    return axk::WUnit<F>::conv(q, 0, sc);
  }
}

template <int F, int EPI>
__global__ __launch_bounds__(256, 2) void mx_gemm_kernel(DgArgs g) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int RB = dg_row_bytes<F>(), STAGE = dg_stage<F>();
  constexpr int kDgBM = dg_bm<F>(), kDgMT = dg_mt<F>(), kDgAI = dg_ai<F>(), kDgAStage = dg_astage<F>();
  constexpr int COLS = EPI == EPI_SWIGLU ? kDgBN / 2 : kDgBN;  // output channels per workgroup
  const int nb = EPI == EPI_PLAIN ? g.cb0[g.count] : (g.n[0] + COLS - 1) / COLS, mb = (g.m + kDgBM - 1) / kDgBM;
  const int total = nb * mb, per = (total + kDgXcds - 1) / kDgXcds;
  const int q = blockIdx.x / kDgXcds, lid = (blockIdx.x % kDgXcds) * per + q;
  if (q >= per || lid >= total) return;
  // groups of kDgGroupRows row blocks, column blocks inner: an XCD's run of tiles (and the 64 it runs at once) covers
  // a few row blocks across the column blocks, so its L2 keeps those activation rows for every column block
  const int gfirst = (lid / (kDgGroupRows * nb)) * kDgGroupRows, gsize = min(mb - gfirst, kDgGroupRows);
  const int inner = lid - gfirst * nb;
  const int rbk = gfirst + inner % gsize, cb = inner / gsize;
  int mat = 0;  // EPI_PLAIN: the matrix whose column blocks hold cb (workgroup-uniform)
  if constexpr (EPI == EPI_PLAIN)
    while (mat + 1 < g.count && cb >= g.cb0[mat + 1]) ++mat;
  const int N = g.n[mat];
  const int col0 = (cb - (EPI == EPI_PLAIN ? g.cb0[mat] : 0)) * COLS, m0 = rbk * kDgBM;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, g4 = lane >> 4;
  const int K = g.k, nk = K / kDgBK;
  const uint32_t lds0 = lds_addr(smem);

  // LDS weight row rho -> weight row (SwiGLU: rho < 128 the gate channel col0 + rho, else the up channel col0 + rho -
  // 128), clamped to the last channel (never stored)
  auto wrow = [&](int rho, bool scale) -> const uint8_t* {
    const int mi = EPI == EPI_SWIGLU ? (rho >= COLS ? 1 : 0) : mat;
    const int c = min(col0 + (EPI == EPI_SWIGLU ? (rho & (COLS - 1)) : rho), N - 1);
    return scale ? g.ws[mi] + (int64_t)c * (K / (axk::is_nv(F) ? 16 : 32))
                 : g.w[mi] + (int64_t)c * axk::row_bytes<F>(K);
  };
  // per-lane sources of this wave's direct loads of a step: A instructions i = kDgAI wave + h (rows 8 i + lane / 8,
  // chunk (lane % 8) ^ (row & 7)); B instructions (RB == 32: 2 per wave, 32 rows each; RB == 64: 4 per wave,
  // 16 rows each)
  constexpr int BI = kDgBN * RB / 1024 / 4;  // B instructions per wave and step
  static_assert(kDgAI * 4 * 1024 == kDgAStage && BI * 4 * 1024 == kDgBN * RB, "the direct loads cover the stage");
  const uint16_t* asrc[kDgAI];
  const uint8_t* bsrc[BI];
#pragma unroll
  for (int h = 0; h < kDgAI; ++h) {
    const int i = kDgAI * wave + h;
    const int r = 8 * i + (lane >> 3), rr = min(m0 + r, g.m - 1), ch = (lane & 7) ^ (r & 7);
    asrc[h] = g.a + (int64_t)rr * g.lda + 8 * ch;
  }
#pragma unroll
  for (int h = 0; h < BI; ++h) {
    const int i = BI * wave + h;
    if constexpr (RB == 32) {
      const int rho = 32 * i + (lane >> 1);
      bsrc[h] = wrow(rho, false) + 16 * ((lane & 1) ^ ((rho >> 3) & 1));
    } else {
      const int rho = 16 * i + (lane >> 2);
      bsrc[h] = wrow(rho, false) + 16 * ((lane & 3) ^ ((rho >> 2) & 3));
    }
  }
  int brow[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    brow[j] = EPI == EPI_SWIGLU ? (j >> 1) * COLS + 32 * wave + 16 * (j & 1) : 64 * wave + 16 * j;
  // the E8M0 bytes of a step (MX formats) join the direct loads: wave w loads the aligned dword holding blocks
  // 4 (ks / 2) .. + 3 of weight rows 64 w + lane into the slot's scale table [256 rows][4 B], so no whole-K scale
  // table takes LDS (which then fits several workgroups a CU) and the loop has no load the compiler waits on
  // (NVFP4: the dword holding the step's four 16-value blocks)
  const uint8_t* ssrc = axk::has_block_scales(F) ? wrow(64 * wave + lane, true) : nullptr;
  // step ks into ring slot BUF (past the last step the last one again: in bounds, unused), so every iteration
  // waits on the same count
  auto issue = [&](int ks, auto buf_c) __attribute__((always_inline)) {
    constexpr int BUF = decltype(buf_c)::value;
    const int kk = min(ks, nk - 1);
    const uint32_t base = lds0 + BUF * STAGE;
#pragma unroll
    for (int h = 0; h < kDgAI; ++h) lds_dma16_cached(asrc[h] + kk * kDgBK, base + (kDgAI * wave + h) * 1024);
#pragma unroll
    for (int h = 0; h < BI; ++h) lds_dma16_cached(bsrc[h] + kk * RB, base + kDgAStage + (BI * wave + h) * 1024);
    if constexpr (axk::is_mx(F))
      lds_dma4_cached(ssrc + 4 * (kk >> 1), base + kDgAStage + kDgBN * RB + 256 * wave);
    if constexpr (axk::is_nv(F)) lds_dma4_cached(ssrc + 4 * kk, base + kDgAStage + kDgBN * RB + 256 * wave);
  };
  constexpr int LPS = kDgAI + BI + (axk::has_block_scales(F) ? 1 : 0);  // vector-memory instructions per step
  issue(0, std::integral_constant<int, 0>{});
  issue(1, std::integral_constant<int, 1>{});
  axk_f32x4 acc[kDgMT][4];
#pragma unroll
  for (int mt = 0; mt < kDgMT; ++mt)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[mt][j] = axk_f32x4{0.f, 0.f, 0.f, 0.f};

  auto step = [&](int ks, auto buf_c) __attribute__((always_inline)) {
    constexpr int BUF = decltype(buf_c)::value;
    wait_vmcnt<LPS>();  // this wave's loads of step ks have landed (step ks + 1's may not have)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's reads of step ks - 1 are done
    __builtin_amdgcn_s_barrier();  // every wave's step-ks loads landed; every wave is done with step ks - 1
    asm volatile("" ::: "memory");
    issue(ks + 2, std::integral_constant<int, (BUF + 2) % kDgStages>{});  // into the slot of step ks - 1
    const unsigned char* sa = smem + BUF * STAGE;
    const unsigned char* sb = sa + kDgAStage;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      axk_bf16x8 af[kDgMT], bf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = brow[j] + l16;
        const float sc = axk::is_mx(F)   ? e8m0_to_f32(sb[kDgBN * RB + 4 * r + 2 * (ks & 1) + kh])
                         : axk::is_nv(F) ? e4m3_to_f32(sb[kDgBN * RB + 4 * r + 2 * kh + (g4 >> 1)])
                                         : 1.0f;
        bf[j] = dg_decode<F>(sb + r * RB, kh, g4, r, sc);
      }
#pragma unroll
      for (int mt = 0; mt < kDgMT; ++mt) {
        const int r = 16 * mt + l16;
        af[mt] = *reinterpret_cast<const axk_bf16x8*>(sa + r * 128 + 16 * ((4 * kh + g4) ^ (r & 7)));
      }
#pragma unroll
      for (int mt = 0; mt < kDgMT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[mt][j] = mfma_bf16_16x16x32(af[mt], bf[j], acc[mt][j]);
    }
  };
  static_assert(kDgStages == 3, "the K loop is unrolled over three ring slots");
  for (int ks = 0; ks < nk; ks += 3) {
    step(ks, std::integral_constant<int, 0>{});
    if (ks + 1 < nk) step(ks + 1, std::integral_constant<int, 1>{});
    if (ks + 2 < nk) step(ks + 2, std::integral_constant<int, 2>{});
  }
  wait_vmcnt<0>();  // the look-ahead loads land before the workgroup's LDS is released

  // element (mt, r) of tile j: row m0 + 16 mt + 4 g4 + r, weight row brow[j] + l16 (the group kernel's epilogue)
  auto fin = [&](int mi, int nn, int m, float v) {
    if (g.row_scale) v *= g.row_scale[m];
    if (g.col_scale[mi]) v *= g.col_scale[mi][nn];
    if (g.gscale[mi]) v *= *g.gscale[mi];
    if (g.bias[mi]) v += g.bias[mi][nn];
    return v;
  };
  if (g.out_f32) {  // fp32 outputs (EPI_PLAIN): stored directly, 64-byte runs of 16 lanes
#pragma unroll
    for (int mt = 0; mt < kDgMT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + 16 * mt + 4 * g4 + r;
        if (m >= g.m) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int nn = col0 + 64 * wave + 16 * j + l16;
          if (nn < N) reinterpret_cast<float*>(g.out[mat])[(int64_t)m * g.ldo[mat] + nn] = fin(mat, nn, m, acc[mt][j][r]);
        }
      }
    return;
  }
  // bf16 outputs go through an LDS tile [BM rows][COLS + 8] over the ring, then leave as 16-byte row segments
  // (EPI_RES: the residual read the same way and added as bf16(res + bf16(v)))
  constexpr int LDO = COLS + 8;
  static_assert(kDgBM * LDO * 2 <= kDgStages * STAGE, "the output tile fits in the ring");
  uint16_t* so = reinterpret_cast<uint16_t*>(smem);
  __syncthreads();  // every wave is done with the ring
#pragma unroll
  for (int mt = 0; mt < kDgMT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * mt + 4 * g4 + r, m = min(m0 + row, g.m - 1);
      if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int nn = min(col0 + 32 * wave + 16 * j + l16, N - 1);
          const float gv = fin(0, nn, m, acc[mt][j][r]), uv = fin(1, nn, m, acc[mt][j + 2][r]);
          so[row * LDO + 32 * wave + 16 * j + l16] =
              (uint16_t)f32_to_bf16_bits(silu_f32(round_bf16(gv)) * round_bf16(uv));
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int nn = min(col0 + 64 * wave + 16 * j + l16, N - 1);
          so[row * LDO + 64 * wave + 16 * j + l16] = (uint16_t)f32_to_bf16_bits(fin(mat, nn, m, acc[mt][j][r]));
        }
      }
    }
  __syncthreads();
  constexpr int SPR = COLS / 8;  // 8-column segments per row
  uint16_t* ob = reinterpret_cast<uint16_t*>(g.out[mat]);
  const int64_t ldo = g.ldo[mat];
  const bool vec = ldo % 8 == 0 && ((uintptr_t)ob & 15) == 0 &&
                   (EPI != EPI_RES || (g.ldr % 8 == 0 && ((uintptr_t)g.res & 15) == 0));
  for (int sidx = tid; sidx < kDgBM * SPR; sidx += 256) {
    const int row = sidx / SPR, seg = sidx - row * SPR, m = m0 + row, nn = col0 + 8 * seg;
    if (m >= g.m || nn >= N) continue;
    const uint16_t* src = so + row * LDO + 8 * seg;
    uint16_t* dst = ob + (int64_t)m * ldo + nn;
    if (vec && nn + 8 <= N) {
      uint4 v = *reinterpret_cast<const uint4*>(src);
      if constexpr (EPI == EPI_RES) {
        const uint4 rv = *reinterpret_cast<const uint4*>(g.res + (int64_t)m * g.ldr + nn);
        const uint32_t vw[4] = {v.x, v.y, v.z, v.w}, rw[4] = {rv.x, rv.y, rv.z, rv.w};
        uint32_t ow[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float lo = bf16_bits_to_f32(rw[i] & 0xffffu) + bf16_bits_to_f32(vw[i] & 0xffffu);
          const float hi = bf16_bits_to_f32(rw[i] >> 16) + bf16_bits_to_f32(vw[i] >> 16);
          ow[i] = f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
        }
        v = make_uint4(ow[0], ow[1], ow[2], ow[3]);
      }
      *reinterpret_cast<uint4*>(dst) = v;
    } else {
      for (int e = 0; e < 8 && nn + e < N; ++e) {
        float v = bf16_bits_to_f32(src[e]);
        if constexpr (EPI == EPI_RES) v = bf16_bits_to_f32(g.res[(int64_t)m * g.ldr + nn + e]) + v;
        dst[e] = (uint16_t)f32_to_bf16_bits(v);
      }
    }
  }
}

// The dense GEMM for a checked group: one launch for all of its matrices (their column blocks end to end; EPI_SWIGLU
// the gate / up pair). dg_fits is false when the shape does not take it (then the group kernel runs).
// MX formats load each step's E8M0 bytes as 4-byte aligned dwords of the scale rows: K a multiple of 128 (whole
// dwords per row) and 4-byte aligned scale matrices.
template <int F>
bool dg_fits(int64_t m, int64_t k, const AxkConvEpi* conv, const MxGroup& g) {
  if constexpr (F == axk::WF_BF16) {
    return false;
  } else {
    if (conv != nullptr || m < kDgMinRows || k % kDgBK != 0 || dg_lds_bytes<F>(k) > 160 * 1024) return false;
    if constexpr (axk::is_mx(F)) {
      if (k % 128 != 0) return false;
      for (int i = 0; i < g.count; ++i)
        if (!axk_aligned(g.ws[i], 4)) return false;
    }
    if constexpr (axk::is_nv(F)) {  // each step's scales one aligned dword of the row (K / 16 bytes, K % 64 == 0)
      for (int i = 0; i < g.count; ++i)
        if (!axk_aligned(g.ws[i], 4)) return false;
    }
    return true;
  }
}

template <int F, int EPI>
int dg_launch(const DgArgs& d, hipStream_t st) {
  static AxkOnce lds_once;  // > 64 KiB of dynamic LDS must be allowed once per kernel
  if (const int rc = axk_raise_lds(lds_once, reinterpret_cast<const void*>(&mx_gemm_kernel<F, EPI>), 160 * 1024))
    return rc;
  constexpr int COLS = EPI == EPI_SWIGLU ? kDgBN / 2 : kDgBN;
  const int64_t nb = EPI == EPI_PLAIN ? d.cb0[d.count] : ((int64_t)d.n[0] + COLS - 1) / COLS;
  const int64_t tiles = nb * (((int64_t)d.m + dg_bm<F>() - 1) / dg_bm<F>());
  const int64_t grid = (tiles + kDgXcds - 1) / kDgXcds * kDgXcds;  // whole rounds over the XCDs
  AXK_REQUIRE(grid <= INT32_MAX, AXK_E_SHAPE);
  hipLaunchKernelGGL((mx_gemm_kernel<F, EPI>), dim3((unsigned)grid), dim3(256), dg_lds_bytes<F>(d.k), st, d);
  return axk_launch_status();
}

template <int F>
int dg_group(const uint16_t* a, int64_t lda, const MxGroup& g, int epi, int64_t m, int64_t k, hipStream_t st) {
  DgArgs d{};
  d.a = a;
  d.lda = lda;
  d.count = g.count;
  d.cb0[0] = 0;
  for (int i = 0; i < g.count; ++i) {
    d.w[i] = g.w[i], d.ws[i] = g.ws[i], d.col_scale[i] = g.col_scale[i], d.bias[i] = g.bias[i];
    d.gscale[i] = g.gscale[i];
    d.out[i] = g.out[i], d.ldo[i] = g.ldo[i], d.n[i] = g.n[i];
    d.cb0[i + 1] = d.cb0[i] + (g.n[i] + kDgBN - 1) / kDgBN;
  }
  d.row_scale = g.row_scale;
  d.res = g.res;
  d.ldr = g.ldr;
  d.out_f32 = g.out_f32;
  d.m = (int)m, d.k = (int)k;
  if (epi == EPI_SWIGLU) return dg_launch<F, EPI_SWIGLU>(d, st);
  if (epi == EPI_RES) return dg_launch<F, EPI_RES>(d, st);
  return dg_launch<F, EPI_PLAIN>(d, st);  // every matrix of the group in one launch
}

// Checks a group and launches it. Matrices need whole 128-byte row segments (and 8-byte aligned MXFP4 scale rows).
template <int F>
int mx_group(const uint16_t* a, int64_t lda, const AxkMxMat* mats, int count, int epi, const uint16_t* res,
             int64_t ldr, const float* row_scale, int out_dtype, int64_t m, int64_t k, const AxkConvEpi* conv,
             hipStream_t st) {
  AXK_REQUIRE(a && mats, AXK_E_NULL);
  AXK_REQUIRE(count >= 1 && count <= AXK_MX_GROUP_MAX, AXK_E_SHAPE);
  AXK_REQUIRE(epi == EPI_PLAIN || epi == EPI_SWIGLU || epi == EPI_RES, AXK_E_SHAPE);
  AXK_REQUIRE(epi != EPI_SWIGLU || (count == 2 && mats[0].n == mats[1].n && mats[0].out == mats[1].out), AXK_E_SHAPE);
  AXK_REQUIRE(epi != EPI_RES || (count == 1 && res), AXK_E_NULL);
  AXK_REQUIRE(m >= 0 && k > 0 && m <= INT32_MAX && axk::row_bytes<F>(k) % axk::kSegBytes == 0, AXK_E_SHAPE);
  AXK_REQUIRE(lda >= k && lda % 8 == 0 && axk_aligned(a, 16), AXK_E_ALIGN);
  AXK_REQUIRE(out_dtype == AXK_DT_BF16 || out_dtype == AXK_DT_F32, AXK_E_DTYPE);
  AXK_REQUIRE(epi == EPI_PLAIN || out_dtype == AXK_DT_BF16, AXK_E_DTYPE);
  if (conv) {  // the conv epilogue: matrix 0, plain bf16 outputs, one token per row
    AXK_REQUIRE(conv->w && conv->state_in && conv->state_out, AXK_E_NULL);
    AXK_REQUIRE(epi == EPI_PLAIN && out_dtype == AXK_DT_BF16 && conv->kernel >= 1 && conv->kernel <= kMaxConvTaps,
                AXK_E_SHAPE);
    const size_t sbytes = (size_t)m * (conv->kernel - 1) * mats[0].n * 2;
    AXK_REQUIRE(conv->state_in == conv->state_out || !axk_overlap(conv->state_in, sbytes, conv->state_out, sbytes),
                AXK_E_ALIAS);
  }
  MxGroup g{};
  g.count = count;
  if (conv) {
    g.conv_w = conv->w;
    g.conv_in = conv->state_in;
    g.conv_out = conv->state_out;
    g.conv_k = (int)conv->kernel;
  }
  g.row_scale = row_scale;
  g.res = res;
  g.ldr = ldr;
  g.out_f32 = out_dtype == AXK_DT_F32;
  const size_t esz = out_dtype == AXK_DT_F32 ? 4 : 2;
  const size_t a_bytes = m > 0 ? (size_t)((m - 1) * lda + k) * 2 : 0;
  int64_t tiles = 0;
  for (int i = 0; i < count; ++i) {
    const AxkMxMat& p = mats[i];
    AXK_REQUIRE(p.w && p.out && (!axk::has_block_scales(F) || p.ws) && (!axk::is_nv(F) || p.gscale), AXK_E_NULL);
    AXK_REQUIRE(p.n > 0 && p.n <= INT32_MAX && p.ldo >= p.n, AXK_E_SHAPE);
    AXK_REQUIRE(axk_aligned(p.w, 16) &&
                    (!axk::has_block_scales(F) ||
                     axk_aligned(p.ws, axk::is_nv(F) ? 16 : F == axk::WF_MXFP4 ? 8 : 4)) &&
                    (!axk::is_nv(F) || axk_aligned(p.gscale, 4)),
                AXK_E_ALIGN);
    const size_t o_bytes = m > 0 ? (size_t)((m - 1) * p.ldo + p.n) * esz : 0;
    AXK_REQUIRE(!axk_overlap(p.out, o_bytes, a, a_bytes), AXK_E_ALIAS);
    if (epi == EPI_RES) {  // in place (out == res, one leading dimension) or disjoint
      AXK_REQUIRE(ldr >= p.n, AXK_E_SHAPE);
      const size_t r_bytes = m > 0 ? (size_t)((m - 1) * ldr + p.n) * 2 : 0;
      AXK_REQUIRE((p.out == res && p.ldo == ldr) || !axk_overlap(p.out, o_bytes, res, r_bytes), AXK_E_ALIAS);
    }
    g.w[i] = p.w;
    g.ws[i] = p.ws;
    g.col_scale[i] = p.col_scale;
    g.bias[i] = p.bias;
    g.gscale[i] = p.gscale;
    g.out[i] = p.out;
    g.ldo[i] = p.ldo;
    g.n[i] = (int)p.n;
    g.tile0[i] = (int)tiles;
    tiles += (p.n + 15) / 16;
  }
  AXK_REQUIRE(tiles <= INT32_MAX / 16, AXK_E_SHAPE);
  for (int i = count; i <= AXK_MX_GROUP_MAX; ++i) g.tile0[i] = (int)tiles;
  if (m == 0) return AXK_OK;
  AXK_LAUNCH_GATE();
  if (dg_fits<F>(m, k, conv, g)) return dg_group<F>(a, lda, g, epi, m, k, st);
  if (epi == EPI_SWIGLU) return group_dispatch<F, EPI_SWIGLU>(a, lda, g, m, k, st);
  if (epi == EPI_RES) return group_dispatch<F, EPI_RES>(a, lda, g, m, k, st);
  return group_dispatch<F, EPI_PLAIN>(a, lda, g, m, k, st);
}

template <int F>
int launch_linear(const uint16_t* a, int64_t lda, const uint8_t* w, const uint8_t* ws, const float* row_scale,
                  const float* col_scale, const float* bias, void* out, int out_dtype, int64_t m, int64_t n,
                  int64_t k, axk_stream_t stream, const float* gscale = nullptr) {
  AXK_REQUIRE(a && w && out, AXK_E_NULL);
  AXK_REQUIRE(!axk::has_block_scales(F) || ws, AXK_E_NULL);
  AXK_REQUIRE(!axk::is_nv(F) || gscale, AXK_E_NULL);
  AXK_REQUIRE(m >= 0 && n >= 0 && k > 0 && k % 32 == 0, AXK_E_SHAPE);
  AXK_REQUIRE(m <= INT32_MAX && n <= INT32_MAX, AXK_E_SHAPE);
  AXK_REQUIRE(lda >= k && lda % 8 == 0, AXK_E_ALIGN);
  AXK_REQUIRE(axk_aligned(a, 16) && axk_aligned(w, 16), AXK_E_ALIGN);
  AXK_REQUIRE(out_dtype == AXK_DT_BF16 || out_dtype == AXK_DT_F32, AXK_E_DTYPE);
  if (m == 0 || n == 0) return AXK_OK;
  const size_t out_bytes = (size_t)m * n * (out_dtype == AXK_DT_F32 ? 4 : 2);
  const size_t a_bytes = (size_t)((m - 1) * lda + k) * 2;
  AXK_REQUIRE(!axk_overlap(out, out_bytes, a, a_bytes), AXK_E_ALIAS);

  hipStream_t st = axk_stream(stream);
  // staged group kernel when rows are whole 128-byte segments (and scale rows 8-byte (MXFP4) / 4-byte (MXFP8)
  // aligned)
  if (axk::row_bytes<F>(k) % axk::kSegBytes == 0 &&
      (!axk::has_block_scales(F) || axk_aligned(ws, axk::is_nv(F) ? 16 : F == WF_MXFP4 ? 8 : 4))) {
    const AxkMxMat mat{w, ws, col_scale, bias, out, n, n, gscale};
    return mx_group<F>(a, lda, &mat, 1, EPI_PLAIN, nullptr, 0, row_scale, out_dtype, m, k, nullptr, st);
  }
  constexpr int CH = 4 * WUnit<F>::V;
  const int64_t nc = (k + CH - 1) / CH;  // K chunks
  const int waves = (int)(nc < kMaxWaves ? nc : kMaxWaves);
  const int mt = m <= 16 ? 1 : 2;
  dim3 grid((unsigned)((n + 15) / 16), (unsigned)((m + 16 * mt - 1) / (16 * mt)));
  dim3 block(64 * waves);
  const int of32 = out_dtype == AXK_DT_F32;
  if (mt == 1)
    hipLaunchKernelGGL((mx_linear_kernel<F, 1>), grid, block, 0, st, a, lda, w, ws, row_scale, col_scale, bias, gscale,
                       out, of32, (int)m, (int)n, k);
  else
    hipLaunchKernelGGL((mx_linear_kernel<F, 2>), grid, block, 0, st, a, lda, w, ws, row_scale, col_scale, bias, gscale,
                       out, of32, (int)m, (int)n, k);
  return axk_launch_status();
}

}  // namespace

int axk_mx_group(int fmt, const uint16_t* a, int64_t lda, const AxkMxMat* mats, int count, int epi,
                 const uint16_t* res, int64_t ldr, const float* row_scale, int out_dtype, int64_t m, int64_t k,
                 const AxkConvEpi* conv, hipStream_t stream) {
  if (fmt == AXK_MX_FP8)
    return mx_group<WF_FP8>(a, lda, mats, count, epi, res, ldr, row_scale, out_dtype, m, k, conv, stream);
  if (fmt == AXK_MX_MXFP4)
    return mx_group<WF_MXFP4>(a, lda, mats, count, epi, res, ldr, row_scale, out_dtype, m, k, conv, stream);
  if (fmt == AXK_MX_MXFP8)
    return mx_group<axk::WF_MXFP8>(a, lda, mats, count, epi, res, ldr, row_scale, out_dtype, m, k, conv, stream);
  if (fmt == AXK_MX_NVFP4)
    return mx_group<axk::WF_NVFP4>(a, lda, mats, count, epi, res, ldr, row_scale, out_dtype, m, k, conv, stream);
  return AXK_E_DTYPE;
}

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

extern "C" int axk_nvfp4_gemm(const uint16_t* a, int64_t lda, const uint8_t* b_fp4, const uint8_t* b_scale,
                              const float* b_scale2, const float* bias, void* out, int out_dtype, int64_t m,
                              int64_t n, int64_t k, axk_stream_t stream) {
  AXK_REQUIRE(b_scale2, AXK_E_NULL);
  AXK_REQUIRE(axk_aligned(b_scale2, 4), AXK_E_ALIGN);
  return launch_linear<axk::WF_NVFP4>(a, lda, b_fp4, b_scale, nullptr, nullptr, bias, out, out_dtype, m, n, k, stream,
                                      b_scale2);
}

extern "C" int axk_fp8_gemm(const uint16_t* a, int64_t lda, const uint8_t* b_fp8, const float* scale_a,
                            const float* scale_b, const float* bias, void* out, int out_dtype, int64_t m, int64_t n,
                            int64_t k, axk_stream_t stream) {
  AXK_REQUIRE(scale_b, AXK_E_NULL);
  return launch_linear<WF_FP8>(a, lda, b_fp8, nullptr, scale_a, scale_b, bias, out, out_dtype, m, n, k, stream);
}

extern "C" int axk_mxfp8_gemm(const uint16_t* a, int64_t lda, const uint8_t* b_fp8, const uint8_t* b_scale,
                              int fp8_dtype, const float* bias, void* out, int out_dtype, int64_t m, int64_t n,
                              int64_t k, axk_stream_t stream) {
  if (fp8_dtype == AXK_DT_FP8E4M3)
    return launch_linear<axk::WF_MXFP8>(a, lda, b_fp8, b_scale, nullptr, nullptr, bias, out, out_dtype, m, n, k,
                                        stream);
  if (fp8_dtype == AXK_DT_FP8E5M2)
    return launch_linear<axk::WF_MXBF8>(a, lda, b_fp8, b_scale, nullptr, nullptr, bias, out, out_dtype, m, n, k,
                                        stream);
  return AXK_E_DTYPE;
}

extern "C" int axk_bf16_gemm(const uint16_t* a, int64_t lda, const uint16_t* b, const float* bias, void* out,
                             int out_dtype, int64_t m, int64_t n, int64_t k, axk_stream_t stream) {
  return launch_linear<WF_BF16>(a, lda, reinterpret_cast<const uint8_t*>(b), nullptr, nullptr, nullptr, bias, out,
                                out_dtype, m, n, k, stream);
}
