// Per-layer glue of the Qwen3.5 hybrid decode layer for gfx950: RMSNorm (plain, fused with the residual add,
// gated by silu(z)), the stateful causal depthwise conv1d + SiLU, q / k RMSNorm with partial NeoX RoPE, and the
// elementwise gates. Semantics (models/qwen35_35b_a3b/src/70b0fbc/q35_step.py):
//   rmsnorm(x, w)  = x * rsqrt(mean(x^2) + eps) * w  in fp32, bf16 out; layer / q / k norms take w = 1 + weight
//                    as the reference's runtime input (one_plus, q35_step.py:346-348)
//   gdn core norm  = bf16(rmsnorm(core, norm_w)) * silu(z), fp32 activation, bf16 out (q35_step.py:179-181)
//   conv1d + SiLU  = per channel sum over the kernel window of x_{t-j} w[c, j] (column 0 multiplies the current
//                    token, gdn_args q35_step.py:365-368), accumulated tap by tap from the current token backwards
//                    with a bf16 rounding after each tap, then silu in fp32 (the golden
//                    causal_conv1d_silu_reference, models/qwen35_35b_a3b/sgl/tests/test_gdn_attn.py:241-256);
//                    the state holds the last kernel - 1 inputs, oldest first
//   rope           = NeoX halves of the first `rot` channels: y_i = x_i cos_i - x_{i+h} sin_i,
//                    y_{i+h} = x_{i+h} cos_i + x_i sin_i, h = rot / 2, on the bf16 normalised q / k
//                    (attn_block q35_step.py:191-197; models/qwen38_27b/mtp/mtp_ref.py:176-187)
//   sigmoid gate   = bf16(attn * sigmoid(gate)); MLP = bf16(silu(g) * u); residual = bf16(x + y)
//                    (q35_step.py:136-139, 276-279)
// All are bandwidth- or latency-bound row operations: one wave per row for the norms (4 rows per workgroup),
// 16-byte vector loads and stores, fp32 arithmetic.
#include "axk_common.h"
#include "axk_host.h"

namespace {

constexpr int kRowsPerWg = 4;
constexpr int kMaxConvKernel = kMaxConvTaps;
constexpr int kMaxRopeDim = 512;

AXK_DEV void unpack8(const uint4& v, float (&f)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

AXK_DEV uint4 pack8(const float (&f)[8]) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7]));
}

// MODE 0: out = rmsnorm(x) w.  MODE 1: s = bf16(x + y) -> sum_out, out = rmsnorm(s) w.
// MODE 2: out = bf16(bf16(rmsnorm(x) w) * silu(z)).  One wave per row; lane c takes 8-element chunks c, c + 64, ...
template <int MODE>
__global__ __launch_bounds__(64 * kRowsPerWg) void rmsnorm_rows_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                       const uint16_t* __restrict__ y,
                                                                       const float* __restrict__ w,
                                                                       const uint16_t* __restrict__ z,
                                                                       uint16_t* sum_out, uint16_t* __restrict__ out,
                                                                       int64_t ldo, int64_t rows, int n, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerWg + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nch = n >> 3;
  const uint16_t* xr = x + row * ldx;
  float ss = 0.f;
  for (int c = lane; c < nch; c += 64) {
    float f[8];
    unpack8(*reinterpret_cast<const uint4*>(xr + 8 * c), f);
    if (MODE == 1) {
      float g[8];
      unpack8(*reinterpret_cast<const uint4*>(y + row * n + 8 * c), g);
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = round_bf16(f[i] + g[i]);
      *reinterpret_cast<uint4*>(sum_out + row * n + 8 * c) = pack8(f);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += f[i] * f[i];
  }
  const float inv = rsqrtf(wave_sum(ss) / (float)n + eps);
  // second pass: the row again (the sum as this lane wrote it)
  const uint16_t* src = MODE == 1 ? sum_out + row * n : xr;
  for (int c = lane; c < nch; c += 64) {
    float f[8];
    unpack8(*reinterpret_cast<const uint4*>(src + 8 * c), f);
    const float4 w0 = *reinterpret_cast<const float4*>(w + 8 * c), w1 = *reinterpret_cast<const float4*>(w + 8 * c + 4);
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = f[i] * inv * wv[i];
    if (MODE == 2) {
      float g[8];
      unpack8(*reinterpret_cast<const uint4*>(z + row * n + 8 * c), g);
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = round_bf16(f[i]) * silu_f32(g[i]);
    }
    *reinterpret_cast<uint4*>(out + row * ldo + 8 * c) = pack8(f);
  }
}

// Register-resident variant for n <= 8192: TPR threads per row (16 or 32: a lane group of a wave, 64: a wave, 256: the
// workgroup), each holding CPT 8-element chunks (c = rank + TPR i); every load of the row (x, y, z, w) is issued
// before the reduction, so a row costs one memory round trip. Same rounding points as rmsnorm_rows_kernel.
template <int MODE, int TPR, int CPT>
__global__ __launch_bounds__(256) void rmsnorm_reg_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                          const uint16_t* __restrict__ y, const float* __restrict__ w,
                                                          const uint16_t* __restrict__ z, uint16_t* sum_out,
                                                          uint16_t* __restrict__ out, int64_t ldo, int64_t rows, int n,
                                                          float eps) {
  __shared__ float part[256 / 64];
  const int rank = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * (256 / TPR) + threadIdx.x / TPR;
  if (TPR <= 64 && row >= rows) return;  // whole lane groups; TPR == 256 rows are always in range (grid = rows)
  const int nch = n >> 3;
  float f[CPT][8], wv[CPT][8], zv[CPT][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = rank + TPR * i;
    if (c < nch) {
      unpack8(*reinterpret_cast<const uint4*>(x + row * ldx + 8 * c), f[i]);
      const float4 w0 = *reinterpret_cast<const float4*>(w + 8 * c), w1 = *reinterpret_cast<const float4*>(w + 8 * c + 4);
      wv[i][0] = w0.x; wv[i][1] = w0.y; wv[i][2] = w0.z; wv[i][3] = w0.w;
      wv[i][4] = w1.x; wv[i][5] = w1.y; wv[i][6] = w1.z; wv[i][7] = w1.w;
      if (MODE == 1) {
        float g[8];
        unpack8(*reinterpret_cast<const uint4*>(y + row * n + 8 * c), g);
#pragma unroll
        for (int k = 0; k < 8; ++k) f[i][k] = round_bf16(f[i][k] + g[k]);
        *reinterpret_cast<uint4*>(sum_out + row * n + 8 * c) = pack8(f[i]);
      }
      if (MODE == 2) unpack8(*reinterpret_cast<const uint4*>(z + row * n + 8 * c), zv[i]);
#pragma unroll
      for (int k = 0; k < 8; ++k) ss += f[i][k] * f[i][k];
    }
  }
  if constexpr (TPR < 64) {  // the row's lane group (aligned, whole: it returned or stayed together)
#pragma unroll
    for (int o = TPR / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  } else {
    ss = wave_sum(ss);
  }
  if (TPR == 256) {
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (part[0] + part[1]) + (part[2] + part[3]);
  }
  const float inv = rsqrtf(ss / (float)n + eps);
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = rank + TPR * i;
    if (c < nch) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        f[i][k] = f[i][k] * inv * wv[i][k];
        if (MODE == 2) f[i][k] = round_bf16(f[i][k]) * silu_f32(zv[i][k]);
      }
      *reinterpret_cast<uint4*>(out + row * ldo + 8 * c) = pack8(f[i]);
    }
  }
}

// Thread = (sequence b, 8 channels, a tile of kConvTile tokens): the K - 1 inputs before the tile (conv-state rows or
// x rows) and the tile's rows loaded into registers up front, then the tile's tokens in order; 16-byte loads and
// stores along the channels. The conv state after the last token (the last K - 1 rows of [state_in | x]) is written
// by one thread per (sequence, channels): with one tile, from its registers at the end; with more (then T > K - 1
// and those rows are all x rows), by the tile-0 thread, the only one that reads state_in, after its own reads, so
// an in-place state is read before it is overwritten.
constexpr int kConvTile = 8;
template <int K>
__global__ __launch_bounds__(256) void conv1d_silu_tiled_kernel(const uint16_t* __restrict__ x,
                                                                const uint16_t* __restrict__ w,
                                                                const uint16_t* state_in, uint16_t* state_out,
                                                                uint16_t* __restrict__ out, int B, int T, int C) {
  const int c8 = C / 8, tiles = (T + kConvTile - 1) / kConvTile;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)B * tiles * c8) return;
  const int cg = (int)(i % c8);
  const int64_t rest = i / c8;
  const int tile = (int)(rest % tiles), b = (int)(rest / tiles);
  const int c0 = 8 * cg, t0 = tile * kConvTile, t1 = min(T, t0 + kConvTile);
  float wk[8][kMaxConvKernel], hist[8][kMaxConvKernel];
#pragma unroll
  for (int q = 0; q < 8; ++q)
#pragma unroll
    for (int j = 0; j < kMaxConvKernel; ++j) {
      wk[q][j] = j < K ? bf16_bits_to_f32(w[(int64_t)(c0 + q) * K + j]) : 0.f;
      hist[q][j] = 0.f;
    }
#pragma unroll
  for (int j = 0; j < kMaxConvKernel; ++j) {  // input rows t0 - (K - 1) .. t0 - 1, oldest first
    if (j < K - 1) {
      const int r = t0 - (K - 1) + j;
      const uint16_t* src = r < 0 ? state_in + ((int64_t)b * (K - 1) + (K - 1) + r) * C
                                  : x + ((int64_t)b * T + r) * C;
      float f[8];
      unpack8(*reinterpret_cast<const uint4*>(src + c0), f);
#pragma unroll
      for (int q = 0; q < 8; ++q) hist[q][j] = f[q];
    }
  }
  uint4 rows[kConvTile];  // the tile's input rows, all loads in flight together
#pragma unroll
  for (int u = 0; u < kConvTile; ++u)
    if (t0 + u < t1) rows[u] = *reinterpret_cast<const uint4*>(x + ((int64_t)b * T + t0 + u) * C + c0);
#pragma unroll
  for (int u = 0; u < kConvTile; ++u) {
    if (t0 + u < t1) {
      const int64_t o = ((int64_t)b * T + t0 + u) * C + c0;
      float xt[8], y[8];
      unpack8(rows[u], xt);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        // tap j multiplies x_{t-j}: j = 0 the current token, then back through the history (a bf16 rounding per tap)
        y[q] = silu_f32(conv_taps(xt[q], wk[q], hist[q], K));
#pragma unroll
        for (int j = 0; j + 1 < kMaxConvKernel; ++j)
          if (j + 1 < K - 1) hist[q][j] = hist[q][j + 1];
        if (K > 1) hist[q][K - 2] = xt[q];
      }
      *reinterpret_cast<uint4*>(out + o) = pack8(y);
    }
  }
  if (K > 1 && tiles == 1) {
#pragma unroll
    for (int j = 0; j < kMaxConvKernel; ++j)
      if (j < K - 1) {
        float f[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) f[q] = hist[q][j];
        *reinterpret_cast<uint4*>(state_out + ((int64_t)b * (K - 1) + j) * C + c0) = pack8(f);
      }
  } else if (K > 1 && tile == 0) {
#pragma unroll
    for (int j = 0; j < kMaxConvKernel; ++j)
      if (j < K - 1)
        *reinterpret_cast<uint4*>(state_out + ((int64_t)b * (K - 1) + j) * C + c0) =
            *reinterpret_cast<const uint4*>(x + ((int64_t)b * T + T - (K - 1) + j) * C + c0);
  }
}

// One thread per (sequence, channel): the window slides over the tokens; history in registers (channel counts that
// are not a multiple of 8, or rows not 16-byte aligned).
__global__ __launch_bounds__(256) void conv1d_silu_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ w,
                                                          const uint16_t* state_in, uint16_t* state_out,
                                                          uint16_t* __restrict__ out, int B, int T, int C, int K) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)B * C) return;
  const int b = (int)(i / C), c = (int)(i - (int64_t)b * C);
  float wk[kMaxConvKernel], hist[kMaxConvKernel];  // hist[0 .. K-2]: the K - 1 previous inputs, oldest first
#pragma unroll
  for (int j = 0; j < kMaxConvKernel; ++j) {
    wk[j] = j < K ? bf16_bits_to_f32(w[(int64_t)c * K + j]) : 0.f;
    hist[j] = j < K - 1 ? bf16_bits_to_f32(state_in[((int64_t)b * (K - 1) + j) * C + c]) : 0.f;
  }
  for (int t = 0; t < T; ++t) {
    const int64_t o = ((int64_t)b * T + t) * C + c;
    const float xt = bf16_bits_to_f32(x[o]);
    // tap j multiplies x_{t-j}: j = 0 the current token, then back through the history (a bf16 rounding per tap)
    out[o] = (uint16_t)f32_to_bf16_bits(silu_f32(conv_taps(xt, wk, hist, K)));
#pragma unroll
    for (int j = 0; j + 1 < kMaxConvKernel; ++j)
      if (j + 1 < K - 1) hist[j] = hist[j + 1];
    if (K > 1) hist[K - 2] = xt;
  }
#pragma unroll
  for (int j = 0; j < kMaxConvKernel; ++j)
    if (j < K - 1) state_out[((int64_t)b * (K - 1) + j) * C + c] = (uint16_t)f32_to_bf16_bits(hist[j]);
}

// One wave, one row of D = 64 EPL values (lane l: channels EPL l .. EPL l + EPL - 1): RMSNorm to bf16, then NeoX
// RoPE on the first rot channels with the row's cos / sin (channel e pairs with e + rot / 2); with norm == false
// the row is copied. The wave must be whole (the norm and the rotation exchange values across lanes).
template <int EPL>
AXK_DEV void norm_rope_row(const uint16_t* __restrict__ xr, const float* __restrict__ w,
                           const uint16_t* __restrict__ cosr, const uint16_t* __restrict__ sinr, uint16_t* orow,
                           int rot, float eps, bool norm) {
  constexpr int D = 64 * EPL;
  const int lane = threadIdx.x & 63;
  float v[EPL];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    v[j] = bf16_bits_to_f32(xr[EPL * lane + j]);
    ss += v[j] * v[j];
  }
  if (norm) {
    const float inv = rsqrtf(wave_sum(ss) / (float)D + eps);
#pragma unroll
    for (int j = 0; j < EPL; ++j) v[j] = round_bf16(v[j] * inv * w[EPL * lane + j]);
  }
  const int half = rot >> 1, lofs = half / EPL;  // partner lane offset (half % EPL == 0)
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = EPL * lane + j;
    const bool low = e < half;
    const int plane = low ? lane + lofs : lane - lofs;
    const float pv = __shfl(v[j], (plane >= 0 && plane < 64) ? plane : lane, 64);
    float r = v[j];
    if (norm && e < rot) {
      const int ci = low ? e : e - half;
      const float cs = bf16_bits_to_f32(cosr[ci]), sn = bf16_bits_to_f32(sinr[ci]);
      r = low ? v[j] * cs - pv * sn : v[j] * cs + pv * sn;
    }
    orow[e] = (uint16_t)f32_to_bf16_bits(r);
  }
}

// One wave per (sequence, head) row: norm_rope_row over x rows ldx apart, into contiguous out rows.
template <int EPL>
__global__ __launch_bounds__(64 * kRowsPerWg) void qk_norm_rope_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                       const float* __restrict__ w,
                                                                       const uint16_t* __restrict__ cosv,
                                                                       const uint16_t* __restrict__ sinv,
                                                                       uint16_t* __restrict__ out, int64_t rows,
                                                                       int heads, int rot, float eps) {
  constexpr int D = 64 * EPL;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerWg + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t b = row / heads;
  const int half = rot >> 1;
  norm_rope_row<EPL>(x + row * ldx, w, cosv + b * half, sinv + b * half, out + row * D, rot, eps, true);
}

// The attention layer's q / k / v preparation in one launch, one wave per row of the rows b (HQ + 2 HKV) + r:
// r < HQ: q head r of the [q | gate] projection rows (2D apart) -> norm (q_norm) + RoPE -> q_out [B, HQ, D];
// HQ <= r < HQ + HKV: k head -> norm (k_norm) + RoPE -> the K plane of the paged cache at loc[b] = (page, slot);
// the last HKV rows: v head -> the V plane (store_paged_kv; a location outside the cache writes nothing).
template <int EPL>
__global__ __launch_bounds__(64 * kRowsPerWg) void attn_prep_kernel(
    const uint16_t* __restrict__ qg, const uint16_t* __restrict__ kk, const uint16_t* __restrict__ vv,
    const float* __restrict__ q_norm, const float* __restrict__ k_norm, const uint16_t* __restrict__ cosv,
    const uint16_t* __restrict__ sinv, uint16_t* __restrict__ q_out, uint16_t* __restrict__ cache,
    const int* __restrict__ loc, int batch, int hq, int hkv, int rot, int page_size, int64_t num_pages, float eps) {
  constexpr int D = 64 * EPL;
  const int per = hq + 2 * hkv;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerWg + (threadIdx.x >> 6);
  if (row >= (int64_t)batch * per) return;
  const int b = (int)(row / per), r = (int)(row - (int64_t)b * per);
  const int half = rot >> 1;
  const uint16_t *cr = cosv + (int64_t)b * half, *sr = sinv + (int64_t)b * half;
  if (r < hq) {
    norm_rope_row<EPL>(qg + ((int64_t)b * hq + r) * 2 * D, q_norm, cr, sr, q_out + ((int64_t)b * hq + r) * D, rot,
                       eps, true);
    return;
  }
  const int plane = r >= hq + hkv, kvh = r - hq - plane * hkv;
  const int page = loc[2 * b], off = loc[2 * b + 1];
  if (page < 0 || page >= num_pages || off < 0 || off >= page_size) return;
  uint16_t* dst = cache + ((((int64_t)page * 2 + plane) * page_size + off) * hkv + kvh) * D;
  const uint16_t* src = (plane ? vv : kk) + ((int64_t)b * hkv + kvh) * D;
  norm_rope_row<EPL>(src, k_norm, cr, sr, dst, rot, eps, !plane);
}

// Elementwise over rows x n (n % 8 == 0): OP 0 bf16(x * sigmoid(g)), OP 1 bf16(silu(x) * g), OP 2 bf16(x + g).
// g rows are ldg elements apart (the attention gate sits inside the q projection's rows).
template <int OP>
__global__ __launch_bounds__(256) void eltwise_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ g,
                                                      int64_t ldg, uint16_t* __restrict__ out, int64_t rows, int n) {
  const int nch = n >> 3;
  const int64_t total = rows * nch;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / nch, c = i - r * nch;
    float a[8], b[8];
    unpack8(*reinterpret_cast<const uint4*>(x + r * n + 8 * c), a);
    unpack8(*reinterpret_cast<const uint4*>(g + r * ldg + 8 * c), b);
#pragma unroll
    for (int k = 0; k < 8; ++k) a[k] = OP == 0 ? a[k] * sigmoid_f32(b[k]) : (OP == 1 ? silu_f32(a[k]) * b[k] : a[k] + b[k]);
    *reinterpret_cast<uint4*>(out + r * n + 8 * c) = pack8(a);
  }
}

unsigned row_grid(int64_t rows) { return (unsigned)((rows + kRowsPerWg - 1) / kRowsPerWg); }

unsigned elt_grid(int64_t work) {
  const int64_t g = (work + 255) / 256;
  return (unsigned)(g < 65536 ? (g > 0 ? g : 1) : 65536);
}

// Launches the register-resident kernel when the row fits (n <= 8192), else the looping one.
template <int MODE>
void launch_rmsnorm(const uint16_t* x, int64_t ldx, const uint16_t* y, const float* w, const uint16_t* z,
                    uint16_t* sum_out, uint16_t* out, int64_t ldo, int64_t rows, int n, float eps, hipStream_t st) {
  const int nch = n >> 3;
#define AXK_RMS(TPR, CPT)                                                                                          \
  hipLaunchKernelGGL((rmsnorm_reg_kernel<MODE, TPR, CPT>), dim3((unsigned)((rows + 256 / TPR - 1) / (256 / TPR))), \
                     dim3(256), 0, st, x, ldx, y, w, z, sum_out, out, ldo, rows, n, eps)
  if (nch <= 16) AXK_RMS(16, 1);  // a head's row (128 values): 4 rows per wave
  else if (nch <= 32) AXK_RMS(32, 1);
  else if (nch <= 64) AXK_RMS(64, 1);
  else if (nch <= 128) AXK_RMS(64, 2);
  else if (nch <= 256) AXK_RMS(256, 1);
  else if (nch <= 512) AXK_RMS(256, 2);
  else if (nch <= 768) AXK_RMS(256, 3);
  else if (nch <= 1024) AXK_RMS(256, 4);
  else
    hipLaunchKernelGGL(rmsnorm_rows_kernel<MODE>, dim3(row_grid(rows)), dim3(64 * kRowsPerWg), 0, st, x, ldx, y, w, z,
                       sum_out, out, ldo, rows, n, eps);
#undef AXK_RMS
}

bool aligned16(const void* p) { return axk_aligned(p, 16); }

}  // namespace

extern "C" int axk_rmsnorm(const uint16_t* x, int64_t ldx, const float* w, uint16_t* out, int64_t ldo, int64_t rows,
                           int64_t n, float eps, axk_stream_t stream) {
  AXK_REQUIRE(x && w && out, AXK_E_NULL);
  AXK_REQUIRE(rows > 0 && n > 0 && n % 8 == 0 && n <= INT32_MAX && ldx >= n && ldo >= n, AXK_E_SHAPE);
  AXK_REQUIRE(ldx % 8 == 0 && ldo % 8 == 0 && aligned16(x) && aligned16(w) && aligned16(out), AXK_E_ALIGN);
  AXK_LAUNCH_GATE();
  launch_rmsnorm<0>(x, ldx, nullptr, w, nullptr, nullptr, out, ldo, rows, (int)n, eps, axk_stream(stream));
  return axk_launch_status();
}

extern "C" int axk_add_rmsnorm(const uint16_t* x, const uint16_t* y, const float* w, uint16_t* sum_out,
                               uint16_t* norm_out, int64_t rows, int64_t n, float eps, axk_stream_t stream) {
  AXK_REQUIRE(x && y && w && sum_out && norm_out, AXK_E_NULL);
  AXK_REQUIRE(rows > 0 && n > 0 && n % 8 == 0 && n <= INT32_MAX, AXK_E_SHAPE);
  AXK_REQUIRE(aligned16(x) && aligned16(y) && aligned16(w) && aligned16(sum_out) && aligned16(norm_out), AXK_E_ALIGN);
  const size_t bytes = (size_t)rows * n * 2;
  AXK_REQUIRE(!axk_overlap(norm_out, bytes, sum_out, bytes) && !axk_overlap(norm_out, bytes, x, bytes) &&
                  !axk_overlap(norm_out, bytes, y, bytes),
              AXK_E_ALIAS);
  AXK_LAUNCH_GATE();
  launch_rmsnorm<1>(x, n, y, w, nullptr, sum_out, norm_out, n, rows, (int)n, eps, axk_stream(stream));
  return axk_launch_status();
}

extern "C" int axk_gated_rmsnorm_silu(const uint16_t* x, const float* w, const uint16_t* z, uint16_t* out,
                                      int64_t rows, int64_t n, float eps, axk_stream_t stream) {
  AXK_REQUIRE(x && w && z && out, AXK_E_NULL);
  AXK_REQUIRE(rows > 0 && n > 0 && n % 8 == 0 && n <= INT32_MAX, AXK_E_SHAPE);
  AXK_REQUIRE(aligned16(x) && aligned16(w) && aligned16(z) && aligned16(out), AXK_E_ALIGN);
  AXK_LAUNCH_GATE();
  launch_rmsnorm<2>(x, n, nullptr, w, z, nullptr, out, n, rows, (int)n, eps, axk_stream(stream));
  return axk_launch_status();
}

extern "C" int axk_causal_conv1d_silu(const uint16_t* x, const uint16_t* w, const uint16_t* state_in,
                                      uint16_t* state_out, uint16_t* out, int64_t batch, int64_t tokens,
                                      int64_t channels, int64_t kernel, axk_stream_t stream) {
  AXK_REQUIRE(x && w && out && (kernel == 1 || (state_in && state_out)), AXK_E_NULL);
  AXK_REQUIRE(batch > 0 && tokens > 0 && channels > 0 && kernel >= 1 && kernel <= kMaxConvKernel, AXK_E_SHAPE);
  AXK_REQUIRE(batch * channels <= INT32_MAX && tokens <= INT32_MAX, AXK_E_SHAPE);
  const size_t sbytes = (size_t)batch * (kernel - 1) * channels * 2, obytes = (size_t)batch * tokens * channels * 2;
  // in place state is allowed (each thread reads its history before writing it); the output may not overlap it
  AXK_REQUIRE(kernel == 1 || state_in == state_out || !axk_overlap(state_in, sbytes, state_out, sbytes), AXK_E_ALIAS);
  AXK_REQUIRE(kernel == 1 || !axk_overlap(out, obytes, state_out, sbytes), AXK_E_ALIAS);
  AXK_LAUNCH_GATE();
  if (channels % 8 == 0 && aligned16(x) && aligned16(out) &&
      (kernel == 1 || (aligned16(state_in) && aligned16(state_out)))) {
    const int64_t n = batch * ((tokens + kConvTile - 1) / kConvTile) * (channels / 8);
    const dim3 grid((unsigned)((n + 255) / 256));
    const hipStream_t st = axk_stream(stream);
    const int Bi = (int)batch, Ti = (int)tokens, Ci = (int)channels;
    switch (kernel) {  // the tap count is a template argument: every register index is then constant
#define AXK_CONV_CASE(KK)                                                                                          \
  case KK:                                                                                                         \
    hipLaunchKernelGGL(conv1d_silu_tiled_kernel<KK>, grid, dim3(256), 0, st, x, w, state_in, state_out, out, Bi, Ti, \
                       Ci);                                                                                        \
    break;
      AXK_CONV_CASE(1) AXK_CONV_CASE(2) AXK_CONV_CASE(3) AXK_CONV_CASE(4)
      AXK_CONV_CASE(5) AXK_CONV_CASE(6) AXK_CONV_CASE(7) AXK_CONV_CASE(8)
#undef AXK_CONV_CASE
    }
  } else {
    const int64_t n = batch * channels;
    hipLaunchKernelGGL(conv1d_silu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, axk_stream(stream), x,
                       w, state_in, state_out, out, (int)batch, (int)tokens, (int)channels, (int)kernel);
  }
  return axk_launch_status();
}

namespace {
// Thread = (snapshot t, sequence b, row i, 8 channels).
__global__ __launch_bounds__(256) void conv_snapshots_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ state_in,
                                                             uint16_t* __restrict__ snap, int64_t snap_ld, int B, int T,
                                                             int C, int K) {
  const int c8 = C / 8;
  const int64_t n = (int64_t)T * B * (K - 1) * c8;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int cc = (int)(e % c8);
    int64_t r = e / c8;
    const int i = (int)(r % (K - 1));
    r /= K - 1;
    const int b = (int)(r % B), t = (int)(r / B);
    const int src = t + 1 + i;  // row of [state_in (K - 1 rows) | x rows]
    const uint16_t* from = src < K - 1 ? state_in + ((int64_t)b * (K - 1) + src) * C
                                       : x + ((int64_t)b * T + (src - (K - 1))) * C;
    *reinterpret_cast<uint4*>(snap + t * snap_ld + ((int64_t)b * (K - 1) + i) * C + 8 * cc) =
        *reinterpret_cast<const uint4*>(from + 8 * cc);
  }
}

__global__ __launch_bounds__(256) void fill_iota_kernel(int32_t* out, int n, int step) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i <= n) out[i] = i * step;
}
}  // namespace

int axk_conv_snapshots(const uint16_t* x, const uint16_t* state_in, uint16_t* snap, int64_t snap_ld, int64_t batch,
                       int64_t tokens, int64_t channels, int64_t kernel, hipStream_t stream) {
  AXK_REQUIRE(x && state_in && snap, AXK_E_NULL);
  AXK_REQUIRE(batch > 0 && tokens > 0 && kernel >= 2 && kernel <= kMaxConvKernel && channels % 8 == 0, AXK_E_SHAPE);
  AXK_REQUIRE(snap_ld >= batch * (kernel - 1) * channels && snap_ld % 8 == 0, AXK_E_SHAPE);
  AXK_REQUIRE(axk_aligned(x, 16) && axk_aligned(state_in, 16) && axk_aligned(snap, 16), AXK_E_ALIGN);
  AXK_REQUIRE(batch * tokens <= INT32_MAX, AXK_E_SHAPE);
  const int64_t n = tokens * batch * (kernel - 1) * (channels / 8);
  const int64_t grid = (n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096;
  AXK_LAUNCH_GATE();
  hipLaunchKernelGGL(conv_snapshots_kernel, dim3((unsigned)grid), dim3(256), 0, stream, x, state_in, snap, snap_ld,
                     (int)batch, (int)tokens, (int)channels, (int)kernel);
  return axk_launch_status();
}

int axk_fill_iota_i32(int32_t* out, int64_t n, int64_t step, hipStream_t stream) {
  AXK_REQUIRE(out, AXK_E_NULL);
  AXK_REQUIRE(n >= 0 && n < INT32_MAX && step >= 0 && n * step <= INT32_MAX, AXK_E_SHAPE);
  AXK_LAUNCH_GATE();
  hipLaunchKernelGGL(fill_iota_kernel, dim3((unsigned)(n / 256 + 1)), dim3(256), 0, stream, out, (int)n, (int)step);
  return axk_launch_status();
}

extern "C" int axk_qk_norm_rope(const uint16_t* x, int64_t ldx, const float* w, const uint16_t* cos,
                                const uint16_t* sin, uint16_t* out, int64_t batch, int64_t heads, int64_t head_dim,
                                int64_t rot, float eps, axk_stream_t stream) {
  AXK_REQUIRE(x && w && out && (rot == 0 || (cos && sin)), AXK_E_NULL);
  AXK_REQUIRE(batch > 0 && heads > 0 && ldx >= head_dim, AXK_E_SHAPE);
  AXK_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == kMaxRopeDim, AXK_E_SHAPE);
  const int64_t epl = head_dim / 64;
  AXK_REQUIRE(rot >= 0 && rot <= head_dim && rot % 2 == 0 && (rot / 2) % epl == 0, AXK_E_SHAPE);
  const int64_t rows = batch * heads;
  const size_t obytes = (size_t)rows * head_dim * 2;
  AXK_REQUIRE(!axk_overlap(out, obytes, x, (size_t)((rows - 1) * ldx + head_dim) * 2), AXK_E_ALIAS);
  hipStream_t st = axk_stream(stream);
  AXK_LAUNCH_GATE();
#define AXK_QKR(E)                                                                                                 \
  hipLaunchKernelGGL(qk_norm_rope_kernel<E>, dim3(row_grid(rows)), dim3(64 * kRowsPerWg), 0, st, x, ldx, w, cos, sin, \
                     out, rows, (int)heads, (int)rot, eps)
  if (epl == 1) AXK_QKR(1);
  else if (epl == 2) AXK_QKR(2);
  else if (epl == 4) AXK_QKR(4);
  else AXK_QKR(8);
#undef AXK_QKR
  return axk_launch_status();
}

namespace {
template <int OP>
int launch_eltwise(const uint16_t* x, const uint16_t* g, int64_t ldg, uint16_t* out, int64_t rows, int64_t n,
                   axk_stream_t stream) {
  AXK_REQUIRE(x && g && out, AXK_E_NULL);
  AXK_REQUIRE(rows > 0 && n > 0 && n % 8 == 0 && ldg >= n && n <= INT32_MAX, AXK_E_SHAPE);
  AXK_REQUIRE(ldg % 8 == 0 && aligned16(x) && aligned16(g) && aligned16(out), AXK_E_ALIGN);
  AXK_LAUNCH_GATE();
  hipLaunchKernelGGL(eltwise_kernel<OP>, dim3(elt_grid(rows * (n / 8))), dim3(256), 0, axk_stream(stream), x, g, ldg,
                     out, rows, (int)n);
  return axk_launch_status();
}
}  // namespace

extern "C" int axk_sigmoid_mul(const uint16_t* x, const uint16_t* gate, int64_t ldg, uint16_t* out, int64_t rows,
                               int64_t n, axk_stream_t stream) {
  return launch_eltwise<0>(x, gate, ldg, out, rows, n, stream);
}

extern "C" int axk_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* out, int64_t rows, int64_t n,
                            axk_stream_t stream) {
  return launch_eltwise<1>(g, u, n, out, rows, n, stream);
}

extern "C" int axk_add(const uint16_t* x, const uint16_t* y, uint16_t* out, int64_t rows, int64_t n,
                       axk_stream_t stream) {
  return launch_eltwise<2>(x, y, n, out, rows, n, stream);
}

int axk_attn_qkv_prep(const uint16_t* qg, const uint16_t* kk, const uint16_t* vv, const float* q_norm,
                      const float* k_norm, const uint16_t* cos, const uint16_t* sin, uint16_t* q_out,
                      uint16_t* kv_cache, const int32_t* cache_location, int64_t batch, int64_t hq, int64_t hkv,
                      int64_t head_dim, int64_t rot, int64_t page_size, int64_t num_pages, float eps,
                      hipStream_t stream) {
  AXK_REQUIRE(qg && kk && vv && q_norm && k_norm && q_out && kv_cache && cache_location && (rot == 0 || (cos && sin)),
              AXK_E_NULL);
  AXK_REQUIRE(batch > 0 && hq > 0 && hkv > 0 && page_size > 0 && num_pages > 0, AXK_E_SHAPE);
  AXK_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == kMaxRopeDim, AXK_E_SHAPE);
  const int64_t epl = head_dim / 64;
  AXK_REQUIRE(rot >= 0 && rot <= head_dim && rot % 2 == 0 && (rot / 2) % epl == 0, AXK_E_SHAPE);
  const int64_t rows = batch * (hq + 2 * hkv);
  AXK_REQUIRE(rows <= INT32_MAX, AXK_E_SHAPE);
  AXK_LAUNCH_GATE();
#define AXK_PREP(E)                                                                                             \
  hipLaunchKernelGGL(attn_prep_kernel<E>, dim3(row_grid(rows)), dim3(64 * kRowsPerWg), 0, stream, qg, kk, vv,  \
                     q_norm, k_norm, cos, sin, q_out, kv_cache, cache_location, (int)batch, (int)hq, (int)hkv, \
                     (int)rot, (int)page_size, num_pages, eps)
  if (epl == 1) AXK_PREP(1);
  else if (epl == 2) AXK_PREP(2);
  else if (epl == 4) AXK_PREP(4);
  else AXK_PREP(8);
#undef AXK_PREP
  return axk_launch_status();
}
