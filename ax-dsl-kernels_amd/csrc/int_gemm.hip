// Integer-weight GEMMs for gfx950: the int8_gemm and int4_gemm of sgl_kernel_axera/gemm.py (479-492, 662-677).
//
// axk_int8_gemm: out = (a_int8 * scale_a[:, None]) @ (b_int8 * scale_b[:, None])^T + bias (_scaled_gemm, 119-181),
// int8 activations and weights. The products are exact in int32 on v_mfma_i32_16x16x64_i8 (64 int8 products per
// lane step, no rounding), and the two scales and the bias are applied once to each int32 sum in fp32, rounding once
// to the output dtype. (The reference first scales both operands into the output dtype, then runs an fp32 matmul:
// for fp32 outputs the two differ by fp32 rounding only, for bf16 outputs this form also skips the bf16 rounding of
// the scaled operands.)
//
// axk_int4_gemm: out = a @ (b_int4 * b_scale[n, k / group])^T + bias (_mx_gemm, 564-623), bf16 activations, signed
// int4 weights one per byte, an fp32 scale per `group` consecutive K of each channel. Weight values are exact in bf16,
// so each 32-wide K slice is one v_mfma_f32_16x16x32_bf16 of the activations with the raw integers (exact products,
// fp32 sums), and its 16 x 16 partial is scaled by the slice's group scale (one per output channel = one per lane)
// into the fp32 accumulator: group % 32 == 0.
//
// m <= 64 (decode batches) takes the skinny kernels below; m and n of at least 128 the 128 x 128 tiles; the rest the
// 64 x 64 tiles: workgroup = 64 output rows x 64 output channels, 4 waves as 2 x 2 blocks of 32 x 32 (2 x 2 MFMA
// tiles). Each
// 64-wide K step of A and B is loaded one step ahead into registers (16 or 32 bytes a thread, 4 lanes per row),
// written to one of two LDS buffers (rows padded by 16 bytes: the 16-byte fragment reads of a wave spread over the
// banks) and read back in the MFMA layout: lane (row l % 16, K group l / 16) takes its row's K slice of group l / 16
// for the A operand, likewise for B; one barrier per step.
#include "axk_common.h"
#include "axk_host.h"

namespace {

typedef int axk_i32x4 __attribute__((ext_vector_type(4)));

constexpr int kI8Tile = 64, kI8Bk = 64, kI8Ld = kI8Bk + 16;

__global__ __launch_bounds__(256) void int8_gemm_kernel(const int8_t* __restrict__ a, int64_t lda,
                                                        const int8_t* __restrict__ b, const float* __restrict__ sa,
                                                        const float* __restrict__ sb, const float* __restrict__ bias,
                                                        void* __restrict__ out, int out_f32, int M, int N, int K) {
  __shared__ __align__(16) int8_t sA[2][kI8Tile * kI8Ld];
  __shared__ __align__(16) int8_t sB[2][kI8Tile * kI8Ld];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, g4 = lane >> 4;
  const int n0 = blockIdx.x * kI8Tile, m0 = blockIdx.y * kI8Tile;
  const int wm = wave >> 1, wn = wave & 1;
  // this thread's 16 bytes of a step: row r of the tile, bytes 16 c .. of the step
  const int r = tid >> 2, c = tid & 3;
  const int8_t* ap = a + (int64_t)min(m0 + r, M - 1) * lda + 16 * c;
  const int8_t* bp = b + (int64_t)min(n0 + r, N - 1) * K + 16 * c;
  const int nk = (K + kI8Bk - 1) / kI8Bk;
  // p already points at byte 16 c of its row; the chunk is wholly inside K or wholly past it (K % 16 == 0)
  auto load = [&](const int8_t* p, int ks) -> uint4 {
    const int kb = ks * kI8Bk;
    return kb + 16 * c < K ? *reinterpret_cast<const uint4*>(p + kb) : make_uint4(0u, 0u, 0u, 0u);
  };
  axk_i32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = axk_i32x4{0, 0, 0, 0};

  uint4 ra = load(ap, 0), rb = load(bp, 0);
  for (int ks = 0; ks < nk; ++ks) {
    const int buf = ks & 1;
    *reinterpret_cast<uint4*>(&sA[buf][r * kI8Ld + 16 * c]) = ra;
    *reinterpret_cast<uint4*>(&sB[buf][r * kI8Ld + 16 * c]) = rb;
    __syncthreads();  // the step's tiles are in LDS; every wave is done with the buffer written two steps ago
    if (ks + 1 < nk) {  // uniform: the next step lands while this one is computed
      ra = load(ap, ks + 1);
      rb = load(bp, ks + 1);
    }
    axk_i32x4 af[2], bf[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      af[i] = *reinterpret_cast<const axk_i32x4*>(&sA[buf][(32 * wm + 16 * i + l16) * kI8Ld + 16 * g4]);
      bf[i] = *reinterpret_cast<const axk_i32x4*>(&sB[buf][(32 * wn + 16 * i + l16) * kI8Ld + 16 * g4]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
  }
  // element (i, j, q): row m0 + 32 wm + 16 i + 4 g4 + q, channel n0 + 32 wn + 16 j + l16
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = m0 + 32 * wm + 16 * i + 4 * g4 + q, n = n0 + 32 * wn + 16 * j + l16;
        if (m >= M || n >= N) continue;
        float v = (float)acc[i][j][q] * sa[m] * sb[n];
        if (bias) v += bias[n];
        if (out_f32)
          reinterpret_cast<float*>(out)[(int64_t)m * N + n] = v;
        else
          reinterpret_cast<uint16_t*>(out)[(int64_t)m * N + n] = (uint16_t)f32_to_bf16_bits(v);
      }
}

// The large-tile int8 form (m and n of at least 128): workgroup = 128 x 128 outputs, 4 waves as 2 x 2 blocks of
// 64 x 64 (4 x 4 MFMA tiles each, 64 accumulator registers), so each 16-byte fragment read from LDS feeds 4 MFMAs
// instead of 2; the same 64-K steps double-buffered in LDS, each thread moving 2 + 2 16-byte pieces a step.
constexpr int kI8Big = 128;

__global__ __launch_bounds__(256) void int8_gemm_big_kernel(const int8_t* __restrict__ a, int64_t lda,
                                                            const int8_t* __restrict__ b, const float* __restrict__ sa,
                                                            const float* __restrict__ sb,
                                                            const float* __restrict__ bias, void* __restrict__ out,
                                                            int out_f32, int M, int N, int K) {
  __shared__ __align__(16) int8_t sA[2][kI8Big * kI8Ld];
  __shared__ __align__(16) int8_t sB[2][kI8Big * kI8Ld];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, g4 = lane >> 4;
  const int n0 = blockIdx.x * kI8Big, m0 = blockIdx.y * kI8Big;
  const int wm = wave >> 1, wn = wave & 1;
  // this thread's pieces of a step: rows r and r + 64 of each tile, bytes 16 c .. 16 c + 15 of the step
  const int r = tid >> 2, c = tid & 3;
  const int8_t* ap0 = a + (int64_t)min(m0 + r, M - 1) * lda + 16 * c;
  const int8_t* ap1 = a + (int64_t)min(m0 + r + 64, M - 1) * lda + 16 * c;
  const int8_t* bp0 = b + (int64_t)min(n0 + r, N - 1) * K + 16 * c;
  const int8_t* bp1 = b + (int64_t)min(n0 + r + 64, N - 1) * K + 16 * c;
  const int nk = (K + kI8Bk - 1) / kI8Bk;
  const axk_i32x4 z = {0, 0, 0, 0};
  // K % 16 == 0: a piece is wholly inside K or wholly past it
  auto load = [&](const int8_t* p, int ks) -> axk_i32x4 {
    const int kb = ks * kI8Bk;
    return kb + 16 * c < K ? *reinterpret_cast<const axk_i32x4*>(p + kb) : z;
  };
  axk_i32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = z;

  axk_i32x4 ra0 = load(ap0, 0), ra1 = load(ap1, 0), rb0 = load(bp0, 0), rb1 = load(bp1, 0);
  for (int ks = 0; ks < nk; ++ks) {
    const int buf = ks & 1;
    *reinterpret_cast<axk_i32x4*>(&sA[buf][r * kI8Ld + 16 * c]) = ra0;
    *reinterpret_cast<axk_i32x4*>(&sA[buf][(r + 64) * kI8Ld + 16 * c]) = ra1;
    *reinterpret_cast<axk_i32x4*>(&sB[buf][r * kI8Ld + 16 * c]) = rb0;
    *reinterpret_cast<axk_i32x4*>(&sB[buf][(r + 64) * kI8Ld + 16 * c]) = rb1;
    __syncthreads();  // the step's tiles are in LDS; every wave is done with the buffer written two steps ago
    if (ks + 1 < nk) {  // uniform: the next step lands while this one is computed
      ra0 = load(ap0, ks + 1);
      ra1 = load(ap1, ks + 1);
      rb0 = load(bp0, ks + 1);
      rb1 = load(bp1, ks + 1);
    }
    axk_i32x4 af[4], bf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      af[i] = *reinterpret_cast<const axk_i32x4*>(&sA[buf][(64 * wm + 16 * i + l16) * kI8Ld + 16 * g4]);
      bf[i] = *reinterpret_cast<const axk_i32x4*>(&sB[buf][(64 * wn + 16 * i + l16) * kI8Ld + 16 * g4]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
  }
  // element (i, j, q): row m0 + 64 wm + 16 i + 4 g4 + q, channel n0 + 64 wn + 16 j + l16
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + 64 * wn + 16 * j + l16;
    if (n >= N) continue;
    const float sbn = sb[n], bn = bias ? bias[n] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = m0 + 64 * wm + 16 * i + 4 * g4 + q;
        if (m >= M) continue;
        float v = (float)acc[i][j][q] * sa[m] * sbn;
        if (bias) v += bn;
        if (out_f32)
          reinterpret_cast<float*>(out)[(int64_t)m * N + n] = v;
        else
          reinterpret_cast<uint16_t*>(out)[(int64_t)m * N + n] = (uint16_t)f32_to_bf16_bits(v);
      }
  }
}

// 8 signed bytes -> 8 bf16 (exact: |v| <= 128 needs 8 significant bits).
AXK_DEV axk_bf16x8 i8x8_to_bf16x8(uint2 w) {
  axk_u32x4 r;
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const uint32_t d = h < 2 ? w.x : w.y, sh = 16 * (h & 1);
    const float lo = (float)(int8_t)(d >> sh), hi = (float)(int8_t)(d >> (sh + 8));
    r[h] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
  }
  return __builtin_bit_cast(axk_bf16x8, r);
}

constexpr int kI4LdA = 2 * kI8Bk + 16;  // bytes per bf16 activation row of a step in LDS

__global__ __launch_bounds__(256) void int4_gemm_kernel(const uint16_t* __restrict__ a, int64_t lda,
                                                        const int8_t* __restrict__ b, const float* __restrict__ bs,
                                                        int group, const float* __restrict__ bias,
                                                        void* __restrict__ out, int out_f32, int M, int N, int K) {
  __shared__ __align__(16) uint8_t sA[2][kI8Tile * kI4LdA];
  __shared__ __align__(16) int8_t sB[2][kI8Tile * kI8Ld];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, g4 = lane >> 4;
  const int n0 = blockIdx.x * kI8Tile, m0 = blockIdx.y * kI8Tile;
  const int wm = wave >> 1, wn = wave & 1;
  // this thread's share of a step: row r of the tile, K 16 c .. 16 c + 15 of the step (32 bytes of A, 16 of B)
  const int r = tid >> 2, c = tid & 3;
  const uint16_t* ap = a + (int64_t)min(m0 + r, M - 1) * lda + 16 * c;
  const int8_t* bp = b + (int64_t)min(n0 + r, N - 1) * K + 16 * c;
  const int nk = (K + kI8Bk - 1) / kI8Bk, ngroups = K / group;
  // group scales of the two output channels this lane's accumulators hold (tile column j)
  const float* srow0 = bs + (int64_t)min(n0 + 32 * wn + l16, N - 1) * ngroups;
  const float* srow1 = bs + (int64_t)min(n0 + 32 * wn + 16 + l16, N - 1) * ngroups;
  const axk_u32x4 z = {0u, 0u, 0u, 0u};
  axk_f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = axk_f32x4{0.f, 0.f, 0.f, 0.f};

  // K % 32 == 0: a 16-wide chunk is wholly inside K or wholly past it
  bool in = 16 * c < K;
  axk_u32x4 ra0 = in ? *reinterpret_cast<const axk_u32x4*>(ap) : z;
  axk_u32x4 ra1 = in ? *reinterpret_cast<const axk_u32x4*>(ap + 8) : z;
  axk_u32x4 rb = in ? *reinterpret_cast<const axk_u32x4*>(bp) : z;
  for (int ks = 0; ks < nk; ++ks) {
    const int buf = ks & 1;
    *reinterpret_cast<axk_u32x4*>(&sA[buf][r * kI4LdA + 32 * c]) = ra0;
    *reinterpret_cast<axk_u32x4*>(&sA[buf][r * kI4LdA + 32 * c + 16]) = ra1;
    *reinterpret_cast<axk_u32x4*>(&sB[buf][r * kI8Ld + 16 * c]) = rb;
    __syncthreads();  // the step's tiles are in LDS; every wave is done with the buffer written two steps ago
    if (ks + 1 < nk) {
      const int kb = (ks + 1) * kI8Bk;
      in = kb + 16 * c < K;
      ra0 = in ? *reinterpret_cast<const axk_u32x4*>(ap + kb) : z;
      ra1 = in ? *reinterpret_cast<const axk_u32x4*>(ap + kb + 8) : z;
      rb = in ? *reinterpret_cast<const axk_u32x4*>(bp + kb) : z;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k32 = ks * kI8Bk + 32 * h;
      if (k32 >= K) break;  // uniform
      axk_bf16x8 af[2], bf[2];
      const float sc[2] = {srow0[k32 / group], srow1[k32 / group]};
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        af[i] = *reinterpret_cast<const axk_bf16x8*>(&sA[buf][(32 * wm + 16 * i + l16) * kI4LdA + 64 * h + 16 * g4]);
        bf[i] = i8x8_to_bf16x8(
            *reinterpret_cast<const uint2*>(&sB[buf][(32 * wn + 16 * i + l16) * kI8Ld + 32 * h + 8 * g4]));
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const axk_f32x4 p = mfma_bf16_16x16x32(af[i], bf[j], axk_f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[i][j][q] = __builtin_fmaf(p[q], sc[j], acc[i][j][q]);
        }
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = m0 + 32 * wm + 16 * i + 4 * g4 + q, n = n0 + 32 * wn + 16 * j + l16;
        if (m >= M || n >= N) continue;
        float v = acc[i][j][q];
        if (bias) v += bias[n];
        if (out_f32)
          reinterpret_cast<float*>(out)[(int64_t)m * N + n] = v;
        else
          reinterpret_cast<uint16_t*>(out)[(int64_t)m * N + n] = (uint16_t)f32_to_bf16_bits(v);
      }
}

// The large-tile int4 form (m and n of at least 128): 128 x 128 outputs per workgroup, 4 waves of 64 x 64 (4 x 4
// MFMA tiles), 64-K steps double-buffered in LDS (each thread moving 4 16-byte activation pieces and 2 weight pieces a
// step); each 32-wide K slice's 16 x 16 partial scaled by its group scale as in the 64 x 64 form, or with CH (group %
// 64 == 0: a step lies in one group) the step's two slices chained into one partial, scaled once.
template <bool CH>
__global__ __launch_bounds__(256) void int4_gemm_big_kernel(const uint16_t* __restrict__ a, int64_t lda,
                                                            const int8_t* __restrict__ b, const float* __restrict__ bs,
                                                            int group, const float* __restrict__ bias,
                                                            void* __restrict__ out, int out_f32, int M, int N, int K) {
  __shared__ __align__(16) uint8_t sA[2][kI8Big * kI4LdA];
  __shared__ __align__(16) int8_t sB[2][kI8Big * kI8Ld];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, g4 = lane >> 4;
  const int n0 = blockIdx.x * kI8Big, m0 = blockIdx.y * kI8Big;
  const int wm = wave >> 1, wn = wave & 1;
  // this thread's share of a step: rows r and r + 64 of each tile, K 16 c .. 16 c + 15 of the step
  const int r = tid >> 2, c = tid & 3;
  const uint16_t* ap0 = a + (int64_t)min(m0 + r, M - 1) * lda + 16 * c;
  const uint16_t* ap1 = a + (int64_t)min(m0 + r + 64, M - 1) * lda + 16 * c;
  const int8_t* bp0 = b + (int64_t)min(n0 + r, N - 1) * K + 16 * c;
  const int8_t* bp1 = b + (int64_t)min(n0 + r + 64, N - 1) * K + 16 * c;
  const int nk = (K + kI8Bk - 1) / kI8Bk, ngroups = K / group;
  const float* srow[4];  // group scales of the four output channels this lane's accumulators hold (tile column j)
#pragma unroll
  for (int j = 0; j < 4; ++j) srow[j] = bs + (int64_t)min(n0 + 64 * wn + 16 * j + l16, N - 1) * ngroups;
  const axk_u32x4 z = {0u, 0u, 0u, 0u};
  axk_f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = axk_f32x4{0.f, 0.f, 0.f, 0.f};

  // K % 32 == 0: a 16-wide chunk is wholly inside K or wholly past it
  axk_u32x4 ra[4], rb[2];
  auto load = [&](int kb) {
    const bool in = kb + 16 * c < K;
    ra[0] = in ? *reinterpret_cast<const axk_u32x4*>(ap0 + kb) : z;
    ra[1] = in ? *reinterpret_cast<const axk_u32x4*>(ap0 + kb + 8) : z;
    ra[2] = in ? *reinterpret_cast<const axk_u32x4*>(ap1 + kb) : z;
    ra[3] = in ? *reinterpret_cast<const axk_u32x4*>(ap1 + kb + 8) : z;
    rb[0] = in ? *reinterpret_cast<const axk_u32x4*>(bp0 + kb) : z;
    rb[1] = in ? *reinterpret_cast<const axk_u32x4*>(bp1 + kb) : z;
  };
  load(0);
  for (int ks = 0; ks < nk; ++ks) {
    const int buf = ks & 1;
    *reinterpret_cast<axk_u32x4*>(&sA[buf][r * kI4LdA + 32 * c]) = ra[0];
    *reinterpret_cast<axk_u32x4*>(&sA[buf][r * kI4LdA + 32 * c + 16]) = ra[1];
    *reinterpret_cast<axk_u32x4*>(&sA[buf][(r + 64) * kI4LdA + 32 * c]) = ra[2];
    *reinterpret_cast<axk_u32x4*>(&sA[buf][(r + 64) * kI4LdA + 32 * c + 16]) = ra[3];
    *reinterpret_cast<axk_u32x4*>(&sB[buf][r * kI8Ld + 16 * c]) = rb[0];
    *reinterpret_cast<axk_u32x4*>(&sB[buf][(r + 64) * kI8Ld + 16 * c]) = rb[1];
    __syncthreads();  // the step's tiles are in LDS; every wave is done with the buffer written two steps ago
    if (ks + 1 < nk) load((ks + 1) * kI8Bk);  // uniform
    if constexpr (CH) {  // K % 64 == 0: the whole step, one group
      axk_bf16x8 af[2][4], bf[2][4];
      float sc[4];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          af[h][i] =
              *reinterpret_cast<const axk_bf16x8*>(&sA[buf][(64 * wm + 16 * i + l16) * kI4LdA + 64 * h + 16 * g4]);
          bf[h][i] = i8x8_to_bf16x8(
              *reinterpret_cast<const uint2*>(&sB[buf][(64 * wn + 16 * i + l16) * kI8Ld + 32 * h + 8 * g4]));
        }
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[j] = srow[j][ks * kI8Bk / group];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          axk_f32x4 p = mfma_bf16_16x16x32(af[0][i], bf[0][j], axk_f32x4{0.f, 0.f, 0.f, 0.f});
          p = mfma_bf16_16x16x32(af[1][i], bf[1][j], p);
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[i][j][q] = __builtin_fmaf(p[q], sc[j], acc[i][j][q]);
        }
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k32 = ks * kI8Bk + 32 * h;
        if (k32 >= K) break;  // uniform
        axk_bf16x8 af[4], bf[4];
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          af[i] =
              *reinterpret_cast<const axk_bf16x8*>(&sA[buf][(64 * wm + 16 * i + l16) * kI4LdA + 64 * h + 16 * g4]);
          bf[i] = i8x8_to_bf16x8(
              *reinterpret_cast<const uint2*>(&sB[buf][(64 * wn + 16 * i + l16) * kI8Ld + 32 * h + 8 * g4]));
          sc[i] = srow[i][k32 / group];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const axk_f32x4 p = mfma_bf16_16x16x32(af[i], bf[j], axk_f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[i][j][q] = __builtin_fmaf(p[q], sc[j], acc[i][j][q]);
          }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + 64 * wn + 16 * j + l16;
    if (n >= N) continue;
    const float bn = bias ? bias[n] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = m0 + 64 * wm + 16 * i + 4 * g4 + q;
        if (m >= M) continue;
        float v = acc[i][j][q];
        if (bias) v += bn;
        if (out_f32)
          reinterpret_cast<float*>(out)[(int64_t)m * N + n] = v;
        else
          reinterpret_cast<uint16_t*>(out)[(int64_t)m * N + n] = (uint16_t)f32_to_bf16_bits(v);
      }
  }
}

// Skinny forms (m <= 64, decode batches): a workgroup per 16 output channels, so n / 16 workgroups stream the
// weights; its 4 waves take interleaved K steps (neighbouring waves read neighbouring pieces of the same weight
// rows, nt) with MT = ceil(m / 16) row tiles of the activations each (read straight from global: every workgroup
// reads them, so they stay in L2), several steps in flight per wave (at least 64 weight bytes a lane); the 4
// partial sums meet in LDS.
constexpr int kSkU = 4;

template <int MT>
__global__ __launch_bounds__(256) void int8_skinny_kernel(const int8_t* __restrict__ a, int64_t lda,
                                                          const int8_t* __restrict__ b, const float* __restrict__ sa,
                                                          const float* __restrict__ sb, const float* __restrict__ bias,
                                                          void* __restrict__ out, int out_f32, int M, int N, int K) {
  // A wave step is 128 K: lane (l % 16, l / 16) reads bytes 32 (l / 16) .. + 31 of its weight row as two 16-byte
  // loads, so a step's two load instructions cover 16 whole 128-byte lines; the first MFMA takes every lane's first
  // 16 bytes, the second its last 16 (the activations are read with the same offsets, so each K meets its own).
  __shared__ axk_i32x4 red[4 * MT * 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, g4 = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int8_t* bp = b + (int64_t)min(n0 + l16, N - 1) * K + 32 * g4;
  const int8_t* ap[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) ap[t] = a + (int64_t)min(16 * t + l16, M - 1) * lda + 32 * g4;
  const int nk = (K + 127) / 128;
  axk_i32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = axk_i32x4{0, 0, 0, 0};
  constexpr int U = MT == 1 ? kSkU : kSkU / 2;
  for (int s0 = wave; s0 < nk; s0 += 4 * U) {
    axk_i32x4 bv[U][2], av[U][MT][2];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kb = (s0 + 4 * u) * 128 + 16 * h;
        const bool in = kb + 32 * g4 < K;  // K % 16 == 0: each 16-byte piece is wholly inside K or past it
        bv[u][h] = in ? (axk_i32x4)load_nt(bp + kb) : axk_i32x4{0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < MT; ++t)
          av[u][t][h] = in ? *reinterpret_cast<const axk_i32x4*>(ap[t] + kb) : axk_i32x4{0, 0, 0, 0};
      }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int t = 0; t < MT; ++t)
          acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[u][t][h], bv[u][h], acc[t], 0, 0, 0);
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) red[(wave * MT + t) * 64 + lane] = acc[t];
  __syncthreads();
  // element e = (t * 64 + lane) * 4 + q of every wave's partial: row 16 t + 4 (lane / 16) + q, channel lane % 16
  const int* ri = reinterpret_cast<const int*>(red);
  for (int e = threadIdx.x; e < MT * 256; e += 256) {
    const int t = e >> 8, ln = (e >> 2) & 63, q = e & 3;
    const int m = 16 * t + 4 * (ln >> 4) + q, n = n0 + (ln & 15);
    if (m >= M || n >= N) continue;
    const int sum = ri[e] + ri[MT * 256 + e] + ri[2 * MT * 256 + e] + ri[3 * MT * 256 + e];
    float v = (float)sum * sa[m] * sb[n];
    if (bias) v += bias[n];
    if (out_f32)
      reinterpret_cast<float*>(out)[(int64_t)m * N + n] = v;
    else
      reinterpret_cast<uint16_t*>(out)[(int64_t)m * N + n] = (uint16_t)f32_to_bf16_bits(v);
  }
}

// The int4 skinny form: steps of KS = 64 K when group % 64 == 0 (lane (l % 16, l / 16) reads 16 weight bytes and 16
// activations at K offset 16 (l / 16) of the step: two chained v_mfma_f32_16x16x32_bf16 per row tile, the first on
// each lane's low 8, the second on its high 8, both inside one group), else KS = 32 (8 bytes and 8 activations at
// offset 8 (l / 16), one MFMA); each step's 16 x 16 partial is scaled by the step's group scale.
template <int MT, int KS>
__global__ __launch_bounds__(256) void int4_skinny_kernel(const uint16_t* __restrict__ a, int64_t lda,
                                                          const int8_t* __restrict__ b, const float* __restrict__ bs,
                                                          int group, const float* __restrict__ bias,
                                                          void* __restrict__ out, int out_f32, int M, int N, int K) {
  static_assert(KS == 32 || KS == 64, "step of 32 or 64 K");
  constexpr int BL = KS / 4, H = KS / 32;  // bytes (and activations) a lane reads per step; MFMAs per step
  constexpr int U = KS == 32 ? 2 * kSkU : (MT == 1 ? 2 * kSkU : kSkU);
  __shared__ axk_f32x4 red[4 * MT * 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, g4 = lane >> 4;
  const int n0 = blockIdx.x * 16, nc = min(n0 + l16, N - 1);
  const int8_t* bp = b + (int64_t)nc * K + BL * g4;
  const float* srow = bs + (int64_t)nc * (K / group);
  const uint16_t* ap[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) ap[t] = a + (int64_t)min(16 * t + l16, M - 1) * lda + BL * g4;
  const int nk = K / KS;  // K % group == 0 and group % KS == 0
  axk_f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = axk_f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s0 = wave; s0 < nk; s0 += 4 * U) {
    uint2 bv[U][H];
    axk_bf16x8 av[U][MT][H];
    float sc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + 4 * u;
      const bool in = s < nk;  // uniform
      if (KS == 64) {
        const axk_u32x4 w = in ? load_nt(bp + KS * s) : axk_u32x4{0u, 0u, 0u, 0u};
        bv[u][0] = make_uint2(w[0], w[1]);
        bv[u][H - 1] = make_uint2(w[2], w[3]);
      } else if (in) {
        const axk_i32x2 w = __builtin_nontemporal_load(reinterpret_cast<const axk_i32x2*>(bp + KS * s));
        bv[u][0] = make_uint2((uint32_t)w[0], (uint32_t)w[1]);
      } else {
        bv[u][0] = make_uint2(0u, 0u);
      }
      sc[u] = in ? srow[KS * s / group] : 0.f;
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int h = 0; h < H; ++h)
          av[u][t][h] = in ? *reinterpret_cast<const axk_bf16x8*>(ap[t] + KS * s + 8 * h) : axk_bf16x8{};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      axk_bf16x8 w[H];
#pragma unroll
      for (int h = 0; h < H; ++h) w[h] = i8x8_to_bf16x8(bv[u][h]);
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        axk_f32x4 p = mfma_bf16_16x16x32(av[u][t][0], w[0], axk_f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int h = 1; h < H; ++h) p = mfma_bf16_16x16x32(av[u][t][h], w[h], p);
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[t][q] = __builtin_fmaf(p[q], sc[u], acc[t][q]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) red[(wave * MT + t) * 64 + lane] = acc[t];
  __syncthreads();
  const float* rf = reinterpret_cast<const float*>(red);
  for (int e = threadIdx.x; e < MT * 256; e += 256) {
    const int t = e >> 8, ln = (e >> 2) & 63, q = e & 3;
    const int m = 16 * t + 4 * (ln >> 4) + q, n = n0 + (ln & 15);
    if (m >= M || n >= N) continue;
    float v = ((rf[e] + rf[MT * 256 + e]) + rf[2 * MT * 256 + e]) + rf[3 * MT * 256 + e];
    if (bias) v += bias[n];
    if (out_f32)
      reinterpret_cast<float*>(out)[(int64_t)m * N + n] = v;
    else
      reinterpret_cast<uint16_t*>(out)[(int64_t)m * N + n] = (uint16_t)f32_to_bf16_bits(v);
  }
}

}  // namespace

extern "C" int axk_int8_gemm(const int8_t* a, int64_t lda, const int8_t* b_int8, const float* scale_a,
                             const float* scale_b, const float* bias, void* out, int out_dtype, int64_t m, int64_t n,
                             int64_t k, axk_stream_t stream) {
  AXK_REQUIRE(a && b_int8 && scale_a && scale_b && out, AXK_E_NULL);
  AXK_REQUIRE(m >= 0 && n >= 0 && k > 0 && k % 16 == 0 && m <= INT32_MAX && n <= INT32_MAX && k <= INT32_MAX,
              AXK_E_SHAPE);
  AXK_REQUIRE(lda >= k && lda % 16 == 0 && axk_aligned(a, 16) && axk_aligned(b_int8, 16), AXK_E_ALIGN);
  AXK_REQUIRE(out_dtype == AXK_DT_BF16 || out_dtype == AXK_DT_F32, AXK_E_DTYPE);
  if (m == 0 || n == 0) return AXK_OK;
  const size_t out_bytes = (size_t)m * n * (out_dtype == AXK_DT_F32 ? 4 : 2);
  AXK_REQUIRE(!axk_overlap(out, out_bytes, a, (size_t)((m - 1) * lda + k)) &&
                  !axk_overlap(out, out_bytes, b_int8, (size_t)(n * k)),
              AXK_E_ALIAS);
  const dim3 grid((unsigned)((n + kI8Tile - 1) / kI8Tile), (unsigned)((m + kI8Tile - 1) / kI8Tile));
  AXK_REQUIRE(grid.x <= INT32_MAX && grid.y <= 65535, AXK_E_SHAPE);
  AXK_LAUNCH_GATE();
  const int f32 = out_dtype == AXK_DT_F32 ? 1 : 0;
  if (m <= 64) {
    const dim3 sg((unsigned)((n + 15) / 16));
    const hipStream_t st = axk_stream(stream);
    if (m <= 16)
      hipLaunchKernelGGL(int8_skinny_kernel<1>, sg, dim3(256), 0, st, a, lda, b_int8, scale_a, scale_b, bias, out,
                         f32, (int)m, (int)n, (int)k);
    else if (m <= 32)
      hipLaunchKernelGGL(int8_skinny_kernel<2>, sg, dim3(256), 0, st, a, lda, b_int8, scale_a, scale_b, bias, out,
                         f32, (int)m, (int)n, (int)k);
    else
      hipLaunchKernelGGL(int8_skinny_kernel<4>, sg, dim3(256), 0, st, a, lda, b_int8, scale_a, scale_b, bias, out,
                         f32, (int)m, (int)n, (int)k);
    return axk_launch_status();
  }
  if (m >= kI8Big && n >= kI8Big) {
    const dim3 bg((unsigned)((n + kI8Big - 1) / kI8Big), (unsigned)((m + kI8Big - 1) / kI8Big));
    hipLaunchKernelGGL(int8_gemm_big_kernel, bg, dim3(256), 0, axk_stream(stream), a, lda, b_int8, scale_a, scale_b,
                       bias, out, f32, (int)m, (int)n, (int)k);
    return axk_launch_status();
  }
  hipLaunchKernelGGL(int8_gemm_kernel, grid, dim3(256), 0, axk_stream(stream), a, lda, b_int8, scale_a, scale_b, bias,
                     out, out_dtype == AXK_DT_F32 ? 1 : 0, (int)m, (int)n, (int)k);
  return axk_launch_status();
}

extern "C" int axk_int4_gemm(const uint16_t* a, int64_t lda, const int8_t* b_int4, const float* b_scale, int64_t group,
                             const float* bias, void* out, int out_dtype, int64_t m, int64_t n, int64_t k,
                             axk_stream_t stream) {
  AXK_REQUIRE(a && b_int4 && b_scale && out, AXK_E_NULL);
  AXK_REQUIRE(m >= 0 && n >= 0 && k > 0 && k % 32 == 0 && group > 0 && group % 32 == 0 && k % group == 0 &&
                  m <= INT32_MAX && n <= INT32_MAX && k <= INT32_MAX,
              AXK_E_SHAPE);
  AXK_REQUIRE(lda >= k && lda % 8 == 0 && axk_aligned(a, 16) && axk_aligned(b_int4, 16) && axk_aligned(b_scale, 4),
              AXK_E_ALIGN);
  AXK_REQUIRE(out_dtype == AXK_DT_BF16 || out_dtype == AXK_DT_F32, AXK_E_DTYPE);
  if (m == 0 || n == 0) return AXK_OK;
  const size_t out_bytes = (size_t)m * n * (out_dtype == AXK_DT_F32 ? 4 : 2);
  AXK_REQUIRE(!axk_overlap(out, out_bytes, a, (size_t)((m - 1) * lda + k) * 2) &&
                  !axk_overlap(out, out_bytes, b_int4, (size_t)(n * k)) &&
                  !axk_overlap(out, out_bytes, b_scale, (size_t)(n * (k / group)) * 4),
              AXK_E_ALIAS);
  const dim3 grid((unsigned)((n + kI8Tile - 1) / kI8Tile), (unsigned)((m + kI8Tile - 1) / kI8Tile));
  AXK_REQUIRE(grid.x <= INT32_MAX && grid.y <= 65535, AXK_E_SHAPE);
  AXK_LAUNCH_GATE();
  const int f32 = out_dtype == AXK_DT_F32 ? 1 : 0;
  if (m <= 64) {
    const dim3 sg((unsigned)((n + 15) / 16));
    const hipStream_t st = axk_stream(stream);
    auto go = [&](auto kern) {
      hipLaunchKernelGGL(kern, sg, dim3(256), 0, st, a, lda, b_int4, b_scale, (int)group, bias, out, f32, (int)m,
                         (int)n, (int)k);
    };
    const bool wide = group % 64 == 0;
    if (m <= 16)
      wide ? go(int4_skinny_kernel<1, 64>) : go(int4_skinny_kernel<1, 32>);
    else if (m <= 32)
      wide ? go(int4_skinny_kernel<2, 64>) : go(int4_skinny_kernel<2, 32>);
    else
      wide ? go(int4_skinny_kernel<4, 64>) : go(int4_skinny_kernel<4, 32>);
    return axk_launch_status();
  }
  if (m >= kI8Big && n >= kI8Big) {
    const dim3 bg((unsigned)((n + kI8Big - 1) / kI8Big), (unsigned)((m + kI8Big - 1) / kI8Big));
    if (group % 64 == 0)
      hipLaunchKernelGGL(int4_gemm_big_kernel<true>, bg, dim3(256), 0, axk_stream(stream), a, lda, b_int4, b_scale,
                         (int)group, bias, out, f32, (int)m, (int)n, (int)k);
    else
      hipLaunchKernelGGL(int4_gemm_big_kernel<false>, bg, dim3(256), 0, axk_stream(stream), a, lda, b_int4, b_scale,
                         (int)group, bias, out, f32, (int)m, (int)n, (int)k);
    return axk_launch_status();
  }
  hipLaunchKernelGGL(int4_gemm_kernel, grid, dim3(256), 0, axk_stream(stream), a, lda, b_int4, b_scale, (int)group,
                     bias, out, out_dtype == AXK_DT_F32 ? 1 : 0, (int)m, (int)n, (int)k);
  return axk_launch_status();
}
