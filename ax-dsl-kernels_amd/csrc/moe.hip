// MoE layer with MXFP4 experts for gfx950: router top-K, shared expert with sigmoid gate, routed SwiGLU
// experts, combine. Semantics of moe_full (models/qwen35_35b_a3b/src/70b0fbc/q35_layer_mc.py:797-853):
//   logits = h2 W_router^T (fp32); p = softmax(logits); top-K by value (ties: lower expert id), rw = p / sum p
//   shared: act = bf16(silu(bf16(h2 Wg^T)) * bf16(h2 Wu^T)); sh = act Wd^T (fp32); gate = sigmoid(h2 . w_shg)
//   base = x_res + gate * sh;  out = bf16(base + sum_k rw_k * down_k(silu(gate_k) * up_k))
// The reference also rounds `base` to bf16 before the sum (the layer kernel's bf16 `out`); here it stays fp32
// so the output is rounded once: a value within half an ulp of a bf16 midpoint would otherwise flip by one
// ulp of |base| between any two summation orders.
// Routed experts are planar MXFP4 tensors: gate-up e_gw [E, 2F, H/2] (gate rows, then up rows), e_gs
// [E, 2F, H/32]; down e_dw [E, H, F/2], e_ds [E, H, F/32] (models/qwen35_35b_a3b/qwen35_35b_a3b.manifest.json).
//
// Router (axk_moe_decode; q35_layer_mc.py:820-829):
//   router       — decode: GEMV split over K, workgroup = (16 experts, 16 tokens, K slice), partial logits per
//                  slice; one extra expert block forms the shared gate's partial logit h2 . w_shg per slice
//   router_tile  — prefill: 64 x 64 MFMA tiles of tokens x experts over two K halves
//   route_part   — one wave per token: the partials summed in slice order into the logits (and, in decode, the
//                  gate logit), softmax, top-K by ballot rounds (ties: lower id), renormalised weights
//   route        — the same selection from caller logits (axk_moe_route)
// Experts, decode (tokens <= kDecodeTokens, tokens x top_k <= kMaxPairs):
//   gateup  — workgroup = (active expert or the shared expert, run of 16-row weight tiles). The workgroup groups
//             the pairs itself: it reads the top-K ids once, finds the slot-th active expert in ascending id order
//             from an LDS bitmap and ranks that expert's pairs by ballots (stable, deterministic, no grouping
//             launch). Each wave streams its MXFP4 gate and up rows over the full K; for small row counts the
//             weights pass through a wave-private LDS tile in 128-byte row segments (whole cache lines per
//             load) and are read back in the MFMA layout; SwiGLU in the epilogue, activations by pair
//   down    — the same grouping and streaming over hidden-row tiles: act x Wd^T, scaled by the routing weight,
//             written to y by pair
//   combine — workgroup = (token, columns): shared gate (from the router's gate logit, or a dot here), residual,
//             sum over the token's K pairs in slot order, one bf16 rounding
// Every expert's weights are read once per call, whatever the number of its tokens.
//
// Prefill (tokens > kDecodeTokens; moe_slots_px + moe_combine of q35_moe_prefill.py:150-214):
//   pcount / pscan / pscatter — the pairs grouped by expert in 256-token blocks (per-block bitmask counts, one
//             scan of the (expert, block) bases, stable scatter), plus a tile list of kBM-row tiles per active
//             expert and for the shared expert over all tokens
//   ggemm   — a grouped GEMM on MFMA: workgroup = (tile, 256 weight rows), workgroups spread over the XCDs so
//             that each XCD takes a contiguous run of the expert-ordered tiles; A rows gathered by token and
//             B MXFP4 rows land in an LDS ring by direct loads; per-wave 64 x 64 blocks; gate-up with the
//             SwiGLU epilogue, then down with the routing-weight epilogue into bf16 y by pair
//   combine — as decode
#include "axk_common.h"
#include "axk_host.h"
#include "axk_mx_tile.h"

namespace {

using axk::WF_MXFP4;

constexpr int kMaxExperts = 1024;
constexpr int kMaxTopK = 32;  // <= 64: lane k of the routing wave keeps selection k
constexpr int kMaxPairs = 8192;
constexpr int kMaskWords = 4;  // token bitmask words per expert in a 256-token block of the prefill grouping
constexpr size_t kMaxStageLds = 160 * 1024;  // dynamic LDS of the prefill GEMMs (the whole CU's LDS)
// dynamic LDS of the decode streaming kernels (activation rows of K + 8 bf16, the wave tiles): the CU's LDS less
// 4 KiB for their static grouping state
constexpr size_t kMaxStreamLds = 156 * 1024;
constexpr int kDecodeTokens = 64 * kMaskWords;  // above this the prefill path runs
constexpr int64_t kMaxPrefillTokens = 1 << 16;
constexpr int64_t kMaxPrefillPairs = 1 << 19;
constexpr int kBlkTokens = 256;  // tokens per block of the prefill grouping
constexpr int kBM = 128, kBK = 64;  // prefill GEMM tile rows, K step

struct MoeWs {
  int* counts;      // [E]
  int* offsets;     // [E + 1]
  int4* active;     // [E] active expert i: {rows, expert, first sorted row, 0}; rows 0 past the list
  int* n_active;    // [2]: the active experts; [1] the decode routing's finished-workgroup count
  int* pair_pos;    // [P] sorted row of pair p = t * K + k
  int* row_tok;     // [P] token of sorted row
  float* row_w;     // [P] routing weight of sorted row
  uint16_t* act;    // [P, F] bf16 routed activations (sorted rows)
  uint16_t* act_sh; // [T, Fs] bf16 shared-expert activations
  float* y;         // [P, H] routed outputs x routing weight, row t * K + k for pair (t, k): fp32 (decode) or
                    // bf16 (prefill: the first P H bf16 of the buffer)
  float* y_sh;      // [T, H] fp32 shared-expert output
  int* blk;         // [NB, E] prefill: per-block expert counts, then per-block row bases
  int4* tiles;      // [max tiles] prefill GEMM tiles: {expert (-1: shared), first row, rows, 0}
  int* n_tiles;     // [1]
  int* row_pair;    // [P] pair t * K + k of sorted row (y is indexed by pair)
  float* rpart;     // [S, T, E] router partial logits of K slice s
  float* gate_logit; // [T] decode: the shared expert's gate logit h2 . w_shg, summed from
  float* gpart;      // [S, T] its slice partials
};

int64_t prefill_blocks(int64_t T) { return (T + kBlkTokens - 1) / kBlkTokens; }
int64_t prefill_max_tiles(int64_t T, int64_t E, int64_t K) {
  return (T * K + kBM - 1) / kBM + E + (T + kBM - 1) / kBM;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Router partial logits, summed in slice order by the routing kernel. Decode: K slices of 8 steps of 32 (1..16 slices),
// prefill: two K halves.
constexpr int kMaxRouterSplits = 16;
constexpr int kPrefillRouterSplits = 2;
int router_splits(int64_t H) {
  const int64_t s = (H / 32) / 8;
  return (int)(s < 1 ? 1 : (s > kMaxRouterSplits ? kMaxRouterSplits : s));
}

constexpr int kWsParts = 17;

size_t moe_ws_layout(int64_t T, int64_t H, int64_t E, int64_t K, int64_t F, int64_t Fs, size_t* off) {
  const int64_t P = T * K;
  const bool prefill = T > kDecodeTokens;
  const size_t nb = prefill ? (size_t)prefill_blocks(T) : 0, nt = prefill ? (size_t)prefill_max_tiles(T, E, K) : 0;
  const size_t S = prefill ? kPrefillRouterSplits : router_splits(H);
  const size_t rp = S * T * E * 4;
  size_t o = 0;
  const size_t sizes[kWsParts] = {(size_t)E * 4,      (size_t)(E + 1) * 4, (size_t)E * 16,    8,
                                  (size_t)P * 4,      (size_t)P * 4,       (size_t)P * 4,     (size_t)P * F * 2,
                                  (size_t)T * Fs * 2, (size_t)P * H * 4,   (size_t)T * H * 4, nb * E * 4,
                                  nt * 16,            4,                   (size_t)P * 4,     rp,
                                  (S + 1) * T * 4};
  for (int i = 0; i < kWsParts; ++i) {
    off[i] = o;
    o = align256(o + sizes[i]);
  }
  return o;
}

MoeWs moe_ws(void* ws, int64_t T, int64_t H, int64_t E, int64_t K, int64_t F, int64_t Fs) {
  size_t off[kWsParts];
  moe_ws_layout(T, H, E, K, F, Fs, off);
  unsigned char* b = reinterpret_cast<unsigned char*>(ws);
  return {reinterpret_cast<int*>(b + off[0]),       reinterpret_cast<int*>(b + off[1]),
          reinterpret_cast<int4*>(b + off[2]),      reinterpret_cast<int*>(b + off[3]),
          reinterpret_cast<int*>(b + off[4]),       reinterpret_cast<int*>(b + off[5]),
          reinterpret_cast<float*>(b + off[6]),     reinterpret_cast<uint16_t*>(b + off[7]),
          reinterpret_cast<uint16_t*>(b + off[8]),  reinterpret_cast<float*>(b + off[9]),
          reinterpret_cast<float*>(b + off[10]),    reinterpret_cast<int*>(b + off[11]),
          reinterpret_cast<int4*>(b + off[12]),     reinterpret_cast<int*>(b + off[13]),
          reinterpret_cast<int*>(b + off[14]),      reinterpret_cast<float*>(b + off[15]),
          reinterpret_cast<float*>(b + off[16]),    reinterpret_cast<float*>(b + off[16]) + T};
}

// ---------------------------------------------------------------------------------------------
// route: one wave per token
// ---------------------------------------------------------------------------------------------
// Softmax and top-K of one token's logits, lane l holding experts l + 64 i (x[i] = -inf past E). Selection k is
// the largest remaining logit (the softmax is monotonic), ties to the lower expert id: a DPP wave maximum, then
// one ballot per register finds the lowest id holding it. Lane k keeps selection k.
template <int V>
AXK_DEV int route_select(const float (&x)[V], int lane, int E, int K, int norm_topk, int32_t* __restrict__ ids,
                         float* __restrict__ wts) {
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < V; ++i) mx = fmaxf(mx, x[i]);
  mx = wave_max(mx);
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) sum += (i * 64 + lane < E) ? __expf(x[i] - mx) : 0.f;
  const float inv = 1.0f / wave_sum(sum);
  unsigned taken = 0u;  // bit i: x[i] already selected
  float myp = 0.f, psum = 0.f;
  int myid = 0;
  for (int k = 0; k < K; ++k) {
    float bv = -INFINITY;
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (i * 64 + lane < E && !(taken >> i & 1u)) bv = fmaxf(bv, x[i]);
    const float m = wave_max(bv);
    int id = -1;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const unsigned long long hit = __ballot(i * 64 + lane < E && !(taken >> i & 1u) && x[i] == m);
      if (id < 0 && hit) id = i * 64 + __builtin_ctzll(hit);
    }
    if (id < 0) {  // no remaining logit compares equal (NaN): the lowest remaining id
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const unsigned long long left = __ballot(i * 64 + lane < E && !(taken >> i & 1u));
        if (id < 0 && left) id = i * 64 + __builtin_ctzll(left);
      }
    }
    if ((id & 63) == lane) taken |= 1u << (id >> 6);
    const float p = __expf(m - mx) * inv;
    if (lane == k) {
      myp = p;
      myid = id;
    }
    psum += p;
  }
  if (lane < K) {
    ids[lane] = myid;
    wts[lane] = norm_topk ? myp / psum : myp;
  }
  return lane < K ? myid : -1;  // lane k: selection k
}

template <int V>  // expert logits per lane (num_experts <= 64 V)
__global__ __launch_bounds__(256) void moe_route_kernel(const float* __restrict__ logits, int T, int E, int K,
                                                        int norm_topk, int32_t* __restrict__ ids,
                                                        float* __restrict__ wts) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* lg = logits + (int64_t)t * E;
  float x[V];
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int e = i * 64 + lane;
    const float v = lg[min(e, E - 1)];  // unconditional (clamped) loads
    x[i] = e < E ? v : -INFINITY;
  }
  route_select<V>(x, lane, E, K, norm_topk, ids + (int64_t)t * K, wts + (int64_t)t * K);
}

// Routing from the router's partial logits: logit = sum of the S K-slice partials in slice order (written out as the
// layer's logits), then route_select. With gpart (decode), lane 0 of token t's wave also sums the shared gate's S
// partial logits in slice order into gate_logit[t]. With blk (prefill), each selection is counted into its
// (256-token block, expert) count blk[block E + e], zeroed by the router launch: the counts the prefill grouping
// scans (a token's K selections are distinct experts, so this is each block's per-expert token count).
template <int V, int MAXS>  // MAXS: bound on the number of partials
__global__ __launch_bounds__(256) void moe_route_part_kernel(const float* __restrict__ part,
                                                             const float* __restrict__ gpart, int S, int T, int E,
                                                             int K, int norm_topk, float* __restrict__ logits,
                                                             float* __restrict__ gate_logit,
                                                             int32_t* __restrict__ ids, float* __restrict__ wts,
                                                             int* __restrict__ blk) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;
  // all S x V partial loads unconditional (slices past S clamped, then dropped): one memory round trip
  float pv[MAXS][V];
#pragma unroll
  for (int sl = 0; sl < MAXS; ++sl)
#pragma unroll
    for (int i = 0; i < V; ++i)
      pv[sl][i] = part[((int64_t)min(sl, S - 1) * T + t) * E + min(i * 64 + lane, E - 1)];
  float gp[MAXS];
  if (gpart) {
#pragma unroll
    for (int sl = 0; sl < MAXS; ++sl) gp[sl] = gpart[(int64_t)min(sl, S - 1) * T + t];
  }
  float x[V];
#pragma unroll
  for (int i = 0; i < V; ++i) {
    float v = pv[0][i];
#pragma unroll
    for (int sl = 1; sl < MAXS; ++sl)
      if (sl < S) v += pv[sl][i];
    x[i] = v;
  }
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int e = i * 64 + lane;
    if (e < E) logits[(int64_t)t * E + e] = x[i];
    else x[i] = -INFINITY;
  }
  if (gpart && lane == 0) {
    float gv = gp[0];
#pragma unroll
    for (int sl = 1; sl < MAXS; ++sl)
      if (sl < S) gv += gp[sl];
    gate_logit[t] = gv;
  }
  const int id = route_select<V>(x, lane, E, K, norm_topk, ids + (int64_t)t * K, wts + (int64_t)t * K);
  if (blk && id >= 0 && id < E) atomicAdd(blk + (int64_t)(t / kBlkTokens) * E + id, 1);
}

// Prefill router GEMM: workgroup (64 tokens, 64 experts, K slice s), waves 2 x 2 with 32 x 32 each; both operands
// staged in LDS per 64-wide K step from line-coalesced loads (8 lanes per 128-byte row segment), loaded two
// steps ahead in register stages. Writes the slice's partial logits like the decode router.
__global__ __launch_bounds__(256) void moe_router_tile_kernel(const uint16_t* __restrict__ h2,
                                                              const uint16_t* __restrict__ wr, int T, int H, int E,
                                                              int S, float* __restrict__ part, int* __restrict__ blk,
                                                              int nblk) {
  {  // the routing launch's (block, expert) counts to zero, spread over the grid
    const int64_t wg = blockIdx.x + (int64_t)gridDim.x * (blockIdx.y + (int64_t)gridDim.y * blockIdx.z);
    const int64_t nth = (int64_t)gridDim.x * gridDim.y * gridDim.z * blockDim.x;
    for (int64_t i = wg * blockDim.x + threadIdx.x; i < nblk; i += nth) blk[i] = 0;
  }
  constexpr int kLd = 72;
  __shared__ __align__(16) uint16_t sA[2][64 * kLd];
  __shared__ __align__(16) uint16_t sB[2][64 * kLd];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l16 = lane & 15, g4 = lane >> 4;
  const int t0 = blockIdx.x * 64, e0 = blockIdx.y * 64, sl = blockIdx.z;
  const int nall = H / 64, kb = (int)((int64_t)sl * nall / S), nk = (int)((int64_t)(sl + 1) * nall / S) - kb;
  const int r = tid >> 3, c = tid & 7;
  const uint16_t* ap0 = h2 + (int64_t)min(t0 + r, T - 1) * H + 8 * c;
  const uint16_t* ap1 = h2 + (int64_t)min(t0 + r + 32, T - 1) * H + 8 * c;
  const uint16_t* bp0 = wr + (int64_t)min(e0 + r, E - 1) * H + 8 * c;
  const uint16_t* bp1 = wr + (int64_t)min(e0 + r + 32, E - 1) * H + 8 * c;
  const int wm = wave >> 1, wn = wave & 1;
  if (nk <= 0) return;
#define AXK_RT_LOAD(A0, A1, B0, B1, ks)                        \
  do {                                                         \
    const int k_ = (kb + min((ks), nk - 1)) * 64;              \
    A0 = *reinterpret_cast<const uint4*>(ap0 + k_);            \
    A1 = *reinterpret_cast<const uint4*>(ap1 + k_);            \
    B0 = *reinterpret_cast<const uint4*>(bp0 + k_);            \
    B1 = *reinterpret_cast<const uint4*>(bp1 + k_);            \
  } while (0)
#define AXK_RT_STORE(A0, A1, B0, B1, buf)                                  \
  do {                                                                     \
    *reinterpret_cast<uint4*>(&sA[buf][r * kLd + 8 * c]) = A0;             \
    *reinterpret_cast<uint4*>(&sA[buf][(r + 32) * kLd + 8 * c]) = A1;      \
    *reinterpret_cast<uint4*>(&sB[buf][r * kLd + 8 * c]) = B0;             \
    *reinterpret_cast<uint4*>(&sB[buf][(r + 32) * kLd + 8 * c]) = B1;      \
  } while (0)
  axk_f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = axk_f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      axk_bf16x8 af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        af[i] = load_bf16x8(&sA[buf][(32 * wm + 16 * i + l16) * kLd + 32 * kh + 8 * g4]);
        bf[i] = load_bf16x8(&sB[buf][(32 * wn + 16 * i + l16) * kLd + 32 * kh + 8 * g4]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma_bf16_16x16x32(af[i], bf[j], acc[i][j]);
    }
  };
  uint4 a00, a10, b00, b10, a01, a11, b01, b11, a02, a12, b02, b12;
  AXK_RT_LOAD(a00, a10, b00, b10, 0);
  AXK_RT_LOAD(a01, a11, b01, b11, 1);
  AXK_RT_STORE(a00, a10, b00, b10, 0);
  __syncthreads();
  for (int ks = 0; ks < nk; ks += 3) {  // one exit; steps past nk only move clamped data
    AXK_RT_LOAD(a02, a12, b02, b12, ks + 2);
    compute(ks & 1);
    AXK_RT_STORE(a01, a11, b01, b11, (ks + 1) & 1);
    __syncthreads();
    AXK_RT_LOAD(a00, a10, b00, b10, ks + 3);
    if (ks + 1 < nk) compute((ks + 1) & 1);
    AXK_RT_STORE(a02, a12, b02, b12, ks & 1);
    __syncthreads();
    AXK_RT_LOAD(a01, a11, b01, b11, ks + 4);
    if (ks + 2 < nk) compute(ks & 1);
    AXK_RT_STORE(a00, a10, b00, b10, (ks + 1) & 1);
    __syncthreads();
  }
#undef AXK_RT_LOAD
#undef AXK_RT_STORE
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int t = t0 + 32 * wm + 16 * i + 4 * g4 + q, e = e0 + 32 * wn + 16 * j + l16;
        if (t < T && e < E) part[((int64_t)sl * T + t) * E + e] = acc[i][j][q];
      }
}

// Decode router GEMM, split over K: workgroup (16 experts, 16 tokens, K slice s); wave w multiplies the slice's
// 32-wide K steps w, w + 4, ... on MFMA (h2 rows as A, router rows as B), the four waves are summed in LDS and
// the partial logits written to part[s]. With gpart, expert block ceil(E / 16) multiplies the shared expert's gate
// vector w_shg instead and writes the partial gate logit (h2 . w_shg over the slice) to gpart[s, t]. Rows past T or
// E are clamped for the loads and never stored.
__global__ __launch_bounds__(256) void moe_router_kernel(const uint16_t* __restrict__ h2,
                                                         const uint16_t* __restrict__ wr,
                                                         const uint16_t* __restrict__ w_shg, int T, int H, int E,
                                                         int S, float* __restrict__ part, float* __restrict__ gpart) {
  __shared__ float4 red[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nl = lane & 15, g = lane >> 4;
  const bool gate_blk = (int)blockIdx.x * 16 >= E;  // the extra block (launched only with gpart)
  const int e0 = blockIdx.x * 16, t0 = blockIdx.y * 16, sl = blockIdx.z;
  const int ns = H / 32, st0 = (int)((int64_t)sl * ns / S), st1 = (int)((int64_t)(sl + 1) * ns / S);
  const uint16_t* arow = h2 + (int64_t)min(t0 + nl, T - 1) * H + 8 * g;
  const uint16_t* brow = gate_blk ? w_shg + 8 * g : wr + (int64_t)min(e0 + nl, E - 1) * H + 8 * g;
  axk_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int i = st0 + wave; i < st1; i += 8) {
    const int j = min(i + 4, st1 - 1);
    const axk_bf16x8 a0 = load_bf16x8(arow + 32 * i), b0 = load_bf16x8(brow + 32 * i);
    const axk_bf16x8 a1 = load_bf16x8(arow + 32 * j), b1 = load_bf16x8(brow + 32 * j);
    acc = mfma_bf16_16x16x32(a0, b0, acc);
    if (i + 4 < st1) acc = mfma_bf16_16x16x32(a1, b1, acc);
  }
  red[wave][lane] = make_float4(acc[0], acc[1], acc[2], acc[3]);
  __syncthreads();
  if (wave != 0) return;
  const float4 v0 = red[0][lane], v1 = red[1][lane], v2 = red[2][lane], v3 = red[3][lane];
  const float v[4] = {((v0.x + v1.x) + v2.x) + v3.x, ((v0.y + v1.y) + v2.y) + v3.y, ((v0.z + v1.z) + v2.z) + v3.z,
                      ((v0.w + v1.w) + v2.w) + v3.w};
  const int e = e0 + nl;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = t0 + 4 * g + r;
    if (t >= T) continue;
    if (gate_blk) {
      if (nl == 0) gpart[(int64_t)sl * T + t] = v[r];
    } else if (e < E) {
      part[((int64_t)sl * T + t) * E + e] = v[r];
    }
  }
}

// Block-wide exclusive scan of one int per thread (256 threads); returns the exclusive prefix, *total the sum.
__device__ __forceinline__ int block_exclusive_scan256(int v, int* s_tmp, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int x = __shfl_up(incl, o, 64);
    if (lane >= o) incl += x;
  }
  if (lane == 63 && wave < 4) s_tmp[wave] = incl;  // wider workgroups: only threads 0 .. 255 take part
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave && w < 4; ++w) base += s_tmp[w];
  *total = s_tmp[0] + s_tmp[1] + s_tmp[2] + s_tmp[3];
  __syncthreads();
  return base + incl - v;
}

// ---------------------------------------------------------------------------------------------
// Decode expert streaming. A workgroup owns one slot (an active expert, or the shared expert) and a run of
// 16-row weight tiles; the slot's gathered activation rows (8 or 16 per pass) are staged in LDS once, and every wave
// then streams its own tiles over the full K with the next batch of 16-byte weight units in flight while the
// current one feeds the MFMAs: no cross-wave reduction and no barrier inside the stream.
//
// The pairs are grouped by the streaming workgroups themselves (no grouping launch): each reads the T K top-K ids
// once, marks the active experts in an LDS bitmap, takes the slot-th active expert in ascending id order, and ranks
// that expert's pairs in pair order (token order: a token's K experts are distinct) by ballots. An id outside [0, E)
// selects no expert. Activations and routed outputs are indexed by pair.
// ---------------------------------------------------------------------------------------------
#ifndef AXK_SW
#define AXK_SW 4
#endif
constexpr int kStreamWaves = AXK_SW;
#ifndef AXK_BC
#define AXK_BC 2
#endif
#ifndef AXK_ROWS
#define AXK_ROWS 16
#endif
constexpr int kBatchChunks = AXK_BC;  // 128-wide K chunks per streamed batch (each lane: one unit per chunk)
constexpr int kStageRows = AXK_ROWS;  // activation rows staged per pass (MFMA rows past it are zero)
#ifndef AXK_GU_TPW
#define AXK_GU_TPW 1
#endif
#ifndef AXK_DN_TPW
#define AXK_DN_TPW 4
#endif
#ifndef AXK_GU_NB
#define AXK_GU_NB 3
#endif
#ifndef AXK_DN_NB
#define AXK_DN_NB 3
#endif
constexpr int kGateUpTilesPerWave = AXK_GU_TPW;  // 16-row tiles each wave streams (gate-up / down)
constexpr int kDownTilesPerWave = AXK_DN_TPW;
constexpr int kGateUpBufs = AXK_GU_NB;  // weight batches in rotation per wave (NB - 1 in flight while one is used)
constexpr int kDownBufs = AXK_DN_NB;
constexpr int kStageLd = 64 * kBatchChunks + 16;    // bytes per staged weight row segment of a batch (+16 pad)
constexpr int kWaveStageBytes = 32 * kStageLd;      // a wave's LDS tile: gate and up, 16 rows each
constexpr int kStageLpr = 4 * kBatchChunks;         // staged loads: lanes per row segment,
constexpr int kStageRpi = 64 / kStageLpr;           // rows per load instruction (kBatchChunks instructions a tile)
constexpr int kSmallRows = 8;                       // activation rows per pass of the staged kernels
constexpr int kStreamThreads = 64 * kStreamWaves;
// byte offset of the wave tiles after the activation rows ([rows][K + 8] bf16), 16-byte aligned
__host__ __device__ inline size_t stream_stage_off(int rows, int K) { return ((size_t)rows * (K + 8) * 2 + 15) & ~(size_t)15; }

// A routed slot's grouping in LDS.
struct SlotLds {
  unsigned long long act[kMaxExperts / 64];  // active experts
  int pair[kDecodeTokens];                  // the expert's pairs in pair order (at most one per token)
  int wcnt[kStreamWaves];
};
static_assert(sizeof(SlotLds) + kMaxStreamLds <= 160 * 1024, "streaming LDS over the CU's 160 KiB");

// The slot-th active expert (ascending id), or -1 past the last. id0: the id of pair threadIdx.x (when < P), kept
// for decode_rank_rows.
AXK_DEV int decode_find_expert(const int32_t* __restrict__ ids, int P, int E, int slot, SlotLds& L, int& id0) {
  const int tid = threadIdx.x;
  id0 = ids[min(tid, P - 1)];
  for (int i = tid; i < kMaxExperts / 64; i += kStreamThreads) L.act[i] = 0ull;
  __syncthreads();
  if (tid < P && id0 >= 0 && id0 < E) atomicOr(&L.act[id0 >> 6], 1ull << (id0 & 63));
#pragma unroll 4
  for (int p = tid + kStreamThreads; p < P; p += kStreamThreads) {
    const int e = ids[p];
    if (e >= 0 && e < E) atomicOr(&L.act[e >> 6], 1ull << (e & 63));
  }
  __syncthreads();
  int base = 0;
  for (int wd = 0; wd < (E + 63) / 64; ++wd) {  // uniform
    unsigned long long m = L.act[wd];
    const int c = __popcll(m);
    if (slot < base + c) {  // the r-th set bit of m, by halving
      int r = slot - base, pos = 0;
#pragma unroll
      for (int h = 32; h >= 1; h >>= 1) {
        const int cl = __popcll(m & ((1ull << h) - 1ull));
        if (r >= cl) {
          r -= cl;
          m >>= h;
          pos += h;
        }
      }
      return wd * 64 + pos;
    }
    base += c;
  }
  return -1;
}

// Expert e's pairs in pair order into L.pair; returns their count. Past the first kStreamThreads pairs (id0) the ids
// are read again (L2 hits). A token's K ids are distinct (top-K), so an expert has at most T <= kDecodeTokens pairs;
// rows past that bound (repeated ids) are dropped. Ends with a barrier.
AXK_DEV int decode_rank_rows(const int32_t* __restrict__ ids, int P, int e, int id0, SlotLds& L) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int cnt = 0;
  for (int p0 = 0; p0 < P; p0 += kStreamThreads) {  // uniform
    const int p = p0 + tid;
    const bool hit = p < P && (p0 == 0 ? id0 : ids[min(p, P - 1)]) == e;
    const unsigned long long b = __ballot(hit);
    if (lane == 0) L.wcnt[wave] = __popcll(b);
    __syncthreads();
    int before = cnt, tot = cnt;
#pragma unroll
    for (int w = 0; w < kStreamWaves; ++w) {
      const int c = L.wcnt[w];
      before += w < wave ? c : 0;
      tot += c;
    }
    const int r = before + __popcll(b & ((1ull << lane) - 1ull));
    if (hit && r < kDecodeTokens) L.pair[r] = p;  // more rows than tokens needs repeated ids within a token
    cnt = tot;
    __syncthreads();
  }
  return min(cnt, kDecodeTokens);
}

// Stage activation rows [m0, m0 + ROWS) of the slot into LDS as [ROWS][K + 8] bf16 (rows past cnt are skipped).
// Source row of row m: idx[m] / div (gathered), or m.
template <int ROWS>
__device__ void stage_rows(uint16_t* sA, const uint16_t* __restrict__ src, const int* idx, int div, int m0, int cnt,
                           int K) {
  const int ld = K + 8, units = K / 8;
  const int rows = min(ROWS, cnt - m0);
  for (int i = threadIdx.x; i < rows * units; i += blockDim.x) {
    const int r = i / units, u = i - r * units;
    const int64_t srow = idx ? idx[m0 + r] / div : (int64_t)(m0 + r);
    *reinterpret_cast<uint4*>(sA + r * ld + 8 * u) = *reinterpret_cast<const uint4*>(src + srow * K + 8 * u);
  }
}

// A batch's E8M0 scales of one weight row when K % (128 kBatchChunks) == 0: kBatchChunks consecutive words,
// word j holding chunk j's four lane-group scales (byte g).
AXK_DEV void load_scale_words(uint32_t (&w)[kBatchChunks], const uint8_t* p) {
  static_assert(kBatchChunks == 4 || kBatchChunks == 2, "batch of 2 or 4 chunks");
  if constexpr (kBatchChunks == 4) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    w[0] = v.x; w[1] = v.y;
  }
}

struct GateUpArgs {
  const uint16_t* h2;  // [T, H]
  const uint8_t *e_gw, *e_gs;
  const uint8_t *sg_w, *sg_s, *su_w, *su_s;  // shared gate / up (nullable: no shared expert)
  const int32_t* ids;  // [T, K] top-K expert ids
  int T, H, F, Fs, E, K, ngrp, tpw;          // tpw: tiles per wave; ngrp: workgroups per slot
  int nsp;                                   // grid slots of the shared expert (ROWS tokens each)
  MoeWs w;
};

// gate-up + SwiGLU: workgroup (slot, ngrp-th run of kStreamWaves * tpw tiles); wave w streams tiles
// run + w + kStreamWaves i.
// WIDE (K a multiple of the batch's 128 kBatchChunks values): a batch's E8M0 scales are 4 kBatchChunks
// consecutive bytes of the row (chunks x lane groups), fetched with one load per matrix; otherwise one byte load
// per unit.
// STAGE (with WIDE): each batch's weights are loaded as whole row segments of 64 kBatchChunks bytes (16 / kBatchChunks
// rows per load instruction, which keeps the address path's per-line work low), written to a wave-private LDS tile
// and read back in the MFMA layout; ROWS activation rows per pass.
template <bool WIDE, int ROWS, bool STAGE>
__global__ __launch_bounds__(kStreamThreads) void moe_gateup_kernel(GateUpArgs a) {
  static_assert(!STAGE || WIDE, "staged weights need whole batches");
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ SlotLds L;
  uint16_t* sA = reinterpret_cast<uint16_t*>(smem);
  unsigned char* sW = smem + stream_stage_off(ROWS, a.H) + (threadIdx.x >> 6) * kWaveStageBytes;
  // grid slots [0, nsp): the shared expert, ROWS tokens each (first, so the shared rows start early);
  // slot s >= nsp: active expert s - nsp
  const int gslot = blockIdx.x / a.ngrp, grp = blockIdx.x - gslot * a.ngrp;
  const bool shared = gslot < a.nsp;
  const int Fo = shared ? a.Fs : a.F;
  const int ntiles = (Fo + 15) / 16;
  const int tb = grp * kStreamWaves * a.tpw;
  if (tb >= ntiles) return;
  const int P = a.T * a.K;
  int cnt, mbeg = 0, eid = -1, id0 = -1;
  const uint8_t *gw, *gs, *uw, *us;
  if (shared) {
    mbeg = gslot * ROWS;
    cnt = min(a.T, mbeg + ROWS);
    gw = a.sg_w; gs = a.sg_s; uw = a.su_w; us = a.su_s;
  } else {
    const int e = decode_find_expert(a.ids, P, a.E, gslot - a.nsp, L, id0);
    if (e < 0) return;  // past the active experts (uniform)
    eid = e;
    cnt = -1;           // ranked in the first pass, behind the first weight loads
    const int64_t rows = 2 * (int64_t)a.F;
    gw = a.e_gw + e * rows * (a.H / 2);
    gs = a.e_gs + e * rows * (a.H / 32);
    uw = gw + (int64_t)a.F * (a.H / 2);
    us = gs + (int64_t)a.F * (a.H / 32);
  }
  // the wave index as a scalar: the step count and the past-the-end test derived from it stay uniform, so the
  // look-ahead loads select their address instead of branching around the load
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nl = lane & 15,
            g = lane >> 4;
  const int H = a.H, ldA = H + 8;
  const int nc = (H + 127) / 128, nb = (nc + kBatchChunks - 1) / kBatchChunks;  // chunks, batches per tile
  // this wave's tiles: tb + wave + kStreamWaves i, i < nmine
  const int nmine = max(0, min(a.tpw, (ntiles - tb - wave + kStreamWaves - 1) / kStreamWaves));
  const int steps = nmine * nb;

  struct Batch {  // native vectors: arrays of them stay in registers
    axk_u32x4 qg[kBatchChunks], qu[kBatchChunks];  // STAGE: [h] = rows kStageRpi h + lane / kStageLpr
    uint32_t sg[kBatchChunks], su[kBatchChunks];
  };
  // Loads are unconditional, from addresses clamped into the weights (a row past Fo is never stored, a unit past
  // K is zeroed where it is used): a branch around a load would make every later wait drain the queue. Steps past
  // the wave's last (the look-ahead at the end of its stream) load the first bytes of h2, already in L2 from the
  // row staging, instead of repeating the last weight batch: those non-temporal re-reads missed L2 and came from
  // HBM again. Each such load takes its own 16-byte unit: two loads of one address are merged by the compiler
  // into one load and a register copy, and the copy waits for the whole load queue.
  const uint8_t* idle = reinterpret_cast<const uint8_t*>(a.h2);
  auto load_batch = [&](Batch& bt, int step) {
    const bool past = step >= steps;  // wave-uniform
    step = min(step, max(steps - 1, 0));
    const int i = step / nb, bi = step - i * nb;
    const int64_t n = min((int64_t)(tb + wave + kStreamWaves * i) * 16 + nl, (int64_t)Fo - 1);
    if (STAGE) {
#pragma unroll
      for (int h = 0; h < kBatchChunks; ++h) {
        const int64_t r = min((int64_t)(tb + wave + kStreamWaves * i) * 16 + kStageRpi * h + lane / kStageLpr,
                              (int64_t)Fo - 1);
        const int64_t off = (int64_t)bi * (64 * kBatchChunks) + 16 * (lane % kStageLpr);
        bt.qg[h] = load_nt(past ? idle + 32 * h : gw + r * (H / 2) + off);  // expert weights: read once per step
        bt.qu[h] = load_nt(past ? idle + 32 * h + 16 : uw + r * (H / 2) + off);
      }
    } else {
#pragma unroll
      for (int j = 0; j < kBatchChunks; ++j) {
        const int64_t kb = min((int64_t)(bi * kBatchChunks + j) * 128 + 32 * g, (int64_t)H - 32);
        bt.qg[j] = load_nt(past ? idle + 32 * j : gw + n * (H / 2) + kb / 2);
        bt.qu[j] = load_nt(past ? idle + 32 * j + 16 : uw + n * (H / 2) + kb / 2);
        if (!WIDE) {
          bt.sg[j] = gs[n * (H / 32) + kb / 32];
          bt.su[j] = us[n * (H / 32) + kb / 32];
        }
      }
    }
    if (WIDE) {
      load_scale_words(bt.sg, gs + n * (H / 32) + 4 * kBatchChunks * bi);
      load_scale_words(bt.su, us + n * (H / 32) + 4 * kBatchChunks * bi);
    }
  };

  int m0 = mbeg;
  do {
    axk_f32x4 accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
    auto proc = [&](const Batch& cur, int st) {
      const int i = st / nb, bi = st - i * nb;
      axk_u32x4 wg[kBatchChunks], wu[kBatchChunks];  // this lane's MFMA units of the batch
      if (STAGE) {  // through the wave's LDS tile [gate, up][16 rows][kStageLd] (in-order LDS: no barrier)
#pragma unroll
        for (int h = 0; h < kBatchChunks; ++h) {
          const int r = kStageRpi * h + lane / kStageLpr;
          *reinterpret_cast<axk_u32x4*>(sW + r * kStageLd + 16 * (lane % kStageLpr)) = cur.qg[h];
          *reinterpret_cast<axk_u32x4*>(sW + (16 + r) * kStageLd + 16 * (lane % kStageLpr)) = cur.qu[h];
        }
#pragma unroll
        for (int j = 0; j < kBatchChunks; ++j) {
          wg[j] = *reinterpret_cast<const axk_u32x4*>(sW + nl * kStageLd + 64 * j + 16 * g);
          wu[j] = *reinterpret_cast<const axk_u32x4*>(sW + (16 + nl) * kStageLd + 64 * j + 16 * g);
        }
      } else {
#pragma unroll
        for (int j = 0; j < kBatchChunks; ++j) {
          wg[j] = cur.qg[j];
          wu[j] = cur.qu[j];
        }
      }
#pragma unroll
      for (int j = 0; j < kBatchChunks; ++j) {
        const int c = bi * kBatchChunks + j;
        if (!WIDE && c * 128 >= H) continue;  // whole chunk past K (uniform)
        const int kb = c * 128 + 32 * g;
        const bool kv = WIDE || kb < H;       // this lane's unit (a chunk can straddle the end of K)
        const int kc = kv ? kb : H - 32;
        const uint32_t bg = WIDE ? (cur.sg[j] >> (8 * g)) & 0xffu : cur.sg[j];
        const uint32_t bu = WIDE ? (cur.su[j] >> (8 * g)) & 0xffu : cur.su[j];
        const float scg = kv ? e8m0_to_f32(bg) : 0.f, scu = kv ? e8m0_to_f32(bu) : 0.f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          // only lanes of staged rows read (LDS bandwidth); the other MFMA rows are zero and never stored
          const axk_bf16x8 af = (kv && nl < ROWS) ? load_bf16x8(sA + nl * ldA + kc + 8 * s) : zero_bf16x8();
          accg = mfma_bf16_16x16x32(af, axk::WUnit<WF_MXFP4>::conv(__builtin_bit_cast(uint4, wg[j]), s, scg), accg);
          accu = mfma_bf16_16x16x32(af, axk::WUnit<WF_MXFP4>::conv(__builtin_bit_cast(uint4, wu[j]), s, scu), accu);
        }
      }
      if (bi == nb - 1) {  // tile done: SwiGLU of rows m0 + 4 g + r, column tile * 16 + nl
        const int col = (tb + wave + kStreamWaves * i) * 16 + nl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + 4 * g + r;
          if (4 * g + r < ROWS && m < cnt && col < Fo) {
            const float gv = round_bf16(accg[r]), uv = round_bf16(accu[r]);
            const uint16_t act = (uint16_t)f32_to_bf16_bits(silu_f32(gv) * uv);
            if (shared)
              a.w.act_sh[(int64_t)m * a.Fs + col] = act;
            else
              a.w.act[(int64_t)L.pair[m] * a.F + col] = act;  // by pair
          }
        }
        accg = accu = axk_f32x4{0.f, 0.f, 0.f, 0.f};
      }
    };
    // NB batches in rotation: batch st + NB - 1 is loaded while batch st is used. The first two are issued
    // before the activation rows are ranked and staged, so they overlap the slot's grouping and row gathers; the
    // rest after the gathers (whose in-order wait would otherwise take them all)
    constexpr int NB = kGateUpBufs, NPRE = NB - 1 < 2 ? NB - 1 : 2;
    Batch bt[NB];
    __syncthreads();  // the previous pass's readers are done with sA
#pragma unroll
    for (int j = 0; j < NPRE; ++j) load_batch(bt[j], j);
    if (cnt < 0) cnt = decode_rank_rows(a.ids, P, eid, id0, L);
    if (shared)
      stage_rows<ROWS>(sA, a.h2, nullptr, 1, m0, cnt, H);
    else
      stage_rows<ROWS>(sA, a.h2, L.pair, a.K, m0, cnt, H);  // token = pair / K
#pragma unroll
    for (int j = NPRE; j < NB - 1; ++j) load_batch(bt[j], j);
    __syncthreads();
    for (int st = 0; st < steps; st += NB) {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        load_batch(bt[(j + NB - 1) % NB], st + j + NB - 1);
        if (st + j < steps) proc(bt[j], st + j);
      }
    }
    m0 += ROWS;
  } while (m0 < cnt);
}

struct DownArgs {
  const uint8_t *e_dw, *e_ds;
  const uint8_t *sd_w, *sd_s;
  const int32_t* ids;  // [T, K]
  const float* wts;    // [T, K] routing weights
  int T, H, F, Fs, E, K, ngrp, tpw, nsp;
  MoeWs w;
};

// down: workgroup (slot, run of kStreamWaves * tpw 16-row tiles of H); routed rows scaled by their routing weight.
template <bool WIDE, int ROWS, bool STAGE>
__global__ __launch_bounds__(kStreamThreads) void moe_down_kernel(DownArgs a) {
  static_assert(!STAGE || WIDE, "staged weights need whole batches");
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ SlotLds L;
  uint16_t* sA = reinterpret_cast<uint16_t*>(smem);
  unsigned char* sW = smem + stream_stage_off(ROWS, a.Fs > a.F ? a.Fs : a.F) + (threadIdx.x >> 6) * kWaveStageBytes;
  const int gslot = blockIdx.x / a.ngrp, grp = blockIdx.x - gslot * a.ngrp;
  const bool shared = gslot < a.nsp;
  const int ntiles = (a.H + 15) / 16;
  const int tb = grp * kStreamWaves * a.tpw;
  if (tb >= ntiles) return;
  const int P = a.T * a.K;
  int cnt, K, mbeg = 0, eid = -1, id0 = -1;
  const uint8_t *dw, *ds;
  const uint16_t* act;
  if (shared) {
    mbeg = gslot * ROWS;
    cnt = min(a.T, mbeg + ROWS);
    K = a.Fs;
    dw = a.sd_w; ds = a.sd_s;
    act = a.w.act_sh;
  } else {
    const int e = decode_find_expert(a.ids, P, a.E, gslot - a.nsp, L, id0);
    if (e < 0) return;
    eid = e;
    cnt = -1;
    K = a.F;
    dw = a.e_dw + e * (int64_t)a.H * (a.F / 2);
    ds = a.e_ds + e * (int64_t)a.H * (a.F / 32);
    act = a.w.act;
  }
  // the wave index as a scalar: the step count and the past-the-end test derived from it stay uniform, so the
  // look-ahead loads select their address instead of branching around the load
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nl = lane & 15,
            g = lane >> 4;
  const int ldA = K + 8;
  const int nc = (K + 127) / 128, nb = (nc + kBatchChunks - 1) / kBatchChunks;
  const int nmine = max(0, min(a.tpw, (ntiles - tb - wave + kStreamWaves - 1) / kStreamWaves));
  const int steps = nmine * nb;

  struct Batch {  // native vectors: arrays of them stay in registers
    axk_u32x4 q[kBatchChunks];  // STAGE: [h] = rows kStageRpi h + lane / kStageLpr of the batch
    uint32_t s[kBatchChunks];
  };
  // unconditional, clamped, and past the wave's last step from the slot's first activation bytes (as in the
  // gate-up kernel)
  const uint8_t* idle = reinterpret_cast<const uint8_t*>(act);
  auto load_batch = [&](Batch& bt, int step) {
    const bool past = step >= steps;  // wave-uniform
    step = min(step, max(steps - 1, 0));
    const int i = step / nb, bi = step - i * nb;
    const int64_t n = min((int64_t)(tb + wave + kStreamWaves * i) * 16 + nl, (int64_t)a.H - 1);
    if (STAGE) {
#pragma unroll
      for (int h = 0; h < kBatchChunks; ++h) {
        const int64_t r = min((int64_t)(tb + wave + kStreamWaves * i) * 16 + kStageRpi * h + lane / kStageLpr,
                              (int64_t)a.H - 1);
        bt.q[h] = load_nt(past ? idle + 16 * h
                                : dw + r * (K / 2) + (int64_t)bi * (64 * kBatchChunks) + 16 * (lane % kStageLpr));
      }
    } else {
#pragma unroll
      for (int j = 0; j < kBatchChunks; ++j) {
        const int64_t kb = min((int64_t)(bi * kBatchChunks + j) * 128 + 32 * g, (int64_t)K - 32);
        bt.q[j] = load_nt(past ? idle + 16 * j : dw + n * (K / 2) + kb / 2);
        if (!WIDE) bt.s[j] = ds[n * (K / 32) + kb / 32];
      }
    }
    if (WIDE) load_scale_words(bt.s, ds + n * (K / 32) + 4 * kBatchChunks * bi);
  };

  int m0 = mbeg;
  do {
    constexpr int NB = kDownBufs, NPRE = NB - 1 < 2 ? NB - 1 : 2;  // as in the gate-up kernel
    Batch bt[NB];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NPRE; ++j) load_batch(bt[j], j);
    if (cnt < 0) cnt = decode_rank_rows(a.ids, P, eid, id0, L);
    if (shared)
      stage_rows<ROWS>(sA, act, nullptr, 1, m0, cnt, K);
    else
      stage_rows<ROWS>(sA, act, L.pair, 1, m0, cnt, K);  // activation rows by pair
    float rw[4];
    int pr[4];  // the rows' pair indices (y is indexed by pair); their routing weights are used after the stream
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = min(m0 + 4 * g + r, max(cnt - 1, 0));
      pr[r] = shared ? 0 : L.pair[m];
      rw[r] = shared ? 1.0f : a.wts[pr[r]];
    }
#pragma unroll
    for (int j = NPRE; j < NB - 1; ++j) load_batch(bt[j], j);
    __syncthreads();
    axk_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    auto proc = [&](const Batch& cur, int st) {
      const int i = st / nb, bi = st - i * nb;
      axk_u32x4 wq[kBatchChunks];
      if (STAGE) {  // through the wave's LDS tile [16 rows][kStageLd] (in-order LDS: no barrier)
#pragma unroll
        for (int h = 0; h < kBatchChunks; ++h)
          *reinterpret_cast<axk_u32x4*>(sW + (kStageRpi * h + lane / kStageLpr) * kStageLd + 16 * (lane % kStageLpr)) =
              cur.q[h];
#pragma unroll
        for (int j = 0; j < kBatchChunks; ++j)
          wq[j] = *reinterpret_cast<const axk_u32x4*>(sW + nl * kStageLd + 64 * j + 16 * g);
      } else {
#pragma unroll
        for (int j = 0; j < kBatchChunks; ++j) wq[j] = cur.q[j];
      }
#pragma unroll
      for (int j = 0; j < kBatchChunks; ++j) {
        const int c = bi * kBatchChunks + j;
        if (!WIDE && c * 128 >= K) continue;
        const int kb = c * 128 + 32 * g;
        const bool kv = WIDE || kb < K;
        const int kc = kv ? kb : K - 32;
        const uint32_t sb = WIDE ? (cur.s[j] >> (8 * g)) & 0xffu : cur.s[j];
        const float sc = kv ? e8m0_to_f32(sb) : 0.f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          acc = mfma_bf16_16x16x32((kv && nl < ROWS) ? load_bf16x8(sA + nl * ldA + kc + 8 * s) : zero_bf16x8(),
                                   axk::WUnit<WF_MXFP4>::conv(__builtin_bit_cast(uint4, wq[j]), s, sc), acc);
        }
      }
      if (bi == nb - 1) {
        const int64_t col = (int64_t)(tb + wave + kStreamWaves * i) * 16 + nl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + 4 * g + r;
          if (4 * g + r < ROWS && m < cnt && col < a.H) {
            if (shared)
              a.w.y_sh[(int64_t)m * a.H + col] = acc[r];
            else
              a.w.y[(int64_t)pr[r] * a.H + col] = acc[r] * rw[r];
          }
        }
        acc = axk_f32x4{0.f, 0.f, 0.f, 0.f};
      }
    };
    for (int st = 0; st < steps; st += NB) {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        load_batch(bt[(j + NB - 1) % NB], st + j + NB - 1);
        if (st + j < steps) proc(bt[j], st + j);
      }
    }
    m0 += ROWS;
  } while (m0 < cnt);
}

// ---------------------------------------------------------------------------------------------
// combine
// ---------------------------------------------------------------------------------------------
struct CombineArgs {
  const uint16_t* h2;     // [T, H]
  const uint16_t* x_res;  // [T, H] or null
  const uint16_t* w_shg;  // [H] or null (gate = 1)
  const float* gate_logit;  // [T] h2 . w_shg from the decode router, or null (computed here)
  const int32_t* ids;       // [T, K] top-K expert ids
  int has_shared, T, H, E, K;
  MoeWs w;
  uint16_t* out;  // [T, H]
};

// Workgroup (token, block of columns), 4 columns per thread and pass: base = x_res + gate * y_sh, + the K routed
// rows in slot order (y is indexed by pair t K + k; a pair whose id is outside [0, E) selected nothing), one bf16
// rounding. A pass's loads (all KM routed rows, clamped to K) are issued together, before the shared-gate dot
// (h2 . w_shg, reduced across the workgroup) where the router did not already form it, so they share one memory
// round trip. Few tokens: one block per 1024 columns; many tokens: one block per token (the gate is then computed
// once per token). YB: the routed rows are bf16 (the prefill path's slot outputs), else fp32. KM: a bound on K.
template <bool YB, int KM>
__global__ __launch_bounds__(256) void moe_combine_kernel(CombineArgs a) {
  __shared__ float s_part[4];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = (int64_t)t * a.H, pair0 = (int64_t)t * a.K;
  bool sel[KM];  // pair k selected an expert (uniform over the workgroup)
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    const int e = a.ids[pair0 + min(k, a.K - 1)];
    sel[k] = k < a.K && e >= 0 && e < a.E;
  }
  auto gather = [&](int i, float4& acc, float4& ys) {
    acc = make_float4(0.f, 0.f, 0.f, 0.f);
    ys = acc;
    if (a.x_res) {
      const uint2 xv = *reinterpret_cast<const uint2*>(a.x_res + row + i);
      acc = make_float4(__uint_as_float(xv.x << 16), __uint_as_float(xv.x & 0xffff0000u),
                        __uint_as_float(xv.y << 16), __uint_as_float(xv.y & 0xffff0000u));
    }
    if (a.has_shared) ys = *reinterpret_cast<const float4*>(a.w.y_sh + row + i);
    float4 yv[KM];
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      const int64_t pr = pair0 + min(k, a.K - 1);
      if constexpr (YB) {
        const uint2 b = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(a.w.y) + pr * a.H + i);
        yv[k] = make_float4(__uint_as_float(b.x << 16), __uint_as_float(b.x & 0xffff0000u),
                            __uint_as_float(b.y << 16), __uint_as_float(b.y & 0xffff0000u));
      } else {
        yv[k] = *reinterpret_cast<const float4*>(a.w.y + pr * a.H + i);
      }
    }
#pragma unroll
    for (int k = 0; k < KM; ++k)
      if (sel[k]) {
        acc.x += yv[k].x; acc.y += yv[k].y; acc.z += yv[k].z; acc.w += yv[k].w;
      }
  };
  auto finish = [&](int i, float4 acc, const float4& ys, float gate) {
    acc.x += gate * ys.x; acc.y += gate * ys.y; acc.z += gate * ys.z; acc.w += gate * ys.w;
    *reinterpret_cast<uint2*>(a.out + row + i) = make_uint2(pack_bf16x2(acc.x, acc.y), pack_bf16x2(acc.z, acc.w));
  };
  const int step = 4 * blockDim.x * gridDim.y, i0 = blockIdx.y * 4 * blockDim.x + 4 * tid;
  float4 acc0, ys0;
  gather(min(i0, a.H - 4), acc0, ys0);
  const bool gated = a.has_shared && a.w_shg;
  float gate = 1.0f;
  if (gated && a.gate_logit) {
    gate = sigmoid_f32(a.gate_logit[t]);
  } else if (gated) {
    const uint16_t* hrow = a.h2 + row;
    float d = 0.f;
    for (int i = 8 * tid; i < a.H; i += 8 * blockDim.x) {
      const uint4 hv = *reinterpret_cast<const uint4*>(hrow + i);
      const uint4 wv = *reinterpret_cast<const uint4*>(a.w_shg + i);
      const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w}, ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
      for (int j = 0; j < 4; ++j)
        d += __uint_as_float(hw[j] << 16) * __uint_as_float(ww[j] << 16) +
             __uint_as_float(hw[j] & 0xffff0000u) * __uint_as_float(ww[j] & 0xffff0000u);
    }
    d = wave_sum(d);
    if (lane == 0) s_part[wave] = d;
    __syncthreads();
    gate = sigmoid_f32(s_part[0] + s_part[1] + s_part[2] + s_part[3]);
  }
  if (i0 < a.H) finish(i0, acc0, ys0, gate);
  for (int i = i0 + step; i < a.H; i += step) {
    float4 acc, ys;
    gather(i, acc, ys);
    finish(i, acc, ys, gate);
  }
}

// The combine launch: routed-row loads unrolled to a bound on K.
template <bool YB>
void launch_combine(const CombineArgs& ca, hipStream_t st) {
  const dim3 grid((unsigned)ca.T, (unsigned)(ca.T >= 1024 ? 1 : (ca.H + 1023) / 1024)), block(256);
  if (ca.K <= 8)
    hipLaunchKernelGGL((moe_combine_kernel<YB, 8>), grid, block, 0, st, ca);
  else
    hipLaunchKernelGGL((moe_combine_kernel<YB, kMaxTopK>), grid, block, 0, st, ca);
}

// ---------------------------------------------------------------------------------------------
// prefill grouping: 256-token blocks
// ---------------------------------------------------------------------------------------------
// Per-expert token bitmasks of block `blk` in LDS (4 words per expert); pairs with an id outside [0, E) are
// left out.
__device__ void block_masks(const int32_t* __restrict__ ids, int T, int E, int K, int blk,
                            unsigned long long* s_mask) {
  const int t0 = blk * kBlkTokens, nt = min(kBlkTokens, T - t0);
  for (int i = threadIdx.x; i < E * kMaskWords; i += blockDim.x) s_mask[i] = 0ull;
  __syncthreads();
  for (int p = threadIdx.x; p < nt * K; p += blockDim.x) {
    const int t = p / K, e = ids[(int64_t)t0 * K + p];
    if (e >= 0 && e < E) atomicOr(&s_mask[e * kMaskWords + (t >> 6)], 1ull << (t & 63));
  }
  __syncthreads();
}

__global__ __launch_bounds__(256) void moe_pcount_kernel(const int32_t* __restrict__ ids, int T, int E, int K,
                                                         MoeWs w) {
  __shared__ unsigned long long s_mask[kMaxExperts * kMaskWords];
  block_masks(ids, T, E, K, blockIdx.x, s_mask);
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int c = 0;
#pragma unroll
    for (int i = 0; i < kMaskWords; ++i) c += __popcll(s_mask[e * kMaskWords + i]);
    w.blk[(int64_t)blockIdx.x * E + e] = c;
  }
}

// One workgroup: expert totals, offsets and active list; per-(block, expert) row bases (in place of the
// counts); the GEMM tile list (routed experts in expert order, then the shared expert's tiles).
__global__ __launch_bounds__(256) void moe_pscan_kernel(int T, int E, int NB, int has_shared, MoeWs w) {
  __shared__ int s_tmp[12];
  constexpr int EPT = kMaxExperts / 256;
  const int tid = threadIdx.x;
  // the per-block counts are read in chunks of kChunk blocks for all of the thread's experts at once (independent
  // loads: one memory round trip per chunk, not one per block)
  constexpr int kChunk = 8;
  int cnt[EPT], sum = 0, nact = 0, ntile = 0;
#pragma unroll
  for (int j = 0; j < EPT; ++j) cnt[j] = 0;
  for (int b0 = 0; b0 < NB; b0 += kChunk) {
    int v[EPT][kChunk];
#pragma unroll
    for (int j = 0; j < EPT; ++j)
#pragma unroll
      for (int i = 0; i < kChunk; ++i) {
        const int e = tid * EPT + j, b = b0 + i;
        v[j][i] = (e < E && b < NB) ? w.blk[(int64_t)b * E + e] : 0;
      }
#pragma unroll
    for (int j = 0; j < EPT; ++j)
#pragma unroll
      for (int i = 0; i < kChunk; ++i) cnt[j] += v[j][i];
  }
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    sum += cnt[j];
    nact += cnt[j] > 0;
    ntile += (cnt[j] + kBM - 1) / kBM;
  }
  int tot, tota, tott;
  int off = block_exclusive_scan256(sum, s_tmp, &tot);
  int aoff = block_exclusive_scan256(nact, s_tmp + 4, &tota);
  int toff = block_exclusive_scan256(ntile, s_tmp + 8, &tott);
  int base[EPT];
  {
    int o = off;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      base[j] = o;
      o += cnt[j];
    }
  }
  // per-(block, expert) row bases in place of the counts, chunk by chunk as above
  for (int b0 = 0; b0 < NB; b0 += kChunk) {
    int v[EPT][kChunk];
#pragma unroll
    for (int j = 0; j < EPT; ++j)
#pragma unroll
      for (int i = 0; i < kChunk; ++i) {
        const int e = tid * EPT + j, b = b0 + i;
        v[j][i] = (e < E && b < NB) ? w.blk[(int64_t)b * E + e] : 0;
      }
#pragma unroll
    for (int j = 0; j < EPT; ++j)
#pragma unroll
      for (int i = 0; i < kChunk; ++i) {
        const int e = tid * EPT + j, b = b0 + i;
        if (e < E && b < NB) w.blk[(int64_t)b * E + e] = base[j];
        base[j] += v[j][i];
      }
  }
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int e = tid * EPT + j;
    if (e < E) {
      w.counts[e] = cnt[j];
      w.offsets[e] = off;
      if (cnt[j] > 0) {
        w.active[aoff] = make_int4(cnt[j], e, off, 0);
        ++aoff;
      }
      for (int r = 0; r < cnt[j]; r += kBM) w.tiles[toff++] = make_int4(e, off + r, min(kBM, cnt[j] - r), 0);
    }
    off += cnt[j];
  }
  const int nsh = has_shared ? (T + kBM - 1) / kBM : 0;
  for (int i = tid; i < nsh; i += blockDim.x) w.tiles[tott + i] = make_int4(-1, i * kBM, min(kBM, T - i * kBM), 0);
  if (tid == 0) {
    w.offsets[E] = tot;
    *w.n_active = tota;
    *w.n_tiles = tott + nsh;
  }
}

__global__ __launch_bounds__(256) void moe_pscatter_kernel(const int32_t* __restrict__ ids,
                                                           const float* __restrict__ wts, int T, int E, int K,
                                                           MoeWs w) {
  __shared__ unsigned long long s_mask[kMaxExperts * kMaskWords];
  const int blk = blockIdx.x, t0 = blk * kBlkTokens, nt = min(kBlkTokens, T - t0);
  block_masks(ids, T, E, K, blk, s_mask);
  for (int q = threadIdx.x; q < nt * K; q += blockDim.x) {
    const int64_t p = (int64_t)t0 * K + q;
    const int e = ids[p], t = q / K;
    if (e < 0 || e >= E) {
      w.pair_pos[p] = -1;
      continue;
    }
    const unsigned long long* m = s_mask + e * kMaskWords;
    int rank = __popcll(m[t >> 6] & ((1ull << (t & 63)) - 1ull));
    for (int i = 0; i < (t >> 6); ++i) rank += __popcll(m[i]);
    const int pos = w.blk[(int64_t)blk * E + e] + rank;
    w.pair_pos[p] = pos;
    w.row_tok[pos] = t0 + t;
    w.row_w[pos] = wts[p];
    w.row_pair[pos] = (int)p;
  }
}

// ---------------------------------------------------------------------------------------------
// prefill grouped GEMM: workgroup (tile of kBM rows of one expert, 256 weight rows), wave w a 64 x 64 block of
// the output (four 16-row x four 16-column MFMA tiles: every A fragment feeds four MFMAs and every B fragment
// four). MODE 0: weight rows = 128 gate + the same 128 up columns (SwiGLU pairs gate and up tiles in the same
// lanes); MODE 1: 256 columns of H.
// The A rows (gathered by token) and the packed weights of each 64-wide K step land in LDS by direct loads (no
// register staging) into a ring of kGStages steps, two steps ahead, with one barrier per step; the E8M0 scales of
// the whole reduction are staged once per workgroup. A stage holds A [64 rows][128 B] with the 16-byte chunk c of
// row r at position c ^ (r & 7), and B [256 weight rows][32 B] with the 16-byte half h of row r at position
// h ^ ((r >> 3) & 1): the fragment reads of either are then free of bank conflicts. Workgroups are mapped so that
// all tiles and column blocks of one expert run on one XCD: its weights are fetched into that XCD's L2 once.
// SDMA (reductions of whole 128-element scale dwords, 4-byte aligned scales): each step's E8M0 bytes come with the
// step's direct loads, one dword per weight row, LDS kGStages x (A 8 KiB + B 8 KiB + 1 KiB), so three workgroups
// share a CU; otherwise the scales of the whole reduction are staged once, LDS kGStages x 16 KiB + [256][Kd/32 + 16].
// ---------------------------------------------------------------------------------------------
struct GGemmArgs {
  const uint16_t* a;     // gate-up: h2 [T, H]; down: act [P, F]
  const uint16_t* a_sh;  // down: act_sh [T, Fs]
  const uint8_t *w, *s;  // routed: gate-up e_gw / e_gs [E, 2F, H/2 | H/32]; down e_dw / e_ds [E, H, F/2 | F/32]
  const uint8_t *w_sh, *s_sh, *u_sh, *us_sh;  // shared: gate-up gate and up [Fs, H/2]; down [H, Fs/2] (w_sh, s_sh)
  int T, H, F, Fs, Fmax;  // Fmax = max(F, Fs): sets the gate-up column-block count
  MoeWs ws;
};

constexpr int kG2Rows = 256;          // weight rows per workgroup
constexpr int kG2Cols0 = kG2Rows / 2;  // gate-up: output (act) columns per workgroup
constexpr int kG2Cols1 = kG2Rows;      // down: output columns per workgroup
constexpr int kXcds = 8;              // MI355X: consecutive workgroups go round-robin over 8 XCDs
constexpr int kGStages = 3;
// rows per workgroup: the gate-up GEMM takes a whole kBM-row tile (each decoded weight fragment feeds 8 MFMAs); the
// down GEMM (K = F, a short reduction) a half tile, so twice the workgroups share its fixed costs
template <int MODE>
constexpr int g_bm() { return MODE == 0 ? kBM : kBM / 2; }
template <int MODE>
constexpr int g_astage() { return g_bm<MODE>() * kBK * 2; }
constexpr int kGBStage = kG2Rows * kBK / 2;  // 8 KiB
template <int MODE>
constexpr int g_stage() { return g_astage<MODE>() + kGBStage; }
constexpr int kGSStage = kG2Rows * 4;  // SDMA: one scale dword per weight row and step
template <int MODE>
size_t gemm_lds_bytes(int Kd, bool sdma) {
  return sdma ? (size_t)kGStages * (g_stage<MODE>() + kGSStage)
              : (size_t)kGStages * g_stage<MODE>() + (size_t)kG2Rows * (Kd / 32 + 16);
}

template <int MODE, bool SDMA>
__global__ __launch_bounds__(256, 2) void moe_ggemm_kernel(GGemmArgs g) {
  constexpr int BM = g_bm<MODE>(), SUB = kBM / BM;              // rows per workgroup, workgroups per tile
  constexpr int kGAStage = g_astage<MODE>(), kGStage = g_stage<MODE>();
  constexpr int kGAI = kGAStage / 1024 / 4;                        // A direct-load instructions per wave and step
  constexpr int kGMT = BM / 16;                                    // 16-row MFMA tiles per wave (all rows of the tile)
  constexpr int STAGE = kGStage + (SDMA ? kGSStage : 0);
  extern __shared__ __align__(16) unsigned char smem[];
  const int nblk = MODE == 0 ? (g.Fmax + kG2Cols0 - 1) / kG2Cols0 : (g.H + kG2Cols1 - 1) / kG2Cols1;
  const int total = *g.ws.n_tiles * SUB * nblk, per = (total + kXcds - 1) / kXcds;
  const int k = blockIdx.x / kXcds, lid = (blockIdx.x % kXcds) * per + k;
  if (k >= per || lid >= total) return;
  const int sub = lid / nblk, cblk = lid - sub * nblk, tile = sub / SUB, part = sub - tile * SUB;
  const int4 tl = g.ws.tiles[tile];
  const int e = tl.x, row0 = tl.y + part * BM, rows = min(BM, tl.z - part * BM);
  if (rows <= 0) return;
  const bool shared = e < 0;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;

  const int Kd = MODE == 0 ? g.H : (shared ? g.Fs : g.F);
  const int No = MODE == 0 ? (shared ? g.Fs : g.F) : g.H;
  const int col0 = cblk * (MODE == 0 ? kG2Cols0 : kG2Cols1);
  if (col0 >= No) return;
  const uint32_t lds0 = lds_addr(smem);
  unsigned char* sS = smem + kGStages * STAGE;  // whole-reduction scales (not SDMA)
  const int ldS = Kd / 32 + 16;
  const int nk = Kd / kBK;

  const uint8_t *wgate, *wup, *sgate, *sup;
  if (MODE == 0) {
    if (shared) {
      wgate = g.w_sh; wup = g.u_sh; sgate = g.s_sh; sup = g.us_sh;
    } else {
      const int64_t rows2 = 2 * (int64_t)g.F;
      wgate = g.w + (int64_t)e * rows2 * (g.H / 2);
      wup = wgate + (int64_t)g.F * (g.H / 2);
      sgate = g.s + (int64_t)e * rows2 * (g.H / 32);
      sup = sgate + (int64_t)g.F * (g.H / 32);
    }
  } else {
    wgate = wup = shared ? g.w_sh : g.w + (int64_t)e * g.H * (g.F / 2);
    sgate = sup = shared ? g.s_sh : g.s + (int64_t)e * g.H * (g.F / 32);
  }
  // LDS weight row rho -> weight row (gate-up: rho < 128 gate column col0 + rho, else up column col0 + rho - 128;
  // down: column col0 + rho), clamped to the last column (never stored)
  auto wrow = [&](int rho, bool scale) -> const uint8_t* {
    const bool up = MODE == 0 && rho >= kG2Cols0;
    const int c = min(col0 + (MODE == 0 ? (rho & (kG2Cols0 - 1)) : rho), No - 1);
    return scale ? (up ? sup : sgate) + (int64_t)c * (Kd / 32) : (up ? wup : wgate) + (int64_t)c * (Kd / 2);
  };

  // per-lane sources of this wave's two A and two B load instructions of a step (instruction i = 2 wave + h):
  // A: row 8 i + lane / 8 (rows past the tile re-read its last row, never stored), chunk (lane % 8) ^ (row & 7);
  // B: weight row 32 i + lane / 2, half (lane % 2) ^ ((row >> 3) & 1)
  const uint16_t* asrc[kGAI];
  const uint8_t* bsrc[2];
#pragma unroll
  for (int h = 0; h < kGAI; ++h) {
    const int i = kGAI * wave + h;
    const int r = 8 * i + (lane >> 3), rr = min(r, rows - 1), ch = (lane & 7) ^ (r & 7);
    if (MODE == 0) {
      const int tok = shared ? row0 + rr : g.ws.row_tok[row0 + rr];
      asrc[h] = g.a + (int64_t)tok * g.H + 8 * ch;
    } else {
      asrc[h] = (shared ? g.a_sh + (int64_t)(row0 + rr) * g.Fs : g.a + (int64_t)(row0 + rr) * g.F) + 8 * ch;
    }
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int rho = 32 * (2 * wave + h) + (lane >> 1);
    bsrc[h] = wrow(rho, false) + 16 * ((lane & 1) ^ ((rho >> 3) & 1));
  }
  // SDMA: wave w loads the aligned dword holding blocks 4 (ks / 2) .. + 3 of weight rows 64 w + lane
  const uint8_t* ssrc = SDMA ? wrow(64 * wave + lane, true) : nullptr;
  // step ks into ring slot buf; past the last step the last one is loaded again (in bounds, unused), so every
  // iteration waits on the same count
  auto issue = [&](int ks, int buf) {
    const int kk = min(ks, nk - 1);
    const uint32_t base = lds0 + buf * STAGE;
#pragma unroll
    for (int h = 0; h < kGAI; ++h) lds_dma16_cached(asrc[h] + kk * kBK, base + (kGAI * wave + h) * 1024);
#pragma unroll
    for (int h = 0; h < 2; ++h) lds_dma16_cached(bsrc[h] + kk * (kBK / 2), base + kGAStage + (2 * wave + h) * 1024);
    if constexpr (SDMA) lds_dma4_cached(ssrc + 4 * (kk >> 1), base + kGStage + 256 * wave);
  };
  issue(0, 0);
  issue(1, 1);

  // the E8M0 scales of the whole reduction (while the first steps load): 16-byte units when the row length
  // allows, else 2-byte units
  if constexpr (!SDMA) {
    const int sb = Kd / 32;
    if (sb % 16 == 0 && (((uintptr_t)sgate | (uintptr_t)sup) & 15) == 0) {
      const int u = sb / 16;
      for (int idx = tid; idx < kG2Rows * u; idx += 256) {
        const int rho = idx / u, q = idx - rho * u;
        *reinterpret_cast<uint4*>(sS + rho * ldS + 16 * q) = *reinterpret_cast<const uint4*>(wrow(rho, true) + 16 * q);
      }
    } else {
      const int u = sb / 2;
      for (int idx = tid; idx < kG2Rows * u; idx += 256) {
        const int rho = idx / u, q = idx - rho * u;
        *reinterpret_cast<uint16_t*>(sS + rho * ldS + 2 * q) = *reinterpret_cast<const uint16_t*>(wrow(rho, true) + 2 * q);
      }
    }
  }

  int brow[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    brow[j] = MODE == 0 ? (j >> 1) * kG2Cols0 + 32 * wave + 16 * (j & 1) : 64 * wave + 16 * j;

  axk_f32x4 acc[kGMT][4];
#pragma unroll
  for (int mt = 0; mt < kGMT; ++mt)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[mt][j] = axk_f32x4{0.f, 0.f, 0.f, 0.f};

  // step ks from ring slot BUF (a constant: the loop is unrolled over the ring, so every LDS offset is immediate)
  auto step = [&](int ks, auto buf_c) __attribute__((always_inline)) {
    constexpr int BUF = decltype(buf_c)::value;
    wait_vmcnt<kGAI + 2 + (SDMA ? 1 : 0)>();  // this wave's loads of step ks have landed (step ks + 1's may not)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's reads of step ks - 1 are done
    __builtin_amdgcn_s_barrier();  // every wave's step-ks loads landed; every wave is done with step ks - 1
    asm volatile("" ::: "memory");
    issue(ks + 2, (BUF + 2) % kGStages);  // into the slot of step ks - 1
    const unsigned char* sa = smem + BUF * STAGE;
    const unsigned char* sb = sa + kGAStage;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      axk_bf16x8 af[kGMT], bf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = brow[j] + l16;
        const uint32_t w = *reinterpret_cast<const uint32_t*>(sb + r * 32 + 16 * (kh ^ ((r >> 3) & 1)) + 4 * g4);
        // one E8M0 byte: two VALU to an fp32 scale
        const uint32_t sbyte = SDMA ? sb[kGBStage + 4 * r + 2 * (ks & 1) + kh] : sS[r * ldS + 2 * ks + kh];
        bf[j] = fp4x8_to_bf16x8(w, e8m0_to_f32(sbyte));
      }
#pragma unroll
      for (int mt = 0; mt < kGMT; ++mt) {
        const int r = 16 * mt + l16;
        af[mt] = *reinterpret_cast<const axk_bf16x8*>(sa + r * 128 + 16 * ((4 * kh + g4) ^ (r & 7)));
      }
#pragma unroll
      for (int mt = 0; mt < kGMT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[mt][j] = mfma_bf16_16x16x32(af[mt], bf[j], acc[mt][j]);
    }
  };
  static_assert(kGStages == 3, "the K loop is unrolled over three ring slots");
  for (int ks = 0; ks < nk; ks += 3) {
    step(ks, std::integral_constant<int, 0>{});
    if (ks + 1 < nk) step(ks + 1, std::integral_constant<int, 1>{});
    if (ks + 2 < nk) step(ks + 2, std::integral_constant<int, 2>{});
  }
  wait_vmcnt<0>();  // the look-ahead loads land before the workgroup's LDS is released

  // Epilogue. The bf16 outputs (gate-up: act / act_sh; down, routed: bf16(rw * y) by pair) go through an LDS tile
  // [BM rows][COLS + 8] over the ring, so that each row leaves as 16-byte stores of whole row segments instead of
  // 2-byte stores of 16 lanes; the shared expert's fp32 down rows are stored directly.
  constexpr int COLS = MODE == 0 ? kG2Cols0 : kG2Cols1, LDO = COLS + 8;
  const bool staged = MODE == 0 || !shared;
  uint16_t* so = reinterpret_cast<uint16_t*>(smem);
  if (staged) __syncthreads();  // every wave is done with the ring
#pragma unroll
  for (int mt = 0; mt < kGMT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * mt + 4 * g4 + r;
      const int64_t prow = row0 + row;
      if (MODE == 0) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float gv = round_bf16(acc[mt][j][r]), uv = round_bf16(acc[mt][j + 2][r]);
          so[row * LDO + 32 * wave + 16 * j + l16] =
              (uint16_t)f32_to_bf16_bits(gv * __builtin_amdgcn_rcpf(1.0f + __expf(-gv)) * uv);
        }
      } else if (!shared) {
        // a routed slot is stored as bf16(rw * y), as the reference's delivered slot kernels store it
        // (qwen35moe_slots*_bo: SLOT_OUT=bf16, q35_moe_prefill.py:41, 100, 165) and its combine reads it
        const float rw = row < rows ? g.ws.row_w[prow] : 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          so[row * LDO + 64 * wave + 16 * j + l16] = (uint16_t)f32_to_bf16_bits(acc[mt][j][r] * rw);
      } else {
        if (row >= rows) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int col = col0 + 64 * wave + 16 * j + l16;
          if (col < No) g.ws.y_sh[prow * g.H + col] = acc[mt][j][r];
        }
      }
    }
  if (!staged) return;
  __syncthreads();
  // row segments of 8 columns: thread t takes segments t, t + 256, ...; 16-byte stores where the output rows are
  // 16-byte aligned (row lengths a multiple of 8)
  constexpr int SPR = COLS / 8;  // segments per row
  const bool vec = (MODE == 0 ? (shared ? g.Fs : g.F) : g.H) % 8 == 0;
#pragma unroll
  for (int i = 0; i < BM * SPR / 256; ++i) {
    const int sidx = tid + 256 * i, row = sidx / SPR, seg = sidx - row * SPR;
    if (row >= rows) continue;
    const int64_t prow = row0 + row;
    const int col = col0 + 8 * seg;
    uint16_t* dst;
    if (MODE == 0)
      dst = shared ? g.ws.act_sh + prow * g.Fs + col : g.ws.act + prow * g.F + col;
    else
      dst = reinterpret_cast<uint16_t*>(g.ws.y) + (int64_t)g.ws.row_pair[prow] * g.H + col;
    const uint16_t* src = so + row * LDO + 8 * seg;
    if (vec && col + 8 <= No) {
      *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
    } else {
      for (int e = 0; e < 8 && col + e < No; ++e) dst[e] = src[e];
    }
  }
}

struct MoeDims {
  int64_t T, H, E, K, F, Fs;
};

int check_dims(const MoeDims& d) {
  AXK_REQUIRE(d.T > 0 && d.H > 0 && d.E > 0 && d.K > 0 && d.F > 0, AXK_E_SHAPE);
  AXK_REQUIRE(d.E <= kMaxExperts && d.K <= kMaxTopK && d.K <= d.E, AXK_E_SHAPE);
  if (d.T <= kDecodeTokens) {
    AXK_REQUIRE(d.T * d.K <= kMaxPairs, AXK_E_SHAPE);
    AXK_REQUIRE(d.H % 64 == 0 && d.F % 32 == 0 && d.Fs % 32 == 0 && d.Fs >= 0, AXK_E_SHAPE);
  } else {  // prefill GEMM: whole 64-wide K steps and 64-column gate / up tiles
    AXK_REQUIRE(d.T <= kMaxPrefillTokens && d.T * d.K <= kMaxPrefillPairs, AXK_E_SHAPE);
    AXK_REQUIRE(d.H % 64 == 0 && d.F % 64 == 0 && d.Fs % 64 == 0 && d.Fs >= 0, AXK_E_SHAPE);
    AXK_REQUIRE(d.H <= 8192 && d.F <= 8192 && d.Fs <= 8192, AXK_E_SHAPE);  // whole-K scales staged in LDS
  }
  AXK_REQUIRE(d.H <= INT32_MAX && d.F <= INT32_MAX, AXK_E_SHAPE);
  return AXK_OK;
}

}  // namespace

extern "C" size_t axk_moe_workspace_size(int64_t tokens, int64_t hidden, int64_t num_experts, int64_t top_k,
                                         int64_t inter, int64_t shared_inter) {
  if (check_dims({tokens, hidden, num_experts, top_k, inter, shared_inter}) != AXK_OK) return 0;
  size_t off[kWsParts];
  return moe_ws_layout(tokens, hidden, num_experts, top_k, inter, shared_inter, off);
}

extern "C" int axk_moe_route(const float* logits, int32_t* topk_ids, float* topk_weights, int64_t tokens,
                             int64_t num_experts, int64_t top_k, int norm_topk_prob, axk_stream_t stream) {
  AXK_REQUIRE(logits && topk_ids && topk_weights, AXK_E_NULL);
  AXK_REQUIRE(tokens > 0 && num_experts > 0 && num_experts <= kMaxExperts, AXK_E_SHAPE);
  AXK_REQUIRE(top_k > 0 && top_k <= kMaxTopK && top_k <= num_experts && tokens <= INT32_MAX, AXK_E_SHAPE);
  const dim3 grid((unsigned)((tokens + 3) / 4)), block(256);
  const int T = (int)tokens, E = (int)num_experts, K = (int)top_k;
  hipStream_t st = axk_stream(stream);
  if (E <= 64)
    hipLaunchKernelGGL(moe_route_kernel<1>, grid, block, 0, st, logits, T, E, K, norm_topk_prob, topk_ids, topk_weights);
  else if (E <= 256)
    hipLaunchKernelGGL(moe_route_kernel<4>, grid, block, 0, st, logits, T, E, K, norm_topk_prob, topk_ids, topk_weights);
  else
    hipLaunchKernelGGL(moe_route_kernel<kMaxExperts / 64>, grid, block, 0, st, logits, T, E, K, norm_topk_prob,
                       topk_ids, topk_weights);
  return axk_launch_status();
}

namespace {
// The experts half. gate_given: the decode router formed the shared gate's logit in the workspace; check_only: run the
// contract checks and return before any launch. y_sh_given (optional, with no MXFP4 shared expert): the shared
// expert's fp32 output [T, H], computed by the caller; the combine gates and adds it as its own.
int moe_experts_impl(const uint16_t* h2, const uint16_t* x_res, const uint16_t* w_shg, const uint8_t* sh_gate_w,
                     const uint8_t* sh_gate_s, const uint8_t* sh_up_w, const uint8_t* sh_up_s,
                     const uint8_t* sh_down_w, const uint8_t* sh_down_s, const uint8_t* e_gw, const uint8_t* e_gs,
                     const uint8_t* e_dw, const uint8_t* e_ds, const int32_t* topk_ids, const float* topk_weights,
                     uint16_t* out, int64_t tokens, int64_t hidden, int64_t num_experts, int64_t top_k, int64_t inter,
                     int64_t shared_inter, void* workspace, size_t workspace_bytes, axk_stream_t stream, bool gate_given,
                     bool check_only, const float* y_sh_given = nullptr, bool counted = false) {
  AXK_REQUIRE(h2 && e_gw && e_gs && e_dw && e_ds && topk_ids && topk_weights && out, AXK_E_NULL);
  const bool has_shared = sh_gate_w != nullptr;
  AXK_REQUIRE(!has_shared || (sh_gate_s && sh_up_w && sh_up_s && sh_down_w && sh_down_s), AXK_E_NULL);
  AXK_REQUIRE(!(has_shared && y_sh_given), AXK_E_NULL);  // one shared expert or the other
  AXK_REQUIRE(!y_sh_given || axk_aligned(y_sh_given, 16), AXK_E_ALIGN);
  AXK_REQUIRE(!y_sh_given || !axk_overlap(y_sh_given, (size_t)tokens * hidden * 4, out, (size_t)tokens * hidden * 2),
              AXK_E_ALIAS);
  const MoeDims d{tokens, hidden, num_experts, top_k, inter, has_shared ? shared_inter : 0};
  const int rc = check_dims(d);
  if (rc != AXK_OK) return rc;
  AXK_REQUIRE(!has_shared || shared_inter > 0, AXK_E_SHAPE);
  AXK_REQUIRE(axk_aligned(h2, 16) && axk_aligned(e_gw, 16) && axk_aligned(e_dw, 16), AXK_E_ALIGN);
  AXK_REQUIRE((!w_shg || axk_aligned(w_shg, 16)) && (!x_res || axk_aligned(x_res, 8)), AXK_E_ALIGN);
  AXK_REQUIRE(!has_shared || (axk_aligned(sh_gate_w, 16) && axk_aligned(sh_up_w, 16) && axk_aligned(sh_down_w, 16)),
              AXK_E_ALIGN);
  const size_t need = axk_moe_workspace_size(tokens, hidden, num_experts, top_k, inter, d.Fs);
  AXK_REQUIRE(workspace && workspace_bytes >= need && axk_aligned(workspace, 256), AXK_E_WORKSPACE);
  const size_t obytes = (size_t)tokens * hidden * 2;
  AXK_REQUIRE(!axk_overlap(out, obytes, h2, obytes) && !axk_overlap(out, obytes, workspace, workspace_bytes),
              AXK_E_ALIAS);
  if (check_only) return AXK_OK;
  hipStream_t st = axk_stream(stream);
  MoeWs w = moe_ws(workspace, tokens, hidden, num_experts, top_k, inter, d.Fs);
  if (y_sh_given) w.y_sh = const_cast<float*>(y_sh_given);  // read only (by the combine)
  const int combine_shared = (has_shared || y_sh_given) ? 1 : 0;
  const int T = (int)tokens, H = (int)hidden, E = (int)num_experts, K = (int)top_k, F = (int)inter, Fs = (int)d.Fs;
  if (T > kDecodeTokens) {
    const int NB = (int)prefill_blocks(T);
    // the (block, expert) counts: counted by the routing launch when it ran in this call, else from the ids
    if (!counted) hipLaunchKernelGGL(moe_pcount_kernel, dim3((unsigned)NB), dim3(256), 0, st, topk_ids, T, E, K, w);
    hipLaunchKernelGGL(moe_pscan_kernel, dim3(1), dim3(256), 0, st, T, E, NB, has_shared ? 1 : 0, w);
    hipLaunchKernelGGL(moe_pscatter_kernel, dim3((unsigned)NB), dim3(256), 0, st, topk_ids, topk_weights, T, E, K, w);
    const unsigned tiles = (unsigned)prefill_max_tiles(T, E, K);
    const int fmax = F > Fs ? F : Fs;
    GGemmArgs gu{h2, nullptr, e_gw, e_gs, sh_gate_w, sh_gate_s, sh_up_w, sh_up_s, T, H, F, Fs, fmax, w};
    // per-step scale dwords (SDMA) where every scale row of the reduction is whole, aligned dwords
    auto a4 = [](const void* p) { return p == nullptr || axk_aligned(p, 4); };
    const bool sdma0 = H % 128 == 0 && a4(e_gs) && a4(sh_gate_s) && a4(sh_up_s);
    const bool sdma1 = F % 128 == 0 && Fs % 128 == 0 && a4(e_ds) && a4(sh_down_s);
    const size_t lds0 = gemm_lds_bytes<0>(H, sdma0), lds1 = gemm_lds_bytes<1>(fmax, sdma1);
    static AxkOnce gemm_once;  // > 64 KiB of dynamic LDS must be allowed once per kernel
    const int raised = axk_once(gemm_once, [] {
      const void* fns[4] = {reinterpret_cast<const void*>(&moe_ggemm_kernel<0, false>),
                            reinterpret_cast<const void*>(&moe_ggemm_kernel<1, false>),
                            reinterpret_cast<const void*>(&moe_ggemm_kernel<0, true>),
                            reinterpret_cast<const void*>(&moe_ggemm_kernel<1, true>)};
      for (const void* f : fns) {
        const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxStageLds);
        if (e != hipSuccess) return e;
      }
      return hipSuccess;
    });
    if (raised != AXK_OK) return raised;
    const unsigned nb0 = (unsigned)((fmax + kG2Cols0 - 1) / kG2Cols0), nb1 = (unsigned)((H + kG2Cols1 - 1) / kG2Cols1);
    auto xgrid = [](unsigned n) { return dim3((n + kXcds - 1) / kXcds * kXcds); };  // whole rounds over the XCDs
    if (sdma0)
      hipLaunchKernelGGL((moe_ggemm_kernel<0, true>), xgrid(tiles * nb0), dim3(256), lds0, st, gu);
    else
      hipLaunchKernelGGL((moe_ggemm_kernel<0, false>), xgrid(tiles * nb0), dim3(256), lds0, st, gu);
    GGemmArgs dn{w.act, w.act_sh, e_dw, e_ds, sh_down_w, sh_down_s, nullptr, nullptr, T, H, F, Fs, fmax, w};
    constexpr unsigned sub1 = kBM / g_bm<1>();  // down workgroups per tile
    if (sdma1)
      hipLaunchKernelGGL((moe_ggemm_kernel<1, true>), xgrid(tiles * sub1 * nb1), dim3(256), lds1, st, dn);
    else
      hipLaunchKernelGGL((moe_ggemm_kernel<1, false>), xgrid(tiles * sub1 * nb1), dim3(256), lds1, st, dn);
    CombineArgs ca{h2, x_res, w_shg, nullptr, topk_ids, combine_shared, T, H, E, K, w, out};
    launch_combine<true>(ca, st);
    return axk_launch_status();
  }
  const int max_slots = E < T * K ? E : T * K;
  const int fmax = F > Fs ? F : Fs;
  // runs of 4 x tpw tiles per workgroup; activation rows staged in dynamic LDS ([rows][K + 8] bf16). Small batches
  // (tokens <= 64, K a multiple of 256) take the staged-weight kernels with 8 activation rows per pass (their
  // LDS tiles fit beside 8 rows, not 16); the others stream MFMA-layout units with 16 rows per pass.
  const int gu_tpw = kGateUpTilesPerWave, dn_tpw = kDownTilesPerWave;
  const int run_gu = kStreamWaves * gu_tpw, run_dn = kStreamWaves * dn_tpw;
  const int gu_grp = ((fmax + 15) / 16 + run_gu - 1) / run_gu;
  const int dn_grp = ((H + 15) / 16 + run_dn - 1) / run_dn;
  const int wide_k = 128 * kBatchChunks;
  const bool gu_wide = H % wide_k == 0, dn_wide = F % wide_k == 0 && Fs % wide_k == 0;
  const bool gu_stage = gu_wide && T <= 64, dn_stage = dn_wide && T <= 64;
  const int gu_rows = gu_stage ? kSmallRows : kStageRows, dn_rows = dn_stage ? kSmallRows : kStageRows;
  const size_t gu_lds = stream_stage_off(gu_rows, H) + (gu_stage ? kStreamWaves * kWaveStageBytes : 0);
  const size_t dn_lds = stream_stage_off(dn_rows, fmax) + (dn_stage ? kStreamWaves * kWaveStageBytes : 0);
  AXK_REQUIRE(gu_lds <= kMaxStreamLds && dn_lds <= kMaxStreamLds, AXK_E_SHAPE);
  static AxkOnce lds_once;  // > 64 KiB of dynamic LDS must be allowed once per kernel
  const int raised = axk_once(lds_once, [] {
    const void* fns[6] = {reinterpret_cast<const void*>(&moe_gateup_kernel<false, kStageRows, false>),
                          reinterpret_cast<const void*>(&moe_gateup_kernel<true, kStageRows, false>),
                          reinterpret_cast<const void*>(&moe_gateup_kernel<true, kSmallRows, true>),
                          reinterpret_cast<const void*>(&moe_down_kernel<false, kStageRows, false>),
                          reinterpret_cast<const void*>(&moe_down_kernel<true, kStageRows, false>),
                          reinterpret_cast<const void*>(&moe_down_kernel<true, kSmallRows, true>)};
    for (const void* f : fns) {
      const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxStreamLds);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  });
  if (raised != AXK_OK) return raised;
  const int gu_nsp = has_shared ? (T + gu_rows - 1) / gu_rows : 0, dn_nsp = has_shared ? (T + dn_rows - 1) / dn_rows : 0;
  GateUpArgs ga{h2, e_gw, e_gs, sh_gate_w, sh_gate_s, sh_up_w, sh_up_s, topk_ids, T, H, F, Fs, E, K, gu_grp, gu_tpw,
                gu_nsp, w};
  const dim3 gu_grid((unsigned)((max_slots + gu_nsp) * gu_grp)), dn_grid((unsigned)((max_slots + dn_nsp) * dn_grp));
  if (gu_stage)
    hipLaunchKernelGGL((moe_gateup_kernel<true, kSmallRows, true>), gu_grid, dim3(64 * kStreamWaves), gu_lds, st, ga);
  else if (gu_wide)
    hipLaunchKernelGGL((moe_gateup_kernel<true, kStageRows, false>), gu_grid, dim3(64 * kStreamWaves), gu_lds, st, ga);
  else
    hipLaunchKernelGGL((moe_gateup_kernel<false, kStageRows, false>), gu_grid, dim3(64 * kStreamWaves), gu_lds, st, ga);
  DownArgs da{e_dw, e_ds, sh_down_w, sh_down_s, topk_ids, topk_weights, T, H, F, Fs, E, K, dn_grp, dn_tpw, dn_nsp, w};
  if (dn_stage)
    hipLaunchKernelGGL((moe_down_kernel<true, kSmallRows, true>), dn_grid, dim3(64 * kStreamWaves), dn_lds, st, da);
  else if (dn_wide)
    hipLaunchKernelGGL((moe_down_kernel<true, kStageRows, false>), dn_grid, dim3(64 * kStreamWaves), dn_lds, st, da);
  else
    hipLaunchKernelGGL((moe_down_kernel<false, kStageRows, false>), dn_grid, dim3(64 * kStreamWaves), dn_lds, st, da);
  // the decode router formed the shared gate's logit when the routing ran in this call (gate_given)
  CombineArgs ca{h2, x_res, w_shg, gate_given ? w.gate_logit : nullptr, topk_ids, combine_shared, T, H, E, K, w, out};
  launch_combine<false>(ca, st);
  return axk_launch_status();
}
}  // namespace

extern "C" int axk_moe_experts(const uint16_t* h2, const uint16_t* x_res, const uint16_t* w_shg,
                               const uint8_t* sh_gate_w, const uint8_t* sh_gate_s, const uint8_t* sh_up_w,
                               const uint8_t* sh_up_s, const uint8_t* sh_down_w, const uint8_t* sh_down_s,
                               const uint8_t* e_gw, const uint8_t* e_gs, const uint8_t* e_dw, const uint8_t* e_ds,
                               const int32_t* topk_ids, const float* topk_weights, uint16_t* out, int64_t tokens,
                               int64_t hidden, int64_t num_experts, int64_t top_k, int64_t inter,
                               int64_t shared_inter, void* workspace, size_t workspace_bytes, axk_stream_t stream) {
  return moe_experts_impl(h2, x_res, w_shg, sh_gate_w, sh_gate_s, sh_up_w, sh_up_s, sh_down_w, sh_down_s, e_gw, e_gs,
                          e_dw, e_ds, topk_ids, topk_weights, out, tokens, hidden, num_experts, top_k, inter,
                          shared_inter, workspace, workspace_bytes, stream, false, false);
}

namespace {
int moe_decode_impl(const uint16_t* h2, const uint16_t* x_res, const uint16_t* w_router, const uint16_t* w_shg,
                    const uint8_t* sh_gate_w, const uint8_t* sh_gate_s, const uint8_t* sh_up_w, const uint8_t* sh_up_s,
                    const uint8_t* sh_down_w, const uint8_t* sh_down_s, const uint8_t* e_gw, const uint8_t* e_gs,
                    const uint8_t* e_dw, const uint8_t* e_ds, uint16_t* out, float* logits, int32_t* topk_ids,
                    float* topk_weights, int64_t tokens, int64_t hidden, int64_t num_experts, int64_t top_k,
                    int64_t inter, int64_t shared_inter, int norm_topk_prob, void* workspace, size_t workspace_bytes,
                    axk_stream_t stream, const float* y_sh_given) {
  AXK_REQUIRE(w_router && logits, AXK_E_NULL);
  AXK_REQUIRE(h2 && topk_ids && topk_weights, AXK_E_NULL);
  int rc = check_dims({tokens, hidden, num_experts, top_k, inter, sh_gate_w ? shared_inter : 0});
  if (rc != AXK_OK) return rc;
  AXK_REQUIRE(axk_aligned(h2, 16) && axk_aligned(w_router, 16), AXK_E_ALIGN);
  const size_t need = axk_moe_workspace_size(tokens, hidden, num_experts, top_k, inter, sh_gate_w ? shared_inter : 0);
  AXK_REQUIRE(workspace && workspace_bytes >= need && axk_aligned(workspace, 256), AXK_E_WORKSPACE);
  // the experts half's checks before anything is launched (a nonzero status means nothing was enqueued)
  rc = moe_experts_impl(h2, x_res, w_shg, sh_gate_w, sh_gate_s, sh_up_w, sh_up_s, sh_down_w, sh_down_s, e_gw, e_gs,
                        e_dw, e_ds, topk_ids, topk_weights, out, tokens, hidden, num_experts, top_k, inter,
                        shared_inter, workspace, workspace_bytes, stream, false, true, y_sh_given);
  if (rc != AXK_OK) return rc;
  AXK_LAUNCH_GATE();
  const MoeWs w = moe_ws(workspace, tokens, hidden, num_experts, top_k, inter, sh_gate_w ? shared_inter : 0);
  const int T = (int)tokens, H = (int)hidden, E = (int)num_experts, K = (int)top_k;
  const bool prefill = T > kDecodeTokens;
  hipStream_t st = axk_stream(stream);
  // the router as K-slice partial logits in the workspace (decode: also the shared gate's), summed in slice order
  // by the routing kernel, which writes the logits and the top-K
  const int S = prefill ? (int)std::min<int64_t>(kPrefillRouterSplits, hidden / 64) : router_splits(hidden);
  const bool gate = !prefill && w_shg != nullptr;
  if (prefill)
    hipLaunchKernelGGL(moe_router_tile_kernel, dim3((unsigned)((T + 63) / 64), (unsigned)((E + 63) / 64), (unsigned)S),
                       dim3(256), 0, st, h2, w_router, T, H, E, S, w.rpart, w.blk, (int)(prefill_blocks(T) * E));
  else
    hipLaunchKernelGGL(moe_router_kernel, dim3((unsigned)((E + 15) / 16 + (gate ? 1 : 0)), (unsigned)((T + 15) / 16),
                       (unsigned)S), dim3(256), 0, st, h2, w_router, w_shg, T, H, E, S, w.rpart, w.gpart);
  const dim3 grid((unsigned)((T + 3) / 4)), block(256);
  float* const gp = gate ? w.gpart : nullptr;
#define AXK_ROUTE_PART(V, MS)                                                                                     \
  hipLaunchKernelGGL((moe_route_part_kernel<V, MS>), grid, block, 0, st, w.rpart, gp, S, T, E, K, norm_topk_prob, \
                     logits, w.gate_logit, topk_ids, topk_weights, prefill ? w.blk : nullptr)
  if (prefill) {
    if (E <= 64) AXK_ROUTE_PART(1, kPrefillRouterSplits);
    else if (E <= 256) AXK_ROUTE_PART(4, kPrefillRouterSplits);
    else AXK_ROUTE_PART(kMaxExperts / 64, kPrefillRouterSplits);
  } else if (S <= 8) {  // the partial loads are unrolled to the bound: keep it tight
    if (E <= 64) AXK_ROUTE_PART(1, 8);
    else if (E <= 256) AXK_ROUTE_PART(4, 8);
    else AXK_ROUTE_PART(kMaxExperts / 64, 8);
  } else {
    if (E <= 64) AXK_ROUTE_PART(1, kMaxRouterSplits);
    else if (E <= 256) AXK_ROUTE_PART(4, kMaxRouterSplits);
    else AXK_ROUTE_PART(kMaxExperts / 64, kMaxRouterSplits);
  }
#undef AXK_ROUTE_PART
  rc = axk_launch_status();
  if (rc != AXK_OK) return rc;
  return moe_experts_impl(h2, x_res, w_shg, sh_gate_w, sh_gate_s, sh_up_w, sh_up_s, sh_down_w, sh_down_s, e_gw, e_gs,
                          e_dw, e_ds, topk_ids, topk_weights, out, tokens, hidden, num_experts, top_k, inter,
                          shared_inter, workspace, workspace_bytes, stream, gate, false, y_sh_given, prefill);
}
}  // namespace

extern "C" int axk_moe_decode(const uint16_t* h2, const uint16_t* x_res, const uint16_t* w_router,
                              const uint16_t* w_shg, const uint8_t* sh_gate_w, const uint8_t* sh_gate_s,
                              const uint8_t* sh_up_w, const uint8_t* sh_up_s, const uint8_t* sh_down_w,
                              const uint8_t* sh_down_s, const uint8_t* e_gw, const uint8_t* e_gs,
                              const uint8_t* e_dw, const uint8_t* e_ds, uint16_t* out, float* logits,
                              int32_t* topk_ids, float* topk_weights, int64_t tokens, int64_t hidden,
                              int64_t num_experts, int64_t top_k, int64_t inter, int64_t shared_inter,
                              int norm_topk_prob, void* workspace, size_t workspace_bytes, axk_stream_t stream) {
  return moe_decode_impl(h2, x_res, w_router, w_shg, sh_gate_w, sh_gate_s, sh_up_w, sh_up_s, sh_down_w, sh_down_s,
                         e_gw, e_gs, e_dw, e_ds, out, logits, topk_ids, topk_weights, tokens, hidden, num_experts,
                         top_k, inter, shared_inter, norm_topk_prob, workspace, workspace_bytes, stream, nullptr);
}

int axk_moe_decode_shared_given(const uint16_t* h2, const uint16_t* x_res, const uint16_t* w_router,
                                const uint16_t* w_shg, const float* y_sh, const uint8_t* e_gw, const uint8_t* e_gs,
                                const uint8_t* e_dw, const uint8_t* e_ds, uint16_t* out, float* logits,
                                int32_t* topk_ids, float* topk_weights, int64_t tokens, int64_t hidden,
                                int64_t num_experts, int64_t top_k, int64_t inter, int norm_topk_prob,
                                void* workspace, size_t workspace_bytes, axk_stream_t stream) {
  AXK_REQUIRE(y_sh, AXK_E_NULL);
  return moe_decode_impl(h2, x_res, w_router, w_shg, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, e_gw, e_gs,
                         e_dw, e_ds, out, logits, topk_ids, topk_weights, tokens, hidden, num_experts, top_k, inter, 0,
                         norm_topk_prob, workspace, workspace_bytes, stream, y_sh);
}
