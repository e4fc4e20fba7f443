// Gated DeltaNet chunked prefill (chunk-parallel WY form) for gfx950.
//
// Reference: gdn_stable_chunk (sgl_kernel_axera/attention/gdn.py:1122-1212) with the unit-lower solve of
// inverse_unit_lower_recursive (gdn.py:1048-1119) and chunk_prefix_sum_fp32 (gdn.py:992-1009), driven chunk by
// chunk as gdn_prefill_impl does (gdn.py:1628-1790) and as q35_prefill.gdn_chunked
// (models/qwen35_35b_a3b/src/70b0fbc/q35_prefill.py:144-169).
//
// Per chunk of C = 64 tokens and value head, with the gate prefix G = cumsum(g) inside the chunk,
// Gamma_t = exp(G_t) and decay_ij = exp(G_i - G_j) for i >= j:
//   L = beta_i (k_i . k_j) decay_ij (i > j);   Tinv = (I + L)^-1          (fp32 solve, rounded to bf16)
//   u = Tinv (beta v);   w = Tinv (beta Gamma k);   P = (q k^T) * decay   (bf16 MatMul operands and results)
//   v_new = u - w S;   o = Gamma (q S) + P v_new;   S <- Gamma_last S + k^T (v_new * decay_last,:)
// q and k are the L2-normalised head vectors (q also scaled by DK^-0.5), as in gdn_prefill_impl.
//
// Two launches:
//   gdn_chunk_prep_kernel  one workgroup per (sequence, value head, chunk); every chunk in parallel. The
//                          state-independent half: l2norm, gates, prefix, K K^T and Q K^T on MFMA, the
//                          triangular solve (16 x 16 diagonal blocks by substitution, then two levels of block
//                          products on fp32 MFMA), u and w on MFMA. Writes w, u, P, Gamma and the last decay
//                          row to the workspace, and once per key head the normalised q and k^T.
//   gdn_chunk_scan_kernel  one workgroup per (sequence, value head, slice of kScanSW state columns): the state's
//                          columns evolve independently, so 128 / kScanSW workgroups carry one head's 128 x 128
//                          fp32 state through the chunks in order, held in MFMA accumulators, with each chunk's
//                          operands loaded two chunks ahead.
#include "axk_common.h"
#include "axk_host.h"

namespace {

constexpr int kC = 64;    // chunk length
constexpr int kD = 128;   // key / value head dim

// Workspace: per (sequence, value head, chunk) w [C][D] bf16, u in the scan's accumulator order
// [D/16 slices][4 waves][64 lanes][4 rows] bf16, P [C][C] bf16, Gamma and last-row decay [C] fp32; per
// (sequence, key head, chunk) normalised q [C][D] bf16 and k^T [D][C] bf16.
struct ChunkWs {
  uint16_t* w;
  uint16_t* u;
  uint16_t* p;
  float* gam;
  float* dec;
  uint16_t* qn;
  uint16_t* kt;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t chunk_ws_layout(int64_t B, int64_t NK, int64_t NV, int64_t NC, size_t* off) {
  const size_t vc = (size_t)(B * NV * NC), kc = (size_t)(B * NK * NC);
  const size_t sizes[7] = {vc * kC * kD * 2, vc * kC * kD * 2, vc * kC * kC * 2, vc * kC * 4,
                           vc * kC * 4,      kc * kC * kD * 2, kc * kD * kC * 2};
  size_t o = 0;
  for (int i = 0; i < 7; ++i) {
    off[i] = o;
    o = align256(o + sizes[i]);
  }
  return o;
}

ChunkWs chunk_ws(void* ws, int64_t B, int64_t NK, int64_t NV, int64_t NC) {
  size_t off[7];
  chunk_ws_layout(B, NK, NV, NC, off);
  unsigned char* p = reinterpret_cast<unsigned char*>(ws);
  return {reinterpret_cast<uint16_t*>(p + off[0]), reinterpret_cast<uint16_t*>(p + off[1]),
          reinterpret_cast<uint16_t*>(p + off[2]), reinterpret_cast<float*>(p + off[3]),
          reinterpret_cast<float*>(p + off[4]),    reinterpret_cast<uint16_t*>(p + off[5]),
          reinterpret_cast<uint16_t*>(p + off[6])};
}

AXK_DEV float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
AXK_DEV float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

AXK_DEV axk_f32x4 mfma_f32_16x16x4(float a, float b, axk_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------------------------
// prep: the state-independent half of every chunk
// ---------------------------------------------------------------------------------------------
constexpr int kLdK = kD + 8;  // bf16 row stride of token-major [C][D] tiles in LDS
constexpr int kLdT = kC + 8;  // bf16 row stride of [D][C] and [C][C] tiles
constexpr int kLdL = kC + 4;  // fp32 row stride of [C][C] tiles
constexpr int kLdX = 32 + 1;  // fp32 scratch of the solve's block products

// Three regions, each reused as its contents die (52.7 KiB: three workgroups per CU):
//   K: normalised k (bf16 [C][LdK]) until the K K^T products; then, in place, beta Gamma k for w.
//   Q: normalised q (bf16 [C][LdK]) until the Q K^T products; P staging (bf16 [C][LdT]); the solve's fp32 scratch
//      [32][LdX]; bf16 Tinv [C][LdT]; w staging (bf16 [C][LdK]).
//   L: L (fp32 [C][LdL]), inverted in place into Tinv (each entry of Tinv overwrites the entry of L it replaces,
//      after that entry was read); then beta v (bf16 [C][LdK]).
constexpr int kOffK = 0;
constexpr int kSzK = kC * kLdK * 2;
constexpr int kOffQ = kOffK + kSzK;
constexpr int kSzQ = kC * kLdK * 2;
constexpr int kOffL = kOffQ + kSzQ;
constexpr int kSzL = kC * kLdL * 4;
constexpr int kOffG = kOffL + kSzL;       // G, beta: fp32 [C] each
constexpr int kPrepLds = kOffG + 2 * kC * 4;
static_assert(kSzQ >= kC * kLdT * 2 && kSzQ >= 32 * kLdX * 4 && kSzL >= kC * kLdK * 2, "LDS carve");
static_assert(3 * kPrepLds <= 160 * 1024, "three prep workgroups per CU");

struct PrepArgs {
  const uint16_t *q, *k, *v, *a, *b;
  const float *a_log, *dt_bias;
  ChunkWs ws;
  int B, T, NK, NV, NC;
  int64_t ldq, ldk, ldv;  // elements between consecutive (sequence, token) rows of q, k, v
  int kdiv;               // value head h reads key head (h / kdiv) % NK: NV / NK grouped, 1 tiled
};

__global__ __launch_bounds__(256) void gdn_chunk_prep_kernel(PrepArgs p) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* sK = reinterpret_cast<uint16_t*>(smem + kOffK);
  uint16_t* sQ = reinterpret_cast<uint16_t*>(smem + kOffQ);
  float* sL = reinterpret_cast<float*>(smem + kOffL);  // L, then Tinv in place
  float* sX = reinterpret_cast<float*>(smem + kOffQ);  // the solve's scratch (q is dead by then)
  float* sG = reinterpret_cast<float*>(smem + kOffG);
  float* sBeta = sG + kC;

  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int kh = (h / p.kdiv) % p.NK;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;
  const int t0 = c * kC;
  const int n = min(kC, p.T - t0);
  const int64_t vidx = ((int64_t)b * p.NV + h) * p.NC + c;   // (sequence, value head, chunk)
  const int64_t kidx = ((int64_t)b * p.NK + kh) * p.NC + c;  // (sequence, key head, chunk)

  // the gate inputs of wave 0 (lane = token), issued with the q / k / v loads: one memory round trip
  float a_in = 0.f, b_in = 0.f;
  if (wave == 0 && lane < n) {
    const int64_t vh = ((int64_t)b * p.T + t0 + lane) * p.NV + h;
    a_in = bf16_bits_to_f32(p.a[vh]);
    b_in = bf16_bits_to_f32(p.b[vh]);
  }
  const float dtb = p.dt_bias[h], alog = p.a_log[h];

  // ---- 1. q, k, v rows: thread = (token tt, 32-dim quarter qd); L2 norms over the 4 threads of a token ----
  const int tt = tid >> 2, qd = tid & 3;
  uint4 qr[4], kr[4], vr[4];
  if (tt < n) {
    const int64_t tok = (int64_t)b * p.T + t0 + tt;
    const uint4* qp = reinterpret_cast<const uint4*>(p.q + tok * p.ldq + kh * kD + 32 * qd);
    const uint4* kp = reinterpret_cast<const uint4*>(p.k + tok * p.ldk + kh * kD + 32 * qd);
    const uint4* vp = reinterpret_cast<const uint4*>(p.v + tok * p.ldv + h * kD + 32 * qd);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qr[i] = qp[i];
      kr[i] = kp[i];
      vr[i] = vp[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) qr[i] = kr[i] = vr[i] = make_uint4(0u, 0u, 0u, 0u);
  }
  float qs = 0.f, ks = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t qw[4] = {qr[i].x, qr[i].y, qr[i].z, qr[i].w};
    const uint32_t kw[4] = {kr[i].x, kr[i].y, kr[i].z, kr[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qs += bf16_lo(qw[j]) * bf16_lo(qw[j]) + bf16_hi(qw[j]) * bf16_hi(qw[j]);
      ks += bf16_lo(kw[j]) * bf16_lo(kw[j]) + bf16_hi(kw[j]) * bf16_hi(kw[j]);
    }
  }
  qs = group_sum<4>(qs);
  ks = group_sum<4>(ks);
  {
    // one reciprocal per row instead of a division per element (x * (1 / n) is within an fp32 ulp of x / n)
    const float rq = 1.0f / sqrtf(qs + 1e-6f), rk = 1.0f / sqrtf(ks + 1e-6f);
    const float qscale = 0.08838834764831845f;  // 128^-0.5
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t qw[4] = {qr[i].x, qr[i].y, qr[i].z, qr[i].w};
      const uint32_t kw[4] = {kr[i].x, kr[i].y, kr[i].z, kr[i].w};
      uint4 qo, ko;
      uint32_t* qop = reinterpret_cast<uint32_t*>(&qo);
      uint32_t* kop = reinterpret_cast<uint32_t*>(&ko);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // q: bf16(bf16(q / |q|) * DK^-0.5) (l2norm_lastdim, then the q scale; gdn.py:1631)
        qop[j] = pack_bf16x2(round_bf16(bf16_lo(qw[j]) * rq) * qscale, round_bf16(bf16_hi(qw[j]) * rq) * qscale);
        kop[j] = pack_bf16x2(bf16_lo(kw[j]) * rk, bf16_hi(kw[j]) * rk);
      }
      *reinterpret_cast<uint4*>(sQ + tt * kLdK + 32 * qd + 8 * i) = qo;
      *reinterpret_cast<uint4*>(sK + tt * kLdK + 32 * qd + 8 * i) = ko;
    }
  }
  // gates and the in-chunk prefix of g (wave 0, lane = token); padded tokens: g = 0, beta = 0
  if (wave == 0) {
    float g = 0.f, beta = 0.f;
    if (lane < n) {
      const float x = a_in + dtb;
      const float sp = x > 20.f ? x : log1pf(expf(x));
      g = -expf(alog) * sp;
      beta = round_bf16(1.0f / (1.0f + expf(-b_in)));
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float x = __shfl_up(g, o, 64);
      if (lane >= o) g += x;
    }
    sG[lane] = g;
    sBeta[lane] = beta;
  }
  __syncthreads();

  // ---- 2. normalised q and k^T of this key head (written once, by its first value head, kh * kdiv) ----
  if (h == kh * p.kdiv) {
    uint16_t* qn_g = p.ws.qn + kidx * kC * kD;
    uint16_t* kt_g = p.ws.kt + kidx * kD * kC;
    for (int i = tid; i < kC * kD / 8; i += 256) {  // fragment order: unit i of the destination
      const int row = 16 * (i >> 8) + (i & 15), col = 32 * ((i >> 6) & 3) + 8 * ((i >> 4) & 3);
      *reinterpret_cast<uint4*>(qn_g + 8 * i) = *reinterpret_cast<const uint4*>(sQ + row * kLdK + col);
    }
    for (int i = tid; i < kD * kC / 8; i += 256) {  // k^T [d][token] in fragment order
      const int d = 16 * (i >> 7) + (i & 15), t8 = 4 * ((i >> 6) & 1) + ((i >> 4) & 3);
      uint4 o;
      uint32_t* op = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        op[e] = (uint32_t)sK[(8 * t8 + 2 * e) * kLdK + d] | ((uint32_t)sK[(8 * t8 + 2 * e + 1) * kLdK + d] << 16);
      *reinterpret_cast<uint4*>(kt_g + 8 * i) = o;
    }
  }

  // ---- 3. K K^T and Q K^T: wave w owns token rows 16w .. 16w + 15 ----
  axk_f32x4 kk[4], qk[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) kk[j] = qk[j] = axk_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < kD / 32; ++st) {
    const int ko = 32 * st + 8 * g4;
    const axk_bf16x8 ak = load_bf16x8(sK + (16 * wave + l16) * kLdK + ko);
    const axk_bf16x8 aq = load_bf16x8(sQ + (16 * wave + l16) * kLdK + ko);
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      const axk_bf16x8 bk = load_bf16x8(sK + (16 * jt + l16) * kLdK + ko);
      kk[jt] = mfma_bf16_16x16x32(ak, bk, kk[jt]);
      qk[jt] = mfma_bf16_16x16x32(aq, bk, qk[jt]);
    }
  }

  // ---- 4. L (fp32, strictly lower), P = bf16((q k^T) * decay) staged (over q) for a coalesced write ----
  uint16_t* sP = sQ;
  __syncthreads();  // every wave's reads of q (and of k for the products) are done
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * wave + 4 * g4 + r, j = 16 * jt + l16;
      const float dij = i >= j ? __expf(sG[i] - sG[j]) : 0.f;  // hardware exp2: ~1e-6 relative, far below bf16
      sL[i * kLdL + j] = i > j ? kk[jt][r] * sBeta[i] * dij : 0.f;
      sP[i * kLdT + j] = i >= j ? (uint16_t)f32_to_bf16_bits(qk[jt][r] * dij) : (uint16_t)0;
    }
  if (tid < kC) {
    p.ws.gam[vidx * kC + tid] = __expf(sG[tid]);
    p.ws.dec[vidx * kC + tid] = __expf(sG[kC - 1] - sG[tid]);  // padded tokens keep G: row of the last valid token
  }
  __syncthreads();
  {
    uint16_t* p_g = p.ws.p + vidx * kC * kC;
    for (int i = tid; i < kC * kC / 8; i += 256) {  // fragment order
      const int row = 16 * (i >> 7) + (i & 15), col = 32 * ((i >> 6) & 1) + 8 * ((i >> 4) & 3);
      *reinterpret_cast<uint4*>(p_g + 8 * i) = *reinterpret_cast<const uint4*>(sP + row * kLdT + col);
    }
  }
  __syncthreads();

  // ---- 5. Tinv = (I + L)^-1 ----
  // In place over L: L is zero on and above the diagonal (step 4 writes every entry), which is what Tinv holds
  // above the diagonal, and every step writes a block of Tinv only after the block of L it replaces was read.
  // 5a. the four 16 x 16 diagonal blocks by forward substitution (wave 0: lane = 16 * block + column; a lane
  //     reads rows of its block, every read of the wave precedes its writes)
  if (wave == 0) {
    const int base = 16 * g4, col = l16;
    float t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float acc = i == col ? 1.f : 0.f;
#pragma unroll
      for (int j = 0; j < i; ++j) acc -= sL[(base + i) * kLdL + base + j] * t[j];
      t[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sL[(base + i) * kLdL + base + col] = t[i];
  }
  __syncthreads();
  // 5b. 32 x 32 blocks: T21 = -T22 (L21 T11) with 16 x 16 parts (waves 0, 1: one 32-block each)
  if (wave < 2) {
    const int base = 32 * wave;
    axk_f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int kq = 4 * st + g4;
      x = mfma_f32_16x16x4(sL[(base + 16 + l16) * kLdL + base + kq], sL[(base + kq) * kLdL + base + l16], x);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) sX[wave * 16 * 17 + (4 * g4 + r) * 17 + l16] = x[r];
  }
  __syncthreads();
  if (wave < 2) {
    const int base = 32 * wave;
    axk_f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int kq = 4 * st + g4;
      y = mfma_f32_16x16x4(sL[(base + 16 + l16) * kLdL + base + 16 + kq], sX[wave * 16 * 17 + kq * 17 + l16], y);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) sL[(base + 16 + 4 * g4 + r) * kLdL + base + l16] = -y[r];  // over L21 (read above)
  }
  __syncthreads();
  // 5c. the 64 x 64 level: T21 = -T22 (L21 T11) with 32 x 32 parts (wave w: output tile (w / 2, w % 2))
  {
    const int rt = wave >> 1, ct = wave & 1;
    axk_f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const int kq = 4 * st + g4;
      x = mfma_f32_16x16x4(sL[(32 + 16 * rt + l16) * kLdL + kq], sL[kq * kLdL + 16 * ct + l16], x);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) sX[(16 * rt + 4 * g4 + r) * kLdX + 16 * ct + l16] = x[r];
    __syncthreads();
    axk_f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const int kq = 4 * st + g4;
      y = mfma_f32_16x16x4(sL[(32 + 16 * rt + l16) * kLdL + 32 + kq], sX[kq * kLdX + 16 * ct + l16], y);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) sL[(32 + 16 * rt + 4 * g4 + r) * kLdL + 16 * ct + l16] = -y[r];  // over L21 (read above)
  }
  __syncthreads();

  // ---- 6. bf16 operands: Tinv [C][LdT] (over the scratch), beta v (over fp32 Tinv), beta Gamma k (over k) ----
  uint16_t* sTb = sQ;
  for (int i = tid; i < kC * kC; i += 256) {
    const int r = i >> 6, cc = i & 63;
    sTb[r * kLdT + cc] = (uint16_t)f32_to_bf16_bits(sL[r * kLdL + cc]);
  }
  __syncthreads();
  // beta v and beta Gamma k row-major [token][LdK] (16-byte writes); step 7 reads them transposed. Each thread
  // rewrites the k entries it reads (its own token and columns), so k -> beta Gamma k in place is safe.
  uint16_t* sVB = reinterpret_cast<uint16_t*>(sL);
  uint16_t* sKB = sK;
  {
    const float beta = sBeta[tt], gm = __expf(sG[tt]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d0 = 32 * qd + 8 * i;
      const uint4 kq = *reinterpret_cast<const uint4*>(sK + tt * kLdK + d0);
      const uint32_t vw[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w}, kw[4] = {kq.x, kq.y, kq.z, kq.w};
      uint32_t vo[4], ko[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        vo[j] = pack_bf16x2(bf16_lo(vw[j]) * beta, bf16_hi(vw[j]) * beta);
        ko[j] = pack_bf16x2(bf16_lo(kw[j]) * beta * gm, bf16_hi(kw[j]) * beta * gm);
      }
      *reinterpret_cast<uint4*>(sVB + tt * kLdK + d0) = make_uint4(vo[0], vo[1], vo[2], vo[3]);
      *reinterpret_cast<uint4*>(sKB + tt * kLdK + d0) = make_uint4(ko[0], ko[1], ko[2], ko[3]);
    }
  }
  __syncthreads();

  // ---- 7. u = Tinv (beta v), w = Tinv (beta Gamma k): wave w owns token rows 16w .. 16w + 15 ----
  axk_f32x4 ua[8], wa[8];
#pragma unroll
  for (int ct = 0; ct < 8; ++ct) ua[ct] = wa[ct] = axk_f32x4{0.f, 0.f, 0.f, 0.f};
  // B fragments (tokens 8 g .. 8 g + 7 of column 16 ct + l16) by two transposing reads: source lane 4 j + a of
  // group g points at token 8 g + j (+ 4), columns 16 ct + 4 a .. + 3
  auto bfrag = [&](const uint16_t* m, int tok, int col) __attribute__((always_inline)) -> axk_bf16x8 {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 lo = __builtin_bit_cast(u32x2, lds_read_tr16(m + tok * kLdK + col));
    const u32x2 hi = __builtin_bit_cast(u32x2, lds_read_tr16(m + (tok + 4) * kLdK + col));
    return __builtin_bit_cast(axk_bf16x8, axk_u32x4{lo.x, lo.y, hi.x, hi.y});  // whole-register moves only
  };
#pragma unroll
  for (int st = 0; st < kC / 32; ++st) {
    const int ko = 32 * st + 8 * g4;
    const axk_bf16x8 at = load_bf16x8(sTb + (16 * wave + l16) * kLdT + ko);
    const int tok = ko + (l16 >> 2);
#pragma unroll
    for (int ct = 0; ct < 8; ++ct) {
      const int col = 16 * ct + 4 * (l16 & 3);
      ua[ct] = mfma_bf16_16x16x32(at, bfrag(sVB, tok, col), ua[ct]);
      wa[ct] = mfma_bf16_16x16x32(at, bfrag(sKB, tok, col), wa[ct]);
    }
  }
  __syncthreads();

  // ---- 8. u straight from the accumulators in the scan's order; w staged (over Tinv) for row-major writes ----
  uint16_t* u_g = p.ws.u + vidx * kC * kD;
#pragma unroll
  for (int ct = 0; ct < 8; ++ct)
    *reinterpret_cast<uint2*>(u_g + ((ct * 4 + wave) * 64 + lane) * 4) =
        make_uint2(pack_bf16x2(ua[ct][0], ua[ct][1]), pack_bf16x2(ua[ct][2], ua[ct][3]));
  uint16_t* sW = sQ;
#pragma unroll
  for (int ct = 0; ct < 8; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) sW[(16 * wave + 4 * g4 + r) * kLdK + 16 * ct + l16] = (uint16_t)f32_to_bf16_bits(wa[ct][r]);
  __syncthreads();
  uint16_t* w_g = p.ws.w + vidx * kC * kD;
  for (int i = tid; i < kC * kD / 8; i += 256) {  // fragment order
    const int row = 16 * (i >> 8) + (i & 15), col = 32 * ((i >> 6) & 3) + 8 * ((i >> 4) & 3);
    *reinterpret_cast<uint4*>(w_g + 8 * i) = *reinterpret_cast<const uint4*>(sW + row * kLdK + col);
  }
}

// ---------------------------------------------------------------------------------------------
// scan: the state through the chunks, one 16-column slice per workgroup
// ---------------------------------------------------------------------------------------------
constexpr int kLdS = kD + 8;  // bf16 state slice in LDS, [slice columns][LdS] (8 consecutive rows per lane read)
constexpr int kLdV = kC + 8;  // bf16 v_new and its decayed copy, [slice columns][LdV]
#ifndef AXK_GDN_SW
#define AXK_GDN_SW 16
#endif
#ifndef AXK_GDN_NW
#define AXK_GDN_NW 4
#endif
constexpr int kScanSW = AXK_GDN_SW;  // state columns per scan workgroup
constexpr int kScanNW = AXK_GDN_NW;  // waves per scan workgroup

struct ScanArgs {
  const float* state_in;
  float* state_out;
  uint16_t* out;
  ChunkWs ws;
  int B, T, NK, NV, NC;
  int kdiv;  // value head h reads key head (h / kdiv) % NK
};

// Scan workgroup (sequence, value head, slice of SW state columns) with NW waves. Wave w: token tile
// tt = w % 4 (rows 16 tt .. of w, q, P and of the outputs; state rows 32 tt .. 32 tt + 31) and CPW of the slice's
// 16-column tiles (column group w / 4).
template <int SW, int NW>
struct ScanShape {
  static constexpr int CT = SW / 16;   // column tiles in the slice
  static constexpr int CG = NW / 4;    // column groups
  static constexpr int CPW = CT / CG;  // column tiles per wave
  static_assert(NW % 4 == 0 && CT % CG == 0 && CPW >= 1, "scan shape");
};

// One chunk's operands for one wave (plain members: the struct stays in registers).
template <int CPW>
struct ScanOps {
  axk_bf16x8 wf[4], qf[4], pf[2], kf[2][2];
  uint2 u[CPW];
  float4 gm, dc;
  float glast;
};

// A wave's operand pointers at chunk 0 (operands stored in MFMA fragment order, 16-row x 32-column fragments of 64
// lanes x 16 bytes: every load instruction reads 1 KiB contiguous); chunk c adds c times the per-chunk stride.
struct ScanBase {
  const uint16_t *w, *q, *p, *kt, *u;
  const float *gam, *dec, *glast;
};

template <int CPW>
AXK_DEV void scan_load(ScanOps<CPW>& s, const ScanBase& sb, int c) {
  const int64_t cc = c;
  const uint16_t* wg = sb.w + cc * (kC * kD);    // fragments (tt, st), st < 4
  const uint16_t* qg = sb.q + cc * (kC * kD);
  const uint16_t* pg = sb.p + cc * (kC * kC);    // fragments (tt, st), st < 2
  const uint16_t* ktg = sb.kt + cc * (kD * kC);  // fragments (2 tt + i, st), st < 2
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    s.wf[st] = load_bf16x8(wg + st * 512);
    s.qf[st] = load_bf16x8(qg + st * 512);
  }
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    s.pf[st] = load_bf16x8(pg + st * 512);
    s.kf[0][st] = load_bf16x8(ktg + st * 512);
    s.kf[1][st] = load_bf16x8(ktg + (2 + st) * 512);
  }
#pragma unroll
  for (int j = 0; j < CPW; ++j) s.u[j] = *reinterpret_cast<const uint2*>(sb.u + cc * (kC * kD) + j * (4 * 64 * 4));
  s.gm = *reinterpret_cast<const float4*>(sb.gam + cc * kC);
  s.dc = *reinterpret_cast<const float4*>(sb.dec + cc * kC);
  // a per-lane load (an index the compiler cannot prove uniform): a scalar load here would be waited for at once
  int z = 0;
  asm volatile("" : "+v"(z));
  s.glast = sb.glast[cc * kC + z];
}

template <int SW, int NW>
__global__ __launch_bounds__(64 * NW) void gdn_chunk_scan_kernel(ScanArgs p) {
  using Sh = ScanShape<SW, NW>;
  constexpr int CPW = Sh::CPW;
  __shared__ __align__(16) uint16_t sS[SW * kLdS];
  __shared__ __align__(16) uint16_t sV[SW * kLdV];
  __shared__ __align__(16) uint16_t sXd[SW * kLdV];
  __shared__ __align__(16) uint16_t sO[NW][16 * SW];  // a wave's 16 output rows, staged for 16-byte stores
  static_assert(Sh::CG == 1, "each wave holds all the slice's columns of its rows (the staged stores)");
  const int nbh = p.B * p.NV;
  const int slice = blockIdx.x / nbh, bh = blockIdx.x - slice * nbh;  // slices of a head share an XCD
  const int b = bh / p.NV, h = bh - b * p.NV, kh = (h / p.kdiv) % p.NK;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, g4 = lane >> 4;
  const int tt = wave & 3;
  const int ct_l = (wave >> 2) * CPW;         // first column tile of this wave inside the slice
  const int ct0 = slice * Sh::CT + ct_l;      // ... inside the head (the u layout's column tile)
  const int col0 = 16 * ct0;                  // first state / output column of the wave
  const int64_t vbase = (int64_t)bh * p.NC, kbase = ((int64_t)b * p.NK + kh) * p.NC;  // chunk 0's indices
  ScanBase sbase;
  sbase.w = p.ws.w + vbase * kC * kD + (4 * tt * 64 + lane) * 8;
  sbase.q = p.ws.qn + kbase * kC * kD + (4 * tt * 64 + lane) * 8;
  sbase.p = p.ws.p + vbase * kC * kC + (2 * tt * 64 + lane) * 8;
  sbase.kt = p.ws.kt + kbase * kD * kC + (4 * tt * 64 + lane) * 8;
  sbase.u = p.ws.u + vbase * kC * kD + ((ct0 * 4 + tt) * 64 + lane) * 4;
  sbase.gam = p.ws.gam + vbase * kC + 16 * tt + 4 * g4;
  sbase.dec = p.ws.dec + vbase * kC + 16 * tt + 4 * g4;
  sbase.glast = p.ws.gam + vbase * kC + kC - 1;
  // output rows leave as 16-byte stores: lane i < 2 SW of the wave writes 8 columns of token row 16 tt + i / (SW / 8)
  constexpr int OL = 16 * SW / 8;  // lanes storing a wave's 16 rows
  const int otok = lane / (SW / 8), ocol = 8 * (lane % (SW / 8));
  uint16_t* obase = p.out + ((int64_t)b * p.T * p.NV + h) * kD + 16 * slice * Sh::CT + ocol;
  const int64_t ostride = (int64_t)p.NV * kD;

  // state rows 32 tt + 16 i + 4 g + r, columns col0 + 16 j + l16, in MFMA accumulator tiles
  const float* sin = p.state_in + (int64_t)bh * kD * kD;
  axk_f32x4 S[2][CPW];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < CPW; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) S[i][j][r] = sin[(32 * tt + 16 * i + 4 * g4 + r) * kD + col0 + 16 * j + l16];
  auto put_state = [&]() {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < CPW; ++j)
        *reinterpret_cast<uint2*>(sS + (16 * (ct_l + j) + l16) * kLdS + 32 * tt + 16 * i + 4 * g4) =
            make_uint2(pack_bf16x2(S[i][j][0], S[i][j][1]), pack_bf16x2(S[i][j][2], S[i][j][3]));
  };
  put_state();
  __syncthreads();

  auto process = [&](const ScanOps<CPW>& o, int c) {
    // v_new = u - w S;  base = q S  (S as a bf16 operand, as the reference casts it)
    axk_f32x4 vfs[CPW], base[CPW];
#pragma unroll
    for (int j = 0; j < CPW; ++j) vfs[j] = base[j] = axk_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int j = 0; j < CPW; ++j) {
        const axk_bf16x8 sf = load_bf16x8(sS + (16 * (ct_l + j) + l16) * kLdS + 32 * st + 8 * g4);
        vfs[j] = mfma_bf16_16x16x32(o.wf[st], sf, vfs[j]);
        base[j] = mfma_bf16_16x16x32(o.qf[st], sf, base[j]);
      }
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      float vn[4];
      vn[0] = bf16_lo(o.u[j].x) - vfs[j][0];
      vn[1] = bf16_hi(o.u[j].x) - vfs[j][1];
      vn[2] = bf16_lo(o.u[j].y) - vfs[j][2];
      vn[3] = bf16_hi(o.u[j].y) - vfs[j][3];
      const int lc = 16 * (ct_l + j) + l16;
      *reinterpret_cast<uint2*>(sV + lc * kLdV + 16 * tt + 4 * g4) =
          make_uint2(pack_bf16x2(vn[0], vn[1]), pack_bf16x2(vn[2], vn[3]));
      *reinterpret_cast<uint2*>(sXd + lc * kLdV + 16 * tt + 4 * g4) =
          make_uint2(pack_bf16x2(vn[0] * o.dc.x, vn[1] * o.dc.y), pack_bf16x2(vn[2] * o.dc.z, vn[3] * o.dc.w));
    }
    __syncthreads();
    // o = Gamma (q S) + P v_new
    const float gmr[4] = {o.gm.x, o.gm.y, o.gm.z, o.gm.w};
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const int lc = 16 * (ct_l + j) + l16;
      axk_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 2; ++st) acc = mfma_bf16_16x16x32(o.pf[st], load_bf16x8(sV + lc * kLdV + 32 * st + 8 * g4), acc);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sO[wave][(4 * g4 + r) * SW + 16 * (ct_l + j) + l16] = (uint16_t)f32_to_bf16_bits(base[j][r] * gmr[r] + acc[r]);
    }
    // the wave's rows out of its own staging (in order after its writes: no barrier)
    if (lane < OL) {
      const int t = c * kC + 16 * tt + otok;
      const uint4 v = *reinterpret_cast<const uint4*>(&sO[wave][otok * SW + ocol]);
      if (t < p.T) *reinterpret_cast<uint4*>(obase + t * ostride) = v;
    }
    // S <- Gamma_last S + k^T (v_new * decay_last)
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const int lc = 16 * (ct_l + j) + l16;
      axk_bf16x8 xf[2];
#pragma unroll
      for (int st = 0; st < 2; ++st) xf[st] = load_bf16x8(sXd + lc * kLdV + 32 * st + 8 * g4);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) S[i][j][r] *= o.glast;
#pragma unroll
        for (int st = 0; st < 2; ++st) S[i][j] = mfma_bf16_16x16x32(o.kf[i][st], xf[st], S[i][j]);
      }
    }
    put_state();
    __syncthreads();
  };

  // Four operand sets in rotation: chunk c + 3 is loaded while chunk c is processed (the loads have three chunk
  // steps to land; one wave per SIMD leaves the registers for it). The loads are unconditional (past the end they
  // repeat the last chunk, unused) so every path through the loop has the same loads in flight and the waits
  // before each use stay three sets deep.
  const int last = p.NC - 1;
  ScanOps<CPW> o0, o1, o2, o3;
  scan_load(o0, sbase, 0);
  scan_load(o1, sbase, min(1, last));
  scan_load(o2, sbase, min(2, last));
  for (int c = 0; c < p.NC; c += 4) {
    scan_load(o3, sbase, min(c + 3, last));
    process(o0, c);
    scan_load(o0, sbase, min(c + 4, last));
    if (c + 1 < p.NC) process(o1, c + 1);
    scan_load(o1, sbase, min(c + 5, last));
    if (c + 2 < p.NC) process(o2, c + 2);
    scan_load(o2, sbase, min(c + 6, last));
    if (c + 3 < p.NC) process(o3, c + 3);
  }

  float* sout = p.state_out + (int64_t)bh * kD * kD;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < CPW; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) sout[(32 * tt + 16 * i + 4 * g4 + r) * kD + col0 + 16 * j + l16] = S[i][j][r];
}

int check_chunk_dims(int64_t batch, int64_t tokens, int64_t nk, int64_t nv, int64_t dk, int64_t dv,
                     int64_t chunk) {
  AXK_REQUIRE(dk == kD && dv == kD && chunk == kC, AXK_E_SHAPE);
  AXK_REQUIRE(batch > 0 && tokens > 0 && nk > 0 && nv > 0 && nv % nk == 0, AXK_E_SHAPE);
  AXK_REQUIRE(batch <= 65535 && nv <= 65535 && batch * nv * (kD / kScanSW) <= INT32_MAX, AXK_E_SHAPE);
  AXK_REQUIRE(tokens <= INT32_MAX - kC, AXK_E_SHAPE);
  return AXK_OK;
}

}  // namespace

extern "C" size_t axk_gdn_chunk_workspace_size(int64_t batch, int64_t tokens, int64_t num_k_heads,
                                               int64_t num_v_heads, int64_t head_k_dim, int64_t head_v_dim,
                                               int64_t chunk_size) {
  if (check_chunk_dims(batch, tokens, num_k_heads, num_v_heads, head_k_dim, head_v_dim, chunk_size) != AXK_OK)
    return 0;
  size_t off[7];
  return chunk_ws_layout(batch, num_k_heads, num_v_heads, (tokens + kC - 1) / kC, off);
}

namespace {
int chunk_prefill_impl(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* a, const uint16_t* b,
                       const float* a_log, const float* dt_bias, const float* state_in, float* state_out,
                       uint16_t* out, int64_t batch, int64_t tokens, int64_t num_k_heads, int64_t num_v_heads,
                       int64_t head_k_dim, int64_t head_v_dim, int64_t chunk_size, int64_t ldq, int64_t ldk,
                       int64_t ldv, int v_order, void* workspace, size_t workspace_bytes, axk_stream_t stream) {
  AXK_REQUIRE(q && k && v && a && b && a_log && dt_bias && state_in && state_out && out, AXK_E_NULL);
  AXK_REQUIRE(v_order == AXK_VORDER_GROUPED || v_order == AXK_VORDER_TILED, AXK_E_SHAPE);
  const int rc = check_chunk_dims(batch, tokens, num_k_heads, num_v_heads, head_k_dim, head_v_dim, chunk_size);
  if (rc != AXK_OK) return rc;
  AXK_REQUIRE(axk_aligned(q, 16) && axk_aligned(k, 16) && axk_aligned(v, 16), AXK_E_ALIGN);
  AXK_REQUIRE(ldq >= num_k_heads * kD && ldk >= num_k_heads * kD && ldv >= num_v_heads * kD, AXK_E_SHAPE);
  AXK_REQUIRE(ldq % 8 == 0 && ldk % 8 == 0 && ldv % 8 == 0, AXK_E_ALIGN);
  AXK_REQUIRE(axk_aligned(state_in, 16) && axk_aligned(state_out, 16), AXK_E_ALIGN);
  const size_t need =
      axk_gdn_chunk_workspace_size(batch, tokens, num_k_heads, num_v_heads, head_k_dim, head_v_dim, chunk_size);
  AXK_REQUIRE(workspace && workspace_bytes >= need && axk_aligned(workspace, 256), AXK_E_WORKSPACE);
  const size_t sbytes = (size_t)batch * num_v_heads * kD * kD * 4;
  const size_t obytes = (size_t)batch * tokens * num_v_heads * kD * 2;
  // in place is allowed (each workgroup reads its state slice before writing it); partial overlap is not
  AXK_REQUIRE(state_in == state_out || !axk_overlap(state_in, sbytes, state_out, sbytes), AXK_E_ALIAS);
  AXK_REQUIRE(!axk_overlap(out, obytes, state_out, sbytes) && !axk_overlap(out, obytes, workspace, need) &&
                  !axk_overlap(state_out, sbytes, workspace, need),
              AXK_E_ALIAS);
  const int NC = (int)((tokens + kC - 1) / kC);
  const ChunkWs ws = chunk_ws(workspace, batch, num_k_heads, num_v_heads, NC);
  AXK_LAUNCH_GATE();
  hipStream_t st = axk_stream(stream);
  static AxkOnce lds_once;  // > 64 KiB of dynamic LDS must be allowed once
  if (const int rc = axk_raise_lds(lds_once, reinterpret_cast<const void*>(&gdn_chunk_prep_kernel), kPrepLds))
    return rc;
  const int kdiv = v_order == AXK_VORDER_TILED ? 1 : (int)(num_v_heads / num_k_heads);
  PrepArgs pa{q, k, v, a, b, a_log, dt_bias, ws, (int)batch, (int)tokens, (int)num_k_heads, (int)num_v_heads, NC,
              ldq, ldk, ldv, kdiv};
  hipLaunchKernelGGL(gdn_chunk_prep_kernel, dim3((unsigned)NC, (unsigned)num_v_heads, (unsigned)batch), dim3(256),
                     kPrepLds, st, pa);
  int lrc = axk_launch_status();
  if (lrc != AXK_OK) return lrc;
  ScanArgs sa{state_in, state_out, out, ws, (int)batch, (int)tokens, (int)num_k_heads, (int)num_v_heads, NC, kdiv};
  hipLaunchKernelGGL((gdn_chunk_scan_kernel<kScanSW, kScanNW>), dim3((unsigned)((kD / kScanSW) * batch * num_v_heads)),
                     dim3(64 * kScanNW), 0, st, sa);
  return axk_launch_status();
}
}  // namespace

extern "C" int axk_gdn_chunk_prefill(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* a,
                                     const uint16_t* b, const float* a_log, const float* dt_bias,
                                     const float* state_in, float* state_out, uint16_t* out, int64_t batch,
                                     int64_t tokens, int64_t num_k_heads, int64_t num_v_heads, int64_t head_k_dim,
                                     int64_t head_v_dim, int64_t chunk_size, void* workspace, size_t workspace_bytes,
                                     axk_stream_t stream) {
  return chunk_prefill_impl(q, k, v, a, b, a_log, dt_bias, state_in, state_out, out, batch, tokens, num_k_heads,
                            num_v_heads, head_k_dim, head_v_dim, chunk_size, num_k_heads * kD, num_k_heads * kD,
                            num_v_heads * kD, AXK_VORDER_GROUPED, workspace, workspace_bytes, stream);
}

int axk_gdn_chunk_prefill_strided(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* a,
                                  const uint16_t* b, const float* a_log, const float* dt_bias, const float* state_in,
                                  float* state_out, uint16_t* out, int64_t batch, int64_t tokens, int64_t num_k_heads,
                                  int64_t num_v_heads, int64_t ldq, int64_t ldk, int64_t ldv, int v_order,
                                  void* workspace, size_t workspace_bytes, axk_stream_t stream) {
  return chunk_prefill_impl(q, k, v, a, b, a_log, dt_bias, state_in, state_out, out, batch, tokens, num_k_heads,
                            num_v_heads, kD, kD, kC, ldq, ldk, ldv, v_order, workspace, workspace_bytes, stream);
}
