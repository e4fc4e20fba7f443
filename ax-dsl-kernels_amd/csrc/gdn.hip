// Gated DeltaNet (GDN) recurrent step for gfx950: gate, q/k L2 norm and the delta-rule state update.
//
// Per (sequence b, value head h), token by token (T >= 1; T = 1 is decode):
//   q, k  <- L2-normalised key-head vectors (x / sqrt(sum x^2 + 1e-6)), q *= DK^-0.5
//            (l2norm_lastdim, sgl_kernel_axera/attention/gdn.py:919-931; models/.../q35_step.py:164-169)
//   g      = -exp(A_log[h]) * softplus(a + dt_bias[h]);  beta = sigmoid(b)          (gdn_gate, gdn.py:934-949)
//   S     <- exp(g) S;  pred = k^T S;  err = beta (v - pred);  S <- S + k err^T;  o = q^T S
//            (gdn_recurrent_step, gdn.py:952-989)
// Value head h reads key head (h / kdiv) % NK: kdiv = NV / NK in the grouped order (h / (NV / NK), the operators'
// order, test_gdn_attn.py:268-277), kdiv = 1 in the tiled order (h % NK, the layer kernels' default order,
// models/qwen35_35b_a3b/src/70b0fbc/q35_step.py:82-85, 171).
// The state S [DK, DV] fp32 is the kernel's whole HBM traffic: a workgroup holds its 128 x 128 tile in
// registers (64 floats per thread, float4 loads along DV) from one read to one write, across all T tokens.
// Arithmetic is fp32 throughout (the reference rounds the state to bf16 for its two products; the
// difference is well inside the bf16 output tolerance and is checked against both formulations).
// With GATE (the decode layer), the output row of each head goes through the GDN output norm before it is
// stored: out = bf16(bf16(rmsnorm(bf16 o) * norm_w) * silu(z)) (q35_step.py:179-180), the same rounding points
// as the separate gated-norm kernel.
#include "axk_common.h"
#include "axk_host.h"

namespace {

constexpr int kDK = 128, kDV = 128;
constexpr int kThreads = 256;
constexpr int kColGroups = kDV / 4;               // 32 threads across DV, 4 columns each
constexpr int kRowGroups = kThreads / kColGroups; // 8 row groups
constexpr int kRows = kDK / kRowGroups;           // 16 state rows per thread

struct GdnArgs {
  const uint16_t* q;   // [B, T, NK, DK] bf16
  const uint16_t* k;   // [B, T, NK, DK] bf16
  const uint16_t* v;   // [B, T, NV, DV] bf16
  const uint16_t* a;   // [B, T, NV] bf16
  const uint16_t* b;   // [B, T, NV] bf16
  const float* a_log;  // [NV]
  const float* dt_bias;  // [NV]
  const float* state_in;  // [B, NV, DK, DV]
  float* state_out;       // [B, NV, DK, DV] (may alias state_in)
  uint16_t* out;          // [B, T, NV, DV] bf16
  int B, T, NK, NV;
  int64_t ldq, ldk, ldv, ldab;  // elements between consecutive (sequence, token) rows of q, k, v, a / b
  const float* norm_w;          // GATE: the output norm's weight [DV] and gate z [B, T, NV, DV]
  const uint16_t* z;
  float eps;
  float* snap;                  // optional: the state after token t at snap + t * snap_ld, [B, NV, DK, DV] each
  int64_t snap_ld;
  int kdiv;                     // value head h reads key head (h / kdiv) % NK
};

template <bool GATE>
__global__ __launch_bounds__(kThreads) void gdn_recurrent_kernel(GdnArgs p) {
  __shared__ float s_k[kDK], s_q[kDK];
  __shared__ float s_gn[2];
  __shared__ float s_red[kRowGroups / 2][kDV];  // per-wave partial column sums
  __shared__ float s_vec[kDV];
  __shared__ float s_norm[4];

  const int bh = blockIdx.x;
  const int b = bh / p.NV, h = bh - (bh / p.NV) * p.NV;
  const int kh = (h / p.kdiv) % p.NK;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cg = tid % kColGroups, rg = tid / kColGroups;
  const int c0 = 4 * cg, r0 = kRows * rg;

  // state tile in registers: rows r0 .. r0 + 15, columns c0 .. c0 + 3
  const float* sin = p.state_in + ((int64_t)b * p.NV + h) * kDK * kDV;
  float4 S[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) {  // the tile is read once and written once: non-temporal
    const axk_u32x4 u = load_nt(sin + (r0 + r) * kDV + c0);
    S[r] = make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
  }

  const float a_log = p.a_log[h], dt_bias = p.dt_bias[h];
  const float qscale = rsqrtf((float)kDK);

  for (int t = 0; t < p.T; ++t) {
    const int64_t tok = (int64_t)b * p.T + t;
    // ---- q / k L2 norm (threads 0..127 own one element of each) ----
    float kx = 0.f, qx = 0.f;
    if (tid < kDK) {
      kx = bf16_bits_to_f32(p.k[tok * p.ldk + kh * kDK + tid]);
      qx = bf16_bits_to_f32(p.q[tok * p.ldq + kh * kDK + tid]);
    }
    float ks = wave_sum(kx * kx), qs = wave_sum(qx * qx);
    if (lane == 0 && wave < 2) {
      s_norm[wave] = ks;
      s_norm[2 + wave] = qs;
    }
    const int64_t vh = tok * p.NV + h;  // output row
    const float a = bf16_bits_to_f32(p.a[tok * p.ldab + h]), bb = bf16_bits_to_f32(p.b[tok * p.ldab + h]);
    const uint16_t* vr = p.v + tok * p.ldv + h * kDV + c0;
    const float4 vv = make_float4(bf16_bits_to_f32(vr[0]), bf16_bits_to_f32(vr[1]), bf16_bits_to_f32(vr[2]),
                                  bf16_bits_to_f32(vr[3]));
    __syncthreads();
    if (tid < kDK) {
      const float kn = sqrtf(s_norm[0] + s_norm[1] + 1e-6f), qn = sqrtf(s_norm[2] + s_norm[3] + 1e-6f);
      s_k[tid] = kx / kn;
      s_q[tid] = qx / qn * qscale;
    }
    // ---- gate ----
    const float g = -__expf(a_log) * softplus_f32(a + dt_bias);
    const float decay = __expf(g);
    const float beta = sigmoid_f32(bb);
    __syncthreads();

    // ---- S <- decay S; pred = k^T S (column sums over this thread's rows, then over row groups) ----
    float4 pr = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const float kr = s_k[r0 + r];
      S[r].x *= decay; S[r].y *= decay; S[r].z *= decay; S[r].w *= decay;
      pr.x += kr * S[r].x; pr.y += kr * S[r].y; pr.z += kr * S[r].z; pr.w += kr * S[r].w;
    }
    // the two row groups of a wave: lanes l and l ^ 32
    pr.x = xor32_sum(pr.x); pr.y = xor32_sum(pr.y);
    pr.z = xor32_sum(pr.z); pr.w = xor32_sum(pr.w);
    if (lane < 32) *reinterpret_cast<float4*>(&s_red[wave][c0]) = pr;
    __syncthreads();
    if (tid < kDV) {
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < kRowGroups / 2; ++w) sum += s_red[w][tid];
      s_vec[tid] = sum;
    }
    __syncthreads();
    // ---- err = beta (v - pred); S += k err^T; o = q^T S ----
    const float4 pd = *reinterpret_cast<const float4*>(&s_vec[c0]);
    const float4 er = make_float4(beta * (vv.x - pd.x), beta * (vv.y - pd.y), beta * (vv.z - pd.z), beta * (vv.w - pd.w));
    float4 ov = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const float kr = s_k[r0 + r], qr = s_q[r0 + r];
      S[r].x += kr * er.x; S[r].y += kr * er.y; S[r].z += kr * er.z; S[r].w += kr * er.w;
      ov.x += qr * S[r].x; ov.y += qr * S[r].y; ov.z += qr * S[r].z; ov.w += qr * S[r].w;
    }
    ov.x = xor32_sum(ov.x); ov.y = xor32_sum(ov.y);
    ov.z = xor32_sum(ov.z); ov.w = xor32_sum(ov.w);
    __syncthreads();  // s_red / s_vec reuse
    if (lane < 32) *reinterpret_cast<float4*>(&s_red[wave][c0]) = ov;
    __syncthreads();
    if (!GATE) {
      if (tid < kDV) {
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < kRowGroups / 2; ++w) sum += s_red[w][tid];
        p.out[vh * kDV + tid] = (uint16_t)f32_to_bf16_bits(sum);
      }
    } else {
      float core = 0.f;  // the head's bf16 output, element tid (threads 0 .. 127: waves 0 and 1)
      if (tid < kDV) {
#pragma unroll
        for (int w = 0; w < kRowGroups / 2; ++w) core += s_red[w][tid];
        core = round_bf16(core);
      }
      const float ss = wave_sum(core * core);
      if (lane == 0 && wave < 2) s_gn[wave] = ss;
      __syncthreads();
      if (tid < kDV) {
        const float inv = rsqrtf((s_gn[0] + s_gn[1]) / (float)kDV + p.eps);
        const float zz = bf16_bits_to_f32(p.z[vh * kDV + tid]);
        p.out[vh * kDV + tid] = (uint16_t)f32_to_bf16_bits(round_bf16(core * inv * p.norm_w[tid]) * silu_f32(zz));
      }
    }
    if (p.snap) {  // the state after this token (speculative verification's per-row snapshots)
      float* sn = p.snap + t * p.snap_ld + ((int64_t)b * p.NV + h) * kDK * kDV;
#pragma unroll
      for (int r = 0; r < kRows; ++r)
        store_nt(sn + (r0 + r) * kDV + c0, axk_u32x4{__float_as_uint(S[r].x), __float_as_uint(S[r].y),
                                                     __float_as_uint(S[r].z), __float_as_uint(S[r].w)});
    }
    __syncthreads();  // s_k / s_q / s_red / s_gn reuse by the next token
  }

  float* sout = p.state_out + ((int64_t)b * p.NV + h) * kDK * kDV;
#pragma unroll
  for (int r = 0; r < kRows; ++r)
    store_nt(sout + (r0 + r) * kDV + c0, axk_u32x4{__float_as_uint(S[r].x), __float_as_uint(S[r].y), __float_as_uint(S[r].z), __float_as_uint(S[r].w)});
}

}  // namespace

int axk_gdn_recurrent_strided(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* a,
                              const uint16_t* b, const float* a_log, const float* dt_bias, const float* state_in,
                              float* state_out, uint16_t* out, int64_t batch, int64_t tokens, int64_t num_k_heads,
                              int64_t num_v_heads, const AxkGdnStrides& ld, const AxkGdnGate* gate, int v_order,
                              hipStream_t stream, float* state_snap, int64_t snap_ld) {
  AXK_REQUIRE(q && k && v && a && b && a_log && dt_bias && state_in && state_out && out, AXK_E_NULL);
  AXK_REQUIRE(v_order == AXK_VORDER_GROUPED || v_order == AXK_VORDER_TILED, AXK_E_SHAPE);
  AXK_REQUIRE(!gate || (gate->norm_w && gate->z), AXK_E_NULL);
  AXK_REQUIRE(batch > 0 && tokens > 0 && num_k_heads > 0 && num_v_heads > 0, AXK_E_SHAPE);
  AXK_REQUIRE(num_v_heads % num_k_heads == 0, AXK_E_SHAPE);
  AXK_REQUIRE(batch * num_v_heads <= INT32_MAX && tokens <= INT32_MAX, AXK_E_SHAPE);
  AXK_REQUIRE(ld.q >= num_k_heads * kDK && ld.k >= num_k_heads * kDK && ld.v >= num_v_heads * kDV &&
                  ld.ab >= num_v_heads,
              AXK_E_SHAPE);
  AXK_REQUIRE(axk_aligned(state_in, 16) && axk_aligned(state_out, 16), AXK_E_ALIGN);
  const size_t sbytes = (size_t)batch * num_v_heads * kDK * kDV * 4;
  // in place is allowed (each workgroup reads its whole tile before writing it); partial overlap is not
  AXK_REQUIRE(state_in == state_out || !axk_overlap(state_in, sbytes, state_out, sbytes), AXK_E_ALIAS);
  const size_t obytes = (size_t)batch * tokens * num_v_heads * kDV * 2;
  AXK_REQUIRE(!axk_overlap(out, obytes, state_out, sbytes), AXK_E_ALIAS);
  if (state_snap) {  // snapshot t: [B, NV, DK, DV] at state_snap + t * snap_ld, none overlapping the states
    const int64_t per = batch * num_v_heads * kDK * kDV;
    AXK_REQUIRE(snap_ld >= per && axk_aligned(state_snap, 16) && snap_ld % 4 == 0, AXK_E_SHAPE);
    const size_t nbytes = (size_t)((tokens - 1) * snap_ld + per) * 4;
    AXK_REQUIRE(!axk_overlap(state_snap, nbytes, state_in, sbytes) && !axk_overlap(state_snap, nbytes, state_out, sbytes) &&
                    !axk_overlap(state_snap, nbytes, out, obytes),
                AXK_E_ALIAS);
  }
  GdnArgs p{q, k, v, a, b, a_log, dt_bias, state_in, state_out, out, (int)batch, (int)tokens, (int)num_k_heads,
            (int)num_v_heads, ld.q, ld.k, ld.v, ld.ab, gate ? gate->norm_w : nullptr, gate ? gate->z : nullptr,
            gate ? gate->eps : 0.f, state_snap, snap_ld,
            v_order == AXK_VORDER_TILED ? 1 : (int)(num_v_heads / num_k_heads)};
  AXK_LAUNCH_GATE();
  if (gate)
    hipLaunchKernelGGL(gdn_recurrent_kernel<true>, dim3((unsigned)(batch * num_v_heads)), dim3(kThreads), 0, stream, p);
  else
    hipLaunchKernelGGL(gdn_recurrent_kernel<false>, dim3((unsigned)(batch * num_v_heads)), dim3(kThreads), 0, stream, p);
  return axk_launch_status();
}

extern "C" int axk_gdn_recurrent(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* a,
                                 const uint16_t* b, const float* a_log, const float* dt_bias, const float* state_in,
                                 float* state_out, uint16_t* out, int64_t batch, int64_t tokens, int64_t num_k_heads,
                                 int64_t num_v_heads, int64_t head_k_dim, int64_t head_v_dim, axk_stream_t stream) {
  AXK_REQUIRE(head_k_dim == kDK && head_v_dim == kDV, AXK_E_SHAPE);
  const AxkGdnStrides ld{num_k_heads * kDK, num_k_heads * kDK, num_v_heads * kDV, num_v_heads};
  return axk_gdn_recurrent_strided(q, k, v, a, b, a_log, dt_bias, state_in, state_out, out, batch, tokens,
                                   num_k_heads, num_v_heads, ld, nullptr, AXK_VORDER_GROUPED, axk_stream(stream));
}
