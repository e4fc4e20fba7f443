// One hybrid decode layer per call, composed from the library's kernels on the caller's stream: the GDN layer
// (models/qwen35_35b_a3b/src/70b0fbc/q35_step.py gdn_layer 149-183) and the attention layer (attn_block 186-280),
// each followed by the MLP block (mlp_block 118-142). The projections of the attention / GDN paths and the MLP each take
// a weight format (AXK_WFMT_*): FP8 E4M3 with per-output-channel fp32 scales (the config of the hybrid decode group),
// MXFP8 (the 35B manifest's layer weights) or MXFP4 (the 9B / 27B manifests' and the group's MLP). Every intermediate is
// a bf16 tensor in the caller's workspace, rounded where the reference rounds (each projection's output, each
// glue op's output). Projections that share an input run as one grouped launch (GDN: qkv | z | b | a, whose qkv
// epilogue also runs the causal conv1d + SiLU; attention: q | k | v); the GDN kernel applies the gated output norm
// to each head's row; one launch prepares q / k / v (norms, RoPE, the paged KV write); the MLP's gate and up
// projections run as one launch whose epilogue applies SwiGLU, and the down projection's epilogue adds the
// residual. Every fused step rounds exactly where the separate op rounds. No allocation, no host
// synchronisation: a layer is graph-capturable.
#include "axk_host.h"

namespace {

size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

// Carves consecutive 256-byte aligned buffers out of a workspace (or, with base == nullptr, only sizes them).
struct Carver {
  unsigned char* base;
  size_t off = 0;
  template <typename T>
  T* take(size_t count) {
    T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
    off = al256(off + count * sizeof(T));
    return p;
  }
};

struct MlpWeights {
  const uint8_t *gate_w, *up_w, *down_w;
  const void *gate_s, *up_s, *down_s;
};

// The grouped kernel's format of a weight format code (AXK_WFMT_*), or -1.
int mx_fmt_of(int wfmt) {
  switch (wfmt) {
    case AXK_WFMT_FP8_CHANNEL: return AXK_MX_FP8;
    case AXK_WFMT_MXFP8: return AXK_MX_MXFP8;
    case AXK_WFMT_MXFP4: return AXK_MX_MXFP4;
    case AXK_WFMT_NVFP4: return AXK_MX_NVFP4;
    default: return -1;
  }
}

// One projection of the group: per-channel f32 scales [N] (FP8) or E8M0 block scales [N, K/32] (MX formats).
AxkMxMat proj_mat(int wfmt, const uint8_t* w, const void* s, void* out, int64_t n) {
  if (wfmt == AXK_WFMT_FP8_CHANNEL) return AxkMxMat{w, nullptr, static_cast<const float*>(s), nullptr, out, n, n};
  if (wfmt == AXK_WFMT_NVFP4) {  // s: the host descriptor of the E4M3 block scales and the fp32 scale2
    const axk_nvfp4_scales* ns = static_cast<const axk_nvfp4_scales*>(s);
    return AxkMxMat{w, ns ? ns->block_scales : nullptr, nullptr, nullptr, out, n, n, ns ? ns->scale2 : nullptr};
  }
  return AxkMxMat{w, static_cast<const uint8_t*>(s), nullptr, nullptr, out, n, n};
}

struct MlpBufs {
  uint16_t *x1, *h2, *act;
};

MlpBufs carve_mlp(Carver& c, int64_t B, int64_t H, int64_t F) {
  MlpBufs m;
  m.x1 = c.take<uint16_t>(B * H);
  m.h2 = c.take<uint16_t>(B * H);
  m.act = c.take<uint16_t>(B * F);
  return m;
}

#define AXK_TRY(call)            \
  do {                           \
    const int rc_ = (call);      \
    if (rc_ != AXK_OK) return rc_; \
  } while (0)

// x1 = x + y; h2 = rmsnorm(x1, ln2); out = x1 + down(silu(gate h2) * up h2)  (mlp_block, q35_step.py:118-142):
// three launches (the norm, gate | up with SwiGLU, down with the residual add). wfmt: the MLP weights' format.
int mlp_residual(const uint16_t* x, const uint16_t* y, const float* ln2, const MlpWeights& w, int wfmt, uint16_t* out,
                 const MlpBufs& m, int64_t B, int64_t H, int64_t F, float eps, axk_stream_t st) {
  AXK_TRY(axk_add_rmsnorm(x, y, ln2, m.x1, m.h2, B, H, eps, st));
  const AxkMxMat gate_up[2] = {proj_mat(wfmt, w.gate_w, w.gate_s, m.act, F), proj_mat(wfmt, w.up_w, w.up_s, m.act, F)};
  AXK_TRY(axk_mx_group(mx_fmt_of(wfmt), m.h2, H, gate_up, 2, AXK_MX_EPI_SWIGLU, nullptr, 0, nullptr, AXK_DT_BF16, B,
                       H, nullptr, axk_stream(st)));
  const AxkMxMat down = proj_mat(wfmt, w.down_w, w.down_s, out, H);
  return axk_mx_group(mx_fmt_of(wfmt), m.act, F, &down, 1, AXK_MX_EPI_RES, m.x1, H, nullptr, AXK_DT_BF16, B, F,
                      nullptr, axk_stream(st));
}

// The MoE block's buffers beside the dense MLP's (whose act holds the shared expert's activations).
struct MoeBufs {
  float* y_sh;     // [B, H] the shared expert's fp32 output
  float* logits;   // [B, E]
  int32_t* ids;    // [B, K]
  float* wts;      // [B, K]
  void* mws;       // the routed experts' workspace
  size_t mws_bytes;
};

// Shapes the MoE block takes beside the layer's (0 when unsupported).
size_t moe_ws_bytes(int64_t B, int64_t H, const axk_moe_block& m) {
  if (m.num_experts <= 0 || m.top_k <= 0 || m.expert_inter <= 0) return 0;
  return axk_moe_workspace_size(B, H, m.num_experts, m.top_k, m.expert_inter, 0);
}

MoeBufs carve_moe(Carver& c, int64_t B, int64_t H, const axk_moe_block& m) {
  MoeBufs e;
  e.y_sh = c.take<float>(B * H);
  e.logits = c.take<float>(B * m.num_experts);
  e.ids = c.take<int32_t>(B * m.top_k);
  e.wts = c.take<float>(B * m.top_k);
  if (c.base) {  // the caller's routing outputs where given
    if (m.logits) e.logits = m.logits;
    if (m.topk_ids) e.ids = m.topk_ids;
    if (m.topk_weights) e.wts = m.topk_weights;
  }
  e.mws_bytes = moe_ws_bytes(B, H, m);
  e.mws = c.take<unsigned char>(e.mws_bytes);
  return e;
}

// moe_full (q35_layer_mc.py:797-853) after the layer's first half: x1 = x + y; h2 = rmsnorm(x1, ln2); the shared
// expert (the layer's MLP weights in wfmt: gate | up with SwiGLU, then down into fp32 y_sh); the router, top-K and
// the routed MXFP4 experts, whose combine writes out = x1 + sigmoid(h2 . w_shg) y_sh + the routed sum.
int moe_residual(const uint16_t* x, const uint16_t* y, const float* ln2, const MlpWeights& w, int wfmt,
                 const axk_moe_block& m, uint16_t* out, const MlpBufs& mb, const MoeBufs& eb, int64_t B, int64_t H,
                 int64_t F, float eps, axk_stream_t st) {
  AXK_TRY(axk_add_rmsnorm(x, y, ln2, mb.x1, mb.h2, B, H, eps, st));
  const AxkMxMat gate_up[2] = {proj_mat(wfmt, w.gate_w, w.gate_s, mb.act, F), proj_mat(wfmt, w.up_w, w.up_s, mb.act, F)};
  AXK_TRY(axk_mx_group(mx_fmt_of(wfmt), mb.h2, H, gate_up, 2, AXK_MX_EPI_SWIGLU, nullptr, 0, nullptr, AXK_DT_BF16, B,
                       H, nullptr, axk_stream(st)));
  const AxkMxMat down = proj_mat(wfmt, w.down_w, w.down_s, eb.y_sh, H);
  AXK_TRY(axk_mx_group(mx_fmt_of(wfmt), mb.act, F, &down, 1, AXK_MX_EPI_PLAIN, nullptr, 0, nullptr, AXK_DT_F32, B, F,
                       nullptr, axk_stream(st)));
  return axk_moe_decode_shared_given(mb.h2, mb.x1, m.w_router, m.w_shg, eb.y_sh, m.e_gw, m.e_gs, m.e_dw, m.e_ds, out,
                                     eb.logits, eb.ids, eb.wts, B, H, m.num_experts, m.top_k, m.expert_inter,
                                     m.norm_topk_prob, eb.mws, eb.mws_bytes, st);
}

// Projections of one input a [m, k] in weight format wfmt (bf16 outputs) as one grouped launch; conv (optional)
// runs the causal conv1d + SiLU on the first matrix's output.
int projs(int wfmt, const uint16_t* a, int64_t lda, const AxkMxMat* mats, int count, int64_t m, int64_t k,
          axk_stream_t st, const AxkConvEpi* conv = nullptr) {
  return axk_mx_group(mx_fmt_of(wfmt), a, lda, mats, count, AXK_MX_EPI_PLAIN, nullptr, 0, nullptr, AXK_DT_BF16, m, k,
                      conv, axk_stream(st));
}

struct GdnBufs {
  uint16_t *h, *z, *bb, *aa, *mixed, *gated, *y;
  MlpBufs mlp;
};

GdnBufs carve_gdn(Carver& c, int64_t B, int64_t H, int64_t NK, int64_t NV, int64_t DH, int64_t F) {
  const int64_t KD = NK * DH, VD = NV * DH, C = 2 * KD + VD;
  GdnBufs g;
  g.h = c.take<uint16_t>(B * H);
  g.z = c.take<uint16_t>(B * VD);
  g.bb = c.take<uint16_t>(B * NV);
  g.aa = c.take<uint16_t>(B * NV);
  g.mixed = c.take<uint16_t>(B * C);
  g.gated = c.take<uint16_t>(B * VD);
  g.y = c.take<uint16_t>(B * H);
  g.mlp = carve_mlp(c, B, H, F);
  return g;
}

struct AttnBufs {
  uint16_t *h, *qg, *kk, *vv, *q, *attn, *gated, *y;
  void* pws;
  size_t pws_bytes;
  MlpBufs mlp;
};

AttnBufs carve_attn(Carver& c, int64_t B, int64_t H, int64_t HQ, int64_t HKV, int64_t D, int64_t F) {
  AttnBufs a;
  a.h = c.take<uint16_t>(B * H);
  a.qg = c.take<uint16_t>(B * HQ * 2 * D);
  a.kk = c.take<uint16_t>(B * HKV * D);
  a.vv = c.take<uint16_t>(B * HKV * D);
  a.q = c.take<uint16_t>(B * HQ * D);
  a.attn = c.take<uint16_t>(B * HQ * D);
  a.gated = c.take<uint16_t>(B * HQ * D);
  a.y = c.take<uint16_t>(B * H);
  a.pws_bytes = axk_paged_decode_workspace_size(B, HQ, HKV, D);
  a.pws = c.take<unsigned char>(a.pws_bytes);
  a.mlp = carve_mlp(c, B, H, F);
  return a;
}

int check_common(int64_t B, int64_t H, int64_t F) {
  AXK_REQUIRE(B > 0 && B <= 4096 && H > 0 && F > 0, AXK_E_SHAPE);
  AXK_REQUIRE(H % 256 == 0 && F % 256 == 0, AXK_E_SHAPE);  // whole MXFP4 / FP8 row segments
  return AXK_OK;
}

}  // namespace

namespace {

// Workspace of a GDN decode layer, with the MoE block's buffers after the layer's when moe is given.
size_t gdn_ws_bytes(int64_t B, int64_t H, int64_t NK, int64_t NV, int64_t DH, int64_t F, const axk_moe_block* moe) {
  if (check_common(B, H, F) != AXK_OK || DH != 128 || NK <= 0 || NV <= 0 || NV % NK != 0) return 0;
  if (moe && moe_ws_bytes(B, H, *moe) == 0) return 0;
  Carver c{nullptr};
  carve_gdn(c, B, H, NK, NV, DH, F);
  if (moe) carve_moe(c, B, H, *moe);
  return c.off;
}

int gdn_layer_impl(const uint16_t* x, const float* ln1, const uint8_t* w_qkv, const void* s_qkv, const uint8_t* w_z,
                   const void* s_z, const uint8_t* w_b, const void* s_b, const uint8_t* w_a, const void* s_a,
                   const uint16_t* conv_w, const float* a_log, const float* dt_bias, const float* norm_w,
                   const uint8_t* w_out, const void* s_out, const float* ln2, const uint8_t* mlp_gate_w,
                   const void* mlp_gate_s, const uint8_t* mlp_up_w, const void* mlp_up_s, const uint8_t* mlp_down_w,
                   const void* mlp_down_s, const axk_moe_block* moe, const float* state_in, const uint16_t* conv_in,
                   uint16_t* out, float* state_out, uint16_t* conv_out, int64_t batch, int64_t hidden,
                   int64_t num_k_heads, int64_t num_v_heads, int64_t head_dim, int64_t conv_kernel, int64_t inter,
                   float eps, int proj_fmt, int mlp_fmt, int v_order, void* workspace, size_t workspace_bytes,
                   axk_stream_t stream) {
  AXK_REQUIRE(x && ln1 && w_qkv && s_qkv && w_z && s_z && w_b && s_b && w_a && s_a && conv_w && a_log && dt_bias &&
                  norm_w && w_out && s_out && ln2 && mlp_gate_w && mlp_gate_s && mlp_up_w && mlp_up_s &&
                  mlp_down_w && mlp_down_s && state_in && conv_in && out && state_out && conv_out,
              AXK_E_NULL);
  AXK_REQUIRE(mx_fmt_of(proj_fmt) >= 0 && mx_fmt_of(mlp_fmt) >= 0, AXK_E_DTYPE);
  const size_t need = gdn_ws_bytes(batch, hidden, num_k_heads, num_v_heads, head_dim, inter, moe);
  AXK_REQUIRE(need > 0, AXK_E_SHAPE);
  AXK_REQUIRE(workspace && workspace_bytes >= need && axk_aligned(workspace, 256), AXK_E_WORKSPACE);
  const int64_t B = batch, H = hidden, NK = num_k_heads, NV = num_v_heads, DH = head_dim, F = inter;
  const int64_t KD = NK * DH, VD = NV * DH, C = 2 * KD + VD;
  Carver c{static_cast<unsigned char*>(workspace)};
  const GdnBufs g = carve_gdn(c, B, H, NK, NV, DH, F);
  const MoeBufs eb = moe ? carve_moe(c, B, H, *moe) : MoeBufs{};
  const MlpWeights mw{mlp_gate_w, mlp_up_w, mlp_down_w, mlp_gate_s, mlp_up_s, mlp_down_s};
  auto body = [&]() -> int {
    AXK_TRY(axk_rmsnorm(x, H, ln1, g.h, H, B, H, eps, stream));
    // qkv | z | b | a, the qkv output through the causal conv1d + SiLU (mixed) as it is stored
    const AxkMxMat proj[4] = {proj_mat(proj_fmt, w_qkv, s_qkv, g.mixed, C), proj_mat(proj_fmt, w_z, s_z, g.z, VD),
                              proj_mat(proj_fmt, w_b, s_b, g.bb, NV), proj_mat(proj_fmt, w_a, s_a, g.aa, NV)};
    const AxkConvEpi conv{conv_w, conv_in, conv_out, conv_kernel};
    AXK_TRY(projs(proj_fmt, g.h, H, proj, 4, B, H, stream, &conv));
    // q, k, v are the conv output's channel ranges [0, KD), [KD, 2 KD), [2 KD, C) of each sequence's row; each
    // head's output row leaves through the gated output norm
    const AxkGdnStrides ld{C, C, C, NV};
    const AxkGdnGate gate{norm_w, g.z, eps};
    AXK_TRY(axk_gdn_recurrent_strided(g.mixed, g.mixed + KD, g.mixed + 2 * KD, g.aa, g.bb, a_log, dt_bias, state_in,
                                      state_out, g.gated, B, 1, NK, NV, ld, &gate, v_order, axk_stream(stream)));
    const AxkMxMat o = proj_mat(proj_fmt, w_out, s_out, g.y, H);
    AXK_TRY(projs(proj_fmt, g.gated, VD, &o, 1, B, VD, stream));
    if (moe) return moe_residual(x, g.y, ln2, mw, mlp_fmt, *moe, out, g.mlp, eb, B, H, F, eps, stream);
    return mlp_residual(x, g.y, ln2, mw, mlp_fmt, out, g.mlp, B, H, F, eps, stream);
  };
  {
    const AxkValidateScope check_only;  // every sub-call's checks before the first launch
    AXK_TRY(body());
  }
  return body();
}

// Workspace of an attention decode layer, with the MoE block's buffers after the layer's when moe is given.
size_t attn_ws_bytes(int64_t B, int64_t H, int64_t HQ, int64_t HKV, int64_t D, int64_t F, const axk_moe_block* moe) {
  if (check_common(B, H, F) != AXK_OK || axk_paged_decode_workspace_size(B, HQ, HKV, D) == 0) return 0;
  if (moe && moe_ws_bytes(B, H, *moe) == 0) return 0;
  Carver c{nullptr};
  carve_attn(c, B, H, HQ, HKV, D, F);
  if (moe) carve_moe(c, B, H, *moe);
  return c.off;
}

int attn_layer_impl(const uint16_t* x, const float* ln1, const uint8_t* w_q, const void* s_q, const uint8_t* w_k,
                    const void* s_k, const uint8_t* w_v, const void* s_v, const float* q_norm, const float* k_norm,
                    const uint16_t* cos, const uint16_t* sin, uint16_t* kv_cache, const int32_t* indptr,
                    const int32_t* indices, const int32_t* last_page_len, const int32_t* cache_location,
                    const uint8_t* w_o, const void* s_o, const float* ln2, const uint8_t* mlp_gate_w,
                    const void* mlp_gate_s, const uint8_t* mlp_up_w, const void* mlp_up_s, const uint8_t* mlp_down_w,
                    const void* mlp_down_s, const axk_moe_block* moe, uint16_t* out, int64_t batch, int64_t hidden,
                    int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t rot, int64_t page_size,
                    int64_t num_pages, int64_t inter, float eps, float sm_scale, int proj_fmt, int mlp_fmt,
                    void* workspace, size_t workspace_bytes, axk_stream_t stream) {
  AXK_REQUIRE(x && ln1 && w_q && s_q && w_k && s_k && w_v && s_v && q_norm && k_norm && kv_cache && indptr &&
                  indices && last_page_len && cache_location && w_o && s_o && ln2 && mlp_gate_w && mlp_gate_s &&
                  mlp_up_w && mlp_up_s && mlp_down_w && mlp_down_s && out && (rot == 0 || (cos && sin)),
              AXK_E_NULL);
  AXK_REQUIRE(mx_fmt_of(proj_fmt) >= 0 && mx_fmt_of(mlp_fmt) >= 0, AXK_E_DTYPE);
  const size_t need = attn_ws_bytes(batch, hidden, num_qo_heads, num_kv_heads, head_dim, inter, moe);
  AXK_REQUIRE(need > 0, AXK_E_SHAPE);
  AXK_REQUIRE(workspace && workspace_bytes >= need && axk_aligned(workspace, 256), AXK_E_WORKSPACE);
  const int64_t B = batch, H = hidden, HQ = num_qo_heads, HKV = num_kv_heads, D = head_dim, F = inter;
  Carver c{static_cast<unsigned char*>(workspace)};
  const AttnBufs a = carve_attn(c, B, H, HQ, HKV, D, F);
  const MoeBufs eb = moe ? carve_moe(c, B, H, *moe) : MoeBufs{};
  const MlpWeights mw{mlp_gate_w, mlp_up_w, mlp_down_w, mlp_gate_s, mlp_up_s, mlp_down_s};
  auto body = [&]() -> int {
    AXK_TRY(axk_rmsnorm(x, H, ln1, a.h, H, B, H, eps, stream));
    const AxkMxMat proj[3] = {proj_mat(proj_fmt, w_q, s_q, a.qg, HQ * 2 * D),  // per head [q | gate]
                              proj_mat(proj_fmt, w_k, s_k, a.kk, HKV * D), proj_mat(proj_fmt, w_v, s_v, a.vv, HKV * D)};
    AXK_TRY(projs(proj_fmt, a.h, H, proj, 3, B, H, stream));
    AXK_TRY(axk_attn_qkv_prep(a.qg, a.kk, a.vv, q_norm, k_norm, cos, sin, a.q, kv_cache, cache_location, B, HQ, HKV,
                              D, rot, page_size, num_pages, eps, axk_stream(stream)));
    // the attention with its output gate applied as each row is written: gated = bf16(attn * sigmoid(gate))
    AXK_TRY(axk_paged_decode_gated(a.q, kv_cache, indptr, indices, last_page_len, a.qg + D, 2 * D, a.gated, B, HQ,
                                   HKV, D, page_size, num_pages, sm_scale, a.pws, a.pws_bytes, axk_stream(stream)));
    const AxkMxMat o = proj_mat(proj_fmt, w_o, s_o, a.y, H);
    AXK_TRY(projs(proj_fmt, a.gated, HQ * D, &o, 1, B, HQ * D, stream));
    if (moe) return moe_residual(x, a.y, ln2, mw, mlp_fmt, *moe, out, a.mlp, eb, B, H, F, eps, stream);
    return mlp_residual(x, a.y, ln2, mw, mlp_fmt, out, a.mlp, B, H, F, eps, stream);
  };
  {
    const AxkValidateScope check_only;  // every sub-call's checks before the first launch
    AXK_TRY(body());
  }
  return body();
}

}  // namespace

extern "C" size_t axk_gdn_layer_workspace_size(int64_t batch, int64_t hidden, int64_t num_k_heads,
                                               int64_t num_v_heads, int64_t head_dim, int64_t inter) {
  return gdn_ws_bytes(batch, hidden, num_k_heads, num_v_heads, head_dim, inter, nullptr);
}

extern "C" int axk_gdn_layer_decode(
    const uint16_t* x, const float* ln1, const uint8_t* w_qkv, const void* s_qkv, const uint8_t* w_z, const void* s_z,
    const uint8_t* w_b, const void* s_b, const uint8_t* w_a, const void* s_a, const uint16_t* conv_w,
    const float* a_log, const float* dt_bias, const float* norm_w, const uint8_t* w_out, const void* s_out,
    const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s, const uint8_t* mlp_up_w,
    const void* mlp_up_s, const uint8_t* mlp_down_w, const void* mlp_down_s, const float* state_in,
    const uint16_t* conv_in, uint16_t* out, float* state_out, uint16_t* conv_out, int64_t batch, int64_t hidden,
    int64_t num_k_heads, int64_t num_v_heads, int64_t head_dim, int64_t conv_kernel, int64_t inter, float eps,
    int proj_fmt, int mlp_fmt, int v_order, void* workspace, size_t workspace_bytes, axk_stream_t stream) {
  return gdn_layer_impl(x, ln1, w_qkv, s_qkv, w_z, s_z, w_b, s_b, w_a, s_a, conv_w, a_log, dt_bias, norm_w, w_out,
                        s_out, ln2, mlp_gate_w, mlp_gate_s, mlp_up_w, mlp_up_s, mlp_down_w, mlp_down_s, nullptr,
                        state_in, conv_in, out, state_out, conv_out, batch, hidden, num_k_heads, num_v_heads,
                        head_dim, conv_kernel, inter, eps, proj_fmt, mlp_fmt, v_order, workspace, workspace_bytes,
                        stream);
}

extern "C" size_t axk_gdn_layer_moe_workspace_size(int64_t batch, int64_t hidden, int64_t num_k_heads,
                                                   int64_t num_v_heads, int64_t head_dim, int64_t inter,
                                                   const axk_moe_block* moe) {
  return moe ? gdn_ws_bytes(batch, hidden, num_k_heads, num_v_heads, head_dim, inter, moe) : 0;
}

extern "C" int axk_gdn_layer_decode_moe(
    const uint16_t* x, const float* ln1, const uint8_t* w_qkv, const void* s_qkv, const uint8_t* w_z, const void* s_z,
    const uint8_t* w_b, const void* s_b, const uint8_t* w_a, const void* s_a, const uint16_t* conv_w,
    const float* a_log, const float* dt_bias, const float* norm_w, const uint8_t* w_out, const void* s_out,
    const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s, const uint8_t* mlp_up_w,
    const void* mlp_up_s, const uint8_t* mlp_down_w, const void* mlp_down_s, const axk_moe_block* moe,
    const float* state_in, const uint16_t* conv_in, uint16_t* out, float* state_out, uint16_t* conv_out,
    int64_t batch, int64_t hidden, int64_t num_k_heads, int64_t num_v_heads, int64_t head_dim, int64_t conv_kernel,
    int64_t inter, float eps, int proj_fmt, int mlp_fmt, int v_order, void* workspace, size_t workspace_bytes,
    axk_stream_t stream) {
  AXK_REQUIRE(moe, AXK_E_NULL);
  return gdn_layer_impl(x, ln1, w_qkv, s_qkv, w_z, s_z, w_b, s_b, w_a, s_a, conv_w, a_log, dt_bias, norm_w, w_out,
                        s_out, ln2, mlp_gate_w, mlp_gate_s, mlp_up_w, mlp_up_s, mlp_down_w, mlp_down_s, moe,
                        state_in, conv_in, out, state_out, conv_out, batch, hidden, num_k_heads, num_v_heads,
                        head_dim, conv_kernel, inter, eps, proj_fmt, mlp_fmt, v_order, workspace, workspace_bytes,
                        stream);
}

extern "C" size_t axk_attn_layer_workspace_size(int64_t batch, int64_t hidden, int64_t num_qo_heads,
                                                int64_t num_kv_heads, int64_t head_dim, int64_t inter) {
  return attn_ws_bytes(batch, hidden, num_qo_heads, num_kv_heads, head_dim, inter, nullptr);
}

extern "C" int axk_attn_layer_decode(
    const uint16_t* x, const float* ln1, const uint8_t* w_q, const void* s_q, const uint8_t* w_k, const void* s_k,
    const uint8_t* w_v, const void* s_v, const float* q_norm, const float* k_norm, const uint16_t* cos,
    const uint16_t* sin, uint16_t* kv_cache, const int32_t* indptr, const int32_t* indices,
    const int32_t* last_page_len, const int32_t* cache_location, const uint8_t* w_o, const void* s_o,
    const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s, const uint8_t* mlp_up_w,
    const void* mlp_up_s, const uint8_t* mlp_down_w, const void* mlp_down_s, uint16_t* out, int64_t batch,
    int64_t hidden, int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t rot, int64_t page_size,
    int64_t num_pages, int64_t inter, float eps, float sm_scale, int proj_fmt, int mlp_fmt, void* workspace,
    size_t workspace_bytes, axk_stream_t stream) {
  return attn_layer_impl(x, ln1, w_q, s_q, w_k, s_k, w_v, s_v, q_norm, k_norm, cos, sin, kv_cache, indptr, indices,
                         last_page_len, cache_location, w_o, s_o, ln2, mlp_gate_w, mlp_gate_s, mlp_up_w, mlp_up_s,
                         mlp_down_w, mlp_down_s, nullptr, out, batch, hidden, num_qo_heads, num_kv_heads, head_dim,
                         rot, page_size, num_pages, inter, eps, sm_scale, proj_fmt, mlp_fmt, workspace,
                         workspace_bytes, stream);
}

extern "C" size_t axk_attn_layer_moe_workspace_size(int64_t batch, int64_t hidden, int64_t num_qo_heads,
                                                    int64_t num_kv_heads, int64_t head_dim, int64_t inter,
                                                    const axk_moe_block* moe) {
  return moe ? attn_ws_bytes(batch, hidden, num_qo_heads, num_kv_heads, head_dim, inter, moe) : 0;
}

extern "C" int axk_attn_layer_decode_moe(
    const uint16_t* x, const float* ln1, const uint8_t* w_q, const void* s_q, const uint8_t* w_k, const void* s_k,
    const uint8_t* w_v, const void* s_v, const float* q_norm, const float* k_norm, const uint16_t* cos,
    const uint16_t* sin, uint16_t* kv_cache, const int32_t* indptr, const int32_t* indices,
    const int32_t* last_page_len, const int32_t* cache_location, const uint8_t* w_o, const void* s_o,
    const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s, const uint8_t* mlp_up_w,
    const void* mlp_up_s, const uint8_t* mlp_down_w, const void* mlp_down_s, const axk_moe_block* moe,
    uint16_t* out, int64_t batch, int64_t hidden, int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim,
    int64_t rot, int64_t page_size, int64_t num_pages, int64_t inter, float eps, float sm_scale, int proj_fmt,
    int mlp_fmt, void* workspace, size_t workspace_bytes, axk_stream_t stream) {
  AXK_REQUIRE(moe, AXK_E_NULL);
  return attn_layer_impl(x, ln1, w_q, s_q, w_k, s_k, w_v, s_v, q_norm, k_norm, cos, sin, kv_cache, indptr, indices,
                         last_page_len, cache_location, w_o, s_o, ln2, mlp_gate_w, mlp_gate_s, mlp_up_w, mlp_up_s,
                         mlp_down_w, mlp_down_s, moe, out, batch, hidden, num_qo_heads, num_kv_heads, head_dim, rot,
                         page_size, num_pages, inter, eps, sm_scale, proj_fmt, mlp_fmt, workspace, workspace_bytes,
                         stream);
}

// ---------------------------------------------------------------------------------------------
// Speculative verification: the decode layers over T consecutive new rows per sequence in one call
// (models/qwen38_27b/verify/verify_group_m4.py:1-9: every projection shared by the T rows, so each weight is read
// once; only the row recurrences run in order: the GDN conv and delta-rule state, each row's KV write and causal
// attention). Row t of sequence b is x row b T + t. The GDN state and conv state after every row are written to
// optional per-row snapshots (the verify group's ssnap / cqsnap / cksnap / cvsnap), so a host that accepts a draft
// prefix rolls back to that row's snapshot.
// ---------------------------------------------------------------------------------------------
namespace {

constexpr int64_t kMaxVerifyTokens = 16;

struct GdnVerifyBufs {
  uint16_t *h, *qkv, *z, *bb, *aa, *mixed, *gated, *y;
  MlpBufs mlp;
};

GdnVerifyBufs carve_gdn_verify(Carver& c, int64_t R, int64_t H, int64_t NK, int64_t NV, int64_t DH, int64_t F) {
  const int64_t KD = NK * DH, VD = NV * DH, C = 2 * KD + VD;
  GdnVerifyBufs g;
  g.h = c.take<uint16_t>(R * H);
  g.qkv = c.take<uint16_t>(R * C);
  g.z = c.take<uint16_t>(R * VD);
  g.bb = c.take<uint16_t>(R * NV);
  g.aa = c.take<uint16_t>(R * NV);
  g.mixed = c.take<uint16_t>(R * C);
  g.gated = c.take<uint16_t>(R * VD);
  g.y = c.take<uint16_t>(R * H);
  g.mlp = carve_mlp(c, R, H, F);
  return g;
}

struct AttnVerifyBufs {
  uint16_t *h, *qg, *kk, *vv, *q, *attn, *gated, *y;
  int32_t* qo_indptr;
  MlpBufs mlp;
};

AttnVerifyBufs carve_attn_verify(Carver& c, int64_t B, int64_t R, int64_t H, int64_t HQ, int64_t HKV, int64_t D,
                                 int64_t F) {
  AttnVerifyBufs a;
  a.h = c.take<uint16_t>(R * H);
  a.qg = c.take<uint16_t>(R * HQ * 2 * D);
  a.kk = c.take<uint16_t>(R * HKV * D);
  a.vv = c.take<uint16_t>(R * HKV * D);
  a.q = c.take<uint16_t>(R * HQ * D);
  a.attn = c.take<uint16_t>(R * HQ * D);
  a.gated = c.take<uint16_t>(R * HQ * D);
  a.y = c.take<uint16_t>(R * H);
  a.qo_indptr = c.take<int32_t>(B + 1);
  a.mlp = carve_mlp(c, R, H, F);
  return a;
}

int check_verify(int64_t B, int64_t T, int64_t H, int64_t F) {
  AXK_REQUIRE(T >= 1 && T <= kMaxVerifyTokens && B > 0 && B <= 4096 / T, AXK_E_SHAPE);
  return check_common(B * T, H, F);
}

// Prefill: up to kMaxPrefillTokens new tokens per sequence, kMaxPrefillRows rows per call.
constexpr int64_t kMaxPrefillTokens = 1 << 16, kMaxPrefillRows = 1 << 17;
int check_prefill(int64_t B, int64_t T, int64_t H, int64_t F) {
  AXK_REQUIRE(T >= 1 && T <= kMaxPrefillTokens && B > 0 && B <= kMaxPrefillRows / T, AXK_E_SHAPE);
  AXK_REQUIRE(H > 0 && F > 0 && H % 256 == 0 && F % 256 == 0, AXK_E_SHAPE);
  return AXK_OK;
}

size_t attn_rows_ws(int64_t B, int64_t T, int64_t H, int64_t HQ, int64_t HKV, int64_t D, int64_t F,
                    const axk_moe_block* moe = nullptr) {
  if (HQ <= 0 || HKV <= 0 || HQ % HKV != 0 || !(D == 64 || D == 128 || D == 256)) return 0;
  if (moe && moe_ws_bytes(B * T, H, *moe) == 0) return 0;
  Carver c{nullptr};
  carve_attn_verify(c, B, B * T, H, HQ, HKV, D, F);
  if (moe) carve_moe(c, B * T, H, *moe);
  return c.off;
}

// The attention layer over T new rows per sequence (verify and prefill): every projection over the B T rows; each
// row's K / V into the cache at its own location; causal attention of the rows over the history and the rows up to
// themselves (the T rows are the last T tokens of the sequence's page table); the output gate, o projection and MLP.
int attn_rows_impl(const uint16_t* x, const float* ln1, const uint8_t* w_q, const void* s_q, const uint8_t* w_k,
                   const void* s_k, const uint8_t* w_v, const void* s_v, const float* q_norm, const float* k_norm,
                   const uint16_t* cos, const uint16_t* sin, uint16_t* kv_cache, const int32_t* indptr,
                   const int32_t* indices, const int32_t* last_page_len, const int32_t* cache_location,
                   const uint8_t* w_o, const void* s_o, const float* ln2, const uint8_t* mlp_gate_w,
                   const void* mlp_gate_s, const uint8_t* mlp_up_w, const void* mlp_up_s, const uint8_t* mlp_down_w,
                   const void* mlp_down_s, const axk_moe_block* moe, uint16_t* out, int64_t batch, int64_t tokens,
                   int64_t hidden, int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t rot,
                   int64_t page_size, int64_t num_pages, int64_t inter, float eps, float sm_scale, int proj_fmt,
                   int mlp_fmt, void* workspace, size_t workspace_bytes, axk_stream_t stream, size_t need) {
  AXK_REQUIRE(x && ln1 && w_q && s_q && w_k && s_k && w_v && s_v && q_norm && k_norm && kv_cache && indptr &&
                  indices && last_page_len && cache_location && w_o && s_o && ln2 && mlp_gate_w && mlp_gate_s &&
                  mlp_up_w && mlp_up_s && mlp_down_w && mlp_down_s && out && (rot == 0 || (cos && sin)),
              AXK_E_NULL);
  AXK_REQUIRE(mx_fmt_of(proj_fmt) >= 0 && mx_fmt_of(mlp_fmt) >= 0, AXK_E_DTYPE);
  AXK_REQUIRE(need > 0, AXK_E_SHAPE);
  AXK_REQUIRE(workspace && workspace_bytes >= need && axk_aligned(workspace, 256), AXK_E_WORKSPACE);
  const int64_t B = batch, T = tokens, R = B * T, H = hidden, HQ = num_qo_heads, HKV = num_kv_heads, D = head_dim,
                F = inter;
  Carver c{static_cast<unsigned char*>(workspace)};
  const AttnVerifyBufs a = carve_attn_verify(c, B, R, H, HQ, HKV, D, F);
  const MoeBufs eb = moe ? carve_moe(c, R, H, *moe) : MoeBufs{};
  const MlpWeights mw{mlp_gate_w, mlp_up_w, mlp_down_w, mlp_gate_s, mlp_up_s, mlp_down_s};
  auto body = [&]() -> int {
    AXK_TRY(axk_rmsnorm(x, H, ln1, a.h, H, R, H, eps, stream));
    const AxkMxMat proj[3] = {proj_mat(proj_fmt, w_q, s_q, a.qg, HQ * 2 * D),  // per head [q | gate]
                              proj_mat(proj_fmt, w_k, s_k, a.kk, HKV * D), proj_mat(proj_fmt, w_v, s_v, a.vv, HKV * D)};
    AXK_TRY(projs(proj_fmt, a.h, H, proj, 3, R, H, stream));
    AXK_TRY(axk_attn_qkv_prep(a.qg, a.kk, a.vv, q_norm, k_norm, cos, sin, a.q, kv_cache, cache_location, R, HQ, HKV,
                              D, rot, page_size, num_pages, eps, axk_stream(stream)));
    AXK_TRY(axk_fill_iota_i32(a.qo_indptr, B, T, axk_stream(stream)));
    // the attention with its output gate applied as each row is written: gated = bf16(attn * sigmoid(gate))
    AXK_TRY(axk_paged_prefill_gated(a.q, kv_cache, a.qo_indptr, indptr, indices, last_page_len, a.qg + D, 2 * D,
                                    a.gated, B, R, HQ, HKV, D, page_size, num_pages, sm_scale, axk_stream(stream)));
    const AxkMxMat o = proj_mat(proj_fmt, w_o, s_o, a.y, H);
    AXK_TRY(projs(proj_fmt, a.gated, HQ * D, &o, 1, R, HQ * D, stream));
    if (moe) return moe_residual(x, a.y, ln2, mw, mlp_fmt, *moe, out, a.mlp, eb, R, H, F, eps, stream);
    return mlp_residual(x, a.y, ln2, mw, mlp_fmt, out, a.mlp, R, H, F, eps, stream);
  };
  {
    const AxkValidateScope check_only;  // every sub-call's checks before the first launch
    AXK_TRY(body());
  }
  return body();
}

}  // namespace

extern "C" size_t axk_gdn_layer_verify_workspace_size(int64_t batch, int64_t tokens, int64_t hidden,
                                                      int64_t num_k_heads, int64_t num_v_heads, int64_t head_dim,
                                                      int64_t inter) {
  if (check_verify(batch, tokens, hidden, inter) != AXK_OK || head_dim != 128 || num_k_heads <= 0 ||
      num_v_heads <= 0 || num_v_heads % num_k_heads != 0)
    return 0;
  Carver c{nullptr};
  carve_gdn_verify(c, batch * tokens, hidden, num_k_heads, num_v_heads, head_dim, inter);
  return c.off;
}

extern "C" int axk_gdn_layer_verify(
    const uint16_t* x, const float* ln1, const uint8_t* w_qkv, const void* s_qkv, const uint8_t* w_z, const void* s_z,
    const uint8_t* w_b, const void* s_b, const uint8_t* w_a, const void* s_a, const uint16_t* conv_w,
    const float* a_log, const float* dt_bias, const float* norm_w, const uint8_t* w_out, const void* s_out,
    const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s, const uint8_t* mlp_up_w,
    const void* mlp_up_s, const uint8_t* mlp_down_w, const void* mlp_down_s, const float* state_in,
    const uint16_t* conv_in, uint16_t* out, float* state_out, uint16_t* conv_out, float* state_snap,
    uint16_t* conv_snap, int64_t batch, int64_t tokens, int64_t hidden, int64_t num_k_heads, int64_t num_v_heads,
    int64_t head_dim, int64_t conv_kernel, int64_t inter, float eps, int proj_fmt, int mlp_fmt, int v_order,
    void* workspace, size_t workspace_bytes, axk_stream_t stream) {
  AXK_REQUIRE(x && ln1 && w_qkv && s_qkv && w_z && s_z && w_b && s_b && w_a && s_a && conv_w && a_log && dt_bias &&
                  norm_w && w_out && s_out && ln2 && mlp_gate_w && mlp_gate_s && mlp_up_w && mlp_up_s &&
                  mlp_down_w && mlp_down_s && state_in && conv_in && out && state_out && conv_out,
              AXK_E_NULL);
  AXK_REQUIRE(mx_fmt_of(proj_fmt) >= 0 && mx_fmt_of(mlp_fmt) >= 0, AXK_E_DTYPE);
  const size_t need = axk_gdn_layer_verify_workspace_size(batch, tokens, hidden, num_k_heads, num_v_heads, head_dim,
                                                          inter);
  AXK_REQUIRE(need > 0 && conv_kernel >= 2, AXK_E_SHAPE);
  AXK_REQUIRE(workspace && workspace_bytes >= need && axk_aligned(workspace, 256), AXK_E_WORKSPACE);
  const int64_t B = batch, T = tokens, R = B * T, H = hidden, NK = num_k_heads, NV = num_v_heads, DH = head_dim,
                F = inter, K = conv_kernel;
  const int64_t KD = NK * DH, VD = NV * DH, C = 2 * KD + VD;
  if (conv_snap) {  // [T, B, K - 1, C], apart from the conv states it is taken from
    const size_t sb = (size_t)B * (K - 1) * C * 2, nb = (size_t)T * sb;
    AXK_REQUIRE(!axk_overlap(conv_snap, nb, conv_in, sb) && !axk_overlap(conv_snap, nb, conv_out, sb), AXK_E_ALIAS);
  }
  Carver c{static_cast<unsigned char*>(workspace)};
  const GdnVerifyBufs g = carve_gdn_verify(c, R, H, NK, NV, DH, F);
  const MlpWeights mw{mlp_gate_w, mlp_up_w, mlp_down_w, mlp_gate_s, mlp_up_s, mlp_down_s};
  auto body = [&]() -> int {
    AXK_TRY(axk_rmsnorm(x, H, ln1, g.h, H, R, H, eps, stream));
    // qkv | z | b | a for all rows at once; the conv then runs over each sequence's rows in order
    const AxkMxMat proj[4] = {proj_mat(proj_fmt, w_qkv, s_qkv, g.qkv, C), proj_mat(proj_fmt, w_z, s_z, g.z, VD),
                              proj_mat(proj_fmt, w_b, s_b, g.bb, NV), proj_mat(proj_fmt, w_a, s_a, g.aa, NV)};
    AXK_TRY(projs(proj_fmt, g.h, H, proj, 4, R, H, stream));
    if (conv_snap)  // before the conv, which may advance the state in place
      AXK_TRY(axk_conv_snapshots(g.qkv, conv_in, conv_snap, B * (K - 1) * C, B, T, C, K, axk_stream(stream)));
    AXK_TRY(axk_causal_conv1d_silu(g.qkv, conv_w, conv_in, conv_out, g.mixed, B, T, C, K, stream));
    const AxkGdnStrides ld{C, C, C, NV};
    const AxkGdnGate gate{norm_w, g.z, eps};
    AXK_TRY(axk_gdn_recurrent_strided(g.mixed, g.mixed + KD, g.mixed + 2 * KD, g.aa, g.bb, a_log, dt_bias, state_in,
                                      state_out, g.gated, B, T, NK, NV, ld, &gate, v_order, axk_stream(stream),
                                      state_snap, B * NV * DH * DH));
    const AxkMxMat o = proj_mat(proj_fmt, w_out, s_out, g.y, H);
    AXK_TRY(projs(proj_fmt, g.gated, VD, &o, 1, R, VD, stream));
    return mlp_residual(x, g.y, ln2, mw, mlp_fmt, out, g.mlp, R, H, F, eps, stream);
  };
  {
    const AxkValidateScope check_only;  // every sub-call's checks before the first launch
    AXK_TRY(body());
  }
  return body();
}

extern "C" size_t axk_attn_layer_verify_workspace_size(int64_t batch, int64_t tokens, int64_t hidden,
                                                       int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim,
                                                       int64_t inter) {
  if (check_verify(batch, tokens, hidden, inter) != AXK_OK) return 0;
  return attn_rows_ws(batch, tokens, hidden, num_qo_heads, num_kv_heads, head_dim, inter);
}

extern "C" int axk_attn_layer_verify(
    const uint16_t* x, const float* ln1, const uint8_t* w_q, const void* s_q, const uint8_t* w_k, const void* s_k,
    const uint8_t* w_v, const void* s_v, const float* q_norm, const float* k_norm, const uint16_t* cos,
    const uint16_t* sin, uint16_t* kv_cache, const int32_t* indptr, const int32_t* indices,
    const int32_t* last_page_len, const int32_t* cache_location, const uint8_t* w_o, const void* s_o,
    const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s, const uint8_t* mlp_up_w,
    const void* mlp_up_s, const uint8_t* mlp_down_w, const void* mlp_down_s, uint16_t* out, int64_t batch,
    int64_t tokens, int64_t hidden, int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t rot,
    int64_t page_size, int64_t num_pages, int64_t inter, float eps, float sm_scale, int proj_fmt, int mlp_fmt,
    void* workspace, size_t workspace_bytes, axk_stream_t stream) {
  const size_t need = axk_attn_layer_verify_workspace_size(batch, tokens, hidden, num_qo_heads, num_kv_heads,
                                                           head_dim, inter);
  return attn_rows_impl(x, ln1, w_q, s_q, w_k, s_k, w_v, s_v, q_norm, k_norm, cos, sin, kv_cache, indptr, indices,
                        last_page_len, cache_location, w_o, s_o, ln2, mlp_gate_w, mlp_gate_s, mlp_up_w, mlp_up_s,
                        mlp_down_w, mlp_down_s, nullptr, out, batch, tokens, hidden, num_qo_heads, num_kv_heads, head_dim, rot,
                        page_size, num_pages, inter, eps, sm_scale, proj_fmt, mlp_fmt, workspace, workspace_bytes,
                        stream, need);
}

// ---------------------------------------------------------------------------------------------
// Prefill: T new tokens per sequence through a layer in one call (models/qwen35_35b_a3b/src/70b0fbc/q35_prefill.py
// gdn_layer_prefill 57-141 and attn_layer_prefill 172-336): every projection and the MLP as B T-row matrix products
// (the dense GEMM path from 128 rows), the GDN conv over the T tokens with its state, the delta rule in the chunked
// form (axk_gdn_chunk_prefill: chunk-parallel solves, then the state through the chunks); the attention layer as
// the verify layer's rows. Row t of sequence b is x row b T + t.
// ---------------------------------------------------------------------------------------------
namespace {

struct GdnPrefillBufs {
  uint16_t *h, *qkv, *z, *bb, *aa, *mixed, *core, *gated, *y;
  void* cws;
  size_t cws_bytes;
  MlpBufs mlp;
};

GdnPrefillBufs carve_gdn_prefill(Carver& c, int64_t B, int64_t T, int64_t H, int64_t NK, int64_t NV, int64_t F) {
  const int64_t R = B * T, KD = NK * 128, VD = NV * 128, C = 2 * KD + VD;
  GdnPrefillBufs g;
  g.h = c.take<uint16_t>(R * H);
  g.qkv = c.take<uint16_t>(R * C);
  g.z = c.take<uint16_t>(R * VD);
  g.bb = c.take<uint16_t>(R * NV);
  g.aa = c.take<uint16_t>(R * NV);
  g.mixed = c.take<uint16_t>(R * C);
  g.core = c.take<uint16_t>(R * VD);
  g.gated = c.take<uint16_t>(R * VD);
  g.y = c.take<uint16_t>(R * H);
  g.cws_bytes = axk_gdn_chunk_workspace_size(B, T, NK, NV, 128, 128, 64);
  g.cws = c.take<unsigned char>(g.cws_bytes);
  g.mlp = carve_mlp(c, R, H, F);
  return g;
}

size_t gdn_prefill_ws(int64_t batch, int64_t tokens, int64_t hidden, int64_t num_k_heads, int64_t num_v_heads,
                      int64_t head_dim, int64_t inter, const axk_moe_block* moe) {
  if (check_prefill(batch, tokens, hidden, inter) != AXK_OK || head_dim != 128 || num_k_heads <= 0 ||
      num_v_heads <= 0 || num_v_heads % num_k_heads != 0 ||
      axk_gdn_chunk_workspace_size(batch, tokens, num_k_heads, num_v_heads, 128, 128, 64) == 0)
    return 0;
  if (moe && moe_ws_bytes(batch * tokens, hidden, *moe) == 0) return 0;
  Carver c{nullptr};
  carve_gdn_prefill(c, batch, tokens, hidden, num_k_heads, num_v_heads, inter);
  if (moe) carve_moe(c, batch * tokens, hidden, *moe);
  return c.off;
}

int gdn_prefill_impl(const uint16_t* x, const float* ln1, const uint8_t* w_qkv, const void* s_qkv, const uint8_t* w_z,
                     const void* s_z, const uint8_t* w_b, const void* s_b, const uint8_t* w_a, const void* s_a,
                     const uint16_t* conv_w, const float* a_log, const float* dt_bias, const float* norm_w,
                     const uint8_t* w_out, const void* s_out, const float* ln2, const uint8_t* mlp_gate_w,
                     const void* mlp_gate_s, const uint8_t* mlp_up_w, const void* mlp_up_s,
                     const uint8_t* mlp_down_w, const void* mlp_down_s, const axk_moe_block* moe,
                     const float* state_in, const uint16_t* conv_in, uint16_t* out, float* state_out,
                     uint16_t* conv_out, int64_t batch, int64_t tokens, int64_t hidden, int64_t num_k_heads,
                     int64_t num_v_heads, int64_t head_dim, int64_t conv_kernel, int64_t inter, float eps,
                     int proj_fmt, int mlp_fmt, int v_order, void* workspace, size_t workspace_bytes,
                     axk_stream_t stream) {
  AXK_REQUIRE(x && ln1 && w_qkv && s_qkv && w_z && s_z && w_b && s_b && w_a && s_a && conv_w && a_log && dt_bias &&
                  norm_w && w_out && s_out && ln2 && mlp_gate_w && mlp_gate_s && mlp_up_w && mlp_up_s &&
                  mlp_down_w && mlp_down_s && state_in && conv_in && out && state_out && conv_out,
              AXK_E_NULL);
  AXK_REQUIRE(mx_fmt_of(proj_fmt) >= 0 && mx_fmt_of(mlp_fmt) >= 0, AXK_E_DTYPE);
  const size_t need =
      gdn_prefill_ws(batch, tokens, hidden, num_k_heads, num_v_heads, head_dim, inter, moe);
  AXK_REQUIRE(need > 0, AXK_E_SHAPE);
  AXK_REQUIRE(workspace && workspace_bytes >= need && axk_aligned(workspace, 256), AXK_E_WORKSPACE);
  const int64_t B = batch, T = tokens, R = B * T, H = hidden, NK = num_k_heads, NV = num_v_heads, F = inter;
  const int64_t KD = NK * 128, VD = NV * 128, C = 2 * KD + VD;
  Carver c{static_cast<unsigned char*>(workspace)};
  const GdnPrefillBufs g = carve_gdn_prefill(c, B, T, H, NK, NV, F);
  const MoeBufs eb = moe ? carve_moe(c, R, H, *moe) : MoeBufs{};
  const MlpWeights mw{mlp_gate_w, mlp_up_w, mlp_down_w, mlp_gate_s, mlp_up_s, mlp_down_s};
  auto body = [&]() -> int {
    AXK_TRY(axk_rmsnorm(x, H, ln1, g.h, H, R, H, eps, stream));
    const AxkMxMat proj[4] = {proj_mat(proj_fmt, w_qkv, s_qkv, g.qkv, C), proj_mat(proj_fmt, w_z, s_z, g.z, VD),
                              proj_mat(proj_fmt, w_b, s_b, g.bb, NV), proj_mat(proj_fmt, w_a, s_a, g.aa, NV)};
    AXK_TRY(projs(proj_fmt, g.h, H, proj, 4, R, H, stream));
    // the causal conv1d + SiLU over each sequence's T tokens, from and into the conv state
    AXK_TRY(axk_causal_conv1d_silu(g.qkv, conv_w, conv_in, conv_out, g.mixed, B, T, C, conv_kernel, stream));
    // the delta rule over the chunks, q / k / v the channel ranges of the conv output's rows
    AXK_TRY(axk_gdn_chunk_prefill_strided(g.mixed, g.mixed + KD, g.mixed + 2 * KD, g.aa, g.bb, a_log, dt_bias,
                                          state_in, state_out, g.core, B, T, NK, NV, C, C, C, v_order, g.cws,
                                          g.cws_bytes, stream));
    AXK_TRY(axk_gated_rmsnorm_silu(g.core, norm_w, g.z, g.gated, R * NV, 128, eps, stream));
    const AxkMxMat o = proj_mat(proj_fmt, w_out, s_out, g.y, H);
    AXK_TRY(projs(proj_fmt, g.gated, VD, &o, 1, R, VD, stream));
    if (moe) return moe_residual(x, g.y, ln2, mw, mlp_fmt, *moe, out, g.mlp, eb, R, H, F, eps, stream);
    return mlp_residual(x, g.y, ln2, mw, mlp_fmt, out, g.mlp, R, H, F, eps, stream);
  };
  {
    const AxkValidateScope check_only;  // every sub-call's checks before the first launch
    AXK_TRY(body());
  }
  return body();
}

}  // namespace

extern "C" size_t axk_gdn_layer_prefill_workspace_size(int64_t batch, int64_t tokens, int64_t hidden,
                                                       int64_t num_k_heads, int64_t num_v_heads, int64_t head_dim,
                                                       int64_t inter) {
  return gdn_prefill_ws(batch, tokens, hidden, num_k_heads, num_v_heads, head_dim, inter, nullptr);
}

extern "C" size_t axk_gdn_layer_prefill_moe_workspace_size(int64_t batch, int64_t tokens, int64_t hidden,
                                                           int64_t num_k_heads, int64_t num_v_heads,
                                                           int64_t head_dim, int64_t inter,
                                                           const axk_moe_block* moe) {
  return moe ? gdn_prefill_ws(batch, tokens, hidden, num_k_heads, num_v_heads, head_dim, inter, moe) : 0;
}

extern "C" int axk_gdn_layer_prefill(
    const uint16_t* x, const float* ln1, const uint8_t* w_qkv, const void* s_qkv, const uint8_t* w_z, const void* s_z,
    const uint8_t* w_b, const void* s_b, const uint8_t* w_a, const void* s_a, const uint16_t* conv_w,
    const float* a_log, const float* dt_bias, const float* norm_w, const uint8_t* w_out, const void* s_out,
    const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s, const uint8_t* mlp_up_w,
    const void* mlp_up_s, const uint8_t* mlp_down_w, const void* mlp_down_s, const float* state_in,
    const uint16_t* conv_in, uint16_t* out, float* state_out, uint16_t* conv_out, int64_t batch, int64_t tokens,
    int64_t hidden, int64_t num_k_heads, int64_t num_v_heads, int64_t head_dim, int64_t conv_kernel, int64_t inter,
    float eps, int proj_fmt, int mlp_fmt, int v_order, void* workspace, size_t workspace_bytes,
    axk_stream_t stream) {
  return gdn_prefill_impl(x, ln1, w_qkv, s_qkv, w_z, s_z, w_b, s_b, w_a, s_a, conv_w, a_log, dt_bias, norm_w, w_out,
                          s_out, ln2, mlp_gate_w, mlp_gate_s, mlp_up_w, mlp_up_s, mlp_down_w, mlp_down_s, nullptr,
                          state_in, conv_in, out, state_out, conv_out, batch, tokens, hidden, num_k_heads,
                          num_v_heads, head_dim, conv_kernel, inter, eps, proj_fmt, mlp_fmt, v_order, workspace,
                          workspace_bytes, stream);
}

extern "C" int axk_gdn_layer_prefill_moe(
    const uint16_t* x, const float* ln1, const uint8_t* w_qkv, const void* s_qkv, const uint8_t* w_z, const void* s_z,
    const uint8_t* w_b, const void* s_b, const uint8_t* w_a, const void* s_a, const uint16_t* conv_w,
    const float* a_log, const float* dt_bias, const float* norm_w, const uint8_t* w_out, const void* s_out,
    const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s, const uint8_t* mlp_up_w,
    const void* mlp_up_s, const uint8_t* mlp_down_w, const void* mlp_down_s, const axk_moe_block* moe,
    const float* state_in, const uint16_t* conv_in, uint16_t* out, float* state_out, uint16_t* conv_out,
    int64_t batch, int64_t tokens, int64_t hidden, int64_t num_k_heads, int64_t num_v_heads, int64_t head_dim,
    int64_t conv_kernel, int64_t inter, float eps, int proj_fmt, int mlp_fmt, int v_order, void* workspace,
    size_t workspace_bytes, axk_stream_t stream) {
  AXK_REQUIRE(moe, AXK_E_NULL);
  return gdn_prefill_impl(x, ln1, w_qkv, s_qkv, w_z, s_z, w_b, s_b, w_a, s_a, conv_w, a_log, dt_bias, norm_w, w_out,
                          s_out, ln2, mlp_gate_w, mlp_gate_s, mlp_up_w, mlp_up_s, mlp_down_w, mlp_down_s, moe,
                          state_in, conv_in, out, state_out, conv_out, batch, tokens, hidden, num_k_heads,
                          num_v_heads, head_dim, conv_kernel, inter, eps, proj_fmt, mlp_fmt, v_order, workspace,
                          workspace_bytes, stream);
}

extern "C" size_t axk_attn_layer_prefill_workspace_size(int64_t batch, int64_t tokens, int64_t hidden,
                                                        int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim,
                                                        int64_t inter) {
  if (check_prefill(batch, tokens, hidden, inter) != AXK_OK) return 0;
  return attn_rows_ws(batch, tokens, hidden, num_qo_heads, num_kv_heads, head_dim, inter);
}

extern "C" size_t axk_attn_layer_prefill_moe_workspace_size(int64_t batch, int64_t tokens, int64_t hidden,
                                                            int64_t num_qo_heads, int64_t num_kv_heads,
                                                            int64_t head_dim, int64_t inter,
                                                            const axk_moe_block* moe) {
  if (!moe || check_prefill(batch, tokens, hidden, inter) != AXK_OK) return 0;
  return attn_rows_ws(batch, tokens, hidden, num_qo_heads, num_kv_heads, head_dim, inter, moe);
}

extern "C" int axk_attn_layer_prefill(
    const uint16_t* x, const float* ln1, const uint8_t* w_q, const void* s_q, const uint8_t* w_k, const void* s_k,
    const uint8_t* w_v, const void* s_v, const float* q_norm, const float* k_norm, const uint16_t* cos,
    const uint16_t* sin, uint16_t* kv_cache, const int32_t* indptr, const int32_t* indices,
    const int32_t* last_page_len, const int32_t* cache_location, const uint8_t* w_o, const void* s_o,
    const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s, const uint8_t* mlp_up_w,
    const void* mlp_up_s, const uint8_t* mlp_down_w, const void* mlp_down_s, uint16_t* out, int64_t batch,
    int64_t tokens, int64_t hidden, int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t rot,
    int64_t page_size, int64_t num_pages, int64_t inter, float eps, float sm_scale, int proj_fmt, int mlp_fmt,
    void* workspace, size_t workspace_bytes, axk_stream_t stream) {
  const size_t need = axk_attn_layer_prefill_workspace_size(batch, tokens, hidden, num_qo_heads, num_kv_heads,
                                                            head_dim, inter);
  return attn_rows_impl(x, ln1, w_q, s_q, w_k, s_k, w_v, s_v, q_norm, k_norm, cos, sin, kv_cache, indptr, indices,
                        last_page_len, cache_location, w_o, s_o, ln2, mlp_gate_w, mlp_gate_s, mlp_up_w, mlp_up_s,
                        mlp_down_w, mlp_down_s, nullptr, out, batch, tokens, hidden, num_qo_heads, num_kv_heads,
                        head_dim, rot, page_size, num_pages, inter, eps, sm_scale, proj_fmt, mlp_fmt, workspace,
                        workspace_bytes, stream, need);
}

extern "C" int axk_attn_layer_prefill_moe(
    const uint16_t* x, const float* ln1, const uint8_t* w_q, const void* s_q, const uint8_t* w_k, const void* s_k,
    const uint8_t* w_v, const void* s_v, const float* q_norm, const float* k_norm, const uint16_t* cos,
    const uint16_t* sin, uint16_t* kv_cache, const int32_t* indptr, const int32_t* indices,
    const int32_t* last_page_len, const int32_t* cache_location, const uint8_t* w_o, const void* s_o,
    const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s, const uint8_t* mlp_up_w,
    const void* mlp_up_s, const uint8_t* mlp_down_w, const void* mlp_down_s, const axk_moe_block* moe,
    uint16_t* out, int64_t batch, int64_t tokens, int64_t hidden, int64_t num_qo_heads, int64_t num_kv_heads,
    int64_t head_dim, int64_t rot, int64_t page_size, int64_t num_pages, int64_t inter, float eps, float sm_scale,
    int proj_fmt, int mlp_fmt, void* workspace, size_t workspace_bytes, axk_stream_t stream) {
  AXK_REQUIRE(moe, AXK_E_NULL);
  const size_t need = axk_attn_layer_prefill_moe_workspace_size(batch, tokens, hidden, num_qo_heads, num_kv_heads,
                                                                head_dim, inter, moe);
  return attn_rows_impl(x, ln1, w_q, s_q, w_k, s_k, w_v, s_v, q_norm, k_norm, cos, sin, kv_cache, indptr, indices,
                        last_page_len, cache_location, w_o, s_o, ln2, mlp_gate_w, mlp_gate_s, mlp_up_w, mlp_up_s,
                        mlp_down_w, mlp_down_s, moe, out, batch, tokens, hidden, num_qo_heads, num_kv_heads,
                        head_dim, rot, page_size, num_pages, inter, eps, sm_scale, proj_fmt, mlp_fmt, workspace,
                        workspace_bytes, stream, need);
}
