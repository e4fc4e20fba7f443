// Host-side helpers for the C-ABI entry points: argument checks and launch status.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "axk.h"

#define AXK_REQUIRE(cond, code) \
  do {                          \
    if (!(cond)) return (code); \
  } while (0)

static inline bool axk_aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

static inline int axk_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? AXK_OK : AXK_E_LAUNCH;
}

// Byte ranges [a, a+na) and [b, b+nb) overlap.
static inline bool axk_overlap(const void* a, size_t na, const void* b, size_t nb) {
  if (!a || !b || !na || !nb) return false;
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + nb && y < x + na;
}

static inline hipStream_t axk_stream(axk_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// A one-time host step (raising a kernel's dynamic-LDS limit) that is retried until it succeeds once, safe when
// several host threads make their first call together.
struct AxkOnce {
  std::atomic<bool> done{false};
  std::mutex mu;
};
// Runs fn (returning hipError_t) unless an earlier call succeeded; AXK_OK, or AXK_E_LAUNCH when fn fails.
template <class Fn>
static inline int axk_once(AxkOnce& once, Fn&& fn) {
  if (once.done.load(std::memory_order_acquire)) return AXK_OK;
  std::lock_guard<std::mutex> lock(once.mu);
  if (once.done.load(std::memory_order_relaxed)) return AXK_OK;
  if (fn() != hipSuccess) return AXK_E_LAUNCH;
  once.done.store(true, std::memory_order_release);
  return AXK_OK;
}
// A kernel's dynamic-LDS limit raised to `bytes` once per process.
static inline int axk_raise_lds(AxkOnce& once, const void* kernel, size_t bytes) {
  return axk_once(once, [&] {
    return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  });
}

// Validate-only mode of the calling thread: while it is set, entry points run every argument check and return
// AXK_OK just before their first launch. The composed layer entry points run their whole call sequence once this way
// before running it for real, so a contract error in a late sub-call is returned before an early one has advanced a
// state, a conv state or the KV cache (a nonzero status means nothing was enqueued). Kept in a POSIX thread key.
__attribute__((visibility("hidden"))) int axk_validate_only();
__attribute__((visibility("hidden"))) void axk_validate_add(int delta);
struct AxkValidateScope {
  AxkValidateScope() { axk_validate_add(1); }
  ~AxkValidateScope() { axk_validate_add(-1); }
  AxkValidateScope(const AxkValidateScope&) = delete;
  AxkValidateScope& operator=(const AxkValidateScope&) = delete;
};
#define AXK_LAUNCH_GATE()                    \
  do {                                       \
    if (axk_validate_only()) return AXK_OK; \
  } while (0)

// Internal (not exported): the GDN recurrence with row strides, in elements between consecutive (sequence, token)
// rows, for q, k, v and a / b. axk_gdn_recurrent passes the contiguous strides; the decode layer reads q / k / v
// straight out of the conv output. state_snap (optional): the fp32 state after token t, [batch, NV, DK, DV] at
// state_snap + t * snap_ld elements. Returns an AXK status.
// With gate (optional), out is the GDN output norm of each head's row: bf16(bf16(rmsnorm(o) * norm_w) * silu(z)),
// z [batch, tokens, num_v_heads, 128] contiguous. v_order: AXK_VORDER_GROUPED or AXK_VORDER_TILED (which key head
// each value head reads).
struct AxkGdnStrides {
  int64_t q, k, v, ab;
};
struct AxkGdnGate {
  const float* norm_w;
  const uint16_t* z;
  float eps;
};
__attribute__((visibility("hidden"))) int axk_gdn_recurrent_strided(
    const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* a, const uint16_t* b, const float* a_log,
    const float* dt_bias, const float* state_in, float* state_out, uint16_t* out, int64_t batch, int64_t tokens,
    int64_t num_k_heads, int64_t num_v_heads, const AxkGdnStrides& ld, const AxkGdnGate* gate, int v_order,
    hipStream_t stream, float* state_snap = nullptr, int64_t snap_ld = 0);

// Internal (not exported): the conv state after each of a sequence's `tokens` new rows (speculative verification's
// per-row snapshots): snapshot t holds the last kernel - 1 inputs of [state_in | x rows 0 .. t] (oldest first), written
// at snap + t * snap_ld elements as [batch, kernel - 1, channels]. x bf16 [batch, tokens, channels] (the raw
// projection rows the conv consumes), state_in bf16 [batch, kernel - 1, channels]. Returns an AXK status.
__attribute__((visibility("hidden"))) int axk_conv_snapshots(const uint16_t* x, const uint16_t* state_in,
                                                             uint16_t* snap, int64_t snap_ld, int64_t batch,
                                                             int64_t tokens, int64_t channels, int64_t kernel,
                                                             hipStream_t stream);

// Internal (not exported): out[i] = i * step for i = 0 .. n (n + 1 values), int32 (a uniform row index, e.g. the
// qo_indptr of `step` query rows per sequence). Returns an AXK status.
__attribute__((visibility("hidden"))) int axk_fill_iota_i32(int32_t* out, int64_t n, int64_t step, hipStream_t stream);

// Internal (not exported): one launch of up to AXK_MX_GROUP_MAX weight matrices that share the activations a
// [m, k] (the projections of one decode layer). Matrix i: weights w [n, k] (FP8 bytes with a per-channel scale, or
// MXFP4 codes / MXFP8 E4M3 bytes with E8M0 scales ws [n, k/32]), optional per-channel scale and bias, output
// out [m, n] with leading dimension ldo.
// epi: AXK_MX_EPI_PLAIN; AXK_MX_EPI_SWIGLU (mats[0] gate, mats[1] up, one shape and one out:
// out = bf16(silu(bf16 g) * bf16 u)); AXK_MX_EPI_RES (one matrix: out = bf16(res + bf16 y), res [m, n] with
// leading dimension ldr). Rows must be whole 128-byte segments. Returns an AXK status.
#define AXK_MX_GROUP_MAX 4
enum { AXK_MX_EPI_PLAIN = 0, AXK_MX_EPI_SWIGLU = 1, AXK_MX_EPI_RES = 2 };
enum { AXK_MX_MXFP4 = 0, AXK_MX_FP8 = 1, AXK_MX_MXFP8 = 2, AXK_MX_NVFP4 = 3 };
struct AxkMxMat {
  const uint8_t* w;
  const uint8_t* ws;
  const float* col_scale;
  const float* bias;
  void* out;
  int64_t ldo;
  int64_t n;
  const float* gscale;  // NVFP4 (AXK_MX_NVFP4): the fp32 scale2 [1] in device memory; E4M3 ws [n, k/16]
};
// Optional conv epilogue on mats[0] (plain bf16): each row is one token of its sequence; the output is
// silu(causal_conv1d) over the projection's bf16 output with taps w [n, kernel] (tap 0 = the current token) and
// the state [m, kernel - 1, n] oldest first, advanced into state_out (which may be state_in).
struct AxkConvEpi {
  const uint16_t* w;
  const uint16_t* state_in;
  uint16_t* state_out;
  int64_t kernel;
};
__attribute__((visibility("hidden"))) int axk_mx_group(int fmt, const uint16_t* a, int64_t lda, const AxkMxMat* mats,
                                                       int count, int epi, const uint16_t* res, int64_t ldr,
                                                       const float* row_scale, int out_dtype, int64_t m, int64_t k,
                                                       const AxkConvEpi* conv, hipStream_t stream);

// Internal (not exported): the attention decode layer's q / k / v preparation in one launch. q heads of the
// [q | gate] projection qg [B, HQ, 2 D] -> rmsnorm(q_norm) + NeoX RoPE -> q_out [B, HQ, D]; k [B, HKV, D] ->
// rmsnorm(k_norm) + RoPE and v [B, HKV, D] as is -> the paged cache [P, 2, page, HKV, D] at cache_location [B, 2]
// (page, slot); a location outside the cache writes nothing. Returns an AXK status.
__attribute__((visibility("hidden"))) int axk_attn_qkv_prep(
    const uint16_t* qg, const uint16_t* kk, const uint16_t* vv, const float* q_norm, const float* k_norm,
    const uint16_t* cos, const uint16_t* sin, uint16_t* q_out, uint16_t* kv_cache, const int32_t* cache_location,
    int64_t batch, int64_t hq, int64_t hkv, int64_t head_dim, int64_t rot, int64_t page_size, int64_t num_pages,
    float eps, hipStream_t stream);

// Internal (not exported): axk_paged_decode with the attention output gate applied where each output row is written:
// out[b, h, :] = bf16(bf16(attention) * sigmoid(gate[(b hq + h) ldg + :])), bit-identical to axk_paged_decode followed
// by the elementwise sigmoid-mul, one launch fewer. Returns an AXK status.
__attribute__((visibility("hidden"))) int axk_paged_decode_gated(
    const uint16_t* q, const uint16_t* kv_cache, const int32_t* indptr, const int32_t* indices,
    const int32_t* last_page_len, const uint16_t* gate, int64_t ldg, uint16_t* out, int64_t batch, int64_t num_qo_heads,
    int64_t num_kv_heads, int64_t head_dim, int64_t page_size, int64_t num_pages, float sm_scale, void* workspace,
    size_t workspace_bytes, hipStream_t stream);

// Internal (not exported): axk_paged_prefill with the attention output gate applied where each output row is
// written, as axk_paged_decode_gated (gate rows ldg elements apart, one per (token, query head) row). Returns an
// AXK status.
__attribute__((visibility("hidden"))) int axk_paged_prefill_gated(
    const uint16_t* q, const uint16_t* kv_cache, const int32_t* qo_indptr, const int32_t* indptr,
    const int32_t* indices, const int32_t* last_page_len, const uint16_t* gate, int64_t ldg, uint16_t* out,
    int64_t batch, int64_t total_q, int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
    int64_t num_pages, float sm_scale, hipStream_t stream);

// Internal (not exported): axk_moe_decode with the shared expert computed by the caller: y_sh [tokens, hidden] fp32
// is its down projection (any weight format), gated by sigmoid(h2 . w_shg) in the combine as the library's own
// shared expert is; the routed experts and routing as axk_moe_decode. Size the workspace with
// axk_moe_workspace_size(..., shared_inter = 0). Returns an AXK status; a nonzero one means nothing was launched.
__attribute__((visibility("hidden"))) int axk_moe_decode_shared_given(
    const uint16_t* h2, const uint16_t* x_res, const uint16_t* w_router, const uint16_t* w_shg, const float* y_sh,
    const uint8_t* e_gw, const uint8_t* e_gs, const uint8_t* e_dw, const uint8_t* e_ds, uint16_t* out, float* logits,
    int32_t* topk_ids, float* topk_weights, int64_t tokens, int64_t hidden, int64_t num_experts, int64_t top_k,
    int64_t inter, int norm_topk_prob, void* workspace, size_t workspace_bytes, axk_stream_t stream);

// Internal (not exported): axk_gdn_chunk_prefill (chunk 64, head dims 128) with q, k, v read at row strides ldq, ldk,
// ldv (elements between consecutive (sequence, token) rows; the heads of a row contiguous), so the prefill layer
// reads them straight out of the conv output, and the value-head order v_order (AXK_VORDER_*). Returns an AXK status.
__attribute__((visibility("hidden"))) int axk_gdn_chunk_prefill_strided(
    const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* a, const uint16_t* b, const float* a_log,
    const float* dt_bias, const float* state_in, float* state_out, uint16_t* out, int64_t batch, int64_t tokens,
    int64_t num_k_heads, int64_t num_v_heads, int64_t ldq, int64_t ldk, int64_t ldv, int v_order, void* workspace,
    size_t workspace_bytes, axk_stream_t stream);
