/* axk — C-ABI of the MI355X (gfx950) kernels for the per-layer Qwen3.5 decode/prefill hot path.
 *
 * Conventions (the same for every entry point):
 *  - All tensor arguments are DEVICE pointers owned by the caller. No entry point allocates,
 *    converts, pads, copies or slices on the caller's behalf; scratch memory is a caller-provided
 *    workspace whose size is returned by the matching *_workspace_size() query. This is the
 *    ownership rule of the reference operator API
 *    (models/qwen35_35b_a3b/sgl/python/sgl_kernel_axera/attention/flash_attn.py:2573-2588).
 *  - Weights are runtime inputs. FP4 (E2M1) codes and E8M0 scales travel as uint8_t:
 *    codes [N, K/2] with the LOW nibble holding the EVEN column, scales [N, K/32]
 *    (models/qwen35_35b_a3b/src/70b0fbc/q35_moe.py:46-63, board_io.py:1-38).
 *  - bf16 tensors are passed as uint16_t bit patterns; fp8 E4M3 weights as uint8_t.
 *  - `stream` is a hipStream_t (NULL = the legacy default stream). Every entry point is
 *    asynchronous on `stream` and reentrant across streams.
 *  - Return value: AXK_OK (0) or one of the AXK_E_* codes below, in the spirit of the AX engine's
 *    int status (tools/board/axrun.cc:106-110). Contract checks happen before any launch, so a
 *    nonzero return means nothing was enqueued.
 *  - Outputs may alias inputs only where an entry point says so (in-place state / KV), following
 *    tools/board/axrun.cc:74-99 and tools/board/inplace_test.cc:1-3.
 */
#ifndef AXK_H
#define AXK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* axk_stream_t; /* hipStream_t */

/* status codes */
#define AXK_OK 0
#define AXK_E_NULL 1      /* a required pointer is NULL */
#define AXK_E_SHAPE 2     /* a size / shape contract is violated */
#define AXK_E_ALIGN 3     /* a pointer or leading dimension is not aligned as required */
#define AXK_E_DTYPE 4     /* unsupported dtype code */
#define AXK_E_ALIAS 5     /* buffers overlap where that is not allowed */
#define AXK_E_WORKSPACE 6 /* workspace missing or smaller than *_workspace_size() */
#define AXK_E_LAUNCH 7    /* the HIP runtime rejected the launch */
#define AXK_E_ROLE 8      /* unknown role name in an IO-table query */
#define AXK_E_BUFFER 9    /* a host-side output buffer is too small */
#define AXK_E_SCRATCH 10  /* the call needs more than the library's static scratch (no-allocation entry points) */

/* AX dtype codes used on the boundary (tools/manifest/onnx_io.py:18-29) */
#define AXK_DT_U8 1
#define AXK_DT_F32 3
#define AXK_DT_I32 6
#define AXK_DT_BF16 9
#define AXK_DT_F16 10
#define AXK_DT_FP8E4M3 11
#define AXK_DT_FP8E5M2 12
#define AXK_DT_FP4 15

/* Weight formats of the decode layers' projections and MLP (proj_fmt / mlp_fmt):
 *   AXK_WFMT_FP8_CHANNEL  E4M3 bytes [N, K] + f32 per-output-channel scale [N]   (sgl gemm.py:119-181)
 *   AXK_WFMT_MXFP8        E4M3 bytes [N, K] + E8M0 bytes [N, K/32]              (q35_mx_build.py:60-72; the 35B manifest)
 *   AXK_WFMT_MXFP4        E2M1 pairs [N, K/2] + E8M0 bytes [N, K/32]            (q35_moe.py:46-63; the 9B / 27B manifests)
 *   AXK_WFMT_NVFP4        E2M1 pairs [N, K/2] + E4M3 bytes [N, K/16] + f32 scale2 [1] (q35_mx_build.py:168-200, the
 *                         WFMT=nv4 projections; sgl quantize_nvfp4): the s_<name> argument of a layer entry then points
 *                         to an axk_nvfp4_scales in host memory naming both device arrays (the reference's s_<name> and
 *                         t_<name> inputs), read while the call is made */
#define AXK_WFMT_FP8_CHANNEL 0
#define AXK_WFMT_MXFP8 1
#define AXK_WFMT_MXFP4 2
#define AXK_WFMT_NVFP4 3

typedef struct axk_nvfp4_scales {
  const uint8_t* block_scales; /* E4M3 [N, K/16], 16-byte aligned */
  const float* scale2;         /* f32 [1] */
} axk_nvfp4_scales;

/* Value-head order of the GDN layers when num_v_heads > num_k_heads: which key head value head vh reads
 * (models/qwen35_35b_a3b/src/70b0fbc/q35_step.py:82-85; the weights of the value heads, w_qkv's v rows, conv_w's
 * v rows, w_z, w_b, w_a, a_log, dt_bias, w_out's columns and the state, are in the same order). */
#define AXK_VORDER_GROUPED 0 /* vh / (NV / NK): the checkpoint's order, the GDN operators' */
#define AXK_VORDER_TILED 1   /* vh % NK: the order the reference's layer kernels are built with by default */

/* Library identification and error text. */
const char* axk_version(void);
const char* axk_status_string(int status);

/* ---------------------------------------------------------------------------------------------
 * IO tables: the named IO of each role libaxk serves, as the AX engine reports a kernel's IO (AX_ENGINE_GetIOInfo's
 * {pName, nSize, eDataType, pShape, nShapeSize}, dumped by tools/board/iojson.c:23-34 as [name, bytes, dtype, shape])
 * and as manifest.json records it (tools/manifest/mkmanifest.py:183-199, 296-311). Names, dtype codes (AXK_DT_*, the
 * board's codes of tools/manifest/onnx_io.py:18-29) and byte counts are the reference's, so a host can check its
 * buffers name -> bytes the way models/qwen35_35b_a3b/sgl/scripts/check_adapter_abi.py:20-56 does.
 * ------------------------------------------------------------------------------------------- */

#define AXK_IO_NAME_MAX 48
#define AXK_IO_RANK_MAX 6
typedef struct {
  char name[AXK_IO_NAME_MAX]; /* NUL-terminated */
  int64_t bytes;              /* storage bytes (E2M1: two values per byte) */
  int32_t dtype;              /* AXK_DT_* */
  int32_t output;             /* 0: input, 1: output */
  int32_t rank;
  int64_t shape[AXK_IO_RANK_MAX]; /* logical elements (E2M1: values, as the board reports them) */
} axk_io_entry;

/* Fills entries[0 .. *count) with the IO of `role` at the dimensions dims[0 .. ndims), inputs first, in the
 * reference's order; a dimension left out takes its default (in brackets). Roles and their dims:
 *   "lm_head"     n, k [, m = 1]          mul_mat_mx4_n<n>_k<k>: x bf16 [m, k]; w E2M1 [n, k]; s E8M0 [n, k/32] ->
 *                                         out f32 [m, n] (axk_mx_gemm with f32 output)
 *   "layer.gdn"   hidden, num_k_heads, num_v_heads, inter [, conv_kernel = 4, proj_fmt = AXK_WFMT_MXFP4,
 *                 mlp_fmt = AXK_WFMT_MXFP4, num_experts = 0, batch = 1]
 *                 x, the layer's parameters in the manifest's order (params.gdn: ln1, w_qkv, s_qkv, w_z, s_z, w_b, s_b,
 *                 w_a, s_a, conv_w, a_log, dt_bias, norm_w, w_out, s_out, ln2, w_gate .. s_down, and with num_experts
 *                 the MoE layer's w_router, w_shg), state_in, conv_in -> out, state_out, conv_out (axk_gdn_layer_decode;
 *                 the MoE half through axk_moe_decode)
 *   "layer.attn"  hidden, num_qo_heads, num_kv_heads, head_dim, inter [, proj_fmt = AXK_WFMT_MXFP4,
 *                 mlp_fmt = AXK_WFMT_MXFP4, num_experts = 0, batch = 1, rot = 64, page_size = 256, num_pages = 1]
 *                 x, the parameters (params.attn: ln1, w_q, s_q, w_k, s_k, w_v, s_v, q_norm, k_norm, w_o, s_o, ln2,
 *                 the MLP, and with num_experts w_router, w_shg), cos, sin, the paged cache and page table -> out,
 *                 kv_cache (in place) (axk_attn_layer_decode)
 *   "experts"     num_experts, hidden, inter   e_gw, e_gs, e_dw, e_ds (params.experts; axk_moe_experts)
 * Weight w_<x> / s_<x> by format: FP8_CHANNEL E4M3 [N, K] + f32 [N]; MXFP8 E4M3 [N, K] + E8M0 [N, K/32]; MXFP4
 * E2M1 [N, K] + E8M0 [N, K/32]. Returns AXK_E_ROLE for an unknown role, AXK_E_SHAPE for missing or invalid dims,
 * AXK_E_BUFFER when more than `capacity` entries are needed (*count is then the number needed). Host only: makes no
 * HIP call. */
int axk_io_table(const char* role, const int64_t* dims, int ndims, axk_io_entry* entries, int capacity, int* count);

/* ---------------------------------------------------------------------------------------------
 * MXFP4 codec and MX / FP8 runtime-weight linear
 * ------------------------------------------------------------------------------------------- */

/* Exact dequantisation: out[n, k] = E2M1(code) * 2^(scale - 127) in fp32, bit-identical to
 * dequant_mxfp4 (models/qwen35_35b_a3b/src/70b0fbc/q35_moe.py:60-63) and
 * dequantize_mxfp4 (models/qwen38_27b/head/mx4_common.py:37-49).
 * codes u8 [n, k/2], scales u8 [n, k/32], out f32 [n, k]; k % 32 == 0. */
int axk_mxfp4_dequant(const uint8_t* codes, const uint8_t* scales, float* out, int64_t n, int64_t k,
                      axk_stream_t stream);

/* MXFP4 GEMM: output = a @ dequant(b_fp4, b_scale).T + bias, fp32 accumulation.
 * Replaces sgl_kernel_axera.gemm.mxfp4_gemm
 * (models/qwen35_35b_a3b/sgl/python/sgl_kernel_axera/gemm.py:626-641, kernel 564-598) and the MX
 * `linear()` projections of models/qwen35_35b_a3b/src/70b0fbc/q35_mx_build.py:100-115.
 *   a       bf16 [m, k] (row stride lda elements, lda % 8 == 0)
 *   b_fp4   u8   [n, k/2]   b_scale u8 [n, k/32]
 *   bias    f32  [n] or NULL (already rounded to the output dtype, as the reference does)
 *   out     [m, n]: bf16 when out_dtype == AXK_DT_BF16, f32 when AXK_DT_F32
 * k % 32 == 0; a, b_fp4 16-byte aligned. */
int axk_mxfp4_gemm(const uint16_t* a, int64_t lda, const uint8_t* b_fp4, const uint8_t* b_scale,
                   const float* bias, void* out, int out_dtype, int64_t m, int64_t n, int64_t k,
                   axk_stream_t stream);

/* FP8 E4M3 linear with per-output-channel fp32 scales (and optional per-row activation scales):
 * output = (a * scale_a[:, None]) @ (b_fp8 * scale_b[:, None]).T + bias.
 * Replaces the scaled GEMM of sgl_kernel_axera.gemm (gemm.py:119-181, fp8_gemm 457-466) for bf16
 * activations, as used by the attention / GDN projections of the hybrid decode group.
 *   a bf16 [m, k]; b_fp8 u8 (E4M3) [n, k]; scale_b f32 [n]; scale_a f32 [m] or NULL;
 *   bias f32 [n] or NULL; out bf16/f32 [m, n]; k % 32 == 0. */
int axk_fp8_gemm(const uint16_t* a, int64_t lda, const uint8_t* b_fp8, const float* scale_a,
                 const float* scale_b, const float* bias, void* out, int out_dtype, int64_t m, int64_t n,
                 int64_t k, axk_stream_t stream);

/* MXFP8 GEMM: output = a @ dequant(b_fp8, b_scale).T + bias, fp32 accumulation, where
 * dequant(w)[n, k] = FP8(b_fp8[n, k]) * 2^(b_scale[n, k / 32] - 127). Replaces sgl_kernel_axera.gemm.mxfp8_gemm
 * (models/qwen35_35b_a3b/sgl/python/sgl_kernel_axera/gemm.py:644-659) and the MXFP8 projections of
 * models/qwen35_35b_a3b/src/70b0fbc/q35_mx_build.py:60-72 (quant_mxfp8 / dequant).
 *   a        bf16 [m, k] (row stride lda elements, lda % 8 == 0)
 *   b_fp8    u8   [n, k]: OCP FP8 codes, E4M3 (fp8_dtype == AXK_DT_FP8E4M3) or E5M2 (AXK_DT_FP8E5M2)
 *   b_scale  u8   [n, k/32] E8M0
 *   bias f32 [n] or NULL; out bf16 / f32 [m, n]; k % 32 == 0; a, b_fp8 16-byte aligned.
 * Each weight is decoded to bf16 in registers by gfx950's scaled converts, exactly while code * 2^(s-127) is a bf16
 * normal (every finite code at scale bytes 10 .. 246 for E4M3, 17 .. 239 for E5M2). */
int axk_mxfp8_gemm(const uint16_t* a, int64_t lda, const uint8_t* b_fp8, const uint8_t* b_scale, int fp8_dtype,
                   const float* bias, void* out, int out_dtype, int64_t m, int64_t n, int64_t k, axk_stream_t stream);

/* NVFP4 GEMM: output = a @ dequant(b_fp4, b_scale, b_scale2).T + bias, fp32 accumulation, where
 * dequant(w)[n, k] = E2M1(code[n, k]) * E4M3(b_scale[n, k / 16]) * b_scale2[0]. Replaces sgl_kernel_axera.gemm.nvfp4_gemm
 * (models/qwen35_35b_a3b/sgl/python/sgl_kernel_axera/gemm.py:495-561) on weights packed by quantize_nvfp4
 * (sgl_kernel_axera/quantization.py:8-37), the NVFP4 projections of q35_mx_build.py:168-200.
 *   a         bf16 [m, k] (row stride lda elements, lda % 8 == 0)
 *   b_fp4     u8   [n, k/2]: E2M1 pairs, low nibble = even k (the reference's packed layout)
 *   b_scale   u8   [n, k/16]: E4M3 block scales
 *   b_scale2  f32  [1] in device memory (a runtime input, as the reference keeps it)
 *   bias f32 [n] or NULL; out bf16 / f32 [m, n]; k % 32 == 0; a, b_fp4 16-byte aligned.
 * Each code times its block scale is exact in bf16; b_scale2 multiplies the fp32 sums. */
int axk_nvfp4_gemm(const uint16_t* a, int64_t lda, const uint8_t* b_fp4, const uint8_t* b_scale,
                   const float* b_scale2, const float* bias, void* out, int out_dtype, int64_t m, int64_t n,
                   int64_t k, axk_stream_t stream);

/* Dense bf16-weight linear (router logits and other small bf16 projections):
 * output = a @ b.T + bias, fp32 accumulation. Replaces sgl_kernel_axera.gemm.fp16_gemm / bf16_gemm
 * (gemm.py:81-116, 469-476). a bf16 [m, k]; b bf16 [n, k]; k % 32 == 0. */
int axk_bf16_gemm(const uint16_t* a, int64_t lda, const uint16_t* b, const float* bias, void* out,
                  int out_dtype, int64_t m, int64_t n, int64_t k, axk_stream_t stream);

/* INT8 scaled GEMM: output = (a * scale_a[:, None]) @ (b_int8 * scale_b[:, None]).T + bias. Replaces
 * sgl_kernel_axera.gemm.int8_gemm (gemm.py:479-492 over _scaled_gemm 119-181); int32 MFMA accumulation, the
 * scales applied to each exact int32 sum in fp32.
 *   a       int8 [m, k], row stride lda bytes (lda % 16 == 0, 16-byte aligned)
 *   b_int8  int8 [n, k] contiguous (16-byte aligned); k % 16 == 0
 *   scale_a f32 [m], scale_b f32 [n] (a scalar scale is broadcast by the caller, as _normalize_scale does) */
int axk_int8_gemm(const int8_t* a, int64_t lda, const int8_t* b_int8, const float* scale_a, const float* scale_b,
                  const float* bias, void* out, int out_dtype, int64_t m, int64_t n, int64_t k,
                  axk_stream_t stream);

/* INT4-weight GEMM: output = a @ (b_int4 * b_scale[:, k / group]).T + bias. Replaces
 * sgl_kernel_axera.gemm.int4_gemm (gemm.py:662-677 over _mx_gemm 564-623); fp32 accumulation.
 *   a       bf16 [m, k], row stride lda elements (lda % 8 == 0, 16-byte aligned)
 *   b_int4  int8 [n, k] contiguous: one signed int4 value (-8..7) per byte, as the reference stores it
 *   b_scale f32 [n, k / group]: one scale per `group` consecutive K of a channel; group % 32 == 0, k % group == 0 */
int axk_int4_gemm(const uint16_t* a, int64_t lda, const int8_t* b_int4, const float* b_scale, int64_t group,
                  const float* bias, void* out, int out_dtype, int64_t m, int64_t n, int64_t k,
                  axk_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Paged flash-attention decode and the paged KV write
 * ------------------------------------------------------------------------------------------- */

/* Workspace bytes axk_paged_decode needs for this batch / head configuration (0 = invalid shape). */
size_t axk_paged_decode_workspace_size(int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads,
                                       int64_t head_dim);

/* Split-KV work partition for axk_paged_decode_run, computed on the device from indptr /
 * last_page_len into the workspace (pages per split, one descriptor per work item). It depends only on
 * the page-table shape, so one plan serves every attention layer of a decode step. Up to 63 sequences
 * the run kernels derive the same partition from the page table themselves and this call launches
 * nothing (it still validates its arguments). */
int axk_paged_decode_plan(const int32_t* indptr, const int32_t* last_page_len, int64_t batch,
                          int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                          void* workspace, size_t workspace_bytes, axk_stream_t stream);

/* First half of axk_paged_decode_run (one launch): attention of every work item of the plan. A
 * sequence handled by a single item gets its final output; the others leave fp32 partials
 * (running max, sum, unnormalised O) in the workspace for axk_paged_decode_merge. */
int axk_paged_decode_split(const uint16_t* q, const uint16_t* kv_cache, const int32_t* indptr,
                           const int32_t* indices, const int32_t* last_page_len, uint16_t* out, int64_t batch,
                           int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                           int64_t num_pages, float sm_scale, void* workspace, size_t workspace_bytes,
                           axk_stream_t stream);

/* Second half (one launch): log-sum-exp merge of the split partials, as the split-KV merge of
 * models/qwen35_35b_a3b/src/70b0fbc/q35_layer_mc.py:330-349; zero output for empty sequences. */
int axk_paged_decode_merge(const int32_t* indptr, const int32_t* last_page_len, uint16_t* out, int64_t batch,
                           int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                           void* workspace, size_t workspace_bytes, axk_stream_t stream);

/* The decode attention itself, using the plan held in `workspace` (same batch / heads / indptr):
 * axk_paged_decode_split then axk_paged_decode_merge. Arguments as axk_paged_decode. */
int axk_paged_decode_run(const uint16_t* q, const uint16_t* kv_cache, const int32_t* indptr,
                         const int32_t* indices, const int32_t* last_page_len, uint16_t* out, int64_t batch,
                         int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                         int64_t num_pages, float sm_scale, void* workspace, size_t workspace_bytes,
                         axk_stream_t stream);

/* Decode attention of one query token per sequence over a paged KV cache (GQA, split-KV):
 * axk_paged_decode_plan followed by axk_paged_decode_run.
 * Replaces the page loop of sgl_kernel_axera.attention.flash_attn.paged_attention
 * (models/qwen35_35b_a3b/sgl/python/sgl_kernel_axera/attention/flash_attn.py:1421-1596, page-id
 * lookup 1478-1495, tail mask 87-104) and attention_split_qa of
 * models/qwen38_27b/decode/q35_group.py:317-385 (split-KV + LSE merge).
 *   q             bf16 [batch, num_qo_heads, head_dim]
 *   kv_cache      bf16 [num_pages, 2, page_size, num_kv_heads, head_dim] (plane 0 = K, 1 = V)
 *   indptr        i32  [batch + 1]   CSR offsets into indices
 *   indices       i32  [indptr[batch]] physical page ids (each < num_pages)
 *   last_page_len i32  [batch]        valid tokens in each sequence's last page (1..page_size)
 *   out           bf16 [batch, num_qo_heads, head_dim]
 * The query attends every valid cached token of its sequence (write the current token with
 * axk_paged_kv_write first: the reference's "history + current token" merge is the same sum).
 * A sequence with no pages yields zeros. head_dim in {64, 128, 256}; num_qo_heads / num_kv_heads
 * <= 16; page_size a multiple of 16, at most 4096. Page ids outside [0, num_pages) are skipped, never read.
 * workspace >= axk_paged_decode_workspace_size(...), 256-byte aligned. */
int axk_paged_decode(const uint16_t* q, const uint16_t* kv_cache, const int32_t* indptr,
                     const int32_t* indices, const int32_t* last_page_len, uint16_t* out, int64_t batch,
                     int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                     int64_t num_pages, float sm_scale, void* workspace, size_t workspace_bytes,
                     axk_stream_t stream);

/* axk_paged_decode without a workspace argument, for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. The split partials live in
 * a static device array of the library (AXK_PAGED_NOALLOC_SCRATCH_BYTES, held by each GPU the library runs on until the
 * process ends); nothing is allocated or freed. A configuration whose axk_paged_decode_workspace_size exceeds it is
 * rejected with AXK_E_SCRATCH before anything is launched. Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (different streams, or host threads) race and must be serialised by the caller. The first call
 * on a device does host set-up (the array's address on that device, the split kernel's LDS limit): made while its
 * stream is capturing it returns AXK_E_LAUNCH and enqueues nothing, so make one eager call before capturing; later
 * calls may be captured and the graph replayed. Other arguments and the result as axk_paged_decode. */
#define AXK_PAGED_NOALLOC_SCRATCH_BYTES (24u << 20)
int axk_paged_decode_noalloc(const uint16_t* q, const uint16_t* kv_cache, const int32_t* indptr,
                             const int32_t* indices, const int32_t* last_page_len, uint16_t* out, int64_t batch,
                             int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                             int64_t num_pages, float sm_scale, axk_stream_t stream);

/* The sgl decode operator's page-table convention (models/qwen35_35b_a3b/sgl/python/sgl_kernel_axera/attention/
 * flash_attn.py:2335-2357 and 1421-1596; its test models/qwen35_35b_a3b/sgl/tests/test_qwen35_runtime.py:96-118):
 * last_page_len counts the HISTORY tokens on each sequence's last page (0 .. page_size - 1, so the cached length is
 * (pages - 1) * page_size + last_page_len and may be 0), the page list already holds the page the current token goes
 * to, and cache_location[b] = (page, offset) is that token's slot (offset == last_page_len[b]). The current token's
 * k, v bf16 [batch, num_kv_heads, head_dim] are written there first (as axk_paged_kv_write; a location outside the
 * pool is skipped and sets *status), then q attends the history plus the current token, the same sum as the
 * reference's history loop merged with the current token's score. Every sequence holds at least one page. Other
 * arguments and the workspace as axk_paged_decode. */
int axk_paged_attention_decode(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* kv_cache,
                               const int32_t* indptr, const int32_t* indices, const int32_t* last_page_len,
                               const int32_t* cache_location, uint16_t* out, int64_t batch, int64_t num_qo_heads,
                               int64_t num_kv_heads, int64_t head_dim, int64_t page_size, int64_t num_pages,
                               float sm_scale, int32_t* status, void* workspace, size_t workspace_bytes,
                               axk_stream_t stream);

/* Scatter the current token's K and V rows into the paged cache in place:
 *   kv_cache[loc[b,0], 0, loc[b,1], :, :] = k[b]; kv_cache[loc[b,0], 1, loc[b,1], :, :] = v[b].
 * Replaces store_paged_kv (flash_attn.py:53-84, cache_location = [page, offset]) and
 * kv_write_paged (models/qwen38_27b/decode/q35_group.py:237-264). Every other cache byte is left
 * untouched. k, v bf16 [batch, num_kv_heads, head_dim]; cache_location i32 [batch, 2].
 * A location outside the pool is skipped and *status (if non-NULL, device i32) is set to 1. */
int axk_paged_kv_write(const uint16_t* k, const uint16_t* v, uint16_t* kv_cache, const int32_t* cache_location,
                       int64_t batch, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                       int64_t num_pages, int32_t* status, axk_stream_t stream);

/* FP8 KV cache (models/qwen38_27b/decode/q35_group.py:44-54, KV8=2): K and V stored as OCP E4M3 bytes of
 * bf16(x * kv_scale) with one static power-of-two kv_scale (the reference's KV8_SCALE, 8 for the 27B); attention
 * reads stored / kv_scale, exact in bf16. Same page table, shapes and result as axk_paged_decode, with
 * kv_cache u8 [num_pages, 2, page_size, num_kv_heads, head_dim] (half the bytes); head_dim 128 or 256.
 * Same workspace (axk_paged_decode_workspace_size). */
int axk_paged_decode_fp8(const uint16_t* q, const uint8_t* kv_cache, const int32_t* indptr, const int32_t* indices,
                         const int32_t* last_page_len, uint16_t* out, int64_t batch, int64_t num_qo_heads,
                         int64_t num_kv_heads, int64_t head_dim, int64_t page_size, int64_t num_pages,
                         float sm_scale, float kv_scale, void* workspace, size_t workspace_bytes,
                         axk_stream_t stream);

/* The FP8 cache's KV write (kv_write_paged with KV8=2, q35_group.py:244-247): the cache bytes at the token's
 * (page, slot) become e4m3(bf16(k * kv_scale)) and e4m3(bf16(v * kv_scale)), rounded to nearest even as torch's
 * float8_e4m3fn cast (a magnitude past 464 becomes NaN); every other byte is left untouched. Arguments as
 * axk_paged_kv_write. */
int axk_paged_kv_write_fp8(const uint16_t* k, const uint16_t* v, uint8_t* kv_cache, const int32_t* cache_location,
                           int64_t batch, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                           int64_t num_pages, float kv_scale, int32_t* status, axk_stream_t stream);

/* INT8 paged KV cache with a bf16 scale per row and KV head (models/qwen38_27b/decode/q35_group.py:44-47, KV8=1):
 * kv_cache int8 [num_pages, 2, page_size, num_kv_heads, head_dim] and kv_scales bf16 [num_pages, 2, page_size,
 * num_kv_heads], the layout of the reference's kv<j> / kvs<j> inputs. The write quantizes each row and head as
 * kv_quant_row does (q35_group.py:197-205): s = bf16(max(amax, bf16(1e-5)) * bf16(1 / 127)), codes
 * int8(bf16(x * bf16(1 / s))) rounded to nearest even and saturated; decode reads bf16(q * s) (kv_page, 208-221).
 * Arguments otherwise as axk_paged_kv_write / axk_paged_decode; head_dim 128 or 256; decode takes num_kv_heads <= 16
 * and 4-byte aligned scales. */
int axk_paged_kv_write_i8(const uint16_t* k, const uint16_t* v, int8_t* kv_cache, uint16_t* kv_scales,
                          const int32_t* cache_location, int64_t batch, int64_t num_kv_heads, int64_t head_dim,
                          int64_t page_size, int64_t num_pages, int32_t* status, axk_stream_t stream);
int axk_paged_decode_i8(const uint16_t* q, const int8_t* kv_cache, const uint16_t* kv_scales, const int32_t* indptr,
                        const int32_t* indices, const int32_t* last_page_len, uint16_t* out, int64_t batch,
                        int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                        int64_t num_pages, float sm_scale, void* workspace, size_t workspace_bytes,
                        axk_stream_t stream);

/* Prefill / speculative-verify attention over the paged cache, causal (the history pages and the current block of
 * sgl_kernel_axera/attention/flash_attn.py:471-611 paged_flash_attention, flash_attn.py:1044 flash_attn_with_kvcache;
 * the G x P-row block attention of models/qwen35_35b_a3b/src/70b0fbc/q35_prefill.py:264-336). Sequence b's new tokens
 * are rows qo_indptr[b] .. qo_indptr[b + 1] of q bf16 [total_q, num_qo_heads, head_dim]; their K / V are already in
 * the cache (axk_paged_kv_write) as the sequence's last tokens, so new token t of a sequence with kv_len cached tokens
 * attends positions 0 .. kv_len - qlen + t. Same cache layout and page table as axk_paged_decode; head_dim 64, 128 or
 * 256; page_size a multiple of 16. out bf16 like q. No workspace. A page id outside the pool (page skipped) or a
 * query range outside q (sequence skipped) sets *status (if non-NULL, device i32) to 1. */
int axk_paged_prefill(const uint16_t* q, const uint16_t* kv_cache, const int32_t* qo_indptr, const int32_t* indptr,
                      const int32_t* indices, const int32_t* last_page_len, uint16_t* out, int64_t batch,
                      int64_t total_q, int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim,
                      int64_t page_size, int64_t num_pages, float sm_scale, int32_t* status, axk_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Gated DeltaNet (GDN)
 * ------------------------------------------------------------------------------------------- */

/* GDN recurrence over `tokens` consecutive tokens (1 = decode), fused with the gate and the q/k L2 norm:
 *   q, k <- x / sqrt(sum x^2 + 1e-6), q *= head_k_dim^-0.5; g = -exp(a_log) softplus(a + dt_bias);
 *   beta = sigmoid(b); S <- exp(g) S; S <- S + k (beta (v - k^T S))^T; o = q^T S.
 * Replaces gdn_gate + gdn_recurrent_step of
 * models/qwen35_35b_a3b/sgl/python/sgl_kernel_axera/attention/gdn.py:919-989 (l2norm 919-931, gate 934-949)
 * with the golden of models/qwen35_35b_a3b/sgl/tests/test_gdn_attn.py:259-296. Value head h uses key head
 * h / (num_v_heads / num_k_heads).
 *   q, k  bf16 [batch, tokens, num_k_heads, 128];  v bf16 [batch, tokens, num_v_heads, 128]
 *   a, b  bf16 [batch, tokens, num_v_heads];        a_log, dt_bias f32 [num_v_heads]
 *   state_in / state_out f32 [batch, num_v_heads, 128, 128] (state_out == state_in: in place)
 *   out   bf16 [batch, tokens, num_v_heads, 128]
 * head_k_dim = head_v_dim = 128. */
int axk_gdn_recurrent(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* a,
                      const uint16_t* b, const float* a_log, const float* dt_bias, const float* state_in,
                      float* state_out, uint16_t* out, int64_t batch, int64_t tokens, int64_t num_k_heads,
                      int64_t num_v_heads, int64_t head_k_dim, int64_t head_v_dim, axk_stream_t stream);

/* Workspace bytes for axk_gdn_chunk_prefill (0 = unsupported shape). */
size_t axk_gdn_chunk_workspace_size(int64_t batch, int64_t tokens, int64_t num_k_heads, int64_t num_v_heads,
                                    int64_t head_k_dim, int64_t head_v_dim, int64_t chunk_size);

/* GDN over `tokens` tokens in the chunked (WY / unit-lower solve) form: the same recurrence as
 * axk_gdn_recurrent, computed chunk-parallel. Replaces gdn_stable_chunk + inverse_unit_lower_recursive +
 * chunk_prefix_sum_fp32 (models/qwen35_35b_a3b/sgl/python/sgl_kernel_axera/attention/gdn.py:992-1212) as driven
 * by gdn_prefill_impl (gdn.py:1628-1790) and q35_prefill.gdn_chunked
 * (models/qwen35_35b_a3b/src/70b0fbc/q35_prefill.py:144-169). Rounding points as the reference: bf16 operands
 * for every product (normalised q / k, beta, the inverse, u, w, q k^T * decay, the state, v_new), fp32
 * accumulation and an fp32 state.
 *   Tensors as axk_gdn_recurrent; chunk_size = 64; head dims 128. state_out == state_in: in place.
 *   workspace >= axk_gdn_chunk_workspace_size(...), 256-byte aligned (per-chunk solve results; reused
 *   freely between calls). */
int axk_gdn_chunk_prefill(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* a,
                          const uint16_t* b, const float* a_log, const float* dt_bias, const float* state_in,
                          float* state_out, uint16_t* out, int64_t batch, int64_t tokens, int64_t num_k_heads,
                          int64_t num_v_heads, int64_t head_k_dim, int64_t head_v_dim, int64_t chunk_size,
                          void* workspace, size_t workspace_bytes, axk_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * MoE with MXFP4 experts (router top-K, shared expert with sigmoid gate, routed SwiGLU experts)
 * ------------------------------------------------------------------------------------------- */

/* Workspace bytes for axk_moe_experts / axk_moe_decode (0 = unsupported shape). Always: num_experts <= 1024,
 * top_k <= 32, top_k <= num_experts, hidden % 64 == 0. Decode (tokens <= 256): tokens x top_k <= 8192,
 * inter and shared_inter % 32 == 0. Prefill (tokens > 256): tokens <= 65536, tokens x top_k <= 524288,
 * inter and shared_inter % 64 == 0, hidden, inter, shared_inter <= 8192. */
size_t axk_moe_workspace_size(int64_t tokens, int64_t hidden, int64_t num_experts, int64_t top_k, int64_t inter,
                              int64_t shared_inter);

/* Router top-K on fp32 logits [tokens, num_experts]: p = softmax(logits); the top_k experts by logit
 * (descending, ties to the lower expert id); weights = p / sum(p) when norm_topk_prob, else p.
 * Replaces route() of models/qwen35_35b_a3b/src/70b0fbc/q35_moe.py:293-297 and the softmax / topk /
 * renormalisation of q35_layer_mc.py:825-829 (tie rule: q35_layer_mc.py:1461-1466).
 * topk_ids i32 [tokens, top_k]; topk_weights f32 [tokens, top_k]. */
int axk_moe_route(const float* logits, int32_t* topk_ids, float* topk_weights, int64_t tokens, int64_t num_experts,
                  int64_t top_k, int norm_topk_prob, axk_stream_t stream);

/* Experts half of the MoE layer for given routing (moe_full, q35_layer_mc.py:797-853; moe_pre +
 * moe_experts_gu, q35_moe.py:96-137):
 *   act_s = bf16(silu(bf16(h2 Wsg^T)) * bf16(h2 Wsu^T)); sh = act_s Wsd^T; gate = sigmoid(h2 . w_shg)
 *   base = x_res + gate * sh;  out = bf16(base + sum_k w_k * down_e(bf16(silu(gate_e) * up_e)))
 *   (fp32 throughout; the reference rounds base to bf16 first, a difference of at most one bf16 ulp of base)
 *   h2, x_res (nullable) bf16 [tokens, hidden]; w_shg bf16 [hidden] (nullable: gate 1)
 *   shared expert (sh_* all NULL: none): gate / up MXFP4 [shared_inter, hidden/2] + [.., hidden/32],
 *     down [hidden, shared_inter/2] + [hidden, shared_inter/32]
 *   e_gw u8 [E, 2*inter, hidden/2] (gate rows, then up rows), e_gs u8 [E, 2*inter, hidden/32],
 *   e_dw u8 [E, hidden, inter/2], e_ds u8 [E, hidden, inter/32]
 *   topk_ids i32 / topk_weights f32 [tokens, top_k]: a row holds distinct expert ids (as the router's
 *     top-K does); an id outside [0, num_experts) selects nothing; out bf16 [tokens, hidden]. */
int axk_moe_experts(const uint16_t* h2, const uint16_t* x_res, const uint16_t* w_shg, const uint8_t* sh_gate_w,
                    const uint8_t* sh_gate_s, const uint8_t* sh_up_w, const uint8_t* sh_up_s,
                    const uint8_t* sh_down_w, const uint8_t* sh_down_s, const uint8_t* e_gw, const uint8_t* e_gs,
                    const uint8_t* e_dw, const uint8_t* e_ds, const int32_t* topk_ids, const float* topk_weights,
                    uint16_t* out, int64_t tokens, int64_t hidden, int64_t num_experts, int64_t top_k,
                    int64_t inter, int64_t shared_inter, void* workspace, size_t workspace_bytes,
                    axk_stream_t stream);

/* The whole decode MoE layer: logits = h2 w_router^T (bf16 router [E, hidden], fp32 logits out), then
 * axk_moe_route and axk_moe_experts. Outputs out, logits, topk_ids, topk_weights (the layer kernel's
 * h2 / logits_out / topk_i / topk_v IO of q35_layer_mc.py:437-449). */
int axk_moe_decode(const uint16_t* h2, const uint16_t* x_res, const uint16_t* w_router, const uint16_t* w_shg,
                   const uint8_t* sh_gate_w, const uint8_t* sh_gate_s, const uint8_t* sh_up_w,
                   const uint8_t* sh_up_s, const uint8_t* sh_down_w, const uint8_t* sh_down_s,
                   const uint8_t* e_gw, const uint8_t* e_gs, const uint8_t* e_dw, const uint8_t* e_ds,
                   uint16_t* out, float* logits, int32_t* topk_ids, float* topk_weights, int64_t tokens,
                   int64_t hidden, int64_t num_experts, int64_t top_k, int64_t inter, int64_t shared_inter,
                   int norm_topk_prob, void* workspace, size_t workspace_bytes, axk_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Per-layer glue of the hybrid decode layer (models/qwen35_35b_a3b/src/70b0fbc/q35_step.py gdn_layer 149-183,
 * attn_block 186-280, mlp_block 118-142). bf16 tensors as uint16_t, fp32 arithmetic, one bf16 rounding per op.
 * ------------------------------------------------------------------------------------------- */

/* RMSNorm of `rows` rows of n values: out = x * rsqrt(mean(x^2) + eps) * w (w f32 [n]: the reference's runtime
 * weight, 1 + weight for the layer / q / k norms, q35_step.py:346-348). Rows ldx / ldo elements apart.
 * Replaces rmsnorm(...) of q35_step.py:151, 190-194, 138. n % 8 == 0; x, w, out 16-byte aligned. */
int axk_rmsnorm(const uint16_t* x, int64_t ldx, const float* w, uint16_t* out, int64_t ldo, int64_t rows, int64_t n,
                float eps, axk_stream_t stream);

/* Residual add fused with the next RMSNorm: sum_out = bf16(x + y); norm_out = rmsnorm(sum_out, w).
 * Replaces x1 = add(xt, proj(...)) followed by rmsnorm(x1, ln2) (q35_step.py:181 / 279 and 138).
 * Contiguous [rows, n]; norm_out may not overlap the others. */
int axk_add_rmsnorm(const uint16_t* x, const uint16_t* y, const float* w, uint16_t* sum_out, uint16_t* norm_out,
                    int64_t rows, int64_t n, float eps, axk_stream_t stream);

/* GDN output norm: out = bf16(bf16(rmsnorm(x) * w) * silu(z)), per head row of n values (w = norm_w f32 [n],
 * not 1 + w). Replaces rmsnorm(core, norm_w) + silu_gate(normed, z) (q35_step.py:179-180). Contiguous
 * [rows, n]. */
int axk_gated_rmsnorm_silu(const uint16_t* x, const float* w, const uint16_t* z, uint16_t* out, int64_t rows,
                           int64_t n, float eps, axk_stream_t stream);

/* Stateful causal depthwise conv1d + SiLU over `tokens` tokens per sequence:
 *   out[b, t, c] = silu(sum_j x[b, t - j, c] * w[c, j]), j = 0 .. kernel - 1 (column 0 multiplies the current
 *   token, gdn_args q35_step.py:365-368), x[b, t - j] for t - j < 0 taken from state_in (oldest first);
 *   accumulated from j = 0 upwards with a bf16 rounding after each tap, silu in fp32 (the golden
 *   causal_conv1d_silu_reference, models/qwen35_35b_a3b/sgl/tests/test_gdn_attn.py:241-256).
 *   state_out = the last kernel - 1 inputs. Replaces stateful_runtime_causal_depthwise_conv1d_silu
 *   (q35_step.py:156).
 *   x, out bf16 [batch, tokens, channels]; w bf16 [channels, kernel]; state_in / state_out bf16
 *   [batch, kernel - 1, channels] (state_out == state_in: in place). kernel <= 8. */
int axk_causal_conv1d_silu(const uint16_t* x, const uint16_t* w, const uint16_t* state_in, uint16_t* state_out,
                           uint16_t* out, int64_t batch, int64_t tokens, int64_t channels, int64_t kernel,
                           axk_stream_t stream);

/* q / k head norm and partial NeoX RoPE: per (sequence b, head) row of head_dim values (rows ldx elements apart),
 * r = bf16(rmsnorm(x) * w); the first rot channels rotate by halves with cos / sin of sequence b:
 * y_i = r_i cos_i - r_{i+h} sin_i, y_{i+h} = r_{i+h} cos_i + r_i sin_i (h = rot / 2); the rest pass through.
 * Replaces rmsnorm(q, q_norm) / rmsnorm(k, k_norm) + rope(..., rotary_dim=ROT) (q35_step.py:192-197;
 * models/qwen38_27b/mtp/mtp_ref.py:176-187).
 *   x bf16 rows [batch * heads] x head_dim; w f32 [head_dim]; cos, sin bf16 [batch, rot / 2];
 *   out bf16 [batch, heads, head_dim] contiguous. head_dim in {64, 128, 256, 512}; (rot / 2) % (head_dim / 64) == 0. */
int axk_qk_norm_rope(const uint16_t* x, int64_t ldx, const float* w, const uint16_t* cos, const uint16_t* sin,
                     uint16_t* out, int64_t batch, int64_t heads, int64_t head_dim, int64_t rot, float eps,
                     axk_stream_t stream);

/* out = bf16(x * sigmoid(gate)) over rows x n (gate rows ldg apart: the gate half of the q projection).
 * Replaces sigmoid_mul(attn, gate) (q35_step.py:276-277). */
int axk_sigmoid_mul(const uint16_t* x, const uint16_t* gate, int64_t ldg, uint16_t* out, int64_t rows, int64_t n,
                    axk_stream_t stream);

/* out = bf16(silu(g) * u): the MLP activation, silu_mul (q35_step.py:136-137). Contiguous [rows, n]. */
int axk_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* out, int64_t rows, int64_t n, axk_stream_t stream);

/* out = bf16(x + y): the residual add (q35_step.py:139). Contiguous [rows, n]. */
int axk_add(const uint16_t* x, const uint16_t* y, uint16_t* out, int64_t rows, int64_t n, axk_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Decode layers of the hybrid group (one token per sequence, `batch` sequences), composed from the kernels above
 * on `stream`. The attention / GDN projections are in weight format proj_fmt and the MLP in mlp_fmt (AXK_WFMT_*):
 * each weight w_<x> with its scales s_<x> (f32 [N] for AXK_WFMT_FP8_CHANNEL, E8M0 bytes [N, K/32] for the MX formats,
 * hence `const void*`). Every intermediate lives in the caller's workspace (256-byte aligned, *_workspace_size bytes);
 * nothing is allocated or synchronised, so a layer can be captured in a HIP graph. hidden, inter % 256 == 0; every
 * projection's K a whole number of 128-byte weight rows. All checks run before the first launch: a nonzero status
 * means no state, conv state or cache byte changed.
 * ------------------------------------------------------------------------------------------- */

/* Workspace bytes of axk_gdn_layer_decode (0 = unsupported shape; head_dim must be 128). */
size_t axk_gdn_layer_workspace_size(int64_t batch, int64_t hidden, int64_t num_k_heads, int64_t num_v_heads,
                                    int64_t head_dim, int64_t inter);

/* The GDN layer, gdn_layer of models/qwen35_35b_a3b/src/70b0fbc/q35_step.py:149-183 (IO GDN_ORDER, :415-416):
 *   h = rmsnorm(x, ln1); qkv, z, b, a = h W^T; mixed = conv1d_silu(qkv) (state conv_in -> conv_out);
 *   core = GDN(q, k, v = mixed's channel ranges, a, b; state_in -> state_out);
 *   x1 = x + (bf16(rmsnorm(core, norm_w)) * silu(z)) W_out^T; out = x1 + MLP(rmsnorm(x1, ln2)).
 *   x, out bf16 [batch, hidden]; ln1, ln2 f32 [hidden] (1 + weight); w_qkv [2 KD + VD, hidden], w_z [VD, hidden],
 *   w_b, w_a [num_v_heads, hidden], w_out [hidden, VD] (FP8, scales f32 [N]); conv_w bf16 [2 KD + VD, conv_kernel];
 *   a_log, dt_bias f32 [num_v_heads]; norm_w f32 [head_dim]; MLP gate / up [inter, hidden], down [hidden, inter]
 *   (MXFP4); state f32 [batch, num_v_heads, 128, 128] (in place allowed); conv state bf16
 *   [batch, conv_kernel - 1, 2 KD + VD] (in place allowed). KD = num_k_heads * 128, VD = num_v_heads * 128.
 *   v_order: AXK_VORDER_TILED for weights exported in the reference's default layer order, AXK_VORDER_GROUPED for
 *   the checkpoint's (the same for every GDN layer entry). */
int axk_gdn_layer_decode(const uint16_t* x, const float* ln1, const uint8_t* w_qkv, const void* s_qkv,
                         const uint8_t* w_z, const void* s_z, const uint8_t* w_b, const void* s_b,
                         const uint8_t* w_a, const void* s_a, const uint16_t* conv_w, const float* a_log,
                         const float* dt_bias, const float* norm_w, const uint8_t* w_out, const void* s_out,
                         const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s,
                         const uint8_t* mlp_up_w, const void* mlp_up_s, const uint8_t* mlp_down_w,
                         const void* mlp_down_s, const float* state_in, const uint16_t* conv_in, uint16_t* out,
                         float* state_out, uint16_t* conv_out, int64_t batch, int64_t hidden, int64_t num_k_heads,
                         int64_t num_v_heads, int64_t head_dim, int64_t conv_kernel, int64_t inter, float eps,
                         int proj_fmt, int mlp_fmt, int v_order, void* workspace, size_t workspace_bytes,
                         axk_stream_t stream);

/* Workspace bytes of axk_attn_layer_decode (0 = unsupported shape). */
size_t axk_attn_layer_workspace_size(int64_t batch, int64_t hidden, int64_t num_qo_heads, int64_t num_kv_heads,
                                     int64_t head_dim, int64_t inter);

/* The attention layer, attn_block + mlp of q35_step.py:186-293 (IO ATTN_ORDER, :417-418) on the paged KV cache:
 *   h = rmsnorm(x, ln1); [q | gate] = h W_q^T per head; q = rope(rmsnorm(q, q_norm)); k = rope(rmsnorm(h W_k^T,
 *   k_norm)); v = h W_v^T; k, v written at cache_location; o = attention of q over each sequence's pages
 *   (indptr / indices / last_page_len including the new token); x1 = x + (o * sigmoid(gate)) W_o^T;
 *   out = x1 + MLP(rmsnorm(x1, ln2)).
 *   w_q [2 D num_qo_heads, hidden], w_k, w_v [D num_kv_heads, hidden], w_o [hidden, D num_qo_heads] (FP8 + f32
 *   scales); q_norm, k_norm f32 [D] (1 + weight); cos, sin bf16 [batch, rot / 2] (each sequence's position);
 *   kv_cache and the page table as axk_paged_decode, cache_location as axk_paged_kv_write. */
int axk_attn_layer_decode(const uint16_t* x, const float* ln1, const uint8_t* w_q, const void* s_q,
                          const uint8_t* w_k, const void* s_k, const uint8_t* w_v, const void* s_v,
                          const float* q_norm, const float* k_norm, const uint16_t* cos, const uint16_t* sin,
                          uint16_t* kv_cache, const int32_t* indptr, const int32_t* indices,
                          const int32_t* last_page_len, const int32_t* cache_location, const uint8_t* w_o,
                          const void* s_o, const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s,
                          const uint8_t* mlp_up_w, const void* mlp_up_s, const uint8_t* mlp_down_w,
                          const void* mlp_down_s, uint16_t* out, int64_t batch, int64_t hidden,
                          int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t rot,
                          int64_t page_size, int64_t num_pages, int64_t inter, float eps, float sm_scale,
                          int proj_fmt, int mlp_fmt, void* workspace, size_t workspace_bytes, axk_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * MoE decode layers: the decode layers above with the MLP replaced by the 35B's MoE block, moe_full of
 * models/qwen35_35b_a3b/src/70b0fbc/q35_layer_mc.py:797-853 (inside gdn_layer_full_mx / attn_layer_full_mx, :855-880):
 *   x1 = x + y (y: the attention / GDN half's output projection); h2 = rmsnorm(x1, ln2);
 *   sh = bf16(silu(bf16(h2 gate^T)) * bf16(h2 up^T)) down^T in fp32: the shared expert, the layer's MLP weights
 *        mlp_gate / mlp_up [inter, hidden], mlp_down [hidden, inter] in mlp_fmt (MXFP8 in the 35B manifest);
 *   logits = h2 w_router^T (fp32); the top_k experts by logit (ties: the lower id) weighted by their softmax
 *        probabilities, renormalised over the selection when norm_topk_prob;
 *   out = bf16(x1 + sigmoid(h2 . w_shg) sh + sum_k weight_k bf16(silu(g_k) u_k) down_k^T), the routed experts in
 *        MXFP4 as axk_moe_decode takes them (the manifest's planar e_gw / e_gs / e_dw / e_ds).
 * The reference rounds x1 + gate * sh to bf16 before adding the routed sum; here it stays fp32 up to the one final
 * rounding (at most one bf16 ulp of that sum apart). Decode routes (batch <= 256) run the decode experts; larger
 * batches the grouped prefill GEMMs. Other arguments, checks and workspace rules as the decode layers.
 * ------------------------------------------------------------------------------------------- */
typedef struct axk_moe_block {
  const uint16_t* w_router; /* bf16 [num_experts, hidden] */
  const uint16_t* w_shg;    /* bf16 [hidden]: the shared expert's sigmoid gate; null = gate 1 */
  const uint8_t* e_gw;      /* MXFP4 codes [num_experts, 2 expert_inter, hidden / 2] (gate rows, then up rows) */
  const uint8_t* e_gs;      /* E8M0 [num_experts, 2 expert_inter, hidden / 32] */
  const uint8_t* e_dw;      /* MXFP4 codes [num_experts, hidden, expert_inter / 2] */
  const uint8_t* e_ds;      /* E8M0 [num_experts, hidden, expert_inter / 32] */
  int64_t num_experts;
  int64_t top_k;
  int64_t expert_inter;
  int32_t norm_topk_prob;
  int32_t reserved; /* 0 */
  /* optional outputs (null: kept in the workspace), as the reference's MoE layer kernel stores logits_out / topk
   * (q35_layer_mc.py:435-449): */
  float* logits;        /* f32 [batch, num_experts] */
  int32_t* topk_ids;    /* i32 [batch, top_k], the experts by descending logit */
  float* topk_weights;  /* f32 [batch, top_k], their routing weights */
} axk_moe_block;

/* Workspace bytes of axk_gdn_layer_decode_moe / axk_attn_layer_decode_moe (0 = unsupported shape). */
size_t axk_gdn_layer_moe_workspace_size(int64_t batch, int64_t hidden, int64_t num_k_heads, int64_t num_v_heads,
                                        int64_t head_dim, int64_t inter, const axk_moe_block* moe);
size_t axk_attn_layer_moe_workspace_size(int64_t batch, int64_t hidden, int64_t num_qo_heads, int64_t num_kv_heads,
                                         int64_t head_dim, int64_t inter, const axk_moe_block* moe);

/* gdn_layer_full_mx (q35_layer_mc.py:855-866): axk_gdn_layer_decode with the MoE block as its MLP. */
int axk_gdn_layer_decode_moe(const uint16_t* x, const float* ln1, const uint8_t* w_qkv, const void* s_qkv,
                             const uint8_t* w_z, const void* s_z, const uint8_t* w_b, const void* s_b,
                             const uint8_t* w_a, const void* s_a, const uint16_t* conv_w, const float* a_log,
                             const float* dt_bias, const float* norm_w, const uint8_t* w_out, const void* s_out,
                             const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s,
                             const uint8_t* mlp_up_w, const void* mlp_up_s, const uint8_t* mlp_down_w,
                             const void* mlp_down_s, const axk_moe_block* moe, const float* state_in,
                             const uint16_t* conv_in, uint16_t* out, float* state_out, uint16_t* conv_out,
                             int64_t batch, int64_t hidden, int64_t num_k_heads, int64_t num_v_heads,
                             int64_t head_dim, int64_t conv_kernel, int64_t inter, float eps, int proj_fmt,
                             int mlp_fmt, int v_order, void* workspace, size_t workspace_bytes, axk_stream_t stream);

/* attn_layer_full_mx (q35_layer_mc.py:867-880): axk_attn_layer_decode with the MoE block as its MLP. */
int axk_attn_layer_decode_moe(const uint16_t* x, const float* ln1, const uint8_t* w_q, const void* s_q,
                              const uint8_t* w_k, const void* s_k, const uint8_t* w_v, const void* s_v,
                              const float* q_norm, const float* k_norm, const uint16_t* cos, const uint16_t* sin,
                              uint16_t* kv_cache, const int32_t* indptr, const int32_t* indices,
                              const int32_t* last_page_len, const int32_t* cache_location, const uint8_t* w_o,
                              const void* s_o, const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s,
                              const uint8_t* mlp_up_w, const void* mlp_up_s, const uint8_t* mlp_down_w,
                              const void* mlp_down_s, const axk_moe_block* moe, uint16_t* out, int64_t batch,
                              int64_t hidden, int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim,
                              int64_t rot, int64_t page_size, int64_t num_pages, int64_t inter, float eps,
                              float sm_scale, int proj_fmt, int mlp_fmt, void* workspace, size_t workspace_bytes,
                              axk_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Speculative verification: the decode layers over `tokens` (1 .. 16) consecutive new rows per sequence in one call,
 * the decode.verify role of models/qwen38_27b/README.md:11 (verify/verify_group_m4.py:1-9: a draft of up to 3 tokens
 * after the last cell checked in one pass; every projection shared by the rows, so each weight is read once; the row
 * recurrences in order). Row t of sequence b is row b * tokens + t of x / out bf16 [batch * tokens, hidden]. The
 * result equals `tokens` successive decode-layer calls, one row each. Arguments otherwise as the decode layers.
 * ------------------------------------------------------------------------------------------- */

/* Workspace bytes of axk_gdn_layer_verify / axk_attn_layer_verify (0 = unsupported shape; batch * tokens <= 4096). */
size_t axk_gdn_layer_verify_workspace_size(int64_t batch, int64_t tokens, int64_t hidden, int64_t num_k_heads,
                                           int64_t num_v_heads, int64_t head_dim, int64_t inter);
size_t axk_attn_layer_verify_workspace_size(int64_t batch, int64_t tokens, int64_t hidden, int64_t num_qo_heads,
                                            int64_t num_kv_heads, int64_t head_dim, int64_t inter);

/* The GDN layer over the rows of each sequence in order (verify_group_m4.py gdn_rows 147-243). state_out / conv_out:
 * after the last row (may be the inputs: in place). Per-row snapshots (each optional, NULL = none), the verify
 * group's ssnap / cqsnap / cksnap / cvsnap: state_snap f32 [tokens, batch, NV, 128, 128] = the state after row t,
 * conv_snap bf16 [tokens, batch, conv_kernel - 1, 2 KD + VD] = the conv state after row t (oldest first; the q / k / v
 * channel ranges of the reference's three conv states). conv_kernel >= 2. */
int axk_gdn_layer_verify(const uint16_t* x, const float* ln1, const uint8_t* w_qkv, const void* s_qkv,
                         const uint8_t* w_z, const void* s_z, const uint8_t* w_b, const void* s_b, const uint8_t* w_a,
                         const void* s_a, const uint16_t* conv_w, const float* a_log, const float* dt_bias,
                         const float* norm_w, const uint8_t* w_out, const void* s_out, const float* ln2,
                         const uint8_t* mlp_gate_w, const void* mlp_gate_s, const uint8_t* mlp_up_w,
                         const void* mlp_up_s, const uint8_t* mlp_down_w, const void* mlp_down_s,
                         const float* state_in, const uint16_t* conv_in, uint16_t* out, float* state_out,
                         uint16_t* conv_out, float* state_snap, uint16_t* conv_snap, int64_t batch, int64_t tokens,
                         int64_t hidden, int64_t num_k_heads, int64_t num_v_heads, int64_t head_dim,
                         int64_t conv_kernel, int64_t inter, float eps, int proj_fmt, int mlp_fmt, int v_order,
                         void* workspace, size_t workspace_bytes, axk_stream_t stream);

/* The attention layer over the rows (verify_group_m4.py attn_rows 226-300): every row's K / V is written at its
 * cache_location (i32 [batch * tokens, 2]), then row t attends its sequence's history and rows 0 .. t (the page table
 * covers all the new rows; they are the sequence's last `tokens` tokens). cos, sin bf16 [batch * tokens, rot / 2]:
 * each row's position. page_size a multiple of 16; head_dim 64, 128 or 256. */
int axk_attn_layer_verify(const uint16_t* x, const float* ln1, const uint8_t* w_q, const void* s_q, const uint8_t* w_k,
                          const void* s_k, const uint8_t* w_v, const void* s_v, const float* q_norm,
                          const float* k_norm, const uint16_t* cos, const uint16_t* sin, uint16_t* kv_cache,
                          const int32_t* indptr, const int32_t* indices, const int32_t* last_page_len,
                          const int32_t* cache_location, const uint8_t* w_o, const void* s_o, const float* ln2,
                          const uint8_t* mlp_gate_w, const void* mlp_gate_s, const uint8_t* mlp_up_w,
                          const void* mlp_up_s, const uint8_t* mlp_down_w, const void* mlp_down_s, uint16_t* out,
                          int64_t batch, int64_t tokens, int64_t hidden, int64_t num_qo_heads, int64_t num_kv_heads,
                          int64_t head_dim, int64_t rot, int64_t page_size, int64_t num_pages, int64_t inter,
                          float eps, float sm_scale, int proj_fmt, int mlp_fmt, void* workspace,
                          size_t workspace_bytes, axk_stream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Prefill: `tokens` (1 .. 65536) new tokens per sequence through a layer in one call, batch * tokens <= 131072
 * (models/qwen35_35b_a3b/src/70b0fbc/q35_prefill.py: gdn_layer_prefill 57-141, attn_layer_prefill 172-336). Row t of
 * sequence b is row b * tokens + t of x / out bf16 [batch * tokens, hidden]. Every projection and the MLP are
 * matrix products over the batch * tokens rows; the recurrences run over each sequence's tokens in order. No
 * per-row snapshots (the verify layers keep those). Arguments otherwise as the verify layers.
 * ------------------------------------------------------------------------------------------- */

/* Workspace bytes of axk_gdn_layer_prefill / axk_attn_layer_prefill (0 = unsupported shape). */
size_t axk_gdn_layer_prefill_workspace_size(int64_t batch, int64_t tokens, int64_t hidden, int64_t num_k_heads,
                                            int64_t num_v_heads, int64_t head_dim, int64_t inter);
size_t axk_attn_layer_prefill_workspace_size(int64_t batch, int64_t tokens, int64_t hidden, int64_t num_qo_heads,
                                             int64_t num_kv_heads, int64_t head_dim, int64_t inter);

/* The GDN layer over each sequence's tokens (q35_prefill.py gdn_layer_prefill 57-141): the causal conv over the
 * tokens from conv_in, the delta rule in the chunked form (64-token chunks, as axk_gdn_chunk_prefill) from state_in.
 * state_out f32 [batch, NV, 128, 128] / conv_out bf16 [batch, conv_kernel - 1, 2 KD + VD]: after the last token (may
 * be the inputs: in place). head_dim 128. */
int axk_gdn_layer_prefill(const uint16_t* x, const float* ln1, const uint8_t* w_qkv, const void* s_qkv,
                          const uint8_t* w_z, const void* s_z, const uint8_t* w_b, const void* s_b, const uint8_t* w_a,
                          const void* s_a, const uint16_t* conv_w, const float* a_log, const float* dt_bias,
                          const float* norm_w, const uint8_t* w_out, const void* s_out, const float* ln2,
                          const uint8_t* mlp_gate_w, const void* mlp_gate_s, const uint8_t* mlp_up_w,
                          const void* mlp_up_s, const uint8_t* mlp_down_w, const void* mlp_down_s,
                          const float* state_in, const uint16_t* conv_in, uint16_t* out, float* state_out,
                          uint16_t* conv_out, int64_t batch, int64_t tokens, int64_t hidden, int64_t num_k_heads,
                          int64_t num_v_heads, int64_t head_dim, int64_t conv_kernel, int64_t inter, float eps,
                          int proj_fmt, int mlp_fmt, int v_order, void* workspace, size_t workspace_bytes,
                          axk_stream_t stream);

/* The attention layer over each sequence's tokens (q35_prefill.py attn_layer_prefill 172-336): every token's K / V
 * is written at its cache_location (i32 [batch * tokens, 2]), then token t attends its sequence's history and tokens
 * 0 .. t (the page table covers the history and all the new tokens). cos, sin bf16 [batch * tokens, rot / 2]. */
int axk_attn_layer_prefill(const uint16_t* x, const float* ln1, const uint8_t* w_q, const void* s_q,
                           const uint8_t* w_k, const void* s_k, const uint8_t* w_v, const void* s_v,
                           const float* q_norm, const float* k_norm, const uint16_t* cos, const uint16_t* sin,
                           uint16_t* kv_cache, const int32_t* indptr, const int32_t* indices,
                           const int32_t* last_page_len, const int32_t* cache_location, const uint8_t* w_o,
                           const void* s_o, const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s,
                           const uint8_t* mlp_up_w, const void* mlp_up_s, const uint8_t* mlp_down_w,
                           const void* mlp_down_s, uint16_t* out, int64_t batch, int64_t tokens, int64_t hidden,
                           int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim, int64_t rot,
                           int64_t page_size, int64_t num_pages, int64_t inter, float eps, float sm_scale,
                           int proj_fmt, int mlp_fmt, void* workspace, size_t workspace_bytes, axk_stream_t stream);

/* The 35B's MoE prefill layers (models/qwen35_35b_a3b/src/70b0fbc/q35_moe_prefill.py: qwen35moe_gdn_prefill /
 * qwen35moe_attn_prefill 47-77, the layer up to its MLP then moe_pre on the P rows, q35_moe.py:123-137; the routed
 * experts of the P tokens grouped by expert and combined, moe_slots_px / moe_combine 150-214): the prefill layers
 * with the MoE block of axk_gdn_layer_decode_moe as their MLP, over the batch * tokens rows (more than 256 rows take
 * the grouped prefill expert GEMMs, whose per-(token, slot) outputs are bf16 as the reference's slot kernels store
 * them). moe's optional routing outputs are [batch * tokens, ...]. Arguments otherwise as the prefill layers. */
size_t axk_gdn_layer_prefill_moe_workspace_size(int64_t batch, int64_t tokens, int64_t hidden, int64_t num_k_heads,
                                                int64_t num_v_heads, int64_t head_dim, int64_t inter,
                                                const axk_moe_block* moe);
size_t axk_attn_layer_prefill_moe_workspace_size(int64_t batch, int64_t tokens, int64_t hidden, int64_t num_qo_heads,
                                                 int64_t num_kv_heads, int64_t head_dim, int64_t inter,
                                                 const axk_moe_block* moe);
int axk_gdn_layer_prefill_moe(const uint16_t* x, const float* ln1, const uint8_t* w_qkv, const void* s_qkv,
                              const uint8_t* w_z, const void* s_z, const uint8_t* w_b, const void* s_b,
                              const uint8_t* w_a, const void* s_a, const uint16_t* conv_w, const float* a_log,
                              const float* dt_bias, const float* norm_w, const uint8_t* w_out, const void* s_out,
                              const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s,
                              const uint8_t* mlp_up_w, const void* mlp_up_s, const uint8_t* mlp_down_w,
                              const void* mlp_down_s, const axk_moe_block* moe, const float* state_in,
                              const uint16_t* conv_in, uint16_t* out, float* state_out, uint16_t* conv_out,
                              int64_t batch, int64_t tokens, int64_t hidden, int64_t num_k_heads,
                              int64_t num_v_heads, int64_t head_dim, int64_t conv_kernel, int64_t inter, float eps,
                              int proj_fmt, int mlp_fmt, int v_order, void* workspace, size_t workspace_bytes,
                              axk_stream_t stream);
int axk_attn_layer_prefill_moe(const uint16_t* x, const float* ln1, const uint8_t* w_q, const void* s_q,
                               const uint8_t* w_k, const void* s_k, const uint8_t* w_v, const void* s_v,
                               const float* q_norm, const float* k_norm, const uint16_t* cos, const uint16_t* sin,
                               uint16_t* kv_cache, const int32_t* indptr, const int32_t* indices,
                               const int32_t* last_page_len, const int32_t* cache_location, const uint8_t* w_o,
                               const void* s_o, const float* ln2, const uint8_t* mlp_gate_w, const void* mlp_gate_s,
                               const uint8_t* mlp_up_w, const void* mlp_up_s, const uint8_t* mlp_down_w,
                               const void* mlp_down_s, const axk_moe_block* moe, uint16_t* out, int64_t batch,
                               int64_t tokens, int64_t hidden, int64_t num_qo_heads, int64_t num_kv_heads,
                               int64_t head_dim, int64_t rot, int64_t page_size, int64_t num_pages, int64_t inter,
                               float eps, float sm_scale, int proj_fmt, int mlp_fmt, void* workspace,
                               size_t workspace_bytes, axk_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* AXK_H */
