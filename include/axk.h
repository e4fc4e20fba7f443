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

/* AX dtype codes used on the boundary (tools/manifest/onnx_io.py:18-29) */
#define AXK_DT_U8 1
#define AXK_DT_F32 3
#define AXK_DT_I32 6
#define AXK_DT_BF16 9
#define AXK_DT_F16 10
#define AXK_DT_FP8E4M3 11
#define AXK_DT_FP8E5M2 12
#define AXK_DT_FP4 15

/* Library identification and error text. */
const char* axk_version(void);
const char* axk_status_string(int status);

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

/* Dense bf16-weight linear (router logits and other small bf16 projections):
 * output = a @ b.T + bias, fp32 accumulation. Replaces sgl_kernel_axera.gemm.fp16_gemm / bf16_gemm
 * (gemm.py:81-116, 469-476). a bf16 [m, k]; b bf16 [n, k]; k % 32 == 0. */
int axk_bf16_gemm(const uint16_t* a, int64_t lda, const uint16_t* b, const float* bias, void* out,
                  int out_dtype, int64_t m, int64_t n, int64_t k, axk_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* AXK_H */
