/* Oracle (test infrastructure only): plain-C restatement of the MXFP4 codec and the MXFP4 linear.
 *
 *  oracle_mxfp4_dequant  follows models/qwen35_35b_a3b/src/70b0fbc/q35_moe.py:60-63
 *                        (value = E2M1[code & 7] * (code >= 8 ? -1 : 1) * 2^(scale - 127), fp32)
 *  oracle_mxfp4_linear   follows the golden pattern of q35_moe.py:234-238 / sgl gemm.py:564-598:
 *                        out = x(bf16 values, fp32) . dequant(W)^T, fp32 accumulation in K order.
 * Used by tests (checked against oracle/mx.py and the exhaustive table) and as bench.py's CPU
 * baseline (OpenMP over output channels). Never linked into the product library.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static const float kE2M1[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

static float e8m0(uint8_t s) { return ldexpf(1.0f, (int)s - 127); }

static float fp4(uint8_t c) {
  const float m = kE2M1[c & 7];
  return (c & 8) ? -m : m;
}

static float bf16(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void oracle_mxfp4_dequant(const uint8_t* codes, const uint8_t* scales, float* out, int64_t n, int64_t k) {
  for (int64_t r = 0; r < n; ++r)
    for (int64_t j = 0; j < k; ++j) {
      const uint8_t byte = codes[r * (k / 2) + j / 2];
      const uint8_t c = (j & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 15);
      out[r * k + j] = fp4(c) * e8m0(scales[r * (k / 32) + j / 32]);
    }
}

/* x: bf16 bits [m, k]; out: fp32 [m, n]. */
void oracle_mxfp4_linear(const uint16_t* x, int64_t m, const uint8_t* codes, const uint8_t* scales, float* out,
                         int64_t n, int64_t k, int nthreads) {
#pragma omp parallel for schedule(static) num_threads(nthreads)
  for (int64_t r = 0; r < n; ++r) {
    for (int64_t i = 0; i < m; ++i) {
      float acc = 0.0f;
      for (int64_t b = 0; b < k / 32; ++b) {
        const float sc = e8m0(scales[r * (k / 32) + b]);
        for (int j = 0; j < 32; ++j) {
          const int64_t kk = b * 32 + j;
          const uint8_t byte = codes[r * (k / 2) + kk / 2];
          const uint8_t c = (kk & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 15);
          acc += bf16(x[i * k + kk]) * (fp4(c) * sc);
        }
      }
      out[i * n + r] = acc;
    }
  }
}
