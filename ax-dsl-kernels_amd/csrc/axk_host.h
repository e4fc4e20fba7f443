// Host-side helpers for the C-ABI entry points: argument checks and launch status.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

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

// Internal (not exported): the GDN recurrence with row strides, in elements between consecutive (sequence, token)
// rows, for q, k, v and a / b. axk_gdn_recurrent passes the contiguous strides; the decode layer reads q / k / v
// straight out of the conv output. Returns an AXK status.
struct AxkGdnStrides {
  int64_t q, k, v, ab;
};
__attribute__((visibility("hidden"))) int axk_gdn_recurrent_strided(
    const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* a, const uint16_t* b, const float* a_log,
    const float* dt_bias, const float* state_in, float* state_out, uint16_t* out, int64_t batch, int64_t tokens,
    int64_t num_k_heads, int64_t num_v_heads, const AxkGdnStrides& ld, hipStream_t stream);
