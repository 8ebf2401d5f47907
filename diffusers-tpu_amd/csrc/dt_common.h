// Shared device/host helpers for the gfx950 attention-path kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dt_attention.h"

namespace dt {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Records a message for dt_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);

// bf16 <-> fp32, round-to-nearest-even (what the hardware convert does).
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// The key length a kernel runs with for batch element b: the host value,
// or, when the caller passed the length in device memory (a runtime scalar
// that one captured graph can vary between replays), the value read at run
// time: one int32 for every batch element (count <= 1) or one per batch
// element (count > 1, entry b).  A device value <= 0 means no keys (the
// kernels then write the empty-row result), one above `limit` means
// `limit`.
__device__ __forceinline__ int resolve_len(const int32_t* dev, int count,
                                           int b, int host, int limit) {
  if (dev == nullptr) return host;
  const int n = __builtin_amdgcn_readfirstlane(dev[count > 1 ? b : 0]);
  return n <= 0 ? 0 : (n > limit ? limit : n);
}

// Host side of a device length argument: with `dev` given, the ABI's host
// length argument `host` is the number of int32 entries `dev` points to:
// 0 or 1 (one length for every batch element) or B (one per batch element).
// Stores the count for resolve_len; returns DT_OK or DT_ERR_ARG.
inline int dev_len_count(const int32_t* dev, int host, int B, const char* who,
                         int* count) {
  *count = 0;
  if (dev == nullptr) return 0;
  if (host != 0 && host != 1 && host != B)
    return set_error(DT_ERR_ARG,
                     "%s: with a device length the length argument is its "
                     "entry count (0 or 1: one for the batch, or B = %d), "
                     "got %d",
                     who, B, host);
  *count = host;
  return 0;
}

}  // namespace dt
