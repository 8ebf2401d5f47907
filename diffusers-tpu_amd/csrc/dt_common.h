// Shared device/host helpers for the gfx950 attention-path kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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

// The key length a kernel runs with: the host value, or when the caller
// passed the length in device memory (a runtime scalar that one captured
// graph can vary between replays), that value read at run time, with
// n <= 0 or n > limit meaning `limit` (every key).
__device__ __forceinline__ int resolve_len(const int32_t* dev, int host,
                                           int limit) {
  if (dev == nullptr) return host;
  const int n = __builtin_amdgcn_readfirstlane(*dev);
  return (n <= 0 || n > limit) ? limit : n;
}

}  // namespace dt
