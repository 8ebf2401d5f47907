// HBM bandwidth calibration for the benchmark (not part of the attention
// path or its C ABI): a device-to-device copy of a given size with
// 16-byte non-temporal accesses, so that bench.py can report, in the same
// run, what a plain copy of the prologue's bytes sustains on this part.
//
//   variant 0..3: grid-stride loop, (2048 | 8192) workgroups of 256 lanes,
//                 (4 | 8) loads in flight per lane before their stores
//   variant 4:    one-shot grid, every lane one 64-byte span (4 loads)
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int U>
__global__ __launch_bounds__(256) void copy_stride(const u32x4* __restrict__ a,
                                                   u32x4* __restrict__ b,
                                                   int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 256 * U;
  for (int64_t i = (int64_t)blockIdx.x * 256 * U + threadIdx.x; i < n;
       i += stride) {
    u32x4 r[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i + u * 256 < n) r[u] = __builtin_nontemporal_load(a + i + u * 256);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i + u * 256 < n) __builtin_nontemporal_store(r[u], b + i + u * 256);
  }
}

}  // namespace

extern "C" int dt_calib_copy_variants(void) { return 5; }

// Copies `bytes` (a multiple of 16; both pointers 16-byte aligned) from src
// to dst on `stream`.  Returns 0, or -1 on a bad argument or launch error.
extern "C" int dt_calib_copy(const void* src, void* dst, size_t bytes,
                             int variant, void* stream) {
  if (!src || !dst || bytes % 16 || ((uintptr_t)src & 15) ||
      ((uintptr_t)dst & 15) || variant < 0 || variant > 4)
    return -1;
  const int64_t n = (int64_t)(bytes / 16);
  const u32x4* a = (const u32x4*)src;
  u32x4* b = (u32x4*)dst;
  hipStream_t st = (hipStream_t)stream;
  const int grid = (variant & 1) ? 8192 : 2048;
  switch (variant) {
    case 0:
    case 1:
      hipLaunchKernelGGL(copy_stride<4>, dim3(grid), dim3(256), 0, st, a, b, n);
      break;
    case 2:
    case 3:
      hipLaunchKernelGGL(copy_stride<8>, dim3(grid), dim3(256), 0, st, a, b, n);
      break;
    default: {
      const int64_t g = (n + 256 * 4 - 1) / (256 * 4);
      if (g > 0x7fffffff) return -1;
      hipLaunchKernelGGL(copy_stride<4>, dim3((unsigned)g), dim3(256), 0, st,
                         a, b, n);
    }
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
