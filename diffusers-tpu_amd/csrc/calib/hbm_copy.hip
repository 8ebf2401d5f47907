// HBM bandwidth calibration for the benchmark (not part of the attention
// path or its C ABI): a device-to-device copy of a given size with
// 16-byte non-temporal accesses, so that bench.py can report, in the same
// run, what a plain copy of the prologue's bytes sustains on this part.
//
//   variant 0..3: grid-stride loop, (2048 | 8192) workgroups of 256 lanes,
//                 (4 | 8) loads in flight per lane before their stores
//   variant 4:    one-shot grid, every lane one 64-byte span (4 loads)
//
// dt_calib_bshd_copy: the prologue's access pattern without its arithmetic:
// q and k [B, S, H, 128] bf16 in, [B, H, S, 128] out (the BSHD read and
// BHSD write of dt_qk_norm_rope, the same bytes), so that the bench can
// price the prologue against a copy that moves its bytes the same way.
//   variant 0:    the prologue's own mapping: an 8-lane group per token,
//                 a chunk of two of the token's 2H rows per grid row, each
//                 lane two 16-byte pieces of a row (128 B apart)
//   variant 1..3: head-major: 16 lanes per row, a wavefront takes one row
//                 (q or k head) of 4U consecutive tokens, U = 2, 4, 8 loads
//                 in flight per lane; its stores are 4U * 256 contiguous
//                 bytes, its loads 256-byte rows H * 256 bytes apart
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

// the prologue's mapping (qk_norm_rope_kernel<128, 2, false> at rotary 128)
__global__ __launch_bounds__(256) void bshd_copy_prologue(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    uint16_t* __restrict__ qo, uint16_t* __restrict__ ko, int S, int H,
    uint32_t ntok) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 7, grp = lane >> 3;
  const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const uint32_t tok = wave * 8u + grp;
  if (tok >= ntok) return;
  const int b = (int)(tok / (uint32_t)S), s = (int)(tok - (uint32_t)b * S);
  const int r0 = blockIdx.y * 2, r1 = min(r0 + 2, 2 * H);
  const int c0 = li, c1 = li + 8;
  u32x4 v[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = r0 + i;
    if (r >= r1) continue;
    const uint16_t* src = (r >= H ? k : q) +
                          (((int64_t)b * S + s) * H + (r >= H ? r - H : r)) * 128;
    v[i][0] = __builtin_nontemporal_load((const u32x4*)(src + c0 * 8));
    v[i][1] = __builtin_nontemporal_load((const u32x4*)(src + c1 * 8));
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = r0 + i;
    if (r >= r1) continue;
    uint16_t* dst = (r >= H ? ko : qo) +
                    (((int64_t)b * H + (r >= H ? r - H : r)) * S + s) * 128;
    __builtin_nontemporal_store(v[i][0], (u32x4*)(dst + c0 * 8));
    __builtin_nontemporal_store(v[i][1], (u32x4*)(dst + c1 * 8));
  }
}

// head-major: wavefront = one row r of 4U consecutive tokens
template <int U>
__global__ __launch_bounds__(256) void bshd_copy_rows(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    uint16_t* __restrict__ qo, uint16_t* __restrict__ ko, int S, int H,
    uint32_t ntok) {
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, t = lane >> 4;
  const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int r = blockIdx.y;
  const bool isk = r >= H;
  const int h = isk ? r - H : r;
  const uint16_t* src = isk ? k : q;
  uint16_t* dst = isk ? ko : qo;
  u32x4 v[U];
  uint32_t toks[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    toks[u] = wave * (4u * U) + 4u * u + t;
    if (toks[u] < ntok)
      v[u] = __builtin_nontemporal_load(
          (const u32x4*)(src + ((int64_t)toks[u] * H + h) * 128 + c * 8));
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (toks[u] >= ntok) continue;
    const int b = (int)(toks[u] / (uint32_t)S);
    const int s = (int)(toks[u] - (uint32_t)b * S);
    __builtin_nontemporal_store(
        v[u], (u32x4*)(dst + (((int64_t)b * H + h) * S + s) * 128 + c * 8));
  }
}

}  // namespace

extern "C" int dt_calib_bshd_copy_variants(void) { return 4; }

// q, k: contiguous [B, S, H, 128] bf16; qo, ko: contiguous [B, H, S, 128].
// Returns 0, or -1 on a bad argument or launch error.
extern "C" int dt_calib_bshd_copy(const void* q, const void* k, void* qo,
                                  void* ko, int B, int S, int H, int variant,
                                  void* stream) {
  if (!q || !k || !qo || !ko || B <= 0 || S <= 0 || H <= 0 || variant < 0 ||
      variant > 3 || (int64_t)B * S >= (1ll << 31))
    return -1;
  const uint32_t ntok = (uint32_t)((int64_t)B * S);
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* a = (const uint16_t*)q;
  const uint16_t* b = (const uint16_t*)k;
  uint16_t* x = (uint16_t*)qo;
  uint16_t* y = (uint16_t*)ko;
  if (variant == 0) {
    const int64_t waves = ((int64_t)ntok + 7) / 8;
    const dim3 grid((unsigned)((waves + 3) / 4), (unsigned)((2 * H + 1) / 2));
    hipLaunchKernelGGL(bshd_copy_prologue, grid, dim3(256), 0, st, a, b, x, y,
                       S, H, ntok);
  } else {
    const int U = variant == 1 ? 2 : (variant == 2 ? 4 : 8);
    const int64_t waves = ((int64_t)ntok + 4 * U - 1) / (4 * U);
    const dim3 grid((unsigned)((waves + 3) / 4), (unsigned)(2 * H));
    if (U == 2)
      hipLaunchKernelGGL(bshd_copy_rows<2>, grid, dim3(256), 0, st, a, b, x, y,
                         S, H, ntok);
    else if (U == 4)
      hipLaunchKernelGGL(bshd_copy_rows<4>, grid, dim3(256), 0, st, a, b, x, y,
                         S, H, ntok);
    else
      hipLaunchKernelGGL(bshd_copy_rows<8>, grid, dim3(256), 0, st, a, b, x, y,
                         S, H, ntok);
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

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
