// Per-head maximum L2 row norm (gfx950): the reduction behind the fixed-m
// softmax bound.  Replaces fixed_m_bound.max_row_norm_per_head
// (kernels/fixed_m_bound.py:57-73) and the scaled-query form
// fixed_m_query_norms (:76-95), which folds the softmax scale in as a factor.
//
// One HBM pass over x, 16-byte non-temporal loads: D/8 lanes hold one row
// (8 bf16 each), a wavefront covers 64/(D/8) rows per load and each lane
// keeps 8 loads in flight.  Sums of squares reduce across the row's lanes
// with xor-shuffles; the block's maximum goes to out[h] with one
// atomic max on the float bits (non-negative floats order like unsigned
// integers), so blocks of one head need no second pass and several calls
// (q and k shards, batches) can accumulate into one output.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/dt_attention.h"
#include "dt_common.h"

namespace dt {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 8;  // loads in flight per lane (4: 3.5 % slower at V7)

template <int D>
__global__ __launch_bounds__(kThreads) void row_norm_max_kernel(
    const uint16_t* __restrict__ x, int64_t sb, int64_t sh, int64_t ss, int S,
    int H, int rows_per_block, float factor, float* __restrict__ out) {
  constexpr int kLanesPerRow = D / 8;
  constexpr int kRowsPerWave = 64 / kLanesPerRow;
  constexpr int kRowsPerStep = kRowsPerWave * (kThreads / 64);
  __shared__ float s_max[kThreads / 64];

  const int bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  const uint16_t* base = x + b * sb + h * sh;
  const int s_begin = blockIdx.x * rows_per_block;
  const int s_end = min(S, s_begin + rows_per_block);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int part = lane % kLanesPerRow;
  const int row0 = s_begin + wave * kRowsPerWave + lane / kLanesPerRow;

  float best = 0.f;
  for (int s = row0; s < s_end; s += kUnroll * kRowsPerStep) {
    u32x4 raw[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int r = s + u * kRowsPerStep;
      raw[u] = u32x4{0u, 0u, 0u, 0u};
      if (r < s_end)
        raw[u] = __builtin_nontemporal_load(
            (const u32x4*)(base + (int64_t)r * ss + part * 8));
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = __uint_as_float(raw[u][e] << 16);
        const float hi = __uint_as_float(raw[u][e] & 0xffff0000u);
        acc = __builtin_fmaf(lo, lo, acc);
        acc = __builtin_fmaf(hi, hi, acc);
      }
      // every lane of a row group takes the same branches: the shuffles
      // stay inside the group
#pragma unroll
      for (int off = kLanesPerRow / 2; off > 0; off >>= 1)
        acc += __shfl_xor(acc, off, 64);
      best = fmaxf(best, acc);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
    best = fmaxf(best, __shfl_xor(best, off, 64));
  if (lane == 0) s_max[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    float m = s_max[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) m = fmaxf(m, s_max[w]);
    atomicMax((unsigned int*)(out + h), __float_as_uint(sqrtf(m) * factor));
  }
}

}  // namespace
}  // namespace dt

extern "C" int dt_max_row_norm(const uint16_t* x, int B, int H, int S, int D,
                               const int64_t* strides, float factor, float* out,
                               void* stream) {
  using namespace dt;
  if (!x || !strides || !out)
    return set_error(DT_ERR_ARG, "dt_max_row_norm: null pointer argument");
  if (B <= 0 || H <= 0 || S <= 0)
    return set_error(DT_ERR_SHAPE, "dt_max_row_norm: B=%d H=%d S=%d", B, H, S);
  if (D != 64 && D != 128 && D != 256)
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_max_row_norm: head dim %d (supported: 64, 128, 256)",
                     D);
  if (!(factor >= 0.f) || !isfinite(factor))
    return set_error(DT_ERR_ARG, "dt_max_row_norm: factor %g must be >= 0",
                     (double)factor);
  if (((uintptr_t)x & 15u) || strides[0] % 8 || strides[1] % 8 ||
      strides[2] % 8)
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_max_row_norm: x must be 16-byte aligned with strides "
                     "that are multiples of 8 elements");
  if ((int64_t)B * H > 65535)
    return set_error(DT_ERR_SHAPE, "dt_max_row_norm: B*H %d too large", B * H);
  // about 2048 blocks over the grid; whole load steps per block
  const int step = 4 * (64 / (D / 8)) * kUnroll;
  const int per_slice = (2048 + B * H - 1) / (B * H);
  int rows = (S + per_slice - 1) / per_slice;
  rows = ((rows + step - 1) / step) * step;
  const int nblk = (S + rows - 1) / rows;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid(nblk, B * H);
  if (D == 256)
    hipLaunchKernelGGL(row_norm_max_kernel<256>, grid, dim3(kThreads), 0, st, x,
                       strides[0], strides[1], strides[2], S, H, rows, factor,
                       out);
  else if (D == 128)
    hipLaunchKernelGGL(row_norm_max_kernel<128>, grid, dim3(kThreads), 0, st, x,
                       strides[0], strides[1], strides[2], S, H, rows, factor,
                       out);
  else
    hipLaunchKernelGGL(row_norm_max_kernel<64>, grid, dim3(kThreads), 0, st, x,
                       strides[0], strides[1], strides[2], S, H, rows, factor,
                       out);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "dt_max_row_norm: %s", hipGetErrorString(e));
  return DT_OK;
}
