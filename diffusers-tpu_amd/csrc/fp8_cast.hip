// Saturating E4M3 cast of bf16 tensors (gfx950): the qk_fp8 key cast.
// Replaces fp8_cast.quantize_saturating (kernels/fp8_cast.py:28-39), which
// clips to +-448 (E4M3_MAX, kernels/e4m3.py:25) and casts to float8_e4m3fn.
//
// HBM-bound elementwise pass: each lane reads 16 bytes (8 bf16) with a
// non-temporal load and writes 8 bytes; rows are addressed through
// (b, h, s) strides so (B,S,H,D) storage converts to a contiguous
// (B,H,S,D) E4M3 copy in the same pass.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/dt_attention.h"
#include "flash_common.h"

namespace dt {
namespace {

struct CastParams {
  const uint16_t* x;
  uint8_t* y;
  int64_t xs0, xs1, xs2, ys0, ys1, ys2;
  int H, S, lanes_per_row;  // D / 8
  float factor;
};

__global__ __launch_bounds__(256) void e4m3_cast_kernel(CastParams p) {
  // blockIdx.y: one (b, h) slice; x: its S * D/8 16-byte items
  const int h = blockIdx.y % p.H;
  const int64_t b = blockIdx.y / p.H;
  const int n = p.S * p.lanes_per_row;
  for (int it = blockIdx.x * blockDim.x + threadIdx.x; it < n;
       it += gridDim.x * blockDim.x) {
    const int s = it / p.lanes_per_row;
    const int part = it - s * p.lanes_per_row;
    const u32x4 raw = __builtin_nontemporal_load(
        (const u32x4*)(p.x + b * p.xs0 + h * p.xs1 + s * p.xs2 + part * 8));
    u32x2 out;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      uint32_t w[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t v = raw[2 * e + j];
        w[j] = pack_bf16x2(__uint_as_float(v << 16) * p.factor,
                           __uint_as_float(v & 0xffff0000u) * p.factor);
      }
      out[e] = (uint32_t)pack_e4m3x4(w[0], w[1]);
    }
    __builtin_nontemporal_store(
        out, (u32x2*)(p.y + b * p.ys0 + h * p.ys1 + s * p.ys2 + part * 8));
  }
}

}  // namespace
}  // namespace dt

extern "C" int dt_quantize_e4m3(const uint16_t* x, uint8_t* y, int B, int H,
                                int S, int D, const int64_t* x_strides,
                                const int64_t* y_strides, float factor,
                                void* stream) {
  using namespace dt;
  if (!x || !y || !x_strides || !y_strides)
    return set_error(DT_ERR_ARG, "dt_quantize_e4m3: null pointer argument");
  if (B <= 0 || H <= 0 || S <= 0 || D <= 0)
    return set_error(DT_ERR_SHAPE, "dt_quantize_e4m3: B=%d H=%d S=%d D=%d", B,
                     H, S, D);
  if (D % 8)
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_quantize_e4m3: head dim %d not a multiple of 8", D);
  if (!isfinite(factor))
    return set_error(DT_ERR_ARG, "dt_quantize_e4m3: factor not finite");
  for (int i = 0; i < 3; ++i)
    if (x_strides[i] % 8 || y_strides[i] % 8)
      return set_error(DT_ERR_UNSUPPORTED,
                       "dt_quantize_e4m3: strides must be multiples of 8");
  if ((int64_t)S * (D / 8) > 0x7fffffff || (int64_t)B * H > 65535)
    return set_error(DT_ERR_SHAPE, "dt_quantize_e4m3: tensor too large");
  if (((uintptr_t)x & 15u) || ((uintptr_t)y & 7u))
    return set_error(DT_ERR_UNSUPPORTED, "dt_quantize_e4m3: misaligned tensor");
  CastParams p;
  p.x = x;
  p.y = y;
  p.xs0 = x_strides[0];
  p.xs1 = x_strides[1];
  p.xs2 = x_strides[2];
  p.ys0 = y_strides[0];
  p.ys1 = y_strides[1];
  p.ys2 = y_strides[2];
  p.H = H;
  p.S = S;
  p.lanes_per_row = D / 8;
  p.factor = factor;
  // about 8192 blocks over the grid; each thread strides over its slice
  const int64_t want = ((int64_t)S * (D / 8) + 255) / 256;
  const int64_t cap = (8192 + (int64_t)B * H - 1) / ((int64_t)B * H);
  const int bx = (int)(want < cap ? want : cap);
  hipLaunchKernelGGL(e4m3_cast_kernel, dim3(bx, B * H), dim3(256), 0,
                     (hipStream_t)stream, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "dt_quantize_e4m3: %s",
                     hipGetErrorString(e));
  return DT_OK;
}
