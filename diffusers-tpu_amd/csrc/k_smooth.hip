// Key smoothing (gfx950): k - mean_S(k) per (batch, head) and channel, the
// caller contract of the fixed-m softmax.  Replaces the reference's
//   k = k - jnp.mean(k, axis=2, keepdims=True)
// (kernels/mesh_attention.py:234-237, backends/ours_splash_tt.py:136-137)
// and its padded form, the mean over the real rows s < kv_len in float32,
// cast to the key dtype and subtracted, padded rows zeroed
// (models/minimax_h3/jax_server.py:271-289).  Softmax attention does not
// change; the per-head bound of the smoothed rows, which fixed-m needs,
// falls out of the same pass.
//
// Three launches, deterministic (no floating-point atomics):
//   col_sum_kernel  one read of k: per (b, h, row chunk) column sums, in a
//                   fixed order, into the workspace;
//   col_mean_kernel the chunk sums in chunk order -> mean, rounded to bf16;
//   smooth_kernel   a second read of k: bf16(k - mean) (0 for rows at or
//                   past kv_len) written out, and the largest L2 norm of the
//                   written rows max-accumulated per head into norms[h]
//                   (atomic max on the bits of a non-negative float, which
//                   is order independent).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/dt_attention.h"
#include "dt_common.h"

namespace dt {
namespace {

constexpr int kThreads = 256;

struct SmoothParams {
  const uint16_t* k;
  uint16_t* ks;
  int64_t k_sb, k_sh, k_ss, ks_sb, ks_sh, ks_ss;
  int H, S, kv_end, nchunk, rows_per_chunk, rows_per_block;
  float* partial;  // [B*H][nchunk][D]
  float* mean;     // [B*H][D], bf16-rounded values
  float* norms;    // [H] or null
};

__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(v[i] << 16);
    f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ uint32_t bf16_round_bits(float x) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 r = {(__bf16)x, (__bf16)0.f};
  return *reinterpret_cast<uint32_t*>(&r) & 0xffffu;
}

template <int D>
__global__ __launch_bounds__(kThreads) void col_sum_kernel(SmoothParams p) {
  constexpr int LPR = D / 8, RPW = 64 / LPR, RPS = RPW * (kThreads / 64);
  __shared__ float s_acc[kThreads][9];  // padded against bank conflicts
  const int bh = blockIdx.y, chunk = blockIdx.x;
  const int b = bh / p.H, h = bh % p.H;
  const uint16_t* base = p.k + b * p.k_sb + h * p.k_sh;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int part = lane % LPR;
  const int s0 = chunk * p.rows_per_chunk;
  const int s1 = min(p.kv_end, s0 + p.rows_per_chunk);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s = s0 + wave * RPW + lane / LPR; s < s1; s += RPS) {
    float x[8];
    unpack8(__builtin_nontemporal_load(
                (const u32x4*)(base + (int64_t)s * p.k_ss + part * 8)),
            x);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += x[e];
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) s_acc[threadIdx.x][e] = acc[e];
  __syncthreads();
  if (threadIdx.x < D) {
    const int c = threadIdx.x, cp = c / 8, ce = c % 8;
    float sum = 0.f;
    for (int t = cp; t < kThreads; t += LPR) sum += s_acc[t][ce];
    p.partial[((int64_t)bh * p.nchunk + chunk) * D + c] = sum;
  }
}

template <int D>
__global__ __launch_bounds__(D) void col_mean_kernel(SmoothParams p) {
  const int bh = blockIdx.x, c = threadIdx.x;
  const float* src = p.partial + (int64_t)bh * p.nchunk * D + c;
  float sum = 0.f;
  for (int i = 0; i < p.nchunk; ++i) sum += src[(int64_t)i * D];
  const float mean = sum / (float)p.kv_end;
  p.mean[(int64_t)bh * D + c] = __uint_as_float(bf16_round_bits(mean) << 16);
}

template <int D>
__global__ __launch_bounds__(kThreads) void smooth_kernel(SmoothParams p) {
  constexpr int LPR = D / 8, RPW = 64 / LPR, RPS = RPW * (kThreads / 64);
  __shared__ float s_max[kThreads / 64];
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  const uint16_t* src = p.k + b * p.k_sb + h * p.k_sh;
  uint16_t* dst = p.ks + b * p.ks_sb + h * p.ks_sh;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int part = lane % LPR;
  float mu[8];
  {
    const f32x4* m4 = (const f32x4*)(p.mean + (int64_t)bh * D + part * 8);
    const f32x4 a = m4[0], c = m4[1];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      mu[e] = a[e];
      mu[4 + e] = c[e];
    }
  }
  const int s0 = blockIdx.x * p.rows_per_block;
  const int s1 = min(p.S, s0 + p.rows_per_block);
  float best = 0.f;
  for (int s = s0 + wave * RPW + lane / LPR; s < s1; s += RPS) {
    u32x4 out = {0u, 0u, 0u, 0u};
    float ss = 0.f;
    if (s < p.kv_end) {
      float x[8];
      unpack8(__builtin_nontemporal_load(
                  (const u32x4*)(src + (int64_t)s * p.k_ss + part * 8)),
              x);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t lo = bf16_round_bits(x[2 * e] - mu[2 * e]);
        const uint32_t hi = bf16_round_bits(x[2 * e + 1] - mu[2 * e + 1]);
        out[e] = lo | (hi << 16);
        const float flo = __uint_as_float(lo << 16);
        const float fhi = __uint_as_float(hi << 16);
        ss = __builtin_fmaf(flo, flo, ss);
        ss = __builtin_fmaf(fhi, fhi, ss);
      }
    }
    __builtin_nontemporal_store(out, (u32x4*)(dst + (int64_t)s * p.ks_ss + part * 8));
    // every lane of a row group takes the same branches
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    best = fmaxf(best, ss);
  }
  if (p.norms == nullptr) return;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
    best = fmaxf(best, __shfl_xor(best, off, 64));
  if (lane == 0) s_max[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    float m = s_max[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) m = fmaxf(m, s_max[w]);
    atomicMax((unsigned int*)(p.norms + h), __float_as_uint(sqrtf(m)));
  }
}

// chunking of the column sums: about 1024 blocks over the grid, whole load
// steps per chunk
struct SmoothPlan {
  int nchunk, rows_per_chunk;
  size_t ws_bytes;
};

SmoothPlan smooth_plan(int B, int H, int D, int kv_end) {
  const int rps = (64 / (D / 8)) * (kThreads / 64);
  const int64_t bh = (int64_t)B * H;
  int64_t nchunk = (1024 + bh - 1) / bh;
  const int64_t max_chunks = (kv_end + rps - 1) / rps;
  if (nchunk > max_chunks) nchunk = max_chunks;
  if (nchunk < 1) nchunk = 1;
  int64_t rows = (kv_end + nchunk - 1) / nchunk;
  rows = (rows + rps - 1) / rps * rps;
  nchunk = (kv_end + rows - 1) / rows;
  SmoothPlan sp;
  sp.nchunk = (int)nchunk;
  sp.rows_per_chunk = (int)rows;
  sp.ws_bytes = (size_t)(bh * nchunk * D + bh * D) * sizeof(float);
  return sp;
}

}  // namespace
}  // namespace dt

extern "C" size_t dt_smooth_keys_workspace_bytes(int B, int H, int S, int D,
                                                 int kv_len) {
  if (B <= 0 || H <= 0 || S <= 0 || (D != 64 && D != 128)) return 0;
  const int kv_end = (kv_len <= 0 || kv_len > S) ? S : kv_len;
  return dt::smooth_plan(B, H, D, kv_end).ws_bytes;
}

extern "C" int dt_smooth_keys(const uint16_t* k, uint16_t* ks, int B, int H,
                              int S, int D, const int64_t* k_strides,
                              const int64_t* ks_strides, int kv_len,
                              float* norms, void* workspace,
                              size_t workspace_bytes, void* stream) {
  using namespace dt;
  if (!k || !ks || !k_strides || !ks_strides || !workspace)
    return set_error(DT_ERR_ARG, "dt_smooth_keys: null pointer argument");
  if (B <= 0 || H <= 0 || S <= 0)
    return set_error(DT_ERR_SHAPE, "dt_smooth_keys: B=%d H=%d S=%d", B, H, S);
  if (D != 64 && D != 128)
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_smooth_keys: head dim %d (supported: 64, 128)", D);
  if (kv_len > S)
    return set_error(DT_ERR_SHAPE, "dt_smooth_keys: kv_len %d > S %d", kv_len, S);
  for (int i = 0; i < 3; ++i)
    if (k_strides[i] % 8 || ks_strides[i] % 8)
      return set_error(DT_ERR_UNSUPPORTED,
                       "dt_smooth_keys: strides must be multiples of 8 elements");
  if (((uintptr_t)k & 15u) || ((uintptr_t)ks & 15u) ||
      ((uintptr_t)workspace & 15u))
    return set_error(DT_ERR_UNSUPPORTED, "dt_smooth_keys: misaligned pointer");
  if ((int64_t)B * H > 65535)
    return set_error(DT_ERR_SHAPE, "dt_smooth_keys: B*H too large");
  const int kv_end = kv_len > 0 ? kv_len : S;
  const SmoothPlan sp = smooth_plan(B, H, D, kv_end);
  if (workspace_bytes < sp.ws_bytes)
    return set_error(DT_ERR_ARG,
                     "dt_smooth_keys: workspace of %zu bytes, %zu needed",
                     workspace_bytes, sp.ws_bytes);
  SmoothParams p;
  p.k = k;
  p.ks = ks;
  p.k_sb = k_strides[0];
  p.k_sh = k_strides[1];
  p.k_ss = k_strides[2];
  p.ks_sb = ks_strides[0];
  p.ks_sh = ks_strides[1];
  p.ks_ss = ks_strides[2];
  p.H = H;
  p.S = S;
  p.kv_end = kv_end;
  p.nchunk = sp.nchunk;
  p.rows_per_chunk = sp.rows_per_chunk;
  p.partial = (float*)workspace;
  p.mean = p.partial + (int64_t)B * H * sp.nchunk * D;
  p.norms = norms;
  // smoothing pass: about 2048 blocks, whole load steps per block
  const int rps = (64 / (D / 8)) * (kThreads / 64);
  const int per_slice = (2048 + B * H - 1) / (B * H);
  int rows = (S + per_slice - 1) / per_slice;
  rows = (rows + 4 * rps - 1) / (4 * rps) * (4 * rps);
  p.rows_per_block = rows;
  const int nblk = (S + rows - 1) / rows;
  hipStream_t st = (hipStream_t)stream;
  const dim3 g1(sp.nchunk, B * H), g3(nblk, B * H);
  if (D == 128) {
    hipLaunchKernelGGL(col_sum_kernel<128>, g1, dim3(kThreads), 0, st, p);
    hipLaunchKernelGGL(col_mean_kernel<128>, dim3(B * H), dim3(128), 0, st, p);
    hipLaunchKernelGGL(smooth_kernel<128>, g3, dim3(kThreads), 0, st, p);
  } else {
    hipLaunchKernelGGL(col_sum_kernel<64>, g1, dim3(kThreads), 0, st, p);
    hipLaunchKernelGGL(col_mean_kernel<64>, dim3(B * H), dim3(64), 0, st, p);
    hipLaunchKernelGGL(smooth_kernel<64>, g3, dim3(kThreads), 0, st, p);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "dt_smooth_keys: %s", hipGetErrorString(e));
  return DT_OK;
}
