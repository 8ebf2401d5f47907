// Key smoothing and the fixed-m operand (gfx950).
//
// dt_smooth_keys: k - mean_S(k) per (batch, head) and channel, the caller
// contract of the fixed-m softmax.  Replaces the reference's
//   k = k - jnp.mean(k, axis=2, keepdims=True)
// (kernels/mesh_attention.py:234-237, backends/ours_splash_tt.py:136-137)
// and its padded form, the mean over the real rows s < kv_len in float32,
// cast to the key dtype and subtracted, padded rows zeroed
// (models/minimax_h3/jax_server.py:271-289).  Softmax attention does not
// change; the per-head bound of the smoothed rows, which fixed-m needs,
// falls out of the same pass.
//
// dt_fixed_m_prepare: the whole fixed-m preparation of one call, the
// smoothing above (optional) plus the operand of
// kernels/fixed_m_bound.py:98-118 / kernels/splash.py:609-614,
// mk = (ceil(bound), bound <= gate) with bound = max|q| * factor * max|k|
// per head, in three launches instead of a dozen small ones.
//
// Launches, all deterministic (no floating-point atomics on the way to mk):
//   pass1_kernel   one read of k: per (b, h, row chunk) column sums in a
//                  fixed order (or, without smoothing, the chunk's largest
//                  row sum of squares); with a query, in the same grid, one
//                  read of q: each chunk's largest row sum of squares;
//   smooth_kernel  the block's mean from the chunk sums (in chunk order,
//                  rounded to bf16), a second read of k, bf16(k - mean)
//                  written (0 for rows at or past kv_len), and the block's
//                  largest row sum of squares of the written rows: into a
//                  per-block slot (dt_fixed_m_prepare) or max-accumulated
//                  as a norm per head (dt_smooth_keys; an atomic max on the
//                  bits of a non-negative float, order independent);
//   operand_kernel the per-head maxima over the slots, square roots, the
//                  bound, its ceiling and the gate flag.
// Row sums of squares use the lane arithmetic of row_norm_max_kernel (the
// same fused multiply-adds in the same order), so the operand equals the
// one built from dt_max_row_norm.
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
  int B, H, S, kv_end, nchunk, rows_per_chunk, rows_per_block, nblk;
  int smooth;      // 1: column sums + smoothing; 0: k row norms in pass 1
  // runtime key length in device memory, or null (kv_end); planned with
  // kv_end = S when given
  const int32_t* kv_len_dev;
  int kv_len_count;  // entries of kv_len_dev: <= 1 shared, else one per b
  float* partial;  // [B*H][nchunk][D] column sums (smooth)
  float* norms;    // [H] max-accumulated norms (dt_smooth_keys) or null
  float* kmax;     // [B*H][nblk] block maxima of row sums of squares or null
  // the query side of dt_fixed_m_prepare (q null: none)
  const uint16_t* q;
  int64_t q_sb, q_sh, q_ss;
  int Hq, Sq, q_nchunk, q_rows_per_chunk;
  float* qmax;     // [B*Hq][q_nchunk]
  // the operand
  float q_factor, gate;
  float* mk;       // [2][Hq]
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

// sum of squares of a lane's 8 bf16 values, in row_norm_max_kernel's order
__device__ __forceinline__ float sumsq8(const u32x4& raw) {
  float acc = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lo = __uint_as_float(raw[e] << 16);
    const float hi = __uint_as_float(raw[e] & 0xffff0000u);
    acc = __builtin_fmaf(lo, lo, acc);
    acc = __builtin_fmaf(hi, hi, acc);
  }
  return acc;
}

// the block's largest value of `v` (non-negative), in every thread
__device__ __forceinline__ float block_max(float v, float* s_max) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  __syncthreads();  // s_max may still be read from an earlier use
  if ((threadIdx.x & 63) == 0) s_max[threadIdx.x >> 6] = v;
  __syncthreads();
  float m = s_max[0];
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) m = fmaxf(m, s_max[w]);
  return m;
}

// largest row sum of squares over rows [s0, s1) of a [S][D] slice
template <int D>
__device__ float chunk_max_sumsq(const uint16_t* base, int64_t ss, int s0,
                                 int s1, float* s_max) {
  constexpr int LPR = D / 8, RPW = 64 / LPR, RPS = RPW * (kThreads / 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int part = lane % LPR;
  // eight loads in flight per lane (one at a time left this read-only pass
  // latency-bound), then the row sums
  constexpr int U = 8;
  float best = 0.f;
  for (int s = s0 + wave * RPW + lane / LPR; s < s1; s += U * RPS) {
    u32x4 raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      raw[u] = u32x4{0u, 0u, 0u, 0u};
      if (s + u * RPS < s1)
        raw[u] = __builtin_nontemporal_load(
            (const u32x4*)(base + (int64_t)(s + u * RPS) * ss + part * 8));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float acc = sumsq8(raw[u]);
      // every lane of a row group takes the same branches
#pragma unroll
      for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
      best = fmaxf(best, acc);  // rows past s1 add zero
    }
  }
  return block_max(best, s_max);
}

// blockIdx.z 0: the keys (column sums, or row norms without smoothing),
// 1: the query row norms.  x: row chunk, y: (b, head).
template <int D>
__global__ __launch_bounds__(kThreads) void pass1_kernel(SmoothParams p) {
  constexpr int LPR = D / 8, RPW = 64 / LPR, RPS = RPW * (kThreads / 64);
  __shared__ float s_acc[kThreads][9];  // padded against bank conflicts
  __shared__ float s_max[kThreads / 64];
  const int chunk = blockIdx.x, bh = blockIdx.y;
  if (blockIdx.z == 1) {  // query row norms
    if (bh >= p.B * p.Hq || chunk >= p.q_nchunk) return;
    const int b = bh / p.Hq, h = bh % p.Hq;
    const int s0 = chunk * p.q_rows_per_chunk;
    const int s1 = min(p.Sq, s0 + p.q_rows_per_chunk);
    const float m = chunk_max_sumsq<D>(p.q + b * p.q_sb + h * p.q_sh, p.q_ss,
                                       s0, s1, s_max);
    if (threadIdx.x == 0) p.qmax[(int64_t)bh * p.q_nchunk + chunk] = m;
    return;
  }
  if (bh >= p.B * p.H || chunk >= p.nchunk) return;
  const int b = bh / p.H, h = bh % p.H;
  const uint16_t* base = p.k + b * p.k_sb + h * p.k_sh;
  const int s0 = chunk * p.rows_per_chunk;
  if (!p.smooth) {  // key row norms over every row
    const int s1 = min(p.S, s0 + p.rows_per_chunk);
    const float m = chunk_max_sumsq<D>(base, p.k_ss, s0, s1, s_max);
    if (threadIdx.x == 0) p.kmax[(int64_t)bh * p.nblk + chunk] = m;
    return;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int part = lane % LPR;
  const int kv_end = resolve_len(p.kv_len_dev, p.kv_len_count, b, p.kv_end, p.S);
  const int s1 = min(kv_end, s0 + p.rows_per_chunk);
  // few, long chunks (the smoothing pass re-reads every chunk sum of its
  // slice): eight loads in flight per lane keep the HBM reads deep enough
  // (four: 4 % slower for dt_smooth_keys at V7; the lane still adds its
  // rows in row order, so the sums do not change)
  constexpr int U = 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s = s0 + wave * RPW + lane / LPR; s < s1; s += U * RPS) {
    u32x4 raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      raw[u] = u32x4{0u, 0u, 0u, 0u};
      if (s + u * RPS < s1)
        raw[u] = __builtin_nontemporal_load(
            (const u32x4*)(base + (int64_t)(s + u * RPS) * p.k_ss + part * 8));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float x[8];
      unpack8(raw[u], x);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += x[e];
    }
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
__global__ __launch_bounds__(kThreads) void smooth_kernel(SmoothParams p) {
  constexpr int LPR = D / 8, RPW = 64 / LPR, RPS = RPW * (kThreads / 64);
  __shared__ __attribute__((aligned(16))) float s_mean[D];
  __shared__ float s_max[kThreads / 64];
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  const int kv_end = resolve_len(p.kv_len_dev, p.kv_len_count, b, p.kv_end, p.S);
  // this (b, h)'s mean from the chunk sums, in chunk order, rounded to bf16
  if (threadIdx.x < D) {
    const float* src = p.partial + (int64_t)bh * p.nchunk * D + threadIdx.x;
    // in chunk order, eight loads in flight (a load at a time left every
    // block waiting out up to 64 round trips before its first row)
    float sum = 0.f;
    int i = 0;
    for (; i + 8 <= p.nchunk; i += 8) {
      float t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = src[(int64_t)(i + u) * D];
#pragma unroll
      for (int u = 0; u < 8; ++u) sum += t[u];
    }
    for (; i < p.nchunk; ++i) sum += src[(int64_t)i * D];
    // no real rows (a device length of 0): every row comes out zero
    s_mean[threadIdx.x] = kv_end > 0
        ? __uint_as_float(bf16_round_bits(sum / (float)kv_end) << 16)
        : 0.f;
  }
  __syncthreads();
  const uint16_t* src = p.k + b * p.k_sb + h * p.k_sh;
  uint16_t* dst = p.ks + b * p.ks_sb + h * p.ks_sh;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int part = lane % LPR;
  float mu[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) mu[e] = s_mean[part * 8 + e];
  const int s0 = blockIdx.x * p.rows_per_block;
  const int s1 = min(p.S, s0 + p.rows_per_block);
  float best = 0.f;
  // eight rows per lane in flight: all loads first, then the arithmetic
  constexpr int U = 8;
  for (int s = s0 + wave * RPW + lane / LPR; s < s1; s += U * RPS) {
    u32x4 raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = s + u * RPS;
      raw[u] = u32x4{0u, 0u, 0u, 0u};
      if (r < s1 && r < kv_end)
        raw[u] = __builtin_nontemporal_load(
            (const u32x4*)(src + (int64_t)r * p.k_ss + part * 8));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = s + u * RPS;
      if (r >= s1) break;  // the same for every lane of a row group
      u32x4 out = {0u, 0u, 0u, 0u};
      if (r < kv_end) {
        float x[8];
        unpack8(raw[u], x);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = bf16_round_bits(x[2 * e] - mu[2 * e]);
          const uint32_t hi = bf16_round_bits(x[2 * e + 1] - mu[2 * e + 1]);
          out[e] = lo | (hi << 16);
        }
      }
      __builtin_nontemporal_store(out, (u32x4*)(dst + (int64_t)r * p.ks_ss + part * 8));
      float ss = sumsq8(out);
#pragma unroll
      for (int off = LPR / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
      best = fmaxf(best, ss);
    }
  }
  if (p.norms == nullptr && p.kmax == nullptr) return;
  const float m = block_max(best, s_max);
  if (threadIdx.x == 0) {
    if (p.kmax != nullptr) p.kmax[(int64_t)bh * p.nblk + blockIdx.x] = m;
    if (p.norms != nullptr)
      atomicMax((unsigned int*)(p.norms + h), __float_as_uint(sqrtf(m)));
  }
}

// one block per query head h: mk[0][h] = ceil(bound), mk[1][h] =
// bound <= gate, with bound = sqrt(max q row sum of squares) * q_factor *
// sqrt(max k ...) over the batch; query head h reads kv head h / (Hq / H).
// The block's threads reduce the slots in parallel (max is order free).
__global__ __launch_bounds__(kThreads) void operand_kernel(SmoothParams p, int B) {
  __shared__ float s_max[kThreads / 64];
  const int h = blockIdx.x;
  const int hk = h / (p.Hq / p.H);
  float qm = 0.f, km = 0.f;
  for (int i = threadIdx.x; i < B * p.q_nchunk; i += kThreads) {
    const int b = i / p.q_nchunk, c = i - b * p.q_nchunk;
    qm = fmaxf(qm, p.qmax[((int64_t)b * p.Hq + h) * p.q_nchunk + c]);
  }
  for (int i = threadIdx.x; i < B * p.nblk; i += kThreads) {
    const int b = i / p.nblk, c = i - b * p.nblk;
    km = fmaxf(km, p.kmax[((int64_t)b * p.H + hk) * p.nblk + c]);
  }
  qm = block_max(qm, s_max);
  km = block_max(km, s_max);
  if (threadIdx.x == 0) {
    const float bound = (sqrtf(qm) * p.q_factor) * sqrtf(km);
    p.mk[h] = ceilf(bound);
    p.mk[p.Hq + h] = bound <= p.gate ? 1.f : 0.f;
  }
}

// Chunking: about 1024 blocks over a tensor's (b, head) slices, whole load
// steps per chunk; the smoothing pass: about 2048 blocks.
struct Chunks {
  int n, rows;
};

Chunks chunk_rows(int64_t bh, int D, int rows_total, int blocks,
                  int max_per_slice = 1 << 30) {
  const int rps = (64 / (D / 8)) * (kThreads / 64);
  int64_t n = (blocks + bh - 1) / bh;
  if (n > max_per_slice) n = max_per_slice;
  const int64_t max_chunks = (rows_total + rps - 1) / rps;
  if (n > max_chunks) n = max_chunks;
  if (n < 1) n = 1;
  int64_t rows = (rows_total + n - 1) / n;
  rows = (rows + rps - 1) / rps * rps;
  n = (rows_total + rows - 1) / rows;
  return Chunks{(int)n, (int)rows};
}

struct SmoothPlan {
  Chunks k, q, blk;
  size_t partial_floats, kmax_floats, qmax_floats;
  size_t ws_bytes() const {
    return (partial_floats + kmax_floats + qmax_floats) * sizeof(float);
  }
};

// smooth: k chunks over the real rows, blk over all rows for the
// smoothing pass; without smoothing, k chunks over all rows (their maxima
// are the k slots).  with_q: the query side too.
SmoothPlan smooth_plan(int B, int H, int Hq, int S, int Sq, int D, int kv_end,
                       bool smooth, bool with_q, bool with_kmax) {
  SmoothPlan sp{};
  const int64_t bh = (int64_t)B * H;
  // column-sum chunks: at most 64 per slice, since every block of the
  // smoothing pass sums its slice's chunk sums
  sp.k = smooth ? chunk_rows(bh, D, kv_end, 1024, 64) : chunk_rows(bh, D, S, 1024);
  sp.blk = chunk_rows(bh, D, S, 2048);
  if (with_q) sp.q = chunk_rows((int64_t)B * Hq, D, Sq, 1024);
  sp.partial_floats = smooth ? (size_t)bh * sp.k.n * D : 0;
  sp.kmax_floats =
      with_kmax ? (size_t)bh * (smooth ? sp.blk.n : sp.k.n) : 0;
  sp.qmax_floats = with_q ? (size_t)B * Hq * sp.q.n : 0;
  return sp;
}

int check_tensor(const char* who, const void* t, const int64_t* strides) {
  if (!t || !strides) return set_error(DT_ERR_ARG, "%s: null pointer argument", who);
  for (int i = 0; i < 3; ++i)
    if (strides[i] % 8)
      return set_error(DT_ERR_UNSUPPORTED,
                       "%s: strides must be multiples of 8 elements", who);
  if ((uintptr_t)t & 15u)
    return set_error(DT_ERR_UNSUPPORTED, "%s: misaligned pointer", who);
  return DT_OK;
}

int launch_smooth(SmoothParams& p, const SmoothPlan& sp, int B, int D,
                  bool with_q, hipStream_t st) {
  const int gy = (int)(with_q && (int64_t)B * p.Hq > (int64_t)B * p.H
                           ? (int64_t)B * p.Hq
                           : (int64_t)B * p.H);
  const int gx = with_q && sp.q.n > sp.k.n ? sp.q.n : sp.k.n;
  const dim3 g1(gx, gy, with_q ? 2 : 1);
  if (D == 256)
    hipLaunchKernelGGL(pass1_kernel<256>, g1, dim3(kThreads), 0, st, p);
  else if (D == 128)
    hipLaunchKernelGGL(pass1_kernel<128>, g1, dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL(pass1_kernel<64>, g1, dim3(kThreads), 0, st, p);
  if (p.smooth) {
    const dim3 g2(sp.blk.n, B * p.H);
    if (D == 256)
      hipLaunchKernelGGL(smooth_kernel<256>, g2, dim3(kThreads), 0, st, p);
    else if (D == 128)
      hipLaunchKernelGGL(smooth_kernel<128>, g2, dim3(kThreads), 0, st, p);
    else
      hipLaunchKernelGGL(smooth_kernel<64>, g2, dim3(kThreads), 0, st, p);
  }
  return DT_OK;
}

}  // namespace
}  // namespace dt

extern "C" size_t dt_smooth_keys_workspace_bytes(int B, int H, int S, int D,
                                                 int kv_len) {
  if (B <= 0 || H <= 0 || S <= 0 || (D != 64 && D != 128 && D != 256)) return 0;
  const int kv_end = (kv_len <= 0 || kv_len > S) ? S : kv_len;
  return dt::smooth_plan(B, H, H, S, S, D, kv_end, true, false, false)
      .ws_bytes();
}

extern "C" int dt_smooth_keys(const uint16_t* k, uint16_t* ks, int B, int H,
                              int S, int D, const int64_t* k_strides,
                              const int64_t* ks_strides, int kv_len,
                              const int32_t* kv_len_dev, float* norms,
                              void* workspace, size_t workspace_bytes,
                              void* stream) {
  using namespace dt;
  if (int rc = check_tensor("dt_smooth_keys", k, k_strides)) return rc;
  if (int rc = check_tensor("dt_smooth_keys", ks, ks_strides)) return rc;
  if (!workspace) return set_error(DT_ERR_ARG, "dt_smooth_keys: null workspace");
  if (B <= 0 || H <= 0 || S <= 0)
    return set_error(DT_ERR_SHAPE, "dt_smooth_keys: B=%d H=%d S=%d", B, H, S);
  if (D != 64 && D != 128 && D != 256)
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_smooth_keys: head dim %d (supported: 64, 128, 256)", D);
  // a length in device memory: kv_len is its entry count
  int kv_len_count = 0;
  if (int rc = dev_len_count(kv_len_dev, kv_len, B, "dt_smooth_keys",
                             &kv_len_count))
    return rc;
  if (kv_len_dev != nullptr) kv_len = 0;
  if (kv_len > S)
    return set_error(DT_ERR_SHAPE, "dt_smooth_keys: kv_len %d > S %d", kv_len, S);
  if ((uintptr_t)workspace & 15u)
    return set_error(DT_ERR_UNSUPPORTED, "dt_smooth_keys: misaligned workspace");
  if ((int64_t)B * H > 65535)
    return set_error(DT_ERR_SHAPE, "dt_smooth_keys: B*H too large");
  // a length in device memory: chunks planned over every row
  const int kv_end = (kv_len > 0 && kv_len_dev == nullptr) ? kv_len : S;
  const SmoothPlan sp = smooth_plan(B, H, H, S, S, D, kv_end, true, false, false);
  if (workspace_bytes < sp.ws_bytes())
    return set_error(DT_ERR_ARG,
                     "dt_smooth_keys: workspace of %zu bytes, %zu needed",
                     workspace_bytes, sp.ws_bytes());
  SmoothParams p{};
  p.k = k;
  p.ks = ks;
  p.k_sb = k_strides[0];
  p.k_sh = k_strides[1];
  p.k_ss = k_strides[2];
  p.ks_sb = ks_strides[0];
  p.ks_sh = ks_strides[1];
  p.ks_ss = ks_strides[2];
  p.B = B;
  p.H = H;
  p.Hq = H;
  p.S = S;
  p.kv_end = kv_end;
  p.kv_len_dev = kv_len_dev;
  p.kv_len_count = kv_len_count;
  p.smooth = 1;
  p.nchunk = sp.k.n;
  p.rows_per_chunk = sp.k.rows;
  p.rows_per_block = sp.blk.rows;
  p.nblk = sp.blk.n;
  p.partial = (float*)workspace;
  p.norms = norms;
  p.kmax = nullptr;
  p.q = nullptr;
  launch_smooth(p, sp, B, D, false, (hipStream_t)stream);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "dt_smooth_keys: %s", hipGetErrorString(e));
  return DT_OK;
}

extern "C" size_t dt_fixed_m_prepare_workspace_bytes(int B, int Hq, int Hkv,
                                                     int Sq, int Skv, int D,
                                                     int kv_len, int smooth) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Sq <= 0 || Skv <= 0 ||
      (D != 64 && D != 128 && D != 256))
    return 0;
  const int kv_end = (kv_len <= 0 || kv_len > Skv) ? Skv : kv_len;
  return dt::smooth_plan(B, Hkv, Hq, Skv, Sq, D, kv_end, smooth != 0, true,
                         true)
      .ws_bytes();
}

extern "C" int dt_fixed_m_prepare(
    const uint16_t* q, const uint16_t* k, uint16_t* ks, int B, int Hq,
    int Hkv, int Sq, int Skv, int D, const int64_t* q_strides,
    const int64_t* k_strides, const int64_t* ks_strides, int kv_len,
    const int32_t* kv_len_dev, float q_factor, float gate, int smooth,
    float* mk, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace dt;
  const char* who = "dt_fixed_m_prepare";
  if (int rc = check_tensor(who, q, q_strides)) return rc;
  if (int rc = check_tensor(who, k, k_strides)) return rc;
  if (smooth)
    if (int rc = check_tensor(who, ks, ks_strides)) return rc;
  if (!mk || !workspace) return set_error(DT_ERR_ARG, "%s: null mk or workspace", who);
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Sq <= 0 || Skv <= 0)
    return set_error(DT_ERR_SHAPE, "%s: B=%d Hq=%d Hkv=%d Sq=%d Skv=%d", who, B,
                     Hq, Hkv, Sq, Skv);
  if (Hq % Hkv)
    return set_error(DT_ERR_SHAPE, "%s: Hq %d not a multiple of Hkv %d", who, Hq,
                     Hkv);
  if (D != 64 && D != 128 && D != 256)
    return set_error(DT_ERR_UNSUPPORTED, "%s: head dim %d (supported: 64, 128, 256)",
                     who, D);
  int kv_len_count = 0;
  if (int rc = dev_len_count(kv_len_dev, kv_len, B, who, &kv_len_count))
    return rc;
  if (kv_len_dev != nullptr) kv_len = 0;
  if (kv_len > Skv)
    return set_error(DT_ERR_SHAPE, "%s: kv_len %d > Skv %d", who, kv_len, Skv);
  if (!(q_factor > 0.f) || !isfinite(q_factor) || isnan(gate))
    return set_error(DT_ERR_ARG, "%s: q_factor %g, gate %g", who,
                     (double)q_factor, (double)gate);
  if ((uintptr_t)workspace & 15u)
    return set_error(DT_ERR_UNSUPPORTED, "%s: misaligned workspace", who);
  if ((int64_t)B * (Hq > Hkv ? Hq : Hkv) > 65535)
    return set_error(DT_ERR_SHAPE, "%s: B*heads too large", who);
  const int kv_end = (kv_len > 0 && kv_len_dev == nullptr) ? kv_len : Skv;
  const SmoothPlan sp =
      smooth_plan(B, Hkv, Hq, Skv, Sq, D, kv_end, smooth != 0, true, true);
  if (workspace_bytes < sp.ws_bytes())
    return set_error(DT_ERR_ARG, "%s: workspace of %zu bytes, %zu needed", who,
                     workspace_bytes, sp.ws_bytes());
  SmoothParams p{};
  p.k = k;
  p.ks = ks;
  p.k_sb = k_strides[0];
  p.k_sh = k_strides[1];
  p.k_ss = k_strides[2];
  if (smooth) {
    p.ks_sb = ks_strides[0];
    p.ks_sh = ks_strides[1];
    p.ks_ss = ks_strides[2];
  }
  p.B = B;
  p.H = Hkv;
  p.S = Skv;
  p.kv_end = kv_end;
  p.kv_len_dev = kv_len_dev;
  p.kv_len_count = kv_len_count;
  p.smooth = smooth ? 1 : 0;
  p.nchunk = sp.k.n;
  p.rows_per_chunk = sp.k.rows;
  p.rows_per_block = sp.blk.rows;
  p.nblk = smooth ? sp.blk.n : sp.k.n;
  p.partial = (float*)workspace;
  p.kmax = p.partial + sp.partial_floats;
  p.qmax = p.kmax + sp.kmax_floats;
  p.norms = nullptr;
  p.q = q;
  p.q_sb = q_strides[0];
  p.q_sh = q_strides[1];
  p.q_ss = q_strides[2];
  p.Hq = Hq;
  p.Sq = Sq;
  p.q_nchunk = sp.q.n;
  p.q_rows_per_chunk = sp.q.rows;
  p.q_factor = q_factor;
  p.gate = gate;
  p.mk = mk;
  hipStream_t st = (hipStream_t)stream;
  launch_smooth(p, sp, B, D, true, st);
  hipLaunchKernelGGL(operand_kernel, dim3(Hq), dim3(kThreads), 0, st, p, B);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
  return DT_OK;
}
