// Fused QK-RMSNorm + RoPE prologue for gfx950.
//
// Replaces the per-layer q/k prologue of the reference's DiT attention
// blocks: RMSNorm models/minimax_h3/jax_dit.py:191-195 (applied :362-363),
// RoPE apply_rope :251-262 with tables rope_angles :603-617 (applied
// :365-366), padded-row zeroing :367-381; Qwen interleaved-pair RoPE
// models/qwen_image_21/jax_dit.py:214-220.
//
// HBM-bound: per (token, head) row it reads D bf16 and writes D bf16, for q
// and for k.  Layout of the work:
//   * one wavefront owns one token at a time (grid-stride over B*S tokens)
//     and walks all 2*H rows of that token (H q-heads, then H k-heads);
//   * a row of D channels is covered by LPR = D/16 lanes, each holding two
//     8-channel chunks (two 16-byte loads), so a wavefront covers 64/LPR rows
//     per step and each 16-byte access is naturally aligned;
//   * the chunks a lane holds are chosen so every rotation pair sits inside
//     one lane: rotate-half pairs chunk c with chunk c + rotary/16, the
//     interleaved form keeps (2j, 2j+1) inside a chunk, pass-through chunks
//     are handed out two per lane after the rotating ones;
//   * the RMS reduction is a butterfly over the LPR lanes of a row
//     (__shfl_xor within a 16-lane group);
//   * the 8 rotation angles a lane needs depend only on the token, so their
//     cos/sin are computed once per token and reused by all 2*H rows.
//     Angles are carried in revolutions (frequency / 2pi) and reduced to
//     [0, 1) before the hardware sin/cos, which take revolutions.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/dt_attention.h"
#include "dt_common.h"

namespace dt {

struct NormRopeParams {
  const uint16_t* q;
  const uint16_t* k;
  uint16_t* qo;
  uint16_t* ko;
  const float* wq;
  const float* wk;
  const float* head_scale;
  const int32_t* pos;
  int64_t in_sb, in_ss, in_sh;
  int64_t out_sb, out_ss, out_sh;
  int B, S, H;
  float eps;
  int valid_len;
  int mode;
  int rot;  // rotated channels (even, <= D)
  // Per rotation pair j < rot/2: frequency in revolutions per position unit
  // and the position axis it reads.
  float freq_rev[64];
  int8_t pair_axis[64];
};

template <int D>
struct Layout {
  static constexpr int LPR = D / 16;          // lanes per row
  static constexpr int ROWS = 64 / LPR;       // rows per wavefront step
  static constexpr int CHUNKS = D / 8;        // 8-channel chunks per row
};

// Chunk indices (in units of 8 channels) owned by lane `li` of a row.
template <int D>
__device__ __forceinline__ void lane_chunks(int li, int mode, int rot, int& c0,
                                            int& c1) {
  if (mode == DT_ROPE_HALF) {
    const int hc = rot / 16;  // rotating chunks in the first half
    if (li < hc) {
      c0 = li;
      c1 = li + hc;
    } else {
      const int kk = li - hc;
      c0 = rot / 8 + 2 * kk;
      c1 = c0 + 1;
    }
  } else {
    c0 = 2 * li;
    c1 = 2 * li + 1;
  }
}

__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(v[i] << 16);
    f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ uint32_t f32_to_bf16_rne(float x) {
  uint32_t u = __float_as_uint(x);
  // NaN stays NaN (quiet bit set); finite values round to nearest even.
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    r[i] = f32_to_bf16_rne(f[2 * i]) | (f32_to_bf16_rne(f[2 * i + 1]) << 16);
  return r;
}

template <int D>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(NormRopeParams p) {
  using L = Layout<D>;
  const int lane = threadIdx.x & 63;
  const int li = lane % L::LPR;   // lane within row
  const int grp = lane / L::LPR;  // row group within wavefront
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int nwaves = (gridDim.x * blockDim.x) >> 6;

  int c0, c1;
  lane_chunks<D>(li, p.mode, p.rot, c0, c1);

  // Channel-resident RMSNorm weights for this lane's 16 channels.
  float wq[16], wk[16];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    wq[i] = p.wq[c0 * 8 + i];
    wq[8 + i] = p.wq[c1 * 8 + i];
    wk[i] = p.wk[c0 * 8 + i];
    wk[8 + i] = p.wk[c1 * 8 + i];
  }

  // Rotation pairs of this lane: pair index per slot, -1 = pass-through.
  // HALF: slot i pairs element i (chunk c0) with element 8+i (chunk c1).
  // PAIR: slot i pairs elements (2i, 2i+1) of the 16 (c0 then c1).
  int pj[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (p.mode == DT_ROPE_HALF) {
      const int ch = c0 * 8 + i;
      pj[i] = (ch < p.rot / 2) ? ch : -1;
    } else if (p.mode == DT_ROPE_PAIR) {
      const int ch = (i < 4 ? c0 * 8 + 2 * i : c1 * 8 + 2 * (i - 4));
      pj[i] = (ch < p.rot) ? ch / 2 : -1;
    } else {
      pj[i] = -1;
    }
  }

  const int64_t ntok = (int64_t)p.B * p.S;
  const int rows = 2 * p.H;
  for (int64_t tok = wave; tok < ntok; tok += nwaves) {
    const int b = (int)(tok / p.S);
    const int s = (int)(tok - (int64_t)b * p.S);
    const bool zero = (p.valid_len >= 0) && (s >= p.valid_len);

    float cs[8], sn[8];
    if (!zero) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        cs[i] = 1.0f;
        sn[i] = 0.0f;
        if (pj[i] >= 0) {
          const int j = pj[i];
          const float pos = (float)p.pos[s * 3 + p.pair_axis[j]];
          float rev = pos * p.freq_rev[j];
          rev = rev - floorf(rev);
          sn[i] = __builtin_amdgcn_sinf(rev);
          cs[i] = __builtin_amdgcn_cosf(rev);
        }
      }
    }

    for (int r = grp; r < rows; r += L::ROWS) {
      const bool isk = r >= p.H;
      const int h = isk ? r - p.H : r;
      uint16_t* dst = (isk ? p.ko : p.qo) + b * p.out_sb + s * p.out_ss +
                      h * p.out_sh;
      if (zero) {
        const u32x4 z = {0u, 0u, 0u, 0u};
        *(u32x4*)(dst + c0 * 8) = z;
        *(u32x4*)(dst + c1 * 8) = z;
        continue;
      }
      const uint16_t* src =
          (isk ? p.k : p.q) + b * p.in_sb + s * p.in_ss + h * p.in_sh;
      const u32x4 v0 = *(const u32x4*)(src + c0 * 8);
      const u32x4 v1 = *(const u32x4*)(src + c1 * 8);
      float x[16];
      unpack8(v0, x);
      unpack8(v1, x + 8);
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) ss += x[i] * x[i];
#pragma unroll
      for (int off = 1; off < L::LPR; off <<= 1) ss += __shfl_xor(ss, off, 64);
      const float rr = rsqrtf(ss * (1.0f / D) + p.eps);
      const float* w = isk ? wk : wq;
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = x[i] * rr * w[i];
      if (p.mode == DT_ROPE_HALF) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float a = x[i], bb = x[8 + i];
          x[i] = a * cs[i] - bb * sn[i];
          x[8 + i] = bb * cs[i] + a * sn[i];
        }
      } else if (p.mode == DT_ROPE_PAIR) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float a = x[2 * i], bb = x[2 * i + 1];
          x[2 * i] = a * cs[i] - bb * sn[i];
          x[2 * i + 1] = a * sn[i] + bb * cs[i];
        }
      }
      if (!isk && p.head_scale != nullptr) {
        const float f = p.head_scale[h];
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] *= f;
      }
      *(u32x4*)(dst + c0 * 8) = pack8(x);
      *(u32x4*)(dst + c1 * 8) = pack8(x + 8);
    }
  }
}

static bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace dt

extern "C" int dt_qk_norm_rope(const uint16_t* q, const uint16_t* k,
                               uint16_t* q_out, uint16_t* k_out, int B, int S,
                               int H, int D, const int64_t* in_strides,
                               const int64_t* out_strides, const float* wq,
                               const float* wk, float eps,
                               const float* q_head_scale, int mode,
                               const int32_t* pos, const int32_t* axis_dims,
                               float theta, int valid_len, void* stream) {
  using namespace dt;
  if (!q || !k || !q_out || !k_out || !wq || !wk || !in_strides ||
      !out_strides)
    return set_error(DT_ERR_ARG, "dt_qk_norm_rope: null pointer argument");
  if (B <= 0 || S <= 0 || H <= 0)
    return set_error(DT_ERR_SHAPE, "dt_qk_norm_rope: B=%d S=%d H=%d", B, S, H);
  if (D != 64 && D != 128)
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_qk_norm_rope: head dim %d (supported: 64, 128)", D);
  if (mode < DT_ROPE_NONE || mode > DT_ROPE_PAIR)
    return set_error(DT_ERR_ARG, "dt_qk_norm_rope: rope mode %d", mode);
  if (!(eps >= 0.f)) return set_error(DT_ERR_ARG, "dt_qk_norm_rope: eps");
  for (int i = 0; i < 3; ++i) {
    if (in_strides[i] % 8 || out_strides[i] % 8)
      return set_error(DT_ERR_UNSUPPORTED,
                       "dt_qk_norm_rope: strides must be multiples of 8");
  }
  if (!aligned16(q) || !aligned16(k) || !aligned16(q_out) || !aligned16(k_out))
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_qk_norm_rope: tensors must be 16-byte aligned");
  NormRopeParams p;
  p.q = q;
  p.k = k;
  p.qo = q_out;
  p.ko = k_out;
  p.wq = wq;
  p.wk = wk;
  p.head_scale = q_head_scale;
  p.pos = pos;
  p.in_sb = in_strides[0];
  p.in_ss = in_strides[1];
  p.in_sh = in_strides[2];
  p.out_sb = out_strides[0];
  p.out_ss = out_strides[1];
  p.out_sh = out_strides[2];
  p.B = B;
  p.S = S;
  p.H = H;
  p.eps = eps;
  p.valid_len = valid_len < 0 ? -1 : valid_len;
  p.mode = mode;
  p.rot = 0;
  if (mode != DT_ROPE_NONE) {
    if (!pos || !axis_dims)
      return set_error(DT_ERR_ARG, "dt_qk_norm_rope: rope needs pos, axis_dims");
    if (!(theta > 0.f)) return set_error(DT_ERR_ARG, "dt_qk_norm_rope: theta");
    int rot = 0;
    for (int a = 0; a < 3; ++a) {
      if (axis_dims[a] < 0 || axis_dims[a] % 2)
        return set_error(DT_ERR_ARG, "dt_qk_norm_rope: axis dim %d not even",
                         axis_dims[a]);
      rot += axis_dims[a];
    }
    if (rot > D || rot == 0)
      return set_error(DT_ERR_ARG, "dt_qk_norm_rope: rotary %d vs D %d", rot, D);
    if (mode == DT_ROPE_HALF && (rot / 2) % 8)
      return set_error(DT_ERR_UNSUPPORTED,
                       "dt_qk_norm_rope: rotate-half needs rotary/2 %% 8 == 0");
    p.rot = rot;
    int j = 0;
    for (int a = 0; a < 3; ++a) {
      for (int i = 0; i < axis_dims[a] / 2; ++i, ++j) {
        const double f = pow((double)theta, -2.0 * i / axis_dims[a]);
        p.freq_rev[j] = (float)(f / (2.0 * M_PI));
        p.pair_axis[j] = (int8_t)a;
      }
    }
  }
  const int64_t ntok = (int64_t)B * S;
  // Enough wavefronts to keep every CU busy with several waves in flight;
  // each wavefront then strides over tokens.
  int64_t blocks = (ntok + 3) / 4;
  if (blocks > 4096) blocks = 4096;
  hipStream_t st = (hipStream_t)stream;
  if (D == 128)
    hipLaunchKernelGGL(qk_norm_rope_kernel<128>, dim3((unsigned)blocks),
                       dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL(qk_norm_rope_kernel<64>, dim3((unsigned)blocks),
                       dim3(256), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "dt_qk_norm_rope: %s", hipGetErrorString(e));
  return DT_OK;
}
