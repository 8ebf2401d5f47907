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
//   * a token's 2H rows (r < H a q head, r >= H a k head) are split into
//     blockIdx.y chunks of two rows; a group of LPR lanes owns one token
//     and walks its chunk, so one cos/sin evaluation serves both rows of
//     the chunk; the token index splits into (b, s) by multiply-high
//     division by S;
//   * a row of D channels is covered by LPR = D/16 lanes, each holding two
//     8-channel chunks (two 16-byte loads), so a wavefront covers 64/LPR
//     tokens and each 16-byte access is naturally aligned;
//   * the chunks a lane holds are chosen so every rotation pair sits inside
//     one lane: rotate-half pairs chunk c with chunk c + rotary/16, the
//     interleaved form keeps (2j, 2j+1) inside a chunk, pass-through chunks
//     are handed out two per lane after the rotating ones;
//   * wavefronts are one-shot: each issues all of its chunk's
//     (non-temporal) loads, then computes and stores and retires, which keeps
//     the most bytes in flight per register (a persistent loop measured
//     slower);
//   * the RMS reduction is a butterfly over the LPR lanes of a row;
//   * angles are carried in revolutions (frequency / 2pi, position axis per
//     slot from a per-block LDS table) and reduced to [0, 1) before the
//     hardware sin/cos, which take revolutions.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include <type_traits>

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
  // runtime valid length in device memory, or null (valid_len): rows
  // s >= the value are zeroed (<= 0: every row, > S: none); one value for
  // the batch (valid_len_count <= 1) or one per batch element
  const int32_t* valid_len_dev;
  int valid_len_count;
  int mode;
  int rot;  // rotated channels (even, <= D)
  // table-driven rotation (dt_qk_norm_rope_table): per-pair cos / sin rows
  // of token (b, s) at b*tab_sb + s*tab_ss (floats); null otherwise
  const float* cos_tab;
  const float* sin_tab;
  int64_t tab_sb, tab_ss;
  // table rows 16-byte aligned and every lane-chunk's pairs all rotating or
  // all passing through: cos/sin are read as float4
  int tab_vec;
  uint32_t ntok;         // B * S
  int rc;                 // rows per chunk (blockIdx.y selects the chunk)
  uint32_t divs_m, divs_s;  // multiply-high division by S
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

// Chunk indices (in units of 8 channels) owned by lane `li` of a row.  The
// first chunk of every lane is, as far as the rotation allows, the lane's
// own position, so one load instruction of the LPR lanes of a row covers
// contiguous memory.
template <int D>
__device__ __host__ __forceinline__ void lane_chunks(int li, int mode, int rot,
                                                     int& c0, int& c1) {
  constexpr int LPR = D / 16;
  if (mode == DT_ROPE_HALF) {
    const int hc = rot / 16;  // rotating chunks in the first half
    if (li < hc) {
      c0 = li;           // pairs with chunk li + hc
      c1 = li + hc;
    } else {
      c0 = li + hc;      // pass-through chunks [2hc, 2*LPR)
      c1 = li + LPR;
    }
  } else {
    c0 = li;
    c1 = li + LPR;
  }
}

__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(v[i] << 16);
    f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}

// Two fp32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 r = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return r;
}

// n / d for n < 2^31 with a precomputed multiplier (Granlund-Montgomery):
// q = (umulhi(n, m) + n) >> s.
__device__ __forceinline__ uint32_t fast_div(uint32_t n, uint32_t m,
                                             uint32_t s) {
  return (__umulhi(n, m) + n) >> s;
}

constexpr int kThreads = 256;  // threads per block (4 wavefronts)

// F32IN: q and k are fp32 (each 8-channel chunk two 16-byte loads) instead
// of bf16; the arithmetic and the bf16 output are the same.
template <int D, int RC, bool TABLE, bool F32IN = false>
__global__ __launch_bounds__(kThreads) void qk_norm_rope_kernel(NormRopeParams p) {
  using L = Layout<D>;
  // the LDS tables below are filled by one thread per entry
  static_assert(kThreads >= L::LPR * 16 + L::LPR * 8, "block too small");
  const int lane = threadIdx.x & 63;
  const int li = lane % L::LPR;   // lane within row
  const int grp = lane / L::LPR;  // row group = token slot within wavefront

  int c0, c1;
  lane_chunks<D>(li, p.mode, p.rot, c0, c1);

  // Per-block tables in LDS, one entry per thread: weights of q and of
  // (k - q) in lane-chunk order, and each lane-in-row's 8 rotation slots as
  // (frequency in revolutions, axis).  Slots that do not rotate get
  // frequency 0 (identity rotation).  Indexed [element][lane in row]: the
  // LPR lanes of a row read LPR consecutive words (distinct banks) and
  // every row group reads the same ones (a broadcast), so the reads are
  // free of bank conflicts.
  __shared__ __attribute__((aligned(16))) float s_wq[16][L::LPR];
  __shared__ __attribute__((aligned(16))) float s_dw[16][L::LPR];
  __shared__ __attribute__((aligned(16))) float s_fr[8][L::LPR];
  __shared__ __attribute__((aligned(16))) int s_ax[8][L::LPR];
  {
    const int t = threadIdx.x;
    if (t < L::LPR * 16) {
      const int tl = t / 16, e = t % 16;
      int t0, t1;
      lane_chunks<D>(tl, p.mode, p.rot, t0, t1);
      const int ch = (e < 8 ? t0 * 8 + e : t1 * 8 + e - 8);
      const float a = p.wq[ch];
      s_wq[e][tl] = a;
      s_dw[e][tl] = p.wk[ch] - a;
    } else if (t < L::LPR * 16 + L::LPR * 8) {
      const int tt = t - L::LPR * 16;
      const int tl = tt / 8, i = tt % 8;
      int t0, t1;
      lane_chunks<D>(tl, p.mode, p.rot, t0, t1);
      // HALF: slot i pairs element i (chunk t0) with element 8+i (chunk t1).
      // PAIR: slot i pairs elements (2i, 2i+1) of the 16 (t0 then t1).
      int j = -1;
      if (p.mode == DT_ROPE_HALF) {
        const int ch = t0 * 8 + i;
        j = (ch < p.rot / 2) ? ch : -1;
      } else if (p.mode == DT_ROPE_PAIR) {
        const int ch = (i < 4 ? t0 * 8 + 2 * i : t1 * 8 + 2 * (i - 4));
        j = (ch < p.rot) ? ch / 2 : -1;
      }
      // The tables are read in place from the kernel-argument segment (the
      // parameter block is this kernel's only argument, at offset 0), so
      // the indexing does not copy the block to scratch.
      const NormRopeParams* kp =
          (const NormRopeParams*)__builtin_amdgcn_kernarg_segment_ptr();
      if constexpr (!TABLE) {
        s_fr[i][tl] = j >= 0 ? kp->freq_rev[j] : 0.f;
        s_ax[i][tl] = j >= 0 ? kp->pair_axis[j] : 0;
      }
    }
  }

  // Token of this lane group; rows [r0, r0 + rc) of it (r < H: q head r,
  // else k head r - H).
  const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const uint32_t tok = wave * (uint32_t)L::ROWS + grp;
  const int r0 = blockIdx.y * p.rc;
  const int r1 = min(r0 + p.rc, 2 * p.H);
  const bool live = tok < p.ntok;
  const int b = live ? (int)fast_div(tok, p.divs_m, p.divs_s) : 0;
  const int s = live ? (int)(tok - (uint32_t)b * (uint32_t)p.S) : 0;
  // (b may differ between the lane groups of a wavefront: a per-lane read)
  int vl = p.valid_len;
  if (p.valid_len_dev != nullptr) {
    const int n = p.valid_len_dev[p.valid_len_count > 1 ? b : 0];
    vl = n <= 0 ? 0 : (n > p.S ? p.S : n);
  }
  const bool zero = (vl >= 0) && (s >= vl);
  using TIn = std::conditional_t<F32IN, float, uint16_t>;
  const TIn* qsrc = (const TIn*)p.q + b * p.in_sb + s * p.in_ss;
  const TIn* ksrc = (const TIn*)p.k + b * p.in_sb + s * p.in_ss;
  uint16_t* qdst = p.qo + b * p.out_sb + s * p.out_ss;
  uint16_t* kdst = p.ko + b * p.out_sb + s * p.out_ss;

  // cos/sin of this lane's 8 rotation slots, shared by the token's rows.
  // Table mode loads them here, with the rows, so their latency overlaps;
  // slot i's pair follows the same rule as the LDS slot table above.
  float cs[8], sn[8];
  if constexpr (TABLE) {
    if (live && !zero) {
      const float* cr = p.cos_tab + b * p.tab_sb + (int64_t)s * p.tab_ss;
      const float* sr = p.sin_tab + b * p.tab_sb + (int64_t)s * p.tab_ss;
      if (p.tab_vec) {
        // HALF: slots 0..7 are pairs c0*8 .. c0*8+7.  PAIR: slots 0..3 are
        // pairs c0*4 .. +3, slots 4..7 pairs c1*4 .. +3.
        const bool half = p.mode == DT_ROPE_HALF;
        const int j0 = half ? c0 * 8 : c0 * 4;
        const int j1 = half ? c0 * 8 + 4 : c1 * 4;
        const bool v0 = half ? j0 < p.rot / 2 : c0 * 8 < p.rot;
        const bool v1 = half ? v0 : c1 * 8 < p.rot;
        const f32x4 one = {1.f, 1.f, 1.f, 1.f}, nil = {0.f, 0.f, 0.f, 0.f};
        const f32x4 ca = v0 ? *(const f32x4*)(cr + j0) : one;
        const f32x4 sa = v0 ? *(const f32x4*)(sr + j0) : nil;
        const f32x4 cb = v1 ? *(const f32x4*)(cr + j1) : one;
        const f32x4 sb = v1 ? *(const f32x4*)(sr + j1) : nil;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          cs[i] = ca[i];
          sn[i] = sa[i];
          cs[4 + i] = cb[i];
          sn[4 + i] = sb[i];
        }
      } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int j;
        if (p.mode == DT_ROPE_HALF) {
          const int ch = c0 * 8 + i;
          j = ch < p.rot / 2 ? ch : -1;
        } else {
          const int ch = (i < 4 ? c0 * 8 + 2 * i : c1 * 8 + 2 * (i - 4));
          j = ch < p.rot ? ch / 2 : -1;
        }
        cs[i] = j >= 0 ? cr[j] : 1.f;
        sn[i] = j >= 0 ? sr[j] : 0.f;
      }
      }
    }
  }

  // a row's two chunks: bf16, one 16-byte load each; fp32, two
  constexpr int NV = F32IN ? 4 : 2;
  u32x4 v[RC][NV];
#pragma unroll
  for (int i = 0; i < RC; ++i) {
    const int r = r0 + i;
    if (!live || zero || r >= r1) continue;
    const bool isk = r >= p.H;
    const TIn* src = (isk ? ksrc + (r - p.H) * p.in_sh : qsrc + r * p.in_sh);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int ch = (j < NV / 2 ? c0 : c1) * 8 + (F32IN ? 4 * (j & 1) : 0);
      v[i][j] = __builtin_nontemporal_load((const u32x4*)(src + ch));
    }
  }
  __syncthreads();  // LDS tables (their global loads overlap the row loads)
  if (!live) return;

  if (zero) {
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < RC; ++i) {
      const int r = r0 + i;
      if (r >= r1) continue;
      const bool isk = r >= p.H;
      uint16_t* dst = (isk ? kdst + (r - p.H) * p.out_sh : qdst + r * p.out_sh);
      __builtin_nontemporal_store(z, (u32x4*)(dst + c0 * 8));
      __builtin_nontemporal_store(z, (u32x4*)(dst + c1 * 8));
    }
    return;
  }

  if (p.mode != DT_ROPE_NONE) {
    if constexpr (!TABLE) {
      const int32_t* ps = p.pos + (int64_t)s * 3;
      const float pt = (float)ps[0], ph = (float)ps[1], pw = (float)ps[2];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int ax = s_ax[i][li];
        const float pv = ax == 0 ? pt : (ax == 1 ? ph : pw);
        float rev = pv * s_fr[i][li];
        rev = rev - floorf(rev);
        sn[i] = __builtin_amdgcn_sinf(rev);
        cs[i] = __builtin_amdgcn_cosf(rev);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < RC; ++i) {
    const int r = r0 + i;
    if (r >= r1) continue;
    const bool isk = r >= p.H;
    const int h = isk ? r - p.H : r;
    uint16_t* dst = (isk ? kdst : qdst) + h * p.out_sh;
    float x[16];
    if constexpr (F32IN) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) x[4 * j + e] = __uint_as_float(v[i][j][e]);
    } else {
      unpack8(v[i][0], x);
      unpack8(v[i][1], x + 8);
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) ss += x[e] * x[e];
#pragma unroll
    for (int off = 1; off < L::LPR; off <<= 1) ss += __shfl_xor(ss, off, 64);
    float rr = rsqrtf(ss * (1.0f / D) + p.eps);
    const float kf = isk ? 1.f : 0.f;
    if (!isk && p.head_scale != nullptr) rr *= p.head_scale[h];
#pragma unroll
    for (int e = 0; e < 16; ++e)
      x[e] *= __builtin_fmaf(kf, s_dw[e][li], s_wq[e][li]);
    if (p.mode == DT_ROPE_HALF) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float a = x[e], bb = x[8 + e];
        x[e] = a * cs[e] - bb * sn[e];
        x[8 + e] = bb * cs[e] + a * sn[e];
      }
    } else if (p.mode == DT_ROPE_PAIR) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float a = x[2 * e], bb = x[2 * e + 1];
        x[2 * e] = a * cs[e] - bb * sn[e];
        x[2 * e + 1] = a * sn[e] + bb * cs[e];
      }
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) x[e] *= rr;
    __builtin_nontemporal_store(pack8(x), (u32x4*)(dst + c0 * 8));
    __builtin_nontemporal_store(pack8(x + 8), (u32x4*)(dst + c1 * 8));
  }
}

// Rows of one token per lane group (a chunk).  Two: a lane then has four
// 16-byte loads in flight, as the best plain copy of the same bytes does.
// Chunks of 4, 5 and 8 rows kept more bytes per lane in flight and measured
// 3-12 % slower (V7, V4, I1, I2: bit-identical output); one row per chunk
// evaluates cos/sin for every row and lost 2-6 % against two.
constexpr int kChunk = 2;
// Table mode reads the token's cos/sin row once per chunk, so it keeps
// chunks of up to kTableChunk rows (balanced: 10 -> 2 x 5, 48 -> 6 x 8):
// with two-row chunks the table reads took it from 0.331 to 0.378 ms at V7.
constexpr int kTableChunk = 8;

static void magic_u32(uint32_t d, uint32_t& m, uint32_t& s) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  m = (uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1);
  s = l;
}

static bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace dt

namespace dt {
namespace {

template <bool TABLE, bool F32IN = false>
int launch_norm_rope(NormRopeParams& p, int D, hipStream_t st) {
  const int64_t ntok = (int64_t)p.B * p.S;
  if (ntok >= (1ll << 31))
    return set_error(DT_ERR_SHAPE, "dt_qk_norm_rope: B*S >= 2^31 tokens");
  p.ntok = (uint32_t)ntok;
  magic_u32((uint32_t)p.S, p.divs_m, p.divs_s);
  // Each lane group takes one token and a chunk of its 2H rows (rows
  // c*rc .. c*rc + rc - 1 of the order q heads, then k heads).
  const int cmax = TABLE ? kTableChunk : kChunk;
  const int nchunk = (2 * p.H + cmax - 1) / cmax;
  p.rc = (2 * p.H + nchunk - 1) / nchunk;
  const int tok_per_wave = (D == 128) ? Layout<128>::ROWS : Layout<64>::ROWS;
  const int64_t waves = (ntok + tok_per_wave - 1) / tok_per_wave;
  constexpr int kWaves = kThreads / 64;
  const dim3 grid((unsigned)((waves + kWaves - 1) / kWaves), (unsigned)nchunk);
  // the row buffer is sized to the chunk (registers decide how many
  // wavefronts stay resident)
  if constexpr (!TABLE) {
    if (D == 128)
      hipLaunchKernelGGL((qk_norm_rope_kernel<128, kChunk, TABLE, F32IN>),
                         grid, dim3(kThreads), 0, st, p);
    else
      hipLaunchKernelGGL((qk_norm_rope_kernel<64, kChunk, TABLE, F32IN>),
                         grid, dim3(kThreads), 0, st, p);
  } else if (D == 128) {
    if (p.rc <= 4)
      hipLaunchKernelGGL((qk_norm_rope_kernel<128, 4, TABLE, F32IN>), grid, dim3(kThreads), 0, st, p);
    else if (p.rc <= 5)
      hipLaunchKernelGGL((qk_norm_rope_kernel<128, 5, TABLE, F32IN>), grid, dim3(kThreads), 0, st, p);
    else if (p.rc <= 6)
      hipLaunchKernelGGL((qk_norm_rope_kernel<128, 6, TABLE, F32IN>), grid, dim3(kThreads), 0, st, p);
    else
      hipLaunchKernelGGL((qk_norm_rope_kernel<128, 8, TABLE, F32IN>), grid, dim3(kThreads), 0, st, p);
  } else {
    if (p.rc <= 4)
      hipLaunchKernelGGL((qk_norm_rope_kernel<64, 4, TABLE, F32IN>), grid, dim3(kThreads), 0, st, p);
    else
      hipLaunchKernelGGL((qk_norm_rope_kernel<64, 8, TABLE, F32IN>), grid, dim3(kThreads), 0, st, p);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "dt_qk_norm_rope: %s", hipGetErrorString(e));
  return DT_OK;
}

// Argument checks and parameter block shared by both entry points.
int fill_params(NormRopeParams& p, const void* q, const void* k,
                uint16_t* q_out, uint16_t* k_out, int B, int S, int H, int D,
                const int64_t* in_strides, const int64_t* out_strides,
                const float* wq, const float* wk, float eps,
                const float* q_head_scale, int mode, int valid_len,
                const int32_t* valid_len_dev) {
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
  p.q = (const uint16_t*)q;  // fp32 inputs are re-typed in the kernel
  p.k = (const uint16_t*)k;
  p.qo = q_out;
  p.ko = k_out;
  p.wq = wq;
  p.wk = wk;
  p.head_scale = q_head_scale;
  p.pos = nullptr;
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
  // a length in device memory: valid_len is its entry count
  if (int rc = dev_len_count(valid_len_dev, valid_len, B, "dt_qk_norm_rope",
                             &p.valid_len_count))
    return rc;
  p.valid_len = (valid_len < 0 || valid_len_dev != nullptr) ? -1 : valid_len;
  p.valid_len_dev = valid_len_dev;
  p.mode = mode;
  p.rot = 0;
  p.cos_tab = p.sin_tab = nullptr;
  p.tab_sb = p.tab_ss = 0;
  p.tab_vec = 0;
  return DT_OK;
}

// rotary width checks shared by both entry points
int check_rot(int mode, int rot, int D) {
  if (rot > D || rot <= 0 || rot % 2)
    return set_error(DT_ERR_ARG, "dt_qk_norm_rope: rotary %d vs D %d", rot, D);
  if (mode == DT_ROPE_HALF && (rot / 2) % 8)
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_qk_norm_rope: rotate-half needs rotary/2 %% 8 == 0");
  return DT_OK;
}

}  // namespace
}  // namespace dt

namespace dt {
namespace {

// dt_qk_norm_rope and dt_qk_norm_rope_f32 (F32IN: fp32 q and k).
template <bool F32IN>
int norm_rope_entry(const void* q, const void* k,
                               uint16_t* q_out, uint16_t* k_out, int B, int S,
                               int H, int D, const int64_t* in_strides,
                               const int64_t* out_strides, const float* wq,
                               const float* wk, float eps,
                               const float* q_head_scale, int mode,
                               const int32_t* pos, const int32_t* axis_dims,
                               float theta, int valid_len,
                               const int32_t* valid_len_dev, void* stream) {
  NormRopeParams p;
  if (int rc = fill_params(p, q, k, q_out, k_out, B, S, H, D, in_strides,
                           out_strides, wq, wk, eps, q_head_scale, mode,
                           valid_len, valid_len_dev))
    return rc;
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
    if (int rc = check_rot(mode, rot, D)) return rc;
    p.rot = rot;
    p.pos = pos;
    int j = 0;
    for (int a = 0; a < 3; ++a) {
      for (int i = 0; i < axis_dims[a] / 2; ++i, ++j) {
        const double f = pow((double)theta, -2.0 * i / axis_dims[a]);
        p.freq_rev[j] = (float)(f / (2.0 * M_PI));
        p.pair_axis[j] = (int8_t)a;
      }
    }
  }
  return launch_norm_rope<false, F32IN>(p, D, (hipStream_t)stream);
}

}  // namespace
}  // namespace dt



extern "C" int dt_qk_norm_rope(const uint16_t* q, const uint16_t* k,
                               uint16_t* q_out, uint16_t* k_out, int B, int S,
                               int H, int D, const int64_t* in_strides,
                               const int64_t* out_strides, const float* wq,
                               const float* wk, float eps,
                               const float* q_head_scale, int mode,
                               const int32_t* pos, const int32_t* axis_dims,
                               float theta, int valid_len,
                               const int32_t* valid_len_dev, void* stream) {
  return dt::norm_rope_entry<false>(q, k, q_out, k_out, B, S, H, D, in_strides,
                                    out_strides, wq, wk, eps, q_head_scale,
                                    mode, pos, axis_dims, theta, valid_len,
                                    valid_len_dev, stream);
}

extern "C" int dt_qk_norm_rope_f32(const float* q, const float* k,
                                   uint16_t* q_out, uint16_t* k_out, int B,
                                   int S, int H, int D,
                                   const int64_t* in_strides,
                                   const int64_t* out_strides, const float* wq,
                                   const float* wk, float eps,
                                   const float* q_head_scale, int mode,
                                   const int32_t* pos,
                                   const int32_t* axis_dims, float theta,
                                   int valid_len, const int32_t* valid_len_dev,
                                   void* stream) {
  return dt::norm_rope_entry<true>(q, k, q_out, k_out, B, S, H, D, in_strides,
                                   out_strides, wq, wk, eps, q_head_scale,
                                   mode, pos, axis_dims, theta, valid_len,
                                   valid_len_dev, stream);
}

namespace dt {
namespace {

template <bool F32IN>
int norm_rope_table_entry(const void* q, const void* k, uint16_t* q_out,
                          uint16_t* k_out, int B, int S, int H, int D,
                          const int64_t* in_strides,
                          const int64_t* out_strides, const float* wq,
                          const float* wk, float eps,
                          const float* q_head_scale, int mode,
                          const float* cos_tab, const float* sin_tab,
                          const int64_t* tab_strides, int rot, int valid_len,
                          const int32_t* valid_len_dev, void* stream) {
  NormRopeParams p;
  if (int rc = fill_params(p, q, k, q_out, k_out, B, S, H, D, in_strides,
                           out_strides, wq, wk, eps, q_head_scale, mode,
                           valid_len, valid_len_dev))
    return rc;
  if (mode == DT_ROPE_NONE)
    return set_error(DT_ERR_ARG,
                     "dt_qk_norm_rope_table: mode must be HALF or PAIR");
  if (!cos_tab || !sin_tab || !tab_strides)
    return set_error(DT_ERR_ARG, "dt_qk_norm_rope_table: null table argument");
  if (int rc = check_rot(mode, rot, D)) return rc;
  p.rot = rot;
  p.cos_tab = cos_tab;
  p.sin_tab = sin_tab;
  p.tab_sb = tab_strides[0];
  p.tab_ss = tab_strides[1];
  p.tab_vec = aligned16(cos_tab) && aligned16(sin_tab) &&
              p.tab_sb % 4 == 0 && p.tab_ss % 4 == 0 &&
              (mode == DT_ROPE_HALF || rot % 8 == 0);
  return launch_norm_rope<true, F32IN>(p, D, (hipStream_t)stream);
}

}  // namespace
}  // namespace dt

extern "C" int dt_qk_norm_rope_table(
    const uint16_t* q, const uint16_t* k, uint16_t* q_out, uint16_t* k_out,
    int B, int S, int H, int D, const int64_t* in_strides,
    const int64_t* out_strides, const float* wq, const float* wk, float eps,
    const float* q_head_scale, int mode, const float* cos_tab,
    const float* sin_tab, const int64_t* tab_strides, int rot, int valid_len,
    const int32_t* valid_len_dev, void* stream) {
  return dt::norm_rope_table_entry<false>(
      q, k, q_out, k_out, B, S, H, D, in_strides, out_strides, wq, wk, eps,
      q_head_scale, mode, cos_tab, sin_tab, tab_strides, rot, valid_len,
      valid_len_dev, stream);
}

extern "C" int dt_qk_norm_rope_table_f32(
    const float* q, const float* k, uint16_t* q_out, uint16_t* k_out, int B,
    int S, int H, int D, const int64_t* in_strides,
    const int64_t* out_strides, const float* wq, const float* wk, float eps,
    const float* q_head_scale, int mode, const float* cos_tab,
    const float* sin_tab, const int64_t* tab_strides, int rot, int valid_len,
    const int32_t* valid_len_dev, void* stream) {
  return dt::norm_rope_table_entry<true>(
      q, k, q_out, k_out, B, S, H, D, in_strides, out_strides, wq, wk, eps,
      q_head_scale, mode, cos_tab, sin_tab, tab_strides, rot, valid_len,
      valid_len_dev, stream);
}
