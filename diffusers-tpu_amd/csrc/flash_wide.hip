// Flash attention forward for head dim 256 (gfx950): the head dims above
// 128 that kernels/splash.py accepts (it requires only D_v % 8 == 0,
// kernels/splash.py:156-160); dims 136..248 run zero-padded to 256 by the
// Python layer, as the smaller dims pad to 64 or 128.  Same contract as
// flash_attn_kernel (kernels/splash.py:566-650 and the residual form
// :665-742): GQA, a host or device key length (one for the batch or one per
// batch element), residual (o, m, l) outputs, the fixed-m operand.  Not
// here: E4M3 keys, block-sparse tables, packed V and the tail split.
//
// The D = 128 kernel's layout does not fit this width: two wavefronts per
// SIMD leave 256 registers each, and Q^T (64) + O^T (128) + the scores do
// not fit in them.  Here one wavefront runs per SIMD (a workgroup is 4
// wavefronts x 32 query rows), with O^T in the accumulation registers, and
// the key tile is 32 keys, so a ring of 4 stages of K and V stays at
// 128 KiB of LDS.
//   * S^T = K Q^T on v_mfma_f32_32x32x16_bf16, 16 channel steps, Q^T (the
//     query rows scaled by c = scale*log2 e, rounded to bf16) in registers;
//   * lazy exp2-domain softmax as in flash_attn_kernel: a re-base only on
//     the first tile and when a tile's per-lane sum leaves its range, the
//     internal reference 24 below the row's for online heads;
//   * O^T = V^T P^T: the packed probabilities are the B operand; V^T comes
//     from row-major V in LDS through ds_read_b64_tr_b16;
//   * K and V tiles move global -> LDS with buffer_load ... lds, two tiles
//     ahead, one barrier per tile.
// The softmax is not overlapped with the MFMAs (one wavefront per SIMD has
// no partner to fill the matrix pipe meanwhile): a correct, moderate-rate
// path for shapes the reference's models do not use.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <atomic>

#include "../../include/dt_attention.h"
#include "flash_common.h"

namespace dt {
namespace {

constexpr int kWD = 256;                  // head dim
constexpr int kWNW = 4;                   // wavefronts, one per SIMD
constexpr int kWBQ = kWNW * 32;           // 128 query rows per workgroup
constexpr int kWBKV = 32;                 // keys per tile
constexpr int kWStages = 4;               // LDS ring depth
constexpr int kWDist = 2;                 // tiles requested ahead of use
constexpr int kWRow = 2 * kWD;            // bytes of a K or V row (512)
constexpr int kWTileB = kWBKV * kWRow;    // 16 KiB
constexpr int kWVOff = kWStages * kWTileB;  // V stages after the K stages
constexpr int kWLds = 2 * kWVOff;         // 128 KiB
constexpr int kWLoads = kWTileB / 1024 / kWNW;  // 1 KiB DMAs per wave, K or V
constexpr int kWSteps = kWD / 16;         // QK channel steps
constexpr int kWNB = kWD / 32;            // 32-channel output blocks
constexpr float kWTrip = 4096.0f;
constexpr float kWShift = 24.0f;          // online heads' reference offset
constexpr float kWTripShifted = kWTrip * 16777216.0f;  // 2^(12 + 24)
constexpr float kWRecenter = 88.0f;       // kernels/fixed_m_bound.py:42

__device__ __forceinline__ float dot2_acc(uint32_t w, float acc) {
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), one,
                                         acc, false);
}

__global__ __launch_bounds__(kWNW * 64) void flash_wide_kernel(FlashParams p) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds_raw[];
  lds_u8* lds = (lds_u8*)lds_raw;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31;
  const int hf = lane >> 5;

  const int wg = xcd_remap(blockIdx.x, p.n_wg);
  const int qblk = wg % p.n_qblk;
  const int bh = wg / p.n_qblk;
  const int h = bh % p.Hq;
  const int b = bh / p.Hq;
  const int hk = h / (p.Hq / p.Hkv);
  const uint16_t* qbase = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* kbase = p.k + b * p.k_sb + hk * p.k_sh;
  const uint16_t* vbase = p.v + b * p.v_sb + hk * p.v_sh;
  const int q0 = qblk * kWBQ + wave * 32;
  const int row = q0 + l32;  // this lane's query row
  const int kv_end =
      resolve_len(p.kv_len_dev, p.kv_len_count, b, p.kv_end, p.Skv);
  const int ntiles = (kv_end + kWBKV - 1) / kWBKV;

  if (ntiles <= 0) {  // no keys (a device length of 0): the empty result
    if (row < p.Sq) {
      const int64_t bhrow = ((int64_t)b * p.Hq + h) * p.Sq + row;
#pragma unroll
      for (int j = 0; j < kWD / 8; ++j) {
        if (p.o32 != nullptr)
          *(u32x4*)(p.o32 + bhrow * kWD + (kWD / 2) * hf + 4 * j) =
              u32x4{0u, 0u, 0u, 0u};
        if (p.o != nullptr)
          *(u32x2*)(p.o + b * p.o_sb + h * p.o_sh + (int64_t)row * p.o_ss +
                    (kWD / 2) * hf + 4 * j) = u32x2{0u, 0u};
      }
      if (p.o32 != nullptr && hf == 0) {
        p.m[bhrow] = 0.f;
        p.l[bhrow] = 0.f;
      }
    }
    return;
  }

  // Q^T: lane holds row `row`, channels 16t + 8hf .. +8 for step t, scaled
  // by c and rounded to bf16 (kernels/splash.py:607-609).  Rows past Sq
  // load row Sq - 1 and are zeroed.
  bf16x8 qf[kWSteps];
  {
    const bool live = row < p.Sq;
    const uint16_t* qrow = qbase + (int64_t)(live ? row : p.Sq - 1) * p.q_ss;
    const uint32_t keep = live ? 0xffffffffu : 0u;
    u32x4 raws[kWSteps];
#pragma unroll
    for (int t = 0; t < kWSteps; ++t)
      raws[t] = *(const u32x4*)(qrow + 16 * t + 8 * hf);
#pragma unroll
    for (int t = 0; t < kWSteps; ++t) {
      u32x4 r = raws[t];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = r[e] & keep;
        r[e] = pack_bf16x2(__uint_as_float(w << 16) * p.c,
                           __uint_as_float(w & 0xffff0000u) * p.c);
      }
      qf[t] = __builtin_bit_cast(bf16x8, r);
    }
  }

  // Tile DMA: wave w fills key rows 8w .. 8w+7 of the K and V tiles, two
  // 512-byte rows per 1 KiB instruction; lane -> (row 8w + 2i + lane/32,
  // physical 16-byte chunk lane % 32).  K chunk c of key r sits at
  // c ^ (r & 15), V chunk c at c ^ (4 * (r & 3)) (the swizzles of the
  // D = 128 kernel's 256-byte rows, within each 256-byte half).
  const uint32_t krow = (uint32_t)p.k_ss * 2u;
  const uint32_t vrow = (uint32_t)p.v_ss * 2u;
  uint32_t kvo[kWLoads], vvo[kWLoads];
#pragma unroll
  for (int i = 0; i < kWLoads; ++i) {
    const int r = wave * 8 + 2 * i + (lane >> 5);
    const int pc = lane & 31;
    kvo[i] = r * krow + ((pc ^ (r & 15)) * 16);
    vvo[i] = r * vrow + ((pc ^ (4 * (r & 3))) * 16);
  }
  const uint32_t lds_k = (uint32_t)(uintptr_t)lds + (uint32_t)wave * 8 * kWRow;
  const uint32_t lds_v = lds_k + kWVOff;
  auto issue_tile = [&](int t) {
    const int kv0 = t * kWBKV;
    const int rows = kv_end - kv0 < kWBKV ? kv_end - kv0 : kWBKV;
    // descriptor ranges end at kv_end: rows past it arrive as zeros
    const u32x4 rk = make_rsrc((uint64_t)(uintptr_t)kbase + (uint64_t)kv0 * krow,
                               (uint32_t)rows * krow);
    const u32x4 rv = make_rsrc((uint64_t)(uintptr_t)vbase + (uint64_t)kv0 * vrow,
                               (uint32_t)rows * vrow);
    const uint32_t so = (uint32_t)(t % kWStages) * kWTileB;
#pragma unroll
    for (int i = 0; i < kWLoads; ++i)
      lds_dma16_buf(rk, kvo[i], lds_k + so + i * 1024);
#pragma unroll
    for (int i = 0; i < kWLoads; ++i)
      lds_dma16_buf(rv, vvo[i], lds_v + so + i * 1024);
  };

  // Operand offsets within a stage.  K (A operand of S^T): row l32, logical
  // chunk 2t + hf.  V^T (A operand of O^T) through ds_read_b64_tr_b16: in
  // each 16-lane group g, source lane j names 4 channels of one key
  // (key 4(g >> 1) + j/4, channels 16(g & 1) + 4(j % 4) of the block) and
  // lane i receives channel 16(g & 1) + i of 4 consecutive keys; the read
  // 8 rows further gives the other 4 of the 8 keys the lane's half of the
  // probability operand holds (keys 0-3 and 8-11, or 4-7 and 12-15).
  int kread[kWSteps];
#pragma unroll
  for (int t = 0; t < kWSteps; ++t)
    kread[t] = l32 * kWRow + (((2 * t + hf) ^ (l32 & 15)) * 16);
  const int g = lane >> 4, j16 = lane & 15;
  const int vkey = 4 * (g >> 1) + (j16 >> 2);
  const int vd0 = 16 * (g & 1) + 4 * (j16 & 3);
  const int vsw = 4 * (vkey & 3);
  int vread[kWNB];
#pragma unroll
  for (int mb = 0; mb < kWNB; ++mb) {
    const int d0 = 32 * mb + vd0;
    vread[mb] = kWVOff + vkey * kWRow + (((d0 >> 3) ^ vsw) * 16) + (d0 & 7) * 2;
  }

  f32x16 o[kWNB];
#pragma unroll
  for (int mb = 0; mb < kWNB; ++mb)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[mb][r] = 0.f;
  float m = 0.f, l = 0.f;
  bool fixed = false;
  if (p.mk != nullptr && p.mk[p.Hq + h] > 0.5f) {
    fixed = true;
    m = p.mk[h] - kWRecenter;
  }
  const float trip = fixed ? 3.0e38f : kWTripShifted;
  const float shift = fixed ? 0.f : kWShift;

#pragma unroll
  for (int t = 0; t < kWDist; ++t)
    if (t < ntiles) issue_tile(t);

  for (int jt = 0; jt < ntiles; ++jt) {
    {
      // tile jt resident once at most the next one's loads are in flight
      const int pend = (jt + 1 < ntiles) ? 1 : 0;
      wait_vmcnt(pend * 2 * kWLoads);
      __syncthreads();
    }
    // stage (jt + 2) % 4 was last read in iteration jt - 2
    if (jt + kWDist < ntiles) issue_tile(jt + kWDist);
    const lds_u8* kt = lds + (jt % kWStages) * kWTileB;
    const lds_u8* vt = lds + (jt % kWStages) * kWTileB;

    // ---- S^T = K Q^T, starting from -m: even and odd channel steps in two
    // accumulators (two independent MFMA chains), added at the end
    f32x16 s, s1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = -m;
      s1[r] = 0.f;
    }
    bf16x8 kr[4];
    kr[0] = __builtin_bit_cast(
        bf16x8, *(const __attribute__((address_space(3))) u32x4*)(kt + kread[0]));
    kr[1] = __builtin_bit_cast(
        bf16x8, *(const __attribute__((address_space(3))) u32x4*)(kt + kread[1]));
#pragma unroll
    for (int t = 0; t < kWSteps; ++t) {
      if (t + 2 < kWSteps)
        kr[(t + 2) & 3] = __builtin_bit_cast(
            bf16x8, *(const __attribute__((address_space(3))) u32x4*)(
                        kt + kread[t + 2]));
      if (t & 1)
        s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kr[t & 3], qf[t], s1, 0, 0, 0);
      else
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kr[t & 3], qf[t], s, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] += s1[r];
    // keys at or past kv_end -> -inf (register r holds key 8(r/4) + 4hf + r%4)
    const int kv0 = jt * kWBKV;
    if (kv0 + kWBKV > kv_end) {
      const int lim = kv_end - kv0 - 4 * hf;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rel = 8 * (r >> 2) + (r & 3);
        if (rel >= lim) s[r] = -INFINITY;
      }
    }

    // ---- probabilities against the current reference; re-base on the
    // first tile (online heads) or when the tile's sum leaves its range
    uint32_t pw[8];
    float sa = 0.f, sb = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pw[i] = pack_bf16x2(__builtin_amdgcn_exp2f(s[2 * i]),
                          __builtin_amdgcn_exp2f(s[2 * i + 1]));
      if (i & 1)
        sb = dot2_acc(pw[i], sb);
      else
        sa = dot2_acc(pw[i], sa);
    }
    float sum = sa + sb;
    const bool first = jt == 0 && !fixed;
    if (first || wave_any(!(sum <= trip))) {
      float mx = s[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float delta = first ? mx - shift : fmaxf(mx - shift, 0.f);
      const float alpha = __builtin_amdgcn_exp2f(-delta);
      m += delta;
      sa = 0.f;
      sb = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pw[i] = pack_bf16x2(__builtin_amdgcn_exp2f(s[2 * i] - delta),
                            __builtin_amdgcn_exp2f(s[2 * i + 1] - delta));
        if (i & 1)
          sb = dot2_acc(pw[i], sb);
        else
          sa = dot2_acc(pw[i], sa);
      }
      sum = sa + sb;
      l *= alpha;
#pragma unroll
      for (int mb = 0; mb < kWNB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[mb][r] *= alpha;
    }
    l += sum;

    // ---- O^T += V^T P^T: key step u (16 keys), output block mb
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const u32x4 pr = {pw[4 * u], pw[4 * u + 1], pw[4 * u + 2], pw[4 * u + 3]};
#pragma unroll
      for (int mb = 0; mb < kWNB; ++mb) {
        const lds_u8* a = vt + vread[mb] + u * 16 * kWRow;
        const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16*)(a));
        const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16*)(a + 8 * kWRow));
        const bf16x8 va = __builtin_bit_cast(
            bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        o[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            va, __builtin_bit_cast(bf16x8, pr), o[mb], 0, 0, 0);
      }
    }
  }

  // ---- epilogue: lane holds row `row`, channels 32mb + 8j + 4hf + e of
  // block mb (register 4j + e); the residual (m, l, o) of the reference
  // itself (the online offset taken out)
  if (row >= p.Sq) return;
  const float ltot = l + __shfl_xor(l, 32, 64);
  const float unshift = fixed ? 1.0f : 1.0f / 16777216.0f;  // 2^-kWShift
  const int64_t bhrow = ((int64_t)b * p.Hq + h) * p.Sq + row;
  if (p.o32 != nullptr) {
    float* dst = p.o32 + bhrow * kWD;
#pragma unroll
    for (int mb = 0; mb < kWNB; ++mb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = o[mb][4 * j + e] * unshift;
        *(f32x4*)(dst + 32 * mb + 8 * j + 4 * hf) = w;
      }
    if (hf == 0) {
      p.m[bhrow] = m + shift;
      p.l[bhrow] = ltot * unshift;
    }
  }
  if (p.o != nullptr) {
    const float inv = 1.0f / ltot;
    uint16_t* dst = p.o + b * p.o_sb + h * p.o_sh + (int64_t)row * p.o_ss;
#pragma unroll
    for (int mb = 0; mb < kWNB; ++mb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u32x2 w;
        w[0] = pack_bf16x2(o[mb][4 * j] * inv, o[mb][4 * j + 1] * inv);
        w[1] = pack_bf16x2(o[mb][4 * j + 2] * inv, o[mb][4 * j + 3] * inv);
        *(u32x2*)(dst + 32 * mb + 8 * j + 4 * hf) = w;
      }
  }
}

}  // namespace

int launch_flash_wide(const FlashParams& base, hipStream_t st) {
  if (base.k8 != nullptr || base.vt != nullptr || base.tile_span != nullptr)
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_flash_fwd: head dim 256 takes bf16 keys, row-major V "
                     "and no tile table");
  FlashParams p = base;
  p.n_qblk = (p.Sq + kWBQ - 1) / kWBQ;
  const int64_t nwg = (int64_t)p.n_qblk * p.Hq * p.B;
  if (nwg > 0x7fffffff)
    return set_error(DT_ERR_SHAPE, "dt_flash_fwd: grid too large");
  // byte offsets of one (b, h) slice's rows are 32-bit in the descriptors
  if ((int64_t)p.kv_end * p.k_ss * 2 >= (1ll << 32) ||
      (int64_t)p.kv_end * p.v_ss * 2 >= (1ll << 32))
    return set_error(DT_ERR_SHAPE, "dt_flash_fwd: K/V slice above 4 GiB");
  p.n_wg = (int)nwg;
  p.n_main = p.n_wg;
  p.n_split = 1;
  p.n_tail = 0;
  p.ws = nullptr;
  static std::atomic<uint64_t> lds_set{0};
  if (int rc = ensure_lds_limit((const void*)flash_wide_kernel, kWLds, lds_set,
                                "dt_flash_fwd"))
    return rc;
  hipLaunchKernelGGL(flash_wide_kernel, dim3(p.n_wg), dim3(kWNW * 64), kWLds,
                     st, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "dt_flash_fwd: %s", hipGetErrorString(e));
  return DT_OK;
}

}  // namespace dt
